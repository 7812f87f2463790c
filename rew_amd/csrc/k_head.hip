// A classifier's last layer in one launch: rew's Linear -> softmax -> argmax
// (src/rew/nn/linear.nim:43-49, nn/activation.nim:64-77,
// ops/reduce.nim:202-225) over fp32 rows, as at the end of the MNIST MLP's
// forward.  The logits and probabilities never reach memory.
//
// Each workgroup owns kHeadRows rows: the rows and the weight sit in LDS
// (every load issued before the first store), thread (row, class) runs that
// logit's chain, and one thread per row runs the softmax and the argmax.
// Every value takes the ops, order and roundings of the unfused kernels:
// each logit is the sequential fmaf chain over k = 0, 1, ... of
// gemm_f32_small_kernel (zero terms past K to a multiple of 16) plus the
// bias, the softmax is softmax_tile_kernel's (max, then expf and the running
// sum, then the quotients), and the argmax keeps the lowest index of the
// maximum, INT32_MAX where a row holds NaN.  So the ids equal the unfused
// path's bit for bit.
#include "kernels.h"
#include "vm_device.h"

namespace rew {

namespace {

constexpr int kHeadRows = 4;     // rows per workgroup
constexpr int kHeadK = 1024;     // most inputs per row
constexpr int kHeadN = 64;       // most classes
constexpr int kHeadW = 8192;     // most weight elements (K N)

__global__ void __launch_bounds__(256) class_head_kernel(HeadArgs a) {
  __shared__ __attribute__((aligned(16))) float xs[kHeadRows][kHeadK];
  __shared__ float ws[kHeadW];
  __shared__ float ls[kHeadRows][kHeadN];
  const int t = threadIdx.x;
  const int64_t r0 = (int64_t)blockIdx.x * kHeadRows;
  const int nr = (int)(a.M - r0 < kHeadRows ? a.M - r0 : kHeadRows);
  const int K = (int)a.K, N = (int)a.N;
  const int K16 = (K + 15) & ~15;
  const int cpr = K16 / 4;  // 16-byte chunks per staged row

  // loads in batches of four per thread, each batch's loads issued before
  // its LDS stores (clamped addresses, no branches around the loads); rows
  // past M, columns past K and weights past K are zeros
  const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  const int nx = kHeadRows * cpr;  // 16-byte x chunks
#pragma unroll 1
  for (int e0 = 0; e0 < nx; e0 += 4 * 256) {
    float4 vx[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = e0 + t + 256 * i;
      const int r = e / cpr, k4 = (e - r * cpr) * 4;
      const int rc = r < nr ? r : 0, kc = k4 < K ? k4 : 0;
      vx[i] = *(const float4*)(a.x + (r0 + rc) * a.x_rs + kc);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = e0 + t + 256 * i;
      const int r = e / cpr, k4 = (e - r * cpr) * 4;
      if (e < nx) *(float4*)&xs[r][k4] = (r < nr && k4 < K) ? vx[i] : z;
    }
  }
  const int nw = K16 * N;
#pragma unroll 1
  for (int e0 = 0; e0 < nw; e0 += 4 * 256) {
    float vw[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = e0 + t + 256 * i;
      vw[i] = a.w[e < K * N ? e : 0];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = e0 + t + 256 * i;
      if (e < nw) ws[e] = e < K * N ? vw[i] : 0.0f;
    }
  }
  __syncthreads();

  // logits: thread (row, class)
  if (t < kHeadRows * N) {
    const int r = t / N, j = t - (t / N) * N;
    float acc = 0.0f;
    for (int k = 0; k < K16; ++k) acc = fmaf(xs[r][k], ws[k * N + j], acc);
    ls[r][j] = acc + a.b[j];
  }
  __syncthreads();

  // softmax and argmax of each row
  if (t < nr) {
    float* l = ls[t];
    float m = -INFINITY;
    for (int j = 0; j < N; ++j) m = vm::fmax_prop(m, l[j]);
    float sum = 0.0f;
    for (int j = 0; j < N; ++j) {
      const float e = expf(l[j] - m);
      l[j] = e;
      sum = sum + e;
    }
    float best = 0.0f;
    int bi = -1, nan = 0;
    for (int j = 0; j < N; ++j) {
      const float p = l[j] / sum;
      if (a.probs) a.probs[(r0 + t) * N + j] = p;
      if (p != p) nan = 1;
      else if (bi < 0 || p > best) {
        best = p;
        bi = j;
      }
    }
    a.ids[r0 + t] = (nan || bi < 0) ? INT32_MAX : bi;
  }
}

}  // namespace

bool class_head_ok(const HeadArgs& a) {
  const int64_t k16 = (a.K + 15) & ~(int64_t)15;
  return a.M > 0 && a.K > 0 && k16 <= kHeadK && a.K % 4 == 0 && a.N > 0 && a.N <= kHeadN &&
         k16 * a.N <= kHeadW && a.x_rs % 4 == 0 && ((uintptr_t)a.x & 15) == 0 &&
         a.M / kHeadRows < (1 << 30);
}

void launch_class_head(const HeadArgs& a, hipStream_t stream) {
  if (!class_head_ok(a)) fail(REW_MI355X_ERR_INVALID, "internal: class head launch outside its limits");
  const unsigned blocks = (unsigned)((a.M + kHeadRows - 1) / kHeadRows);
  hipLaunchKernelGGL(class_head_kernel, dim3(blocks), dim3(256), 0, stream, a);
  REW_HIP(hipGetLastError());
}

}  // namespace rew
