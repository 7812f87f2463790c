// A classifier's last layer in one launch: rew's Linear -> softmax -> argmax
// (src/rew/nn/linear.nim:43-49, nn/activation.nim:64-77,
// ops/reduce.nim:202-225) over fp32 rows, as at the end of the MNIST MLP's
// forward.  The logits and probabilities never reach memory.
//
// Each workgroup owns kHeadRows rows, one wave per row: the rows and the
// weight (transposed, k-contiguous per class) are staged in LDS in one round
// of loads (every load issued before the first store), lane j < N of a
// row's wave runs logit j's chain, and the wave then holds the row's logits
// in registers for the softmax and the argmax.  Every value takes the ops,
// order and roundings of the unfused kernels: each logit is the sequential
// fmaf chain over k = 0, 1, ... of gemm_f32_small_kernel (zero terms past K
// to a multiple of 16) plus the bias; the softmax is softmax_tile_kernel's
// (the max, which is order-free as it only enters as x - m; expf per lane;
// the sum of the exps in column order, read across the lanes one at a time;
// the quotients per lane); the argmax keeps the lowest index of the maximum
// (a total order, so the shuffle reduction picks what the sequential scan
// picks), INT32_MAX where a row holds NaN.  So the ids equal the unfused
// path's bit for bit.
#include "kernels.h"
#include "vm_device.h"

namespace rew {

namespace {

constexpr int kHeadRows = 4;     // rows per workgroup (one wave each)
constexpr int kHeadK = 1024;     // most inputs per row
constexpr int kHeadN = 64;       // most classes
constexpr int kHeadW = 8192;     // most weight elements (K N)

__global__ void __launch_bounds__(256) class_head_kernel(HeadArgs a) {
  __shared__ __attribute__((aligned(16))) float xs[kHeadRows][kHeadK];
  // the weight transposed, [class][k] at a pitch of K16 + 4 floats (the
  // classes' 16-byte reads of one k land on distinct banks)
  __shared__ __attribute__((aligned(16))) float ws[kHeadW + 4 * kHeadN];
  const int t = threadIdx.x, lane = t & 63, r = t >> 6;
  const int64_t r0 = (int64_t)blockIdx.x * kHeadRows;
  const int nr = (int)(a.M - r0 < kHeadRows ? a.M - r0 : kHeadRows);
  const int K = (int)a.K, N = (int)a.N;
  const int K16 = (K + 15) & ~15, WP = K16 + 4;
  const int cpr = K16 / 4;  // 16-byte chunks per staged row

  // one round: up to 4 x chunks and 8 weight chunks per thread, all loads
  // (clamped addresses) before any store; rows past M, columns past K and
  // weights past K are zeros
  const int nx = kHeadRows * cpr, nw4 = K * N / 4;
  float4 vx[4], vw[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = t + 256 * i;
    const int rr = e / cpr, k4 = (e - rr * cpr) * 4;
    const int rc = rr < nr ? rr : 0, kc = k4 < K ? k4 : 0;
    vx[i] = *(const float4*)(a.x + (r0 + rc) * a.x_rs + kc);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int e = t + 256 * i;
    vw[i] = *(const float4*)(a.w + 4 * (e < nw4 ? e : 0));
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = t + 256 * i;
    const int rr = e / cpr, k4 = (e - rr * cpr) * 4;
    // (per-component selects: a float4 select went through scratch memory)
    const bool in = rr < nr && k4 < K;
    if (e < nx)
      *(float4*)&xs[rr][k4] = make_float4(in ? vx[i].x : 0.0f, in ? vx[i].y : 0.0f,
                                          in ? vx[i].z : 0.0f, in ? vx[i].w : 0.0f);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int e = t + 256 * i;  // elements 4 e .. 4 e + 3 of the [K, N] weight
    if (e < nw4) {
      const int k0 = (4 * e) / N, j0 = 4 * e - k0 * N;
      const int k1 = (4 * e + 1) / N, j1 = 4 * e + 1 - k1 * N;
      const int k2 = (4 * e + 2) / N, j2 = 4 * e + 2 - k2 * N;
      const int k3 = (4 * e + 3) / N, j3 = 4 * e + 3 - k3 * N;
      ws[j0 * WP + k0] = vw[i].x;
      ws[j1 * WP + k1] = vw[i].y;
      ws[j2 * WP + k2] = vw[i].z;
      ws[j3 * WP + k3] = vw[i].w;
    }
  }
  // the weight's zero pad k = K .. K16 - 1 of every class
  for (int e = t; e < N * (K16 - K); e += 256) {
    const int j = e / (K16 - K);
    ws[j * WP + K + (e - j * (K16 - K))] = 0.0f;
  }
  __syncthreads();

  // logit j of row r on lane j: four k-steps of both operands per pair of
  // 16-byte reads, eight such pairs issued before their fmas
  float l = 0.0f;
  if (lane < N) {
    const float* xr = xs[r];
    const float* wr = ws + lane * WP;
    float acc = 0.0f;
#pragma unroll 8
    for (int k = 0; k < K16; k += 4) {
      const float4 xv = *(const float4*)(xr + k), wv = *(const float4*)(wr + k);
      acc = fmaf(xv.x, wv.x, acc);
      acc = fmaf(xv.y, wv.y, acc);
      acc = fmaf(xv.z, wv.z, acc);
      acc = fmaf(xv.w, wv.w, acc);
    }
    l = acc + a.b[lane];
  }
  if (r >= nr) return;  // whole waves; no barrier follows

  // softmax: the max over the row's lanes, the exps per lane, their sum in
  // column order (each lane's exp read in turn), the quotients per lane
  float m = lane < N ? l : -INFINITY;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) m = vm::fmax_prop(m, __shfl_xor(m, off));
  const float e = lane < N ? expf(l - m) : 0.0f;
  float sum = 0.0f;
  for (int j = 0; j < N; ++j) sum = sum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), j));
  const float p = e / sum;
  if (a.probs && lane < N) a.probs[(r0 + r) * N + lane] = p;
  // argmax: NaN anywhere gives INT32_MAX; otherwise the larger value, the
  // lower index on ties
  const bool nan = __ballot(lane < N && p != p) != 0;
  float bv = p;
  int bi = lane < N ? lane : 0x7fffffff;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(bv, off);
    const int oi = __shfl_xor(bi, off);
    if (oi != 0x7fffffff && (bi == 0x7fffffff || ov > bv || (ov == bv && oi < bi))) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane == 0) a.ids[r0 + r] = nan ? INT32_MAX : bi;
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
