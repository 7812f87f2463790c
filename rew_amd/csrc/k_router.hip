// A mixture-of-experts router in one launch: rew's DeepSeekMoE.route
// (src/rew/models/deepseek.nim:132-137), over token rows of x:
//   logits = Linear(astype(x, f32))      (nn/linear.nim:43-49)
//   probs  = softmax(logits, 1)          (nn/activation.nim:64-77)
//   topW, topI = topK(probs, k, 1, true) (ops/sort.nim:36-90)
//   topWeights = topW / reduceSum(topW, [1])
// The logits, probabilities and unnormalised values never reach memory.
//
// The product is gemm_f32_narrow_kernel's (16 rows per workgroup, thread t
// owns row t / 16 and columns 4 (t % 16) .. + 3, 32-deep k-steps in two
// register sets): every logit is the same sequential fmaf chain over k from
// 0, then the bias add.  x may be bf16: its conversion to f32 is exact and
// happens on the load.  Then the 16 lanes of each row take
// softmax_tile_kernel's steps (the max, expf, the running sum in column
// order, the quotients), topk_rows_kernel's ranking (larger first, NaN last,
// the lower column on ties) and the renormalisation in rank order, as the
// [T, k] row reduction and the divide compute it; the max and each round's
// best are order-free reductions over the lanes, the two sums run on one
// lane in the reference order.  So every output equals the six-launch
// path's bit for bit.
#include <type_traits>

#include "kernels.h"
#include "vm_device.h"

namespace rew {

namespace {

constexpr int kNoCol = 0x7fffffff;

// a ranks before b under "larger first, NaN last, lower index on ties"
__device__ __forceinline__ bool rank_first(float av, int ai, float bv, int bi) {
  if (ai == kNoCol) return false;
  if (bi == kNoCol) return true;
  const bool an = av != av, bn = bv != bv;
  if (an != bn) return !an;
  if (!an && av != bv) return av > bv;
  return ai < bi;
}

template <bool XBF16>
__global__ void __launch_bounds__(256) moe_router_kernel(RouterArgs a) {
  __shared__ __attribute__((aligned(16))) float As[32][17];  // [k][row]
  __shared__ __attribute__((aligned(16))) float Bs[32][64];  // [k][column]
  __shared__ float lg[16][kRouterMaxE + 1];  // the row's exps, then its sum
  const int tid = threadIdx.x;
  const int r = tid >> 4, c4 = (tid & 15) * 4;
  const int64_t m0 = (int64_t)blockIdx.x * 16;
  const int E = a.E;
  // loaders: A, 16 rows x 32 k (threads 0..127, four elements each); B,
  // 32 k x 64 columns (two 16-byte chunks per thread, k rows bk and bk + 16)
  const int ar = (tid >> 3) & 15, ak = (tid & 7) * 4;
  const int64_t arow = m0 + ar < a.T ? m0 + ar : a.T - 1;
  const int bk = tid >> 4;
  const int bcol = c4 < E ? c4 : E - 4;
  const float* bp = a.w + bk * a.E + bcol;
  const int64_t b16 = 16 * (int64_t)a.E;
  // A stays in its own format in the register sets (bf16: 8 bytes per
  // thread) and becomes f32 at the LDS store, so that no load is waited for
  // before the next k-step's arithmetic
  using RawA = typename std::conditional<XBF16, uint2, float4>::type;
  const char* abase = (const char*)a.x + arow * a.x_rs * (XBF16 ? 2 : 4) + ak * (XBF16 ? 2 : 4);
  RawA pa0{}, pa1{};
  float4 pb00, pb01, pb10, pb11;
  auto gload = [&](RawA& pa, float4& pb0, float4& pb1, int64_t k0) {
    if (tid < 128) pa = *(const RawA*)(abase + k0 * (XBF16 ? 2 : 4));
    pb0 = *(const float4*)(bp + k0 * a.E);
    pb1 = *(const float4*)(bp + k0 * a.E + b16);
  };
  auto sstore = [&](const RawA& pa, const float4& pb0, const float4& pb1) {
    if (tid < 128) {
      float4 v;
      if constexpr (XBF16)
        v = make_float4(vm::as_f(pa.x << 16), vm::as_f(pa.x & 0xffff0000u),
                        vm::as_f(pa.y << 16), vm::as_f(pa.y & 0xffff0000u));
      else
        v = pa;
      As[ak][ar] = v.x;
      As[ak + 1][ar] = v.y;
      As[ak + 2][ar] = v.z;
      As[ak + 3][ar] = v.w;
    }
    *(float4*)&Bs[bk][c4] = pb0;
    *(float4*)&Bs[bk + 16][c4] = pb1;
  };
  // the bias of this thread's columns, read before the k-loop
  float bias[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) bias[j] = a.b[c4 + j < E ? c4 + j : 0];
  float acc0 = 0.0f, acc1 = 0.0f, acc2 = 0.0f, acc3 = 0.0f;
  // eight k-steps of A and B at a time from LDS into registers, then their
  // fmas in k order (the reads of a group are waited for once, not per step)
  auto step = [&]() {
#pragma unroll
    for (int k8 = 0; k8 < 32; k8 += 8) {
      float av[8];
      float4 bv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        av[i] = As[k8 + i][r];
        bv[i] = *(const float4*)&Bs[k8 + i][c4];
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        acc0 = fmaf(av[i], bv[i].x, acc0);
        acc1 = fmaf(av[i], bv[i].y, acc1);
        acc2 = fmaf(av[i], bv[i].z, acc2);
        acc3 = fmaf(av[i], bv[i].w, acc3);
      }
    }
  };
  // H % 64 == 0: the k-steps come in pairs, set 0 then set 1
  gload(pa0, pb00, pb01, 0);
  gload(pa1, pb10, pb11, 32);
  for (int64_t k0 = 0; k0 < a.H; k0 += 64) {
    sstore(pa0, pb00, pb01);
    __syncthreads();
    if (k0 + 64 < a.H) gload(pa0, pb00, pb01, k0 + 64);
    step();
    __syncthreads();
    sstore(pa1, pb10, pb11);
    __syncthreads();
    if (k0 + 96 < a.H) gload(pa1, pb10, pb11, k0 + 96);
    step();
    __syncthreads();
  }
  // the row's 16 lanes (one wave holds four rows) hold its logits, four
  // columns each; columns past E take no part
  const int l16 = tid & 15;
  const bool row_ok = m0 + r < a.T;
  float y[4];
  const float accs[4] = {acc0, acc1, acc2, acc3};
#pragma unroll
  for (int j = 0; j < 4; ++j) y[j] = c4 + j < E ? accs[j] + bias[j] : 0.0f;
  // softmax: the max (order-free) over the 16 lanes, the exps in place, the
  // sum in column order on the row's first lane (the reduction's order),
  // then the quotients
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (c4 + j < E) m = vm::fmax_prop(m, y[j]);
#pragma unroll
  for (int off = 8; off >= 1; off >>= 1) m = vm::fmax_prop(m, __shfl_xor(m, off, 16));
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (c4 + j < E) {
      y[j] = expf(y[j] - m);
      lg[r][c4 + j] = y[j];
    }
  __syncthreads();
  if (l16 == 0) {
    float sum = 0.0f;
    for (int j = 0; j < E; ++j) sum = sum + lg[r][j];
    lg[r][kRouterMaxE] = sum;
  }
  __syncthreads();
  const float sum = lg[r][kRouterMaxE];
#pragma unroll
  for (int j = 0; j < 4; ++j) y[j] = y[j] / sum;
  // top-k: each round the best untaken column of each lane, then the best of
  // the 16 (a total order, so every lane agrees on the winner); the row's
  // first lane keeps the values for the renormalisation in rank order
  uint32_t taken = 0;
  float vals[kRouterMaxK];
  float denom = 0.0f;
  for (int s = 0; s < a.k; ++s) {
    float bv = 0.0f;
    int bi = kNoCol;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (c4 + j < E && !((taken >> j) & 1) && rank_first(y[j], c4 + j, bv, bi)) {
        bv = y[j];
        bi = c4 + j;
      }
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) {
      const float ov = __shfl_xor(bv, off, 16);
      const int oi = __shfl_xor(bi, off, 16);
      if (rank_first(ov, oi, bv, bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if (bi >= c4 && bi < c4 + 4) taken |= 1u << (bi - c4);
    if (l16 == 0) {
      vals[s] = bv;
      denom = denom + bv;
      if (row_ok) {
        const int64_t t = m0 + r;
        a.ids[t * a.k + s] = bi;
        if (a.vals) a.vals[t * a.k + s] = bv;
      }
    }
  }
  if (l16 == 0 && row_ok && a.weights) {
    const int64_t t = m0 + r;
    for (int s = 0; s < a.k; ++s) a.weights[t * a.k + s] = vals[s] / denom;
  }
}

}  // namespace

bool moe_router_ok(const RouterArgs& a) {
  const int64_t xe = a.x_bf16 ? 2 : 4;
  return a.T >= 1 && a.H >= 64 && a.H % 64 == 0 && a.E >= 4 && a.E <= kRouterMaxE &&
         a.E % 4 == 0 && a.k >= 1 && a.k <= kRouterMaxK && a.k <= a.E &&
         (a.x_rs * xe) % 16 == 0 && ((uintptr_t)a.x & 15) == 0 && ((uintptr_t)a.w & 15) == 0 &&
         a.T / 16 < (1 << 30);
}

void launch_moe_router(const RouterArgs& a, hipStream_t stream) {
  if (!moe_router_ok(a)) fail(REW_MI355X_ERR_INVALID, "internal: router launch outside its limits");
  const unsigned blocks = (unsigned)((a.T + 15) / 16);
  if (a.x_bf16)
    hipLaunchKernelGGL(moe_router_kernel<true>, dim3(blocks), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(moe_router_kernel<false>, dim3(blocks), dim3(256), 0, stream, a);
  REW_HIP(hipGetLastError());
}

}  // namespace rew
