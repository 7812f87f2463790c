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

// The rest of the router for one row whose logits (without the bias) 16
// lanes hold, four columns each (lanes 16 q .. 16 q + 15 of a wave; lane
// l16 columns c4 .. c4 + 3): softmax_tile_kernel's steps (the max, expf, the
// running sum in column order on the row's first lane, the quotients),
// topk_rows_kernel's ranking and the renormalisation in rank order.  Every
// thread of the workgroup calls it (it holds barriers); row t >= T stores
// nothing.  lg: the row's LDS scratch of kRouterMaxE + 1 floats.
__device__ __forceinline__ void router_tail(const RouterArgs& a, float (&y)[4], int c4,
                                            int64_t t, float* lg) {
  const int E = a.E;
  const int l16 = threadIdx.x & 15;
  const bool row_ok = t < a.T;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (c4 + j >= E) y[j] = 0.0f;
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
      lg[c4 + j] = y[j];
    }
  __syncthreads();
  if (l16 == 0) {
    float sum = 0.0f;
    for (int j = 0; j < E; ++j) sum = sum + lg[j];
    lg[kRouterMaxE] = sum;
  }
  __syncthreads();
  const float sum = lg[kRouterMaxE];
#pragma unroll
  for (int j = 0; j < 4; ++j) y[j] = y[j] / sum;
  // top-k: each round the best untaken column of each lane, then the best of
  // the 16 (a total order, so every lane agrees on the winner); the row's
  // first lane keeps the values for the renormalisation in rank order
  // (the values wait in lg[0 .. k), which only the row's first lane touches
  // from here on: the exps there are spent)
  uint32_t taken = 0;
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
      lg[s] = bv;
      denom = denom + bv;
      if (row_ok) {
        a.ids[t * a.k + s] = bi;
        if (a.vals) a.vals[t * a.k + s] = bv;
      }
    }
  }
  if (l16 == 0 && row_ok && a.weights)
    for (int s = 0; s < a.k; ++s) a.weights[t * a.k + s] = lg[s] / denom;
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
  const float accs[4] = {acc0, acc1, acc2, acc3};
  float y[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) y[j] = accs[j] + bias[j];
  router_tail(a, y, c4, m0 + r, lg[r]);
}

// The DPP form, for H % 128 == 0: thread (wave w, lane l) owns rows
// 8 w + 2 (l / 16) and the next of the workgroup's 32, and columns
// 4 (l % 16) .. + 3.  x never passes through LDS: for each 128-deep k-chunk,
// lane l holds x[row][k0 + 8 (l % 16) .. + 7] of its two rows in registers,
// and the value at k is broadcast from lane (k - k0) / 8 of each 16-lane row
// by DPP row_newbcast.  W's chunk ([128, 64] f32, 32 KiB) is staged through
// LDS, two stages: W rows loaded into registers during chunk c are written
// to LDS at the start of chunk c + 1 (for chunk c + 2), so a whole chunk of
// arithmetic covers each load.  Each logit is
// the same fmaf chain over k from 0 as the narrow kernel's, so the bits
// agree.  Per k a thread issues 2 broadcasts, 8 fmas and one 16-byte LDS
// read, against 4 fmas, a 16-byte and a 4-byte LDS read in the narrow form:
// the LDS traffic per fma halves and the broadcasts need no LDS.
template <int J>
__device__ __forceinline__ float row_bcast(float v) {
  return __int_as_float(
      __builtin_amdgcn_mov_dpp(__float_as_int(v), 0x150 + J, 0xf, 0xf, true));
}

// k-steps 8 J .. 8 J + 7 of a chunk; bc holds their W rows, read one group ahead
template <int J>
__device__ __forceinline__ void router_chunk(const float (*bs)[64], int c4, const float (&f0)[8],
                                             const float (&f1)[8], const float4 (&bc)[8],
                                             float (&acc0)[4], float (&acc1)[4]) {
  float4 bn[8];
  if constexpr (J + 1 < 16) {
#pragma unroll
    for (int e = 0; e < 8; ++e) bn[e] = *(const float4*)&bs[8 * (J + 1) + e][c4];
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float a0 = row_bcast<J>(f0[e]), a1 = row_bcast<J>(f1[e]);
    acc0[0] = fmaf(a0, bc[e].x, acc0[0]);
    acc0[1] = fmaf(a0, bc[e].y, acc0[1]);
    acc0[2] = fmaf(a0, bc[e].z, acc0[2]);
    acc0[3] = fmaf(a0, bc[e].w, acc0[3]);
    acc1[0] = fmaf(a1, bc[e].x, acc1[0]);
    acc1[1] = fmaf(a1, bc[e].y, acc1[1]);
    acc1[2] = fmaf(a1, bc[e].z, acc1[2]);
    acc1[3] = fmaf(a1, bc[e].w, acc1[3]);
  }
  if constexpr (J + 1 < 16) router_chunk<J + 1>(bs, c4, f0, f1, bn, acc0, acc1);
}

template <bool XBF16>
__global__ void __launch_bounds__(256) moe_router_dpp_kernel(RouterArgs a) {
  __shared__ __attribute__((aligned(16))) float Bs[2][128][64];  // 64 KiB
  __shared__ float lg[32][kRouterMaxE + 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, c4 = l16 * 4;
  const int rp = wave * 8 + (lane >> 4) * 2;  // the thread's first row in the workgroup
  const int64_t m0 = (int64_t)blockIdx.x * 32;
  const int E = a.E;
  constexpr int xe = XBF16 ? 2 : 4;
  constexpr int NV = XBF16 ? 1 : 2;  // 16-byte x vectors per row per chunk
  const int64_t r0 = m0 + rp < a.T ? m0 + rp : a.T - 1;
  const int64_t r1 = m0 + rp + 1 < a.T ? m0 + rp + 1 : a.T - 1;
  const char* x0 = (const char*)a.x + (r0 * a.x_rs + l16 * 8) * xe;
  const char* x1 = (const char*)a.x + (r1 * a.x_rs + l16 * 8) * xe;
  // W chunk loader: 2048 16-byte vectors, thread tid takes k-rows
  // tid / 16 + 16 i and columns 4 (tid % 16) .. + 3 (clamped past E)
  const int bk = tid >> 4, bc4 = (tid & 15) * 4;
  const float* wp = a.w + (int64_t)bk * E + (bc4 < E ? bc4 : E - 4);
  float bias[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) bias[j] = a.b[c4 + j < E ? c4 + j : 0];
  float acc0[4] = {0.0f, 0.0f, 0.0f, 0.0f}, acc1[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const int nch = (int)(a.H / 128);
  // the next chunk's x (as loaded) and W rows, in registers
  uint4 n0[NV], n1[NV];
  // (eight named registers: as an array the compiler kept them in scratch
  // memory across the chunk loop)
  float4 nb0, nb1, nb2, nb3, nb4, nb5, nb6, nb7;
#define REW_NB_LOAD(K0)                                       \
  do {                                                        \
    const float* q_ = wp + (int64_t)(K0) * E;                 \
    nb0 = *(const float4*)(q_);                               \
    nb1 = *(const float4*)(q_ + 16 * (int64_t)E);             \
    nb2 = *(const float4*)(q_ + 32 * (int64_t)E);             \
    nb3 = *(const float4*)(q_ + 48 * (int64_t)E);             \
    nb4 = *(const float4*)(q_ + 64 * (int64_t)E);             \
    nb5 = *(const float4*)(q_ + 80 * (int64_t)E);             \
    nb6 = *(const float4*)(q_ + 96 * (int64_t)E);             \
    nb7 = *(const float4*)(q_ + 112 * (int64_t)E);            \
  } while (0)
#define REW_NB_STORE(ST)                                      \
  do {                                                        \
    float (*bw_)[64] = Bs[ST];                                \
    *(float4*)&bw_[bk][bc4] = nb0;                            \
    *(float4*)&bw_[bk + 16][bc4] = nb1;                       \
    *(float4*)&bw_[bk + 32][bc4] = nb2;                       \
    *(float4*)&bw_[bk + 48][bc4] = nb3;                       \
    *(float4*)&bw_[bk + 64][bc4] = nb4;                       \
    *(float4*)&bw_[bk + 80][bc4] = nb5;                       \
    *(float4*)&bw_[bk + 96][bc4] = nb6;                       \
    *(float4*)&bw_[bk + 112][bc4] = nb7;                      \
  } while (0)
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    n0[i] = *(const uint4*)(x0 + 16 * i);
    n1[i] = *(const uint4*)(x1 + 16 * i);
  }
  REW_NB_LOAD(0);
  REW_NB_STORE(0);
  REW_NB_LOAD(nch > 1 ? 128 : 0);
  __syncthreads();
  for (int c = 0; c < nch; ++c) {
    // chunk c + 1's W rows into the other stage (last read in chunk c - 1,
    // before the barrier that ended it), then chunk c + 2's loads; all
    // chunk indices are clamped, so no branch separates a load from its use
    REW_NB_STORE((c + 1) & 1);
    REW_NB_LOAD((int64_t)(c + 2 < nch ? c + 2 : nch - 1) * 128);
    float f0[8], f1[8];
    if constexpr (XBF16) {
      const uint32_t w0[4] = {n0[0].x, n0[0].y, n0[0].z, n0[0].w};
      const uint32_t w1[4] = {n1[0].x, n1[0].y, n1[0].z, n1[0].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f0[2 * i] = vm::as_f(w0[i] << 16);
        f0[2 * i + 1] = vm::as_f(w0[i] & 0xffff0000u);
        f1[2 * i] = vm::as_f(w1[i] << 16);
        f1[2 * i + 1] = vm::as_f(w1[i] & 0xffff0000u);
      }
    } else {
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        f0[4 * i] = vm::as_f(n0[i].x);
        f0[4 * i + 1] = vm::as_f(n0[i].y);
        f0[4 * i + 2] = vm::as_f(n0[i].z);
        f0[4 * i + 3] = vm::as_f(n0[i].w);
        f1[4 * i] = vm::as_f(n1[i].x);
        f1[4 * i + 1] = vm::as_f(n1[i].y);
        f1[4 * i + 2] = vm::as_f(n1[i].z);
        f1[4 * i + 3] = vm::as_f(n1[i].w);
      }
    }
    // the next chunk's x
    const int64_t kn = (int64_t)(c + 1 < nch ? c + 1 : c) * 128;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      n0[i] = *(const uint4*)(x0 + kn * xe + 16 * i);
      n1[i] = *(const uint4*)(x1 + kn * xe + 16 * i);
    }
    const float (*bs)[64] = Bs[c & 1];
    float4 b0[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) b0[e] = *(const float4*)&bs[e][c4];
    router_chunk<0>(bs, c4, f0, f1, b0, acc0, acc1);
    __syncthreads();
  }
#undef REW_NB_LOAD
#undef REW_NB_STORE
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    float y[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) y[j] = (rr ? acc1[j] : acc0[j]) + bias[j];
    router_tail(a, y, c4, m0 + rp + rr, lg[rp + rr]);
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
  if (a.H % 128 == 0) {
    const unsigned blocks = (unsigned)((a.T + 31) / 32);
    if (a.x_bf16)
      hipLaunchKernelGGL(moe_router_dpp_kernel<true>, dim3(blocks), dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL(moe_router_dpp_kernel<false>, dim3(blocks), dim3(256), 0, stream, a);
    REW_HIP(hipGetLastError());
    return;
  }
  const unsigned blocks = (unsigned)((a.T + 15) / 16);
  if (a.x_bf16)
    hipLaunchKernelGGL(moe_router_kernel<true>, dim3(blocks), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(moe_router_kernel<false>, dim3(blocks), dim3(256), 0, stream, a);
  REW_HIP(hipGetLastError());
}

}  // namespace rew
