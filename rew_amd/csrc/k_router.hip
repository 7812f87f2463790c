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
// 0, then the bias add.  For H % 128 == 0 the matrix-core form below runs
// the same chains on f32 MFMAs, which round each step as fmaf does.  x may
// be bf16: its conversion to f32 is exact and happens on the load.  Then
// the 16 lanes of each row take
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

// The rest of the router for one row whose logits (with the bias) LANES
// lanes of a wave hold, COLS columns each (lanes LANES q .. LANES q +
// LANES - 1; the lane with l = lane % LANES holds columns c0 = COLS l ..
// c0 + COLS - 1): softmax_tile_kernel's steps (the max, expf, the running
// sum in column order on the row's first lane, the quotients),
// topk_rows_kernel's ranking and the renormalisation in rank order.  Every
// thread of the workgroup calls it (it holds barriers); row t >= T stores
// nothing.  lg: the row's LDS scratch of kRouterMaxE + 1 floats.
template <int LANES, int COLS>
__device__ __forceinline__ void router_tail(const RouterArgs& a, float (&y)[COLS], int c0,
                                            int64_t t, float* lg) {
  const int E = a.E;
  const int l = threadIdx.x & (LANES - 1);
  const bool row_ok = t < a.T;
#pragma unroll
  for (int j = 0; j < COLS; ++j)
    if (c0 + j >= E) y[j] = 0.0f;
  // softmax: the max (order-free) over the lanes, the exps in place, the
  // sum in column order on the row's first lane (the reduction's order),
  // then the quotients
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < COLS; ++j)
    if (c0 + j < E) m = vm::fmax_prop(m, y[j]);
#pragma unroll
  for (int off = LANES / 2; off >= 1; off >>= 1) m = vm::fmax_prop(m, __shfl_xor(m, off, LANES));
#pragma unroll
  for (int j = 0; j < COLS; ++j)
    if (c0 + j < E) {
      y[j] = expf(y[j] - m);
      lg[c0 + j] = y[j];
    }
  __syncthreads();
  if (l == 0) {
    float sum = 0.0f;
    for (int j = 0; j < E; ++j) sum = sum + lg[j];
    lg[kRouterMaxE] = sum;
  }
  __syncthreads();
  const float sum = lg[kRouterMaxE];
#pragma unroll
  for (int j = 0; j < COLS; ++j) y[j] = y[j] / sum;
  // top-k: each round the best untaken column of each lane, then the best of
  // the row's lanes (a total order, so every lane agrees on the winner); the
  // row's first lane keeps the values for the renormalisation in rank order
  // (the values wait in lg[0 .. k), which only the row's first lane touches
  // from here on: the exps there are spent)
  uint32_t taken = 0;
  float denom = 0.0f;
  for (int s = 0; s < a.k; ++s) {
    float bv = 0.0f;
    int bi = kNoCol;
#pragma unroll
    for (int j = 0; j < COLS; ++j)
      if (c0 + j < E && !((taken >> j) & 1) && rank_first(y[j], c0 + j, bv, bi)) {
        bv = y[j];
        bi = c0 + j;
      }
#pragma unroll
    for (int off = LANES / 2; off >= 1; off >>= 1) {
      const float ov = __shfl_xor(bv, off, LANES);
      const int oi = __shfl_xor(bi, off, LANES);
      if (rank_first(ov, oi, bv, bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if (bi >= c0 && bi < c0 + COLS) taken |= 1u << (bi - c0);
    if (l == 0) {
      lg[s] = bv;
      denom = denom + bv;
      if (row_ok) {
        a.ids[t * a.k + s] = bi;
        if (a.vals) a.vals[t * a.k + s] = bv;
      }
    }
  }
  if (l == 0 && row_ok && a.weights)
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
  router_tail<16, 4>(a, y, c4, m0 + r, lg[r]);
}

// W chunk staging of the matrix-core form: a [128, 64] f32 chunk
// of W's rows (columns past E clamped to E - 4 .. E - 1) is 2048 16-byte
// vectors; thread tid loads k-rows bk + 16 i (bk = tid / 16) at columns
// bc4 .. bc4 + 3 (bc4 = 4 (tid % 16)) from wp into eight named registers
// (as an array the compiler kept them in scratch memory across the chunk
// loop) and stores them to stage ST of Bs.
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

// The matrix-core form, for H % 128 == 0: wave w owns rows 8 w .. 8 w + 7 of
// the workgroup's 32 as two quads, and each k-step of a quad is one
// v_mfma_f32_4x4x1_16b_f32: sixteen 4 x 4 blocks, block b computing the
// quad's 4 rows by columns 4 b .. 4 b + 3, so lane l accumulates column l of
// the 4 rows.  An f32 MFMA with one k per block rounds each step exactly as
// fmaf(x, w, acc) does (a single rounding of the exact product plus the
// accumulator, denormals kept), so the chain over k from 0 gives every logit
// the bits of the VALU chain, at twice the VALU's multiply-add rate.  x
// reaches the matrix core by the MFMA's A broadcast: lane 4 j + i holds
// x[row i][k0 + 8 j .. + 7] of a 128-deep chunk (one 16-byte load per quad
// for bf16), and the step for k = k0 + 8 j + e takes A from value e of lane
// group j (CBSZ 4, ABID j).  W's [128, 64] chunks are staged through LDS in
// two stages: W rows loaded into registers during chunk c are written to LDS
// at the start of chunk c + 1 (for chunk c + 2), so a whole chunk of
// arithmetic covers each load; lane l reads W[k][l], one 4-byte read per k
// shared by both quads.  A dependent 4x4x1 f32 MFMA waits about 40 cycles for
// the previous step of its chain, and the T x E logits give each SIMD only
// two chains (its wave's two quads), so the chains' latency, not the matrix
// core's rate, sets the time: about 24 cycles per MFMA.
typedef float f4_t __attribute__((ext_vector_type(4)));

// k-steps 8 J .. 8 J + 7 of a chunk; bc and bn hold the W values of groups J
// and J + 1, and group J + 2's are read here, two groups (32 MFMAs) ahead of
// their use (the scheduling barrier keeps the compiler from sinking the
// reads next to their MFMAs)
template <int J>
__device__ __forceinline__ void router_mchunk(const float (*bs)[64], int lane,
                                              const float (&x0)[8], const float (&x1)[8],
                                              const float (&bc)[8], const float (&bn)[8],
                                              f4_t& acc0, f4_t& acc1) {
  float bnn[8];
  if constexpr (J + 2 < 16) {
#pragma unroll
    for (int e = 0; e < 8; ++e) bnn[e] = bs[8 * (J + 2) + e][lane];
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    acc0 = __builtin_amdgcn_mfma_f32_4x4x1f32(x0[e], bc[e], acc0, 4, J, 0);
    acc1 = __builtin_amdgcn_mfma_f32_4x4x1f32(x1[e], bc[e], acc1, 4, J, 0);
  }
  if constexpr (J + 1 < 16) router_mchunk<J + 1>(bs, lane, x0, x1, bn, bnn, acc0, acc1);
}

template <bool XBF16>
__global__ void __launch_bounds__(256) moe_router_mfma_kernel(RouterArgs a) {
  __shared__ __attribute__((aligned(16))) float Bs[2][128][64];  // 64 KiB
  __shared__ float lg[32][kRouterMaxE + 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t m0 = (int64_t)blockIdx.x * 32;
  const int E = a.E;
  constexpr int xe = XBF16 ? 2 : 4;
  constexpr int NV = XBF16 ? 1 : 2;  // 16-byte x vectors per lane per quad per chunk
  // lane 4 j + i: row i of each quad, k offset 8 j within a chunk
  const int64_t q0 = m0 + 8 * wave + (lane & 3), q1 = q0 + 4;
  const int64_t r0 = q0 < a.T ? q0 : a.T - 1, r1 = q1 < a.T ? q1 : a.T - 1;
  const char* x0 = (const char*)a.x + (r0 * a.x_rs + 8 * (lane >> 2)) * xe;
  const char* x1 = (const char*)a.x + (r1 * a.x_rs + 8 * (lane >> 2)) * xe;
  const int bk = tid >> 4, bc4 = (tid & 15) * 4;
  const float* wp = a.w + (int64_t)bk * E + (bc4 < E ? bc4 : E - 4);
  const int nch = (int)(a.H / 128);
  uint4 n0[NV], n1[NV];
  float4 nb0, nb1, nb2, nb3, nb4, nb5, nb6, nb7;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    n0[i] = *(const uint4*)(x0 + 16 * i);
    n1[i] = *(const uint4*)(x1 + 16 * i);
  }
  REW_NB_LOAD(0);
  REW_NB_STORE(0);
  REW_NB_LOAD(nch > 1 ? 128 : 0);
  __syncthreads();
  f4_t acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
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
    float b0[8], b1[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      b0[e] = bs[e][lane];
      b1[e] = bs[8 + e][lane];
    }
    router_mchunk<0>(bs, lane, f0, f1, b0, b1, acc0, acc1);
    __syncthreads();
  }
  // lane l holds column l of the wave's 8 rows: the logits (with the bias)
  // go to the rows' LDS scratch, and each row's 16 lanes read their 4
  // columns back for the tail
  const float bias = a.b[lane < E ? lane : 0];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    lg[8 * wave + i][lane] = acc0[i] + bias;
    lg[8 * wave + 4 + i][lane] = acc1[i] + bias;
  }
  __syncthreads();
  const int c4 = (lane & 15) * 4;
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    const int row = 8 * wave + 4 * rr + (lane >> 4);
    float y[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) y[j] = lg[row][c4 + j];
    router_tail<16, 4>(a, y, c4, m0 + row, lg[row]);
  }
}
#undef REW_NB_LOAD
#undef REW_NB_STORE

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
      hipLaunchKernelGGL(moe_router_mfma_kernel<true>, dim3(blocks), dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL(moe_router_mfma_kernel<false>, dim3(blocks), dim3(256), 0, stream, a);
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
