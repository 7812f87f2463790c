// Fused scaled-dot-product attention (flash style) on bf16 MFMA.
//
// Replaces rew's SDPA op chain (src/rew/nn/attention.nim:36-81):
//   scores = dot_general(q, k)            -> bf16 [B,H,Sq,Sk] (operand dtype)
//   s      = f32(scores) * scale (+ mask)  -> f32
//   attn   = bf16(softmax(s))              -> bf16
//   out    = dot_general(attn, v)          -> bf16 [B,H,Sq,D]
// without materialising anything of size Sq x Sk.  GQA is an index map
// (kv head = h / (H / Hkv)), not a copy.
//
// Per workgroup: 4 waves, 128 queries of one (b, h); each wave owns 32
// queries.  Key tiles of 64 keys stream HBM/L2 -> LDS by DMA (buffer_load
// ... lds with a scalar tile offset when every tile is whole, else
// global_load_lds_dwordx4), two stages, so neither K nor V passes through
// registers.  The wave computes S^T = K Q^T with v_mfma_f32_32x32x16_bf16,
// so every lane holds the scores of ONE query column: the row max / sum of
// the online softmax are lane-local plus one exchange with lane ^ 32
// (v_permlane32_swap).  The output is accumulated transposed,
// O^T = V^T P^T: the probabilities go straight from the S^T accumulators
// into the B operand.
//
// LDS layouts (64 keys x D, 16-byte chunks, XOR-swizzled through the DMA
// source addresses):
//   K: chunk c of key row r at physical chunk c ^ (r % (D/8)) -- ds_read_b128
//      fragments (32 keys x one d-chunk) spread over the bank slots;
//   V: row-major, chunk c of key row r at c ^ (4 (r % 4)), read with
//      ds_read_b64_tr_b16: in each 16-lane group source lane s points at key
//      row kb + s/4, d columns d0 + 4 (s % 4), and output lane i receives 4
//      consecutive keys of d-column d0 + i.  Two such reads give the 8 keys
//      of a lane's P fragment, in the order the S^T accumulator holds them
//      (keys 4g..4g+3 and 8+4g..8+4g+3 of each 16-key step), so V needs no
//      transpose or permutation in registers.
//
// Numerics: fp32 accumulation; scores rounded to bf16 (the dot_general
// result dtype) before the fp32 scale / mask; probabilities rounded to bf16
// before the PV product (the astype before the second dot_general); the
// output rounded to bf16 once.  The softmax works in log2 units,
// t = log2(e) (x * scale + mask) and p = exp2(t - m), with the hardware
// exp2 (1 ulp, results below 2^-126 may flush to zero); on tiles where the
// scale is positive and the mask is 0 or absent, t is formed inside one
// FMA.  The normalisation is applied at the end (online softmax), which
// differs from the two-pass op sequence only in rounding (and the running
// max it subtracts moves only once some row's max grew by more than 8, so
// the unnormalised probabilities stay below e^8).
#include <cstdlib>
#include <string>

#include "kernels.h"
#include "vm_device.h"

namespace rew {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s lds_v4s;
typedef __attribute__((address_space(3))) void lds_void;

namespace fa {
constexpr int BQ = 128;  // queries per workgroup
constexpr int BKV = 64;  // keys per tile
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazy = 8.0f;  // max growth (natural log) absorbed without rescaling
}  // namespace fa

// cmp(i, j) as selects on the (uniform) predicate, not a branch per element
__device__ __forceinline__ bool fa_visible(int cmp, int i, int j) {
  const bool lt = i < j, eq = i == j;
  return cmp == vm::CMP_EQ   ? eq
         : cmp == vm::CMP_NE ? !eq
         : cmp == vm::CMP_LT ? lt
         : cmp == vm::CMP_LE ? (lt || eq)
         : cmp == vm::CMP_GT ? !(lt || eq)
                             : !lt;
}

// Every (query, key) pair of queries [q0, q1] x keys [k0, k1] (inclusive)
// satisfies cmp; only the ordered predicates can be decided from corners.
__device__ __forceinline__ bool fa_all_visible(int cmp, int q0, int q1, int k0, int k1) {
  switch (cmp) {
    case vm::CMP_LE: return q1 <= k0;
    case vm::CMP_LT: return q1 < k0;
    case vm::CMP_GE: return q0 >= k1;
    case vm::CMP_GT: return q0 > k1;
    default: return false;
  }
}

// 2^x with the hardware v_exp_f32 (1 ulp) and no denormal-range fix-up:
// every argument here is <= 0 (a score minus its running max), and results
// below 2^-126 are probabilities far under one bf16 ulp of the row sum.
// (The library exp2f wraps the instruction in a range test and two
// rescales; on the Llama shape the flash kernel ran 9 % faster without.)
__device__ __forceinline__ float fa_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// max(a, b, c) in one v_max3_f32.  fmaxf would first quiet signalling NaNs
// with a v_max_f32 x, x per operand (MFMA results are not known to be
// canonical); a quiet NaN operand is ignored either way.
__device__ __forceinline__ float fa_max3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// Two fp32 values rounded to bf16 (RNE; v_cvt_pk_bf16_f32), packed.
__device__ __forceinline__ uint32_t cvt_bf16x2(float a, float b) {
  const bf16x2_t v = __builtin_convertvector((f32x2_t){a, b}, bf16x2_t);
  uint32_t u;
  __builtin_memcpy(&u, &v, 4);
  return u;
}

__device__ __forceinline__ void dma16(const void* src, uint16_t* lds) {
  __builtin_amdgcn_global_load_lds(src, (lds_void*)lds, 16, 0, 0);
}

// Buffer descriptor over `base` with no range limit (callers keep every
// offset inside the tensor); the base is wave-uniform and readfirstlane
// says so, which keeps the descriptor in SGPRs.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t fa_rsrc(const void* base) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  void* p = (void*)(uintptr_t)(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(p, (short)0, 0x7fffffff, 0x00020000);
}
// 16 bytes per lane from base + voff + soff into LDS (buffer_load ... lds):
// the per-lane offset is fixed, the tile advance is the scalar `soff`.
__device__ __forceinline__ void dma16_buf(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                          uint16_t* lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)lds, 16, voff, soff, 0, 0);
}

// Tile kinds of the softmax step, each straight-line code:
//   0 plain     every key in range and visible, scale > 0: t is formed
//               inside the exp's FMA and the max comes from the raw
//               accumulators (rounding and scaling are monotone);
//   1 diagonal  a whole tile under an ordered mask that adds 0 where
//               visible, scale > 0: t = fma(x, scale log2 e, visible ? 0 :
//               mask_false log2 e), visibility from one per-lane threshold;
//   2 general   anything else: t = (x * scale + mask) log2 e, -inf past Sk.
// The plain tiles of queries [q0, q_last] form one range of key tiles
// [lo, hi), found once per wave group instead of per tile.
struct FaKinds {
  int lo, hi;  // plain key tiles
  int diag;    // kind of the other whole tiles: diagonal up / down, or general
  int whole;   // key tiles below this one are whole
};
__device__ __forceinline__ FaKinds fa_kinds(const FlashArgs& a, int q0, int q_last) {
  FaKinds k;
  k.whole = a.Sk / fa::BKV;
  k.lo = 0;
  k.hi = 0;
  const bool diag_ok = a.scale > 0.0f && a.mask && a.mask_true == 0.0f && a.cmp >= vm::CMP_LT;
  k.diag = !diag_ok ? 2 : (a.cmp == vm::CMP_LE || a.cmp == vm::CMP_LT) ? 1 : 3;
  if (!(a.scale > 0.0f)) return k;
  if (!a.mask) {
    k.hi = k.whole;
    return k;
  }
  if (a.mask_true != 0.0f) return k;
  // every pair visible: LE q_last <= k0, LT q_last < k0, GE q0 >= k0 + 63,
  // GT q0 > k0 + 63 (k0 = 64 kt)
  switch (a.cmp) {
    case vm::CMP_LE: k.lo = (q_last + fa::BKV - 1) / fa::BKV; k.hi = k.whole; break;
    case vm::CMP_LT: k.lo = (q_last + fa::BKV) / fa::BKV; k.hi = k.whole; break;
    case vm::CMP_GE: k.hi = q0 >= fa::BKV - 1 ? (q0 - (fa::BKV - 1)) / fa::BKV + 1 : 0; break;
    case vm::CMP_GT: k.hi = q0 >= fa::BKV ? (q0 - fa::BKV) / fa::BKV + 1 : 0; break;
    default: break;
  }
  k.hi = min(k.hi, k.whole);
  return k;
}
__device__ __forceinline__ int fa_kind(const FaKinds& k, int kt) {
  return (kt >= k.lo && kt < k.hi) ? 0 : (kt < k.whole ? k.diag : 2);
}

// Scores rounded to bf16 in place (the dot_general result dtype; ROUND) and
// their max over the lane's 32 keys.  Rounding is monotone, so the max of
// the rounded scores is the rounded max of the raw ones.  bf16(x) as an
// fp32 value takes one instruction: the pack of (0, x) holds bf16(x) in its
// high half over a zero low half.
template <bool ROUND>
__device__ __forceinline__ float fa_round_max(f32x16_t (&sacc)[2]) {
  float m0 = -INFINITY, m1 = -INFINITY;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int e = 0; e < 16; e += 2) {
      if constexpr (ROUND) {
        sacc[kb][e] = vm::as_f(cvt_bf16x2(0.0f, sacc[kb][e]));
        sacc[kb][e + 1] = vm::as_f(cvt_bf16x2(0.0f, sacc[kb][e + 1]));
      }
      if (kb == 0) m0 = fa_max3(m0, sacc[0][e], sacc[0][e + 1]);
      else m1 = fa_max3(m1, sacc[1][e], sacc[1][e + 1]);
    }
  return fa_max3(m0, m1, -INFINITY);
}

// One online-softmax step over a tile of S^T = K Q^T (64 keys x 32 queries;
// lane (c, g) holds query qi = column c, keys k0 + kb 32 + (e / 4) 8 + g 4 +
// e % 4 in sacc[kb][e]), given the scores as fa_round_max left them and
// their max mr: scores in log2 units, t = log2(e) (bf16(x) scale + mask),
// the tile max, the lazily rescaled running max / sum (O rescaled when the
// max moved), and the probabilities packed as bf16 pairs pk[kb][e/2] for the
// PV product (the running sum is left to fa_row_sum).  One straight-line body per tile
// kind (FA_PLAIN, FA_DIAG_UP / FA_DIAG_DOWN for masks that keep keys above /
// below the diagonal, FA_GENERAL).
enum { FA_PLAIN = 0, FA_DIAG_UP = 1, FA_GENERAL = 2, FA_DIAG_DOWN = 3 };
template <int DT, int KIND>
__device__ __forceinline__ void fa_softmax_tile(const FlashArgs& a, int k0, int qi, int g,
                                                float sl2, f32x16_t (&sacc_in)[2],
                                                float mr, uint32_t (&pk)[2][8], float& m_run,
                                                float& l_run, float& alpha_out) {
  using namespace fa;
  f32x16_t(&t)[2] = sacc_in;  // non-plain kinds: the scores in log2 units, in place
  float mt;
  if constexpr (KIND == FA_PLAIN) {
    mt = mr * sl2;
  } else if constexpr (KIND == FA_DIAG_UP || KIND == FA_DIAG_DOWN) {
    // key j = k0 + off (off = kb 32 + (e / 4) 8 + g 4 + e % 4) is visible
    // iff j - qi >= lo (LE, LT) or j - qi <= -lo (GE, GT)
    constexpr bool kUp = KIND == FA_DIAG_UP;
    const float mf2 = a.mask_false * kLog2e;
    const int lo = (a.cmp == vm::CMP_LT || a.cmp == vm::CMP_GT) ? 1 : 0;
    const int base = k0 - qi + g * 4;
    const int thr = kUp ? lo - base : -lo - base;
    float m0 = -INFINITY, m1 = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; e += 2) {
        const int off = kb * 32 + (e >> 2) * 8 + (e & 3);
        const bool v0 = kUp ? off >= thr : off <= thr;
        const bool v1 = kUp ? off + 1 >= thr : off + 1 <= thr;
        const float t0 = fmaf(sacc_in[kb][e], sl2, v0 ? 0.0f : mf2);
        const float t1 = fmaf(sacc_in[kb][e + 1], sl2, v1 ? 0.0f : mf2);
        t[kb][e] = t0;
        t[kb][e + 1] = t1;
        if (kb == 0) m0 = fa_max3(m0, t0, t1);
        else m1 = fa_max3(m1, t0, t1);
      }
    mt = fa_max3(m0, m1, -INFINITY);
  } else {
    float m0 = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; e += 2) {
        const int j0 = k0 + kb * 32 + (e >> 2) * 8 + g * 4 + (e & 3);
        float x0 = sacc_in[kb][e] * a.scale, x1 = sacc_in[kb][e + 1] * a.scale;
        if (a.mask) {
          x0 += fa_visible(a.cmp, qi, j0) ? a.mask_true : a.mask_false;
          x1 += fa_visible(a.cmp, qi, j0 + 1) ? a.mask_true : a.mask_false;
        }
        x0 = j0 < a.Sk ? x0 * kLog2e : -INFINITY;
        x1 = j0 + 1 < a.Sk ? x1 * kLog2e : -INFINITY;
        t[kb][e] = x0;
        t[kb][e + 1] = x1;
        m0 = fmaxf(m0, fmaxf(x0, x1));
      }
    mt = m0;
  }
  {
    // lanes c and c + 32 hold the two halves of one query's keys
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt),
                                                      false, false);
    mt = fa_max3(__uint_as_float(sw[0]), __uint_as_float(sw[1]), -INFINITY);
  }
  // Lazy rescaling: the probabilities are taken against the running max
  // m_run (log2 units), which moves (rescaling O and the sum) only when
  // some row of the wave saw its max grow by more than kLazy (natural
  // log); otherwise p <= e^kLazy, well inside fp32 and bf16.  O / l is
  // the same either way up to rounding.  Selects, not branches, except for
  // the rare rescale of O.
  const float m_new = fmaxf(m_run, mt);
  const bool grow = !(m_new - m_run <= kLazy * kLog2e);  // (also when m_run is still -inf)
  const bool rescale = __builtin_amdgcn_ballot_w64(grow) != 0;
  const float m_use = rescale ? (m_new == -INFINITY ? 0.0f : m_new) : m_run;
  const float alpha = rescale ? fa_exp2(m_run - m_use) : 1.0f;
  m_run = rescale ? m_new : m_run;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int e = 0; e < 16; e += 2) {
      if constexpr (KIND == FA_PLAIN)
        pk[kb][e >> 1] = cvt_bf16x2(fa_exp2(fmaf(sacc_in[kb][e], sl2, -m_use)),
                                    fa_exp2(fmaf(sacc_in[kb][e + 1], sl2, -m_use)));
      else
        pk[kb][e >> 1] = cvt_bf16x2(fa_exp2(t[kb][e] - m_use), fa_exp2(t[kb][e + 1] - m_use));
    }
  l_run = __fmul_rn(l_run, alpha);  // the caller adds this tile's fa_row_sum
  alpha_out = alpha;                // and rescales O when it is not 1
}

// O *= alpha when the softmax step moved the running max (alpha is 1 on
// every other tile, the same for the whole wave).
template <int DT>
__device__ __forceinline__ void fa_rescale(f32x16_t (&o)[DT], float alpha) {
  if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[dt][e] *= alpha;
  }
}

// Sum of a tile's packed bf16 probabilities over the lane's 32 keys
// (v_dot2_f32_bf16 against (1, 1), four independent partial sums): the
// running sum adds exactly the probabilities the PV product uses.  Added to
// l_run after the softmax step's rescale, without contraction, so that
// both kernels round the same way wherever they place the addition.
__device__ __forceinline__ float fa_row_sum(const uint32_t (&pk)[2][8]) {
  const bf16x2_t ones = {(__bf16)1.0f, (__bf16)1.0f};
  float ps[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    bf16x2_t pv;
    __builtin_memcpy(&pv, &pk[i >> 3][i & 7], 4);
    ps[i & 3] = __builtin_amdgcn_fdot2_f32_bf16(pv, ones, ps[i & 3], false);
  }
  return __fadd_rn(__fadd_rn(ps[0], ps[1]), __fadd_rn(ps[2], ps[3]));
}

// The softmax step of the tile's kind (fa_kind), then the rescale of O.
template <int DT>
__device__ __forceinline__ void fa_softmax_any(int kind, const FlashArgs& a, int k0, int qi,
                                               int g, float sl2, f32x16_t (&sacc)[2],
                                               float mr, uint32_t (&pk)[2][8], f32x16_t (&o)[DT],
                                               float& m_run, float& l_run) {
  float alpha;
  if (kind == FA_PLAIN)
    fa_softmax_tile<DT, FA_PLAIN>(a, k0, qi, g, sl2, sacc, mr, pk, m_run, l_run, alpha);
  else if (kind == FA_DIAG_UP)
    fa_softmax_tile<DT, FA_DIAG_UP>(a, k0, qi, g, sl2, sacc, mr, pk, m_run, l_run, alpha);
  else if (kind == FA_DIAG_DOWN)
    fa_softmax_tile<DT, FA_DIAG_DOWN>(a, k0, qi, g, sl2, sacc, mr, pk, m_run, l_run, alpha);
  else
    fa_softmax_tile<DT, FA_GENERAL>(a, k0, qi, g, sl2, sacc, mr, pk, m_run, l_run, alpha);
  fa_rescale<DT>(o, alpha);
}

// Workgroup barrier without the memory fence of __syncthreads (which would
// also wait for every DMA in flight); callers wait for what they need first.
// No instruction is scheduled across it: the ping-pong phases it separates
// must keep their own MFMA or VALU work.
__device__ __forceinline__ void block_barrier_fa() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
}

// BUF: every key tile is whole (Sk % 64 == 0) and every byte offset into K
// and V is below 2^31, so the tiles move by buffer loads with a scalar tile
// offset (no per-tile address arithmetic on the vector ALU).
// ROUND: scores are rounded to bf16 before the scale (a.round_scores).
template <int D, bool BUF, bool ROUND>
__global__ void __launch_bounds__(256, 2) flash_fwd_kernel(FlashArgs a) {
  using namespace fa;
  constexpr int CPR = D / 8;                       // 16-byte chunks per key row
  constexpr int NT = D / 16;                       // MFMA k-steps of Q K^T
  constexpr int DT = D / 32;                       // 32-row d tiles of O^T
  constexpr int TILE = BKV * D;                    // elements of a K or V tile
  constexpr int ROWS_PER_DMA = 64 / CPR;           // key rows per 1 KiB DMA instruction
  constexpr int DMA_PER_WAVE = (TILE / 512) / 4;   // instructions per wave per tile
  static_assert(CPR >= 4 && CPR <= 16 && DMA_PER_WAVE >= 1, "head dim 32..128");
  __shared__ __attribute__((aligned(1024))) uint16_t Ks0[TILE];
  __shared__ __attribute__((aligned(1024))) uint16_t Ks1[TILE];
  __shared__ __attribute__((aligned(1024))) uint16_t Vs0[TILE];
  __shared__ __attribute__((aligned(1024))) uint16_t Vs1[TILE];

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 31, g = lane >> 5;
  const int nqt = (a.Sq + BQ - 1) / BQ;
  const int nbh = a.B * a.H;
  const int rank = blockIdx.x / nbh;
  int bh = blockIdx.x - rank * nbh;
  // GQA: the G query heads of one KV head go to one XCD (workgroups whose
  // indices agree mod 8 share an XCD) at adjacent dispatch slots, so that
  // XCD's L2 serves the same K/V tiles to all of them.  A bijection on
  // [0, B H) when B Hkv is a multiple of 8.
  if (a.H > a.Hkv && (a.B * a.Hkv) % 8 == 0) {
    const int G = a.H / a.Hkv, x = bh % 8, j = bh / 8;
    const int gi = (j / G) * 8 + x, m = j % G;
    bh = (gi / a.Hkv) * a.H + (gi % a.Hkv) * G + m;
  }
  // the most expensive query tiles are scheduled first
  const int qt = a.heavy_last ? nqt - 1 - rank : rank;
  const int b = bh / a.H, h = bh - b * a.H;
  const int hk = h / (a.H / a.Hkv);
  const int q0 = qt * BQ;
  const int qi = q0 + wave * 32 + c;  // this lane's query
  const int q_last = min(q0 + BQ, a.Sq) - 1;

  const uint16_t* Q = (const uint16_t*)a.q + b * a.q_sb + h * a.q_sh;
  const uint16_t* K = (const uint16_t*)a.k + b * a.k_sb + hk * a.k_sh;
  const uint16_t* V = (const uint16_t*)a.v + b * a.v_sb + hk * a.v_sh;

  // key tile range
  const int nkt = (a.Sk + BKV - 1) / BKV;
  int kt0 = 0, kt1 = nkt;
  if (a.skip) {
    const int q1 = min(q0 + BQ, a.Sq);  // exclusive
    if (a.cmp == vm::CMP_LE) kt0 = q0 / BKV;
    else if (a.cmp == vm::CMP_LT) kt0 = (q0 + 1) / BKV;
    else if (a.cmp == vm::CMP_GE) kt1 = min(nkt, (q1 - 1) / BKV + 1);
    else if (a.cmp == vm::CMP_GT) kt1 = min(nkt, (q1 - 2) / BKV + 1);
  }

  // Q^T fragments stay in registers: lane (c, g) holds d = t*16 + g*8 .. +8
  bf16x8_t qf[NT];
  {
    const bool ok = qi < a.Sq;
    const uint16_t* qp = Q + (int64_t)(ok ? qi : 0) * a.q_ss;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (ok) {
        qf[t] = *(const bf16x8_t*)(qp + t * 16 + g * 8);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) qf[t][e] = (__bf16)0.0f;
      }
    }
  }

  // DMA of one key tile: instruction q of this wave covers key rows
  // ROWS_PER_DMA * (wave * DMA_PER_WAVE + q) + lane / CPR
  const int row_in = lane / CPR, pc = lane % CPR;
  uint32_t vk_off[DMA_PER_WAVE], vv_off[DMA_PER_WAVE];
  __amdgpu_buffer_rsrc_t rk, rv;
  if constexpr (BUF) {
    rk = fa_rsrc(K);
    rv = fa_rsrc(V);
#pragma unroll
    for (int q = 0; q < DMA_PER_WAVE; ++q) {
      const int r = (wave * DMA_PER_WAVE + q) * ROWS_PER_DMA + row_in;
      vk_off[q] = (uint32_t)((r * a.k_ss + (pc ^ (r % CPR)) * 8) * 2);
      vv_off[q] = (uint32_t)((r * a.v_ss + (pc ^ ((4 * (r & 3)) % CPR)) * 8) * 2);
    }
  }
  auto dma_tile = [&](uint16_t* ks, uint16_t* vs, int kt) {
    const int k0 = kt * BKV;
    if constexpr (BUF) {
      const uint32_t sk = (uint32_t)(k0 * a.k_ss * 2), sv = (uint32_t)(k0 * a.v_ss * 2);
#pragma unroll
      for (int q = 0; q < DMA_PER_WAVE; ++q) {
        const int blk = wave * DMA_PER_WAVE + q;
        dma16_buf(rk, vk_off[q], sk, ks + blk * 512);
        dma16_buf(rv, vv_off[q], sv, vs + blk * 512);
      }
      return;
    }
#pragma unroll
    for (int q = 0; q < DMA_PER_WAVE; ++q) {
      const int blk = wave * DMA_PER_WAVE + q;
      const int r = blk * ROWS_PER_DMA + row_in;
      int key = k0 + r;
      key = key < a.Sk ? key : a.Sk - 1;  // rows past Sk: an in-range row (masked below)
      const int ck = pc ^ (r % CPR);
      const int cv = pc ^ ((4 * (r & 3)) % CPR);
      dma16(K + (int64_t)key * a.k_ss + ck * 8, ks + blk * 512);
      dma16(V + (int64_t)key * a.v_ss + cv * 8, vs + blk * 512);
    }
  };

  // K fragment offsets (elements): key row kb*32 + c, d-chunk 2t + g; the
  // swizzle depends on the row only through c % CPR, so block kb = 1 is
  // block 0 plus 32 rows (an immediate offset)
  int k_off[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) k_off[t] = c * D + (((2 * t + g) ^ (c % CPR)) * 8);
  // V fragment offsets: 16-lane group G, source lane s: key row
  // 4 (G >> 1) + s / 4 (+ 8 for the second read), d column
  // dt*32 + 16 (G & 1) + 4 (s % 4)
  const int G = lane >> 4, s16 = lane & 15;
  int v_off[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    const int r = 4 * (G >> 1) + (s16 >> 2);
    const int col = dt * 32 + 16 * (G & 1) + 4 * (s16 & 3);
    v_off[dt] = r * D + (((col >> 3) ^ ((4 * (r & 3)) % CPR)) * 8) + (col & 7);
  }

  f32x16_t o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[dt][e] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;
  const float sl2 = a.scale * kLog2e;
  const FaKinds kinds = fa_kinds(a, q0, q_last);

  auto k_tile = [&](const uint16_t* ks, const uint16_t* vs, uint16_t* ks_n, uint16_t* vs_n,
                    int kt) {
    const bool more = kt + 1 < kt1;
    // branch-free: on the last tile a spare reload of tile kt0 into the idle stage
    dma_tile(ks_n, vs_n, more ? kt + 1 : kt0);

    // S^T tile: 64 keys x 32 queries as two 32x32 accumulators.  The K
    // fragments of k-step t + 2 are read while the MFMAs of step t run (a
    // three-slot ring), and the schedule below keeps that order.
    f32x16_t sacc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; ++e) sacc[kb][e] = 0.0f;
    bf16x8_t kf[3][2];
    auto ld_k = [&](int t) {
      kf[t % 3][0] = *(const bf16x8_t*)(ks + k_off[t]);
      kf[t % 3][1] = *(const bf16x8_t*)(ks + k_off[t] + 32 * D);
    };
    ld_k(0);
    ld_k(1);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (t + 2 < NT) ld_k(t + 2);
      sacc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[t % 3][0], qf[t], sacc[0], 0, 0, 0);
      sacc[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[t % 3][1], qf[t], sacc[1], 0, 0, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // ds reads of steps 0, 1
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (t + 2 < NT) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // step t + 2
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);                  // step t
    }

    // V^T fragments of the first PV k-step, read while the softmax runs
    auto load_v = [&](int u, bf16x8_t* dst) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const uint16_t* p = vs + v_off[dt] + u * 16 * D;
        union {
          v4s h[2];
          bf16x8_t v;
        } vf;
        vf.h[0] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)p);
        vf.h[1] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(p + 8 * D));
        dst[dt] = vf.v;
      }
    };
    bf16x8_t vbuf[2][DT];
    load_v(0, vbuf[0]);

    const int k0 = kt * BKV;
    uint32_t pk[2][8];  // bf16 probability pairs: [kb][e/2]
    const float mr = fa_round_max<ROUND>(sacc);
    fa_softmax_any<DT>(fa_kind(kinds, kt), a, k0, qi, g, sl2, sacc, mr, pk, o, m_run, l_run);
    l_run = __fadd_rn(l_run, fa_row_sum(pk));

    // O^T += V^T P^T over 4 k-steps of 16 keys
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int kb = u >> 1, half = u & 1;
      union {
        uint32_t w[4];
        bf16x8_t v;
      } pf;
#pragma unroll
      for (int i = 0; i < 4; ++i) pf.w[i] = pk[kb][half * 4 + i];
      if (u + 1 < 4) load_v(u + 1, vbuf[(u + 1) & 1]);  // next k-step's fragments
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vbuf[u & 1][dt], pf.v, o[dt], 0, 0, 0);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  };

  if (kt0 < kt1) {
    dma_tile(Ks0, Vs0, kt0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    for (int kt = kt0; kt < kt1; kt += 2) {
      k_tile(Ks0, Vs0, Ks1, Vs1, kt);
      if (kt + 1 < kt1) k_tile(Ks1, Vs1, Ks0, Vs0, kt + 1);
    }
  }

  // normalise and store: lane (c, g) holds O[qi][dt*32 + (e>>2)*8 + g*4 + (e&3)]
  const auto lsw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run), __float_as_uint(l_run),
                                                     false, false);
  const float l_tot = __uint_as_float(lsw[0]) + __uint_as_float(lsw[1]);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  if (qi < a.Sq) {
    uint16_t* O = (uint16_t*)a.o + b * a.o_sb + h * a.o_sh + (int64_t)qi * a.o_ss;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d0 = dt * 32 + r * 8 + g * 4;
        *(uint2*)(O + d0) = make_uint2(cvt_bf16x2(o[dt][r * 4 + 0] * inv, o[dt][r * 4 + 1] * inv),
                                       cvt_bf16x2(o[dt][r * 4 + 2] * inv, o[dt][r * 4 + 3] * inv));
      }
  }
}


// Ping-pong schedule.  Eight waves in two groups of four (group r: waves
// 4r .. 4r + 3; waves w and w + 4 share a SIMD), each group 128 queries and
// both groups over the same key tiles: two query heads of one KV head
// (GQA with an even group size) or, otherwise, two adjacent query tiles of
// one head over the union of their key ranges (the extra tiles of the
// shorter one are computed, not skipped: masked keys add exact zeros).
//
// Time runs in half-steps separated by workgroup barriers.  In each
// half-step one group is in an MFMA phase -- S^T = K Q^T of key tile m and
// O^T += V^T P^T of tile m - 1 -- while the other group is in a softmax
// phase (VALU), and the two swap at every barrier, so each SIMD's matrix
// core is fed by one wave while the other wave's exp / rounding / max work
// issues beside it (the VALU wave slows by about a fifth, the MFMA wave not
// at all).  A single wave that alternates the two serialises them, and two
// independent workgroups per CU overlap them only by chance.
//
//   half-step   0        1        2        3      ...  2n        2n + 1
//   group 0     MFMA 0   soft 0   MFMA 1   soft 1      MFMA n    (store)
//   group 1     -        MFMA 0   soft 0   MFMA 1      soft n-1  MFMA n
//
// MFMA phase m reads stage m = {K tile m, V tile m - 1} from LDS slot
// m % 2; stage m + 1 is requested by DMA at the start of half-step 2m
// (each wave moves its share) into the slot stage m - 1 left free, and
// waited for at the end of half-step 2m + 1.
template <int D, bool ROUND>
__global__ void __launch_bounds__(512, 1) flash_pp_kernel(FlashArgs a) {
  using namespace fa;
  constexpr int CPR = D / 8;                      // 16-byte chunks per key row
  constexpr int NT = D / 16;                      // MFMA k-steps of Q K^T
  constexpr int DT = D / 32;                      // 32-row d tiles of O^T
  constexpr int TILE = BKV * D;                   // elements of a K or V tile
  constexpr int ROWS_PER_DMA = 64 / CPR;          // key rows per 1 KiB DMA instruction
  constexpr int DMA_PER_WAVE = (TILE / 512) / 8;  // instructions per wave per K (or V) tile
  static_assert(DMA_PER_WAVE >= 1 && CPR <= 16, "head dim 64 or 128");
  __shared__ __attribute__((aligned(1024))) uint16_t Ks[2 * TILE];
  __shared__ __attribute__((aligned(1024))) uint16_t Vs[2 * TILE];

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2, wq = wave & 3;
  const int c = lane & 31, g = lane >> 5;
  const int nqt = (a.Sq + BQ - 1) / BQ;
  const int G = a.H / a.Hkv;
  const bool pair = (G & 1) == 0;
  int b, h, qa;  // qa: first query of group 0
  if (pair) {
    // units (b, kv head, head pair); the pairs of one KV head go to one XCD
    // (workgroups whose indices agree mod 8 share an XCD) at adjacent
    // dispatch slots, a bijection when B Hkv is a multiple of 8
    const int P = G / 2, units = a.B * a.Hkv * P;
    const int rank = blockIdx.x / units;
    int u = blockIdx.x - rank * units;
    if ((a.B * a.Hkv) % 8 == 0) {
      const int x = u % 8, j = u / 8;
      u = ((j / P) * 8 + x) * P + j % P;
    }
    const int gi = u / P, pm = u - gi * P;
    b = gi / a.Hkv;
    h = (gi - b * a.Hkv) * G + 2 * pm + grp;
    qa = (a.heavy_last ? nqt - 1 - rank : rank) * BQ;
  } else {
    const int nqp = (nqt + 1) / 2, nbh = a.B * a.H;
    const int rank = blockIdx.x / nbh;
    const int bh = blockIdx.x - rank * nbh;
    b = bh / a.H;
    h = bh - b * a.H;
    qa = 2 * (a.heavy_last ? nqp - 1 - rank : rank) * BQ;
  }
  const int hk = h / G;
  const int q0 = pair ? qa : qa + grp * BQ;  // this group's first query (>= Sq: an idle group)
  const int qi = q0 + wq * 32 + c;           // this lane's query
  const int q_last = min(q0 + BQ, a.Sq) - 1;

  const uint16_t* Q = (const uint16_t*)a.q + b * a.q_sb + h * a.q_sh;
  const uint16_t* K = (const uint16_t*)a.k + b * a.k_sb + hk * a.k_sh;
  const uint16_t* V = (const uint16_t*)a.v + b * a.v_sb + hk * a.v_sh;

  // key tiles [kt0, kt0 + n): the union of both groups' ranges
  const int nkt = a.Sk / BKV;
  auto range = [&](int qs, int* lo, int* hi) {
    *lo = 0;
    *hi = nkt;
    if (a.skip) {
      const int q1 = min(qs + BQ, a.Sq);  // exclusive
      if (a.cmp == vm::CMP_LE) *lo = qs / BKV;
      else if (a.cmp == vm::CMP_LT) *lo = (qs + 1) / BKV;
      else if (a.cmp == vm::CMP_GE) *hi = min(nkt, (q1 - 1) / BKV + 1);
      else if (a.cmp == vm::CMP_GT) *hi = min(nkt, (q1 - 2) / BKV + 1);
    }
  };
  int kt0, kt1;
  range(qa, &kt0, &kt1);
  if (!pair && qa + BQ < a.Sq) {
    int lo, hi;
    range(qa + BQ, &lo, &hi);
    kt0 = min(kt0, lo);
    kt1 = max(kt1, hi);
  }
  const int n = max(kt1 - kt0, 0);

  // Q^T fragments stay in registers: lane (c, g) holds d = t*16 + g*8 .. +8
  bf16x8_t qf[NT];
  {
    const bool ok = qi < a.Sq;
    const uint16_t* qp = Q + (int64_t)(ok ? qi : 0) * a.q_ss;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (ok) {
        qf[t] = *(const bf16x8_t*)(qp + t * 16 + g * 8);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) qf[t][e] = (__bf16)0.0f;
      }
    }
  }

  // DMA of one stage: instruction q of this wave covers key rows
  // ROWS_PER_DMA * (wave * DMA_PER_WAVE + q) + lane / CPR of the K tile and
  // of the V tile, with the swizzles of the single-group kernel
  const int row_in = lane / CPR, pc = lane % CPR;
  const __amdgpu_buffer_rsrc_t rk = fa_rsrc(K), rv = fa_rsrc(V);
  uint32_t vk_off[DMA_PER_WAVE], vv_off[DMA_PER_WAVE];
#pragma unroll
  for (int q = 0; q < DMA_PER_WAVE; ++q) {
    const int r = (wave * DMA_PER_WAVE + q) * ROWS_PER_DMA + row_in;
    vk_off[q] = (uint32_t)((r * a.k_ss + (pc ^ (r % CPR)) * 8) * 2);
    vv_off[q] = (uint32_t)((r * a.v_ss + (pc ^ ((4 * (r & 3)) % CPR)) * 8) * 2);
  }
  // stage s: K tile kt0 + s (s < n) and V tile kt0 + s - 1 (s > 0); the
  // missing halves of stages 0 and n reload an in-range tile nobody reads
  auto dma_stage = [&](int s) {
    const int kk = kt0 + min(s, n - 1), vt = kt0 + max(s - 1, 0);
    const uint32_t sk = (uint32_t)(kk * BKV * a.k_ss * 2), sv = (uint32_t)(vt * BKV * a.v_ss * 2);
    uint16_t* ks = Ks + (s & 1) * TILE;
    uint16_t* vs = Vs + (s & 1) * TILE;
#pragma unroll
    for (int q = 0; q < DMA_PER_WAVE; ++q) {
      const int blk = wave * DMA_PER_WAVE + q;
      dma16_buf(rk, vk_off[q], sk, ks + blk * 512);
      dma16_buf(rv, vv_off[q], sv, vs + blk * 512);
    }
  };

  // K fragment offsets (elements): key row kb*32 + c, d-chunk 2t + g; the
  // swizzle depends on the row only through c % CPR, so block kb = 1 is
  // block 0 plus 32 rows (an immediate offset)
  int k_off[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) k_off[t] = c * D + (((2 * t + g) ^ (c % CPR)) * 8);
  // V fragment offsets (ds_read_b64_tr_b16, as in the single-group kernel)
  const int G16 = lane >> 4, s16 = lane & 15;
  int v_off[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    const int r = 4 * (G16 >> 1) + (s16 >> 2);
    const int col = dt * 32 + 16 * (G16 & 1) + 4 * (s16 & 3);
    v_off[dt] = r * D + (((col >> 3) ^ ((4 * (r & 3)) % CPR)) * 8) + (col & 7);
  }

  f32x16_t o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[dt][e] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;
  const float sl2 = a.scale * kLog2e;
  const FaKinds kinds = fa_kinds(a, q0, q_last);
  f32x16_t sacc[2];
  uint32_t pk[2][8];  // bf16 probability pairs of the last softmax phase: [kb][e/2]

  auto qk = [&](const uint16_t* ks) {
    // S^T tile: 64 keys x 32 queries as two 32x32 accumulators; the K
    // fragments of k-step t + 2 are read while the MFMAs of step t run
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; ++e) sacc[kb][e] = 0.0f;
    bf16x8_t kf[3][2];
    auto ld_k = [&](int t) {
      kf[t % 3][0] = *(const bf16x8_t*)(ks + k_off[t]);
      kf[t % 3][1] = *(const bf16x8_t*)(ks + k_off[t] + 32 * D);
    };
    ld_k(0);
    ld_k(1);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (t + 2 < NT) ld_k(t + 2);
      sacc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[t % 3][0], qf[t], sacc[0], 0, 0, 0);
      sacc[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[t % 3][1], qf[t], sacc[1], 0, 0, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // ds reads of steps 0, 1
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (t + 2 < NT) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // step t + 2
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);                  // step t
    }
  };
  auto pv = [&](const uint16_t* vs) {
    // O^T += V^T P^T over 4 k-steps of 16 keys; the V^T fragments of step
    // u + 1 are read while the MFMAs of step u run
    auto load_v = [&](int u, bf16x8_t* dst) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const uint16_t* p = vs + v_off[dt] + u * 16 * D;
        union {
          v4s h[2];
          bf16x8_t v;
        } vf;
        vf.h[0] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)p);
        vf.h[1] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(p + 8 * D));
        dst[dt] = vf.v;
      }
    };
    bf16x8_t vbuf[2][DT];
    load_v(0, vbuf[0]);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int kb = u >> 1, half = u & 1;
      union {
        uint32_t w[4];
        bf16x8_t v;
      } pf;
#pragma unroll
      for (int i = 0; i < 4; ++i) pf.w[i] = pk[kb][half * 4 + i];
      if (u + 1 < 4) load_v(u + 1, vbuf[(u + 1) & 1]);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vbuf[u & 1][dt], pf.v, o[dt], 0, 0, 0);
    }
  };
  // LDS slot of stage m
  auto kslot = [&](int m) -> const uint16_t* { return Ks + (m & 1) * TILE; };
  auto vslot = [&](int m) -> const uint16_t* { return Vs + (m & 1) * TILE; };
  float mr = -INFINITY;  // max of the rounded scores of the last S tile
  auto soft_phase = [&](int m) {
    const int k0 = (kt0 + m) * BKV;
    fa_softmax_any<DT>(fa_kind(kinds, kt0 + m), a, k0, qi, g, sl2, sacc, mr, pk, o, m_run, l_run);
  };
  // the MFMA phase's share of the softmax: the scores' rounding and max,
  // and the row sum of the last probabilities (in the softmax phase instead
  // the kernel measured the same: 176-177 us on the Llama layer either way)
  auto mfma_side = [&](bool round, bool sum) {
    if (round) mr = fa_round_max<ROUND>(sacc);
    if (sum) l_run = __fadd_rn(l_run, fa_row_sum(pk));
  };
  auto vm_wait = []() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); };

  // MFMA phase m (half-step 2m for group 0, 2m + 1 for group 1) computes S
  // of tile m (m < n) and O += V P of tile m - 1 (m > 0) from stage m in
  // slot m % 2; softmax phase m follows it.  Every wave requests its share of
  // stage s during half-step 2s - 2, after its own fragment reads there
  // (group 0: at the end of MFMA phase s - 1; group 1: at the start of
  // softmax phase s - 2), and waits for it at the end of its next softmax
  // phase.  A wave thus never reads LDS while a DMA of its own is in flight:
  // the slot is a run-time value, so the compiler would otherwise wait for
  // the DMA before every fragment read.  The first and last MFMA phases are
  // peeled, so the loop body has one form and O stays in place across it.
  // The MFMA phase runs at the higher wave priority: when both waves of a
  // SIMD can issue, the matrix core is fed first (otherwise the older group
  // wins whatever its phase).  Both groups pass 2n + 1 barriers after the
  // first.
  if (n > 0) {
    dma_stage(0);
    vm_wait();
    block_barrier_fa();
    if (grp == 0) {
      __builtin_amdgcn_s_setprio(1);
      qk(kslot(0));
      mfma_side(true, false);
      dma_stage(1);
      block_barrier_fa();  // half-step 0
      for (int m = 1; m < n; ++m) {
        __builtin_amdgcn_s_setprio(0);
        soft_phase(m - 1);
        vm_wait();
        block_barrier_fa();  // 2m - 1
        __builtin_amdgcn_s_setprio(1);
        qk(kslot(m));
        pv(vslot(m));
        mfma_side(true, true);
        dma_stage(m + 1);
        block_barrier_fa();  // 2m
      }
      __builtin_amdgcn_s_setprio(0);
      soft_phase(n - 1);
      vm_wait();
      block_barrier_fa();  // 2n - 1
      __builtin_amdgcn_s_setprio(1);
      pv(vslot(n));
      mfma_side(false, true);
      block_barrier_fa();  // 2n
    } else {
      dma_stage(1);
      vm_wait();
      block_barrier_fa();  // half-step 0
      __builtin_amdgcn_s_setprio(1);
      qk(kslot(0));
      mfma_side(true, false);
      block_barrier_fa();  // 1
      for (int m = 1; m < n; ++m) {
        __builtin_amdgcn_s_setprio(0);
        dma_stage(m + 1);
        soft_phase(m - 1);
        vm_wait();
        block_barrier_fa();  // 2m
        __builtin_amdgcn_s_setprio(1);
        qk(kslot(m));
        pv(vslot(m));
        mfma_side(true, true);
        block_barrier_fa();  // 2m + 1
      }
      __builtin_amdgcn_s_setprio(0);
      soft_phase(n - 1);
      block_barrier_fa();  // 2n
      __builtin_amdgcn_s_setprio(1);
      pv(vslot(n));
      mfma_side(false, true);
    }
  }

  // normalise and store: lane (c, g) holds O[qi][dt*32 + (e>>2)*8 + g*4 + (e&3)]
  const auto lsw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run), __float_as_uint(l_run),
                                                     false, false);
  const float l_tot = __uint_as_float(lsw[0]) + __uint_as_float(lsw[1]);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  if (qi < a.Sq) {
    uint16_t* O = (uint16_t*)a.o + b * a.o_sb + h * a.o_sh + (int64_t)qi * a.o_ss;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d0 = dt * 32 + r * 8 + g * 4;
        *(uint2*)(O + d0) = make_uint2(cvt_bf16x2(o[dt][r * 4 + 0] * inv, o[dt][r * 4 + 1] * inv),
                                       cvt_bf16x2(o[dt][r * 4 + 2] * inv, o[dt][r * 4 + 3] * inv));
      }
  }
}


bool flash_supported(const FlashArgs& a) {
  if (a.D != 32 && a.D != 64 && a.D != 128) return false;
  if (a.B <= 0 || a.H <= 0 || a.Hkv <= 0 || a.H % a.Hkv) return false;
  if (a.Sq <= 0 || a.Sk <= 0) return false;
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  if (!al16(a.q) || !al16(a.k) || !al16(a.v) || !al16(a.o)) return false;
  for (int64_t s : {a.q_sb, a.q_sh, a.q_ss, a.k_sb, a.k_sh, a.k_ss, a.v_sb, a.v_sh, a.v_ss,
                    a.o_sb, a.o_sh, a.o_ss})
    if (s % 8 != 0) return false;
  const int64_t blocks = (int64_t)((a.Sq + fa::BQ - 1) / fa::BQ) * a.B * a.H;
  return blocks < (1ll << 31);
}

template <int D, bool BUF>
static void launch_flash_db(const FlashArgs& a, unsigned grid, hipStream_t stream) {
  if (a.round_scores)
    hipLaunchKernelGGL((flash_fwd_kernel<D, BUF, true>), dim3(grid), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((flash_fwd_kernel<D, BUF, false>), dim3(grid), dim3(256), 0, stream, a);
}
template <int D>
static void launch_flash_d(const FlashArgs& a, bool buf, unsigned grid, hipStream_t stream) {
  if (buf) launch_flash_db<D, true>(a, grid, stream);
  else launch_flash_db<D, false>(a, grid, stream);
}

// Kernel choice for head dims 64 and 128 when every key tile is whole and
// every K / V byte offset fits the buffer descriptors' 31 bits; other
// shapes run the single-group kernel.  REW_MI355X_FLASH = single or pp
// forces one (tests compare them).
enum { FA_K_SINGLE = 0, FA_K_PP = 1 };
static int flash_forced() {
  static const int v = [] {
    const char* s = std::getenv("REW_MI355X_FLASH");
    if (!s) return -1;
    const std::string t(s);
    return t == "single" ? FA_K_SINGLE : t == "pp" ? FA_K_PP : -1;
  }();
  return v;
}

static bool flash_buf_ok(const FlashArgs& a) {
  return a.Sk % fa::BKV == 0 && ((int64_t)a.Sk * a.k_ss + a.D) * 2 < (1ll << 31) &&
         ((int64_t)a.Sk * a.v_ss + a.D) * 2 < (1ll << 31);
}

static int flash_kernel_kind(const FlashArgs& a) {
  if (!((a.D == 64 || a.D == 128) && flash_buf_ok(a))) return FA_K_SINGLE;
  const int f = flash_forced();
  return f >= 0 ? f : FA_K_PP;
}

const char* flash_variant(const FlashArgs& a) {
  switch (flash_kernel_kind(a)) {
    case FA_K_PP: return "flash_attn_pp";
    default: return "flash_attn";
  }
}

void launch_flash(const FlashArgs& a, hipStream_t stream) {
  const int nqt = (a.Sq + fa::BQ - 1) / fa::BQ;
  const int kind = flash_kernel_kind(a);
  if (kind == FA_K_PP) {
    const bool pair = ((a.H / a.Hkv) & 1) == 0;
    const unsigned grid =
        pair ? (unsigned)(nqt * a.B * (a.H / 2)) : (unsigned)(((nqt + 1) / 2) * a.B * a.H);
    auto go = [&](auto kern) {
      hipLaunchKernelGGL(kern, dim3(grid), dim3(512), 0, stream, a);
    };
    if (a.D == 64) {
      if (a.round_scores) go(flash_pp_kernel<64, true>);
      else go(flash_pp_kernel<64, false>);
    } else {
      if (a.round_scores) go(flash_pp_kernel<128, true>);
      else go(flash_pp_kernel<128, false>);
    }
    REW_HIP(hipGetLastError());
    return;
  }
  const unsigned grid = (unsigned)(nqt * a.B * a.H);
  const bool buf = flash_buf_ok(a);
  switch (a.D) {
    case 32: launch_flash_d<32>(a, buf, grid, stream); break;
    case 64: launch_flash_d<64>(a, buf, grid, stream); break;
    default: launch_flash_d<128>(a, buf, grid, stream); break;
  }
  REW_HIP(hipGetLastError());
}

}  // namespace rew
