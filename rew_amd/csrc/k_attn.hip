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

template <int V>
struct FaK {
  static constexpr int value = V;
};

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

  // K fragment offsets (elements): key row kb*32 + c, d-chunk 2t + g
  int k_off[2][NT];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int r = kb * 32 + c;
      k_off[kb][t] = r * D + (((2 * t + g) ^ (r % CPR)) * 8);
    }
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
  const bool fold = a.scale > 0.0f;
  const float sl2 = a.scale * kLog2e;

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
      kf[t % 3][0] = *(const bf16x8_t*)(ks + k_off[0][t]);
      kf[t % 3][1] = *(const bf16x8_t*)(ks + k_off[1][t]);
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

    // Scores in log2 units, t = log2(e) * (bf16(x) * scale + mask), and the
    // tile max of t.  Three tile kinds, each straight-line code:
    //   plain     every key in range and visible, scale > 0: t is formed
    //             inside the exp's FMA and the max comes from the raw
    //             accumulators (rounding and scaling are monotone);
    //   diagonal  a whole tile under an ordered mask that adds 0 where
    //             visible, scale > 0: t = fma(x, scale log2 e, visible ? 0 :
    //             mask_false log2 e), visibility from one per-lane threshold;
    //   general   anything else: t = (x * scale + mask) log2 e, -inf past Sk.
    const int k0 = kt * BKV;
    const bool whole = k0 + BKV <= a.Sk;
    int kind = 2;
    if (fold && whole) {
      if (!a.mask || (a.mask_true == 0.0f && fa_all_visible(a.cmp, q0, q_last, k0, k0 + BKV - 1)))
        kind = 0;
      else if (a.mask_true == 0.0f && a.cmp >= vm::CMP_LT)
        kind = 1;
    }
    auto round_in_place = [&]() {
      if constexpr (ROUND) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int e = 0; e < 16; e += 2) {
            const uint32_t pr = cvt_bf16x2(sacc[kb][e], sacc[kb][e + 1]);
            sacc[kb][e] = vm::as_f(pr << 16);
            sacc[kb][e + 1] = vm::as_f(pr & 0xffff0000u);
          }
      }
    };
    float mt;
    if (kind == 0) {
      float m0 = -INFINITY, m1 = -INFINITY;
#pragma unroll
      for (int e = 0; e < 16; e += 2) {
        m0 = fa_max3(m0, sacc[0][e], sacc[0][e + 1]);
        m1 = fa_max3(m1, sacc[1][e], sacc[1][e + 1]);
      }
      float mr = fa_max3(m0, m1, -INFINITY);
      round_in_place();
      if constexpr (ROUND) mr = vm::as_f(cvt_bf16x2(mr, mr) << 16);
      mt = mr * sl2;
    } else if (kind == 1) {
      round_in_place();
      // key j = k0 + off (off = kb 32 + (e / 4) 8 + g 4 + e % 4) is visible
      // iff j - qi >= lo (LE, LT) or j - qi <= -lo (GE, GT)
      const float mf2 = a.mask_false * kLog2e;
      const bool up = a.cmp == vm::CMP_LE || a.cmp == vm::CMP_LT;
      const int lo = (a.cmp == vm::CMP_LT || a.cmp == vm::CMP_GT) ? 1 : 0;
      const int base = k0 - qi + g * 4;
      float m0 = -INFINITY, m1 = -INFINITY;
      auto diag = [&](auto UP) {
        constexpr bool kUp = decltype(UP)::value;
        const int thr = kUp ? lo - base : -lo - base;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int e = 0; e < 16; e += 2) {
            const int off = kb * 32 + (e >> 2) * 8 + (e & 3);
            const bool v0 = kUp ? off >= thr : off <= thr;
            const bool v1 = kUp ? off + 1 >= thr : off + 1 <= thr;
            const float t0 = fmaf(sacc[kb][e], sl2, v0 ? 0.0f : mf2);
            const float t1 = fmaf(sacc[kb][e + 1], sl2, v1 ? 0.0f : mf2);
            sacc[kb][e] = t0;
            sacc[kb][e + 1] = t1;
            if (kb == 0) m0 = fa_max3(m0, t0, t1);
            else m1 = fa_max3(m1, t0, t1);
          }
      };
      if (up) diag(FaK<1>{});
      else diag(FaK<0>{});
      mt = fa_max3(m0, m1, -INFINITY);
    } else {
      round_in_place();
      float m0 = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 16; e += 2) {
          const int j0 = k0 + kb * 32 + (e >> 2) * 8 + g * 4 + (e & 3);
          float x0 = sacc[kb][e] * a.scale, x1 = sacc[kb][e + 1] * a.scale;
          if (a.mask) {
            x0 += fa_visible(a.cmp, qi, j0) ? a.mask_true : a.mask_false;
            x1 += fa_visible(a.cmp, qi, j0 + 1) ? a.mask_true : a.mask_false;
          }
          x0 = j0 < a.Sk ? x0 * kLog2e : -INFINITY;
          x1 = j0 + 1 < a.Sk ? x1 * kLog2e : -INFINITY;
          sacc[kb][e] = x0;
          sacc[kb][e + 1] = x1;
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
    // the same either way up to rounding.
    const float m_new = fmaxf(m_run, mt);
    const bool grow = !(m_new - m_run <= kLazy * kLog2e);  // (also when m_run is still -inf)
    const bool rescale = __builtin_amdgcn_ballot_w64(grow) != 0;
    float m_use, alpha = 1.0f;
    if (rescale) {
      m_use = m_new == -INFINITY ? 0.0f : m_new;
      alpha = fa_exp2(m_run - m_use);
      m_run = m_new;
    } else {
      m_use = m_run;
    }
    float psum = 0.0f;
    uint32_t pk[2][8];  // bf16 pairs: [kb][e/2]
    if (kind == 0) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 16; e += 2) {
          const float p0 = fa_exp2(fmaf(sacc[kb][e], sl2, -m_use));
          const float p1 = fa_exp2(fmaf(sacc[kb][e + 1], sl2, -m_use));
          psum += p0 + p1;
          pk[kb][e >> 1] = cvt_bf16x2(p0, p1);
        }
    } else {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 16; e += 2) {
          const float p0 = fa_exp2(sacc[kb][e] - m_use);
          const float p1 = fa_exp2(sacc[kb][e + 1] - m_use);
          psum += p0 + p1;
          pk[kb][e >> 1] = cvt_bf16x2(p0, p1);
        }
    }
    l_run = l_run * alpha + psum;
    if (rescale) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[dt][e] *= alpha;
    }

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

void launch_flash(const FlashArgs& a, hipStream_t stream) {
  const int nqt = (a.Sq + fa::BQ - 1) / fa::BQ;
  const unsigned grid = (unsigned)(nqt * a.B * a.H);
  const bool buf = a.Sk % fa::BKV == 0 &&
                   ((int64_t)a.Sk * a.k_ss + a.D) * 2 < (1ll << 31) &&
                   ((int64_t)a.Sk * a.v_ss + a.D) * 2 < (1ll << 31);
  switch (a.D) {
    case 32: launch_flash_d<32>(a, buf, grid, stream); break;
    case 64: launch_flash_d<64>(a, buf, grid, stream); break;
    default: launch_flash_d<128>(a, buf, grid, stream); break;
  }
  REW_HIP(hipGetLastError());
}

}  // namespace rew
