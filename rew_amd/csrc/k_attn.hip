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
// queries.  Key tiles of 64 are staged in LDS (double-buffered through
// registers).  The wave computes S^T = K Q^T with v_mfma_f32_32x32x16_bf16,
// so every lane holds the scores of ONE query column: the row max / sum of
// the online softmax are lane-local plus one exchange with lane ^ 32.  The
// output is accumulated transposed, O^T = V^T P^T: the probabilities go
// straight from the S^T accumulators into the B operand, and V is written
// into LDS transposed with the key order permuted to match the accumulator
// row order (bits 2 and 3 of the key index swapped inside each 16-key
// group), so every operand fragment is one 16-byte LDS read.
//
// Numerics: fp32 accumulation; scores rounded to bf16 (the dot_general
// result dtype) before the fp32 scale / mask; probabilities rounded to bf16
// before the PV product (the astype before the second dot_general); the
// output rounded to bf16 once.  The softmax normalisation is applied at the
// end (online softmax), which differs from the two-pass op sequence only in
// rounding.
#include "kernels.h"
#include "vm_device.h"

namespace rew {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

namespace fa {
constexpr int BQ = 128;  // queries per workgroup
constexpr int BKV = 64;  // keys per tile
constexpr float kLog2e = 1.4426950408889634f;
}  // namespace fa

__device__ __forceinline__ bool fa_visible(int cmp, int i, int j) {
  switch (cmp) {
    case vm::CMP_EQ: return i == j;
    case vm::CMP_NE: return i != j;
    case vm::CMP_LT: return i < j;
    case vm::CMP_LE: return i <= j;
    case vm::CMP_GT: return i > j;
    default: return i >= j;
  }
}

// Row-order position of key w (0..15) inside a 16-key group of the V^T tile.
__device__ __forceinline__ int fa_perm16(int w) {
  return (w & 3) | (((w >> 2) & 1) << 3) | (((w >> 3) & 1) << 2);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return (uint32_t)vm::bf16_bits(a) | ((uint32_t)vm::bf16_bits(b) << 16);
}

template <int D>
__global__ void __launch_bounds__(256, 2) flash_fwd_kernel(FlashArgs a) {
  using namespace fa;
  constexpr int KP = D + 8;     // K tile row pitch (elements)
  constexpr int VP = BKV + 8;   // V^T tile row pitch (elements)
  constexpr int NT = D / 16;    // MFMA k-steps of Q K^T
  constexpr int DT = D / 32;    // 32-row d tiles of O^T
  constexpr int KCH = BKV * D / 8;          // 16-byte chunks of a K tile
  constexpr int KPT = (KCH + 255) / 256;    // per thread
  constexpr int VG = (D / 8) * (BKV / 4);   // 4-key x 8-d groups of a V tile
  constexpr int VPT = (VG + 255) / 256;     // per thread
  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][BKV * KP];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[2][D * VP];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 31, g = lane >> 5;
  const int nqt = (a.Sq + BQ - 1) / BQ;
  const int nbh = a.B * a.H;
  const int rank = blockIdx.x / nbh;
  const int bh = blockIdx.x - rank * nbh;
  // the most expensive query tiles are scheduled first
  const int qt = a.heavy_last ? nqt - 1 - rank : rank;
  const int b = bh / a.H, h = bh - b * a.H;
  const int hk = h / (a.H / a.Hkv);
  const int q0 = qt * BQ;
  const int qi = q0 + wave * 32 + c;  // this lane's query

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

  uint4 kst[KPT], vst[VPT][4];
  auto load_tile = [&](int kt) {
    const int k0 = kt * BKV;
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int cid = threadIdx.x + i * 256;
      const int row = cid / (D / 8), col = cid - row * (D / 8);
      const int key = k0 + row;
      if (cid < KCH && key < a.Sk)
        kst[i] = *(const uint4*)(K + (int64_t)key * a.k_ss + col * 8);
      else
        kst[i] = make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int gid = threadIdx.x + i * 256;
      const int dc = gid % (D / 8), kg = gid / (D / 8);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = k0 + kg * 4 + r;
        if (gid < VG && key < a.Sk)
          vst[i][r] = *(const uint4*)(V + (int64_t)key * a.v_ss + dc * 8);
        else
          vst[i][r] = make_uint4(0, 0, 0, 0);
      }
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int cid = threadIdx.x + i * 256;
      const int row = cid / (D / 8), col = cid - row * (D / 8);
      if (cid < KCH) *(uint4*)(&Ks[buf][row * KP + col * 8]) = kst[i];
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int gid = threadIdx.x + i * 256;
      if (gid >= VG) continue;
      const int dc = gid % (D / 8), kg = gid / (D / 8);
      const int kk = kg * 4;
      const int pos = (kk & ~15) + fa_perm16(kk & 15);
#pragma unroll
      for (int dd = 0; dd < 8; ++dd) {
        const int w = dd >> 1, sh = (dd & 1) * 16;
        const uint32_t e0 = ((&vst[i][0].x)[w] >> sh) & 0xffffu;
        const uint32_t e1 = ((&vst[i][1].x)[w] >> sh) & 0xffffu;
        const uint32_t e2 = ((&vst[i][2].x)[w] >> sh) & 0xffffu;
        const uint32_t e3 = ((&vst[i][3].x)[w] >> sh) & 0xffffu;
        *(uint2*)(&Vt[buf][(dc * 8 + dd) * VP + pos]) =
            make_uint2(e0 | (e1 << 16), e2 | (e3 << 16));
      }
    }
  };

  f32x16_t o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[dt][e] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;

  if (kt0 < kt1) {
    load_tile(kt0);
    store_tile(0);
  }
  __syncthreads();

  for (int kt = kt0; kt < kt1; ++kt) {
    const int cur = (kt - kt0) & 1;
    const bool more = kt + 1 < kt1;
    if (more) load_tile(kt + 1);
    const uint16_t* ks = Ks[cur];
    const uint16_t* vt = Vt[cur];

    // S^T tile: 64 keys x 32 queries as two 32x32 accumulators
    f32x16_t s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int e = 0; e < 16; ++e) s[kb][e] = 0.0f;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const bf16x8_t kf = *(const bf16x8_t*)(ks + (kb * 32 + c) * KP + t * 16 + g * 8);
        s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[t], s[kb], 0, 0, 0);
      }
    }

    // scale, mask, online softmax (all 32 scores of this lane are query qi)
    const int k0 = kt * BKV;
    float mt = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int j = k0 + kb * 32 + (e >> 2) * 8 + g * 4 + (e & 3);
        float x = a.round_scores ? vm::round_bf16(s[kb][e]) : s[kb][e];
        x = x * a.scale;
        if (a.mask) x = x + (fa_visible(a.cmp, qi, j) ? a.mask_true : a.mask_false);
        if (j >= a.Sk) x = -INFINITY;
        s[kb][e] = x;
        mt = fmaxf(mt, x);
      }
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float m_new = fmaxf(m_run, mt);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = exp2f((m_run - m_use) * kLog2e);
    m_run = m_new;
    float psum = 0.0f;
    uint32_t pk[2][8];  // bf16 pairs: [kb][e/2]
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; e += 2) {
        const float p0 = exp2f((s[kb][e] - m_use) * kLog2e);
        const float p1 = exp2f((s[kb][e + 1] - m_use) * kLog2e);
        psum += p0 + p1;
        pk[kb][e >> 1] = pack_bf16x2(p0, p1);
      }
    l_run = l_run * alpha + psum;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[dt][e] *= alpha;

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
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const bf16x8_t vf = *(const bf16x8_t*)(vt + (dt * 32 + c) * VP + u * 16 + g * 8);
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf.v, o[dt], 0, 0, 0);
      }
    }

    if (more) store_tile(cur ^ 1);
    __syncthreads();
  }

  // normalise and store: lane (c, g) holds O[qi][dt*32 + (e>>2)*8 + g*4 + (e&3)]
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  if (qi < a.Sq) {
    uint16_t* O = (uint16_t*)a.o + b * a.o_sb + h * a.o_sh + (int64_t)qi * a.o_ss;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d0 = dt * 32 + r * 8 + g * 4;
        *(uint2*)(O + d0) = make_uint2(pack_bf16x2(o[dt][r * 4 + 0] * inv, o[dt][r * 4 + 1] * inv),
                                       pack_bf16x2(o[dt][r * 4 + 2] * inv, o[dt][r * 4 + 3] * inv));
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

void launch_flash(const FlashArgs& a, hipStream_t stream) {
  const int nqt = (a.Sq + fa::BQ - 1) / fa::BQ;
  const unsigned grid = (unsigned)(nqt * a.B * a.H);
  switch (a.D) {
    case 32: hipLaunchKernelGGL(flash_fwd_kernel<32>, dim3(grid), dim3(256), 0, stream, a); break;
    case 64: hipLaunchKernelGGL(flash_fwd_kernel<64>, dim3(grid), dim3(256), 0, stream, a); break;
    default: hipLaunchKernelGGL(flash_fwd_kernel<128>, dim3(grid), dim3(256), 0, stream, a); break;
  }
  REW_HIP(hipGetLastError());
}

}  // namespace rew
