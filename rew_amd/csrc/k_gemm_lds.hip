// bf16 GEMM on CDNA4 with direct global->LDS staging ("gemm_lds").
//
// Output tile 256 x 256 per workgroup, 4 waves of 128 x 128, each a 4 x 4
// grid of v_mfma_f32_32x32x16_bf16 tiles (fp32 accumulators).
//
// Operands travel HBM/L2 -> LDS with buffer_load_dwordx4 ... lds (or
// global_load_lds_dwordx4 on the K-tail path): every lane moves 16 bytes
// and lane l of an instruction lands at LDS base + 16 l, so no VGPRs hold
// staged data and no VALU work writes LDS.  The LDS layout is chosen
// through the source address each lane fetches (k-tiles of BK = 32):
//   * A on the buffer path: k-tile PAIRS, a 256 x 64 tile of 128-byte rows
//     (8 chunks; chunk c of row r at physical chunk c ^ ((r >> 1) & 7)), so
//     each row of a pair is one whole cache line.  Moving A one 64-byte half
//     line per k-tile cost the vector memory pipeline twice the requests
//     (the address unit then stalls on the cache far more than a VGPR-staged
//     kernel does) and measured 3-8 % slower.
//   * K-contiguous operands otherwise (A on the K-tail path, B when it is
//     [N, K]): a 256 x 32 tile, 64-byte rows of four 16-byte chunks, chunk c
//     of row r stored at physical chunk c ^ ((r >> 2) & 3).  The 16 lanes a
//     ds_read_b128 serves per cycle read one logical chunk of 16 consecutive
//     rows; rows r and r + 4 share a 256-byte bank window and the XOR gives
//     them distinct chunks, so the 16 reads hit 16 distinct 16-byte slots.
//   * N-contiguous B (rew's [in, out] Linear weights, the common case): a
//     32 x 256 tile, 512-byte k-rows of 32 chunks, chunk c of row k stored
//     at c ^ (4 (k & 3)).  Fragments are read with ds_read_b64_tr_b16: in
//     each 16-lane group, source lane s points at k-row kb + s/4, columns
//     4 (s % 4) .. +3, and output lane i receives B[kb + j][col0 + i] for
//     j = 0..3 -- four consecutive k of one column, the MFMA B layout, read
//     straight out of the untransposed tile.  Two such reads (kb, kb + 4)
//     give the 8 k-values of one fragment.  The XOR spreads the 8 k-rows x
//     4 chunks of one read over all bank groups.
// The k-tiles stream through a ring: four B stages (16 KiB) and two A pair
// stages (32 KiB) on the buffer path, four 32 KiB A+B stages on the K-tail
// path.  B of tile t + 4 is requested after the barrier that frees tile
// t's stage (right after it for even t, two k-steps later for odd t); an A
// pair two k-steps before its first read.  Every 16-MFMA substep issues
// exactly 4 DMA instructions per wave, one after every fourth MFMA: the
// issue is in order, so a DMA instruction that finds the address unit's
// queue full also holds back the MFMAs behind it, and bursts (8 after
// eight consecutive MFMAs, with none in the other substep) measured 2-4 %
// slower per GEMM.  On the Llama shapes a k-step of MFMAs alone takes 1024
// cycles and the full loop about 1230: the DMA overlaps the MFMAs rather
// than hiding behind them; a fifth stage measured no faster.
//
// Tails: rows / columns past the matrix are read from a clamped in-range
// address (their outputs are never stored); on the K-tail path, k-chunks
// past K are fetched from an in-range address and zeroed in LDS after they
// land, so they add exact zeros.
//
// Modes (template): B N-contiguous or K-contiguous; DUAL (SwiGLU: the tile's
// 256 B columns are 128 gate + 128 up columns of two weight matrices, each
// lane fetching from either); GROUP (routed experts: tile -> group from the
// device tables, A rows gathered through a row list; a group of at most 128
// rows gets 64-row tiles, the four waves side by side on 64 x 64 outputs
// each, with the same B stream and ring).  The MFMAs produce
// C^T blocks, so each lane holds runs of four consecutive output columns:
// the epilogue writes them to a C tile in LDS as 8-byte chunks, then stores
// whole 512-byte row segments with the fused bias / residual / SwiGLU
// arithmetic of GemmArgs.
#include <cstring>

#include "kernels.h"
#include "vm_device.h"

namespace rew {

// 16-byte store of an epilogue's output (REW_GEMM_NT_STORE: nontemporal).
#ifndef REW_GEMM_NT_STORE
#define REW_GEMM_NT_STORE 0
#endif
__device__ __forceinline__ void st_c16(void* p, const uint4& v) {
  if constexpr (REW_GEMM_NT_STORE) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, (u32x4*)p);
  } else {
    *(uint4*)p = v;
  }
}


namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s lds_v4s;
typedef __attribute__((address_space(3))) void lds_void;

constexpr int BM = 256, BN = 256, BK = 32;
constexpr int NS = 4;                     // LDS ring stages
constexpr int A_BYTES = BM * BK * 2;      // 16 KiB
constexpr int B_BYTES = BN * BK * 2;      // 16 KiB
constexpr int STAGE = A_BYTES + B_BYTES;  // 32 KiB
constexpr int DMA_PER_TILE = 8;           // DMA instructions per wave per k-tile
static_assert((NS - 1) * DMA_PER_TILE <= 63, "vmcnt range");

// s_waitcnt immediate (vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] at [15:14])
constexpr int waitcnt_imm(int vm, int lgkm) {
  return (vm & 15) | ((vm >> 4) << 14) | (7 << 4) | ((lgkm & 15) << 8);
}

__device__ __forceinline__ void to_lds16(const void* src, uint8_t* lds) {
  __builtin_amdgcn_global_load_lds(src, (lds_void*)lds, 16, 0, 0);
}
// buffer_load_dwordx4 ... lds: base and extent in the SGPR descriptor, the
// lane's fixed byte offset in a VGPR, the k advance in an SGPR, so a k-tile
// of DMA costs no VALU address arithmetic.
// (the base is wave-uniform; readfirstlane states it, so the descriptor is
// built in SGPRs whatever the rest of the kernel does to register choices)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  void* p = (void*)(uintptr_t)(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(p, (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ void buf_to_lds16(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                             uint32_t soff, uint8_t* lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)lds, 16, voff, soff, 0, 0);
}
// Workgroup barrier without the memory fence of __syncthreads (which would
// wait for every DMA in flight); callers wait for what they need first.
__device__ __forceinline__ void block_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// x * logistic(x) for every bf16 x, as rew's SiLU op sequence computes it
// in fp32 (silu = mul(x, divide(1, add(1, exp(neg(x))))),
// src/rew/nn/activation.nim:28-38): the SwiGLU epilogue's gate takes a
// bf16-rounded input, so it looks the product up instead of running the
// library expf and an IEEE division per output (about 30 VALU
// instructions).  Filled on each device by init_silu_table with the same
// device code as the op-by-op path, so the bits are identical.
__device__ float g_silu_bf16[65536];

__global__ void __launch_bounds__(256) silu_table_kernel() {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  const float x = vm::as_f(i << 16);
  const float e = expf(-x);
  const float den = 1.0f + e;
  const float sig = 1.0f / den;
  g_silu_bf16[i] = x * sig;
}

template <int V>
struct IntK {
  static constexpr int value = V;
};

__device__ __forceinline__ void tile_order(int64_t bid, int64_t tiles_m, int64_t tiles_n,
                                           int64_t batch, int64_t* b, int64_t* tm,
                                           int64_t* tn) {
  // XCD-contiguous ranges (every 8th workgroup shares an XCD), then
  // groups of 4 M-tiles walked down N so an XCD's concurrent tiles share A
  // rows and B columns in its L2.
  const int64_t per = tiles_m * tiles_n, total = per * batch;
  int64_t t = bid;
  if (total % 8 == 0) t = (bid % 8) * (total / 8) + bid / 8;
  *b = t / per;
  t -= *b * per;
  constexpr int64_t GM = 4;
  const int64_t group = GM * tiles_n;
  const int64_t first_m = (t / group) * GM;
  const int64_t gsize = min(GM, tiles_m - first_m);
  const int64_t r = t % group;
  *tm = first_m + r % gsize;
  *tn = r / gsize;
}

}  // namespace

// BUF: K % BK == 0 and every operand byte offset below 2^31 from its
// descriptor base (checked at launch); the K-tail path then never runs.
// FAR (DUAL only): the gate and up matrices lie too far apart for one
// descriptor (allocations need not be near each other), so B moves by
// global_load_lds from per-lane 64-bit addresses (A still through its
// descriptor): a few VALU instructions per B DMA more than one descriptor,
// far fewer than the K-tail path.
template <bool B_KC, bool DUAL, bool GROUP, bool BUF, bool FAR = false>
__global__ void __launch_bounds__(256, 1) gemm_lds_kernel(GemmSegs gs, GroupArgs ga) {
  // LDS, 128 KiB.  K-tail path: four 32 KiB stages, each the A and B halves
  // of one k-tile.  BUF path: two 32 KiB A stages, each a k-tile pair (256
  // rows x 128 bytes, so every A row of a pair is one whole cache line), and
  // four 16 KiB B stages.  Each region is its own __shared__ array so the
  // compiler sees that a DMA into one cannot alias fragment reads of another.
  __shared__ __attribute__((aligned(1024))) uint8_t L0[STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t L1[STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t L2[BUF ? B_BYTES : STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t L3[BUF ? B_BYTES : STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t L4[BUF ? B_BYTES : 16];
  __shared__ __attribute__((aligned(1024))) uint8_t L5[BUF ? B_BYTES : 16];
  auto S = [&](int i) -> uint8_t* {  // K-tail stage i
    return i == 0 ? L0 : i == 1 ? L1 : i == 2 ? L2 : L3;
  };
  auto AS = [&](int p) -> uint8_t* { return p ? L1 : L0; };  // BUF A pair stage
  auto BS = [&](int i) -> uint8_t* {                          // BUF B stage
    return i == 0 ? L2 : i == 1 ? L3 : i == 2 ? L4 : L5;
  };
  // 16 KiB block blk (rows 32 blk .. 32 blk + 31) of the epilogue's C tile
  auto CB = [&](int blk) -> uint8_t* {
    if constexpr (BUF) return blk < 4 ? AS(blk >> 1) + (blk & 1) * B_BYTES : BS(blk - 4);
    else return S(blk >> 1) + (blk & 1) * B_BYTES;
  };
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  constexpr int TN = DUAL ? BN / 2 : BN;  // output columns per workgroup

  // ---- tile (and, over several GEMMs of one A, its segment) ---------------------------
  int64_t b = 0, tm = 0, tn = 0, m_rows, row0;
  int grp = 0, seg = 0;
  bool small = false;  // a kSmallTileM-row tile of a small group
  if constexpr (GROUP) {
    // The grid covers the host's bound on the tiles (max_mtiles rows of
    // them); the routing fixes the real count, read here.  Workgroups past it
    // leave at once, and the real tiles are dealt to the XCDs (workgroups
    // whose indices agree mod 8 share one) in eight contiguous chunks, so
    // each XCD's CUs share A rows in their L2 and every XCD gets an eighth
    // of the work.  (Dealing the whole grid instead left the exits to the
    // last XCD: its CUs finished the grouped SwiGLU at about 290 us, the
    // others at 725-773 us.)
    const int64_t tiles_n = (gs.g[0].N + TN - 1) / TN;
    const int64_t real = (int64_t)ga.mt_start[ga.n_groups] * tiles_n;
    int64_t t = blockIdx.x;
    if (t >= real) return;  // past the routed work (uniform)
    {
      const int64_t q = real / 8, rr = real % 8, x = t % 8;
      t = x * q + (x < rr ? x : rr) + t / 8;
    }
    tm = t / tiles_n;
    tn = t - tm * tiles_n;
    int lo = 0, hi = ga.n_groups - 1;             // last group starting at or before tm
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (ga.mt_start[mid] <= tm) lo = mid;
      else hi = mid - 1;
    }
    grp = lo;
    const int tr = group_tile_rows(ga.off[grp + 1] - ga.off[grp]);
    small = tr == kSmallTileM;
    row0 = ga.off[grp] + (tm - ga.mt_start[grp]) * tr;
    m_rows = min((int64_t)tr, (int64_t)ga.off[grp + 1] - row0);
  } else {
    tile_order(blockIdx.x, (gs.g[0].M + BM - 1) / BM, gs.tn0[gs.n], gs.g[0].batch, &b, &tm,
               &tn);
    while (seg + 1 < gs.n && tn >= gs.tn0[seg + 1]) ++seg;
    tn -= gs.tn0[seg];
    row0 = tm * BM;
    m_rows = min((int64_t)BM, gs.g[0].M - row0);
  }

  // The rest of the kernel is one of two bodies (SM): the 256-row tile, its
  // four waves 2 x 2 of 128 x 128 outputs, or a small group's 64-row tile
  // (grouped, buffer path, N-contiguous B), its four waves side by side,
  // each 64 rows x 64 of the 256 B columns: the same B stream and ring, a
  // quarter of the MFMAs and of the A stream.  (Grouped launches in the
  // other modes run a small group's tiles with the 256-row body.)
  auto run = [&](auto SM) {
  constexpr bool SMALL = decltype(SM)::value;
  static_assert(!SMALL || (GROUP && BUF && !B_KC), "64-row tiles: grouped buffer path");
  constexpr int MI = SMALL ? 2 : 4;    // 32-row blocks per wave
  constexpr int NJ = SMALL ? 2 : 4;    // 32-column blocks per wave
  constexpr int NAQ = SMALL ? 2 : 8;   // A pair DMA instructions per wave
  const int wm = SMALL ? 0 : wave >> 1;                    // rows wm * 128 ..
  const int cb0 = SMALL ? wave * 64 : (wave & 1) * 128;    // the wave's first B column
  const GemmArgs& g = gs.g[seg];
  const int64_t n0 = tn * TN;
  const int K = (int)g.K;
  const int nk = (K + BK - 1) / BK;

  const uint16_t* A = (const uint16_t*)g.a + b * g.a_sb;
  const uint16_t* B1 = GROUP ? (const uint16_t*)ga.b[grp] : (const uint16_t*)g.b + b * g.b_sb;
  const uint16_t* B2 = nullptr;
  if constexpr (DUAL)
    B2 = GROUP ? (const uint16_t*)ga.b2[grp] : (const uint16_t*)g.b2 + b * g.b_sb;
  static_assert(!FAR || (DUAL && BUF), "FAR is a DUAL BUF mode");
  // BUF descriptors: A from its (batch) base; B from the lower of B1 / B2
  const uint16_t* Bbase = (DUAL && B2 < B1) ? B2 : B1;
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(A, 0x7fffffffu);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(Bbase, 0x7fffffffu);

  // ---- per-lane sources of this wave's 4 A and 4 B DMA instructions per k-tile ----
  // Instruction q of wave w fills the stage's 1 KiB block i = 4 w + q of A
  // (and of B).
  const uint16_t* pa[4];
  const uint16_t* pb[4];
  uint32_t va[4], vb[4];  // BUF: byte offsets from the descriptor bases
  // K-tail bookkeeping: the k-chunk (0..3) each lane fetches for A (and B
  // when K-contiguous), or the k-row (0..31) when B is N-contiguous
  int a_kc[4], b_sel[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int i = wave * 4 + q;
    // A block i: rows 16 i .. 16 i + 15, lane -> (row, physical chunk)
    const int r = 16 * i + (lane >> 2);
    const int c = (lane & 3) ^ ((r >> 2) & 3);
    const int rr = r < m_rows ? r : (int)m_rows - 1;
    int64_t arow;
    if constexpr (GROUP)
      arow = ga.rows ? (int64_t)ga.rows[row0 + rr] : row0 + rr;
    else
      arow = row0 + rr;
    pa[q] = A + arow * g.a_sm + c * 8;
    a_kc[q] = c;
    va[q] = (uint32_t)((arow * g.a_sm + c * 8) * 2);
    if constexpr (B_KC) {
      // B [N, K]: block i holds n-rows 16 i .. 16 i + 15 like A
      int64_t nr = n0 + r;
      if (nr >= g.N) nr = g.N - 1;
      pb[q] = B1 + nr * g.b_sn + c * 8;
      b_sel[q] = c;
      vb[q] = (uint32_t)((nr * g.b_sn + c * 8) * 2);
    } else {
      // B [K, N]: block i holds k-rows 2 i, 2 i + 1 (512 bytes each)
      const int kr = 2 * i + (lane >> 5);
      const int cb = (lane & 31) ^ (4 * (kr & 3));  // logical chunk of this lane
      int64_t col;
      const uint16_t* src = B1;
      if (DUAL) {
        const int vcol = cb * 8, quad = vcol >> 6;
        src = (quad & 1) ? B2 : B1;
        col = n0 + (quad >> 1) * 64 + (vcol & 63);
      } else {
        col = n0 + cb * 8;
      }
      if (col > g.N - 8) col = g.N - 8;
      pb[q] = src + (int64_t)kr * g.b_sk + col;
      b_sel[q] = kr;
      vb[q] = FAR ? 0u
                  : (uint32_t)((const uint8_t*)src - (const uint8_t*)Bbase) +
                        (uint32_t)(((int64_t)kr * g.b_sk + col) * 2);
    }
  }

  // BUF: A moves a k-tile pair at a time, NAQ (8; 64-row tiles 2)
  // instructions per wave; lane l of instruction q of wave w covers row
  // r = 8 (NAQ w + q) + l / 8, physical 16-byte chunk l % 8, which holds
  // logical chunk (l % 8) ^ ((r >> 1) & 7) (chunks 0-3 the first k-tile of
  // the pair, 4-7 the second).  The 16 lanes a ds_read_b128 serves per cycle
  // read one logical chunk of 16 rows; rows r and r + 1 fall in different
  // halves of a 256-byte bank window and the XOR spreads the 8 even (odd)
  // rows over 8 distinct chunks.
  uint32_t vap[NAQ];
  if constexpr (BUF) {
#pragma unroll
    for (int q = 0; q < NAQ; ++q) {
      const int r = 8 * (NAQ * wave + q) + (lane >> 3);
      const int c = (lane & 7) ^ ((r >> 1) & 7);
      const int rr = r < m_rows ? r : (int)m_rows - 1;
      int64_t arow;
      if constexpr (GROUP)
        arow = ga.rows ? (int64_t)ga.rows[row0 + rr] : row0 + rr;
      else
        arow = row0 + rr;
      vap[q] = (uint32_t)((arow * g.a_sm + c * 8) * 2);
    }
  }
  // B's k-row stride in bytes, held in an SGPR for the whole loop (left to
  // itself the compiler re-read it from the kernel arguments every other
  // k-step and waited on that scalar load right after the barrier)
  const uint32_t b_kbytes = __builtin_amdgcn_readfirstlane((uint32_t)(B_KC ? 2 : g.b_sk * 2));
  // BUF: the B half of k-tile k0 / BK into B stage bst
  // B DMA instruction q, sob bytes along k (FAR: from the lane's pointer)
  auto dma_b = [&](int q, uint32_t sob, uint8_t* dst) {
    if constexpr (FAR)
      to_lds16((const uint8_t*)pb[q] + sob, dst);
    else
      buf_to_lds16(rb, vb[q], sob, dst);
  };
  auto issue_b = [&](uint8_t* bst, int k0) {
    uint8_t* sb = bst + wave * 4096;
    const uint32_t sob = (uint32_t)k0 * b_kbytes;
#pragma unroll
    for (int q = 0; q < 4; ++q) dma_b(q, sob, sb + q * 1024);
  };
  // BUF: half `half` of this wave's instructions (its rows
  // 8 (NAQ w + NAQ / 2 half) .. + 4 NAQ - 1) for the A of the k-tile pair
  // starting at k0, into A stage ast
  auto issue_a = [&](uint8_t* ast, int k0, int half) {
    uint8_t* sa = ast + wave * NAQ * 1024;
#pragma unroll
    for (int q = NAQ / 2 * half; q < NAQ / 2 * (half + 1); ++q)
      buf_to_lds16(ra, vap[q], (uint32_t)k0 * 2, sa + q * 1024);
  };

  // One k-tile of DMA loads.  Branch-free (it is interleaved with MFMAs).
  // K-tail path: lanes whose chunk lies past K fetch an in-range chunk of
  // the same row instead (a select, not a branch), and clear_tail zeroes
  // those slots once they have landed.
  auto issue = [&](uint8_t* stage, int k0) {
    uint8_t* sa = stage + wave * 4096;
    uint8_t* sb = stage + A_BYTES + wave * 4096;
    if constexpr (BUF) {
      const uint32_t soa = (uint32_t)k0 * 2;
      const uint32_t sob = B_KC ? (uint32_t)k0 * 2 : (uint32_t)(k0 * g.b_sk * 2);
#pragma unroll
      for (int q = 0; q < 4; ++q) buf_to_lds16(ra, va[q], soa, sa + q * 1024);
#pragma unroll
      for (int q = 0; q < 4; ++q) dma_b(q, sob, sb + q * 1024);
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int ka = k0 + a_kc[q] * 8 < K ? k0 : K - 8 - a_kc[q] * 8;
        to_lds16(pa[q] + ka, sa + q * 1024);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (B_KC) {
          const int kb = k0 + b_sel[q] * 8 < K ? k0 : K - 8 - b_sel[q] * 8;
          to_lds16(pb[q] + kb, sb + q * 1024);
        } else {
          const int kb = k0 + b_sel[q] < K ? k0 : K - 1 - b_sel[q];
          to_lds16(pb[q] + (int64_t)kb * g.b_sk, sb + q * 1024);
        }
      }
    }
  };
  // (K-tail path) zero this wave's slots of a partial k-tile and wait for
  // the writes, before the barrier that publishes the tile
  auto clear_tail = [&](uint8_t* stage, int k0) {
    uint8_t* sa = stage + wave * 4096 + lane * 16;
    uint8_t* sb = stage + A_BYTES + wave * 4096 + lane * 16;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (k0 + a_kc[q] * 8 >= K) *(uint4*)(sa + q * 1024) = make_uint4(0, 0, 0, 0);
      const bool dead = B_KC ? k0 + b_sel[q] * 8 >= K : k0 + b_sel[q] >= K;
      if (dead) *(uint4*)(sb + q * 1024) = make_uint4(0, 0, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));
  };

  // ---- per-lane fragment offsets (bytes within a stage) ---------------------------
  // A: rows wm*128 + i*32 + (lane & 31), k-chunk 2 s + (lane >> 5)
  const int a_row = wm * 128 + (lane & 31);
  int a_off[2];      // K-tail stages: per substep
  int ap_off[2][2];  // BUF pair stages: [k-tile of the pair][substep]
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    a_off[s] = a_row * 64 + (((2 * s + (lane >> 5)) ^ ((a_row >> 2) & 3)) * 16);
#pragma unroll
    for (int h = 0; h < 2; ++h)
      ap_off[h][s] = a_row * 128 + (((4 * h + 2 * s + (lane >> 5)) ^ ((a_row >> 1) & 7)) * 16);
  }
  int b_off[NJ];  // per fragment column block j (substep s adds s * 8192), from the B half
  int bk_off[2];  // B_KC: per substep
  if constexpr (B_KC) {
    const int b_row = cb0 + (lane & 31);
#pragma unroll
    for (int s = 0; s < 2; ++s)
      bk_off[s] = b_row * 64 + (((2 * s + (lane >> 5)) ^ ((b_row >> 2) & 3)) * 16);
  } else {
    const int grp16 = lane >> 4, s16 = lane & 15;
    const int kr = 8 * (grp16 >> 1) + (s16 >> 2);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int col = cb0 + j * 32 + 16 * (grp16 & 1) + 4 * (s16 & 3);
      b_off[j] = kr * 512 + ((((col >> 3) ^ (4 * (kr & 3)))) * 16) + (col & 7) * 2;
    }
  }

  f32x16_t acc[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  bf16x8_t fa[2][MI], fb[2][NJ];
  // fragments of one substep: A rows from abase (a row stride of `ast`
  // bytes per 32-row block), B from bbase (the B half of a stage)
  constexpr int AST = BUF ? 32 * 128 : 32 * 64;
  auto read_frags = [&](const uint8_t* abase, int aoff, const uint8_t* bbase, int s, int slot) {
#pragma unroll
    for (int i = 0; i < MI; ++i) fa[slot][i] = *(const bf16x8_t*)(abase + aoff + i * AST);
    if constexpr (B_KC) {
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        fb[slot][j] = *(const bf16x8_t*)(bbase + bk_off[s] + j * 32 * 64);
    } else {
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const uint8_t* p = bbase + b_off[j] + s * 16 * 512;
        const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)p);
        const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(p + 4 * 512));
        v4s both[2] = {lo, hi};
        __builtin_memcpy(&fb[slot][j], both, 16);
      }
    }
  };
  // The B fragment goes in the MFMA's first operand and the A fragment in
  // the second, so the instruction computes the 32 x 32 block of C^T: lane
  // l then holds row l % 32 of the C block, columns 8 (e / 4) + 4 (l / 32)
  // + e % 4 for accumulator element e -- four consecutive columns per group
  // of four elements, which the epilogue stores as one 8-byte chunk.  The
  // products and their k order per element are the same either way.
  auto mfmas = [&](int slot) {
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[slot][j], fa[slot][i], acc[i][j],
                                                            0, 0, 0);
  };

  // ---- main loop -------------------------------------------------------------------
  // k-step kt (its substep-0 fragments already in slot 0; the DMA of the
  // next tiles in flight):
  //   substep 0: 16 MFMAs interleaved one-for-one with the 12 fragment
  //     reads of substep 1;
  //   wait until this wave's DMA of tile kt + 1 has landed (later tiles
  //     stay in flight) and the substep-1 fragments are in, barrier: every
  //     wave is done reading tile kt, tile kt + 1 is complete;
  //   substep 1: 16 MFMAs overlap the reads of tile kt + 1's first
  //     fragments and the DMA into the stages tile kt freed.
  // Past the last tile the DMA re-reads data already resident (an L2 hit;
  // kept branch-free so it can interleave); the final wait drains it.
  auto pin_reads = [&]() {
#pragma unroll
    for (int x = 0; x < 12; ++x) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
  };
  // substep 0 with 4 DMA instructions, one after every fourth MFMA
  auto pin_reads4 = [&]() {
#pragma unroll
    for (int x = 0; x < 16; ++x) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      if (x < 12) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      if ((x & 3) == 0) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM
    }
  };
  // substep 1 with nvm (4 or 8) DMA instructions, evenly spaced
  auto pin_last = [&](int nvm) {
#pragma unroll
    for (int x = 0; x < 16; ++x) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      if (x < 12) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      if (x % (16 / nvm) == 0) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM (DMA)
    }
  };
  // 64-row tiles, either substep: 4 MFMAs with the 6 fragment reads and nvm
  // (1 or 4) DMA instructions
  auto pin_small = [&](int nvm) {
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      if (x < 2) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS reads
      else __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      if (nvm == 4 || x == 0) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM
    }
  };
  // K-tail path: stage kt % NS holds A and B of tile kt; tile kt + NS goes
  // into it once it is free (8 DMA instructions per wave and step).
  auto k_step = [&](uint8_t* cur, uint8_t* nxt, int kt) {
    read_frags(cur, a_off[1], cur + A_BYTES, 1, 1);
    mfmas(0);
    pin_reads();
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(waitcnt_imm((NS - 2) * DMA_PER_TILE, 0));
    if (kt + 2 == nk && K % BK) clear_tail(nxt, (kt + 1) * BK);
    block_barrier();
    // (after the last k-step these reads are dead; keeping them
    // unconditional avoids a branch that costs registers)
    read_frags(nxt, a_off[0], nxt + A_BYTES, 0, 0);
    issue(cur, (kt + NS < nk ? kt + NS : kt) * BK);
    mfmas(1);
    pin_last(8);
    __builtin_amdgcn_sched_barrier(0);
  };
  // BUF path, step kt = 4 t + j: B of tile kt in B stage j, A in pair stage
  // (j >> 1) & 1 (k-tile j & 1 of the pair).  Four DMA instructions per
  // substep, each a quarter of a pair (the first half, rows 0-127, or the
  // second) or one B tile:
  //   even kt: substep 0, the second half of the pair (kt + 2, kt + 3);
  //            substep 1, B of kt + 4 into the stage kt freed;
  //   odd kt:  substep 0, B of kt + 2 into the stage kt - 2 freed;
  //            substep 1, the first half of the pair (kt + 3, kt + 4) into
  //            the pair stage kt freed.
  // Counting back from the wait of step kt, the instructions issued after
  // the last load tile kt + 1 needs are 8 either way: even kt, the two
  // halves of the pair (kt + 2, kt + 3) after B of kt + 1; odd kt, B of
  // kt + 3 and B of kt + 2 after the second half of the pair (kt + 1,
  // kt + 2).
  auto k_step2 = [&](int j, int kt) {
    const int jn = (j + 1) & 3;
    uint8_t* acur = AS((j >> 1) & 1);
    uint8_t* anxt = AS((jn >> 1) & 1);
    read_frags(acur, ap_off[j & 1][1], BS(j), 1, 1);
    if (!(j & 1)) {
      // (past the last pair: the same k as the previous step chose for the
      // first half, its spare reload)
      const int kp = kt + 2 < nk ? kt + 2 : (kt >= 2 ? kt - 2 : 0);
      issue_a(AS(((j + 3) >> 1) & 1), kp * BK, 1);
    } else {
      issue_b(BS((j + 2) & 3), (kt + 2 < nk ? kt + 2 : kt) * BK);
    }
    mfmas(0);
    if constexpr (SMALL) pin_small(j & 1 ? 4 : NAQ / 2);
    else pin_reads4();
    __builtin_amdgcn_sched_barrier(0);
    // (64-row tiles: a pair half is NAQ / 2 instructions, so the even
    // steps' count is NAQ)
    if (j & 1) __builtin_amdgcn_s_waitcnt(waitcnt_imm(8, 0));
    else __builtin_amdgcn_s_waitcnt(waitcnt_imm(NAQ, 0));
    block_barrier();
    read_frags(anxt, ap_off[jn & 1][0], BS(jn), 0, 0);
    if (j & 1) issue_a(acur, (kt + 3 < nk ? kt + 3 : kt - 1) * BK, 0);
    else issue_b(BS(j), (kt + NS < nk ? kt + NS : kt) * BK);
    mfmas(1);
    if constexpr (SMALL) pin_small(j & 1 ? NAQ / 2 : 4);
    else pin_last(4);
    __builtin_amdgcn_sched_barrier(0);
  };

  int kt = 0;
  if constexpr (BUF) {
    // the issue order of the (virtual) steps -4 .. -1 (step 0 requests the
    // second half of the pair (2, 3), step 1 B of tile 3)
    issue_b(BS(0), 0);
    issue_a(AS(0), 0, 0);
    issue_a(AS(0), 0, 1);
    issue_b(BS(2), (2 < nk ? 2 : 0) * BK);
    issue_b(BS(1), (1 < nk ? 1 : 0) * BK);
    issue_a(AS(1), (2 < nk ? 2 : 0) * BK, 0);
    // (the last three requests, 8 + NAQ / 2 instructions, stay in flight)
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(8 + NAQ / 2, 15));
    block_barrier();
    read_frags(AS(0), ap_off[0][0], BS(0), 0, 0);
    // Whole turns of the ring, then the remaining steps (nk is even): no
    // path re-enters the loop with a DMA into a stage it reads first still
    // in flight, so the compiler adds no wait for one.
    for (; kt + NS <= nk; kt += NS) {
#pragma unroll
      for (int j = 0; j < NS; ++j) k_step2(j, kt + j);
    }
    if (kt < nk) {
      k_step2(0, kt);
      k_step2(1, kt + 1);
    }
  } else {
#pragma unroll
    for (int t = 0; t < NS; ++t) issue(S(t), (t < nk ? t : 0) * BK);
    __builtin_amdgcn_s_waitcnt(waitcnt_imm((NS - 1) * DMA_PER_TILE, 15));
    if (nk == 1 && K % BK) clear_tail(L0, 0);
    block_barrier();
    read_frags(L0, a_off[0], L0 + A_BYTES, 0, 0);
    for (; kt + NS <= nk; kt += NS) {
#pragma unroll
      for (int j = 0; j < NS; ++j) k_step(S(j), S((j + 1) % NS), kt + j);
    }
#pragma unroll
    for (int j = 0; j < NS - 1; ++j)
      if (kt + j < nk) k_step(S(j), S(j + 1), kt + j);
  }
  // the dummy DMAs (into the stages past the last tile) must land before
  // the epilogue reuses the LDS
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 15));
  __syncthreads();

  // ---- epilogue ----------------------------------------------------------------------
  // phase 1: bf16(acc) into the C tile in LDS (the ring is free now): rows
  // 32 b .. 32 b + 31 in 16 KiB block b, 512-byte rows, 16-byte chunk ch of
  // row r stored at ch ^ (r & 15).  For block (i, j) and column group q = e / 4
  // a lane holds 4 consecutive columns of one row: one ds_write_b64, and
  // the 32 rows of a write spread over 16 chunk positions (2-way at most).
  auto pack4 = [](const float* v) {
    return make_uint2(vm::bf16x2_bits(v[0], v[1]), vm::bf16x2_bits(v[2], v[3]));
  };
  {
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      uint8_t* cb = CB(wm * 4 + i);  // rows wm * 128 + 32 i + [0, 32)
      const int lr = lane & 31;
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int col = cb0 + j * 32 + q * 8 + (lane >> 5) * 4;
          float v[4];
#pragma unroll
          for (int x = 0; x < 4; ++x) v[x] = acc[i][j][q * 4 + x];
          *(uint2*)(cb + lr * 512 + (((col >> 3) ^ (lr & 15)) * 16) + ((col >> 2) & 1) * 8) =
              pack4(v);
        }
    }
  }
  // Phase 2 gives each thread one fixed 16-byte column chunk of the output
  // (chunk ch of CH per row) on rows r_in, r_in + RPI, ...; its column
  // operands (bias, gate bias) are requested before the barrier.  Operand
  // addresses of rows / columns past the matrix are clamped into it, so
  // every load is unconditional; only the stores are predicated.
  constexpr int OC = DUAL ? 128 : 256;  // output columns per tile
  constexpr int CH = OC / 8;            // 16-byte chunks per output row
  constexpr int RPI = 256 / CH;         // rows per pass of the workgroup
  constexpr int PASSES = (SMALL ? kSmallTileM : BM) / RPI;
  const int ch = tid % CH, r_in = tid / CH;
  const int64_t n = n0 + ch * 8;
  const bool col_ok = n < g.N;
  const int64_t nc = col_ok ? n : g.N - 8;                          // clamped column
  const int lc = DUAL ? (ch >> 3) * 128 + (ch & 7) * 8 : ch * 8;  // column in the C tile
  const int epi = DUAL ? (int)EPI_SWIGLU : g.epi;
  uint4 bv = make_uint4(0, 0, 0, 0), bv2 = make_uint4(0, 0, 0, 0);
  if (epi != EPI_NONE) bv = *(const uint4*)((const uint16_t*)(GROUP ? ga.bias[grp] : g.bias) + nc);
  if constexpr (DUAL)
    bv2 = *(const uint4*)((const uint16_t*)(GROUP ? ga.bias2[grp] : g.bias2) + nc);
  __syncthreads();

  // phase 2: 16-byte row chunks (a row's 512 bytes per 32 lanes) with the
  // bias / residual / gate / rotation arithmetic, one loop per epilogue
  // kind so no per-element test or branch sits inside it.  Row operands
  // (residual, rotation tables) are fetched U passes at a time, the next
  // batch requested before this batch's stores: the wait for a batch then
  // never includes stores (vmcnt counts both, in issue order).
  auto c_chunk = [&](int row, int col) -> uint4 {
    const int lr = row & 31;
    return *(const uint4*)(CB(row >> 5) + lr * 512 + ((((col >> 3) ^ (lr & 15))) * 16));
  };
  auto bf = [](uint16_t h) { return vm::as_f((uint32_t)h << 16); };
  uint16_t* C = (uint16_t*)g.c + b * g.c_sb;
  const uint16_t* bh = (const uint16_t*)&bv;
  auto row_of = [&](int p) { return p * RPI + r_in; };
  auto row_ok = [&](int row) { return row < m_rows && col_ok; };
  auto crow = [&](int row) { return row0 + (row < m_rows ? row : (int)m_rows - 1); };
  constexpr int U = SMALL ? 4 : 8;
  static_assert(PASSES % U == 0, "passes per operand batch");

  if (epi == EPI_SWIGLU) {
    const int64_t c_sm = g.c_sm;
    const uint16_t* buh = (const uint16_t*)&bv2;
    // (runtime loops here: the epilogue runs once per tile, and unrolled it
    // would stream tens of KB of straight-line code through the I-cache)
#pragma unroll 1
    for (int p0 = 0; p0 < PASSES; p0 += U) {
      // all U rows' table lookups are requested before any store (a store
      // under the row predicate is a branch, and the compiler waits for
      // every load in flight at it)
      float act[U][8];
      uint32_t up[U][4];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int row = row_of(p0 + u);
        const uint4 dv = c_chunk(row, lc);
        const uint4 uv = c_chunk(row, lc + 64);
        const uint16_t* dh = (const uint16_t*)&dv;
        const uint16_t* uh = (const uint16_t*)&uv;
#pragma unroll
        for (int x = 0; x < 8; x += 2) {
          // GatedFeedForward's gate, op by op in fp32 (gated_ffn.nim:46-67,
          // activation.nim:28-38): g and u rounded to bf16 two at a time,
          // g * logistic(g) from the table by g's bits
          const uint32_t pg = vm::bf16x2_bits(bf(dh[x]) + bf(bh[x]), bf(dh[x + 1]) + bf(bh[x + 1]));
          up[u][x >> 1] = vm::bf16x2_bits(bf(uh[x]) + bf(buh[x]), bf(uh[x + 1]) + bf(buh[x + 1]));
          act[u][x] = g_silu_bf16[pg & 0xffffu];
          act[u][x + 1] = g_silu_bf16[pg >> 16];
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int row = row_of(p0 + u);
        uint32_t out[4];
#pragma unroll
        for (int x = 0; x < 8; x += 2)
          out[x >> 1] = vm::bf16x2_bits(act[u][x] * vm::as_f(up[u][x >> 1] << 16),
                                        act[u][x + 1] * vm::as_f(up[u][x >> 1] & 0xffff0000u));
        if (row_ok(row)) st_c16(C + (row0 + row) * c_sm + n, *(const uint4*)out);
      }
    }
  } else if (epi == EPI_NONE || epi == EPI_BIAS) {
    const bool add = epi == EPI_BIAS;
    const int64_t c_sm = g.c_sm;
#pragma unroll 1
    for (int p0 = 0; p0 < PASSES; p0 += U) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int row = row_of(p0 + u);
        uint4 dv = c_chunk(row, lc);
        if (add) {
          uint16_t* dh = (uint16_t*)&dv;
#pragma unroll
          for (int x = 0; x < 8; ++x) dh[x] = vm::bf16_bits(bf(dh[x]) + bf(bh[x]));
        }
        if (row_ok(row)) st_c16(C + (row0 + row) * c_sm + n, dv);
      }
    }
  } else if (epi == EPI_BIAS_RES) {
    const uint16_t* res = (const uint16_t*)g.res + b * g.res_sb;
    const int64_t res_sm = g.res_sm, c_sm = g.c_sm;
    // two operand buffers used in turn (a register copy of a pending load
    // would have to wait for it)
    uint4 ra[U], rb[U];
    auto fetch = [&](int p0, uint4* dst) {
#pragma unroll
      for (int u = 0; u < U; ++u)
        dst[u] = *(const uint4*)(res + crow(row_of(p0 + u)) * res_sm + nc);
    };
    auto apply = [&](int p0, const uint4* rv) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int row = row_of(p0 + u);
        const uint4 dv = c_chunk(row, lc);
        const uint16_t* dh = (const uint16_t*)&dv;
        const uint16_t* rh = (const uint16_t*)&rv[u];
        uint16_t out[8];
#pragma unroll
        for (int x = 0; x < 8; ++x) {
          const float y = vm::round_bf16(bf(dh[x]) + bf(bh[x]));
          out[x] = vm::bf16_bits(bf(rh[x]) + y);
        }
        if (row_ok(row)) st_c16(C + (row0 + row) * c_sm + n, *(const uint4*)out);
      }
    };
    fetch(0, ra);
#pragma unroll 1
    for (int p0 = 0; p0 < PASSES; p0 += 2 * U) {
      fetch(p0 + U, rb);
      apply(p0, ra);
      if (p0 + 2 * U < PASSES) fetch(p0 + 2 * U, ra);
      apply(p0 + U, rb);
    }
  } else {
    // EPI_BIAS_ROPE: Linear's bias add, then applyRotate (rope.nim:56-108)
    // on the four pairs of a chunk, scattered into the rotated tensor's
    // layout
    constexpr int UR = 4;
    // (DUAL kernels never take this branch: their epilogue is the SwiGLU)
    static_assert(DUAL || PASSES % (2 * UR) == 0, "rotation operand batches");
    const uint32_t nn = (uint32_t)nc;
    const uint32_t hq = nn / (uint32_t)g.rope_D, dq = nn - hq * (uint32_t)g.rope_D;
    const uint32_t rS = (uint32_t)g.rope_S;
    const int64_t rtb = g.rope_tb, rts = g.rope_ts, rti = g.rope_ti;
    const int64_t hoff = hq * g.rope_th + (dq >> 1) * rti;
    const int64_t ob = g.out_b, os = g.out_s, oh = hq * g.out_h + dq;
    const float* rcos = g.rope_cos;
    const float* rsin = g.rope_sin;
    // The four angles of a chunk sit at tb + x * rti.  Unit or 2-element
    // pair strides (the latter: rew's [S, D] tables with each angle stored
    // twice, read through applyRotate's even-element slice) with 16-byte
    // aligned rows take one or two 16-byte loads per table and row.
    const bool al = ((rtb | rts | g.rope_th) & 3) == 0 &&
                    (((uintptr_t)rcos | (uintptr_t)rsin) & 15) == 0;
    const int vmode = !al ? 0 : rti == 1 ? 1 : rti == 2 ? 2 : 0;
    struct Rot {
      float c[UR][4], s[UR][4];
    };
    auto rotate = [&](auto VM) {
      constexpr int kV = decltype(VM)::value;
      Rot ta, tb2;
      auto fetch = [&](int p0, Rot& t) {
#pragma unroll
        for (int u = 0; u < UR; ++u) {
          const uint32_t mm = (uint32_t)crow(row_of(p0 + u));
          const uint32_t bq = mm / rS, sq = mm - bq * rS;
          const int64_t tb = bq * rtb + sq * rts + hoff;
          if constexpr (kV == 1) {
            const float4 cv = *(const float4*)(rcos + tb);
            const float4 sv = *(const float4*)(rsin + tb);
            t.c[u][0] = cv.x; t.c[u][1] = cv.y; t.c[u][2] = cv.z; t.c[u][3] = cv.w;
            t.s[u][0] = sv.x; t.s[u][1] = sv.y; t.s[u][2] = sv.z; t.s[u][3] = sv.w;
          } else if constexpr (kV == 2) {
            f32x4_t c0 = *(const f32x4_t*)(rcos + tb), c1 = *(const f32x4_t*)(rcos + tb + 4);
            f32x4_t s0 = *(const f32x4_t*)(rsin + tb), s1 = *(const f32x4_t*)(rsin + tb + 4);
            // (whole 16-byte loads: left alone the compiler splits them into
            // the dwords used, four times the memory instructions)
            asm volatile("" : "+v"(c0), "+v"(c1), "+v"(s0), "+v"(s1));
            t.c[u][0] = c0[0]; t.c[u][1] = c0[2]; t.c[u][2] = c1[0]; t.c[u][3] = c1[2];
            t.s[u][0] = s0[0]; t.s[u][1] = s0[2]; t.s[u][2] = s1[0]; t.s[u][3] = s1[2];
          } else {
#pragma unroll
            for (int x = 0; x < 4; ++x) {
              t.c[u][x] = rcos[tb + x * rti];
              t.s[u][x] = rsin[tb + x * rti];
            }
          }
        }
      };
      auto apply = [&](int p0, const Rot& t) {
#pragma unroll
        for (int u = 0; u < UR; ++u) {
          const int row = row_of(p0 + u);
          const uint32_t mm = (uint32_t)(row0 + row);
          const uint32_t bq = mm / rS, sq = mm - bq * rS;
          const uint4 dv = c_chunk(row, lc);
          const uint16_t* dh = (const uint16_t*)&dv;
          uint16_t out[8];
#pragma unroll
          for (int x = 0; x < 4; ++x) {
            const float x0 = vm::round_bf16(bf(dh[2 * x]) + bf(bh[2 * x]));
            const float x1 = vm::round_bf16(bf(dh[2 * x + 1]) + bf(bh[2 * x + 1]));
            const float t1 = t.c[u][x] * x0;
            const float t2 = t.s[u][x] * x1;
            const float t3 = t.s[u][x] * x0;
            const float t4 = t.c[u][x] * x1;
            out[2 * x] = vm::bf16_bits(t1 - t2);
            out[2 * x + 1] = vm::bf16_bits(t3 + t4);
          }
          if (row_ok(row)) st_c16(C + bq * ob + sq * os + oh, *(const uint4*)out);
        }
      };
      fetch(0, ta);
#pragma unroll 1
      for (int p0 = 0; p0 < PASSES; p0 += 2 * UR) {
        fetch(p0 + UR, tb2);
        apply(p0, ta);
        if (p0 + 2 * UR < PASSES) fetch(p0 + 2 * UR, ta);
        apply(p0 + UR, tb2);
      }
    };
    if (vmode == 2) rotate(IntK<2>{});
    else if (vmode == 1) rotate(IntK<1>{});
    else rotate(IntK<0>{});
  }
  };  // run

  if constexpr (GROUP && BUF && !B_KC) {
    if (small) {  // (uniform)
      run(IntK<1>{});
      return;
    }
  }
  run(IntK<0>{});
}

// Conditions of the gemm_lds kernels: bf16 in / out, K-contiguous A with
// 16-byte aligned rows, B either K- or N-contiguous (N-contiguous needs
// N % 8 == 0), 16-byte aligned bf16 C rows and epilogue operands.
bool gemm_lds_ok(const GemmArgs& g, bool* b_kc) {
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  if (g.dtype != REW_DT_BFLOAT16 || g.c_dtype != REW_DT_BFLOAT16) return false;
  if (g.K <= 0 || g.K % 8 || g.N % 8 || g.M <= 0) return false;
  if (g.a_sk != 1 || g.a_sm % 8 || g.a_sb % 8 || !al16(g.a)) return false;
  if (g.b_sk == 1 && g.b_sn % 8 == 0 && g.b_sb % 8 == 0) *b_kc = true;
  else if (g.b_sn == 1 && g.b_sk % 8 == 0 && g.b_sb % 8 == 0) *b_kc = false;
  else return false;
  if (!al16(g.b) || !al16(g.c) || g.c_sm % 8 || g.c_sb % 8) return false;
  if (g.epi != EPI_NONE && !al16(g.bias)) return false;
  if (g.epi == EPI_SWIGLU && (*b_kc || !al16(g.bias2) || !al16(g.b2))) return false;
  if (g.epi == EPI_BIAS_RES && (!al16(g.res) || g.res_sm % 8 || g.res_sb % 8)) return false;
  if (g.epi == EPI_BIAS_ROPE &&
      (g.batch != 1 || g.rope_S <= 0 || g.rope_D <= 0 || g.rope_D % 8 || g.N % g.rope_D ||
       g.M % g.rope_S || g.M >= (1ll << 31) || g.N >= (1ll << 31) || !g.rope_cos ||
       !g.rope_sin || g.out_b % 8 || g.out_s % 8 || g.out_h % 8))
    return false;
  return true;
}

// Whether the buffer-descriptor DMA path can run g: K a multiple of 2 BK
// (A moves in k-tile pairs) and every byte offset the kernel forms (row
// offset + k advance) below 2^31.  0: no; 1: yes; 2: yes with a descriptor
// per SwiGLU matrix (their distance apart is past the limit, each matrix's
// own extent is not).
static int buf_mode(const GemmArgs& g, const GroupArgs* ga, bool bkc, bool dual) {
  constexpr int64_t kLim = (int64_t)1 << 31;
  if (g.K % (2 * BK)) return 0;
  const int64_t a_span = ((g.M - 1) * g.a_sm + g.K) * 2;
  const int64_t b_span = bkc ? ((g.N - 1) * g.b_sn + g.K) * 2 : ((g.K - 1) * g.b_sk + g.N) * 2;
  if (a_span >= kLim || b_span >= kLim) return 0;
  if (dual) {
    int64_t d = -1;
    if (ga) d = ga->dual_span;
    else d = (int64_t)((uintptr_t)g.b2 - (uintptr_t)g.b);
    if (ga && d < 0) return 0;
    if (b_span + (d < 0 ? -d : d) >= kLim) return bkc ? 0 : 2;
  }
  return 1;
}

static void launch_segs(const GemmSegs& gs, const GroupArgs* ga, bool bkc, int buf,
                        hipStream_t stream) {
  const GemmArgs& g = gs.g[0];
  const bool dual = g.epi == EPI_SWIGLU;
  const int64_t tiles = ga ? ga->max_mtiles * gs.tn0[gs.n]
                           : ((g.M + 255) / 256) * gs.tn0[gs.n] * g.batch;
  if (tiles <= 0) return;
  if (tiles >= (1ll << 31)) fail(REW_MI355X_ERR_INVALID, "internal: gemm_lds grid too large");
  const GroupArgs none{};
  const GroupArgs& G = ga ? *ga : none;
  const dim3 grid((unsigned)tiles), block(256);
#define REW_LDS_LAUNCH(BKC, DU, GR)                                                          \
  do {                                                                                      \
    if (DU && buf == 2)                                                                     \
      hipLaunchKernelGGL((gemm_lds_kernel<BKC, DU, GR, true, DU>), grid, block, 0, stream, gs, \
                         G);                                                                \
    else if (buf)                                                                           \
      hipLaunchKernelGGL((gemm_lds_kernel<BKC, DU, GR, true>), grid, block, 0, stream, gs, G); \
    else                                                                                    \
      hipLaunchKernelGGL((gemm_lds_kernel<BKC, DU, GR, false>), grid, block, 0, stream, gs, G); \
  } while (0)
  if (ga) {
    if (dual) REW_LDS_LAUNCH(false, true, true);
    else if (bkc) REW_LDS_LAUNCH(true, false, true);
    else REW_LDS_LAUNCH(false, false, true);
  } else {
    if (dual) REW_LDS_LAUNCH(false, true, false);
    else if (bkc) REW_LDS_LAUNCH(true, false, false);
    else REW_LDS_LAUNCH(false, false, false);
  }
#undef REW_LDS_LAUNCH
  REW_HIP(hipGetLastError());
}

void init_silu_table(hipStream_t stream) {
  hipLaunchKernelGGL(silu_table_kernel, dim3(256), dim3(256), 0, stream);
  REW_HIP(hipGetLastError());
}

void launch_gemm_lds(const GemmArgs& g, const GroupArgs* ga, hipStream_t stream) {
  bool bkc = false;
  if (!gemm_lds_ok(g, &bkc)) fail(REW_MI355X_ERR_INVALID, "internal: gemm_lds not launchable");
  const bool dual = g.epi == EPI_SWIGLU;
  GemmSegs gs;
  std::memset(&gs, 0, sizeof gs);
  gs.n = 1;
  gs.g[0] = g;
  gs.tn0[1] = (g.N + (dual ? 127 : 255)) / (dual ? 128 : 256);
  launch_segs(gs, ga, bkc, buf_mode(g, ga, bkc, dual), stream);
}

bool gemm_multi_ok(const GemmArgs* segs, int n) {
  if (n < 1 || n > kMaxSegs) return false;
  bool bkc0 = false;
  // SwiGLU segments (the dual kernel) go only with SwiGLU segments
  const bool dual = segs[0].epi == EPI_SWIGLU;
  for (int i = 0; i < n; ++i) {
    const GemmArgs& g = segs[i];
    bool bkc;
    if (!gemm_lds_ok(g, &bkc) || (g.epi == EPI_SWIGLU) != dual) return false;
    if (i == 0) {
      bkc0 = bkc;
      continue;
    }
    const GemmArgs& f = segs[0];
    if (bkc != bkc0 || g.a != f.a || g.M != f.M || g.K != f.K || g.a_sm != f.a_sm ||
        g.a_sb != f.a_sb || g.batch != f.batch)
      return false;
  }
  return true;
}

void launch_gemm_multi(const GemmArgs* segs, int n, hipStream_t stream) {
  if (!gemm_multi_ok(segs, n)) fail(REW_MI355X_ERR_INVALID, "internal: GEMM set not launchable");
  GemmSegs gs;
  std::memset(&gs, 0, sizeof gs);
  gs.n = n;
  bool bkc = false;
  int buf = 1;  // the lowest segment's mode, FAR over plain
  const bool dual = segs[0].epi == EPI_SWIGLU;
  const int tn = dual ? 128 : 256;  // output columns per tile
  for (int i = 0; i < n; ++i) {
    gemm_lds_ok(segs[i], &bkc);
    const int m = buf_mode(segs[i], nullptr, bkc, dual);
    buf = (buf == 0 || m == 0) ? 0 : (buf == 2 || m == 2 ? 2 : 1);
    gs.g[i] = segs[i];
    gs.tn0[i + 1] = gs.tn0[i] + (segs[i].N + tn - 1) / tn;
  }
  launch_segs(gs, nullptr, bkc, buf, stream);
}

}  // namespace rew
