// bf16 GEMM on CDNA4 with direct global->LDS staging ("gemm_lds").
//
// Output tile 256 x 256 per workgroup, 4 waves of 128 x 128, each a 4 x 4
// grid of v_mfma_f32_32x32x16_bf16 tiles (fp32 accumulators), BK = 64.
//
// Operands travel HBM/L2 -> LDS with global_load_lds_dwordx4: every lane
// moves 16 bytes and lane l of an instruction lands at LDS base + 16 l, so
// no VGPRs hold staged data and no VALU work writes LDS.  The LDS layout is
// chosen through the source address each lane fetches:
//   * K-contiguous operands (A, and B when it is [N, K]): a 256 x 64 tile,
//     128-byte rows of eight 16-byte chunks, chunk c of row r stored at
//     physical chunk c ^ ((r >> 1) & 7).  Two rows share a 256-byte bank
//     window, so the 16 rows a ds_read_b128 serves per cycle land on 16
//     distinct 16-byte bank slots (a plain c ^ (r & 7) maps rows r and
//     r + 8 to the same slot: a 2-way conflict on every fragment read).
//   * N-contiguous B (rew's [in, out] Linear weights, the common case): a
//     64 x 256 tile, 512-byte k-rows of 32 chunks, chunk c of row k stored
//     at c ^ (4 (k & 3)).  Fragments are read with ds_read_b64_tr_b16: in
//     each 16-lane group, source lane s points at k-row kb + s/4, columns
//     4 (s % 4) .. +3, and output lane i receives B[kb + j][col0 + i] for
//     j = 0..3 -- four consecutive k of one column, the MFMA B layout, read
//     straight out of the untransposed tile.  Two such reads (kb, kb + 4)
//     give the 8 k-values of one fragment.  The XOR spreads the 8 k-rows x
//     4 chunks of one read over all bank groups.
// Two LDS stages: tile k + 1 streams into one while the MFMAs consume the
// other; one s_waitcnt vmcnt(0) + barrier per k-tile.
//
// Tails: rows / columns past the matrix are read from a clamped in-range
// address (their outputs are never stored); k-chunks past K are zeroed in
// LDS after they land, so they add exact zeros.
//
// Modes (template): B N-contiguous or K-contiguous; DUAL (SwiGLU: the tile's
// 256 B columns are 128 gate + 128 up columns of two weight matrices, each
// lane fetching from either); GROUP (routed experts: tile -> group from the
// device tables, A rows gathered through a row list).  The epilogue stages
// the bf16 C tile through LDS and writes 16-byte row chunks with the fused
// bias / residual / SwiGLU arithmetic of GemmArgs.
#include "kernels.h"
#include "vm_device.h"

namespace rew {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s lds_v4s;
typedef __attribute__((address_space(3))) void lds_void;

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int A_BYTES = BM * BK * 2;  // 32 KiB
constexpr int B_BYTES = BN * BK * 2;  // 32 KiB
constexpr int STAGE = A_BYTES + B_BYTES;
constexpr int CP = BN + 8;            // epilogue C tile pitch (elements)
// Each stage is its own __shared__ array (so the compiler sees that the
// DMA into one stage cannot alias fragment reads of the other), sized to
// also hold half of the epilogue's C tile.
constexpr int SBYTES = (BM / 2) * CP * 2 > STAGE ? (BM / 2) * CP * 2 : STAGE;

__device__ __forceinline__ void to_lds16(const void* src, uint8_t* lds) {
  __builtin_amdgcn_global_load_lds(src, (lds_void*)lds, 16, 0, 0);
}

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

template <bool B_KC, bool DUAL, bool GROUP>
__global__ void __launch_bounds__(256, 1) gemm_lds_kernel(GemmArgs g, GroupArgs ga) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem0[SBYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t smem1[SBYTES];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  constexpr int TN = DUAL ? BN / 2 : BN;  // output columns per workgroup
  const int64_t tiles_n = (g.N + TN - 1) / TN;

  // ---- tile ------------------------------------------------------------------------
  int64_t b = 0, tm = 0, tn = 0, m_rows, row0;
  int grp = 0;
  if constexpr (GROUP) {
    const int64_t total = ga.max_mtiles * tiles_n;
    int64_t t = blockIdx.x;
    if (total % 8 == 0) t = (t % 8) * (total / 8) + t / 8;
    tm = t / tiles_n;
    tn = t - tm * tiles_n;
    if (tm >= ga.mt_start[ga.n_groups]) return;  // past the routed work (uniform)
    int lo = 0, hi = ga.n_groups - 1;             // last group starting at or before tm
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (ga.mt_start[mid] <= tm) lo = mid;
      else hi = mid - 1;
    }
    grp = lo;
    row0 = ga.off[grp] + (tm - ga.mt_start[grp]) * BM;
    m_rows = min((int64_t)BM, (int64_t)ga.off[grp + 1] - row0);
  } else {
    tile_order(blockIdx.x, (g.M + BM - 1) / BM, tiles_n, g.batch, &b, &tm, &tn);
    row0 = tm * BM;
    m_rows = min((int64_t)BM, g.M - row0);
  }
  const int64_t n0 = tn * TN;
  const int K = (int)g.K;
  const int nk = (K + BK - 1) / BK;

  const uint16_t* A = (const uint16_t*)g.a + b * g.a_sb;
  const uint16_t* B1 = GROUP ? (const uint16_t*)ga.b[grp] : (const uint16_t*)g.b + b * g.b_sb;
  const uint16_t* B2 = nullptr;
  if constexpr (DUAL)
    B2 = GROUP ? (const uint16_t*)ga.b2[grp] : (const uint16_t*)g.b2 + b * g.b_sb;

  // ---- per-lane source pointers of this wave's 8 A and 8 B load instructions ------
  // Instruction q of wave w fills LDS block i = 8 w + q (1 KiB).
  const uint16_t* pa[8];
  const uint16_t* pb[8];
  // K-tail bookkeeping: the k-chunk (0..7) each lane fetches for A (and B
  // when K-contiguous), or the k-row (0..63) when B is N-contiguous
  int a_kc[8], b_sel[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int i = wave * 8 + q;
    // A block i: rows 8 i .. 8 i + 7, lane -> (row, physical chunk)
    const int r = 8 * i + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    const int rr = r < m_rows ? r : (int)m_rows - 1;
    int64_t arow;
    if constexpr (GROUP)
      arow = ga.rows ? (int64_t)ga.rows[row0 + rr] : row0 + rr;
    else
      arow = row0 + rr;
    pa[q] = A + arow * g.a_sm + c * 8;
    a_kc[q] = c;
    if constexpr (B_KC) {
      // B [N, K]: block i holds n-rows 8 i .. 8 i + 7 like A
      int64_t nr = n0 + r;
      if (nr >= g.N) nr = g.N - 1;
      pb[q] = B1 + nr * g.b_sn + c * 8;
      b_sel[q] = c;
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
    }
  }

  // One k-tile of DMA loads.  Branch-free (it is interleaved with MFMAs):
  // on the partial last k-tile the lanes whose chunk lies past K fetch an
  // in-range chunk of the same row instead (a select, not a branch), and
  // clear_tail zeroes those slots once they have landed.
  auto issue = [&](uint8_t* stage, int k0) {
    uint8_t* sa = stage + wave * 8 * 1024;
    uint8_t* sb = stage + A_BYTES + wave * 8 * 1024;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int ka = k0 + a_kc[q] * 8 < K ? k0 : K - 8 - a_kc[q] * 8;
      to_lds16(pa[q] + ka, sa + q * 1024);
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      if (B_KC) {
        const int kb = k0 + b_sel[q] * 8 < K ? k0 : K - 8 - b_sel[q] * 8;
        to_lds16(pb[q] + kb, sb + q * 1024);
      } else {
        const int kb = k0 + b_sel[q] < K ? k0 : K - 1 - b_sel[q];
        to_lds16(pb[q] + (int64_t)kb * g.b_sk, sb + q * 1024);
      }
    }
  };
  auto clear_tail = [&](uint8_t* stage, int k0) {
    uint8_t* sa = stage + wave * 8 * 1024 + lane * 16;
    uint8_t* sb = stage + A_BYTES + wave * 8 * 1024 + lane * 16;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      if (k0 + a_kc[q] * 8 >= K) *(uint4*)(sa + q * 1024) = make_uint4(0, 0, 0, 0);
      const bool dead = B_KC ? k0 + b_sel[q] * 8 >= K : k0 + b_sel[q] >= K;
      if (dead) *(uint4*)(sb + q * 1024) = make_uint4(0, 0, 0, 0);
    }
  };

  // ---- per-lane fragment offsets (bytes within a stage) ---------------------------
  // A: rows wm*128 + i*32 + (lane & 31), k-chunk 2 s + (lane >> 5)
  const int a_row = wm * 128 + (lane & 31);
  int a_off[4];
#pragma unroll
  for (int s = 0; s < 4; ++s)
    a_off[s] = a_row * 128 + (((2 * s + (lane >> 5)) ^ ((lane >> 1) & 7)) * 16);
  int b_off[4];  // per fragment column block j (substep s adds s * 8192)
  int bk_off[4];  // B_KC: per substep
  if constexpr (B_KC) {
    const int b_row = wn * 128 + (lane & 31);
#pragma unroll
    for (int s = 0; s < 4; ++s)
      bk_off[s] = A_BYTES + b_row * 128 + (((2 * s + (lane >> 5)) ^ ((lane >> 1) & 7)) * 16);
  } else {
    const int grp16 = lane >> 4, s16 = lane & 15;
    const int kr = 8 * (grp16 >> 1) + (s16 >> 2);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = wn * 128 + j * 32 + 16 * (grp16 & 1) + 4 * (s16 & 3);
      b_off[j] = A_BYTES + kr * 512 + ((((col >> 3) ^ (4 * (kr & 3)))) * 16) + (col & 7) * 2;
    }
  }

  f32x16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  bf16x8_t fa[2][4], fb[2][4];
  auto read_frags = [&](const uint8_t* base, int s, int slot) {
#pragma unroll
    for (int i = 0; i < 4; ++i) fa[slot][i] = *(const bf16x8_t*)(base + a_off[s] + i * 32 * 128);
    if constexpr (B_KC) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        fb[slot][j] = *(const bf16x8_t*)(base + bk_off[s] + j * 32 * 128);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint8_t* p = base + b_off[j] + s * 16 * 512;
        const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)p);
        const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(p + 4 * 512));
        v4s both[2] = {lo, hi};
        __builtin_memcpy(&fb[slot][j], both, 16);
      }
    }
  };
  auto mfmas = [&](int slot) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[slot][i], fb[slot][j], acc[i][j],
                                                            0, 0, 0);
  };

  // ---- main loop -------------------------------------------------------------------
  // k-step over stage `cur` (fragments of substep 0 already in slot 0):
  //   substeps 0-2: 16 MFMAs each, interleaved one-for-one with the 12
  //     fragment reads of the next substep; the 16 DMA loads of the next
  //     k-tile (into `nxt`) ride along with substep 0;
  //   then: wait for the substep-3 fragments and this wave's DMA, zero the
  //     K tail, barrier (every wave is done reading `cur`, every DMA into
  //     `nxt` has landed);
  //   substep 3: its 16 MFMAs overlap the reads of `nxt`'s first fragments.
  // On the last k-step the DMA re-reads tile 0 into the unused stage (kept
  // branch-free so it can interleave); the final wait drains it.
  // substep 0: 16 MFMAs interleaved with the 12 fragment reads of substep 1
  // and the 16 DMA loads
  auto pin_first = [&]() {
#pragma unroll
    for (int x = 0; x < 16; ++x) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    // MFMA
      if (x < 12) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);    // VMEM (DMA load)
    }
  };
  auto pin_reads = [&]() {
#pragma unroll
    for (int x = 0; x < 12; ++x) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
  };
  auto k_step = [&](uint8_t* cur, uint8_t* nxt, int kt) {
    const bool more = kt + 1 < nk;
    const int k_next = more ? (kt + 1) * BK : 0;
    // substep 0 (+ first half of the DMA), substep 1 (+ second half)
    read_frags(cur, 1, 1);
    issue(nxt, k_next);
    mfmas(0);
    pin_first();
    __builtin_amdgcn_sched_barrier(0);
    read_frags(cur, 2, 0);
    mfmas(1);
    pin_reads();
    __builtin_amdgcn_sched_barrier(0);
    read_frags(cur, 3, 1);
    mfmas(0);
    pin_reads();
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    if (more && (kt + 2) * BK > K) clear_tail(nxt, k_next);
    __syncthreads();
    // (after the last k-step these reads of the unused stage are dead;
    // keeping them unconditional avoids a branch that costs registers)
    read_frags(nxt, 0, 0);
    mfmas(1);
    pin_reads();
    __builtin_amdgcn_sched_barrier(0);
  };

  issue(smem0, 0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if (K < BK) clear_tail(smem0, 0);
  __syncthreads();
  read_frags(smem0, 0, 0);
  for (int kt = 0; kt < nk; kt += 2) {
    k_step(smem0, smem1, kt);
    if (kt + 1 < nk) k_step(smem1, smem0, kt + 1);
  }
  // a possible last DMA (into the unused stage) must land before the
  // epilogue reuses the LDS
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  // ---- epilogue ----------------------------------------------------------------------
  // phase 1: bf16(acc) into the C tile in LDS (the stages are free now)
  // (rows 0..127 in smem0, rows 128..255 in smem1: wave row wm owns one)
  {
    uint16_t* Ch = (uint16_t*)(wm ? smem1 : smem0);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int col = wn * 128 + j * 32 + (lane & 31);
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int row = i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
          Ch[row * CP + col] = vm::bf16_bits(acc[i][j][e]);
        }
      }
  }
  __syncthreads();
  // phase 2: 16-byte row chunks with the bias / residual / gate operands
  constexpr int OC = DUAL ? 128 : 256;
  constexpr int CH = OC / 8;
  uint16_t* C = (uint16_t*)g.c + b * g.c_sb;
  const uint16_t* bias = (const uint16_t*)(GROUP ? ga.bias[grp] : g.bias);
  const uint16_t* bias2 = nullptr;
  if constexpr (DUAL) bias2 = (const uint16_t*)(GROUP ? ga.bias2[grp] : g.bias2);
  const uint16_t* res = (const uint16_t*)g.res + b * g.res_sb;
  for (int t = tid; t < BM * CH; t += 256) {
    const int row = t / CH, ch = t - row * CH;
    const int64_t m = row0 + row;
    const int64_t n = n0 + ch * 8;
    if (row >= m_rows || n >= g.N) continue;
    const int lc = DUAL ? (ch >> 3) * 128 + (ch & 7) * 8 : ch * 8;
    const uint16_t* Cs = (const uint16_t*)(row >= 128 ? smem1 : smem0) + (row & 127) * CP;
    const uint4 dv = *(const uint4*)(Cs + lc);
    const uint16_t* dh = (const uint16_t*)&dv;
    uint16_t out[8];
    if constexpr (DUAL) {
      const uint4 uv = *(const uint4*)(Cs + lc + 64);
      const uint4 bg = *(const uint4*)(bias + n);
      const uint4 bu = *(const uint4*)(bias2 + n);
      const uint16_t* uh = (const uint16_t*)&uv;
      const uint16_t* bgh = (const uint16_t*)&bg;
      const uint16_t* buh = (const uint16_t*)&bu;
#pragma unroll
      for (int x = 0; x < 8; ++x) {
        // GatedFeedForward's gate, op by op in fp32 (gated_ffn.nim:46-67,
        // activation.nim:28-38)
        const float yg = vm::round_bf16(vm::as_f((uint32_t)dh[x] << 16) +
                                        vm::as_f((uint32_t)bgh[x] << 16));
        const float yu = vm::round_bf16(vm::as_f((uint32_t)uh[x] << 16) +
                                        vm::as_f((uint32_t)buh[x] << 16));
        const float e = expf(-yg);
        const float den = 1.0f + e;
        const float sig = 1.0f / den;
        const float act = yg * sig;
        out[x] = vm::bf16_bits(act * yu);
      }
    } else {
      if (g.epi == EPI_NONE) {
#pragma unroll
        for (int x = 0; x < 8; ++x) out[x] = dh[x];
      } else {
        const uint4 bv = *(const uint4*)(bias + n);
        const uint16_t* bh = (const uint16_t*)&bv;
        uint4 rv = make_uint4(0, 0, 0, 0);
        if (g.epi == EPI_BIAS_RES) rv = *(const uint4*)(res + m * g.res_sm + n);
        const uint16_t* rh = (const uint16_t*)&rv;
#pragma unroll
        for (int x = 0; x < 8; ++x) {
          float y = vm::round_bf16(vm::as_f((uint32_t)dh[x] << 16) +
                                   vm::as_f((uint32_t)bh[x] << 16));
          if (g.epi == EPI_BIAS_RES) y = vm::round_bf16(vm::as_f((uint32_t)rh[x] << 16) + y);
          out[x] = vm::bf16_bits(y);
        }
      }
    }
    *(uint4*)(C + m * g.c_sm + n) = *(const uint4*)out;
  }
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
  return true;
}

void launch_gemm_lds(const GemmArgs& g, const GroupArgs* ga, hipStream_t stream) {
  bool bkc = false;
  if (!gemm_lds_ok(g, &bkc)) fail(REW_MI355X_ERR_INVALID, "internal: gemm_lds not launchable");
  const bool dual = g.epi == EPI_SWIGLU;
  const int64_t tn = (g.N + (dual ? 127 : 255)) / (dual ? 128 : 256);
  const int64_t tiles = ga ? ga->max_mtiles * tn : ((g.M + 255) / 256) * tn * g.batch;
  if (tiles <= 0) return;
  if (tiles >= (1ll << 31)) fail(REW_MI355X_ERR_INVALID, "internal: gemm_lds grid too large");
  const GroupArgs none{};
  const GroupArgs& G = ga ? *ga : none;
  const dim3 grid((unsigned)tiles), block(256);
#define REW_LDS_LAUNCH(BKC, DU, GR) \
  hipLaunchKernelGGL((gemm_lds_kernel<BKC, DU, GR>), grid, block, 0, stream, g, G)
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

}  // namespace rew
