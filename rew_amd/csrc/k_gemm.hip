// dot_general as batched GEMM.
//
// gemm_bf16_mfma: bf16 operands, fp32 accumulation on v_mfma_f32_32x32x16_bf16.
//   Macro tile 128x128x64, 4 waves (2x2), each wave 64x64 = 2x2 MFMA tiles.
//   Both operands are staged in LDS K-contiguous ([rows][BK+8], 144-byte
//   pitch so a ds_read_b128 fragment load is bank-conflict free); an operand
//   that is M/N-contiguous in HBM (rew's [in,out] weights) is transposed in
//   registers on its way to LDS, so no transpose ever touches HBM.
//   Double-buffered: the next tile's global loads are in flight while the
//   current tile feeds the MFMAs.
// gemm_generic: any dtype / strides, 64x64x16 LDS tiles, fp32 accumulation.
#include <cstdlib>
#include <string>

#include "kernels.h"
#include "vm_device.h"

namespace rew {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

// ---- fused epilogues (see GemmArgs) -----------------------------------------

__device__ __forceinline__ float epi_rnd(int dt, float v) {
  return dt == REW_DT_BFLOAT16 ? vm::round_bf16(v) : v;
}
__device__ __forceinline__ float epi_ld(const void* p, int dt, int64_t i) {
  return dt == REW_DT_BFLOAT16 ? vm::as_f((uint32_t)((const uint16_t*)p)[i] << 16)
                               : ((const float*)p)[i];
}
__device__ __forceinline__ void epi_st(void* p, int dt, int64_t i, float v) {
  if (dt == REW_DT_BFLOAT16) ((uint16_t*)p)[i] = vm::bf16_bits(v);
  else ((float*)p)[i] = v;
}
// Value stored at C[b, m, n] for the single-GEMM epilogues.
__device__ __forceinline__ float epi_value(const GemmArgs& g, int64_t b, int64_t m, int64_t n,
                                           float acc) {
  const int dt = g.c_dtype;
  const float d = epi_rnd(dt, acc);
  if (g.epi == EPI_NONE) return d;
  const float y = epi_rnd(dt, d + epi_ld(g.bias, dt, n));
  if (g.epi == EPI_BIAS) return y;
  if (g.epi == EPI_BIAS_RELU)
    return g.relu_first ? vm::fmax_prop(y, g.relu_c) : vm::fmax_prop(g.relu_c, y);
  return epi_rnd(dt, epi_ld(g.res, dt, b * g.res_sb + m * g.res_sm + n) + y);
}
// GatedFeedForward's gate (src/rew/nn/gated_ffn.nim:46-67 with
// activation.nim:28-38), op by op in fp32.
__device__ __forceinline__ float epi_swiglu(const GemmArgs& g, int64_t n, float acc_g,
                                            float acc_u) {
  const int dt = g.c_dtype;
  const float yg = epi_rnd(dt, epi_rnd(dt, acc_g) + epi_ld(g.bias, dt, n));
  const float yu = epi_rnd(dt, epi_rnd(dt, acc_u) + epi_ld(g.bias2, dt, n));
  const float e = expf(-yg);
  const float den = 1.0f + e;
  const float sig = 1.0f / den;
  const float act = yg * sig;
  return act * yu;
}

// ---------------------------------------------------------------------------
// generic
// ---------------------------------------------------------------------------

__device__ __forceinline__ float load_as_float(const void* p, int dt, int64_t i) {
  switch (dt) {
    case REW_DT_FLOAT32: return ((const float*)p)[i];
    case REW_DT_BFLOAT16: return vm::as_f((uint32_t)((const uint16_t*)p)[i] << 16);
    case REW_DT_FLOAT16: return __half2float(((const __half*)p)[i]);
    case REW_DT_INT32: return (float)((const int32_t*)p)[i];
    default: return 0.0f;
  }
}

__global__ void __launch_bounds__(256) gemm_generic_kernel(GemmArgs g) {
  __shared__ float As[16][65];
  __shared__ float Bs[16][65];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int64_t m0 = (int64_t)blockIdx.y * 64, n0 = (int64_t)blockIdx.x * 64;
  for (int64_t b = blockIdx.z; b < g.batch; b += gridDim.z) {
    float acc[4][4] = {};
    for (int64_t k0 = 0; k0 < g.K; k0 += 16) {
      for (int i = 0; i < 4; ++i) {
        int e = threadIdx.x + i * 256;
        int mm = e >> 4, kk = e & 15;
        int64_t m = m0 + mm, k = k0 + kk;
        As[kk][mm] = (m < g.M && k < g.K)
                         ? load_as_float(g.a, g.dtype, b * g.a_sb + m * g.a_sm + k * g.a_sk)
                         : 0.0f;
        int kk2 = e >> 6, nn = e & 63;
        int64_t k2 = k0 + kk2, n = n0 + nn;
        Bs[kk2][nn] = (k2 < g.K && n < g.N)
                          ? load_as_float(g.b, g.dtype, b * g.b_sb + k2 * g.b_sk + n * g.b_sn)
                          : 0.0f;
      }
      __syncthreads();
#pragma unroll
      for (int kk = 0; kk < 16; ++kk) {
        float av[4], bv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) av[i] = As[kk][ty * 4 + i];
#pragma unroll
        for (int j = 0; j < 4; ++j) bv[j] = Bs[kk][tx * 4 + j];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
      }
      __syncthreads();
    }
    for (int i = 0; i < 4; ++i) {
      int64_t m = m0 + ty * 4 + i;
      if (m >= g.M) continue;
      for (int j = 0; j < 4; ++j) {
        int64_t n = n0 + tx * 4 + j;
        if (n >= g.N) continue;
        vm::store_scalar(g.c, g.c_dtype, b * g.c_sb + m * g.c_sm + n,
                         vm::as_u(epi_value(g, b, m, n, acc[i][j])));
      }
    }
  }
}

// Small problems (too few 64x64 tiles to occupy the GPU, e.g. the MNIST
// MLP's 128 x 784 x 128): the time is one output's k-chain plus the memory
// latency in front of it, so every thread owns one output of a 16 x 16 tile
// (sixteen times the generic kernel's workgroups).  WHOLE: the tile's whole
// A (16 x K) and B (K x 16) slabs are loaded into LDS, both k-contiguous
// (A's rows, B's columns, at a pitch of an odd number of 16-byte chunks so
// that the 16 columns' 16-byte reads hit distinct banks), then each chain
// reads four k-steps of both operands per pair of 16-byte LDS reads;
// otherwise 64-deep chunks, the next one loaded into registers while the
// current one is multiplied.
// Each output is the same sequential fmaf chain over k = 0, 1, ... with zero
// terms past K (to a multiple of 16) as gemm_generic_kernel's, so the
// kernels give the same bits.
constexpr int kSmallWholeK = 1024;  // WHOLE mode: 16-padded K up to this (129 KiB of LDS)

template <bool WHOLE>
__global__ void __launch_bounds__(256) gemm_f32_small_kernel(GemmArgs g) {
  // WHOLE: As [16][KP] then Bs [16][KP] (k-contiguous, KP = padded K + 4);
  // chunked: As [64][17] then Bs [64][17]
  extern __shared__ float sm[];
  const int tid = threadIdx.x;
  const int r = tid >> 4, cc = tid & 15;
  const int64_t m0 = (int64_t)blockIdx.y * 16, n0 = (int64_t)blockIdx.x * 16;
  const int K16 = (int)((g.K + 15) & ~15);
  const int KP = K16 + 4;
  float* As = sm;
  float* Bs = sm + (WHOLE ? 16 * KP : 64 * 17);
  for (int64_t b = blockIdx.z; b < g.batch; b += gridDim.z) {
    if constexpr (WHOLE) {
      // A slab 16 x K16: 16 threads per row; B slab K16 x 16: 4 threads per
      // k row.  f32 rows contiguous and 16-byte aligned (the usual
      // [M, K] x [K, N] layout): 16-byte loads; otherwise element loads.
      const int ra = tid >> 4, la = tid & 15, kq = tid >> 2, nq = (tid & 3) * 4;
      const int64_t ma = m0 + ra;
      const bool vec = g.dtype == REW_DT_FLOAT32 && g.a_sk == 1 && g.b_sn == 1 &&
                       g.K % 4 == 0 && g.N % 4 == 0 && g.a_sm % 4 == 0 && g.b_sk % 4 == 0 &&
                       g.a_sb % 4 == 0 && g.b_sb % 4 == 0 && ((uintptr_t)g.a & 15) == 0 &&
                       ((uintptr_t)g.b & 15) == 0;
      if (vec) {
        // A's slab moves HBM/L2 -> LDS by global_load_lds (16 bytes per lane,
        // lane-contiguous 1 KiB per instruction over the padded rows, every
        // instruction of a thread in flight at once and no VGPRs held); B's
        // goes through registers (it is transposed to k-contiguous) in two
        // batches of up to kB 16-byte loads per thread, each batch's loads
        // issued before its LDS stores.  Unconditional loads from clamped
        // addresses; the A pad [K, K16) and B's out-of-range values are
        // zeroed after.
        const int abytes = 16 * KP * 4;
        const float* a0 = (const float*)g.a + b * g.a_sb;
        for (int o = (tid >> 6) * 1024; o < abytes; o += 4096) {
          const int lo = o + (tid & 63) * 16;  // this lane's LDS byte
          const int r = lo / (KP * 4), k = (lo - r * KP * 4) >> 2;
          const int64_t m = m0 + (r < 16 ? r : 15);
          const float* src = a0 + (m < g.M ? m : g.M - 1) * g.a_sm + (k < g.K ? k : 0);
          if (lo < abytes)
            __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)((char*)As + o), 16, 0, 0);
        }
        constexpr int kB = 7;
        const int64_t nb = n0 + nq;
        const float* bp = (const float*)g.b + b * g.b_sb + (nb < g.N ? nb : 0);
        const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll 1
        for (int i0 = 0; 64 * i0 < K16; i0 += kB) {
          float4 vb[kB];
#pragma unroll
          for (int i = 0; i < kB; ++i) {
            const int kb = kq + 64 * (i0 + i);
            vb[i] = *(const float4*)(bp + (int64_t)(kb < g.K ? kb : 0) * g.b_sk);
          }
#pragma unroll
          for (int i = 0; i < kB; ++i) {
            const int kb = kq + 64 * (i0 + i);
            if (kb < K16) {
              const float4 v = (kb < g.K && nb < g.N) ? vb[i] : z;
              Bs[nq * KP + kb] = v.x;
              Bs[(nq + 1) * KP + kb] = v.y;
              Bs[(nq + 2) * KP + kb] = v.z;
              Bs[(nq + 3) * KP + kb] = v.w;
            }
          }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        // zeros where the chain runs past K (K16 > K) and in the rows past M
        for (int e = tid; e < 16 * (K16 - (int)g.K); e += 256) {
          const int r = e / (K16 - (int)g.K);
          As[r * KP + g.K + (e - r * (K16 - (int)g.K))] = 0.0f;
        }
        if (m0 + 16 > g.M)
          for (int e = tid; e < 16 * K16; e += 256) {
            const int r = e / K16;
            if (m0 + r >= g.M) As[r * KP + (e - r * K16)] = 0.0f;
          }
      } else {
        for (int k = la; k < K16; k += 16)
          As[ra * KP + k] = (ma < g.M && k < g.K)
                                ? load_as_float(g.a, g.dtype, b * g.a_sb + ma * g.a_sm + k * g.a_sk)
                                : 0.0f;
        const int nc = tid & 15;
        const int64_t n = n0 + nc;
        for (int k = tid >> 4; k < K16; k += 16)
          Bs[nc * KP + k] = (k < g.K && n < g.N)
                                ? load_as_float(g.b, g.dtype, b * g.b_sb + k * g.b_sk + n * g.b_sn)
                                : 0.0f;
      }
      __syncthreads();
      float acc = 0.0f;
      const float* ar = As + r * KP;
      const float* br = Bs + cc * KP;
#pragma unroll 4
      for (int k = 0; k < K16; k += 4) {
        const float4 av = *(const float4*)(ar + k), bv = *(const float4*)(br + k);
        acc = fmaf(av.x, bv.x, acc);
        acc = fmaf(av.y, bv.y, acc);
        acc = fmaf(av.z, bv.z, acc);
        acc = fmaf(av.w, bv.w, acc);
      }
      __syncthreads();
      const int64_t m = m0 + r, n = n0 + cc;
      if (m < g.M && n < g.N)
        vm::store_scalar(g.c, g.c_dtype, b * g.c_sb + m * g.c_sm + n,
                         vm::as_u(epi_value(g, b, m, n, acc)));
      continue;
    }
    // chunked: element e = tid + 256 i of the 16 x 64 A chunk (row e / 64,
    // k e % 64) and of the 64 x 16 B chunk (k e / 16, column e % 16)
    float pa[4], pb[4];
    auto gload = [&](int64_t k0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = tid + 256 * i;
        const int64_t m = m0 + (e >> 6), ka = k0 + (e & 63);
        pa[i] = (m < g.M && ka < g.K)
                    ? load_as_float(g.a, g.dtype, b * g.a_sb + m * g.a_sm + ka * g.a_sk)
                    : 0.0f;
        const int64_t kb = k0 + (e >> 4), n = n0 + (e & 15);
        pb[i] = (kb < g.K && n < g.N)
                    ? load_as_float(g.b, g.dtype, b * g.b_sb + kb * g.b_sk + n * g.b_sn)
                    : 0.0f;
      }
    };
    float acc = 0.0f;
    gload(0);
    for (int64_t k0 = 0; k0 < g.K; k0 += 64) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = tid + 256 * i;
        As[(e & 63) * 17 + (e >> 6)] = pa[i];
        Bs[(e >> 4) * 17 + (e & 15)] = pb[i];
      }
      __syncthreads();
      if (k0 + 64 < g.K) gload(k0 + 64);
      // the generic kernel's chain ends at the first multiple of 16 >= K
      const int kn = (g.K - k0 >= 64) ? 64 : (int)(((g.K - k0) + 15) & ~15);
      if (kn == 64) {
#pragma unroll
        for (int kk = 0; kk < 64; ++kk) acc = fmaf(As[kk * 17 + r], Bs[kk * 17 + cc], acc);
      } else {
        for (int kk = 0; kk < kn; ++kk) acc = fmaf(As[kk * 17 + r], Bs[kk * 17 + cc], acc);
      }
      __syncthreads();
    }
    const int64_t m = m0 + r, n = n0 + cc;
    if (m < g.M && n < g.N)
      vm::store_scalar(g.c, g.c_dtype, b * g.c_sb + m * g.c_sm + n,
                       vm::as_u(epi_value(g, b, m, n, acc)));
  }
}

// The smallest problems (fewer than 256 of the 16 x 16 tiles, f32 operands
// with k-contiguous A rows and n-contiguous B rows): one wave per 8 x 8
// tile, so four times the 16 x 16 kernel's workgroups, one output per lane.
// With one wave per CU the time is the wave's own instruction stream: the
// slabs' load latency, then per k-step one fma and three quarters of an LDS
// read, each stall of which the wave sits out alone.  So the slabs move in
// 256-deep k-blocks by global_load_lds (16 bytes per lane, all blocks in
// flight at once, A's eight 1 KiB row pieces and B's eight 1 KiB pieces of
// [k][8] rows per block, 16 instructions per block, clamped addresses), and
// the chain starts as soon as the first block has landed: before it reads a
// block it waits only for that block's instructions (vmcnt counts loads in
// issue order; the compiler places these waits, as each block has its own
// arrays).  Each block has its own pair of LDS arrays, A as [8][260]
// (the eight rows' 16-byte reads land on distinct banks) and B as [256][8].
// The chain reads 32 k-steps per group, the next group's reads issued before
// the current group's fmas, in two register sets that trade roles.  Rows past M and columns past N load
// clamped data whose outputs are never stored.  Each output is the same fmaf
// chain over k = 0, 1, ... as gemm_f32_small_kernel's, its zero terms past K
// (to a multiple of 16) applied in registers, so the bits agree.
constexpr int kTinyK = 1024;      // K up to this
constexpr int kTinyBlock = 256;   // k-steps per load block
constexpr int kTinyPitch = 260;   // A row pitch in LDS (floats)

typedef __attribute__((address_space(3))) float tiny_lds;
typedef float tiny_f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t tiny_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  void* p = (void*)(uintptr_t)(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(p, (short)0, (int)bytes, 0x00020000);
}

// block kb's DMA: A row rr's k = 256 kb + 4 lane .. + 3 into sa[rr][..], then
// B's k-rows 256 kb + 32 j + lane / 2 at columns n0 + 4 (lane % 2) .. + 3
// into sb[32 j + lane / 2][..]; addresses clamped into the operands
__device__ __forceinline__ void tiny_dma(const GemmArgs& g, const float* a0, const float* b0,
                                         int64_t m0, int64_t n0, int kb, tiny_lds* sa, tiny_lds* sb) {
  const int lane = threadIdx.x, K = (int)g.K;
  // byte offsets into buffer descriptors over this batch's A rows m0 ..
  // m0 + 7 and B (the operands are small: tiny_ok bounds K, and M and N
  // by the tile count)
  const int64_t ml = m0 + 7 < g.M ? m0 + 7 : g.M - 1;
  const __amdgpu_buffer_rsrc_t ra = tiny_rsrc(a0 + m0 * g.a_sm, (uint32_t)(((ml - m0) * g.a_sm + K) * 4));
  const __amdgpu_buffer_rsrc_t rb = tiny_rsrc(b0, (uint32_t)(((int64_t)(K - 1) * g.b_sk + g.N) * 4));
#pragma unroll
  for (int rr = 0; rr < 8; ++rr) {
    const int k = kb * kTinyBlock + 4 * lane;
    const int64_t m = m0 + rr < g.M ? rr : ml - m0;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (__attribute__((address_space(3))) void*)(sa + rr * kTinyPitch), 16,
                                             (uint32_t)((m * g.a_sm + (k < K ? k : 0)) * 4), 0, 0, 0);
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int k = kb * kTinyBlock + 32 * j + (lane >> 1);
    const int64_t n = n0 + (lane & 1) * 4;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (__attribute__((address_space(3))) void*)(sb + 256 * j), 16,
                                             (uint32_t)(((int64_t)(k < K ? k : 0) * g.b_sk + (n < g.N ? n : 0)) * 4), 0, 0, 0);
  }
}

// 32 k-steps from k0 of one block: A's eight 16-byte reads, B's 32 values
__device__ __forceinline__ void tiny_group_load(const tiny_lds* sa, const tiny_lds* sb, int r, int c,
                                                int k0, tiny_f4 (&a)[8], float (&b)[32]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = *(const __attribute__((address_space(3))) tiny_f4*)(sa + r * kTinyPitch + k0 + 4 * i);
#pragma unroll
  for (int i = 0; i < 32; ++i) b[i] = sb[(k0 + i) * 8 + c];
}
__device__ __forceinline__ void tiny_group_fma(float& acc, const tiny_f4 (&a)[8],
                                               const float (&b)[32]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    acc = fmaf(a[i].x, b[4 * i], acc);
    acc = fmaf(a[i].y, b[4 * i + 1], acc);
    acc = fmaf(a[i].z, b[4 * i + 2], acc);
    acc = fmaf(a[i].w, b[4 * i + 3], acc);
  }
}

// the chain over one block's ng (<= 8) 32-step groups, the next group's
// reads issued before the current group's fmas in two register sets
__device__ __forceinline__ void tiny_chain_block(const tiny_lds* sa, const tiny_lds* sb, int r, int c,
                                                 int ng, float& acc) {
  tiny_f4 a0[8], a1[8];
  float b0[32], b1[32];
  tiny_group_load(sa, sb, r, c, 0, a0, b0);
#pragma unroll
  for (int gi = 0; gi < 8; gi += 2) {
    if (gi >= ng) break;
    if (gi + 1 < ng) tiny_group_load(sa, sb, r, c, 32 * (gi + 1), a1, b1);
    tiny_group_fma(acc, a0, b0);
    if (gi + 1 >= ng) break;
    if (gi + 2 < ng) tiny_group_load(sa, sb, r, c, 32 * (gi + 2), a0, b0);
    tiny_group_fma(acc, a1, b1);
  }
}

// the k-steps from k0 to K (fewer than 32, inside one block), four at a time
__device__ __forceinline__ void tiny_chain_tail(const tiny_lds* sa, const tiny_lds* sb, int r, int c,
                                                int k0, int k1, float& acc) {
  for (int k = k0; k < k1; k += 4) {
    const tiny_f4 av = *(const __attribute__((address_space(3))) tiny_f4*)(sa + r * kTinyPitch + k);
    acc = fmaf(av.x, sb[k * 8 + c], acc);
    acc = fmaf(av.y, sb[(k + 1) * 8 + c], acc);
    acc = fmaf(av.z, sb[(k + 2) * 8 + c], acc);
    acc = fmaf(av.w, sb[(k + 3) * 8 + c], acc);
  }
}

__global__ void __launch_bounds__(64) gemm_f32_tiny_kernel(GemmArgs g) {
  // one pair of arrays per k-block, so that the compiler's waits for an LDS
  // read cover only the DMA of that read's block
  __shared__ __attribute__((aligned(16))) float ta0[8 * kTinyPitch], ta1[8 * kTinyPitch],
      ta2[8 * kTinyPitch], ta3[8 * kTinyPitch];
  __shared__ __attribute__((aligned(16))) float tb0[kTinyBlock * 8], tb1[kTinyBlock * 8],
      tb2[kTinyBlock * 8], tb3[kTinyBlock * 8];
  // LDS-typed pointers (no generic-to-LDS conversions at each use)
  tiny_lds *sa0 = (tiny_lds*)ta0, *sa1 = (tiny_lds*)ta1, *sa2 = (tiny_lds*)ta2, *sa3 = (tiny_lds*)ta3;
  tiny_lds *sb0 = (tiny_lds*)tb0, *sb1 = (tiny_lds*)tb1, *sb2 = (tiny_lds*)tb2, *sb3 = (tiny_lds*)tb3;
  const int lane = threadIdx.x;
  const int r = lane >> 3, c = lane & 7;
  const int K = (int)g.K;
  const int K16 = (K + 15) & ~15, K32 = K & ~31;
  const int nkb = (K + kTinyBlock - 1) / kTinyBlock;
  const int64_t m0 = (int64_t)blockIdx.y * 8, n0 = (int64_t)blockIdx.x * 8;
  auto ng = [&](int kb) {
    const int n = (K32 - kb * kTinyBlock) / 32;
    return n < 0 ? 0 : (n > 8 ? 8 : n);
  };
  for (int64_t b = blockIdx.z; b < g.batch; b += gridDim.z) {
    const float* a0 = (const float*)g.a + b * g.a_sb;
    const float* b0 = (const float*)g.b + b * g.b_sb;
    // all four blocks are issued whatever K is (blocks past K load clamped
    // addresses), in a fixed order with the chain: blocks 0 and 1, block 0's
    // chain, block 2, block 1's chain, block 3, then the rest.  So the
    // compiler's waits before each block's first read count exactly the DMA
    // instructions issued after that block's, and the wave's issue of the
    // later blocks (its outstanding loads are capped) overlaps the chain.
    tiny_dma(g, a0, b0, m0, n0, 0, sa0, sb0);
    tiny_dma(g, a0, b0, m0, n0, 1, sa1, sb1);
    float acc = 0.0f;
    tiny_chain_block(sa0, sb0, r, c, ng(0), acc);
    tiny_dma(g, a0, b0, m0, n0, 2, sa2, sb2);
    if (nkb > 1) tiny_chain_block(sa1, sb1, r, c, ng(1), acc);
    tiny_dma(g, a0, b0, m0, n0, 3, sa3, sb3);
    if (nkb > 2) tiny_chain_block(sa2, sb2, r, c, ng(2), acc);
    if (nkb > 3) tiny_chain_block(sa3, sb3, r, c, ng(3), acc);
    if (K32 < K) {
      // the last k-steps lie in one block
      const int kb = K32 / kTinyBlock, k0 = K32 - kb * kTinyBlock, k1 = K - kb * kTinyBlock;
      if (kb == 0) tiny_chain_tail(sa0, sb0, r, c, k0, k1, acc);
      else if (kb == 1) tiny_chain_tail(sa1, sb1, r, c, k0, k1, acc);
      else if (kb == 2) tiny_chain_tail(sa2, sb2, r, c, k0, k1, acc);
      else tiny_chain_tail(sa3, sb3, r, c, k0, k1, acc);
    }
    for (int k = K; k < K16; ++k) acc = fmaf(0.0f, 0.0f, acc);
    // every DMA landed and every read done before the next batch's loads
    __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));  // vmcnt(0)
    __syncthreads();
    const int64_t m = m0 + r, n = n0 + c;
    if (m < g.M && n < g.N)
      vm::store_scalar(g.c, g.c_dtype, b * g.c_sb + m * g.c_sm + n,
                       vm::as_u(epi_value(g, b, m, n, acc)));
  }
}

static bool tiny_ok(const GemmArgs& g) {
  const int64_t tiles16 = ((g.M + 15) / 16) * ((g.N + 15) / 16) * g.batch;
  return tiles16 < 256 && g.dtype == REW_DT_FLOAT32 && g.a_sk == 1 && g.b_sn == 1 &&
         g.K >= 4 && g.K % 4 == 0 && g.K <= kTinyK && g.N % 4 == 0 && g.a_sm % 4 == 0 &&
         g.b_sk % 4 == 0 && g.a_sb % 4 == 0 && g.b_sb % 4 == 0 &&
         ((uintptr_t)g.a & 15) == 0 && ((uintptr_t)g.b & 15) == 0;
}

static void launch_gemm_small(const GemmArgs& g, hipStream_t stream) {
  dim3 grid((unsigned)((g.N + 15) / 16), (unsigned)((g.M + 15) / 16),
            (unsigned)(g.batch < 65535 ? g.batch : 65535));
  if (tiny_ok(g)) {
    dim3 tgrid((unsigned)((g.N + 7) / 8), (unsigned)((g.M + 7) / 8),
               (unsigned)(g.batch < 65535 ? g.batch : 65535));
    hipLaunchKernelGGL(gemm_f32_tiny_kernel, tgrid, dim3(64), 0, stream, g);
    return;
  }
  const int64_t k16 = (g.K + 15) & ~(int64_t)15;
  if (k16 <= kSmallWholeK) {
    const size_t lds = (size_t)16 * (k16 + 4) * 4 * 2;
    static bool attr = [] {
      return hipFuncSetAttribute((const void*)gemm_f32_small_kernel<true>,
                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                 16 * (kSmallWholeK + 4) * 4 * 2) == hipSuccess;
    }();
    if (attr || lds <= 65536) {
      hipLaunchKernelGGL(gemm_f32_small_kernel<true>, grid, dim3(256), lds, stream, g);
      return;
    }
  }
  hipLaunchKernelGGL(gemm_f32_small_kernel<false>, grid, dim3(256), 64 * 17 * 4 * 2, stream, g);
}

// ---------------------------------------------------------------------------
// bf16 MFMA
// ---------------------------------------------------------------------------

namespace mf {
constexpr int BM = 128, BN = 128, BK = 64, LDK = BK + 8;
}

// Staging registers for one operand tile (4 x 16 bytes per thread).
struct Stage {
  uint4 v[4];
};

// K-contiguous operand: rows x BK tile, 16-byte chunks, 4 per thread.
__device__ __forceinline__ void load_kc(Stage& st, const uint16_t* base,
                                        int64_t s_row, int64_t rows_left,
                                        int64_t k0, int64_t K) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = threadIdx.x + i * 256;
    const int row = c >> 3, kc = c & 7;
    const int64_t k = k0 + kc * 8;
    if (row < rows_left && k < K)
      st.v[i] = *(const uint4*)(base + row * s_row + k);
    else
      st.v[i] = make_uint4(0, 0, 0, 0);
  }
}
__device__ __forceinline__ void store_kc(const Stage& st, uint16_t* lds) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = threadIdx.x + i * 256;
    const int row = c >> 3, kc = c & 7;
    *(uint4*)(lds + row * mf::LDK + kc * 8) = st.v[i];
  }
}

// Row-contiguous operand stored [k][row]: each thread loads a 4(k) x 8(row)
// block and writes it transposed (4 k-values per row) into the K-contiguous
// LDS tile.
__device__ __forceinline__ void load_mc(Stage& st, const uint16_t* base,
                                        int64_t s_k, int64_t rows_left,
                                        int64_t k0, int64_t K) {
  const int kb = threadIdx.x >> 4, rb = threadIdx.x & 15;
  const int row0 = rb * 8;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int64_t k = k0 + kb * 4 + t;
    if (row0 < rows_left && k < K)
      st.v[t] = *(const uint4*)(base + k * s_k + row0);
    else
      st.v[t] = make_uint4(0, 0, 0, 0);
  }
}
__device__ __forceinline__ void store_mc(const Stage& st, uint16_t* lds) {
  const int kb = threadIdx.x >> 4, rb = threadIdx.x & 15;
  const int row0 = rb * 8, kk = kb * 4;
  // st.v[t] holds rows row0..row0+7 at k = kk + t (8 bf16 = 4 dwords).
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int w = r >> 1;
    const int sh = (r & 1) * 16;
    uint32_t e0 = ((&st.v[0].x)[w] >> sh) & 0xffffu;
    uint32_t e1 = ((&st.v[1].x)[w] >> sh) & 0xffffu;
    uint32_t e2 = ((&st.v[2].x)[w] >> sh) & 0xffffu;
    uint32_t e3 = ((&st.v[3].x)[w] >> sh) & 0xffffu;
    *(uint2*)(lds + (row0 + r) * mf::LDK + kk) =
        make_uint2(e0 | (e1 << 16), e2 | (e3 << 16));
  }
}

template <bool A_KC, bool B_KC>
__global__ void __launch_bounds__(256) gemm_bf16_mfma_kernel(GemmArgs g) {
  using namespace mf;
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * LDK];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t tiles_n = (g.N + BN - 1) / BN;
  const int64_t tiles_m = (g.M + BM - 1) / BM;
  const int64_t tiles = tiles_m * tiles_n;

  for (int64_t t = blockIdx.x; t < tiles * g.batch; t += gridDim.x) {
    const int64_t b = t / tiles;
    const int64_t tt = t - b * tiles;
    const int64_t tm = tt / tiles_n, tn = tt - tm * tiles_n;
    const int64_t m0 = tm * BM, n0 = tn * BN;
    const uint16_t* A = (const uint16_t*)g.a + b * g.a_sb;
    const uint16_t* B = (const uint16_t*)g.b + b * g.b_sb;
    // Tile origins in HBM.
    const uint16_t* Abase = A_KC ? A + m0 * g.a_sm : A + m0;  // a_sm == 1 when !A_KC
    const uint16_t* Bbase = B_KC ? B + n0 * g.b_sn : B + n0;  // b_sn == 1 when !B_KC
    const int64_t m_left = g.M - m0, n_left = g.N - n0;

    f32x16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    Stage sa, sb;
    const int64_t nk = (g.K + BK - 1) / BK;
    if (A_KC) load_kc(sa, Abase, g.a_sm, m_left, 0, g.K);
    else load_mc(sa, Abase, g.a_sk, m_left, 0, g.K);
    if (B_KC) load_kc(sb, Bbase, g.b_sn, n_left, 0, g.K);
    else load_mc(sb, Bbase, g.b_sk, n_left, 0, g.K);
    if (A_KC) store_kc(sa, As[0]); else store_mc(sa, As[0]);
    if (B_KC) store_kc(sb, Bs[0]); else store_mc(sb, Bs[0]);
    __syncthreads();

    for (int64_t kt = 0; kt < nk; ++kt) {
      const int cur = (int)(kt & 1);
      const bool more = kt + 1 < nk;
      if (more) {
        const int64_t k0 = (kt + 1) * BK;
        if (A_KC) load_kc(sa, Abase, g.a_sm, m_left, k0, g.K);
        else load_mc(sa, Abase, g.a_sk, m_left, k0, g.K);
        if (B_KC) load_kc(sb, Bbase, g.b_sn, n_left, k0, g.K);
        else load_mc(sb, Bbase, g.b_sk, n_left, k0, g.K);
      }
      const uint16_t* as = As[cur];
      const uint16_t* bs = Bs[cur];
#pragma unroll
      for (int s = 0; s < BK / 16; ++s) {
        bf16x8_t af[2], bfr[2];
        const int koff = s * 16 + (lane >> 5) * 8;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int row = wm * 64 + i * 32 + (lane & 31);
          af[i] = *(const bf16x8_t*)(as + row * LDK + koff);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int col = wn * 64 + j * 32 + (lane & 31);
          bfr[j] = *(const bf16x8_t*)(bs + col * LDK + koff);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j],
                                                                acc[i][j], 0, 0, 0);
      }
      if (more) {
        if (A_KC) store_kc(sa, As[cur ^ 1]); else store_mc(sa, As[cur ^ 1]);
        if (B_KC) store_kc(sb, Bs[cur ^ 1]); else store_mc(sb, Bs[cur ^ 1]);
      }
      __syncthreads();
    }

    // Epilogue: lane holds column (lane & 31) of each 32x32 tile, rows
    // (e/4)*8 + (lane/32)*4 + e%4.
    char* C = (char*)g.c;
    const int esz = g.c_dtype == REW_DT_FLOAT32 ? 4 : 2;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int64_t n = n0 + wn * 64 + j * 32 + (lane & 31);
        if (n >= g.N) continue;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int64_t m = m0 + wm * 64 + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
          if (m >= g.M) continue;
          const int64_t off = b * g.c_sb + m * g.c_sm + n;
          const float v = epi_value(g, b, m, n, acc[i][j][e]);
          if (esz == 4)
            ((float*)C)[off] = v;
          else
            ((uint16_t*)C)[off] = vm::bf16_bits(v);
        }
      }
  }
}

// ---------------------------------------------------------------------------
// bf16 MFMA, large tiles: 256x256x64 per workgroup, 4 waves of 128x128
// ---------------------------------------------------------------------------
//
// Each wave owns a 128x128 block of C as 4x4 v_mfma_f32_32x32x16_bf16 tiles
// (256 fp32 accumulators per lane), so one 16-byte LDS fragment read feeds
// four MFMAs.  Operands are read with buffer loads (one scalar resource per
// operand, one VGPR offset per lane; rows past the tile's extent come back
// as zeros from the hardware range check).  A (K-contiguous rows) is staged
// as 16-byte chunks; B is staged K-contiguous per output column: when it is
// N-contiguous in HBM (rew's [in, out] Linear weights) each thread loads an
// 8(k) x 8(n) block (8 lanes = 8 k-blocks of one n-block: full 128-byte
// lines) and transposes it in registers; those 8 lanes then write 8
// different 16-byte chunks of LDS banks, so the 144-byte row pitch keeps both
// the writes and the fragment reads conflict-free.  A of the next k-tile is
// in flight during the first half of the MFMAs, B during the second half.
// Tiles are ordered so each XCD (every 8th workgroup) walks a contiguous,
// row-grouped range of C, keeping the A rows and B columns its 32 CUs share
// resident in its L2.

namespace mf2 {
constexpr int BM = 256, BN = 256, BK = 64, LDK = BK + 8;
constexpr int GROUP_M = 4;
}  // namespace mf2

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  // dword3 0x00020000: raw 32-bit buffer on gfx9 (CDNA)
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  auto x = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  uint4 v;
  __builtin_memcpy(&v, &x, 16);
  return v;
}

__device__ __forceinline__ void tile_of(int64_t bid, int64_t tiles_m, int64_t tiles_n,
                                        int64_t batch, int64_t* b, int64_t* tm, int64_t* tn) {
  const int64_t per = tiles_m * tiles_n;
  const int64_t total = per * batch;
  int64_t t = bid;
  if (total % 8 == 0) t = (bid % 8) * (total / 8) + bid / 8;  // XCD-contiguous ranges
  *b = t / per;
  t -= *b * per;
  const int64_t group = mf2::GROUP_M * tiles_n;
  const int64_t first_m = (t / group) * mf2::GROUP_M;
  const int64_t gsize = min((int64_t)mf2::GROUP_M, tiles_m - first_m);
  const int64_t r = t % group;
  *tm = first_m + r % gsize;
  *tn = r / gsize;
}

// DUAL (EPI_SWIGLU): the workgroup covers 128 output columns of two GEMMs
// sharing A; wave column wn holds gate columns n0 + wn*64 + [0, 64) in its
// accumulator columns j = 0, 1 and the same up-projection columns in
// j = 2, 3, so the SwiGLU epilogue is lane-local.
// GROUP: grouped mode (see GroupArgs): the tile's group, packed rows and
// operand pointers come from the group tables instead of the batch index.
template <bool B_KC, bool DUAL, bool GROUP>
__global__ void __launch_bounds__(256, 1) gemm_bf16_256_kernel(GemmArgs g, GroupArgs ga) {
  using namespace mf2;
  // operand double buffers; after the main loop the same memory holds the
  // rounded C tile for the epilogue pass
  constexpr int CP = 256 + 8;  // C tile row pitch (elements)
  static_assert(BM * CP <= 2 * (BM + BN) * LDK, "C tile must fit the operand buffers");
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * (BM + BN) * LDK];
  uint16_t (*As)[BM * LDK] = reinterpret_cast<uint16_t (*)[BM * LDK]>(smem);
  uint16_t (*Bs)[BN * LDK] = reinterpret_cast<uint16_t (*)[BN * LDK]>(smem + 2 * BM * LDK);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  constexpr int TN = DUAL ? BN / 2 : BN;  // output columns per workgroup
  const int64_t tiles_n = (g.N + TN - 1) / TN;
  int64_t b = 0, tm = 0, tn = 0;
  int64_t m_rows;     // valid rows of the tile
  int64_t row0;       // C row (dense: of the batch matrix; grouped: packed) of tile row 0
  int grp = 0;
  if constexpr (GROUP) {
    const int64_t total = ga.max_mtiles * tiles_n;
    int64_t t = blockIdx.x;
    if (total % 8 == 0) t = (t % 8) * (total / 8) + t / 8;  // XCD-contiguous ranges
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
    // (a small group's tiles hold group_tile_rows rows, the rest unused)
    const int tr = group_tile_rows(ga.off[grp + 1] - ga.off[grp]);
    row0 = ga.off[grp] + (tm - ga.mt_start[grp]) * tr;
    m_rows = min((int64_t)tr, (int64_t)ga.off[grp + 1] - row0);
  } else {
    const int64_t tiles_m = (g.M + BM - 1) / BM;
    tile_of(blockIdx.x, tiles_m, tiles_n, g.batch, &b, &tm, &tn);
    row0 = tm * BM;
    m_rows = min((int64_t)BM, g.M - row0);
  }
  const int64_t n0 = tn * TN;
  const int64_t n_rows = min((int64_t)BN, g.N - n0);
  const int K = (int)g.K;
  const bool gather = GROUP && ga.rows != nullptr;

  // A: rows row0 .. row0 + m_rows (K-contiguous), or the whole token
  // matrix when the rows are gathered
  const uint16_t* Ab = gather ? (const uint16_t*)g.a
                              : (const uint16_t*)g.a + b * g.a_sb + row0 * g.a_sm;
  const __amdgpu_buffer_rsrc_t ra =
      make_rsrc(Ab, (uint32_t)((((gather ? g.M : m_rows) - 1) * g.a_sm + K) * 2));
  const uint32_t a_sm2 = (uint32_t)(g.a_sm * 2);
  // B: K-contiguous rows n0.. (B_KC) or the whole [K, N] batch matrix
  const uint16_t* Bw = GROUP ? (const uint16_t*)ga.b[grp] : (const uint16_t*)g.b + b * g.b_sb;
  const uint16_t* Bb = B_KC ? Bw + n0 * g.b_sn : Bw;
  const uint32_t b_bytes = B_KC ? (uint32_t)(((n_rows - 1) * g.b_sn + K) * 2)
                                : (uint32_t)(((g.K - 1) * g.b_sk + g.N) * 2);
  // DUAL: odd waves stage the up-projection weights (wave-uniform choice)
  const uint16_t* Bw2 = GROUP ? (const uint16_t*)(DUAL ? ga.b2[grp] : nullptr)
                              : (const uint16_t*)g.b2 + b * g.b_sb;
  const uint16_t* Bsrc = (DUAL && (wave & 1)) ? Bw2 : Bb;
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(Bsrc, b_bytes);
  const uint32_t b_s2 = (uint32_t)((B_KC ? g.b_sn : g.b_sk) * 2);

  // per-lane parts of the staging addresses
  const int row8 = tid >> 3, kc = tid & 7;             // A / B_KC: 16-byte chunk kc of row
  const uint32_t a_voff = row8 * a_sm2 + kc * 16;
  // gathered A: byte offset of each of the lane's 8 rows (rows past the
  // tile's extent point past the buffer and read as zeros)
  uint32_t a_gv[GROUP ? 8 : 1];
  if constexpr (GROUP) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = row8 + i * 32;
      a_gv[i] = (gather && r < m_rows)
                    ? (uint32_t)ga.rows[row0 + r] * a_sm2 + kc * 16
                    : 0x80000000u;
    }
  }
  const int nb = tid >> 3, kb = tid & 7;               // !B_KC: 8x8 block (k-block kb, n-block nb)
  // DUAL: virtual column block nb maps to column n0 + (nb >> 4) * 64 + (nb & 7) * 8
  const int64_t bcol = DUAL ? n0 + (nb >> 4) * 64 + (nb & 7) * 8 : n0 + nb * 8;
  const uint32_t bt_voff = B_KC ? row8 * b_s2 + kc * 16
                                : (kb * 8) * b_s2 + (uint32_t)(bcol * 2);

  uint4 rs[8];
  // K-tail lanes are zeroed when the chunk is written to LDS, not at load
  // time, so the loads stay in flight across the MFMAs.
  bool kok_a = true;
  auto load_a = [&](int k0) {
    kok_a = k0 + kc * 8 < K;
    if (gather) {
#pragma unroll
      for (int i = 0; i < 8; ++i) rs[i] = bload16(ra, a_gv[GROUP ? i : 0], (uint32_t)k0 * 2);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        rs[i] = bload16(ra, a_voff, (uint32_t)(i * 32) * a_sm2 + (uint32_t)k0 * 2);
    }
  };
  auto store_a = [&](int buf) {
    uint16_t* as = As[buf] + row8 * LDK + kc * 8;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      *(uint4*)(as + i * 32 * LDK) = kok_a ? rs[i] : make_uint4(0, 0, 0, 0);
  };
  bool kok_b = true;
  auto load_b = [&](int k0) {
    if (B_KC) {
      kok_b = k0 + kc * 8 < K;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        rs[i] = bload16(rb, bt_voff, (uint32_t)(i * 32) * b_s2 + (uint32_t)k0 * 2);
    } else {
      // rows k >= K fall past the resource's extent and read as zeros
#pragma unroll
      for (int r = 0; r < 8; ++r) rs[r] = bload16(rb, bt_voff, (uint32_t)(k0 + r) * b_s2);
    }
  };
  auto store_b = [&](int buf) {
    if (B_KC) {
      uint16_t* bs = Bs[buf] + row8 * LDK + kc * 8;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        *(uint4*)(bs + i * 32 * LDK) = kok_b ? rs[i] : make_uint4(0, 0, 0, 0);
    } else {
      uint16_t* bs = Bs[buf] + (nb * 8) * LDK + kb * 8;
#pragma unroll
      for (int nn = 0; nn < 8; ++nn) {
        const int w = nn >> 1;
        uint32_t o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t x = (&rs[2 * j].x)[w], y = (&rs[2 * j + 1].x)[w];
          o[j] = (nn & 1) ? ((x >> 16) | (y & 0xffff0000u)) : ((x & 0xffffu) | (y << 16));
        }
        *(uint4*)(bs + nn * LDK) = make_uint4(o[0], o[1], o[2], o[3]);
      }
    }
  };

  f32x16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  const int frag_a = (wm * 128 + (lane & 31)) * LDK + (lane >> 5) * 8;
  const int frag_b = (wn * 128 + (lane & 31)) * LDK + (lane >> 5) * 8;
  // Fragments of substep s + 1 are read while the 16 MFMAs of substep s run.
  bf16x8_t fa[2][4], fb[2][4];
  auto read_frags = [&](const uint16_t* as, const uint16_t* bs, int s, int slot) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      fa[slot][i] = *(const bf16x8_t*)(as + frag_a + i * 32 * LDK + s * 16);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      fb[slot][j] = *(const bf16x8_t*)(bs + frag_b + j * 32 * LDK + s * 16);
  };
  auto mfmas = [&](int slot) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[slot][i], fb[slot][j],
                                                            acc[i][j], 0, 0, 0);
  };

  // One scheduling region per k-substep: the 8 fragment reads of the next
  // substep are interleaved one-for-one with the first 8 of the 16 MFMAs of
  // this one, so LDS latency hides under the matrix pipe.
  auto pin = [&]() {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
  };

  const int nk = (K + BK - 1) / BK;
  load_a(0);
  store_a(0);
  load_b(0);
  store_b(0);
  __syncthreads();
  read_frags(As[0], Bs[0], 0, 0);
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    const uint16_t* as = As[cur];
    const uint16_t* bs = Bs[cur];
    if (more) load_a((kt + 1) * BK);
    __builtin_amdgcn_sched_barrier(0);
    read_frags(as, bs, 1, 1);
    mfmas(0);
    pin();
    __builtin_amdgcn_sched_barrier(0);
    read_frags(as, bs, 2, 0);
    mfmas(1);
    pin();
    __builtin_amdgcn_sched_barrier(0);
    if (more) {
      store_a(cur ^ 1);
      load_b((kt + 1) * BK);
    }
    __builtin_amdgcn_sched_barrier(0);
    read_frags(as, bs, 3, 1);
    mfmas(0);
    pin();
    __builtin_amdgcn_sched_barrier(0);
    mfmas(1);
    if (more) store_b(cur ^ 1);
    __syncthreads();
    if (more) read_frags(As[cur ^ 1], Bs[cur ^ 1], 0, 0);
  }

  // Epilogue, phase 1: every lane writes bf16(acc) of its fragments into
  // the C tile in LDS (the operand buffers are free after the last barrier).
  uint16_t* Cs = smem;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = wn * 128 + j * 32 + (lane & 31);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = wm * 128 + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
        Cs[row * CP + col] = vm::bf16_bits(acc[i][j][e]);
      }
    }
  __syncthreads();
  // Phase 2: row-major pass, 8 output columns (16 bytes) per thread and
  // step, with the bias / residual / up-projection operands read coalesced.
  const int OC = DUAL ? 128 : 256;           // output columns of the tile
  const int CH = OC / 8;                     // 16-byte chunks per row
  uint16_t* C = (uint16_t*)g.c + b * g.c_sb;
  const uint16_t* bias = (const uint16_t*)(GROUP ? ga.bias[grp] : g.bias);
  const uint16_t* bias2 = (const uint16_t*)(GROUP ? (DUAL ? ga.bias2[grp] : nullptr) : g.bias2);
  const uint16_t* res = (const uint16_t*)g.res + b * g.res_sb;
  for (int t = tid; t < BM * CH; t += 256) {
    const int row = t / CH, ch = t - row * CH;
    const int64_t m = row0 + row;
    const int64_t n = n0 + ch * 8;
    if (row >= m_rows || n >= g.N) continue;
    // local column of the value (gate column for DUAL)
    const int lc = DUAL ? (ch >> 3) * 128 + (ch & 7) * 8 : ch * 8;
    const uint4 dv = *(const uint4*)(Cs + row * CP + lc);
    const uint16_t* dh = (const uint16_t*)&dv;
    uint16_t out[8];
    if (DUAL) {
      const uint4 uv = *(const uint4*)(Cs + row * CP + lc + 64);
      const uint4 bg = *(const uint4*)(bias + n);
      const uint4 bu = *(const uint4*)(bias2 + n);
      const uint16_t* uh = (const uint16_t*)&uv;
      const uint16_t* bgh = (const uint16_t*)&bg;
      const uint16_t* buh = (const uint16_t*)&bu;
#pragma unroll
      for (int x = 0; x < 8; ++x) {
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
    } else if (g.epi == EPI_NONE) {
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
    *(uint4*)(C + m * g.c_sm + n) = *(const uint4*)out;
  }
}

// f32 GEMM with a narrow output (N <= 64, N % 4 == 0; a router's
// [T, H] x [H, E]): 16-row tiles, so M / 16 workgroups where the generic
// kernel's 64 x 64 tiles give M / 64 and leave most of the chip idle.  The
// k-steps are 32 deep, loaded as 16-byte vectors into two register sets in
// turn, so each load has two k-steps to land.  Every output is a sequential
// fmaf chain over k = 0, 1, ..., K - 1 from 0, as in gemm_generic_kernel, so
// the two kernels give the same bits.  Thread t computes row t / 16, columns
// 4 (t % 16) .. + 3; columns past N read an in-range chunk and are not stored.
__global__ void __launch_bounds__(256) gemm_f32_narrow_kernel(GemmArgs g) {
  // Bs is read and written as float4: both arrays are declared 16-byte
  // aligned rather than relying on where the compiler places them
  __shared__ __attribute__((aligned(16))) float As[32][17];  // [k][row]
  __shared__ __attribute__((aligned(16))) float Bs[32][64];  // [k][column]
  const int tid = threadIdx.x;
  const int r = tid >> 4, c4 = (tid & 15) * 4;
  const int64_t m0 = (int64_t)blockIdx.x * 16;
  const float* A = (const float*)g.a;
  const float* B = (const float*)g.b;
  // loaders: A, 16 rows x 32 k (threads 0..127, one 16-byte chunk each);
  // B, 32 k x 64 columns (two chunks per thread, k rows bk and bk + 16)
  const int ar = (tid >> 3) & 15, ak = (tid & 7) * 4;
  const float* ap = A + (m0 + ar < g.M ? m0 + ar : g.M - 1) * g.a_sm + ak;
  const int bk = tid >> 4;
  const int64_t bcol = c4 < g.N ? c4 : g.N - 4;
  const float* bp = B + bk * g.b_sk + bcol;
  const int64_t b16 = 16 * g.b_sk;
  // two register sets (named, not indexed: an indexed array went to scratch)
  float4 pa0 = make_float4(0, 0, 0, 0), pa1 = pa0, pb00, pb01, pb10, pb11;
  auto gload = [&](float4& pa, float4& pb0, float4& pb1, int64_t k0) {
    if (tid < 128) pa = *(const float4*)(ap + k0);
    pb0 = *(const float4*)(bp + k0 * g.b_sk);
    pb1 = *(const float4*)(bp + k0 * g.b_sk + b16);
  };
  auto sstore = [&](const float4& pa, const float4& pb0, const float4& pb1) {
    if (tid < 128) {
      As[ak][ar] = pa.x;
      As[ak + 1][ar] = pa.y;
      As[ak + 2][ar] = pa.z;
      As[ak + 3][ar] = pa.w;
    }
    *(float4*)&Bs[bk][c4] = pb0;
    *(float4*)&Bs[bk + 16][c4] = pb1;
  };
  float acc0 = 0.0f, acc1 = 0.0f, acc2 = 0.0f, acc3 = 0.0f;
  auto step = [&]() {
#pragma unroll 8
    for (int kk = 0; kk < 32; ++kk) {
      const float a = As[kk][r];
      const float4 b = *(const float4*)&Bs[kk][c4];
      acc0 = fmaf(a, b.x, acc0);
      acc1 = fmaf(a, b.y, acc1);
      acc2 = fmaf(a, b.z, acc2);
      acc3 = fmaf(a, b.w, acc3);
    }
  };
  // K % 64 == 0: the k-steps come in pairs, set 0 then set 1
  gload(pa0, pb00, pb01, 0);
  gload(pa1, pb10, pb11, 32);
  for (int64_t k0 = 0; k0 < g.K; k0 += 64) {
    sstore(pa0, pb00, pb01);
    __syncthreads();
    if (k0 + 64 < g.K) gload(pa0, pb00, pb01, k0 + 64);
    step();
    __syncthreads();
    sstore(pa1, pb10, pb11);
    __syncthreads();
    if (k0 + 96 < g.K) gload(pa1, pb10, pb11, k0 + 96);
    step();
    __syncthreads();
  }
  const int64_t m = m0 + r;
  if (m >= g.M) return;
  const float accs[4] = {acc0, acc1, acc2, acc3};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t n = c4 + j;
    if (n < g.N)
      vm::store_scalar(g.c, g.c_dtype, m * g.c_sm + n, vm::as_u(epi_value(g, 0, m, n, accs[j])));
  }
}

static bool f32_narrow_ok(const GemmArgs& g) {
  return g.dtype == REW_DT_FLOAT32 && g.batch == 1 && g.M >= 1 && g.N >= 4 && g.N <= 64 &&
         g.N % 4 == 0 && g.K >= 64 && g.K % 64 == 0 && g.a_sk == 1 && g.b_sn == 1 &&
         g.a_sm % 4 == 0 && g.b_sk % 4 == 0 && ((uintptr_t)g.a & 15) == 0 &&
         ((uintptr_t)g.b & 15) == 0 && (g.epi == EPI_NONE || g.epi == EPI_BIAS) &&
         g.M / 16 < (1 << 30);
}

// Problems whose 64x64 tiles would leave most CUs idle run 16x16 tiles.
static bool small_ok(const GemmArgs& g) {
  const int64_t tiles64 = ((g.M + 63) / 64) * ((g.N + 63) / 64) * g.batch;
  return tiles64 < 128 && g.epi != EPI_SWIGLU && g.epi != EPI_BIAS_ROPE;
}

static bool mfma_ok(const GemmArgs& g, bool* a_kc, bool* b_kc) {
  if (g.dtype != REW_DT_BFLOAT16) return false;
  if (g.c_dtype != REW_DT_BFLOAT16 && g.c_dtype != REW_DT_FLOAT32) return false;
  if (g.K % 8 != 0) return false;
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  if (!al16(g.a) || !al16(g.b)) return false;
  // A: K-contiguous rows (a_sk == 1) or M-contiguous (a_sm == 1).
  if (g.a_sk == 1 && g.a_sm % 8 == 0 && g.a_sb % 8 == 0) *a_kc = true;
  else if (g.a_sm == 1 && g.a_sk % 8 == 0 && g.a_sb % 8 == 0 && g.M % 8 == 0) *a_kc = false;
  else return false;
  if (g.b_sk == 1 && g.b_sn % 8 == 0 && g.b_sb % 8 == 0) *b_kc = true;
  else if (g.b_sn == 1 && g.b_sk % 8 == 0 && g.b_sb % 8 == 0 && g.N % 8 == 0) *b_kc = false;
  else return false;
  return true;
}

// The 256x256 kernel needs K-contiguous A and enough tiles to fill the
// 256 CUs at least once; smaller problems run the 128x128 kernel.
// REW_MI355X_GEMM_TILE=256 / 128 forces a kernel (tests use it to cover
// the large-tile kernel's tails at small sizes); unset picks by size.
// REW_MI355X_GEMM_TILE: "lds" (the direct-to-LDS kernels), "256" or "128".
static int forced_tile() {
  static const int v = [] {
    const char* s = std::getenv("REW_MI355X_GEMM_TILE");
    if (s && std::string(s) == "lds") return 1;
    return s ? std::atoi(s) : 0;
  }();
  return v;
}

// The direct-to-LDS kernels run every bf16 GEMM they support once it has
// enough 256x256 tiles to occupy most of the 256 CUs (or when forced).
static bool use_lds(const GemmArgs& g) {
  bool bkc;
  const int f = forced_tile();
  if (f == 128 || f == 256 || !gemm_lds_ok(g, &bkc)) return false;
  const bool dual = g.epi == EPI_SWIGLU;
  const int64_t tiles = ((g.M + 255) / 256) * ((g.N + (dual ? 127 : 255)) / (dual ? 128 : 256)) *
                        g.batch;
  return f == 1 || tiles >= 96;
}

// The epilogue pass of the 256 kernels writes 16-byte chunks of bf16 rows.
static bool epi256_ok(const GemmArgs& g) {
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  if (g.c_dtype != REW_DT_BFLOAT16 || g.N % 8 || g.c_sm % 8 || g.c_sb % 8 || !al16(g.c))
    return false;
  if (g.epi != EPI_NONE && !al16(g.bias)) return false;
  if (g.epi == EPI_SWIGLU && !al16(g.bias2)) return false;
  if (g.epi == EPI_BIAS_RES && (!al16(g.res) || g.res_sm % 8 || g.res_sb % 8)) return false;
  return true;
}

static bool use_256(const GemmArgs& g, bool akc) {
  if (!akc || forced_tile() == 128 || !epi256_ok(g)) return false;
  const int64_t tiles = ((g.M + 255) / 256) * ((g.N + 255) / 256) * g.batch;
  if ((tiles < 256 && forced_tile() != 256) || tiles >= (1ll << 31)) return false;
  // buffer offsets are 32-bit: every operand extent a tile addresses < 2 GiB
  bool bkc = g.b_sk == 1;
  const int64_t a_ext = (256 * g.a_sm + g.K) * 2;
  const int64_t b_ext = bkc ? (256 * g.b_sn + g.K) * 2 : (g.K * g.b_sk + g.N) * 2;
  return a_ext < (1ll << 31) && b_ext < (1ll << 31);
}

bool gemm_epilogue_ok(const GemmArgs& g) {
  if (g.epi == EPI_NONE) return true;
  if (g.epi == EPI_BIAS_ROPE) return false;  // launch_gemm_multi only
  bool akc0, bkc0;
  if (g.epi == EPI_BIAS_RELU)  // the f32 kernels only (generic / small)
    return g.c_dtype == REW_DT_FLOAT32 && !mfma_ok(g, &akc0, &bkc0) && !use_lds(g);
  if (g.c_dtype != REW_DT_BFLOAT16 && g.c_dtype != REW_DT_FLOAT32) return false;
  if (g.epi != EPI_SWIGLU) return true;
  bool lkc;
  if (gemm_lds_ok(g, &lkc)) return true;
  bool akc, bkc;
  if (!mfma_ok(g, &akc, &bkc) || !akc || bkc || !epi256_ok(g)) return false;
  const int64_t a_ext = (256 * g.a_sm + g.K) * 2;
  const int64_t b_ext = (g.K * g.b_sk + g.N) * 2;
  return a_ext < (1ll << 31) && b_ext < (1ll << 31) && ((uintptr_t)g.b2 & 15) == 0;
}

const char* gemm_variant(const GemmArgs& g) {
  bool akc, bkc;
  if (use_lds(g)) {
    gemm_lds_ok(g, &bkc);
    return g.epi == EPI_SWIGLU ? "gemm_lds_swiglu" : (bkc ? "gemm_lds_tn" : "gemm_lds_nn");
  }
  if (g.epi == EPI_SWIGLU) return "gemm_bf16_256_swiglu";
  if (!mfma_ok(g, &akc, &bkc))
    return f32_narrow_ok(g) ? "gemm_f32_narrow" : (small_ok(g) ? "gemm_f32_small" : "gemm_generic");
  if (use_256(g, akc)) return bkc ? "gemm_bf16_256_tn" : "gemm_bf16_256_nn";
  if (akc && bkc) return "gemm_bf16_mfma_tn";
  if (akc) return "gemm_bf16_mfma_nn";
  if (bkc) return "gemm_bf16_mfma_tt";
  return "gemm_bf16_mfma_nt";
}

void launch_gemm(const GemmArgs& g, hipStream_t stream) {
  if (g.M == 0 || g.N == 0 || g.batch == 0) return;
  bool akc, bkc;
  if (use_lds(g)) {
    launch_gemm_lds(g, nullptr, stream);
    return;
  }
  if (g.epi == EPI_SWIGLU) {
    if (!gemm_epilogue_ok(g)) fail(REW_MI355X_ERR_INVALID, "internal: SwiGLU GEMM not launchable");
    const int64_t tiles = ((g.M + 255) / 256) * ((g.N + 127) / 128) * g.batch;
    hipLaunchKernelGGL((gemm_bf16_256_kernel<false, true, false>), dim3((unsigned)tiles),
                       dim3(256), 0, stream, g, GroupArgs{});
  } else if (mfma_ok(g, &akc, &bkc) && use_256(g, akc)) {
    const int64_t tiles = ((g.M + 255) / 256) * ((g.N + 255) / 256) * g.batch;
    if (bkc)
      hipLaunchKernelGGL((gemm_bf16_256_kernel<true, false, false>), dim3((unsigned)tiles),
                         dim3(256), 0, stream, g, GroupArgs{});
    else
      hipLaunchKernelGGL((gemm_bf16_256_kernel<false, false, false>), dim3((unsigned)tiles),
                         dim3(256), 0, stream, g, GroupArgs{});
  } else if (mfma_ok(g, &akc, &bkc)) {
    const int64_t tiles = ((g.M + 127) / 128) * ((g.N + 127) / 128) * g.batch;
    const unsigned grid = (unsigned)(tiles < 1 << 20 ? tiles : 1 << 20);
    if (akc && bkc)
      hipLaunchKernelGGL((gemm_bf16_mfma_kernel<true, true>), dim3(grid), dim3(256), 0, stream, g);
    else if (akc)
      hipLaunchKernelGGL((gemm_bf16_mfma_kernel<true, false>), dim3(grid), dim3(256), 0, stream, g);
    else if (bkc)
      hipLaunchKernelGGL((gemm_bf16_mfma_kernel<false, true>), dim3(grid), dim3(256), 0, stream, g);
    else
      hipLaunchKernelGGL((gemm_bf16_mfma_kernel<false, false>), dim3(grid), dim3(256), 0, stream, g);
  } else if (f32_narrow_ok(g)) {
    hipLaunchKernelGGL(gemm_f32_narrow_kernel, dim3((unsigned)((g.M + 15) / 16)), dim3(256), 0,
                       stream, g);
  } else if (small_ok(g)) {
    launch_gemm_small(g, stream);
  } else {
    dim3 grid((unsigned)((g.N + 63) / 64), (unsigned)((g.M + 63) / 64),
              (unsigned)(g.batch < 65535 ? g.batch : 65535));
    hipLaunchKernelGGL(gemm_generic_kernel, grid, dim3(256), 0, stream, g);
  }
  REW_HIP(hipGetLastError());
}

bool gemm_grouped_ok(const GemmArgs& g) {
  bool lkc;
  if (forced_tile() != 256 && gemm_lds_ok(g, &lkc) && g.batch == 1 &&
      (g.epi == EPI_BIAS || g.epi == EPI_SWIGLU))
    return true;
  bool akc, bkc;
  if (!mfma_ok(g, &akc, &bkc) || !akc || bkc || g.batch != 1) return false;
  if (g.epi != EPI_BIAS && g.epi != EPI_SWIGLU) return false;
  if (g.c_dtype != REW_DT_BFLOAT16 || g.N % 8 || g.c_sm % 8 || ((uintptr_t)g.c & 15)) return false;
  const int64_t a_ext = ((g.M - 1) * g.a_sm + g.K) * 2;
  const int64_t b_ext = ((g.K - 1) * g.b_sk + g.N) * 2;
  return a_ext < (1ll << 31) && b_ext < (1ll << 31);
}

void launch_gemm_grouped(const GemmArgs& g, const GroupArgs& ga, hipStream_t stream) {
  if (ga.n_groups <= 0 || ga.max_mtiles <= 0 || g.N == 0) return;
  if (!gemm_grouped_ok(g)) fail(REW_MI355X_ERR_INVALID, "internal: grouped GEMM not launchable");
  bool lkc;
  if (forced_tile() != 256 && gemm_lds_ok(g, &lkc)) {
    launch_gemm_lds(g, &ga, stream);
    return;
  }
  const bool dual = g.epi == EPI_SWIGLU;
  const int64_t tiles = ga.max_mtiles * ((g.N + (dual ? 127 : 255)) / (dual ? 128 : 256));
  if (tiles >= (1ll << 31)) fail(REW_MI355X_ERR_INVALID, "internal: grouped GEMM grid too large");
  if (dual)
    hipLaunchKernelGGL((gemm_bf16_256_kernel<false, true, true>), dim3((unsigned)tiles),
                       dim3(256), 0, stream, g, ga);
  else
    hipLaunchKernelGGL((gemm_bf16_256_kernel<false, false, true>), dim3((unsigned)tiles),
                       dim3(256), 0, stream, g, ga);
  REW_HIP(hipGetLastError());
}

}  // namespace rew
