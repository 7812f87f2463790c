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
#include "kernels.h"
#include "vm_device.h"

namespace rew {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

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
                         vm::as_u(acc[i][j]));
      }
    }
  }
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
          if (esz == 4)
            ((float*)C)[off] = acc[i][j][e];
          else
            ((uint16_t*)C)[off] = vm::bf16_bits(acc[i][j][e]);
        }
      }
  }
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

const char* gemm_variant(const GemmArgs& g) {
  bool akc, bkc;
  if (!mfma_ok(g, &akc, &bkc)) return "gemm_generic";
  if (akc && bkc) return "gemm_bf16_mfma_tn";
  if (akc) return "gemm_bf16_mfma_nn";
  if (bkc) return "gemm_bf16_mfma_tt";
  return "gemm_bf16_mfma_nt";
}

void launch_gemm(const GemmArgs& g, hipStream_t stream) {
  if (g.M == 0 || g.N == 0 || g.batch == 0) return;
  bool akc, bkc;
  if (mfma_ok(g, &akc, &bkc)) {
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
  } else {
    dim3 grid((unsigned)((g.N + 63) / 64), (unsigned)((g.M + 63) / 64),
              (unsigned)(g.batch < 65535 ? g.batch : 65535));
    hipLaunchKernelGGL(gemm_generic_kernel, grid, dim3(256), 0, stream, g);
  }
  REW_HIP(hipGetLastError());
}

}  // namespace rew
