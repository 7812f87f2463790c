// Row-wise composites of rew's nn layers as single HBM passes.
//
// rmsnorm_rows: rew's rmsNorm (src/rew/nn/norm.nim:204-224) over the last
//   axis, op by op in fp32:
//     s = sum_j x_j * x_j;  r = sqrt(s / n + eps);  y_j = gamma_j * (x_j / r)
//   One workgroup per row; the row is read once into registers (up to
//   kRowRegs elements per thread, re-read from L2 beyond that), reduced with
//   a wave64 butterfly and an LDS step across the 4 waves.  The input may be
//   bf16 (the astype to fp32 in front of the norm happens on load) and the
//   output bf16 (the astype behind it happens on store).
//
// rope_pairs: rew's applyRotate (src/rew/nn/rope.nim:56-108) on adjacent
//   pairs (2i, 2i+1) of the last axis:
//     y_2i   = c_i * x_2i - s_i * x_2i+1
//     y_2i+1 = s_i * x_2i + c_i * x_2i+1
//   with c / s read through their broadcast views of the fp32 tables, each
//   product and sum rounded to fp32 as the separate eager ops are.  Four
//   pairs (16 bytes of bf16) per thread.
#include "kernels.h"
#include "vm_device.h"

namespace rew {

using namespace vm;

__device__ __forceinline__ int dt_bytes(int dt) { return dt == REW_DT_BFLOAT16 ? 2 : 4; }

__device__ __forceinline__ float ld_f(const void* p, int dt, int64_t i) {
  return dt == REW_DT_BFLOAT16 ? as_f((uint32_t)((const uint16_t*)p)[i] << 16)
                               : ((const float*)p)[i];
}
__device__ __forceinline__ void st_f(void* p, int dt, int64_t i, float v) {
  if (dt == REW_DT_BFLOAT16) ((uint16_t*)p)[i] = bf16_bits(v);
  else ((float*)p)[i] = v;
}

constexpr int kRowRegs = 32;  // elements per thread kept in registers

// row of x that feeds output row r (the gather form reads it from ids)
__device__ __forceinline__ int64_t src_row(const RowNormArgs& a, int64_t r) {
  if (!a.ids) return r;
  int64_t i;
  switch (a.ids_dt) {
    case REW_DT_INT32: i = ((const int32_t*)a.ids)[r]; break;
    case REW_DT_UINT32: i = ((const uint32_t*)a.ids)[r]; break;
    case REW_DT_INT64: i = ((const int64_t*)a.ids)[r]; break;
    default: i = (int64_t)((const uint64_t*)a.ids)[r]; break;
  }
  return i < 0 ? 0 : (i >= a.x_rows ? a.x_rows - 1 : i);
}

// Sum of v over the 256 threads of the workgroup: the wave butterfly, then
// the four wave sums as (w0 + w1) + (w2 + w3).  `part` is free again when
// this returns.
__device__ __forceinline__ float block_sum(float v, float (&part)[4]) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
  __syncthreads();
  const float sum = (part[0] + part[1]) + (part[2] + part[3]);
  __syncthreads();
  return sum;
}

// Any row length, stride, alignment and dtype pair: one workgroup per row,
// kRowRegs elements per thread kept in registers, the rest re-read.  Both
// norms; the gather form too (rows by id, the raw row stored to xout).
__global__ void __launch_bounds__(256) rmsnorm_rows_kernel(RowNormArgs a) {
  __shared__ float part[4];
  const int tid = threadIdx.x;
  const int xb = dt_bytes(a.x_dt);
  for (int64_t row = blockIdx.x; row < a.rows; row += gridDim.x) {
    const char* x = (const char*)a.x + src_row(a, row) * a.x_rs * xb;
    char* xo = a.xout ? (char*)a.xout + row * a.n * xb : nullptr;
    float v[kRowRegs];
    // pass 1: sum of squares (rmsNorm) or sum (LayerNorm)
    float s1 = 0.0f;
#pragma unroll
    for (int k = 0; k < kRowRegs; ++k) {
      const int64_t j = tid + (int64_t)k * 256;
      v[k] = j < a.n ? ld_f(x, a.x_dt, j) : 0.0f;
      if (xo && j < a.n) st_f(xo, a.x_dt, j, v[k]);
      if (a.layer) {
        s1 += v[k];
      } else {
        const float sq = v[k] * v[k];
        s1 += sq;
      }
    }
    for (int64_t j = tid + (int64_t)kRowRegs * 256; j < a.n; j += 256) {
      const float xv = ld_f(x, a.x_dt, j);
      if (xo) st_f(xo, a.x_dt, j, xv);
      if (a.layer) {
        s1 += xv;
      } else {
        const float sq = xv * xv;
        s1 += sq;
      }
    }
    const float sum = block_sum(s1, part);
    char* y = (char*)a.y + row * a.n * dt_bytes(a.y_dt);
    if (!a.layer) {
      const float mean = sum / a.divisor;
      const float r = sqrtf(mean + a.eps);
#pragma unroll
      for (int k = 0; k < kRowRegs; ++k) {
        const int64_t j = tid + (int64_t)k * 256;
        if (j < a.n) {
          const float nv = v[k] / r;
          st_f(y, a.y_dt, j, a.gamma[j] * nv);
        }
      }
      for (int64_t j = tid + (int64_t)kRowRegs * 256; j < a.n; j += 256) {
        const float nv = ld_f(x, a.x_dt, j) / r;
        st_f(y, a.y_dt, j, a.gamma[j] * nv);
      }
      continue;
    }
    // LayerNorm pass 2: sum of the centred squares
    const float m = sum / a.divisor;
    float s2 = 0.0f;
#pragma unroll
    for (int k = 0; k < kRowRegs; ++k) {
      const int64_t j = tid + (int64_t)k * 256;
      if (j < a.n) {
        const float c = v[k] - m;
        const float sq = c * c;
        s2 += sq;
      }
    }
    for (int64_t j = tid + (int64_t)kRowRegs * 256; j < a.n; j += 256) {
      const float c = ld_f(x, a.x_dt, j) - m;
      const float sq = c * c;
      s2 += sq;
    }
    const float var = block_sum(s2, part) / a.divisor2;
    const float inv = 1.0f / sqrtf(var + a.eps);  // rsqrt as the elementwise op computes it
#pragma unroll
    for (int k = 0; k < kRowRegs; ++k) {
      const int64_t j = tid + (int64_t)k * 256;
      if (j < a.n) {
        const float nv = (v[k] - m) * inv;
        const float gv = a.gamma[j] * nv;
        st_f(y, a.y_dt, j, gv + a.beta[j]);
      }
    }
    for (int64_t j = tid + (int64_t)kRowRegs * 256; j < a.n; j += 256) {
      const float nv = (ld_f(x, a.x_dt, j) - m) * inv;
      const float gv = a.gamma[j] * nv;
      st_f(y, a.y_dt, j, gv + a.beta[j]);
    }
  }
}

// Fast path: one wave per row, the row held in registers as 16-byte chunks
// (8 bf16 or 4 f32 per load), CH chunks per lane; a wave-only reduction; the
// same op order as rmsnorm_rows_kernel (square, sum, / n, + eps, sqrt,
// x / r, gamma * .).
//
// rms_row: that arithmetic for one row whose chunks are in raw (chunk k of
// lane l holds elements (64 k + l) EPC_X ..); gam(k, e) is gamma of element
// e of chunk k.  FULL: every chunk is in range (n == 64 CH EPC_X).
template <int XB, int YB, int CH, bool FULL, typename Gamma>
__device__ __forceinline__ void rms_row(const RowNormArgs& a, int64_t row, int lane,
                                        const uint4 (&raw)[CH], Gamma gam) {
  constexpr int EPC_X = 16 / XB;
  if (a.xout) {  // gather form: the gathered row itself
    char* xo = (char*)a.xout + row * a.n * XB;
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      const int64_t j = ((int64_t)k * 64 + lane) * EPC_X;
      if (FULL || j < a.n) *(uint4*)(xo + j * XB) = raw[k];
    }
  }
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const uint32_t* w = (const uint32_t*)&raw[k];
#pragma unroll
    for (int e = 0; e < EPC_X; ++e) {
      const float v = XB == 2 ? as_f((e & 1) ? (w[e >> 1] & 0xffff0000u) : (w[e >> 1] << 16))
                              : as_f(w[e]);
      const float sq = v * v;
      ss += sq;
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
  const float mean = ss / a.divisor;
  const float r = sqrtf(mean + a.eps);
  // x / r as x * (1 / r) (within an ulp of the quotient; the row's sum of
  // squares already runs in another order than the op sequence's reduction)
  const float rinv = 1.0f / r;
  char* y = (char*)a.y + row * a.n * YB;
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int64_t j = ((int64_t)k * 64 + lane) * EPC_X;
    if (!FULL && j >= a.n) continue;
    const uint32_t* w = (const uint32_t*)&raw[k];
    float out[EPC_X];
#pragma unroll
    for (int e = 0; e < EPC_X; ++e) {
      const float v = XB == 2 ? as_f((e & 1) ? (w[e >> 1] & 0xffff0000u) : (w[e >> 1] << 16))
                              : as_f(w[e]);
      const float nv = v * rinv;
      out[e] = gam(k, e) * nv;
    }
    if (YB == 2) {
      uint32_t o[EPC_X / 2];
#pragma unroll
      for (int e = 0; e < EPC_X; e += 2) o[e / 2] = bf16x2_bits(out[e], out[e + 1]);
      if (EPC_X == 8) *(uint4*)(y + j * 2) = *(const uint4*)o;
      else *(uint2*)(y + j * 2) = *(const uint2*)o;
    } else {
#pragma unroll
      for (int e = 0; e < EPC_X; e += 4)
        *(float4*)(y + (j + e) * 4) = make_float4(out[e], out[e + 1], out[e + 2], out[e + 3]);
    }
  }
}

template <int XB, int YB, int CH>  // element bytes of x and y; 16-byte chunks per lane
__global__ void __launch_bounds__(256) rmsnorm_wave_kernel(RowNormArgs a) {
  constexpr int EPC_X = 16 / XB;          // elements per x chunk
  const int lane = threadIdx.x & 63;
  const int64_t waves = (int64_t)gridDim.x * 4;
  for (int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); row < a.rows; row += waves) {
    const char* x = (const char*)a.x + src_row(a, row) * a.x_rs * XB;
    uint4 raw[CH];
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      const int64_t j = ((int64_t)k * 64 + lane) * EPC_X;
      raw[k] = j < a.n ? *(const uint4*)(x + j * XB) : make_uint4(0, 0, 0, 0);
    }
    rms_row<XB, YB, CH, false>(a, row, lane, raw, [&](int k, int e) {
      return a.gamma[((int64_t)k * 64 + lane) * EPC_X + e];
    });
  }
}

// Rows of exactly 64 CH EPC_X elements (every chunk in range, no guards):
// each wave walks rows / (4 gridDim) rows, holds gamma in registers for all
// of them (read once per wave, not once per row), and loads its next row
// before the arithmetic of the current one, the rows alternating between two
// register buffers.  The next row's loads are unconditional (past the last
// row the wave re-reads the row it just read): loads under a branch would
// make the compiler wait for every load in flight at the merge.
template <int XB, int YB, int CH>
__global__ void __launch_bounds__(256) rmsnorm_pipe_kernel(RowNormArgs a) {
  constexpr int EPC_X = 16 / XB;
  const int lane = threadIdx.x & 63;
  const int64_t waves = (int64_t)gridDim.x * 4;
  int64_t row = __builtin_amdgcn_readfirstlane((int)(blockIdx.x * 4 + (threadIdx.x >> 6)));
  if (row >= a.rows) return;
  float g[CH][EPC_X];
#pragma unroll
  for (int k = 0; k < CH; ++k)
#pragma unroll
    for (int e = 0; e < EPC_X; e += 4) {
      const float4 t = *(const float4*)(a.gamma + ((int64_t)k * 64 + lane) * EPC_X + e);
      g[k][e] = t.x;
      g[k][e + 1] = t.y;
      g[k][e + 2] = t.z;
      g[k][e + 3] = t.w;
    }
  auto load = [&](int64_t r, uint4 (&raw)[CH]) {
    const char* x = (const char*)a.x + src_row(a, r) * a.x_rs * XB;
#pragma unroll
    for (int k = 0; k < CH; ++k) raw[k] = *(const uint4*)(x + ((int64_t)k * 64 + lane) * 16);
  };
  auto gam = [&](int k, int e) { return g[k][e]; };
  uint4 ra[CH], rb[CH];
  load(row, ra);
  for (;;) {
    const int64_t r1 = row + waves;
    load(r1 < a.rows ? r1 : row, rb);
    __builtin_amdgcn_sched_barrier(0);  // (issued before this row's work)
    rms_row<XB, YB, CH, true>(a, row, lane, ra, gam);
    if (r1 >= a.rows) break;
    const int64_t r2 = r1 + waves;
    load(r2 < a.rows ? r2 : r1, ra);
    __builtin_amdgcn_sched_barrier(0);
    rms_row<XB, YB, CH, true>(a, r1, lane, rb, gam);
    if (r2 >= a.rows) break;
    row = r2;
  }
}

// ---- workgroup per row ----------------------------------------------------------------------
//
// Rows of exactly 256 CPL 16-byte chunks: the four waves of a workgroup
// split one row, thread t holding chunks k 256 + t (k < CPL), so each row's
// arithmetic is a quarter of a wave-per-row kernel's and up to eight
// workgroups per CU keep loads in flight while others compute (no software
// pipeline, no persistent loop).  The row total is the wave butterfly of
// each wave's partials, then the four wave sums as (w0 + w1) + (w2 + w3).
template <int SLOT>
__device__ __forceinline__ float wg_row_sum(float v, float (&part)[2][4]) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  if ((threadIdx.x & 63) == 0) part[SLOT][threadIdx.x >> 6] = v;
  __syncthreads();
  return (part[SLOT][0] + part[SLOT][1]) + (part[SLOT][2] + part[SLOT][3]);
}

template <int XB, int YB, int CPL, int R>  // R rows per workgroup (bytes in flight per CU)
__global__ void __launch_bounds__(256) rmsnorm_wg_kernel(RowNormArgs a) {
  constexpr int EPC = 16 / XB;
  __shared__ float part[R][4];
  const int t = threadIdx.x;
  const int64_t row0 = (int64_t)blockIdx.x * R;
  uint4 raw[R][CPL];
#pragma unroll
  for (int q = 0; q < R; ++q) {
    // past the last row (rows % R != 0) the last row is read again, its
    // results not stored
    const int64_t row = row0 + q < a.rows ? row0 + q : a.rows - 1;
    const char* x = (const char*)a.x + src_row(a, row) * a.x_rs * XB;
#pragma unroll
    for (int k = 0; k < CPL; ++k) raw[q][k] = *(const uint4*)(x + ((int64_t)k * 256 + t) * 16);
  }
  auto elem = [&](int q, int k, int e) {
    const uint32_t* w = (const uint32_t*)&raw[q][k];
    return XB == 2 ? as_f((e & 1) ? (w[e >> 1] & 0xffff0000u) : (w[e >> 1] << 16)) : as_f(w[e]);
  };
  float ss[R];
#pragma unroll
  for (int q = 0; q < R; ++q) {
    ss[q] = 0.0f;
#pragma unroll
    for (int k = 0; k < CPL; ++k)
#pragma unroll
      for (int e = 0; e < EPC; ++e) {
        const float v = elem(q, k, e);
        const float sq = v * v;
        ss[q] += sq;
      }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) ss[q] += __shfl_xor(ss[q], m, 64);
    if ((t & 63) == 0) part[q][t >> 6] = ss[q];
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < R; ++q) {
    const int64_t row = row0 + q;
    if (row >= a.rows) break;
    const float tot = (part[q][0] + part[q][1]) + (part[q][2] + part[q][3]);
    const float mean = tot / a.divisor;
    const float r = sqrtf(mean + a.eps);
    const float rinv = 1.0f / r;  // x / r as x * (1 / r), as in rms_row
    char* y = (char*)a.y + row * a.n * YB;
    char* xo = a.xout ? (char*)a.xout + row * a.n * XB : nullptr;
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
      const int64_t j = ((int64_t)k * 256 + t) * EPC;
      if (xo) *(uint4*)(xo + j * XB) = raw[q][k];  // gather form: the gathered row itself
      float out[EPC];
#pragma unroll
      for (int e = 0; e < EPC; e += 4) {
        const float4 g = *(const float4*)(a.gamma + j + e);
        out[e] = g.x * (elem(q, k, e) * rinv);
        out[e + 1] = g.y * (elem(q, k, e + 1) * rinv);
        out[e + 2] = g.z * (elem(q, k, e + 2) * rinv);
        out[e + 3] = g.w * (elem(q, k, e + 3) * rinv);
      }
      if (YB == 2) {
        uint32_t o[EPC / 2];
#pragma unroll
        for (int e = 0; e < EPC; e += 2) o[e / 2] = bf16x2_bits(out[e], out[e + 1]);
        if (EPC == 8) *(uint4*)(y + j * 2) = *(const uint4*)o;
        else *(uint2*)(y + j * 2) = *(const uint2*)o;
      } else {
#pragma unroll
        for (int e = 0; e < EPC; e += 4)
          *(float4*)(y + (j + e) * 4) = make_float4(out[e], out[e + 1], out[e + 2], out[e + 3]);
      }
    }
  }
}

// LayerNorm, laid out like rmsnorm_wg_kernel (one row per workgroup, thread
// t holding chunks k 256 + t): the row sum, the mean, then the sum of the
// centred squares from the same registers -- one read and one write of the
// row.  Each workgroup-wide sum has its own LDS slot, so the second needs no
// barrier before its writes.
template <int XB, int YB, int CPL>
__global__ void __launch_bounds__(256) layernorm_wg_kernel(RowNormArgs a) {
  constexpr int EPC = 16 / XB;
  __shared__ float part[2][4];
  const int t = threadIdx.x;
  const int64_t row = blockIdx.x;
  uint4 raw[CPL];
  {
    const char* x = (const char*)a.x + src_row(a, row) * a.x_rs * XB;
#pragma unroll
    for (int k = 0; k < CPL; ++k) raw[k] = *(const uint4*)(x + ((int64_t)k * 256 + t) * 16);
  }
  auto elem = [&](int k, int e) {
    const uint32_t* w = (const uint32_t*)&raw[k];
    return XB == 2 ? as_f((e & 1) ? (w[e >> 1] & 0xffff0000u) : (w[e >> 1] << 16)) : as_f(w[e]);
  };
  if (a.xout) {  // gather form: the gathered row itself
    char* xo = (char*)a.xout + row * a.n * XB;
#pragma unroll
    for (int k = 0; k < CPL; ++k) *(uint4*)(xo + ((int64_t)k * 256 + t) * 16) = raw[k];
  }
  float s1 = 0.0f;
#pragma unroll
  for (int k = 0; k < CPL; ++k)
#pragma unroll
    for (int e = 0; e < EPC; ++e) s1 += elem(k, e);
  const float m = wg_row_sum<0>(s1, part) / a.divisor;
  float s2 = 0.0f;
#pragma unroll
  for (int k = 0; k < CPL; ++k)
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      const float c = elem(k, e) - m;
      const float sq = c * c;
      s2 += sq;
    }
  const float var = wg_row_sum<1>(s2, part) / a.divisor2;
  const float inv = 1.0f / sqrtf(var + a.eps);  // rsqrt as the elementwise op computes it
  char* y = (char*)a.y + row * a.n * YB;
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int64_t j = ((int64_t)k * 256 + t) * EPC;
    float out[EPC];
#pragma unroll
    for (int e = 0; e < EPC; e += 4) {
      const float4 g = *(const float4*)(a.gamma + j + e);
      const float4 b = *(const float4*)(a.beta + j + e);
      out[e] = g.x * ((elem(k, e) - m) * inv) + b.x;
      out[e + 1] = g.y * ((elem(k, e + 1) - m) * inv) + b.y;
      out[e + 2] = g.z * ((elem(k, e + 2) - m) * inv) + b.z;
      out[e + 3] = g.w * ((elem(k, e + 3) - m) * inv) + b.w;
    }
    if (YB == 2) {
      uint32_t o[EPC / 2];
#pragma unroll
      for (int e = 0; e < EPC; e += 2) o[e / 2] = bf16x2_bits(out[e], out[e + 1]);
      if (EPC == 8) *(uint4*)(y + j * 2) = *(const uint4*)o;
      else *(uint2*)(y + j * 2) = *(const uint2*)o;
    } else {
#pragma unroll
      for (int e = 0; e < EPC; e += 4)
        *(float4*)(y + (j + e) * 4) = make_float4(out[e], out[e + 1], out[e + 2], out[e + 3]);
    }
  }
}

// REW_MI355X_ROWS=wave keeps the wave-per-row kernels for whole rows.
static bool rows_wg() {
  static const bool on = [] {
    const char* s = std::getenv("REW_MI355X_ROWS");
    return !(s && std::string(s) == "wave");
  }();
  return on;
}

bool rmsnorm_gather_ok(const RowNormArgs& a) {
  const int xb = a.x_dt == REW_DT_BFLOAT16 ? 2 : 4, yb = a.y_dt == REW_DT_BFLOAT16 ? 2 : 4;
  const int epc = 16 / xb;
  const int64_t chunks = (a.n + epc - 1) / epc;
  const bool id_ok = a.ids_dt == REW_DT_INT32 || a.ids_dt == REW_DT_UINT32 ||
                     a.ids_dt == REW_DT_INT64 || a.ids_dt == REW_DT_UINT64;
  return id_ok && a.x_rows > 0 && a.n % epc == 0 && (a.x_rs * xb) % 16 == 0 &&
         ((uintptr_t)a.x & 15) == 0 && ((uintptr_t)a.y & 15) == 0 &&
         ((uintptr_t)a.xout & 15) == 0 && (a.n * yb) % 16 == 0 && chunks <= 64 * 16;
}

void launch_rmsnorm_rows(const RowNormArgs& a, hipStream_t stream) {
  if (a.rows == 0 || a.n == 0) return;
  if (a.ids && !rmsnorm_gather_ok(a))
    fail(REW_MI355X_ERR_INVALID, "internal: gather rmsNorm launch outside its limits");
  const int xb = a.x_dt == REW_DT_BFLOAT16 ? 2 : 4, yb = a.y_dt == REW_DT_BFLOAT16 ? 2 : 4;
  const int epc = 16 / xb;
  const int64_t chunks = (a.n + epc - 1) / epc;  // 16-byte chunks per row
  const bool vec = a.n % epc == 0 && (a.x_rs * xb) % 16 == 0 && ((uintptr_t)a.x & 15) == 0 &&
                   ((uintptr_t)a.y & 15) == 0 && (a.n * yb) % 16 == 0 && chunks <= 64 * 16;
  if (a.layer) {
    // LayerNorm: a workgroup per row of 256, 512 or 1024 chunks, else the
    // general kernel (any shape, the gather form included)
    if (vec && ((uintptr_t)a.gamma & 15) == 0 && ((uintptr_t)a.beta & 15) == 0 &&
        a.rows < (1 << 30) && (chunks == 256 || chunks == 512 || chunks == 1024)) {
      const dim3 grid((unsigned)a.rows), block(256);
#define REW_LN(XB, YB, CPL) \
      hipLaunchKernelGGL((layernorm_wg_kernel<XB, YB, CPL>), grid, block, 0, stream, a)
#define REW_LN_CPL(XB, YB) \
      if (chunks == 256) { REW_LN(XB, YB, 1); } else if (chunks == 512) { REW_LN(XB, YB, 2); } \
      else { REW_LN(XB, YB, 4); }
      if (xb == 2 && yb == 2) { REW_LN_CPL(2, 2); }
      else if (xb == 2) { REW_LN_CPL(2, 4); }
      else if (yb == 2) { REW_LN_CPL(4, 2); }
      else { REW_LN_CPL(4, 4); }
#undef REW_LN_CPL
#undef REW_LN
    } else {
      const unsigned grid = (unsigned)(a.rows < 65536 ? a.rows : 65536);
      hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(grid), dim3(256), 0, stream, a);
    }
    REW_HIP(hipGetLastError());
    return;
  }
  if (vec && rows_wg() && ((uintptr_t)a.gamma & 15) == 0 && a.rows < (1 << 30) &&
      (chunks == 256 || chunks == 512 || chunks == 1024) &&
      !(a.ids && !rmsnorm_gather_ok(a))) {
    // one row per workgroup: two or four rows per workgroup measured 1-8 %
    // slower on [8192, 4096] bf16 and f32
    const dim3 grid((unsigned)a.rows), block(256);
#define REW_RMS(XB, YB, CPL) \
    hipLaunchKernelGGL((rmsnorm_wg_kernel<XB, YB, CPL, 1>), grid, block, 0, stream, a)
#define REW_RMS_CPL(XB, YB) \
    if (chunks == 256) { REW_RMS(XB, YB, 1); } else if (chunks == 512) { REW_RMS(XB, YB, 2); } \
    else { REW_RMS(XB, YB, 4); }
    if (xb == 2 && yb == 2) { REW_RMS_CPL(2, 2); }
    else if (xb == 2) { REW_RMS_CPL(2, 4); }
    else if (yb == 2) { REW_RMS_CPL(4, 2); }
    else { REW_RMS_CPL(4, 4); }
#undef REW_RMS_CPL
#undef REW_RMS
    REW_HIP(hipGetLastError());
    return;
  }
  if (vec) {
    const int64_t blocks = (a.rows + 3) / 4;
    const dim3 grid((unsigned)(blocks < 65536 ? blocks : 65536)), block(256);
    const int ch = (int)((chunks + 63) / 64);
    // whole rows of 2, 4 or 8 chunks per lane: the pipelined kernel, at most
    // 2048 waves (two workgroups per CU)
    if (chunks == 64 * ch && ch <= 8 && ((uintptr_t)a.gamma & 15) == 0) {
      const dim3 grid_pipe((unsigned)(blocks < 512 ? blocks : 512));
#define REW_RMS(XB, YB, CH) hipLaunchKernelGGL((rmsnorm_pipe_kernel<XB, YB, CH>), grid_pipe, block, 0, stream, a)
#define REW_RMS_CH(XB, YB) \
      if (ch == 2) REW_RMS(XB, YB, 2); else if (ch == 4) REW_RMS(XB, YB, 4); else REW_RMS(XB, YB, 8)
      if (xb == 2 && yb == 2) { REW_RMS_CH(2, 2); }
      else if (xb == 2) { REW_RMS_CH(2, 4); }
      else if (yb == 2) { REW_RMS_CH(4, 2); }
      else { REW_RMS_CH(4, 4); }
#undef REW_RMS_CH
#undef REW_RMS
      REW_HIP(hipGetLastError());
      return;
    }
#define REW_RMS(XB, YB, CH) hipLaunchKernelGGL((rmsnorm_wave_kernel<XB, YB, CH>), grid, block, 0, stream, a)
#define REW_RMS_CH(XB, YB) \
    if (ch <= 2) REW_RMS(XB, YB, 2); else if (ch <= 4) REW_RMS(XB, YB, 4); \
    else if (ch <= 8) REW_RMS(XB, YB, 8); else REW_RMS(XB, YB, 16)
    if (xb == 2 && yb == 2) { REW_RMS_CH(2, 2); }
    else if (xb == 2) { REW_RMS_CH(2, 4); }
    else if (yb == 2) { REW_RMS_CH(4, 2); }
    else { REW_RMS_CH(4, 4); }
#undef REW_RMS_CH
#undef REW_RMS
  } else {
    const unsigned grid = (unsigned)(a.rows < 65536 ? a.rows : 65536);
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(grid), dim3(256), 0, stream, a);
  }
  REW_HIP(hipGetLastError());
}

// ---- softmax -------------------------------------------------------------------------------

// rew's softmax (src/rew/nn/activation.nim:64-77) over the last axis in one
// pass: the row is read once and written once.  The compiled row reduction
// (one wave per row, V = 4) has lane l add its 16-byte chunks c = 0, 1, ...
// -- elements 4 (64 c + l) + j, j = 0..3 in order -- then combine lanes by a
// butterfly over xor 32, 16, ..., 1; the sum here runs in exactly that
// order, and the max (order-free) and exp / divide are the same fp32 ops.
// One row per wave; PIPE: each wave walks several rows (grid-stride) and
// loads its next row before computing the current one, the rows alternating
// between two register buffers (no copies, which would wait for the loads),
// so the HBM reads of one row overlap the exp / divide work of the last.
// FULL: n == 256 CH, every chunk in range; the loads then carry no guards
// (a guarded load is a branch, and the compiler waits for every load in
// flight at each one, the next row's included).
// The arithmetic of each row is the same either way.
template <int CH, bool FULL>
__device__ __forceinline__ void softmax_load(const SoftmaxArgs& a, int64_t row, int lane,
                                             float4 (&v)[CH]) {
  const float* x = a.x + row * a.x_rs;
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int64_t j = ((int64_t)k * 64 + lane) * 4;
    if (FULL || j < a.n) v[k] = *(const float4*)(x + j);
  }
}
template <int CH, bool FULL>
__device__ __forceinline__ void softmax_row(const SoftmaxArgs& a, int64_t row, int lane,
                                            float4 (&v)[CH]) {
  // The row max enters only as x - m, so two of reduceMax's rules cannot
  // change a result: +0 and -0 give the same exp(x - m) bits, and with a
  // NaN in the row the sum is NaN and every output NaN however m treats
  // it.  The plain hardware max (one instruction, NaN-dropping, either
  // zero) therefore gives the op-by-op outputs bit for bit, NaN payloads
  // aside.
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int64_t j = ((int64_t)k * 64 + lane) * 4;
    if (FULL || j < a.n) {
      m = __builtin_fmaxf(m, v[k].x);
      m = __builtin_fmaxf(m, v[k].y);
      m = __builtin_fmaxf(m, v[k].z);
      m = __builtin_fmaxf(m, v[k].w);
    }
  }
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) m = __builtin_fmaxf(m, __shfl_xor(m, s, 64));
  float sum = 0.0f;
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int64_t j = ((int64_t)k * 64 + lane) * 4;
    if (FULL || j < a.n) {
      v[k].x = expf(v[k].x - m);
      v[k].y = expf(v[k].y - m);
      v[k].z = expf(v[k].z - m);
      v[k].w = expf(v[k].w - m);
      sum = sum + v[k].x;
      sum = sum + v[k].y;
      sum = sum + v[k].z;
      sum = sum + v[k].w;
    }
  }
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) sum = sum + __shfl_xor(sum, s, 64);
  float* y = a.y + row * a.n;
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int64_t j = ((int64_t)k * 64 + lane) * 4;
    if (FULL || j < a.n)
      *(float4*)(y + j) = make_float4(v[k].x / sum, v[k].y / sum, v[k].z / sum, v[k].w / sum);
  }
}
template <int CH, bool PIPE, bool FULL>  // CH: 16-byte chunks per lane
__global__ void __launch_bounds__(256) softmax_wave_kernel(SoftmaxArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t waves = (int64_t)gridDim.x * 4;
  int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if constexpr (!PIPE) {
    for (; row < a.rows; row += waves) {
      float4 v[CH];
      softmax_load<CH, FULL>(a, row, lane, v);
      softmax_row<CH, FULL>(a, row, lane, v);
    }
  } else {
    // The next row's loads are unconditional (past the last row a wave
    // re-reads the row it just read): a load under a branch would leave the
    // compiler, at the merge, waiting for every load in flight before the
    // current row's arithmetic.
    row = __builtin_amdgcn_readfirstlane((int)row);
    if (row >= a.rows) return;
    float4 va[CH], vb[CH];
    softmax_load<CH, FULL>(a, row, lane, va);
    for (;;) {
      const int64_t r1 = row + waves;
      softmax_load<CH, FULL>(a, r1 < a.rows ? r1 : row, lane, vb);
      __builtin_amdgcn_sched_barrier(0);  // (issued before this row's work)
      softmax_row<CH, FULL>(a, row, lane, va);
      if (r1 >= a.rows) break;
      const int64_t r2 = r1 + waves;
      softmax_load<CH, FULL>(a, r2 < a.rows ? r2 : r1, lane, va);
      __builtin_amdgcn_sched_barrier(0);
      softmax_row<CH, FULL>(a, r1, lane, vb);
      if (r2 >= a.rows) break;
      row = r2;
    }
  }
}

// Rows shorter than 128: a workgroup stages R rows in LDS with coalesced
// loads (row pitch n + 1 against bank conflicts), one thread runs each row's
// three sequential passes -- max, sum of expf(x - m), expf(x - m) / sum --
// in the order of the compiled reductions over short rows, so the result
// equals rew's five-op sequence bit for bit, and the results leave through
// LDS as coalesced stores.  Each exp(x - m) is computed once and kept in
// LDS for the division.
template <int R>
__global__ void __launch_bounds__(256) softmax_tile_kernel(SoftmaxArgs a) {
  extern __shared__ float tile[];
  const int n = (int)a.n, pitch = n + 1;
  const int q = 256 / n, rem = 256 % n;
  for (int64_t r0 = (int64_t)blockIdx.x * R; r0 < a.rows; r0 += (int64_t)gridDim.x * R) {
    const int nr = (int)(a.rows - r0 < R ? a.rows - r0 : R);
    // element i = row * n + col of the tile, walked in steps of 256
    int row = threadIdx.x / n, col = threadIdx.x - row * n;
    for (int i = threadIdx.x; i < nr * n; i += 256) {
      tile[row * pitch + col] = a.x[(r0 + row) * a.x_rs + col];
      col += rem;
      row += q;
      if (col >= n) {
        col -= n;
        ++row;
      }
    }
    __syncthreads();
    if ((int)threadIdx.x < nr) {
      float* t = tile + threadIdx.x * pitch;
      float m = -INFINITY;
      for (int j = 0; j < n; ++j) m = fmax_prop(m, t[j]);
      float sum = 0.0f;
      for (int j = 0; j < n; ++j) {
        const float e = expf(t[j] - m);
        t[j] = e;
        sum = sum + e;
      }
      for (int j = 0; j < n; ++j) t[j] = t[j] / sum;
    }
    __syncthreads();
    row = threadIdx.x / n;
    col = threadIdx.x - row * n;
    float* y = a.y + r0 * n;
    for (int i = threadIdx.x; i < nr * n; i += 256) {
      y[i] = tile[row * pitch + col];
      col += rem;
      row += q;
      if (col >= n) {
        col -= n;
        ++row;
      }
    }
    __syncthreads();
  }
}

// Rows of exactly 1024 CPL fp32 (256 CPL 16-byte chunks): a workgroup per
// row, thread t holding chunks k 256 + t; the max, then the sum of the
// exps, each over the workgroup (wg_row_sum's order), then the quotients.
// The same fp32 ops per element as softmax_row; the sum runs in another
// order than the compiled row reduction's.
template <int CPL>
__global__ void __launch_bounds__(256) softmax_wg_kernel(SoftmaxArgs a) {
  __shared__ float part[2][4];
  const int64_t row = blockIdx.x;
  const int t = threadIdx.x;
  const float* x = a.x + row * a.x_rs;
  float4 v[CPL];
#pragma unroll
  for (int k = 0; k < CPL; ++k) v[k] = *(const float4*)(x + ((int64_t)k * 256 + t) * 4);
  float m = -INFINITY;  // the hardware max, as in softmax_row
#pragma unroll
  for (int k = 0; k < CPL; ++k)
    m = __builtin_fmaxf(__builtin_fmaxf(m, __builtin_fmaxf(v[k].x, v[k].y)),
                        __builtin_fmaxf(v[k].z, v[k].w));
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) m = __builtin_fmaxf(m, __shfl_xor(m, s, 64));
  if ((t & 63) == 0) part[1][t >> 6] = m;
  __syncthreads();
  m = __builtin_fmaxf(__builtin_fmaxf(part[1][0], part[1][1]),
                      __builtin_fmaxf(part[1][2], part[1][3]));
  float sum = 0.0f;
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    v[k].x = expf(v[k].x - m);
    v[k].y = expf(v[k].y - m);
    v[k].z = expf(v[k].z - m);
    v[k].w = expf(v[k].w - m);
    sum = sum + v[k].x;
    sum = sum + v[k].y;
    sum = sum + v[k].z;
    sum = sum + v[k].w;
  }
  sum = wg_row_sum<0>(sum, part);
  float* y = a.y + row * a.n;
#pragma unroll
  for (int k = 0; k < CPL; ++k)
    *(float4*)(y + ((int64_t)k * 256 + t) * 4) =
        make_float4(v[k].x / sum, v[k].y / sum, v[k].z / sum, v[k].w / sum);
}

bool softmax_rows_ok(const SoftmaxArgs& a) {
  if (a.rows <= 0 || a.n <= 0) return false;
  if (a.n < 128) return true;
  return a.n % 4 == 0 && a.n <= kSoftmaxMaxCols && a.x_rs % 4 == 0 &&
         ((uintptr_t)a.x & 15) == 0 && ((uintptr_t)a.y & 15) == 0;
}

void launch_softmax_rows(const SoftmaxArgs& a, hipStream_t stream) {
  if (!softmax_rows_ok(a)) fail(REW_MI355X_ERR_INVALID, "internal: softmax rows not launchable");
  if (a.n < 128) {
    // 32 rows per workgroup: a thread runs each row's passes serially, so
    // the rows spread over as many CUs as there are workgroups
    const int64_t blocks = (a.rows + 31) / 32;
    hipLaunchKernelGGL(softmax_tile_kernel<32>, dim3((unsigned)(blocks < 65536 ? blocks : 65536)),
                       dim3(256), (size_t)32 * (a.n + 1) * 4, stream, a);
  } else {
    // Rows of exactly 1024, 2048 or 4096 use the pipelined unguarded
    // kernels: at most 2048 waves (two workgroups per CU), each walking
    // rows / 2048 rows.  Other widths keep one row per wave.
    const int64_t blocks = (a.rows + 3) / 4;
    const dim3 grid_pipe((unsigned)(blocks < 512 ? blocks : 512));
    const dim3 grid((unsigned)(blocks < 65536 ? blocks : 65536)), block(256);
    const int64_t ch = (a.n / 4 + 63) / 64;
    const dim3 grid_wg((unsigned)(a.rows < (1 << 30) ? a.rows : 1));
    if (rows_wg() && a.rows < (1 << 30) && (a.n == 1024 || a.n == 2048 || a.n == 4096)) {
      if (a.n == 1024) hipLaunchKernelGGL((softmax_wg_kernel<1>), grid_wg, block, 0, stream, a);
      else if (a.n == 2048) hipLaunchKernelGGL((softmax_wg_kernel<2>), grid_wg, block, 0, stream, a);
      else hipLaunchKernelGGL((softmax_wg_kernel<4>), grid_wg, block, 0, stream, a);
    } else if (a.n == 1024) hipLaunchKernelGGL((softmax_wave_kernel<4, true, true>), grid_pipe, block, 0, stream, a);
    else if (a.n == 2048) hipLaunchKernelGGL((softmax_wave_kernel<8, true, true>), grid_pipe, block, 0, stream, a);
    else if (a.n == 4096) hipLaunchKernelGGL((softmax_wave_kernel<16, true, true>), grid_pipe, block, 0, stream, a);
    else if (ch <= 4) hipLaunchKernelGGL((softmax_wave_kernel<4, false, false>), grid, block, 0, stream, a);
    else if (ch <= 8) hipLaunchKernelGGL((softmax_wave_kernel<8, false, false>), grid, block, 0, stream, a);
    else if (ch <= 16) hipLaunchKernelGGL((softmax_wave_kernel<16, false, false>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((softmax_wave_kernel<32, false, false>), grid, block, 0, stream, a);
  }
  REW_HIP(hipGetLastError());
}

// ---- RoPE ------------------------------------------------------------------------------

// VEC: bf16 x and y with contiguous pairs, cos / sin read at pair stride 2
// (rew's duplicated tables): one 16-byte x load, two float4 loads of each
// table, one 16-byte store per four pairs.
template <bool VEC>
__global__ void __launch_bounds__(256) rope_pairs_kernel(RopeArgs a) {
  // pairs are processed in groups of 4 consecutive i (half % 4 == 0)
  const uint32_t g4 = (uint32_t)(a.half / 4);
  const uint32_t total = (uint32_t)(a.d0 * a.d1 * a.S) * g4;
  FastDiv fg = a.fd_g4, fs = a.fd_s, f1 = a.fd_d1;
  for (uint32_t t = blockIdx.x * 256 + threadIdx.x; t < total; t += gridDim.x * 256) {
    uint32_t q = fdiv(t, fg);
    const uint32_t i0 = (t - q * g4) * 4;
    uint32_t q2 = fdiv(q, fs);
    const uint32_t s = q - q2 * (uint32_t)a.S;
    const uint32_t i1 = q2 - fdiv(q2, f1) * (uint32_t)a.d1;
    const uint32_t i0d = fdiv(q2, f1);
    const int64_t xb = i0d * a.x_s0 + i1 * a.x_s1 + s * a.x_ss;
    const int64_t cb = i0d * a.c_s0 + i1 * a.c_s1 + s * a.c_ss;
    const int64_t sb = i0d * a.s_s0 + i1 * a.s_s1 + s * a.s_ss;
    const int64_t yb = ((int64_t)q2 * a.S + s) * (2 * a.half) + 2 * i0;
    if (VEC) {
      const uint4 xv = *(const uint4*)((const uint16_t*)a.x + xb + 2 * i0);
      const float4 c0 = *(const float4*)(a.cos + cb + 2 * i0);
      const float4 c1 = *(const float4*)(a.cos + cb + 2 * i0 + 4);
      const float4 s0 = *(const float4*)(a.sin + sb + 2 * i0);
      const float4 s1 = *(const float4*)(a.sin + sb + 2 * i0 + 4);
      const float cs[4] = {c0.x, c0.z, c1.x, c1.z};
      const float sn[4] = {s0.x, s0.z, s1.x, s1.z};
      const uint32_t* w = (const uint32_t*)&xv;
      uint32_t o[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float x0 = as_f(w[u] << 16), x1 = as_f(w[u] & 0xffff0000u);
        const float t1 = cs[u] * x0;
        const float t2 = sn[u] * x1;
        const float t3 = sn[u] * x0;
        const float t4 = cs[u] * x1;
        o[u] = (uint32_t)bf16_bits(t1 - t2) | ((uint32_t)bf16_bits(t3 + t4) << 16);
      }
      *(uint4*)((uint16_t*)a.y + yb) = make_uint4(o[0], o[1], o[2], o[3]);
      continue;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t i = i0 + u;
      const float x0 = ld_f(a.x, a.x_dt, xb + (2 * i) * a.x_sd);
      const float x1 = ld_f(a.x, a.x_dt, xb + (2 * i + 1) * a.x_sd);
      const float c = a.cos[cb + i * a.c_si];
      const float sn = a.sin[sb + i * a.s_si];
      const float t1 = c * x0;
      const float t2 = sn * x1;
      const float t3 = sn * x0;
      const float t4 = c * x1;
      st_f(a.y, a.y_dt, yb + 2 * u, t1 - t2);
      st_f(a.y, a.y_dt, yb + 2 * u + 1, t3 + t4);
    }
  }
}

void launch_rope(const RopeArgs& a, hipStream_t stream) {
  const int64_t total = a.d0 * a.d1 * a.S * (a.half / 4);
  if (total == 0) return;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 256 * 32) blocks = 256 * 32;
  auto al = [](const void* p, int b) { return ((uintptr_t)p % b) == 0; };
  const bool vec = a.x_dt == REW_DT_BFLOAT16 && a.y_dt == REW_DT_BFLOAT16 && a.x_sd == 1 &&
                   a.x_s0 % 8 == 0 && a.x_s1 % 8 == 0 && a.x_ss % 8 == 0 && al(a.x, 16) &&
                   al(a.y, 16) && a.c_si == 2 && a.s_si == 2 && a.c_s0 % 4 == 0 &&
                   a.c_s1 % 4 == 0 && a.c_ss % 4 == 0 && a.s_s0 % 4 == 0 && a.s_s1 % 4 == 0 &&
                   a.s_ss % 4 == 0 && al(a.cos, 16) && al(a.sin, 16);
  if (vec)
    hipLaunchKernelGGL(rope_pairs_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(rope_pairs_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  REW_HIP(hipGetLastError());
}

}  // namespace rew
