// Index-producing row selections: argmax, topK and the row sort.
//
// argmax (src/rew/ops/reduce.nim:202-225): the reference composite is
//   m = reduceMax(x, [d]); mask = compare(x, broadcast(m), EQ);
//   reduceMin(select(mask, iota(d), INT32_MAX), [d])
// i.e. the lowest index holding the (NaN-propagating) maximum, and INT32_MAX
// for a slice containing NaN (NaN == m is false everywhere).  Both kernels
// below compute that in one pass with a (value, index, saw-NaN) reduction;
// -0 and +0 compare equal, so the lower index wins between them, as in the
// composite.
//
// topK (src/rew/ops/sort.nim:36-90): a stable sort with comparator GE
// (largest) or LE (smallest), then the first k.  Ties keep the lower index;
// NaN never compares GE/LE, so it ranks after every number.  One wave per
// row: the row's keys sit in LDS, and each lane keeps a 64-bit "taken" mask
// of the row slots it owns (slot s of lane l is column s * 64 + l), so a
// row of up to 4096 columns needs no further state.  Each of the k rounds
// is a lane-local scan plus a 6-step shuffle reduction.
#include <hip/hip_runtime.h>

#include "kernels.h"

namespace rew {

namespace {

constexpr int kNone = 0x7fffffff;

struct Best {
  float v;
  int i;     // kNone: nothing yet
};

// a ranks before b under "larger first, NaN last, lower index on ties"
__device__ __forceinline__ bool ranks_before(float av, int ai, float bv, int bi) {
  if (ai == kNone) return false;
  if (bi == kNone) return true;
  const bool an = av != av, bn = bv != bv;
  if (an != bn) return !an;
  if (!an && av != bv) return av > bv;
  return ai < bi;
}

__device__ __forceinline__ Best wave_best(Best b) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float ov = __shfl_xor(b.v, m, 64);
    const int oi = __shfl_xor(b.i, m, 64);
    if (ranks_before(ov, oi, b.v, b.i)) {
      b.v = ov;
      b.i = oi;
    }
  }
  return b;
}

// argmax partial state: best non-NaN value and its lowest index, plus
// whether a NaN was seen (which forces the INT32_MAX result).
struct Arg {
  float v;
  int i;
  int nan;
};

__device__ __forceinline__ void arg_push(Arg& a, float x, int i) {
  if (x != x) {
    a.nan = 1;
  } else if (a.i == kNone || x > a.v || (x == a.v && i < a.i)) {
    a.v = x;
    a.i = i;
  }
}

__device__ __forceinline__ void arg_merge(Arg& a, float v, int i, int nan) {
  a.nan |= nan;
  if (i == kNone) return;
  if (a.i == kNone || v > a.v || (v == a.v && i < a.i)) {
    a.v = v;
    a.i = i;
  }
}

}  // namespace

// Reduced dim innermost: one wave per slice.
__global__ void __launch_bounds__(256) argmax_rows_kernel(ArgmaxArgs g) {
  const int lane = threadIdx.x & 63;
  const int64_t waves = (int64_t)gridDim.x * 4;
  for (int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); r < g.outer; r += waves) {
    const float* x = g.x + r * g.n;
    Arg a{0.0f, kNone, 0};
    for (int64_t c = lane; c < g.n; c += 64) arg_push(a, x[c], (int)c);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      const float ov = __shfl_xor(a.v, m, 64);
      const int oi = __shfl_xor(a.i, m, 64);
      const int on = __shfl_xor(a.nan, m, 64);
      arg_merge(a, ov, oi, on);
    }
    if (lane == 0) g.out[r] = a.nan ? kNone : a.i;
  }
}

// Reduced dim strided (inner > 1): one thread per (outer, inner) slice,
// neighbouring threads read neighbouring inner elements.
__global__ void __launch_bounds__(256) argmax_cols_kernel(ArgmaxArgs g) {
  const int64_t total = g.outer * g.inner;
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += step) {
    const int64_t o = t / g.inner, j = t - o * g.inner;
    const float* x = g.x + o * g.n * g.inner + j;
    Arg a{0.0f, kNone, 0};
    for (int64_t c = 0; c < g.n; ++c) arg_push(a, x[c * g.inner], (int)c);
    g.out[t] = a.nan ? kNone : a.i;
  }
}

__global__ void __launch_bounds__(256) topk_rows_kernel(TopkArgs g) {
  extern __shared__ float keys[];  // 4 waves x cols
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float* row = keys + (int64_t)wave * g.cols;
  const int64_t waves = (int64_t)gridDim.x * 4;
  const float sgn = g.largest ? 1.0f : -1.0f;
  for (int64_t r = (int64_t)blockIdx.x * 4 + wave; r < g.rows; r += waves) {
    const float* x = g.x + r * g.cols;
    // every lane reads back only the slots it wrote (columns lane + 64 s)
    for (int c = lane; c < g.cols; c += 64) row[c] = sgn * x[c];
    uint64_t taken = 0;
    for (int t = 0; t < g.k; ++t) {
      Best b{0.0f, kNone};
      int s = 0;
      for (int c = lane; c < g.cols; c += 64, ++s) {
        if ((taken >> s) & 1) continue;
        const float v = row[c];
        if (ranks_before(v, c, b.v, b.i)) {
          b.v = v;
          b.i = c;
        }
      }
      b = wave_best(b);
      if ((b.i & 63) == lane) taken |= 1ull << (b.i >> 6);
      if (lane == 0) {
        g.vals[r * g.k + t] = sgn * b.v;
        g.idx[r * g.k + t] = b.i;
      }
    }
  }
}

// ---- row sort --------------------------------------------------------------
//
// One workgroup per row: the row's keys become 64-bit composites
// (order key << 32 | column) in LDS, a bitonic network sorts them
// ascending, and the low halves give every output column its source
// column.  The column in the low half makes equal keys keep their original
// order (a stable sort); padding slots are all-ones and sort last.

namespace {

// Monotone unsigned image of one key: ascending order of the image is the
// comparator's order; NaN maps above every number in both directions.
__device__ __forceinline__ uint32_t order_key(const SortArgs& g, int64_t i) {
  uint32_t u;
  bool flt = false;
  switch (g.key_dt) {
    case kF32: u = ((const uint32_t*)g.key)[i]; flt = true; break;
    case kBF16: u = (uint32_t)((const uint16_t*)g.key)[i] << 16; flt = true; break;
    case kF16: u = __float_as_uint((float)((const _Float16*)g.key)[i]); flt = true; break;
    case kI32: u = ((const uint32_t*)g.key)[i] ^ 0x80000000u; break;
    case kI16: u = (uint32_t)(int32_t)((const int16_t*)g.key)[i] ^ 0x80000000u; break;
    case kI8: u = (uint32_t)(int32_t)((const int8_t*)g.key)[i] ^ 0x80000000u; break;
    case kU32: u = ((const uint32_t*)g.key)[i]; break;
    case kU16: u = ((const uint16_t*)g.key)[i]; break;
    default: u = ((const uint8_t*)g.key)[i]; break;  // kU8, kBool
  }
  if (flt) {
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0xffffffffu;  // NaN: last
    if (u == 0x80000000u) u = 0;                              // -0 == +0
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  }
  return g.descending ? ~u : u;
}

__device__ __forceinline__ void copy_elem(const void* src, void* dst, int esize,
                                          int64_t s, int64_t d) {
  switch (esize) {
    case 1: ((uint8_t*)dst)[d] = ((const uint8_t*)src)[s]; break;
    case 2: ((uint16_t*)dst)[d] = ((const uint16_t*)src)[s]; break;
    case 4: ((uint32_t*)dst)[d] = ((const uint32_t*)src)[s]; break;
    default: ((uint64_t*)dst)[d] = ((const uint64_t*)src)[s]; break;
  }
}

}  // namespace

template <int NP, int NT>
__global__ void __launch_bounds__(NT) sort_rows_kernel(SortArgs g) {
  __shared__ uint64_t s[NP];
  for (int64_t r = blockIdx.x; r < g.rows; r += gridDim.x) {
    const int64_t base = r * g.cols;
    for (int i = threadIdx.x; i < NP; i += NT)
      s[i] = i < g.cols ? ((uint64_t)order_key(g, base + i) << 32) | (uint32_t)i : ~0ull;
    __syncthreads();
    for (int k = 2; k <= NP; k <<= 1) {
      for (int j = k >> 1; j > 0; j >>= 1) {
        for (int t = threadIdx.x; t < NP / 2; t += NT) {
          const int lo = 2 * t - (t & (j - 1));
          const int hi = lo + j;
          const uint64_t a = s[lo], b = s[hi];
          const bool up = (lo & k) == 0;
          if ((a > b) == up) {
            s[lo] = b;
            s[hi] = a;
          }
        }
        __syncthreads();
      }
    }
    for (int j = threadIdx.x; j < g.cols; j += NT) {
      const int64_t src = base + (int64_t)(uint32_t)s[j];
      for (int o = 0; o < g.n_ops; ++o) copy_elem(g.in[o], g.out[o], g.esize[o], src, base + j);
    }
    __syncthreads();
  }
}

void launch_sort(const SortArgs& g, hipStream_t stream) {
  if (g.rows == 0 || g.cols == 0) return;
  if (g.cols > kSortMaxCols || g.n_ops < 1 || g.n_ops > kSortMaxOps)
    fail(REW_MI355X_ERR_INVALID, "internal: sort launch outside its limits");
  const unsigned blocks = (unsigned)(g.rows < 65536 ? g.rows : 65536);
#define REW_SORT_LAUNCH(NP, NT)                                                         \
  hipLaunchKernelGGL((sort_rows_kernel<NP, NT>), dim3(blocks), dim3(NT), 0, stream, g)
  if (g.cols <= 64) REW_SORT_LAUNCH(64, 64);
  else if (g.cols <= 256) REW_SORT_LAUNCH(256, 128);
  else if (g.cols <= 1024) REW_SORT_LAUNCH(1024, 256);
  else if (g.cols <= 4096) REW_SORT_LAUNCH(4096, 512);
  else REW_SORT_LAUNCH(8192, 512);
#undef REW_SORT_LAUNCH
  REW_HIP(hipGetLastError());
}

void launch_argmax(const ArgmaxArgs& g, hipStream_t stream) {
  if (g.outer == 0 || g.inner == 0) return;
  if (g.inner == 1) {
    const int64_t blocks = (g.outer + 3) / 4;
    hipLaunchKernelGGL(argmax_rows_kernel, dim3((unsigned)(blocks < 65536 ? blocks : 65536)),
                       dim3(256), 0, stream, g);
  } else {
    const int64_t blocks = (g.outer * g.inner + 255) / 256;
    hipLaunchKernelGGL(argmax_cols_kernel, dim3((unsigned)(blocks < 65536 ? blocks : 65536)),
                       dim3(256), 0, stream, g);
  }
  REW_HIP(hipGetLastError());
}

void launch_topk(const TopkArgs& g, hipStream_t stream) {
  if (g.rows == 0) return;
  if (g.k < 1 || g.k > 64 || g.cols < g.k || g.cols > kTopkMaxCols)
    fail(REW_MI355X_ERR_INVALID, "internal: topK launch outside its limits");
  const int64_t blocks = (g.rows + 3) / 4;
  const size_t lds = (size_t)4 * g.cols * sizeof(float);
  hipLaunchKernelGGL(topk_rows_kernel, dim3((unsigned)(blocks < 65536 ? blocks : 65536)),
                     dim3(256), lds, stream, g);
  REW_HIP(hipGetLastError());
}

}  // namespace rew
