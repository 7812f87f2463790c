// torch_index_select (batch_dims = 0): row gather; and the general
// stablehlo.gather / stablehlo.scatter (thread per element, atomic updates).
//
// One workgroup per output row; rows are copied with 16-byte loads/stores
// when the row size and both base addresses allow it (the embedding case:
// 4096 bf16 = 8 KiB rows).  Indices are clamped into [0, src_dim - 1], the
// clamping rule XLA applies to gather start indices.
#include <hip/hip_runtime.h>

#include "kernels.h"

namespace rew {

__device__ __forceinline__ int64_t load_index(const void* p, int dt, int64_t i) {
  switch (dt) {
    case REW_DT_INT32: return ((const int32_t*)p)[i];
    case REW_DT_UINT32: return ((const uint32_t*)p)[i];
    case REW_DT_INT64: return ((const int64_t*)p)[i];
    case REW_DT_UINT64: return (int64_t)((const uint64_t*)p)[i];
    case REW_DT_INT16: return ((const int16_t*)p)[i];
    case REW_DT_UINT16: return ((const uint16_t*)p)[i];
    case REW_DT_INT8: return ((const int8_t*)p)[i];
    default: return ((const uint8_t*)p)[i];
  }
}

template <int W>  // bytes per access: 16 or 1
__global__ void __launch_bounds__(256) gather_kernel(GatherArgs g) {
  const int64_t rows = g.n_pre * g.n_idx;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const int64_t pre = r / g.n_idx, i = r - pre * g.n_idx;
    int64_t idx = load_index(g.index, g.index_dtype, i);
    idx = idx < 0 ? 0 : (idx >= g.src_dim ? g.src_dim - 1 : idx);
    const char* src = (const char*)g.src + ((pre * g.src_dim + idx) * g.row_bytes);
    char* dst = (char*)g.out + r * g.row_bytes;
    if (W == 16) {
      for (int64_t o = threadIdx.x * 16; o < g.row_bytes; o += 256 * 16)
        *(uint4*)(dst + o) = *(const uint4*)(src + o);
    } else {
      for (int64_t o = threadIdx.x; o < g.row_bytes; o += 256) dst[o] = src[o];
    }
  }
}

void launch_gather(const GatherArgs& g, hipStream_t stream) {
  const int64_t rows = g.n_pre * g.n_idx;
  if (rows == 0 || g.row_bytes == 0) return;
  const unsigned grid = (unsigned)(rows < 65536 ? rows : 65536);
  const bool v16 = g.row_bytes % 16 == 0 && ((uintptr_t)g.src & 15) == 0 &&
                   ((uintptr_t)g.out & 15) == 0;
  if (v16)
    hipLaunchKernelGGL(gather_kernel<16>, dim3(grid), dim3(256), 0, stream, g);
  else
    hipLaunchKernelGGL(gather_kernel<1>, dim3(grid), dim3(256), 0, stream, g);
  REW_HIP(hipGetLastError());
}

}  // namespace rew

// ---- general gather / scatter ----------------------------------------------------

namespace rew {

namespace {

// Linear x offset of iteration element t (false: out of bounds, scatter only).
__device__ __forceinline__ bool map_element(const IndexMapArgs& g, int64_t t, int64_t* x_lin) {
  int64_t c[8];
  int64_t rem = t;
  for (int d = g.rank_it - 1; d >= 0; --d) {
    c[d] = rem % g.dims_it[d];
    rem /= g.dims_it[d];
  }
  int64_t win[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int64_t st[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int64_t ib = 0;
  for (int d = 0; d < g.rank_it; ++d) {
    if (g.role[d] >= 0) win[g.role[d]] = c[d];
    else ib += c[d] * g.stride_idx_batch[-1 - g.role[d]];
  }
  for (int j = 0; j < g.n_map; ++j)
    st[g.map_x[j]] = load_index(g.index, g.index_dtype, ib + j * g.stride_idx_vec);
  for (int i = 0; i < g.n_bat; ++i) st[g.bat_x[i]] = c[g.bat_it[i]];
  int64_t lin = 0;
  for (int d = 0; d < g.rank_x; ++d) {
    int64_t s = st[d];
    if (g.clamp) {
      const int64_t hi = g.dims_x[d] - g.slice[d];
      s = s < 0 ? 0 : (s > hi ? hi : s);
    }
    const int64_t v = s + win[d];
    if (!g.clamp && (v < 0 || v >= g.dims_x[d])) return false;
    lin += v * g.stride_x[d];
  }
  *x_lin = lin;
  return true;
}

__device__ __forceinline__ void copy_bytes(const void* src, int64_t s, void* dst, int64_t d,
                                           int esize) {
  switch (esize) {
    case 1: ((uint8_t*)dst)[d] = ((const uint8_t*)src)[s]; break;
    case 2: ((uint16_t*)dst)[d] = ((const uint16_t*)src)[s]; break;
    case 4: ((uint32_t*)dst)[d] = ((const uint32_t*)src)[s]; break;
    default: ((uint64_t*)dst)[d] = ((const uint64_t*)src)[s]; break;
  }
}

__device__ __forceinline__ float combine_f(int op, float a, float b) {
  switch (op) {
    case kScatterAdd: return a + b;
    case kScatterMax: return (a != a || b != b) ? __builtin_nanf("") : (a > b ? a : b);
    case kScatterMin: return (a != a || b != b) ? __builtin_nanf("") : (a < b ? a : b);
    case kScatterMul: return a * b;
    default: return b;
  }
}

__device__ __forceinline__ uint32_t combine_i(int op, bool sgn, uint32_t a, uint32_t b) {
  switch (op) {
    case kScatterAdd: return a + b;
    case kScatterMax: return sgn ? ((int32_t)a > (int32_t)b ? a : b) : (a > b ? a : b);
    case kScatterMin: return sgn ? ((int32_t)a < (int32_t)b ? a : b) : (a < b ? a : b);
    case kScatterMul: return a * b;
    default: return b;
  }
}

__device__ __forceinline__ float half_to_f(uint32_t h, bool bf) {
  if (bf) return __uint_as_float(h << 16);
  _Float16 x;
  const uint16_t u = (uint16_t)h;
  __builtin_memcpy(&x, &u, 2);
  return (float)x;
}

__device__ __forceinline__ uint32_t f_to_half(float f, bool bf) {
  if (bf) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;  // quiet NaN
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;                   // round to nearest even
  }
  const _Float16 x = (_Float16)f;
  uint16_t u;
  __builtin_memcpy(&u, &x, 2);
  return u;
}

// out[d] = op(out[d], src[s]) as one atomic read-modify-write.
__device__ void update(const IndexMapArgs& g, int64_t s, int64_t d) {
  if (g.op == kScatterReplace) {
    copy_bytes(g.src, s, g.out, d, g.esize);
    return;
  }
  if (g.dtype == kF32) {
    float* p = (float*)g.out + d;
    const float v = ((const float*)g.src)[s];
    if (g.op == kScatterAdd) {
      atomicAdd(p, v);
      return;
    }
    unsigned int* q = (unsigned int*)p;
    unsigned int old = *q, seen;
    do {
      seen = old;
      old = atomicCAS(q, seen, __float_as_uint(combine_f(g.op, __uint_as_float(seen), v)));
    } while (old != seen);
    return;
  }
  if (g.dtype == kI32 || g.dtype == kU32) {
    unsigned int* q = (unsigned int*)g.out + d;
    const uint32_t v = ((const uint32_t*)g.src)[s];
    if (g.op == kScatterAdd) {
      atomicAdd(q, v);
      return;
    }
    unsigned int old = *q, seen;
    do {
      seen = old;
      old = atomicCAS(q, seen, combine_i(g.op, g.dtype == kI32, seen, v));
    } while (old != seen);
    return;
  }
  // bf16 / f16: compare-and-swap on the aligned 32-bit word holding the element
  const bool bf = g.dtype == kBF16;
  const uintptr_t a = (uintptr_t)((uint16_t*)g.out + d);
  unsigned int* q = (unsigned int*)(a & ~(uintptr_t)3);
  const int sh = (int)(a & 2) * 8;
  const float v = half_to_f(((const uint16_t*)g.src)[s], bf);
  unsigned int old = *q, seen;
  do {
    seen = old;
    const float cur = half_to_f((seen >> sh) & 0xffffu, bf);
    const uint32_t nh = f_to_half(combine_f(g.op, cur, v), bf);
    old = atomicCAS(q, seen, (seen & ~(0xffffu << sh)) | (nh << sh));
  } while (old != seen);
}

}  // namespace

__global__ void __launch_bounds__(256) gather_nd_kernel(IndexMapArgs g) {
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < g.total; t += step) {
    int64_t x = 0;
    map_element(g, t, &x);
    copy_bytes(g.src, x, g.out, t, g.esize);
  }
}

__global__ void __launch_bounds__(256) scatter_kernel(IndexMapArgs g) {
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < g.total; t += step) {
    int64_t x = 0;
    if (map_element(g, t, &x)) update(g, t, x);
  }
}

static unsigned index_map_grid(int64_t total) {
  const int64_t b = (total + 255) / 256;
  return (unsigned)(b < 65536 ? b : 65536);
}

void launch_gather_nd(const IndexMapArgs& g, hipStream_t stream) {
  if (g.total == 0) return;
  hipLaunchKernelGGL(gather_nd_kernel, dim3(index_map_grid(g.total)), dim3(256), 0, stream, g);
  REW_HIP(hipGetLastError());
}

void launch_scatter(const IndexMapArgs& g, hipStream_t stream) {
  if (g.total == 0) return;
  hipLaunchKernelGGL(scatter_kernel, dim3(index_map_grid(g.total)), dim3(256), 0, stream, g);
  REW_HIP(hipGetLastError());
}


// ---- pad / dynamicSlice / dynamicUpdateSlice -----------------------------------------

namespace {

// Start scalar d of a dynamic slice / update, clamped into [0, room]
// (stablehlo.dynamic_slice / dynamic_update_slice); a uint64 start above
// INT64_MAX is past every extent, so it clamps to room.
__device__ __forceinline__ int64_t window_start(const WindowArgs& a, int d, int64_t room) {
  int64_t s = load_index(a.start[d], a.start_dt[d], 0);
  if (a.start_dt[d] == REW_DT_UINT64 && s < 0) s = room;
  return s < 0 ? 0 : (s > room ? room : s);
}

__global__ void __launch_bounds__(256) window_kernel(WindowArgs a) {
  int64_t st[8];
  for (int d = 0; d < a.rank; ++d)
    st[d] = a.mode == kWinSlice    ? window_start(a, d, a.x_dims[d] - a.out_dims[d])
            : a.mode == kWinUpdate ? window_start(a, d, a.x_dims[d] - a.y_dims[d])
                                   : 0;
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < a.total; t += step) {
    // coordinates of result element t, innermost dim first
    int64_t rem = t, xl = 0, yl = 0, xs = 1, ys = 1;
    bool in_x = true, in_y = true;
    for (int d = a.rank - 1; d >= 0; --d) {
      const int64_t o = rem % a.out_dims[d];
      rem /= a.out_dims[d];
      if (a.mode == kWinPad) {
        const int64_t p = o - a.lo[d];
        const int64_t i = p / a.step[d];
        in_x = in_x && p >= 0 && p == i * a.step[d] && i < a.x_dims[d];
        xl += i * xs;
      } else if (a.mode == kWinSlice) {
        xl += (o + st[d]) * xs;
      } else {
        const int64_t u = o - st[d];
        in_y = in_y && u >= 0 && u < a.y_dims[d];
        yl += u * ys;
        xl += o * xs;
      }
      xs *= a.x_dims[d];
      ys *= a.y_dims[d];
    }
    if (a.mode == kWinPad) {
      if (in_x) copy_bytes(a.x, xl, a.out, t, a.esize);
      else copy_bytes(a.y, 0, a.out, t, a.esize);
    } else if (a.mode == kWinUpdate && in_y) {
      copy_bytes(a.y, yl, a.out, t, a.esize);
    } else {
      copy_bytes(a.x, xl, a.out, t, a.esize);
    }
  }
}

// One matrix per workgroup, in LDS.  Column j: the pivot
// d = sqrt(a_jj - sum_{k<j} l_jk^2), then every row i > j in parallel
// l_ij = (a_ij - sum_{k<j} l_ik l_jk) / d, the sums in k order.  The upper
// form factors the transpose of the upper triangle the same way.
template <typename T>
__global__ void __launch_bounds__(256) cholesky_kernel(CholeskyArgs a) {
  __shared__ T L[kCholMaxN][kCholMaxN + 1];
  const int n = (int)a.n;
  const T* x = (const T*)a.x + blockIdx.x * a.n * a.n;
  T* out = (T*)a.out + blockIdx.x * a.n * a.n;
  for (int e = threadIdx.x; e < n * n; e += blockDim.x) {
    const int i = e / n, j = e % n;
    // L[i][j] (i >= j) from the referenced triangle
    if (i >= j) L[i][j] = a.lower ? x[(int64_t)i * n + j] : x[(int64_t)j * n + i];
  }
  __syncthreads();
  for (int j = 0; j < n; ++j) {
    if (threadIdx.x == 0) {
      T s = L[j][j];
      for (int k = 0; k < j; ++k) s -= L[j][k] * L[j][k];
      L[j][j] = sqrt(s);
    }
    __syncthreads();
    const T d = L[j][j];
    for (int i = j + 1 + threadIdx.x; i < n; i += blockDim.x) {
      T s = L[i][j];
      for (int k = 0; k < j; ++k) s -= L[i][k] * L[j][k];
      L[i][j] = s / d;
    }
    __syncthreads();
  }
  for (int e = threadIdx.x; e < n * n; e += blockDim.x) {
    const int i = e / n, j = e % n;
    T v = 0;
    if (a.lower && i >= j) v = L[i][j];
    if (!a.lower && j >= i) v = L[j][i];
    out[e] = v;
  }
}

// Triangular solve: T = op(a) restricted to the referenced triangle;
// right-side systems x T = b are T^T x^T = b^T, solved per row of b.
template <typename T>
__global__ void __launch_bounds__(256) trisolve_kernel(TriSolveArgs p) {
  __shared__ T A[kCholMaxN][kCholMaxN + 1];
  const int n = (int)p.n;
  const int64_t m = p.m;
  const T* a = (const T*)p.a + (int64_t)blockIdx.x * n * n;
  const T* b = (const T*)p.b + (int64_t)blockIdx.x * n * m;
  T* x = (T*)p.out + (int64_t)blockIdx.x * n * m;
  for (int e = threadIdx.x; e < n * n; e += blockDim.x) {
    const int i = e / n, j = e % n;
    const bool ref = p.lower ? i >= j : j >= i;
    A[i][j] = ref ? a[e] : T(0);
  }
  __syncthreads();
  // effective matrix of the column system: E = op(a) (left) or op(a)^T
  // (right); E(i, k) = A[k][i] when exactly one of (trans, right) holds
  const bool flip = (bool)p.trans != !p.left;
  const bool low = (bool)p.lower != flip;  // E is lower triangular
  for (int64_t r = threadIdx.x; r < m; r += blockDim.x) {
    // element i of right-hand side r: b[i, r] (left) or b[r, i] (right)
    const int64_t si = p.left ? m : 1, sr = p.left ? 1 : n;
    for (int s = 0; s < n; ++s) {
      const int i = low ? s : n - 1 - s;
      T acc = b[i * si + r * sr];
      if (low) {
        for (int k = 0; k < i; ++k) acc -= (flip ? A[k][i] : A[i][k]) * x[k * si + r * sr];
      } else {
        for (int k = i + 1; k < n; ++k) acc -= (flip ? A[k][i] : A[i][k]) * x[k * si + r * sr];
      }
      x[i * si + r * sr] = p.unit ? acc : acc / A[i][i];
    }
  }
}

__global__ void __launch_bounds__(256) complex_kernel(ComplexArgs a) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= a.n) return;
  const int w = a.esize;
  auto cp = [&](void* dst, const void* src) {
    if (w == 8) *(uint64_t*)dst = *(const uint64_t*)src;
    else if (w == 4) *(uint32_t*)dst = *(const uint32_t*)src;
    else *(uint16_t*)dst = *(const uint16_t*)src;
  };
  uint8_t* o = (uint8_t*)a.out;
  const uint8_t* x = (const uint8_t*)a.x;
  switch (a.mode) {
    case 0:
      cp(o + 2 * i * w, x + i * w);
      cp(o + (2 * i + 1) * w, (const uint8_t*)a.y + i * w);
      break;
    case 1: cp(o + i * w, x + 2 * i * w); break;
    case 2: cp(o + i * w, x + (2 * i + 1) * w); break;
    case 3: cp(o + i * w, x + i * w); break;
    default: {
      const uint64_t z = 0;
      cp(o + i * w, &z);
    }
  }
}

template <typename T>
__global__ void __launch_bounds__(256) fft1_kernel(Fft1Args a) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = a.outer * a.len_out * a.inner;
  if (i >= total) return;
  const int64_t in_ = i % a.inner, k = (i / a.inner) % a.len_out, o = i / (a.inner * a.len_out);
  const int64_t n = a.n;
  const int64_t base = o * a.len_in * a.inner + in_;  // element (o, 0, in_) of x
  const T* x = (const T*)a.x;
  T* out = (T*)a.out;
  double re = 0.0, im = 0.0;
  const double sgn = a.mode == 1 || a.mode == 3 ? 1.0 : -1.0;
  auto tw = [&](int64_t j, double* c, double* s) {
    const int64_t r = (k * j) % n;  // exp(sgn 2 pi i r / n)
    double sp, cp;
    sincospi(2.0 * (double)r / (double)n, &sp, &cp);
    *c = cp;
    *s = sgn * sp;
  };
  if (a.mode == 3) {
    // real output: x[k] = (1/n)(Re X0 + 2 sum_{0<j<(n+1)/2} Re(X_j w^{jk}) + [n even] Re X_{n/2} (-1)^k)
    const int64_t h = (n + 1) / 2;
    for (int64_t j = 0; j < a.len_in && j <= n / 2; ++j) {
      const T* z = x + 2 * (base + j * a.inner);
      double c, s;
      tw(j, &c, &s);
      const double v = (double)z[0] * c - (double)z[1] * s;
      if (j == 0) re += (double)z[0];
      else if (j < h) re += 2.0 * v;
      else re += (double)z[0] * c;  // j == n / 2, n even: (-1)^k Re X
    }
    out[i] = (T)(re / (double)n);
    return;
  }
  for (int64_t j = 0; j < a.len_in; ++j) {
    double xr, xi = 0.0;
    if (a.mode == 2) {
      xr = (double)x[base + j * a.inner];
    } else {
      const T* z = x + 2 * (base + j * a.inner);
      xr = (double)z[0];
      xi = (double)z[1];
    }
    double c, s;
    tw(j, &c, &s);
    re += xr * c - xi * s;
    im += xr * s + xi * c;
  }
  if (a.mode == 1) {
    re /= (double)n;
    im /= (double)n;
  }
  out[2 * i] = (T)re;
  out[2 * i + 1] = (T)im;
}

}  // namespace

void launch_complex(const ComplexArgs& a, hipStream_t stream) {
  if (a.n == 0) return;
  if (a.esize != 2 && a.esize != 4 && a.esize != 8)
    fail(REW_MI355X_ERR_INVALID, "internal: complex launch outside its limits");
  hipLaunchKernelGGL(complex_kernel, dim3((unsigned)((a.n + 255) / 256)), dim3(256), 0, stream, a);
  REW_HIP(hipGetLastError());
}

void launch_fft1(const Fft1Args& a, hipStream_t stream) {
  const int64_t total = a.outer * a.len_out * a.inner;
  if (total == 0) return;
  if (a.n <= 0 || total > (int64_t)0x7fffffff * 256)
    fail(REW_MI355X_ERR_INVALID, "internal: fft launch outside its limits");
  const dim3 grid((unsigned)((total + 255) / 256));
  if (a.f64) hipLaunchKernelGGL(fft1_kernel<double>, grid, dim3(256), 0, stream, a);
  else hipLaunchKernelGGL(fft1_kernel<float>, grid, dim3(256), 0, stream, a);
  REW_HIP(hipGetLastError());
}

void launch_trisolve(const TriSolveArgs& a, hipStream_t stream) {
  if (a.batch == 0 || a.n == 0 || a.m == 0) return;
  if (a.n > kCholMaxN || a.batch > 0x7fffffff)
    fail(REW_MI355X_ERR_INVALID, "internal: triangularSolve launch outside its limits");
  if (a.f64) hipLaunchKernelGGL(trisolve_kernel<double>, dim3((unsigned)a.batch), dim3(256), 0, stream, a);
  else hipLaunchKernelGGL(trisolve_kernel<float>, dim3((unsigned)a.batch), dim3(256), 0, stream, a);
  REW_HIP(hipGetLastError());
}

void launch_window(const WindowArgs& a, hipStream_t stream) {
  if (a.total == 0) return;
  if (a.rank < 0 || a.rank > 8 || (a.esize != 1 && a.esize != 2 && a.esize != 4 && a.esize != 8))
    fail(REW_MI355X_ERR_INVALID, "internal: window launch outside its limits");
  hipLaunchKernelGGL(window_kernel, dim3(index_map_grid(a.total)), dim3(256), 0, stream, a);
  REW_HIP(hipGetLastError());
}

void launch_cholesky(const CholeskyArgs& a, hipStream_t stream) {
  if (a.batch == 0 || a.n == 0) return;
  if (a.n > kCholMaxN || a.batch > 0x7fffffff)
    fail(REW_MI355X_ERR_INVALID, "internal: cholesky launch outside its limits");
  if (a.f64) hipLaunchKernelGGL(cholesky_kernel<double>, dim3((unsigned)a.batch), dim3(256), 0, stream, a);
  else hipLaunchKernelGGL(cholesky_kernel<float>, dim3((unsigned)a.batch), dim3(256), 0, stream, a);
  REW_HIP(hipGetLastError());
}

// ---- batch norm ----------------------------------------------------------------------

namespace {

template <typename T>
__device__ __forceinline__ T bn_norm(T x, T m, T v, double eps) {
  return (x - m) / sqrt(v + (T)eps);
}

template <typename T>
__global__ void __launch_bounds__(256) bn_inference_kernel(BatchNormArgs a) {
  const T *x = (const T*)a.x, *sc = (const T*)a.scale, *of = (const T*)a.offset;
  const T *mu = (const T*)a.mean, *va = (const T*)a.var;
  T* y = (T*)a.out0;
  const int64_t total = a.outer * a.C * a.inner;
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += step) {
    const int64_t c = (t / a.inner) % a.C;
    y[t] = sc[c] * bn_norm<T>(x[t], mu[c], va[c], a.eps) + of[c];
  }
}

// Workgroup sum of v (fixed tree: wave butterfly, then the four wave sums).
template <typename T>
__device__ __forceinline__ T bn_block_sum(T v, T* part) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  __syncthreads();  // part may still be read from the previous sum
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
  __syncthreads();
  return (part[0] + part[1]) + (part[2] + part[3]);
}

template <typename T>
__global__ void __launch_bounds__(256) bn_feature_kernel(BatchNormArgs a) {
  __shared__ T part[4];
  const int64_t c = blockIdx.x;
  const int64_t n = a.outer * a.inner;
  const T *x = (const T*)a.x, *sc = (const T*)a.scale;
  auto at = [&](int64_t i) { return (i / a.inner) * a.C * a.inner + c * a.inner + i % a.inner; };
  if (a.mode == kBnTraining) {
    const T* of = (const T*)a.offset;
    T s = 0;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) s += x[at(i)];
    const T mean = bn_block_sum<T>(s, part) / (T)n;
    T q = 0;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
      const T d = x[at(i)] - mean;
      q += d * d;
    }
    const T var = bn_block_sum<T>(q, part) / (T)n;
    if (threadIdx.x == 0) {
      ((T*)a.out1)[c] = mean;
      ((T*)a.out2)[c] = var;
    }
    T* y = (T*)a.out0;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x)
      y[at(i)] = sc[c] * bn_norm<T>(x[at(i)], mean, var, a.eps) + of[c];
  } else {
    const T *dy = (const T*)a.dy, mean = ((const T*)a.mean)[c], var = ((const T*)a.var)[c];
    T sg = 0, sgx = 0;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
      const T g = dy[at(i)];
      sg += g;
      sgx += g * bn_norm<T>(x[at(i)], mean, var, a.eps);
    }
    const T d_off = bn_block_sum<T>(sg, part);
    const T d_sc = bn_block_sum<T>(sgx, part);
    if (threadIdx.x == 0) {
      ((T*)a.out1)[c] = d_sc;
      ((T*)a.out2)[c] = d_off;
    }
    const T stddev = sqrt(var + (T)a.eps);
    T* dx = (T*)a.out0;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
      const T xn = bn_norm<T>(x[at(i)], mean, var, a.eps);
      dx[at(i)] = sc[c] / stddev * (dy[at(i)] - d_off / (T)n - xn * d_sc / (T)n);
    }
  }
}

}  // namespace

void launch_batchnorm(const BatchNormArgs& a, hipStream_t stream) {
  const int64_t total = a.outer * a.C * a.inner;
  // an empty batch (outer * inner == 0, C > 0) still writes the [C] outputs
  // of training and grad: 0 / 0 = NaN statistics and zero gradient sums, as
  // the feature kernel's empty loops give
  if (a.C == 0 || (total == 0 && a.mode == kBnInference)) return;
  if (a.mode == kBnInference) {
    const unsigned grid = index_map_grid(total);
    if (a.f64) hipLaunchKernelGGL(bn_inference_kernel<double>, dim3(grid), dim3(256), 0, stream, a);
    else hipLaunchKernelGGL(bn_inference_kernel<float>, dim3(grid), dim3(256), 0, stream, a);
  } else {
    if (a.C > 0x7fffffff) fail(REW_MI355X_ERR_INVALID, "internal: batch norm launch outside its limits");
    if (a.f64) hipLaunchKernelGGL(bn_feature_kernel<double>, dim3((unsigned)a.C), dim3(256), 0, stream, a);
    else hipLaunchKernelGGL(bn_feature_kernel<float>, dim3((unsigned)a.C), dim3(256), 0, stream, a);
  }
  REW_HIP(hipGetLastError());
}

}  // namespace rew
