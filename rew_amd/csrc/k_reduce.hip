// Reductions with a fused elementwise prologue.
//
// The kernel space is [kept dims..., reduced dims...]; the prologue program
// produces the value to reduce at each point, so `reduceSum(mul(x, x))` or a
// reduction over a transposed / broadcast view reads its source tensor once.
// Rows of >= 128 elements: one 256-thread workgroup per output, kVec-wide
// loads, wave64 shuffle tree then an LDS tree across the 4 waves.  Short
// rows: one thread per output.
#include "kernels.h"
#include "vm_device.h"

namespace rew {

using namespace vm;

__device__ __forceinline__ uint32_t red_init(int op) {
  switch (op) {
    case RED_SUM: return as_u(0.0f);
    case RED_MAX: return as_u(-INFINITY);
    case RED_MIN: return as_u(INFINITY);
    case RED_PROD: return as_u(1.0f);
    case RED_AND: return 1u;
    case RED_OR: return 0u;
    case RED_MAXI: return 0x80000000u;
    default: return 0x7fffffffu;  // RED_MINI
  }
}

__device__ __forceinline__ uint32_t red_op(int op, uint32_t a, uint32_t b) {
  switch (op) {
    case RED_SUM: return as_u(as_f(a) + as_f(b));
    case RED_MAX: return as_u(fmax_prop(as_f(a), as_f(b)));
    case RED_MIN: return as_u(fmin_prop(as_f(a), as_f(b)));
    case RED_PROD: return as_u(as_f(a) * as_f(b));
    case RED_AND: return (a != 0u) & (b != 0u);
    case RED_OR: return (a != 0u) | (b != 0u);
    case RED_MAXI: return (int32_t)a > (int32_t)b ? a : b;
    default: return (int32_t)a < (int32_t)b ? a : b;
  }
}

__device__ __forceinline__ uint32_t wave_reduce(int op, uint32_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = red_op(op, v, __shfl_xor(v, m, 64));
  return v;
}

template <int V>
__global__ void __launch_bounds__(256) reduce_rows_kernel(Program P, Space S,
                                                          ReduceArgs A) {
  __shared__ uint32_t part[4];
  const int reg = P.out[0].reg;
  for (uint32_t o = blockIdx.x; o < A.n_out; o += gridDim.x) {
    uint32_t acc = red_init(A.op);
    for (uint32_t r = threadIdx.x * V; r < A.n_red; r += 256 * V) {
      const uint32_t lin = o * A.n_red + r;
      int32_t coord[kRank];
      delinearize(S, lin, coord);
      Regs<V> R;
      run<V>(P, S.rank, coord, lin, R);
      uint32_t v[V];
      rget<V>(R, reg, v);
#pragma unroll
      for (int j = 0; j < V; ++j) acc = red_op(A.op, acc, v[j]);
    }
    acc = wave_reduce(A.op, acc);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) part[w] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
      uint32_t x = red_op(A.op, red_op(A.op, part[0], part[1]),
                          red_op(A.op, part[2], part[3]));
      store_scalar(A.out, A.out_dtype, o, x);
    }
    __syncthreads();
  }
}

__global__ void __launch_bounds__(256) reduce_small_kernel(Program P, Space S,
                                                           ReduceArgs A) {
  const int reg = P.out[0].reg;
  for (uint32_t o = blockIdx.x * 256 + threadIdx.x; o < A.n_out;
       o += gridDim.x * 256) {
    uint32_t acc = red_init(A.op);
    for (uint32_t r = 0; r < A.n_red; ++r) {
      const uint32_t lin = o * A.n_red + r;
      int32_t coord[kRank];
      delinearize(S, lin, coord);
      Regs<1> R;
      run<1>(P, S.rank, coord, lin, R);
      uint32_t v[1];
      rget<1>(R, reg, v);
      acc = red_op(A.op, acc, v[0]);
    }
    store_scalar(A.out, A.out_dtype, o, acc);
  }
}

// reduceMean's divide after an interpreted reduction: y = x / d (f32)
__global__ void __launch_bounds__(256) div_scalar_kernel(const float* x, float* y, uint32_t n,
                                                         float d) {
  for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) y[i] = x[i] / d;
}

void launch_reduce(const vm::Program& P, const vm::Space& S,
                   const ReduceArgs& A, bool vec, hipStream_t stream) {
  if (A.n_out == 0) return;
  if (jit_launch_reduce(P, S, A, vec, stream)) return;
  if (A.n_mean > 0) {
    // the interpreter stores the sums, then divides them
    ReduceArgs plain = A;
    plain.n_mean = 0;
    launch_reduce(P, S, plain, vec, stream);
    const unsigned blocks = (A.n_out + 255) / 256 < 65536 ? (A.n_out + 255) / 256 : 65536;
    for (int x = 0; x < A.n_mean; ++x) {
      const void* src = A.mean_src[x] ? A.extra_out[A.mean_src[x] - 1] : A.out;
      hipLaunchKernelGGL(div_scalar_kernel, dim3(blocks), dim3(256), 0, stream,
                         (const float*)src, (float*)A.mean_out[x], A.n_out, A.mean_div[x]);
    }
    REW_HIP(hipGetLastError());
    return;
  }
  if (A.n_extra > 0) {
    // the interpreter reduces one op per pass
    for (int x = -1; x < A.n_extra; ++x) {
      ReduceArgs one = A;
      one.n_extra = 0;
      if (x >= 0) {
        one.op = A.extra_op[x];
        one.out = A.extra_out[x];
      }
      launch_reduce(P, S, one, vec, stream);
    }
    return;
  }
  if (A.n_red >= 128) {
    int64_t blocks = A.n_out < 65536 ? A.n_out : 65536;
    if (vec)
      hipLaunchKernelGGL(reduce_rows_kernel<vm::kVec>, dim3((unsigned)blocks),
                         dim3(256), 0, stream, P, S, A);
    else
      hipLaunchKernelGGL(reduce_rows_kernel<1>, dim3((unsigned)blocks), dim3(256),
                         0, stream, P, S, A);
  } else {
    int64_t blocks = (A.n_out + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(reduce_small_kernel, dim3((unsigned)blocks), dim3(256), 0,
                       stream, P, S, A);
  }
  REW_HIP(hipGetLastError());
}

}  // namespace rew
