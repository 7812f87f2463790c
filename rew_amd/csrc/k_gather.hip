// torch_index_select (batch_dims = 0): row gather.
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
