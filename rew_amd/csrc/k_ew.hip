// Fused elementwise kernel: one vm::Program over a dense output space.
//
// HBM-bound by construction: each lane handles kVec consecutive elements of
// the innermost dimension with 16-byte (f32) / 8-byte (bf16) vector loads
// and stores where the leaf is contiguous; the opcode stream is
// wave-uniform scalar control flow.
#include "kernels.h"
#include "vm_device.h"

namespace rew {

using namespace vm;

template <int V>
__global__ void __launch_bounds__(256) ew_kernel(Program P, Space S) {
  const uint32_t nvec = (uint32_t)(S.numel / V);
  const uint32_t stride = gridDim.x * blockDim.x;
  for (uint32_t t = blockIdx.x * blockDim.x + threadIdx.x; t < nvec; t += stride) {
    const uint32_t lin = t * V;
    int32_t coord[kRank];
    delinearize(S, lin, coord);
    Regs<V> R;
    run<V>(P, S.rank, coord, lin, R);
    for (int o = 0; o < P.n_outs; ++o) {
      uint32_t v[V];
      rget<V>(R, P.out[o].reg, v);
      store_vec<V>(P.out[o].ptr, P.out[o].dtype, (int64_t)P.out[o].off + lin, v);
    }
  }
}

void launch_ew(const vm::Program& P, const vm::Space& S, bool vec,
               hipStream_t stream) {
  if (S.numel == 0) return;
  if (jit_launch_ew(P, S, vec, stream)) return;
  const int V = vec ? vm::kVec : 1;
  const int64_t nvec = S.numel / V;
  int64_t blocks = (nvec + 255) / 256;
  if (blocks > 256 * 64) blocks = 256 * 64;
  if (vec)
    hipLaunchKernelGGL(ew_kernel<vm::kVec>, dim3((unsigned)blocks), dim3(256), 0,
                       stream, P, S);
  else
    hipLaunchKernelGGL(ew_kernel<1>, dim3((unsigned)blocks), dim3(256), 0,
                       stream, P, S);
  REW_HIP(hipGetLastError());
}

}  // namespace rew
