// Routed mixture-of-experts: token placement and the ordered combine.
//
// rew's DeepSeekMoE.forward (src/rew/models/deepseek.nim:122-145) runs every
// routed expert on every token and adds `expert(x) * w_e(x)` into the
// running output in expert order, where
//   w_e(x)[t] = reduceSum(topWeights[t, :] * (topIndices[t, :] == e))
// (routedWeightForExpert, deepseek.nim:114-120) is zero unless e is one of
// token t's top-k experts.  A zero weight makes the whole contribution an
// exact zero, so the backend evaluates each expert only on its routed rows:
//
//   moe_count_kernel  per-member row counts -> row offsets and 256-row tile
//                     starts (the grouped GEMMs' work lists);
//   moe_place_kernel  one workgroup per member: the tokens routed to it in
//                     ascending token order (a stable, ballot-based
//                     compaction, so the layout never depends on timing),
//                     and each (token, k-slot)'s packed row;
//   (grouped SwiGLU and down-projection GEMMs over the packed rows, k_gemm.hip)
//   moe_combine_kernel per token: start from the running sum before the
//                     first routed expert, then for the token's routed
//                     members in chain order add bf16(f32(y) * w) with bf16
//                     rounding after every add -- the dense op sequence's
//                     arithmetic on the only rows where it is non-zero.
#include <hip/hip_runtime.h>

#include "kernels.h"
#include "vm_device.h"

namespace rew {

__global__ void __launch_bounds__(1024) moe_count_kernel(MoeRouteArgs a) {
  extern __shared__ int cnt[];  // n_members
  for (int m = threadIdx.x; m < a.n_members; m += blockDim.x) cnt[m] = 0;
  __syncthreads();
  // a (token, expert) pair counts once even if the id repeats in the row
  // (topK ids are distinct; placement and combine use the first occurrence)
  const int64_t n = a.T * a.k;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
    const int e = a.topi[i];
    const int m = (e >= 0 && e < a.E) ? a.member_of[e] : -1;
    bool first = true;
    for (int64_t q = i - i % a.k; q < i; ++q) first &= a.topi[q] != e;
    if (m >= 0 && first) atomicAdd(&cnt[m], 1);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int off = 0, mt = 0;
    for (int m = 0; m < a.n_members; ++m) {
      a.off[m] = off;
      a.mt_start[m] = mt;
      off += cnt[m];
      mt += (cnt[m] + a.tile_m - 1) / a.tile_m;
    }
    a.off[a.n_members] = off;
    a.mt_start[a.n_members] = mt;
  }
}

__global__ void __launch_bounds__(256) moe_place_kernel(MoeRouteArgs a) {
  __shared__ int wave_tot[4];
  const int m = blockIdx.x;
  const int e = a.members[m];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int base = a.off[m];
  for (int64_t t0 = 0; t0 < a.T; t0 += 256) {
    const int64_t t = t0 + threadIdx.x;
    int j = -1;
    if (t < a.T)
      for (int q = a.k - 1; q >= 0; --q)
        if (a.topi[t * a.k + q] == e) j = q;  // first occurrence
    const uint64_t ball = __ballot(j >= 0);
    const int below = __popcll(ball & ((1ull << lane) - 1ull));
    if (lane == 0) wave_tot[wave] = __popcll(ball);
    __syncthreads();
    int pre = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      pre += w < wave ? wave_tot[w] : 0;
      tot += wave_tot[w];
    }
    if (j >= 0) {
      const int slot = base + pre + below;
      a.perm[slot] = (int32_t)t;
      a.slot_of[t * a.k + j] = slot;
    }
    base += tot;
    __syncthreads();  // wave_tot is rewritten by the next chunk
  }
}

// One workgroup per token row; each thread owns 8 consecutive columns.
// Thread 0 sorts the token's routed members into chain order in LDS.
__global__ void __launch_bounds__(256) moe_combine_kernel(MoeCombineArgs a) {
  __shared__ int s_slot[kMoeMaxK];
  __shared__ float s_w[kMoeMaxK];
  __shared__ int s_n;
  for (int64_t t = blockIdx.x; t < a.T; t += gridDim.x) {
    if (threadIdx.x == 0) {
      int mem[kMoeMaxK];
      int n = 0;
      for (int q = 0; q < a.k; ++q) {
        const int e = a.topi[t * a.k + q];
        const int m = (e >= 0 && e < a.E) ? a.member_of[e] : -1;
        bool first = true;
        for (int q2 = 0; q2 < q; ++q2) first &= a.topi[t * a.k + q2] != e;
        if (m < 0 || !first) continue;
        int p = n++;
        while (p > 0 && mem[p - 1] > m) {
          mem[p] = mem[p - 1];
          s_slot[p] = s_slot[p - 1];
          s_w[p] = s_w[p - 1];
          --p;
        }
        mem[p] = m;
        s_slot[p] = a.slot_of[t * a.k + q];
        s_w[p] = a.topw[t * a.k + q];
      }
      s_n = n;
    }
    __syncthreads();
    const int n = s_n;
    for (int64_t h = (int64_t)threadIdx.x * 8; h < a.H; h += 256 * 8) {
      const uint4 pv = *(const uint4*)(a.prev + t * a.prev_rs + h);
      const uint16_t* ph = (const uint16_t*)&pv;
      float acc[8];
#pragma unroll
      for (int x = 0; x < 8; ++x) acc[x] = vm::as_f((uint32_t)ph[x] << 16);
      for (int i = 0; i < n; ++i) {
        const float w = s_w[i];
        const uint4 yv = *(const uint4*)(a.y + (int64_t)s_slot[i] * a.H + h);
        const uint16_t* yh = (const uint16_t*)&yv;
#pragma unroll
        for (int x = 0; x < 8; ++x) {
          const float c = vm::round_bf16(vm::as_f((uint32_t)yh[x] << 16) * w);
          acc[x] = vm::round_bf16(acc[x] + c);
        }
      }
      uint16_t o[8];
#pragma unroll
      for (int x = 0; x < 8; ++x) o[x] = (uint16_t)(vm::as_u(acc[x]) >> 16);
      *(uint4*)(a.out + t * a.H + h) = *(const uint4*)o;
    }
    __syncthreads();  // the next token rewrites the LDS list
  }
}

void launch_moe_route(const MoeRouteArgs& a, hipStream_t stream) {
  if (a.n_members <= 0) return;
  if (a.k < 1 || a.k > kMoeMaxK || a.tile_m <= 0)
    fail(REW_MI355X_ERR_INVALID, "internal: MoE routing launch outside its limits");
  hipLaunchKernelGGL(moe_count_kernel, dim3(1), dim3(1024), (size_t)a.n_members * sizeof(int),
                     stream, a);
  REW_HIP(hipGetLastError());
  if (a.T == 0) return;
  hipLaunchKernelGGL(moe_place_kernel, dim3((unsigned)a.n_members), dim3(256), 0, stream, a);
  REW_HIP(hipGetLastError());
}

void launch_moe_combine(const MoeCombineArgs& a, hipStream_t stream) {
  if (a.T == 0) return;
  if (a.H % 8 || a.prev_rs % 8 || ((uintptr_t)a.prev & 15) || ((uintptr_t)a.y & 15) ||
      ((uintptr_t)a.out & 15) || a.k > kMoeMaxK)
    fail(REW_MI355X_ERR_INVALID, "internal: MoE combine launch outside its limits");
  const int64_t grid = a.T < 65536 ? a.T : 65536;
  hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)grid), dim3(256), 0, stream, a);
  REW_HIP(hipGetLastError());
}

}  // namespace rew
