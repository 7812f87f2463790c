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
//   moe_count / moe_scan / moe_place  per-member row counts -> row offsets
//                     and 256-row tile starts (the grouped GEMMs' work
//                     lists), and each member's tokens in ascending token
//                     order with each (token, k-slot)'s packed row: counts
//                     and ballot ranks only, so the layout never depends on
//                     timing;
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

// Token placement in three launches over blocks of kMoeRouteBlock tokens
// (256, one per thread):
//   moe_count_kernel  each block's per-member counts (LDS atomics: a count
//                     does not depend on the order of its increments);
//   moe_scan_kernel   per member, the exclusive prefix of the block counts
//                     (in block order) and the total; then the members'
//                     row offsets and tile starts;
//   moe_place_kernel  each block ranks its tokens per member in token order
//                     (per-wave counts, then ballots within each wave) and
//                     writes the packed rows.
// A (token, expert) pair counts once even if the id repeats in the row
// (topK ids are distinct; placement and combine use the first occurrence).

// member of token t's slot q, or -1 (off the chain, or a repeated id)
__device__ __forceinline__ int route_member(const MoeRouteArgs& a, int64_t t, int q) {
  const int e = a.topi[t * a.k + q];
  if (e < 0 || e >= a.E) return -1;
  for (int q2 = 0; q2 < q; ++q2)
    if (a.topi[t * a.k + q2] == e) return -1;
  return a.member_of[e];
}

__global__ void __launch_bounds__(256) moe_count_kernel(MoeRouteArgs a) {
  extern __shared__ int cnt[];  // n_members
  for (int m = threadIdx.x; m < a.n_members; m += 256) cnt[m] = 0;
  __syncthreads();
  const int64_t t = (int64_t)blockIdx.x * kMoeRouteBlock + threadIdx.x;
  if (t < a.T)
    for (int q = 0; q < a.k; ++q) {
      const int m = route_member(a, t, q);
      if (m >= 0) atomicAdd(&cnt[m], 1);
    }
  __syncthreads();
  int32_t* out = a.blk_cnt + (int64_t)blockIdx.x * a.n_members;
  for (int m = threadIdx.x; m < a.n_members; m += 256) out[m] = cnt[m];
}

__global__ void __launch_bounds__(1024) moe_scan_kernel(MoeRouteArgs a, int nblk) {
  extern __shared__ int tot[];  // n_members
  for (int m = threadIdx.x; m < a.n_members; m += 1024) {
    int run = 0;
    for (int b = 0; b < nblk; ++b) {
      int32_t* p = a.blk_cnt + (int64_t)b * a.n_members + m;
      const int c = *p;
      *p = run;
      run += c;
    }
    tot[m] = run;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int off = 0, mt = 0;
    for (int m = 0; m < a.n_members; ++m) {
      a.off[m] = off;
      a.mt_start[m] = mt;
      off += tot[m];
      mt += (tot[m] + a.tile_m - 1) / a.tile_m;
    }
    a.off[a.n_members] = off;
    a.mt_start[a.n_members] = mt;
  }
}

__global__ void __launch_bounds__(256) moe_place_kernel(MoeRouteArgs a) {
  extern __shared__ int sh[];  // base [n], wave counts [4][n]
  int* base = sh;
  int* wcnt = sh + a.n_members;
  const int n = a.n_members;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int32_t* pre = a.blk_cnt + (int64_t)blockIdx.x * n;
  for (int m = threadIdx.x; m < n; m += 256) {
    base[m] = a.off[m] + pre[m];
    for (int w = 0; w < 4; ++w) wcnt[w * n + m] = 0;
  }
  __syncthreads();
  const int64_t t = (int64_t)blockIdx.x * kMoeRouteBlock + threadIdx.x;
  int mem[kMoeMaxK];  // fully unrolled: stays in registers
#pragma unroll
  for (int q = 0; q < kMoeMaxK; ++q) {
    mem[q] = (q < a.k && t < a.T) ? route_member(a, t, q) : -1;
    if (mem[q] >= 0) atomicAdd(&wcnt[wave * n + mem[q]], 1);
  }
  __syncthreads();
  // rows before this wave's: the block's base plus the earlier waves' counts
  const uint64_t lt = (1ull << lane) - 1ull;
  for (int m = 0; m < n; ++m) {
    int j = -1;
#pragma unroll
    for (int q = kMoeMaxK - 1; q >= 0; --q)
      if (mem[q] == m) j = q;
    const uint64_t ball = __ballot(j >= 0);
    if (j >= 0) {
      int slot = base[m] + __popcll(ball & lt);
      for (int w = 0; w < wave; ++w) slot += wcnt[w * n + m];
      a.perm[slot] = (int32_t)t;
      a.slot_of[t * a.k + j] = slot;
    }
  }
}

// One wave per token (four per workgroup).  Lanes q < k take slot q: its
// member (off the chain or a repeated id: none), its packed row and weight,
// and its rank among the token's members in chain order (shuffles, no
// shared memory).  Then each lane owns 8-column chunks of the row: the
// token's expert rows for a chunk are loaded eight at a time before the
// ordered, rounded accumulation runs over them.
__global__ void __launch_bounds__(256) moe_combine_kernel(MoeCombineArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t waves = (int64_t)gridDim.x * 4;
  for (int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); t < a.T; t += waves) {
    int e = -1, m = -1, slot = 0;
    float w = 0.0f;
    if (lane < a.k) e = a.topi[t * a.k + lane];
    bool valid = false;
    if (lane < a.k && e >= 0 && e < a.E) {
      m = a.member_of[e];
      valid = m >= 0;
    }
    for (int q2 = 0; q2 < a.k; ++q2) {
      const int e2 = __shfl(e, q2, 64);
      if (q2 < lane && e2 == e) valid = false;  // a repeated id counts once
    }
    if (valid) {
      slot = a.slot_of[t * a.k + lane];
      w = a.topw[t * a.k + lane];
    }
    int rank = 0;
    for (int q2 = 0; q2 < a.k; ++q2) {
      const int m2 = __shfl(m, q2, 64);
      const int v2 = __shfl(valid ? 1 : 0, q2, 64);
      if (v2 && m2 < m) ++rank;
    }
    const int n = __popcll(__ballot(valid));
    // the i-th member in chain order: its packed row and weight (wave-uniform)
    int si[kMoeMaxK];
    float wi[kMoeMaxK];
#pragma unroll
    for (int i = 0; i < kMoeMaxK; ++i) {
      si[i] = 0;
      wi[i] = 0.0f;
      if (i < n) {
        const uint64_t bi = __ballot(valid && rank == i);
        const int src = (int)__builtin_ctzll(bi);
        si[i] = __builtin_amdgcn_readfirstlane(__shfl(slot, src, 64));
        wi[i] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(__shfl(w, src, 64))));
      }
    }
    for (int64_t h = (int64_t)lane * 8; h < a.H; h += 64 * 8) {
      const uint4 pv = *(const uint4*)(a.prev + t * a.prev_rs + h);
      const uint16_t* ph = (const uint16_t*)&pv;
      float acc[8];
#pragma unroll
      for (int x = 0; x < 8; ++x) acc[x] = vm::as_f((uint32_t)ph[x] << 16);
      // rows in groups of 8, each group's loads issued together
#pragma unroll
      for (int i0 = 0; i0 < kMoeMaxK; i0 += 8) {
        if (i0 >= n) break;
        uint4 yv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (i0 + i < n) yv[i] = *(const uint4*)(a.y + (int64_t)si[i0 + i] * a.H + h);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          if (i0 + i < n) {
            const uint16_t* yh = (const uint16_t*)&yv[i];
#pragma unroll
            for (int x = 0; x < 8; ++x) {
              const float c = vm::round_bf16(vm::as_f((uint32_t)yh[x] << 16) * wi[i0 + i]);
              acc[x] = vm::round_bf16(acc[x] + c);
            }
          }
        }
      }
      uint16_t o[8];
#pragma unroll
      for (int x = 0; x < 8; ++x) o[x] = (uint16_t)(vm::as_u(acc[x]) >> 16);
      *(uint4*)(a.out + t * a.H + h) = *(const uint4*)o;
    }
  }
}

void launch_moe_route(const MoeRouteArgs& a, hipStream_t stream) {
  if (a.n_members <= 0) return;
  if (a.k < 1 || a.k > kMoeMaxK || a.tile_m <= 0 || a.n_members > 3200)
    fail(REW_MI355X_ERR_INVALID, "internal: MoE routing launch outside its limits");
  const int nblk = (int)((a.T + kMoeRouteBlock - 1) / kMoeRouteBlock);
  const size_t n4 = (size_t)a.n_members * sizeof(int);
  if (nblk > 0) {
    hipLaunchKernelGGL(moe_count_kernel, dim3((unsigned)nblk), dim3(256), n4, stream, a);
    REW_HIP(hipGetLastError());
  }
  hipLaunchKernelGGL(moe_scan_kernel, dim3(1), dim3(1024), n4, stream, a, nblk);
  REW_HIP(hipGetLastError());
  if (nblk == 0) return;
  hipLaunchKernelGGL(moe_place_kernel, dim3((unsigned)nblk), dim3(256), 5 * n4, stream, a);
  REW_HIP(hipGetLastError());
}

void launch_moe_combine(const MoeCombineArgs& a, hipStream_t stream) {
  if (a.T == 0) return;
  if (a.H % 8 || a.prev_rs % 8 || ((uintptr_t)a.prev & 15) || ((uintptr_t)a.y & 15) ||
      ((uintptr_t)a.out & 15) || a.k > kMoeMaxK)
    fail(REW_MI355X_ERR_INVALID, "internal: MoE combine launch outside its limits");
  const int64_t blocks = (a.T + 3) / 4;
  const int64_t grid = blocks < 65536 ? blocks : 65536;
  hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)grid), dim3(256), 0, stream, a);
  REW_HIP(hipGetLastError());
}

}  // namespace rew
