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
//   moe_count / moe_place  per-member row counts -> row offsets and
//                     256-row tile starts (the grouped GEMMs' work lists),
//                     each member's tokens in ascending token order, and
//                     each token's packed rows and gate weights in chain
//                     order: counts and ballot ranks only, so the layout
//                     never depends on timing;
//   (grouped SwiGLU and down-projection GEMMs over the packed rows, k_gemm.hip)
//   moe_combine_kernel per token: start from the running sum before the
//                     first routed expert (the caller's rows, or the shared
//                     experts' outputs added in order with bf16 rounding
//                     after each add), then for the token's routed
//                     members in chain order add bf16(f32(y) * w) with bf16
//                     rounding after every add -- the dense op sequence's
//                     arithmetic on the only rows where it is non-zero.
#include <hip/hip_runtime.h>

#include "kernels.h"
#include "vm_device.h"

namespace rew {

// Token placement over blocks of kMoeRouteBlock tokens (256, one per thread):
//   moe_count_kernel  each block's per-member counts (LDS atomics: a count
//                     does not depend on the order of its increments);
//   moe_place_kernel  each block sums the count table per member over the
//                     blocks before its own (the block's base) and over all
//                     blocks (the totals, whose prefixes over the members
//                     are the row offsets and tile starts; block 0 stores
//                     them).  Then every wave ORs 1 << lane into an LDS
//                     mask per (wave, member) for each of its tokens'
//                     members, and a token's rank among the member's tokens
//                     of the block is the popcount of the lower lanes' bits
//                     plus the earlier waves' counts: ascending token order,
//                     O(k) work per token, and OR does not depend on the
//                     order of the atomics.  It writes the packed rows and
//                     each token's rows and weights in chain order
//                     (ord_slot / ord_w, for the combine).
// Past kMoeFusedTable count-table entries the sums over blocks run once in
// moe_scan_kernel instead, and the placement reads its results.
// A (token, expert) pair counts once even if the id repeats in the row, with
// the weights of all its slots summed in slot order, as routedWeightForExpert
// sums topWeights * (topIndices == e) (topK's ids are distinct, so the sum
// is one weight there).

constexpr int kMoeFusedTable = 65536;  // count-table entries a placement block sums
constexpr int kMoeFusedMembers = 1024;

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

// The large-table form: per member, the block counts replaced by their
// exclusive prefix in block order, then the offsets and tile starts.
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
      mt += group_tiles(tot[m]);
    }
    a.off[a.n_members] = off;
    a.mt_start[a.n_members] = mt;
    for (int sh = 1; sh <= a.n_shared; ++sh) {
      a.off[a.n_members + sh] = off + sh * (int)a.T;
      a.mt_start[a.n_members + sh] = mt + sh * group_tiles(a.T);
    }
  }
}

// KM: the most slots per token the unrolled loops cover (k <= KM)
template <bool FUSED, int KM>
__global__ void __launch_bounds__(256) moe_place_kernel(MoeRouteArgs a, int nblk) {
  // lane masks [4][n] (64-bit; in the fused form first the partial sums
  // [2][4][n]), base [n]; fused: totals [n], tile counts [n]
  extern __shared__ __attribute__((aligned(8))) int sh[];
  const int n = a.n_members;
  unsigned long long* bits = reinterpret_cast<unsigned long long*>(sh);
  int* base = sh + 8 * n;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int blk = (int)blockIdx.x;
  if constexpr (FUSED) {
    int* tot = base + n;
    int* til = base + 2 * n;
    int* part = sh;  // [g][n] before this block, then [4 + g][n] all
    // thread (g, m) sums blocks g, g + 4, ...: sixteen loads at a time, all
    // issued before their sums (addresses clamped, no branch around a load)
    for (int i = threadIdx.x; i < 4 * n; i += 256) {
      const int g = i / n, m = i - g * n;
      int pre = 0, all = 0;
      for (int b0 = g; b0 < nblk; b0 += 64) {
        int c[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const int b = b0 + 4 * u;
          c[u] = a.blk_cnt[(int64_t)(b < nblk ? b : g) * n + m];
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const int b = b0 + 4 * u;
          const int v = b < nblk ? c[u] : 0;
          pre += b < blk ? v : 0;
          all += v;
        }
      }
      part[g * n + m] = pre;
      part[(4 + g) * n + m] = all;
    }
    __syncthreads();
    for (int m = threadIdx.x; m < n; m += 256) {
      const int all = part[4 * n + m] + part[5 * n + m] + part[6 * n + m] + part[7 * n + m];
      base[m] = part[m] + part[n + m] + part[2 * n + m] + part[3 * n + m];
      tot[m] = all;
      til[m] = group_tiles(all);
    }
    __syncthreads();
    if (wave == 0) {
      // exclusive prefixes over the members: lane l takes members
      // [l s, l s + s), then an inclusive scan of the lane sums
      const int s = (n + 63) / 64;
      const int lo = lane * s < n ? lane * s : n, hi = lo + s < n ? lo + s : n;
      int s1 = 0, s2 = 0;
      for (int m = lo; m < hi; ++m) {
        s1 += tot[m];
        s2 += til[m];
      }
      int i1 = s1, i2 = s2;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int u1 = __shfl_up(i1, off, 64), u2 = __shfl_up(i2, off, 64);
        if (lane >= off) {
          i1 += u1;
          i2 += u2;
        }
      }
      int r1 = i1 - s1, r2 = i2 - s2;
      for (int m = lo; m < hi; ++m) {
        const int v1 = tot[m], v2 = til[m];
        tot[m] = r1;
        til[m] = r2;
        r1 += v1;
        r2 += v2;
      }
      if (blk == 0 && lane == 63) {
        a.off[n] = i1;
        a.mt_start[n] = i2;
        for (int sh = 1; sh <= a.n_shared; ++sh) {  // groups of all T tokens
          a.off[n + sh] = i1 + sh * (int)a.T;
          a.mt_start[n + sh] = i2 + sh * group_tiles(a.T);
        }
      }
    }
    __syncthreads();
    for (int m = threadIdx.x; m < n; m += 256) {
      base[m] += tot[m];
      if (blk == 0) {
        a.off[m] = tot[m];
        a.mt_start[m] = til[m];
      }
    }
  } else {
    const int32_t* pre = a.blk_cnt + (int64_t)blk * n;
    for (int m = threadIdx.x; m < n; m += 256) base[m] = a.off[m] + pre[m];
  }
  for (int i = threadIdx.x; i < 4 * n; i += 256) bits[i] = 0ull;

  // one token per thread
  const int64_t t = (int64_t)blk * kMoeRouteBlock + threadIdx.x;
  const bool live = t < a.T;
  const int64_t row = t * a.k;
  int id[KM], mem[KM];  // fully unrolled: registers
  float wv[KM];
  {
    // every load unconditional (clamped to a real slot), kept or dropped after
    const int64_t crow = (live ? t : a.T - 1) * a.k;
    int ri[KM];
    float rw[KM];
#pragma unroll
    for (int q = 0; q < KM; ++q) {
      const int qc = q < a.k ? q : a.k - 1;
      ri[q] = a.topi[crow + qc];
      rw[q] = a.topw[crow + qc];
    }
#pragma unroll
    for (int q = 0; q < KM; ++q) {
      const bool in = live && q < a.k;
      id[q] = in ? ri[q] : -1;
      wv[q] = in ? rw[q] : 0.0f;
    }
  }
#pragma unroll
  for (int q = 0; q < KM; ++q) {
    const int e = id[q];
    bool first = q < a.k && e >= 0 && e < a.E;
#pragma unroll
    for (int q2 = 0; q2 < q; ++q2)
      if (id[q2] == e) first = false;
    mem[q] = a.member_of[first ? e : 0];
    if (!first) mem[q] = -1;
  }
  __syncthreads();  // the masks are clear
  const unsigned long long me = 1ull << lane;
#pragma unroll
  for (int q = 0; q < KM; ++q)
    if (mem[q] >= 0) atomicOr(&bits[wave * n + mem[q]], me);
  // a member's weight: the slots holding its id, summed in slot order from
  // zero; its place in the token's chain-order list: the members before it
  int nmem = 0;
#pragma unroll
  for (int q = 0; q < KM; ++q) nmem += mem[q] >= 0 ? 1 : 0;
  __syncthreads();  // the masks are complete
  const unsigned long long lt = me - 1ull;
#pragma unroll
  for (int q = 0; q < KM; ++q) {
    const int m = mem[q];
    if (m < 0) continue;
    float w = 0.0f;
    int p = 0;
#pragma unroll
    for (int q2 = 0; q2 < KM; ++q2) {
      if (q2 < a.k) w = w + (id[q2] == id[q] ? wv[q2] : 0.0f);
      p += (mem[q2] >= 0 && mem[q2] < m) ? 1 : 0;
    }
    int slot = base[m] + __popcll(bits[wave * n + m] & lt);
    for (int w2 = 0; w2 < wave; ++w2) slot += __popcll(bits[w2 * n + m]);
    a.perm[slot] = (int32_t)t;
    a.ord_slot[row + p] = slot;
    a.ord_w[row + p] = w;
  }
  if (live) {
    for (int i = nmem; i < a.k; ++i) {
      a.ord_slot[row + i] = -1;
      a.ord_w[row + i] = 0.0f;
    }
    for (int sh = 0; sh < a.n_shared; ++sh) a.perm[a.T * a.k + sh * a.T + t] = (int32_t)t;
  }
}

// One wave per token (four per workgroup).  Lanes q < k read the token's
// packed rows and weights in chain order (the placement's lists; -1 ends
// them); row i's entry is read from lane i (readlane, wave-uniform).  Each lane owns 16-byte
// chunks h, h + 512 B, ... of the row and takes them two at a time: both
// chunks' loads of the running sum and of every member's row are issued
// before the ordered, rounded accumulation runs over them.  With KC > 0,
// tokens with exactly KC members take straight-line loads (no branch between
// a load and its use); the rest take the general loop.
template <int KC>
__global__ void __launch_bounds__(256) moe_combine_kernel(MoeCombineArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t waves = (int64_t)gridDim.x * 4;
  const int nch = (int)(a.H / 8);  // 16-byte chunks per row
  for (int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); t < a.T; t += waves) {
    int slot = -1;
    float w = 0.0f;
    if (lane < a.k) {
      slot = a.ord_slot[t * a.k + lane];
      w = a.ord_w[t * a.k + lane];
    }
    const int n = __popcll(__ballot(slot >= 0));
    const uint16_t* prow = a.prev + t * a.prev_rs;
    uint16_t* orow = a.out + t * a.H;
    for (int c0 = lane; c0 < nch; c0 += 128) {
      const bool two = c0 + 64 < nch;
      const int64_t h0 = (int64_t)c0 * 8, h1 = two ? h0 + 512 : h0;
      const uint4 p0 = *(const uint4*)(prow + h0);
      const uint4 p1 = *(const uint4*)(prow + h1);
      float acc0[8], acc1[8];
      {
        const uint16_t* x0 = (const uint16_t*)&p0;
        const uint16_t* x1 = (const uint16_t*)&p1;
#pragma unroll
        for (int x = 0; x < 8; ++x) {
          acc0[x] = vm::as_f((uint32_t)x0[x] << 16);
          acc1[x] = vm::as_f((uint32_t)x1[x] << 16);
        }
      }
      // the later shared experts' rows: out = bf16(out + row), as the
      // residual epilogue of rew's chain add
#pragma unroll 1
      for (int s = 1; s < a.n_prev; ++s) {
        const uint4 q0 = *(const uint4*)(prow + s * a.prev_sb + h0);
        const uint4 q1 = *(const uint4*)(prow + s * a.prev_sb + h1);
        const uint16_t* x0 = (const uint16_t*)&q0;
        const uint16_t* x1 = (const uint16_t*)&q1;
#pragma unroll
        for (int x = 0; x < 8; ++x) {
          acc0[x] = vm::round_bf16(acc0[x] + vm::as_f((uint32_t)x0[x] << 16));
          acc1[x] = vm::round_bf16(acc1[x] + vm::as_f((uint32_t)x1[x] << 16));
        }
      }
      auto add = [&](const uint4& y0, const uint4& y1, float wgt) {
        const uint16_t* a0 = (const uint16_t*)&y0;
        const uint16_t* a1 = (const uint16_t*)&y1;
#pragma unroll
        for (int x = 0; x < 8; ++x) {
          acc0[x] = vm::round_bf16(acc0[x] + vm::round_bf16(vm::as_f((uint32_t)a0[x] << 16) * wgt));
          acc1[x] = vm::round_bf16(acc1[x] + vm::round_bf16(vm::as_f((uint32_t)a1[x] << 16) * wgt));
        }
      };
      if (KC > 0 && n == KC) {
        uint4 y0[KC > 0 ? KC : 1], y1[KC > 0 ? KC : 1];
#pragma unroll
        for (int i = 0; i < KC; ++i) {
          const uint16_t* yr = a.y + (int64_t)__builtin_amdgcn_readlane(slot, i) * a.H;
          y0[i] = *(const uint4*)(yr + h0);
          y1[i] = *(const uint4*)(yr + h1);
        }
#pragma unroll
        for (int i = 0; i < KC; ++i)
          add(y0[i], y1[i], __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), i)));
      } else {
        // one row at a time (lane i's entry read by a uniform readlane)
#pragma unroll 1
        for (int i = 0; i < n; ++i) {
          const uint16_t* yr = a.y + (int64_t)__builtin_amdgcn_readlane(slot, i) * a.H;
          const uint4 y0 = *(const uint4*)(yr + h0);
          const uint4 y1 = *(const uint4*)(yr + h1);
          add(y0, y1, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), i)));
        }
      }
      uint16_t o0[8], o1[8];
#pragma unroll
      for (int x = 0; x < 8; ++x) {
        o0[x] = (uint16_t)(vm::as_u(acc0[x]) >> 16);
        o1[x] = (uint16_t)(vm::as_u(acc1[x]) >> 16);
      }
      *(uint4*)(orow + h0) = *(const uint4*)o0;
      if (two) *(uint4*)(orow + h1) = *(const uint4*)o1;
    }
  }
}

int launch_moe_route(const MoeRouteArgs& a, hipStream_t stream) {
  if (a.n_members <= 0) return 0;
  if (a.k < 1 || a.k > kMoeMaxK || a.n_members > kMoeMaxMembers)
    fail(REW_MI355X_ERR_INVALID, "internal: MoE routing launch outside its limits");
  const int nblk = (int)((a.T + kMoeRouteBlock - 1) / kMoeRouteBlock);
  const size_t n4 = (size_t)a.n_members * sizeof(int);
  const bool fused = a.n_members <= kMoeFusedMembers &&
                     (int64_t)nblk * a.n_members <= kMoeFusedTable;
  int launches = 0;
  if (nblk > 0) {
    ++launches;
    hipLaunchKernelGGL(moe_count_kernel, dim3((unsigned)nblk), dim3(256), n4, stream, a);
    REW_HIP(hipGetLastError());
  }
  if (!fused || nblk == 0) {
    ++launches;
    hipLaunchKernelGGL(moe_scan_kernel, dim3(1), dim3(1024), n4, stream, a, nblk);
    REW_HIP(hipGetLastError());
  }
  if (nblk == 0) return launches;
  // LDS: the lane masks (8 n ints, the partial sums before them), base, and
  // in the fused form totals and tile counts
  const size_t lds = (fused ? 11 : 9) * n4;
  if (fused) {
    if (a.k <= 8)
      hipLaunchKernelGGL((moe_place_kernel<true, 8>), dim3((unsigned)nblk), dim3(256), lds,
                         stream, a, nblk);
    else
      hipLaunchKernelGGL((moe_place_kernel<true, kMoeMaxK>), dim3((unsigned)nblk), dim3(256),
                         lds, stream, a, nblk);
  } else {
    if (a.k <= 8)
      hipLaunchKernelGGL((moe_place_kernel<false, 8>), dim3((unsigned)nblk), dim3(256), lds,
                         stream, a, nblk);
    else
      hipLaunchKernelGGL((moe_place_kernel<false, kMoeMaxK>), dim3((unsigned)nblk), dim3(256),
                         lds, stream, a, nblk);
  }
  REW_HIP(hipGetLastError());
  return launches + 1;
}

void launch_moe_combine(const MoeCombineArgs& a, hipStream_t stream) {
  if (a.T == 0) return;
  if (a.H % 8 || a.prev_rs % 8 || a.prev_sb % 8 || a.n_prev < 1 || ((uintptr_t)a.prev & 15) ||
      ((uintptr_t)a.y & 15) || ((uintptr_t)a.out & 15) || a.k < 1 || a.k > kMoeMaxK)
    fail(REW_MI355X_ERR_INVALID, "internal: MoE combine launch outside its limits");
  const int64_t blocks = (a.T + 3) / 4;
  const dim3 grid((unsigned)(blocks < 65536 ? blocks : 65536));
  switch (a.k) {
    case 1: hipLaunchKernelGGL(moe_combine_kernel<1>, grid, dim3(256), 0, stream, a); break;
    case 2: hipLaunchKernelGGL(moe_combine_kernel<2>, grid, dim3(256), 0, stream, a); break;
    case 4: hipLaunchKernelGGL(moe_combine_kernel<4>, grid, dim3(256), 0, stream, a); break;
    case 6: hipLaunchKernelGGL(moe_combine_kernel<6>, grid, dim3(256), 0, stream, a); break;
    case 8: hipLaunchKernelGGL(moe_combine_kernel<8>, grid, dim3(256), 0, stream, a); break;
    default: hipLaunchKernelGGL(moe_combine_kernel<0>, grid, dim3(256), 0, stream, a); break;
  }
  REW_HIP(hipGetLastError());
}

}  // namespace rew
