// The routed-expert FFN of rew's DeepSeekMoE.forward over raw device rows
// (src/rew/models/deepseek.nim:122-145): the launch sequence the deferred
// graph's MoE lowering runs, and the C-ABI entry point that runs it
// directly on caller-owned buffers.
//
// Working memory (one block, carved at 256-byte boundaries):
//   member_of [E] int32    expert id -> chain index, -1 off the chain
//   members   [n] int32    chain index -> expert id
//   tables    [6 n] ptr    per-expert weight / bias device pointers
//   route     [2 (n + 1) + 3 R + nb n] int32   offsets, tile starts,
//                                       packed row -> token, each token's
//                                       packed rows and weights (f32) in
//                                       chain order, per-block counts (nb =
//                                       ceil(T / 256) token blocks)
//   hbuf      [R, I] bf16  SwiGLU outputs of the routed rows
//   ybuf      [R, H] bf16  down-projection outputs of the routed rows
// with R = T k routed rows (with shared experts both hold their T rows
// each after the routed rows: R + n_shared T).  Every byte a kernel reads is written earlier
// in the same sequence, so nothing has to start at zero.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <mutex>

#include "kernels.h"
#include "runtime.h"

namespace rew {

// Experts whose table entries one metadata launch writes (from its
// kernel arguments, so no host staging buffer is involved).  The first
// launch also sets member_of to -1 before the chunks enter their members;
// an entry with id -1 (a shared expert) only fills its table slots.
constexpr int kMetaChunk = 72;

struct MoeMetaChunk {
  int first, count, n;
  int32_t ids[kMetaChunk];
  const void* p[6][kMetaChunk];
};

__global__ void __launch_bounds__(256) moe_meta_kernel(MoeMetaChunk ch, int E, int32_t* members,
                                                       int32_t* member_of, const void** tables) {
  const int i = threadIdx.x;
  if (ch.first == 0) {
    for (int e = i; e < E; e += 256) member_of[e] = -1;
    __syncthreads();
  }
  if (i >= ch.count) return;
  if (ch.ids[i] >= 0) {
    members[ch.first + i] = ch.ids[i];
    member_of[ch.ids[i]] = ch.first + i;  // the ids are distinct
  }
#pragma unroll
  for (int j = 0; j < 6; ++j) tables[(size_t)j * ch.n + ch.first + i] = ch.p[j][i];
}

namespace {

struct Layout {
  size_t member_of, members, tables, route, hbuf, ybuf, total;
};

// (with shared experts: their table entries follow the members', their
// hidden and output rows the routed rows in hbuf and ybuf)
Layout layout_of(const RoutedFfn& a) {
  auto up = [](size_t b) { return (b + 255) & ~(size_t)255; };
  const size_t R = (size_t)a.T * (size_t)a.k, ns = (size_t)a.n_shared;
  const size_t groups = (size_t)a.n + ns;
  Layout L;
  size_t o = 0;
  L.member_of = o;
  o += up((size_t)a.E * 4);
  L.members = o;
  o += up((size_t)a.n * 4);
  L.tables = o;
  o += up(groups * 6 * sizeof(void*));
  L.route = o;
  const size_t nb = ((size_t)a.T + kMoeRouteBlock - 1) / kMoeRouteBlock;
  o += up((2 * (groups + 1) + 3 * R + ns * (size_t)a.T + nb * (size_t)a.n) * 4);
  L.hbuf = o;
  o += up((R + ns * (size_t)a.T) * (size_t)a.I * 2);
  L.ybuf = o;
  o += up((R + ns * (size_t)a.T) * (size_t)a.H * 2);
  L.total = o;
  return L;
}

// The two grouped GEMMs: SwiGLU over x's routed rows, down projection over
// the packed hidden rows, each with the shared experts' groups of all T
// tokens after the members' (operand tables and outputs filled in by the
// caller).
void gemm_args(const RoutedFfn& a, GemmArgs* gs, GemmArgs* gd) {
  *gs = GemmArgs{};
  *gd = GemmArgs{};
  for (GemmArgs* g : {gs, gd}) {
    g->dtype = REW_DT_BFLOAT16;
    g->c_dtype = REW_DT_BFLOAT16;
    g->batch = 1;
    g->a_sk = 1;
    g->b_sn = 1;
  }
  gs->a = a.x;
  gs->M = a.T;
  gs->K = a.H;
  gs->N = a.I;
  gs->a_sm = a.x_rs;
  gs->b_sk = a.I;
  gs->c_sm = a.I;
  gs->epi = EPI_SWIGLU;
  gd->M = a.T * ((int64_t)a.k + a.n_shared);
  gd->K = a.I;
  gd->N = a.H;
  gd->a_sm = a.I;
  gd->b_sk = a.H;
  gd->c_sm = a.H;
  gd->epi = EPI_BIAS;
}

bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

size_t routed_ffn_scratch_bytes(const RoutedFfn& a) { return layout_of(a).total; }

void routed_ffn_check(const RoutedFfn& a) {
  auto bad = [](const std::string& m) { invalid("routed MoE FFN: " + m); };
  if (a.T < 0 || a.H <= 0 || a.I <= 0) bad("tokens must be >= 0, hidden and ffn > 0");
  if (a.H % 8 || a.I % 8) bad("hidden and ffn must be multiples of 8");
  if (a.k < 1 || a.k > kMoeMaxK) bad("k must be in 1.." + std::to_string(kMoeMaxK));
  if (a.E < 1) bad("router_width must be positive");
  if (a.n < 1 || a.n > a.E) bad("n_experts must be in 1..router_width");
  if (a.n > kMoeMaxMembers) bad("at most " + std::to_string(kMoeMaxMembers) + " experts per call");
  if (a.T * (int64_t)a.k >= ((int64_t)1 << 31)) bad("tokens * k must be below 2^31");
  if (!a.expert) bad("null expert_ids");
  for (int i = 0; i < a.n; ++i) {
    if (a.expert[i] < 0 || a.expert[i] >= a.E)
      bad("expert id " + std::to_string(a.expert[i]) + " outside [0, router_width)");
    for (int j = 0; j < i; ++j)
      if (a.expert[j] == a.expert[i])
        bad("expert id " + std::to_string(a.expert[i]) + " repeated");
  }
  static const char* kTable[6] = {"gate_w", "up_w", "gate_b", "up_b", "down_w", "down_b"};
  for (int j = 0; j < 6; ++j) {
    if (!a.ptr[j]) bad(std::string("null ") + kTable[j] + " table");
    for (int i = 0; i < a.n; ++i)
      if (!a.ptr[j][i] || !al16(a.ptr[j][i]))
        bad(std::string(kTable[j]) + "[" + std::to_string(i) +
            "] is null or not 16-byte aligned");
  }
  if (a.n_shared < 0 || a.n + a.n_shared > kMoeMaxMembers)
    bad("at most " + std::to_string(kMoeMaxMembers) + " experts per call");
  for (int j = 0; j < 6 && a.n_shared > 0; ++j) {
    if (!a.sptr[j]) bad(std::string("null shared ") + kTable[j] + " table");
    for (int i = 0; i < a.n_shared; ++i)
      if (!a.sptr[j][i] || !al16(a.sptr[j][i]))
        bad(std::string("shared ") + kTable[j] + "[" + std::to_string(i) +
            "] is null or not 16-byte aligned");
  }
  if (a.T * ((int64_t)a.k + a.n_shared) >= ((int64_t)1 << 31))
    bad("tokens * (k + shared experts) must be below 2^31");
  if (a.T == 0) return;
  const bool own_start = a.n_shared > 0;
  if (!a.x || (!own_start && !a.start) || !a.topi || !a.topw || !a.out)
    bad("null device pointer");
  if (!al16(a.x) || (!own_start && !al16(a.start)) || !al16(a.out))
    bad("rows must be 16-byte aligned");
  if (a.x_rs < a.H || a.x_rs % 8 || (!own_start && (a.start_rs < a.H || a.start_rs % 8)))
    bad("row strides must be >= hidden and multiples of 8 elements");
  GemmArgs gs, gd;
  gemm_args(a, &gs, &gd);
  void* const rows = reinterpret_cast<void*>(uintptr_t(4096));  // scratch rows are aligned
  gs.c = rows;
  gd.a = rows;
  gd.c = rows;
  if (!gemm_grouped_ok(gs) || !gemm_grouped_ok(gd))
    bad("the expert GEMMs exceed the grouped kernel's 32-bit operand extents");
}

void run_routed_ffn(Ctx* c, const RoutedFfn& a, void* scratch) {
  const Layout L = layout_of(a);
  uint8_t* s = static_cast<uint8_t*>(scratch);
  int32_t* member_of = reinterpret_cast<int32_t*>(s + L.member_of);
  int32_t* members = reinterpret_cast<int32_t*>(s + L.members);
  const void** tables = reinterpret_cast<const void**>(s + L.tables);
  int32_t* route = reinterpret_cast<int32_t*>(s + L.route);
  const int n = a.n, ns = a.n_shared, groups = n + ns;
  const int64_t R = a.T * a.k;

  // (profile names are built only while profiling: the allocation-free
  // entry point runs this sequence without touching the host heap)
  if (c->profiling) prof_begin(c, "moe_tables{E" + std::to_string(n) + "}");
  for (int first = 0; first < groups; first += kMetaChunk) {
    MoeMetaChunk ch;
    std::memset(&ch, 0, sizeof ch);
    ch.first = first;
    ch.count = std::min(kMetaChunk, groups - first);
    ch.n = groups;
    for (int i = 0; i < ch.count; ++i) {
      const int e = first + i;  // members, then the shared experts (id -1)
      ch.ids[i] = e < n ? a.expert[e] : -1;
      for (int j = 0; j < 6; ++j) ch.p[j][i] = e < n ? a.ptr[j][e] : a.sptr[j][e - n];
    }
    hipLaunchKernelGGL(moe_meta_kernel, dim3(1), dim3(256), 0, c->stream, ch, (int)a.E, members,
                       member_of, tables);
    REW_HIP(hipGetLastError());
  }
  prof_end(c);

  MoeRouteArgs ra;
  ra.topi = a.topi;
  ra.topw = a.topw;
  ra.T = a.T;
  ra.k = a.k;
  ra.E = a.E;
  ra.member_of = member_of;
  ra.members = members;
  ra.n_members = n;
  ra.n_shared = ns;
  const int64_t RS = R + (int64_t)ns * a.T;  // hidden rows: routed, then shared
  ra.off = route;
  ra.mt_start = route + (groups + 1);
  ra.perm = route + 2 * (groups + 1);
  ra.ord_slot = route + 2 * (groups + 1) + RS;
  ra.ord_w = reinterpret_cast<float*>(route + 2 * (groups + 1) + RS + R);
  ra.blk_cnt = route + 2 * (groups + 1) + RS + 2 * R;
  if (c->profiling)
    prof_begin(c, "moe_route{" + std::to_string(a.T) + "x" + std::to_string(a.k) + ",E" +
                      std::to_string(n) + "}");
  const int route_launches = launch_moe_route(ra, c->stream);
  prof_end(c);

  GemmArgs gs, gd;
  gemm_args(a, &gs, &gd);
  gs.c = s + L.hbuf;
  gd.a = s + L.hbuf;
  gd.c = s + L.ybuf;
  // the SwiGLU launch covers the members and the shared experts (groups of
  // all T tokens); the down launch the members only
  GroupArgs ga;
  ga.off = ra.off;
  ga.mt_start = ra.mt_start;
  ga.n_groups = groups;
  // (a group of r rows takes at most r / 256 + 2 tiles, group_tiles)
  ga.max_mtiles = (R + 255) / 256 + 2 * n + (int64_t)ns * group_tiles(a.T);
  ga.rows = ra.perm;
  ga.b = tables;
  ga.b2 = tables + groups;
  ga.bias = tables + 2 * groups;
  ga.bias2 = tables + 3 * groups;
  ga.dual_span = 0;
  for (int i = 0; i < groups; ++i) {
    const void* g0 = i < n ? a.ptr[0][i] : a.sptr[0][i - n];
    const void* g1 = i < n ? a.ptr[1][i] : a.sptr[1][i - n];
    const int64_t d = (int64_t)((uintptr_t)g1 - (uintptr_t)g0);
    ga.dual_span = std::max(ga.dual_span, d < 0 ? -d : d);
  }
  if (c->profiling) {
    char nm[160];
    std::snprintf(nm, sizeof nm, "moe_gemm_swiglu[%d,%lld,%lld,%lld]", groups, (long long)RS,
                  (long long)a.I, (long long)a.H);
    prof_begin(c, nm);
  }
  launch_gemm_grouped(gs, ga, c->stream);
  prof_end(c);
  // the down launch: the members' and the shared experts' groups again,
  // over the packed hidden rows, each output row a bias epilogue
  ga.rows = nullptr;
  ga.b = tables + 4 * groups;
  ga.b2 = nullptr;
  ga.bias = tables + 5 * groups;
  ga.bias2 = nullptr;
  if (c->profiling) {
    char nm[160];
    std::snprintf(nm, sizeof nm, "moe_gemm_down[%d,%lld,%lld,%lld]", groups, (long long)RS,
                  (long long)a.H, (long long)a.I);
    prof_begin(c, nm);
  }
  launch_gemm_grouped(gd, ga, c->stream);
  prof_end(c);

  // the combine starts from the shared experts' outputs (rew's running
  // sum, each add rounded) or, without them, from the caller's start rows
  MoeCombineArgs ca;
  if (ns) {
    ca.prev = (const uint16_t*)(s + L.ybuf) + (size_t)R * a.H;
    ca.prev_rs = a.H;
  } else {
    ca.prev = (const uint16_t*)a.start;
    ca.prev_rs = a.start_rs;
  }
  ca.n_prev = ns ? ns : 1;
  ca.prev_sb = a.T * a.H;
  ca.y = (const uint16_t*)gd.c;
  ca.ord_slot = ra.ord_slot;
  ca.ord_w = ra.ord_w;
  ca.T = a.T;
  ca.H = a.H;
  ca.k = a.k;
  ca.out = (uint16_t*)a.out;
  if (c->profiling)
    prof_begin(c, "moe_combine{" + std::to_string(a.T) + "x" + std::to_string(a.H) + "}");
  launch_moe_combine(ca, c->stream);
  prof_end(c);
  c->stats.kernels_launched += route_launches + 3 + (groups + kMetaChunk - 1) / kMetaChunk;
  c->stats.fused_groups += 4;
}

// Working memory of rew_mi355x_moe_routed_ffn_noalloc: one array per GPU,
// part of this library's code object, held until the process ends.  Host
// code never passes `scratch` itself (on the host it names a stand-in, not
// device memory): noalloc_scratch_lookup() resolves its device address once
// per device at rew_mi355x_init and the context keeps it.
constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

void* noalloc_scratch_lookup(std::string* err) {
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p) {
    (void)hipGetLastError();
    *err = std::string("allocation-free MoE entry point unavailable: hipGetSymbolAddress "
                       "failed (") + hipGetErrorString(e) + ")";
    return nullptr;
  }
  return p;
}

}  // namespace rew

using namespace rew;

namespace {

RoutedFfn from_abi(const rew_mi355x_moe_args* p) {
  if (!p) invalid("routed MoE FFN: null args");
  RoutedFfn a;
  a.x = p->x;
  a.x_rs = p->x_row_stride;
  a.start = p->start;
  a.start_rs = p->start_row_stride;
  a.topi = p->top_ids;
  a.topw = p->top_weights;
  a.T = p->tokens;
  a.H = p->hidden;
  a.I = p->ffn;
  a.k = p->k;
  a.E = p->router_width;
  a.n = p->n_experts;
  a.expert = p->expert_ids;
  a.ptr[0] = p->gate_w;
  a.ptr[1] = p->up_w;
  a.ptr[2] = p->gate_b;
  a.ptr[3] = p->up_b;
  a.ptr[4] = p->down_w;
  a.ptr[5] = p->down_b;
  a.out = p->out;
  return a;
}

Ctx* ctx_of(rew_mi355x_ctx* ctx) {
  if (!ctx) invalid("null context");
  return reinterpret_cast<Ctx*>(ctx);
}

}  // namespace

extern "C" int rew_mi355x_moe_routed_ffn(rew_mi355x_ctx* ctx, const rew_mi355x_moe_args* args) {
  return guarded([&] {
    Ctx* c = ctx_of(ctx);
    const RoutedFfn a = from_abi(args);
    routed_ffn_check(a);
    std::lock_guard<std::recursive_mutex> g(c->mu);
    REW_HIP(hipSetDevice(c->ordinal));
    Shape s;
    s.rank = 1;
    s.d[0] = (int64_t)routed_ffn_scratch_bytes(a);
    Tensor* w = new_tensor(c, kU8, s);
    w->plan_dead = true;
    try {
      tensor_alloc(w);
      run_routed_ffn(c, a, w->data());
    } catch (...) {
      maybe_destroy(w);
      throw;
    }
    // stream-ordered: the block is reused only by work enqueued after this
    maybe_destroy(w);
  });
}

extern "C" int rew_mi355x_moe_routed_ffn_noalloc(rew_mi355x_ctx* ctx,
                                                 const rew_mi355x_moe_args* args) {
  return guarded([&] {
    Ctx* c = ctx_of(ctx);
    const RoutedFfn a = from_abi(args);
    routed_ffn_check(a);
    const size_t need = routed_ffn_scratch_bytes(a);
    if (need > kNoAllocScratchBytes)
      invalid("routed MoE FFN (allocation-free): needs " + std::to_string(need) +
              " bytes of working memory, the static scratch holds " +
              std::to_string(kNoAllocScratchBytes) +
              "; call rew_mi355x_moe_routed_ffn for this size");
    std::lock_guard<std::recursive_mutex> g(c->mu);
    REW_HIP(hipSetDevice(c->ordinal));
    if (!c->noalloc_scratch) fail(REW_MI355X_ERR_DEVICE, c->noalloc_error);
    run_routed_ffn(c, a, c->noalloc_scratch);
  });
}
