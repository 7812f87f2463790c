// Graph lowering: turns the pending op graph of a context into HIP launches.
//
// 1. Dead nodes (no owner and no consumer) are dropped.
// 2. Each pending tensor is classified: anchors (reductions, dot_general,
//    gathers, ...) always materialize; elementwise results materialize when
//    the caller still holds them, when a consumer needs them in memory, or
//    when several consumers would each recompute a non-trivial expression;
//    view ops (reshape/transpose/broadcast/slice/reverse) never do unless
//    the caller holds them.
// 3. Every materialization of an elementwise tensor becomes one vm::Program
//    whose leaves read materialized tensors through affine index maps built
//    by composing the view ops between them, so chains like rew's RoPE
//    (~26 reshape/slice/mul/concat ops) or a bias-add + SiLU + gate product
//    become a single HBM pass.  Reductions take their input expression as a
//    prologue.  dot_general folds transposes into GEMM strides.
// A graph whose signature was flushed before skips 2 and 3: the launches
// recorded then are replayed over this flush's buffers (plan.cpp).
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <functional>
#include <map>
#include <tuple>

#include "kernels.h"
#include "plan.h"
#include "runtime.h"

namespace rew {

using namespace vm;

static_assert(sizeof(Program) + sizeof(Space) + sizeof(ReduceArgs) < 4000,
              "kernel arguments must stay below 4 KiB");

// ---------------------------------------------------------------------------
// classification
// ---------------------------------------------------------------------------

static bool is_view(int k) {
  return k == K_RESHAPE || k == K_TRANSPOSE || k == K_REVERSE ||
         k == K_BROADCAST_TO || k == K_BROADCAST || k == K_SLICE;
}
static bool is_ew(int k) {
  return k == K_BINARY || k == K_UNARY || k == K_CONVERT || k == K_ISFINITE ||
         k == K_COMPARE || k == K_SELECT || k == K_CLAMP || k == K_IOTA ||
         k == K_CONCAT || k == K_REDUCE_PRECISION || k == K_CONST;
}
// Consumers that read an operand through a fused prologue.
static bool takes_expression(int k) { return is_ew(k) || is_view(k) || k == K_REDUCE; }

// Value of broadcastTo(scalar f32 constant, shape, []) (defined with the matchers).
static bool const_bcast(Tensor* t, float* val);

// ---------------------------------------------------------------------------
// affine index maps: kernel coordinates -> tensor coordinates
// ---------------------------------------------------------------------------

struct Affine {
  int R = 0;  // kernel rank
  int r = 0;  // tensor rank
  int64_t off[kMaxRank] = {0};
  int64_t S[kMaxRank][kMaxRank] = {{0}};

  static Affine identity(int rank) {
    Affine a;
    a.R = a.r = rank;
    for (int i = 0; i < rank; ++i) a.S[i][i] = 1;
    return a;
  }
  bool operator==(const Affine& o) const {
    if (R != o.R || r != o.r) return false;
    for (int i = 0; i < r; ++i) {
      if (off[i] != o.off[i]) return false;
      for (int k = 0; k < R; ++k)
        if (S[i][k] != o.S[i][k]) return false;
    }
    return true;
  }
};

static void dense_strides(const Shape& s, int64_t* st) {
  int64_t acc = 1;
  for (int i = s.rank - 1; i >= 0; --i) {
    st[i] = acc;
    acc *= s.d[i];
  }
}

// Map through u = reshape(x): fine when every group of u dims merges into a
// single x dim (x coordinate = mixed-radix combination of u coordinates).
static bool compose_reshape(const Shape& U, const Shape& X, const Affine& m,
                            Affine* out) {
  out->R = m.R;
  out->r = X.rank;
  for (int j = 0; j < X.rank; ++j) {
    out->off[j] = 0;
    for (int k = 0; k < m.R; ++k) out->S[j][k] = 0;
  }
  // Non-unit dims of each side.
  std::vector<int> ui, xj;
  for (int i = 0; i < U.rank; ++i)
    if (U.d[i] != 1) ui.push_back(i);
  for (int j = 0; j < X.rank; ++j)
    if (X.d[j] != 1) xj.push_back(j);
  size_t a = 0, b = 0;
  while (a < ui.size() || b < xj.size()) {
    if (a >= ui.size() || b >= xj.size()) return false;
    // grow a minimal group with equal products
    size_t a1 = a + 1, b1 = b + 1;
    int64_t pu = U.d[ui[a]], px = X.d[xj[b]];
    while (pu != px) {
      if (pu < px) {
        if (a1 >= ui.size()) return false;
        pu *= U.d[ui[a1++]];
      } else {
        if (b1 >= xj.size()) return false;
        px *= X.d[xj[b1++]];
      }
    }
    if (b1 - b != 1) return false;  // would need a division
    const int j = xj[b];
    int64_t w = 1;
    for (size_t t = a1; t-- > a;) {
      const int i = ui[t];
      out->off[j] += m.off[i] * w;
      for (int k = 0; k < m.R; ++k) out->S[j][k] += m.S[i][k] * w;
      w *= U.d[i];
    }
    a = a1;
    b = b1;
  }
  return true;
}

// Given m: kernel -> coordinates of u = v(x), produce kernel -> x.
static bool compose_view(const Node* v, const Affine& m, Affine* out) {
  const Shape& X = v->in[0]->shape;
  const Shape& U = v->out[0]->shape;
  switch (v->kind) {
    case K_RESHAPE:
      return compose_reshape(U, X, m, out);
    case K_TRANSPOSE: {
      *out = m;
      for (int i = 0; i < U.rank; ++i) {
        const int p = (int)v->l0[i];
        out->off[p] = m.off[i];
        for (int k = 0; k < m.R; ++k) out->S[p][k] = m.S[i][k];
      }
      return true;
    }
    case K_BROADCAST_TO: {
      Affine o;
      o.R = m.R;
      o.r = X.rank;
      for (int j = 0; j < X.rank; ++j) {
        if (X.d[j] == 1) continue;  // row of zeros
        const int i = (int)v->l1[j];
        o.off[j] = m.off[i];
        for (int k = 0; k < m.R; ++k) o.S[j][k] = m.S[i][k];
      }
      *out = o;
      return true;
    }
    case K_BROADCAST: {
      Affine o;
      o.R = m.R;
      o.r = X.rank;
      const int nb = (int)v->l0.size();
      for (int j = 0; j < X.rank; ++j) {
        o.off[j] = m.off[nb + j];
        for (int k = 0; k < m.R; ++k) o.S[j][k] = m.S[nb + j][k];
      }
      *out = o;
      return true;
    }
    case K_SLICE: {
      *out = m;
      for (int i = 0; i < X.rank; ++i) {
        out->off[i] = v->l0[i] + v->l2[i] * m.off[i];
        for (int k = 0; k < m.R; ++k) out->S[i][k] = v->l2[i] * m.S[i][k];
      }
      return true;
    }
    case K_REVERSE: {
      *out = m;
      for (auto d : v->l0) {
        out->off[d] = X.d[d] - 1 - m.off[d];
        for (int k = 0; k < m.R; ++k) out->S[d][k] = -m.S[d][k];
      }
      return true;
    }
    default:
      return false;
  }
}

// ---------------------------------------------------------------------------
// lowering state
// ---------------------------------------------------------------------------

// A recognised SDPA chain (src/rew/nn/attention.nim:36-81): the PV
// dot_general it ends in is lowered to one flash-attention launch.
struct FlashPlan {
  Tensor *q = nullptr, *k = nullptr, *v = nullptr;
  float scale = 1.0f;
  bool round_scores = true;
  bool mask = false;
  int cmp = 0;
  float mask_true = 0.0f, mask_false = 0.0f;
  // When the attention output's only consumer is transpose [0, 2, 1, 3]
  // (GroupedQueryAttention.forward, groupedqueryattention.nim:136-140),
  // the kernel writes that transposed tensor directly.
  Tensor* out_t = nullptr;
};

// A dot_general whose consumers fold into its epilogue (see GemmArgs::epi).
struct GemmPlan {
  Node* dot = nullptr;
  Node* dot2 = nullptr;  // EPI_SWIGLU: the up projection
  int epi = 0;
  Tensor* bias = nullptr;
  Tensor* bias2 = nullptr;
  Tensor* res = nullptr;
  // EPI_BIAS_ROPE: the rotated tensor is [B, H, S, D] (rope_t, the
  // projection reshaped to [B, S, H, D] and transposed) or [B, S, H, D]
  Tensor* rope_cos = nullptr;  // the applyRotate chain's fp32 table views
  Tensor* rope_sin = nullptr;
  bool rope_t = false;
  int64_t rope_B = 0, rope_S = 0, rope_H = 0, rope_D = 0;
  // EPI_BIAS_RELU: maximum(y, relu_c) or maximum(relu_c, y)
  float relu_c = 0.0f;
  bool relu_first = true;
  // projections of one input launched together (GroupedQueryAttention's
  // q / k / v): index into Lower::gemm_groups, or -1
  int group = -1;
};

// rmsNorm chain (src/rew/nn/norm.nim:204-224) or LayerNorm chain
// (norm.nim:41-84, layer) lowered to one row kernel.
struct NormPlan {
  Tensor* src = nullptr;  // bf16 source (astype folded) or the f32 input itself
  Tensor* gamma = nullptr;
  float eps = 0.0f, divisor = 1.0f;
  bool layer = false;
  Tensor* beta = nullptr;  // layer: the shift
  float divisor2 = 1.0f;   // layer: the variance's reduceMean divisor
};

// softmax chain (src/rew/nn/activation.nim:64-77) over the last axis, lowered
// to one row kernel.
struct SoftmaxPlan {
  Tensor* x = nullptr;  // f32 input
};

// applyRotate chain (src/rew/nn/rope.nim:56-108) lowered to one pair kernel.
struct RopePlan {
  Tensor* src = nullptr;   // x (bf16 when the astype to f32 is folded)
  Tensor* cos0 = nullptr;  // [..., S, half] views of the fp32 tables
  Tensor* sin0 = nullptr;
};

// A run of routed-expert contributions of rew's DeepSeekMoE.forward
// (src/rew/models/deepseek.nim:122-145) added into one running sum:
//   out_j = add(out_{j-1}, astype(mul(astype(Y_e, f32),
//                                     broadcastTo(reshape(w_e, [T, 1]))), bf16))
// Y_e = downProj(SwiGLU(x)) of routed expert e, w_e = routedWeightForExpert
// (deepseek.nim:114-120) over the same (topWeights, topIndices).  Lowered to
// routing + two grouped GEMMs over the routed rows + an ordered combine.
struct MoeMember {
  int e = 0;
  GemmPlan sw;  // SwiGLU dual GEMM of x (gate, up)
  GemmPlan dn;  // down projection + bias
};
struct MoePlan {
  Tensor* start = nullptr;  // running sum before the first member
  Tensor* x = nullptr;      // token matrix [T, H] bf16
  Tensor* topi = nullptr;   // [T, k] int32 (topK indices)
  Tensor* topw = nullptr;   // [T, k] f32
  int E = 0;                // router width
  std::vector<MoeMember> mem;
  // matching state, applied only once the whole group is known lowerable:
  // the members' intermediates (never materialized) and the running sums
  // between members
  std::vector<Tensor*> inner, mids;
  // the shared experts whose sum is `start` (e = -1), when the group also
  // owns them: their SwiGLU GEMMs join the members' grouped launch and
  // `start` with their intermediates is never materialized
  std::vector<MoeMember> shared;
  std::vector<Tensor*> shared_inner;
};

// A classifier head, argmax(softmax(Linear(x))) over f32 rows (the end of
// rew's MLP forward, nn/linear.nim:43-49 and nn/activation.nim:64-77), whose
// logits and probabilities nobody else reads: one launch at the argmax.
struct HeadPlan {
  Tensor *x = nullptr, *w = nullptr, *b = nullptr;
};

// DeepSeekMoE.route (src/rew/models/deepseek.nim:132-137): topK of the
// softmax of an f32 Linear of x (or of astype(x, f32) from bf16), and the
// renormalised weights when the chain goes on to them; logits,
// probabilities and (with the renormalisation) the raw values have no
// other reader.  One launch makes the ids and the weights (or values).
struct RouterPlan {
  Tensor *x = nullptr, *w = nullptr, *b = nullptr;
  Tensor *ids = nullptr, *vals = nullptr, *wts = nullptr;
  int k = 0;
};

struct Lower {
  Ctx* c;
  std::vector<Node*> nodes;  // live pending nodes in creation order
  std::unordered_map<Node*, FlashPlan> flash;  // keyed by the PV dot_general
  std::unordered_map<Tensor*, std::vector<Node*>> cons;  // pending consumers
  std::unordered_map<Tensor*, GemmPlan> gemm_out;  // fused GEMM result -> plan
  std::unordered_map<Tensor*, NormPlan> norm_out;
  // an embedding lookup (torchIndexSelect output, pending) read only
  // through reshapes by a planned rmsNorm -> that norm's output: both are
  // written by one launch at the lookup
  std::unordered_map<Tensor*, Tensor*> gather_norm;
  std::unordered_map<Tensor*, RopePlan> rope_out;
  std::unordered_map<Tensor*, SoftmaxPlan> softmax_out;
  std::unordered_map<Tensor*, MoePlan> moe_out;
  std::unordered_map<Tensor*, Node*> flash_out;  // transposed flash output -> PV node
  std::unordered_map<Tensor*, HeadPlan> head_out;  // argmax output -> fused head
  std::unordered_map<Tensor*, RouterPlan> router_out;  // its ids / weights / values -> router
  std::vector<std::vector<Tensor*>> gemm_groups;  // outputs of sibling projections
  // reductions emitted in this flush, by (input, op, dims, dtype): a repeat
  // (reduceMean's reduceSum next to a reduceSum of the same tensor) aliases
  // the first result
  std::map<std::tuple<Tensor*, int, std::vector<int64_t>, int>, Tensor*> reduce_done;
  // dense copies made by emit_permuted_copy and not yet freed: released
  // (stream-ordered) when their consumer is enqueued or at the end of the flush
  std::unordered_set<Tensor*> temps;

  explicit Lower(Ctx* ctx) : c(ctx) {}
  void drop_temp(Tensor* t) {
    if (temps.erase(t)) maybe_destroy(t);
  }

  void match_moe();
  bool moe_lowerable(const MoePlan& p);
  bool match_shared(MoePlan& g, Tensor* first_sum);
  bool emit_moe(Tensor* t, const MoePlan& p);
  void dense_rows(Tensor* x, int64_t n, const void** ptr, int64_t* rs);

  bool match_flash(Node* pv);
  void match_gemm_epilogues();
  void match_rows();
  bool plan_norm(NormPlan np, Tensor* x, int x_uses, Tensor* o, std::vector<Tensor*>& inner);
  bool match_layernorm(Node* ao);
  void match_class_head();
  bool emit_class_head(Node* n, const HeadPlan& p);
  void match_router();
  bool emit_router(const RouterPlan& p);
  bool emit_norm(Tensor* t, const NormPlan& p);
  bool emit_rope(Tensor* t, const RopePlan& p);
  bool emit_softmax(Tensor* t, const SoftmaxPlan& p);
  bool rows_view(Tensor* x, int64_t n, const void** ptr, int64_t* rs);
  bool emit_gemm_fused(Tensor* t, const GemmPlan& p);
  bool gemm_fused_args(Tensor* t, const GemmPlan& p, GemmArgs& g);
  bool fuse_rope(const RopePlan& rp, Tensor* out);
  void match_gemm_groups();
  void view4(Tensor* v, int r, const void** ptr, int64_t* s);
  bool emit_flash(Node* pv, const FlashPlan& fp);
  void match_flash_out();
  bool kv_operand(Tensor* t, int H, const void** ptr, int64_t* sb, int64_t* sh,
                  int64_t* ss, int* hkv);

  void ensure_mat(Tensor* t);
  void emit_ew_root(Tensor* t);
  void emit_anchor(Node* n);
  void emit_reduce(Node* n);
  void emit_dot(Node* n);
  void dot_args(Node* n, GemmArgs& g, Tensor*& ta, Tensor*& tb);
  void emit_gather(Node* n);
  void emit_argmax(Node* n);
  void emit_topk(Node* n);
  void emit_sort(Node* n);
  bool emit_gather_norm(Node* n, Tensor* t, const NormPlan& p);
  void emit_index_map(Node* n);
  void emit_window(Node* n);
  void emit_cholesky(Node* n);
  void emit_trisolve(Node* n);
  void emit_complex(Node* n);
  void emit_fft1(Node* n);
  void emit_batchnorm(Node* n);
  // Materialize `t` (any kind) into a fresh dense tensor whose shape is the
  // permutation `perm` of t's shape.
  Tensor* emit_permuted_copy(Tensor* t, const std::vector<int>& perm);
  // Strides (in elements) of every dim of `t` over a materialized base.
  void operand_strides(Tensor* t, Tensor** base, int64_t* off, int64_t* st);
};

// ---------------------------------------------------------------------------
// expression code generation
// ---------------------------------------------------------------------------

struct GenFail {};

struct Gen {
  Lower& L;
  Shape space;             // kernel index space (before collapsing)
  Program P;
  std::vector<Tensor*> leaf_t;
  struct Memo {
    Tensor* t;
    Affine m;
    int clamp;
    int val;
  };
  std::vector<Memo> memo;
  int clamp_depth = 0;
  int n_vals = 0;

  Gen(Lower& l, const Shape& s) : L(l), space(s) {
    std::memset(&P, 0, sizeof(P));
  }

  int emit(uint8_t op, int a = 0, int b = 0, int cc = 0, uint8_t aux = 0,
           uint32_t imm = 0) {
    if (P.n_ins >= kMaxIns) throw GenFail();
    Ins& I = P.ins[P.n_ins++];
    I.op = op;
    I.a = (uint8_t)a;
    I.b = (uint8_t)b;
    I.c = (uint8_t)cc;
    I.aux = aux;
    I.imm = imm;
    I.dst = 0;
    // Until register allocation, operands and dst hold SSA value ids; ids
    // are instruction indices, kept < 256 by kMaxIns.
    I.pad = 0;
    return n_vals++;
  }

  int add_leaf(Tensor* t, const Affine& m, bool iota) {
    int64_t ds[kMaxRank];
    int64_t off = 0, st[kMaxRank] = {0};
    if (iota) {
      // value = coordinate m.row(iota_dim); the caller passes a 1-row map.
      off = m.off[0];
      for (int k = 0; k < m.R; ++k) st[k] = m.S[0][k];
    } else {
      dense_strides(t->shape, ds);
      for (int i = 0; i < m.r; ++i) {
        off += m.off[i] * ds[i];
        for (int k = 0; k < m.R; ++k) st[k] += m.S[i][k] * ds[i];
      }
    }
    for (int i = 0; i < P.n_leaves; ++i) {
      const Leaf& q = P.leaf[i];
      if (leaf_t[i] == t && q.ptr == (iota ? nullptr : t->data()) && q.off == off &&
          (q.clamp_hi >= 0) == (clamp_depth > 0 && !iota)) {
        bool same = true;
        for (int k = 0; k < m.R; ++k)
          if (q.stride[k] != st[k]) same = false;
        if (same) return i;
      }
    }
    if (P.n_leaves >= kMaxLeaves) throw GenFail();
    const int li = P.n_leaves++;
    Leaf& lf = P.leaf[li];
    std::memset(&lf, 0, sizeof(lf));
    lf.ptr = iota ? nullptr : t->data();
    lf.dtype = iota ? (uint8_t)kI32 : (uint8_t)t->dt;
    lf.mode = LM_STRIDED;
    lf.off = (int32_t)off;
    lf.clamp_hi = (!iota && clamp_depth > 0) ? (int32_t)(t->numel() - 1) : -1;
    for (int k = 0; k < m.R; ++k) lf.stride[k] = (int32_t)st[k];
    leaf_t.push_back(t);
    return li;
  }

  uint32_t const_bits(Tensor* t) {
    uint32_t u = 0;
    switch (t->dt) {
      case kF32: case kI32: case kU32: std::memcpy(&u, t->host, 4); break;
      case kBF16: { uint16_t h; std::memcpy(&h, t->host, 2); u = (uint32_t)h << 16; break; }
      case kF16: {
        uint16_t h; std::memcpy(&h, t->host, 2);
        // f16 -> f32 (exact)
        uint32_t sgn = (h & 0x8000u) << 16, e = (h >> 10) & 0x1f, f = h & 0x3ff;
        if (e == 0) {
          float v = std::ldexp((float)f, -24);
          std::memcpy(&u, &v, 4);
          u |= sgn;
        } else if (e == 31) {
          u = sgn | 0x7f800000u | (f << 13);
        } else {
          u = sgn | ((e + 112) << 23) | (f << 13);
        }
        break;
      }
      case kI16: { int16_t v; std::memcpy(&v, t->host, 2); u = (uint32_t)(int32_t)v; break; }
      case kU16: { uint16_t v; std::memcpy(&v, t->host, 2); u = v; break; }
      case kI8: { int8_t v; std::memcpy(&v, t->host, 1); u = (uint32_t)(int32_t)v; break; }
      default: u = t->host[0]; break;  // bool, u8
    }
    return u;
  }

  // Leaf value of a materialized tensor `t` read at map `m`.
  int load_mat(Tensor* t, const Affine& m) {
    if (t->has_host && t->numel() == 1) return emit(OP_CONST, 0, 0, 0, 0, const_bits(t));
    const int li = add_leaf(t, m, false);
    return emit(OP_LOAD, 0, 0, 0, 0, (uint32_t)li);
  }

  int gen(Tensor* u, const Affine& m);
  int gen_node(Node* p, Tensor* u, const Affine& m);
};

static bool is_float_dt(int dt) { return dt == kF32 || dt == kBF16 || dt == kF16; }

// Re-rounds a float register to the storage precision of `dt`, or narrows
// an integer register to its width.
static int fix_width(Gen& g, int v, int dt) {
  switch (dt) {
    case kBF16: return g.emit(OP_RBF16, v);
    case kF16: return g.emit(OP_RF16, v);
    case kI8: return g.emit(OP_SEXT8, v);
    case kU8: return g.emit(OP_ZEXT8, v);
    case kI16: return g.emit(OP_SEXT16, v);
    case kU16: return g.emit(OP_ZEXT16, v);
    default: return v;
  }
}

int Gen::gen(Tensor* u, const Affine& m) {
  if (u->st || !u->prod) return load_mat(u, m);
  Node* p = u->prod;
  if (u->plan_mat) {
    L.ensure_mat(u);
    return load_mat(u, m);
  }
  if (is_view(p->kind)) {
    Affine m2;
    if (compose_view(p, m, &m2)) return gen(p->in[0], m2);
    // A reshape that would split a coordinate: read its input as a dense
    // buffer instead (same linear order as u).
    Tensor* x = p->in[0];
    L.ensure_mat(x);
    if (x->has_host && x->numel() == 1) return load_mat(x, m);
    int64_t ds[kMaxRank];
    dense_strides(u->shape, ds);
    Affine flat;
    flat.R = m.R;
    flat.r = 1;
    for (int i = 0; i < m.r; ++i) {
      flat.off[0] += m.off[i] * ds[i];
      for (int k = 0; k < m.R; ++k) flat.S[0][k] += m.S[i][k] * ds[i];
    }
    // treat x as a 1-D dense buffer
    Shape saved = x->shape;
    x->shape = Shape(std::vector<int64_t>{x->numel()});
    int v = load_mat(x, flat);
    x->shape = saved;
    return v;
  }
  if (is_ew(p->kind)) {
    for (auto& e : memo)
      if (e.t == u && e.clamp == (clamp_depth > 0) && e.m == m) return e.val;
    int v = gen_node(p, u, m);
    memo.push_back({u, m, clamp_depth > 0, v});
    return v;
  }
  L.ensure_mat(u);
  return load_mat(u, m);
}

int Gen::gen_node(Node* p, Tensor* u, const Affine& m) {
  const int odt = u->dt;
  switch (p->kind) {
    case K_BINARY: {
      const int dt = p->in[0]->dt;
      int a = gen(p->in[0], m);
      int b = gen(p->in[1], m);
      uint8_t op = OP_NOP;
      if (is_float_dt(dt)) {
        static const uint8_t fop[] = {OP_ADDF, OP_SUBF, OP_MULF, OP_DIVF, OP_MAXF,
                                      OP_MINF, OP_ATAN2F, OP_POWF, OP_REMF};
        if (p->sub > 8) throw Error(REW_MI355X_ERR_INVALID, "bad float binary op");
        op = fop[p->sub];
        return fix_width(*this, emit(op, a, b), dt);
      }
      if (dt == kBool) {
        switch (p->sub) {
          case 0: case 4: case 10: op = OP_OR; break;    // add, max, or
          case 2: case 5: case 9: op = OP_AND; break;    // mul, min, and
          case 11: op = OP_XOR; break;
          default:
            throw Error(REW_MI355X_ERR_UNSUPPORTED,
                        "eager '" + p->name + "': not supported on bool");
        }
        return emit(op, a, b);
      }
      const bool un = !dt_is_signed(dt);
      switch (p->sub) {
        case 0: op = OP_ADDI; break;
        case 1: op = OP_SUBI; break;
        case 2: op = OP_MULI; break;
        case 3: op = un ? OP_DIVU : OP_DIVI; break;
        case 4: op = un ? OP_MAXU : OP_MAXI; break;
        case 5: op = un ? OP_MINU : OP_MINI; break;
        case 8: op = un ? OP_REMU : OP_REMI; break;
        case 9: op = OP_AND; break;
        case 10: op = OP_OR; break;
        case 11: op = OP_XOR; break;
        case 12: op = OP_SHL; break;
        case 13: op = OP_SHRA; break;
        case 14: op = OP_SHRL; break;
        default:
          throw Error(REW_MI355X_ERR_UNSUPPORTED,
                      "eager '" + p->name + "': not supported on integers");
      }
      return fix_width(*this, emit(op, a, b), dt);
    }
    case K_UNARY: {
      const int dt = p->in[0]->dt;
      int a = gen(p->in[0], m);
      static const uint8_t fop[] = {
          OP_NEGF, OP_ABSF, OP_EXPF, OP_LOGF, OP_SQRTF, OP_TANHF, OP_CBRTF,
          OP_CEILF, OP_EXPM1F, OP_FLOORF, OP_LOG1PF, OP_LOGISTICF, OP_TANF,
          OP_SIGNF, OP_ROUNDAFZF, OP_ROUNDEVENF, OP_NOP, OP_NOP, OP_NOP, OP_NOP,
          OP_SINF, OP_COSF, OP_RSQRTF};
      if (p->sub == 19) return a;  // optimizationBarrier / stopGradient
      if (is_float_dt(dt)) return fix_width(*this, emit(fop[p->sub], a), dt);
      uint8_t op;
      switch (p->sub) {
        case 0: op = OP_NEGI; break;
        case 1: op = OP_ABSI; break;
        case 13: op = OP_SIGNI; break;
        case 16: op = dt == kBool ? OP_NOTB : OP_NOT; break;
        case 17:
          if (dt_size(dt) != 4)
            throw Error(REW_MI355X_ERR_UNSUPPORTED, "countLeadingZeros: 32-bit only");
          op = OP_CLZ;
          break;
        case 18:
          if (dt_size(dt) != 4) {
            a = emit(dt_size(dt) == 1 ? OP_ZEXT8 : OP_ZEXT16, a);
          }
          op = OP_POPCNT;
          break;
        default:
          throw Error(REW_MI355X_ERR_UNSUPPORTED, "eager '" + p->name + "' on integers");
      }
      int v = emit(op, a);
      return dt == kBool ? v : fix_width(*this, v, dt);
    }
    case K_CONVERT: {
      const int sdt = p->in[0]->dt, ddt = odt;
      int a = gen(p->in[0], m);
      if (sdt == ddt) return a;
      const bool sf = is_float_dt(sdt), df = is_float_dt(ddt);
      if (sf && df) return fix_width(*this, a, ddt);
      if (sf && ddt == kBool) return emit(OP_FTOBOOL, a);
      if (sf) {
        int v = emit(dt_is_signed(ddt) ? OP_F2I : OP_F2U, a);
        return fix_width(*this, v, ddt);
      }
      // integer / bool source
      if (df) {
        int v = emit((dt_is_signed(sdt)) ? OP_I2F : OP_U2F, a);
        return fix_width(*this, v, ddt);
      }
      if (ddt == kBool) return emit(OP_TOBOOL, a);
      return fix_width(*this, a, ddt);
    }
    case K_ISFINITE:
      return emit(OP_ISFINITEF, gen(p->in[0], m));
    case K_REDUCE_PRECISION: {
      int a = gen(p->in[0], m);
      if (p->i1 == 7) return emit(OP_RBF16, a);
      if (p->i1 == 10) return emit(OP_RF16, a);
      return a;
    }
    case K_COMPARE: {
      const int dt = p->in[0]->dt;
      int a = gen(p->in[0], m), b = gen(p->in[1], m);
      uint8_t op = is_float_dt(dt) ? OP_CMPF : (dt_is_signed(dt) ? OP_CMPI : OP_CMPU);
      return emit(op, a, b, 0, (uint8_t)p->cmp);
    }
    case K_SELECT: {
      int pr = gen(p->in[0], m);
      int a = gen(p->in[1], m);
      int b = gen(p->in[2], m);
      return emit(OP_SELECT, pr, a, b);
    }
    case K_CLAMP: {
      const int dt = p->in[1]->dt;
      auto bound = [&](Tensor* t) {
        if (t->shape.rank == 0) {
          Affine z;
          z.R = m.R;
          z.r = 0;
          return gen(t, z);
        }
        return gen(t, m);
      };
      int lo = bound(p->in[0]);
      int x = gen(p->in[1], m);
      int hi = bound(p->in[2]);
      uint8_t op = is_float_dt(dt) ? OP_CLAMPF : (dt_is_signed(dt) ? OP_CLAMPI : OP_CLAMPU);
      return emit(op, lo, x, hi);
    }
    case K_CONST:  // a 32-bit integer scalar fixed by the op
      return emit(OP_CONST, 0, 0, 0, 0, (uint32_t)p->i0);
    case K_IOTA: {
      Affine row;
      row.R = m.R;
      row.r = 1;
      row.off[0] = m.off[p->i0];
      for (int k = 0; k < m.R; ++k) row.S[0][k] = m.S[p->i0][k];
      const int li = add_leaf(u, row, true);
      int v = emit(OP_IOTA, 0, 0, 0, 0, (uint32_t)li);
      if (is_float_dt(odt)) return fix_width(*this, emit(OP_I2F, v), odt);
      return fix_width(*this, v, odt);
    }
    case K_CONCAT: {
      const int dim = (int)p->i0;
      const int nparts = (int)p->in.size();
      std::vector<int> vals(nparts);
      std::vector<int64_t> starts(nparts);
      int64_t o = 0;
      for (int j = 0; j < nparts; ++j) {
        starts[j] = o;
        Affine mj = m;
        mj.off[dim] -= o;
        if (nparts > 1) ++clamp_depth;
        vals[j] = gen(p->in[j], mj);
        if (nparts > 1) --clamp_depth;
        o += p->in[j]->shape.d[dim];
      }
      if (nparts == 1) return vals[0];
      Affine row;
      row.R = m.R;
      row.r = 1;
      row.off[0] = m.off[dim];
      for (int k = 0; k < m.R; ++k) row.S[0][k] = m.S[dim][k];
      const int li = add_leaf(u, row, true);
      int coord = emit(OP_IOTA, 0, 0, 0, 0, (uint32_t)li);
      int r = vals[nparts - 1];
      for (int j = nparts - 2; j >= 0; --j) {
        int lim = emit(OP_CONST, 0, 0, 0, 0, (uint32_t)starts[j + 1]);
        int cond = emit(OP_CMPI, coord, lim, 0, CMP_LT);
        r = emit(OP_SELECT, cond, vals[j], r);
      }
      return r;
    }
    default:
      throw Error(REW_MI355X_ERR_UNSUPPORTED, "cannot fuse op '" + p->name + "'");
  }
}

// ---------------------------------------------------------------------------
// program finishing: dim collapsing, leaf modes, register allocation
// ---------------------------------------------------------------------------

static FastDiv make_fastdiv(uint32_t d) {
  FastDiv f;
  f.d = d;
  uint32_t s = 0;
  while (((uint64_t)1 << s) < d) ++s;
  f.s = s;
  f.m = (uint32_t)((((uint64_t)1 << 32) * (((uint64_t)1 << s) - d)) / d + 1);
  return f;
}

// Collapses the kernel space: drops unit dims and merges neighbours whose
// strides agree for every leaf and output.  `groups` marks dims that must
// not merge across (the kept/reduced boundary of a reduction).
static Space finish_space(Program& P, const Shape& space, int boundary,
                          std::vector<int64_t>* out_dims) {
  const int R = space.rank;
  std::vector<int> keep;
  for (int k = 0; k < R; ++k)
    if (space.d[k] != 1) keep.push_back(k);
  // merged dims as lists of original dims
  std::vector<std::vector<int>> groups;
  std::vector<int64_t> sizes;
  for (int k : keep) {
    bool merged = false;
    if (!groups.empty()) {
      const int prev = groups.back().back();
      const bool cross = boundary >= 0 && prev < boundary && k >= boundary;
      if (!cross) {
        bool ok = true;
        for (int l = 0; l < P.n_leaves && ok; ++l)
          if ((int64_t)P.leaf[l].stride[prev] != (int64_t)P.leaf[l].stride[k] * space.d[k])
            ok = false;
        if (ok) {
          groups.back().push_back(k);
          sizes.back() *= space.d[k];
          merged = true;
        }
      }
    }
    if (!merged) {
      groups.push_back({k});
      sizes.push_back(space.d[k]);
    }
  }
  // rewrite leaf strides: stride of a merged group = stride of its last dim
  for (int l = 0; l < P.n_leaves; ++l) {
    int32_t ns[kRank] = {0};
    for (size_t g = 0; g < groups.size(); ++g) ns[g] = P.leaf[l].stride[groups[g].back()];
    std::memcpy(P.leaf[l].stride, ns, sizeof(ns));
  }
  Space S;
  std::memset(&S, 0, sizeof(S));
  S.rank = (int)groups.size();
  S.numel = space.numel();
  for (size_t g = 0; g < groups.size(); ++g) S.dim[g] = make_fastdiv((uint32_t)sizes[g]);
  if (S.rank == 0) {  // scalar space
    S.rank = 1;
    S.dim[0] = make_fastdiv(1);
    sizes.push_back(1);
  }
  if (out_dims) *out_dims = sizes;
  // reduction boundary after collapsing is recomputed by the caller
  return S;
}

// Refuses to launch a program whose leaves could address outside their
// tensors anywhere in the kernel space (clamped concat leaves excepted):
// a planner bug becomes a host error, never a device fault.
static void check_bounds(const Program& P, const std::vector<Tensor*>& leaf_t,
                         const std::vector<int64_t>& dims) {
  for (int l = 0; l < P.n_leaves; ++l) {
    const Leaf& lf = P.leaf[l];
    if (!lf.ptr || lf.clamp_hi >= 0) continue;
    int64_t lo = lf.off, hi = lf.off;
    for (size_t k = 0; k < dims.size(); ++k) {
      const int64_t e = (int64_t)lf.stride[k] * (dims[k] - 1);
      if (e < 0) lo += e; else hi += e;
    }
    const int64_t n = leaf_t[l]->numel();
    if (lo < 0 || hi >= n)
      throw Error(REW_MI355X_ERR_INVALID,
                  "internal: fused program would read elements [" + std::to_string(lo) +
                      ", " + std::to_string(hi) + "] of a tensor with " + std::to_string(n));
  }
}

// Leaf addressing modes for a kVec-wide lane when `vec`.
static void set_leaf_modes(Program& P, const Space& S, bool vec) {
  const int in = S.rank - 1;
  for (int l = 0; l < P.n_leaves; ++l) {
    Leaf& lf = P.leaf[l];
    lf.mode = LM_STRIDED;
    if (!vec || !lf.ptr || lf.clamp_hi >= 0) continue;
    if (lf.stride[in] == 0) {
      lf.mode = LM_BCAST;
      continue;
    }
    if (lf.stride[in] != 1) continue;
    bool al = (lf.off % kVec) == 0;
    for (int k = 0; k < in; ++k)
      if (lf.stride[k] % kVec != 0) al = false;
    const int esz = dt_size(lf.dtype);
    const uintptr_t need = (uintptr_t)(esz * kVec);
    if (((uintptr_t)lf.ptr % need) != 0) al = false;
    if (al && (lf.dtype == kF32 || lf.dtype == kI32 || lf.dtype == kU32 ||
               lf.dtype == kBF16))
      lf.mode = LM_CONTIG;
  }
}

// Linear-scan register allocation over the SSA program.  `live_out` values
// must survive to the end.
static void alloc_regs(Program& P, const std::vector<int>& live_out,
                       std::vector<int>* phys_of_out) {
  const int n = P.n_ins;
  std::vector<int> last(n, -1);
  auto use = [&](int v, int at) { if (v >= 0 && v < n) last[v] = std::max(last[v], at); };
  for (int i = 0; i < n; ++i) {
    const Ins& I = P.ins[i];
    int ar;
    if (I.op <= OP_IOTA) ar = 0;
    else if (I.op >= OP_SELECT && I.op <= OP_CLAMPU) ar = 3;
    else if ((I.op >= OP_ADDF && I.op <= OP_SHRL) || (I.op >= OP_CMPF && I.op <= OP_CMPU)) ar = 2;
    else ar = 1;
    if (ar >= 1) use(I.a, i);
    if (ar >= 2) use(I.b, i);
    if (ar >= 3) use(I.c, i);
  }
  for (int v : live_out) last[v] = n;
  std::vector<int> phys(n, -1);
  std::vector<int> free_regs;
  for (int r = kMaxRegs - 1; r >= 0; --r) free_regs.push_back(r);
  std::vector<std::vector<int>> expire(n + 1);
  for (int i = 0; i < n; ++i) {
    Ins& I = P.ins[i];
    int ar;
    if (I.op <= OP_IOTA) ar = 0;
    else if (I.op >= OP_SELECT && I.op <= OP_CLAMPU) ar = 3;
    else if ((I.op >= OP_ADDF && I.op <= OP_SHRL) || (I.op >= OP_CMPF && I.op <= OP_CMPU)) ar = 2;
    else ar = 1;
    // operands read before the destination is written, so registers of
    // operands dying here may be reused as the destination
    int pa = ar >= 1 ? phys[I.a] : 0, pb = ar >= 2 ? phys[I.b] : 0,
        pc = ar >= 3 ? phys[I.c] : 0;
    for (int v : expire[i]) free_regs.push_back(phys[v]);
    if (free_regs.empty()) throw GenFail();
    const int r = free_regs.back();
    free_regs.pop_back();
    phys[i] = r;
    I.a = (uint8_t)pa;
    I.b = (uint8_t)pb;
    I.c = (uint8_t)pc;
    I.dst = (uint8_t)r;
    const int end = last[i] < 0 ? i : last[i];
    if (end >= n) continue;
    if (end == i) {
      free_regs.push_back(r);  // dead value
    } else {
      expire[end].push_back(i);
    }
  }
  phys_of_out->clear();
  for (int v : live_out) phys_of_out->push_back(phys[v]);
}

// ---------------------------------------------------------------------------
// emission
// ---------------------------------------------------------------------------

void Lower::ensure_mat(Tensor* t) {
  if (t->st) return;
  auto rtt = router_out.find(t);
  if (rtt != router_out.end()) {
    const RouterPlan rp = rtt->second;
    for (Tensor* o : {rp.ids, rp.vals, rp.wts})
      if (o) router_out.erase(o);
    if (emit_router(rp) && t->st) return;
    // outside the fused kernel's limits: the chain's own plans run
  }
  auto git = gemm_out.find(t);
  if (git != gemm_out.end()) {
    GemmPlan gp = git->second;
    gemm_out.erase(git);
    if (emit_gemm_fused(t, gp)) return;
    // not launchable fused: the expression is rebuilt around a plain GEMM
  }
  auto nit = norm_out.find(t);
  if (nit != norm_out.end()) {
    NormPlan np = nit->second;
    norm_out.erase(nit);
    if (emit_norm(t, np)) return;
  }
  auto rit = rope_out.find(t);
  if (rit != rope_out.end()) {
    RopePlan rp = rit->second;
    rope_out.erase(rit);
    if (emit_rope(t, rp)) return;
  }
  auto sit = softmax_out.find(t);
  if (sit != softmax_out.end()) {
    SoftmaxPlan sp = sit->second;
    softmax_out.erase(sit);
    if (emit_softmax(t, sp)) return;
  }
  auto fit = flash_out.find(t);
  if (fit != flash_out.end()) {
    Node* pv = fit->second;
    flash_out.erase(fit);
    auto pit = flash.find(pv);
    if (pit != flash.end()) {
      FlashPlan fp = pit->second;
      if (emit_flash(pv, fp)) {
        flash.erase(pit);
        return;
      }
      // not launchable: the attention output is produced by the generic path
      // and transposed by the elementwise kernel below
      flash[pv].out_t = nullptr;
    }
  }
  auto mit = moe_out.find(t);
  if (mit != moe_out.end()) {
    MoePlan mp = mit->second;
    moe_out.erase(mit);
    if (emit_moe(t, mp)) return;
    throw Error(REW_MI355X_ERR_UNSUPPORTED, "routed MoE chain could not be lowered");
  }
  Node* p = t->prod;
  if (!p) throw Error(REW_MI355X_ERR_INVALID, "internal: tensor has neither data nor producer");
  if (is_ew(p->kind) || is_view(p->kind)) {
    // a reshape (or a chain of reshapes) of a materialized or materializable
    // dense tensor aliases it
    if (p->kind == K_RESHAPE) {
      Tensor* x = p->in[0];
      Tensor* y = x;
      while (!y->st && !y->plan_mat && y->prod && y->prod->kind == K_RESHAPE) y = y->prod->in[0];
      if (y->st || y->plan_mat || !y->prod) {
        ensure_mat(x);
        tensor_alias(t, x);
        return;
      }
    }
    emit_ew_root(t);
    return;
  }
  emit_anchor(p);
  if (!t->st) throw Error(REW_MI355X_ERR_INVALID, "internal: anchor did not materialize");
}

void Lower::emit_ew_root(Tensor* t) {
  // Kernel space: the deepest reshape source with the same linear order.
  Tensor* root = t;
  while (root->prod && root->prod->kind == K_RESHAPE && !root->prod->in[0]->st &&
         !root->prod->in[0]->plan_mat && root->prod->in[0]->prod &&
         (is_ew(root->prod->in[0]->prod->kind) || is_view(root->prod->in[0]->prod->kind)))
    root = root->prod->in[0];
  for (int attempt = 0; attempt < 64; ++attempt) {
    Gen g(*this, root->shape);
    try {
      Affine id = Affine::identity(root->shape.rank);
      int v;
      if (root == t) {
        // gen(t) would return a load of t once materialized; expand its node
        Node* p = t->prod;
        if (is_view(p->kind)) {
          Affine m2;
          if (!compose_view(p, id, &m2))
            throw Error(REW_MI355X_ERR_INVALID, "internal: view root not composable");
          v = g.gen(p->in[0], m2);
        } else {
          v = g.gen_node(p, t, id);
        }
      } else {
        v = g.gen(root, id);
      }
      tensor_alloc(t);
      std::vector<int64_t> dims;
      Space S = finish_space(g.P, root->shape, -1, &dims);
      check_bounds(g.P, g.leaf_t, dims);
      std::vector<int> outs_phys;
      alloc_regs(g.P, {v}, &outs_phys);
      g.P.n_outs = 1;
      g.P.out[0].ptr = t->data();
      g.P.out[0].dtype = (uint8_t)t->dt;
      g.P.out[0].reg = (uint8_t)outs_phys[0];
      g.P.out[0].off = 0;
      const bool vec = (dims.back() % kVec) == 0 &&
                       ((uintptr_t)t->data() % (dt_size(t->dt) * kVec)) == 0 &&
                       (t->dt == kF32 || t->dt == kI32 || t->dt == kU32 || t->dt == kBF16);
      set_leaf_modes(g.P, S, vec);
      Launch L{EwL{g.P, S, vec}};
      if (c->profiling)
        L.name = "ew_fused{" + std::to_string(S.numel) + "x" + std::to_string(g.P.n_ins) +
                 "," + dt_name(t->dt) + "," + (t->prod ? t->prod->name : "?") + "}";
      L.fused = g.P.n_ins > 2;
      run_launch(c, std::move(L));
      return;
    } catch (GenFail&) {
      tensor_drop_storage(t);
      // Too large for one program: materialize the direct inputs of the
      // root's expression and retry.
      Node* p = root->prod;
      bool progressed = false;
      std::function<void(Node*, int)> mat_inputs = [&](Node* q, int depth) {
        for (Tensor* x : q->in) {
          if (x->st) continue;
          if (x->prod && is_view(x->prod->kind) && depth < 8) {
            mat_inputs(x->prod, depth + 1);
            continue;
          }
          x->plan_mat = true;
          progressed = true;
        }
      };
      mat_inputs(p, 0);
      if (!progressed)
        throw Error(REW_MI355X_ERR_UNSUPPORTED, "expression too large to lower");
    }
  }
  throw Error(REW_MI355X_ERR_UNSUPPORTED, "expression too large to lower");
}

void Lower::emit_anchor(Node* n) {
  switch (n->kind) {
    case K_REDUCE: emit_reduce(n); break;
    case K_DOT_GENERAL: emit_dot(n); break;
    case K_INDEX_SELECT: emit_gather(n); break;
    case K_ARGMAX: emit_argmax(n); break;
    case K_TOPK: emit_topk(n); break;
    case K_SORT: emit_sort(n); break;
    case K_GATHER:
    case K_SCATTER: emit_index_map(n); break;
    case K_WINDOW: emit_window(n); break;
    case K_CHOLESKY: emit_cholesky(n); break;
    case K_TRISOLVE: emit_trisolve(n); break;
    case K_COMPLEX: emit_complex(n); break;
    case K_FFT1: emit_fft1(n); break;
    case K_BATCHNORM: emit_batchnorm(n); break;
    case K_BITCAST: {
      Tensor* x = n->in[0];
      ensure_mat(x);
      tensor_alias(n->out[0], x);
      break;
    }
    default:
      throw Error(REW_MI355X_ERR_UNSUPPORTED, "no lowering for op '" + n->name + "'");
  }
}

void Lower::emit_reduce(Node* n) {
  Tensor* x = n->in[0];
  Tensor* out = n->out[0];
  const auto key = std::make_tuple(x, n->sub, n->l0, out->dt);
  auto done = reduce_done.find(key);
  if (done != reduce_done.end() && done->second->st && done->second->shape == out->shape) {
    tensor_alias(out, done->second);
    return;
  }
  const Shape& X = x->shape;
  std::vector<bool> red(X.rank, false);
  for (auto d : n->l0) red[d] = true;
  std::vector<int> order;
  for (int i = 0; i < X.rank; ++i)
    if (!red[i]) order.push_back(i);
  const int n_kept = (int)order.size();
  for (int i = 0; i < X.rank; ++i)
    if (red[i]) order.push_back(i);
  Shape space;
  space.rank = X.rank;
  Affine m;
  m.R = m.r = X.rank;
  int64_t n_out = 1, n_red = 1;
  for (int k = 0; k < X.rank; ++k) {
    space.d[k] = X.d[order[k]];
    m.S[order[k]][k] = 1;
    if (k < n_kept) n_out *= space.d[k]; else n_red *= space.d[k];
  }
  for (int attempt = 0; attempt < 2; ++attempt) {
    Gen g(*this, space);
    try {
      int v = g.gen(x, m);
      std::vector<int64_t> dims;
      // collapse; keep the kept/reduced boundary
      Space S = finish_space(g.P, space, n_kept, &dims);
      check_bounds(g.P, g.leaf_t, dims);
      std::vector<int> phys;
      alloc_regs(g.P, {v}, &phys);
      g.P.n_outs = 1;
      g.P.out[0].reg = (uint8_t)phys[0];
      tensor_alloc(out);
      ReduceArgs A;
      A.op = n->sub;
      A.n_out = (uint32_t)n_out;
      A.n_red = (uint32_t)n_red;
      A.out = out->data();
      A.out_dtype = out->dt;
      // sibling reductions of the same tensor over the same axes (other ops)
      // ride along in the same pass
      std::vector<Node*> sib;
      for (Node* m : nodes) {
        if (m == n || m->kind != K_REDUCE || m->in[0] != x || m->l0 != n->l0 || m->sub == n->sub)
          continue;
        Tensor* mo = m->out[0];
        if (mo->st || !mo->plan_mat || mo->dt != out->dt || sib.size() == 3) continue;
        bool dup = false;
        for (Node* q : sib) dup = dup || q->sub == m->sub;
        if (dup) continue;
        sib.push_back(m);
      }
      for (Node* m : sib) {
        tensor_alloc(m->out[0]);
        A.extra_op[A.n_extra] = m->sub;
        A.extra_out[A.n_extra++] = m->out[0]->data();
      }
      // reduceMean (reduce.nim:132-150): divide(sum, broadcastTo(n)) of this
      // sum or of a repeat of it in this flush, stored by the same pass
      if (out->dt == kF32 && !cons.empty()) {
        for (int src = 0; src <= (int)sib.size() && A.n_mean < 2; ++src) {
          Node* rn = src ? sib[src - 1] : n;
          if (rn->sub != RED_SUM) continue;
          for (Node* q : nodes) {
            if (q->kind != K_REDUCE || q->in[0] != x || q->l0 != rn->l0 || q->sub != RED_SUM ||
                q->out[0]->dt != kF32)
              continue;
            auto ci = cons.find(q->out[0]);
            if (ci == cons.end()) continue;
            for (Node* d : ci->second) {
              float dv;
              Tensor* dt_ = d->out[0];
              if (A.n_mean == 2 || d->kind != K_BINARY || d->sub != 3 ||
                  d->in[0] != q->out[0] || !const_bcast(d->in[1], &dv) || dt_->dt != kF32 ||
                  dt_->shape != out->shape || dt_->st || !dt_->plan_mat)
                continue;
              tensor_alloc(dt_);
              A.mean_src[A.n_mean] = src;
              A.mean_div[A.n_mean] = dv;
              A.mean_out[A.n_mean++] = dt_->data();
            }
          }
        }
      }
      const bool vec = n_red > 0 && (dims.back() % kVec) == 0 &&
                       (n_red % kVec) == 0 && space.d[X.rank - 1] != 1;
      set_leaf_modes(g.P, S, vec);
      Launch L{ReduceL{g.P, S, A, vec}};
      if (c->profiling)
        L.name = "reduce{" + std::to_string(n_out) + "x" + std::to_string(n_red) + "x" +
                 std::to_string(g.P.n_ins) +
                 (sib.empty() ? "" : "," + std::to_string(1 + sib.size()) + "ops") +
                 (A.n_mean ? ",mean" : "") + "}";
      L.fused = g.P.n_ins > 1 || !sib.empty();
      run_launch(c, std::move(L));
      reduce_done[key] = out;
      for (Node* m : sib) reduce_done[std::make_tuple(x, m->sub, m->l0, out->dt)] = m->out[0];
      return;
    } catch (GenFail&) {
      tensor_drop_storage(out);
      x->plan_mat = true;
      ensure_mat(x);
    }
  }
  throw Error(REW_MI355X_ERR_UNSUPPORTED, "reduction prologue too large");
}

void Lower::operand_strides(Tensor* t, Tensor** base, int64_t* off, int64_t* st) {
  Affine m = Affine::identity(t->shape.rank);
  Tensor* u = t;
  for (;;) {
    if (u->st || !u->prod) break;
    Node* p = u->prod;
    if (u->plan_mat || !is_view(p->kind)) {
      ensure_mat(u);
      break;
    }
    Affine m2;
    if (!compose_view(p, m, &m2)) {
      // reshape that splits a coordinate: read u as dense (its input
      // materialized in the same linear order)
      ensure_mat(u);
      break;
    }
    m = m2;
    u = p->in[0];
  }
  int64_t ds[kMaxRank];
  dense_strides(u->shape, ds);
  *off = 0;
  for (int k = 0; k < m.R; ++k) st[k] = 0;
  for (int i = 0; i < m.r; ++i) {
    *off += m.off[i] * ds[i];
    for (int k = 0; k < m.R; ++k) st[k] += m.S[i][k] * ds[i];
  }
  *base = u;
}

Tensor* Lower::emit_permuted_copy(Tensor* t, const std::vector<int>& perm) {
  Shape s;
  s.rank = t->shape.rank;
  for (int i = 0; i < s.rank; ++i) s.d[i] = t->shape.d[perm[i]];
  Tensor* out = new_tensor(c, t->dt, s);
  out->plan_dead = true;  // marks a planner-private temporary
  temps.insert(out);
  Affine m;
  m.R = m.r = s.rank;
  for (int k = 0; k < s.rank; ++k) m.S[perm[k]][k] = 1;
  Gen g(*this, s);
  int v = g.gen(t, m);
  tensor_alloc(out);
  std::vector<int64_t> dims;
  Space S = finish_space(g.P, s, -1, &dims);
  check_bounds(g.P, g.leaf_t, dims);
  std::vector<int> phys;
  alloc_regs(g.P, {v}, &phys);
  g.P.n_outs = 1;
  g.P.out[0].ptr = out->data();
  g.P.out[0].dtype = (uint8_t)out->dt;
  g.P.out[0].reg = (uint8_t)phys[0];
  const bool vec = (dims.back() % kVec) == 0 &&
                   (out->dt == kF32 || out->dt == kI32 || out->dt == kBF16);
  set_leaf_modes(g.P, S, vec);
  Launch L{EwL{g.P, S, vec}};
  if (c->profiling) L.name = "ew_copy";
  run_launch(c, std::move(L));
  return out;
}

// Merges the dims `dims` (in order) of a strided operand into one
// (size, stride); false when they are not uniformly strided.
static bool merge_group(const Shape& s, const int64_t* st, const std::vector<int64_t>& dims,
                        int64_t* size, int64_t* stride) {
  int64_t sz = 1, str = 0;
  bool have = false;
  int64_t prev_st = 0, prev_sz = 0;
  for (auto d : dims) {
    if (s.d[d] == 1) continue;
    if (have && prev_st != st[d] * s.d[d]) return false;
    prev_st = st[d];
    prev_sz = s.d[d];
    sz *= s.d[d];
    str = st[d];
    have = true;
  }
  (void)prev_sz;
  for (auto d : dims) if (s.d[d] == 0) sz = 0;
  *size = sz;
  *stride = have ? str : 0;
  return true;
}

// GEMM operands of dot_general node `n`: batch / free / contracting groups
// merged into strided [batch, M, K] x [batch, K, N] views (dense copies
// where a group is not uniformly strided); ta / tb are the base tensors.
void Lower::dot_args(Node* n, GemmArgs& g, Tensor*& ta_out, Tensor*& tb_out) {
  Tensor *a = n->in[0], *b = n->in[1], *out = n->out[0];
  (void)out;
  const std::vector<int64_t> &lb = n->l0, &rb = n->l1, &lc = n->l2, &rc = n->l3;
  std::vector<int64_t> lf, rf;
  {
    std::vector<bool> u(a->shape.rank, false);
    for (auto d : lb) u[d] = true;
    for (auto d : lc) u[d] = true;
    for (int i = 0; i < a->shape.rank; ++i) if (!u[i]) lf.push_back(i);
    std::vector<bool> v(b->shape.rank, false);
    for (auto d : rb) v[d] = true;
    for (auto d : rc) v[d] = true;
    for (int i = 0; i < b->shape.rank; ++i) if (!v[i]) rf.push_back(i);
  }
  std::memset(&g, 0, sizeof(g));
  g.dtype = a->dt;
  g.c_dtype = out->dt;

  auto prep = [&](Tensor* t, const std::vector<int64_t>& g0,
                  const std::vector<int64_t>& g1, const std::vector<int64_t>& g2,
                  const void** ptr, int64_t* n0, int64_t* s0, int64_t* n1,
                  int64_t* s1, int64_t* n2, int64_t* s2) {
    for (int attempt = 0; attempt < 2; ++attempt) {
      Tensor* base;
      int64_t off, st[kMaxRank];
      operand_strides(t, &base, &off, st);
      if (merge_group(t->shape, st, g0, n0, s0) && merge_group(t->shape, st, g1, n1, s1) &&
          merge_group(t->shape, st, g2, n2, s2)) {
        *ptr = (const char*)base->data() + off * dt_size(base->dt);
        return base;
      }
      // canonical dense copy [g0..., g1..., g2...]
      std::vector<int> perm;
      for (auto d : g0) perm.push_back((int)d);
      for (auto d : g1) perm.push_back((int)d);
      for (auto d : g2) perm.push_back((int)d);
      Tensor* cp = emit_permuted_copy(t, perm);
      int64_t ds[kMaxRank];
      dense_strides(cp->shape, ds);
      // rebuild groups on the copy
      std::vector<int64_t> h0, h1, h2;
      int k = 0;
      for (size_t i = 0; i < g0.size(); ++i) h0.push_back(k++);
      for (size_t i = 0; i < g1.size(); ++i) h1.push_back(k++);
      for (size_t i = 0; i < g2.size(); ++i) h2.push_back(k++);
      merge_group(cp->shape, ds, h0, n0, s0);
      merge_group(cp->shape, ds, h1, n1, s1);
      merge_group(cp->shape, ds, h2, n2, s2);
      *ptr = cp->data();
      return cp;
    }
    return (Tensor*)nullptr;
  };
  int64_t bA, bB, kA, kB;
  Tensor* ta = prep(a, lb, lf, lc, &g.a, &bA, &g.a_sb, &g.M, &g.a_sm, &kA, &g.a_sk);
  Tensor* tb = prep(b, rb, rc, rf, &g.b, &bB, &g.b_sb, &kB, &g.b_sk, &g.N, &g.b_sn);
  g.batch = bA;
  g.K = kA;
  if (g.M == 1) g.a_sm = 0;
  if (g.N == 1) g.b_sn = 0;
  if (g.batch == 1) { g.a_sb = 0; g.b_sb = 0; }
  if (g.K == 1) { g.a_sk = 0; g.b_sk = 0; }
  // operand extents must stay inside their base tensors
  auto extent_ok = [&](Tensor* base, const void* p, int64_t n0, int64_t s0, int64_t n1,
                       int64_t s1, int64_t n2, int64_t s2) {
    const int64_t off = ((const char*)p - (const char*)base->data()) / dt_size(base->dt);
    int64_t lo = off, hi = off;
    for (auto e : {s0 * (n0 - 1), s1 * (n1 - 1), s2 * (n2 - 1)}) {
      if (e < 0) lo += e; else hi += e;
    }
    return lo >= 0 && hi < base->numel();
  };
  if (g.batch > 0 && g.M > 0 && g.N > 0 && g.K > 0 &&
      (!extent_ok(ta, g.a, g.batch, g.a_sb, g.M, g.a_sm, g.K, g.a_sk) ||
       !extent_ok(tb, g.b, g.batch, g.b_sb, g.K, g.b_sk, g.N, g.b_sn)))
    throw Error(REW_MI355X_ERR_INVALID, "internal: dot_general operand view out of bounds");
  ta_out = ta;
  tb_out = tb;
}

void Lower::emit_dot(Node* n) {
  auto fit = flash.find(n);
  if (fit != flash.end()) {
    FlashPlan fp = fit->second;
    flash.erase(fit);
    if (emit_flash(n, fp)) return;
    // unsupported layout: the chain is rebuilt on demand by the generic path
  }
  Tensor *a = n->in[0], *b = n->in[1], *out = n->out[0];
  GemmArgs g;
  Tensor *ta, *tb;
  dot_args(n, g, ta, tb);
  tensor_alloc(out);
  g.c = out->data();
  g.c_sb = g.M * g.N;
  g.c_sm = g.N;
  if (g.K == 0) {
    // empty contraction: zeros
    run_launch(c, Launch{FillL{out->data(), nullptr, (size_t)out->nbytes()}});
  } else {
    Launch L{GemmL{{g}, false}};
    if (c->profiling) {
      // "<variant>[batch,M,N,K]": the shape fixes the algorithmic FLOPs
      char nm[160];
      std::snprintf(nm, sizeof nm, "%s[%lld,%lld,%lld,%lld]", gemm_variant(g),
                    (long long)g.batch, (long long)g.M, (long long)g.N, (long long)g.K);
      L.name = nm;
    }
    run_launch(c, std::move(L));
  }
  // canonical copies made for this GEMM die with it (stream-ordered free)
  for (Tensor* t : {ta, tb})
    if (t && t != a && t != b) drop_temp(t);
}


// ---------------------------------------------------------------------------
// fused attention: recognition of rew's SDPA op chain
// ---------------------------------------------------------------------------

// Pending (not materialized, not held by the caller) output of a node of
// `kind`, consumed exactly `uses` times inside the graph.
static Node* chain_node(Tensor* t, int kind, int uses) {
  if (!t || t->st || !t->prod || t->ext != 0 || t->uses != uses) return nullptr;
  return t->prod->kind == kind ? t->prod : nullptr;
}

static bool dims_are(const std::vector<int64_t>& v, std::initializer_list<int64_t> w) {
  return v.size() == w.size() && std::equal(v.begin(), v.end(), w.begin());
}

// Value of broadcastTo(scalar f32 constant, shape, []) (src/rew/ops/literal.nim:56-77).
static bool const_bcast(Tensor* t, float* val) {
  if (!t || t->st || !t->prod || t->prod->kind != K_BROADCAST_TO) return false;
  Tensor* s = t->prod->in[0];
  if (s->shape.rank != 0 || s->dt != kF32 || !s->has_host) return false;
  std::memcpy(val, s->host, 4);
  return true;
}

// makeCausalMask (src/rew/nn/attention.nim:18-34):
//   select(compare(iota(dim 0), iota(dim 1), dir), bcast(a), bcast(b))
// broadcast over the two trailing dims of the scores.
static bool match_mask(Tensor* maskB, int64_t Sq, int64_t Sk, FlashPlan* fp) {
  if (!maskB || maskB->st || !maskB->prod || maskB->prod->kind != K_BROADCAST_TO) return false;
  Node* bc = maskB->prod;
  if (!dims_are(bc->l1, {2, 3})) return false;
  Tensor* m = bc->in[0];
  if (m->st || !m->prod || m->prod->kind != K_SELECT || m->dt != kF32) return false;
  if (m->shape.rank != 2 || m->shape.d[0] != Sq || m->shape.d[1] != Sk) return false;
  Node* sel = m->prod;
  float vt, vf;
  if (!const_bcast(sel->in[1], &vt) || !const_bcast(sel->in[2], &vf)) return false;
  Tensor* pr = sel->in[0];
  if (pr->st || !pr->prod || pr->prod->kind != K_COMPARE) return false;
  Node* cm = pr->prod;
  Tensor *x = cm->in[0], *y = cm->in[1];
  auto iota_dim = [](Tensor* t) -> int {
    if (t->st || !t->prod || t->prod->kind != K_IOTA || t->dt != kI32) return -1;
    return (int)t->prod->i0;
  };
  const int dx = iota_dim(x), dy = iota_dim(y);
  int dir = cm->cmp;
  if (dx == 0 && dy == 1) {
    // cmp(i, j)
  } else if (dx == 1 && dy == 0) {
    // cmp(j, i): flip the direction
    static const int flip[] = {CMP_EQ, CMP_NE, CMP_GT, CMP_GE, CMP_LT, CMP_LE};
    dir = flip[dir];
  } else {
    return false;
  }
  fp->mask = true;
  fp->cmp = dir;
  fp->mask_true = vt;
  fp->mask_false = vf;
  return true;
}

bool Lower::match_flash(Node* pv) {
  if (pv->kind != K_DOT_GENERAL || pv->out[0]->dt != kBF16) return false;
  Tensor *attnB = pv->in[0], *v = pv->in[1];
  if (attnB->shape.rank != 4 || v->shape.rank != 4 || v->dt != kBF16) return false;
  if (!dims_are(pv->l0, {0, 1}) || !dims_are(pv->l1, {0, 1}) || !dims_are(pv->l2, {3}) ||
      !dims_are(pv->l3, {2}))
    return false;
  // attnB = astype(attn, bf16); attn = e / bcast(reduceSum(e, [3]))
  Node* cv = chain_node(attnB, K_CONVERT, 1);
  if (!cv || cv->in[0]->dt != kF32) return false;
  Tensor* attn = cv->in[0];
  Node* dv = chain_node(attn, K_BINARY, 1);
  if (!dv || dv->sub != 3 /* divide */) return false;
  Tensor *e = dv->in[0], *sumB = dv->in[1];
  Node* sb = chain_node(sumB, K_BROADCAST_TO, 1);
  if (!sb || !dims_are(sb->l1, {0, 1, 2})) return false;
  Tensor* sumE = sb->in[0];
  Node* rs = chain_node(sumE, K_REDUCE, 1);
  if (!rs || rs->sub != RED_SUM || !dims_are(rs->l0, {3}) || rs->in[0] != e) return false;
  // e = exp(s3 - bcast(reduceMax(s3, [3])))
  Node* ex = chain_node(e, K_UNARY, 2);
  if (!ex || ex->sub != 2 /* exp */) return false;
  Tensor* shifted = ex->in[0];
  Node* sub = chain_node(shifted, K_BINARY, 1);
  if (!sub || sub->sub != 1 /* sub */) return false;
  Tensor *s3 = sub->in[0], *maxB = sub->in[1];
  Node* mb = chain_node(maxB, K_BROADCAST_TO, 1);
  if (!mb || !dims_are(mb->l1, {0, 1, 2})) return false;
  Tensor* maxV = mb->in[0];
  Node* rm = chain_node(maxV, K_REDUCE, 1);
  if (!rm || rm->sub != RED_MAX || !dims_are(rm->l0, {3}) || rm->in[0] != s3) return false;
  if (!s3 || s3->st || !s3->prod || s3->ext != 0 || s3->uses != 2 || s3->dt != kF32)
    return false;
  const int64_t Sq = s3->shape.d[2], Sk = s3->shape.d[3];
  FlashPlan fp;
  std::vector<Tensor*> inner = {attnB, attn, sumB, sumE, e, shifted, maxB, maxV, s3};
  // optional mask: s = s2 + maskB
  Tensor* cur = s3;
  int cur_uses = 2;
  if (cur->prod->kind == K_BINARY && cur->prod->sub == 0 /* add */) {
    Node* ad = cur->prod;
    if (match_mask(ad->in[1], Sq, Sk, &fp)) cur = ad->in[0];
    else if (match_mask(ad->in[0], Sq, Sk, &fp)) cur = ad->in[1];
    else return false;
    cur_uses = 1;
    if (cur->st || !cur->prod || cur->ext != 0 || cur->uses != 1) return false;
    inner.push_back(cur);
  }
  // optional scale: s2 = s32 * bcast(scale)
  if (cur->prod->kind == K_BINARY && cur->prod->sub == 2 /* mul */) {
    Node* mu = cur->prod;
    float sc;
    if (const_bcast(mu->in[1], &sc)) cur = mu->in[0];
    else if (const_bcast(mu->in[0], &sc)) cur = mu->in[1];
    else return false;
    fp.scale = sc;
    if (cur->st || !cur->prod || cur->ext != 0 || cur->uses != 1) return false;
    inner.push_back(cur);
  }
  (void)cur_uses;
  // s32 = astype(scores, f32); scores = dot_general(q, k) over d
  Node* c32 = chain_node(cur, K_CONVERT, 1);
  if (!c32 || c32->in[0]->dt != kBF16) return false;
  Tensor* scores = c32->in[0];
  Node* qk = chain_node(scores, K_DOT_GENERAL, 1);
  if (!qk || !dims_are(qk->l0, {0, 1}) || !dims_are(qk->l1, {0, 1}) ||
      !dims_are(qk->l2, {3}) || !dims_are(qk->l3, {3}))
    return false;
  Tensor *q = qk->in[0], *k = qk->in[1];
  if (q->dt != kBF16 || k->dt != kBF16 || q->shape.rank != 4 || k->shape.rank != 4)
    return false;
  const int64_t D = q->shape.d[3];
  if (D != 32 && D != 64 && D != 128) return false;
  if (v->shape.d[2] != Sk || v->shape.d[3] != D) return false;
  inner.push_back(scores);
  fp.q = q;
  fp.k = k;
  fp.v = v;
  for (Tensor* t : inner) t->plan_mat = false;
  flash[pv] = fp;
  return true;
}

// K / V operand of the fused attention: rew's GQA head expansion
// (src/rew/nn/groupedqueryattention.nim:126-133)
//   reshape(broadcastTo(reshape(x, [B,Hkv,1,S,D]), [B,Hkv,G,S,D]), [B,H,S,D])
// is read as x with kv head h / G; any other operand is read through its
// view strides with Hkv = H.
bool Lower::kv_operand(Tensor* t, int H, const void** ptr, int64_t* sb, int64_t* sh,
                       int64_t* ss, int* hkv) {
  Tensor* x = t;
  int nkv = H;
  if (!t->st && t->prod && !t->plan_mat && t->prod->kind == K_RESHAPE) {
    Tensor* u = t->prod->in[0];
    if (u->shape.rank == 5 && !u->st && u->prod && !u->plan_mat &&
        u->prod->kind == K_BROADCAST_TO && dims_are(u->prod->l1, {0, 1, 2, 3, 4})) {
      Tensor* w = u->prod->in[0];
      if (w->shape.rank == 5 && w->shape.d[2] == 1 && !w->st && w->prod && !w->plan_mat &&
          w->prod->kind == K_RESHAPE) {
        Tensor* y = w->prod->in[0];
        if (y->shape.rank == 4 && y->shape.d[1] == u->shape.d[1] &&
            u->shape.d[1] * u->shape.d[2] == H && y->shape.d[2] == t->shape.d[2] &&
            y->shape.d[3] == t->shape.d[3]) {
          x = y;
          nkv = (int)y->shape.d[1];
        }
      }
    }
  }
  Tensor* base;
  int64_t off, st[kMaxRank];
  operand_strides(x, &base, &off, st);
  if (st[3] != 1) {
    // not d-contiguous: dense copy
    Tensor* cp = emit_permuted_copy(x, {0, 1, 2, 3});
    base = cp;
    off = 0;
    dense_strides(cp->shape, st);
  }
  *ptr = (const char*)base->data() + off * dt_size(base->dt);
  *sb = x->shape.d[0] == 1 ? 0 : st[0];
  *sh = x->shape.d[1] == 1 ? 0 : st[1];
  *ss = st[2];
  *hkv = nkv;
  return true;
}

// REW_MI355X_DEBUG_PLAN=1: the pattern matchers report their decisions on
// stderr (diagnostics only).
static bool debug_plan() {
  static const bool on = [] {
    const char* s = std::getenv("REW_MI355X_DEBUG_PLAN");
    return s && s[0] == '1';
  }();
  return on;
}

void Lower::match_flash_out() {
  for (auto& kv : flash) {
    Node* pv = kv.first;
    Tensor* o = pv->out[0];
    auto it = cons.find(o);
    const size_t nc = it == cons.end() ? 0 : it->second.size();
    if (debug_plan())
      std::fprintf(stderr, "[plan] flash out: ext=%d uses=%d consumers=%zu first=%s\n", o->ext,
                   o->uses, nc, nc ? it->second[0]->name.c_str() : "-");
    if (o->ext != 0 || o->uses != 1 || nc != 1) continue;
    Node* tr = it->second[0];
    if (tr->kind != K_TRANSPOSE || !dims_are(tr->l0, {0, 2, 1, 3})) continue;
    Tensor* t = tr->out[0];
    o->plan_mat = false;
    t->plan_mat = true;
    kv.second.out_t = t;
    flash_out[t] = pv;
  }
}

bool Lower::emit_flash(Node* pv, const FlashPlan& fp) {
  Tensor* out = pv->out[0];
  FlashArgs a;
  std::memset(&a, 0, sizeof(a));
  const Shape& Q = fp.q->shape;
  a.B = (int)Q.d[0];
  a.H = (int)Q.d[1];
  a.Sq = (int)Q.d[2];
  a.D = (int)Q.d[3];
  a.Sk = (int)fp.k->shape.d[2];
  {
    Tensor* base;
    int64_t off, st[kMaxRank];
    Tensor* q = fp.q;
    operand_strides(q, &base, &off, st);
    if (st[3] != 1) {
      base = emit_permuted_copy(q, {0, 1, 2, 3});
      off = 0;
      dense_strides(base->shape, st);
    }
    a.q = (const char*)base->data() + off * dt_size(base->dt);
    a.q_sb = Q.d[0] == 1 ? 0 : st[0];
    a.q_sh = Q.d[1] == 1 ? 0 : st[1];
    a.q_ss = st[2];
  }
  int hk_k, hk_v;
  kv_operand(fp.k, a.H, &a.k, &a.k_sb, &a.k_sh, &a.k_ss, &hk_k);
  kv_operand(fp.v, a.H, &a.v, &a.v_sb, &a.v_sh, &a.v_ss, &hk_v);
  if (hk_k != hk_v) {
    // mixed head mappings: read the expanded K and V directly
    kv_operand(fp.k, -1, &a.k, &a.k_sb, &a.k_sh, &a.k_ss, &hk_k);
    kv_operand(fp.v, -1, &a.v, &a.v_sb, &a.v_sh, &a.v_ss, &hk_v);
    hk_k = hk_v = a.H;
  }
  a.Hkv = hk_k;
  if (fp.out_t) {
    // [B, Sq, H, D] dense: the consumer's transposed layout
    out = fp.out_t;
    a.o_sb = (int64_t)a.Sq * a.H * a.D;
    a.o_sh = a.D;
    a.o_ss = (int64_t)a.H * a.D;
  } else {
    a.o_sb = (int64_t)a.H * a.Sq * a.D;
    a.o_sh = (int64_t)a.Sq * a.D;
    a.o_ss = a.D;
  }
  tensor_alloc(out);
  a.o = out->data();
  a.scale = fp.scale;
  a.round_scores = fp.round_scores ? 1 : 0;
  a.mask = fp.mask ? 1 : 0;
  a.cmp = fp.cmp;
  a.mask_true = fp.mask_true;
  a.mask_false = fp.mask_false;
  // Skipping key tiles that are masked everywhere is exact when the masked
  // value underflows exp() against every visible score and every query row
  // keeps at least one visible key.
  bool rows_ok = false;
  switch (a.cmp) {
    case CMP_LE: rows_ok = a.Sq <= a.Sk; break;
    case CMP_LT: rows_ok = a.Sq <= a.Sk - 1; break;
    case CMP_GE: rows_ok = true; break;
    default: rows_ok = false; break;
  }
  a.skip = (a.mask && rows_ok && a.mask_false - a.mask_true <= -1e8f) ? 1 : 0;
  a.heavy_last = (a.mask && (a.cmp == CMP_GE || a.cmp == CMP_GT)) ? 1 : 0;
  if (!flash_supported(a)) {
    tensor_drop_storage(out);
    return false;
  }
  Launch L{a};
  if (c->profiling) {
    char nm[160];
    std::snprintf(nm, sizeof nm, "%s[%d,%d,%d,%d,%d,%d,%d,%d]",
                  flash_variant(a), a.B, a.H, a.Hkv, a.Sq,
                  a.Sk, a.D, a.mask ? a.cmp : -1, a.skip);
    L.name = nm;
  }
  L.fused = true;
  run_launch(c, std::move(L));
  return true;
}


// ---------------------------------------------------------------------------
// GEMM epilogue fusion: rew's Linear bias add (src/rew/nn/linear.nim:43-49),
// the decoder's residual adds (src/rew/models/llama.nim:106-117) and
// GatedFeedForward's SiLU gate (src/rew/nn/gated_ffn.nim:46-67,
// src/rew/nn/activation.nim:28-38) run inside the GEMM that feeds them.
// ---------------------------------------------------------------------------

static Node* sole_consumer(Lower& L, Tensor* t) {
  if (!t || t->st || t->ext != 0 || t->uses != 1) return nullptr;
  auto it = L.cons.find(t);
  if (it == L.cons.end() || it->second.size() != 1) return nullptr;
  return it->second[0];
}

// broadcastTo(bias[N], [M, N], [1]) of a same-dtype vector
static bool bias_of(Tensor* t, const Shape& ys, Tensor** bias) {
  if (!t || t->st || !t->prod || t->prod->kind != K_BROADCAST_TO) return false;
  Node* bc = t->prod;
  Tensor* v = bc->in[0];
  if (t->shape != ys || ys.rank != 2 || !dims_are(bc->l1, {1})) return false;
  if (v->shape.rank != 1 || v->shape.d[0] != ys.d[1] || v->dt != t->dt) return false;
  *bias = v;
  return true;
}

// y = add(D, bias) / add(bias, D) for the pending matmul output D
static Node* bias_add(Lower& L, Tensor* D, Tensor** bias) {
  Node* ad = sole_consumer(L, D);
  if (!ad || ad->kind != K_BINARY || ad->sub != 0) return nullptr;
  Tensor* other = ad->in[0] == D ? ad->in[1] : ad->in[0];
  if (!bias_of(other, D->shape, bias)) return nullptr;
  return ad;
}

static bool plain_matmul(Node* n) {
  return n && n->kind == K_DOT_GENERAL && n->l0.empty() && n->l1.empty() &&
         n->in[0]->shape.rank == 2 && n->in[1]->shape.rank == 2 && dims_are(n->l2, {1}) &&
         dims_are(n->l3, {0}) && (n->out[0]->dt == kBF16 || n->out[0]->dt == kF32);
}

static bool is_one(Tensor* t) {
  float v;
  return const_bcast(t, &v) && v == 1.0f;
}

void Lower::match_gemm_epilogues() {
  // 1. SwiGLU: hb = astype(mul(silu(astype(yg)), astype(yu)), bf16)
  for (Node* cv : nodes) {
    if (cv->kind != K_CONVERT || cv->out[0]->dt != kBF16 || cv->in[0]->dt != kF32) continue;
    Tensor* hb = cv->out[0];
    Node* mu = chain_node(cv->in[0], K_BINARY, 1);
    if (!mu || mu->sub != 2) continue;
    for (int ord = 0; ord < 2; ++ord) {
      Tensor* act = mu->in[ord];
      Tensor* u32 = mu->in[1 - ord];
      Node* am = chain_node(act, K_BINARY, 1);
      if (!am || am->sub != 2) continue;
      Tensor *g32 = nullptr, *sig = nullptr;
      for (int o2 = 0; o2 < 2 && !g32; ++o2) {
        Node* dv = chain_node(am->in[1 - o2], K_BINARY, 1);
        if (dv && dv->sub == 3 && is_one(dv->in[0])) {
          g32 = am->in[o2];
          sig = am->in[1 - o2];
        }
      }
      if (!g32) continue;
      Node* dv = sig->prod;
      Tensor* den = dv->in[1];
      Node* da = chain_node(den, K_BINARY, 1);
      if (!da || da->sub != 0) continue;
      Tensor* ex = is_one(da->in[0]) ? da->in[1] : (is_one(da->in[1]) ? da->in[0] : nullptr);
      Node* en = chain_node(ex, K_UNARY, 1);
      if (!en || en->sub != 2) continue;
      Node* ng = chain_node(en->in[0], K_UNARY, 1);
      if (!ng || ng->sub != 0 || ng->in[0] != g32) continue;
      Node* gc = chain_node(g32, K_CONVERT, 2);
      Node* uc = chain_node(u32, K_CONVERT, 1);
      if (!gc || !uc || gc->in[0]->dt != kBF16 || uc->in[0]->dt != kBF16) continue;
      Tensor *yg = gc->in[0], *yu = uc->in[0];
      Node* ga = chain_node(yg, K_BINARY, 1);
      Node* ua = chain_node(yu, K_BINARY, 1);
      if (!ga || !ua || ga->sub != 0 || ua->sub != 0) continue;
      auto split = [](Node* ad, Tensor** D, Tensor** bias) {
        for (int o = 0; o < 2; ++o) {
          Tensor* d = ad->in[o];
          if (d->prod && !d->st && d->ext == 0 && d->uses == 1 && plain_matmul(d->prod) &&
              bias_of(ad->in[1 - o], d->shape, bias)) {
            *D = d;
            return true;
          }
        }
        return false;
      };
      Tensor *Dg, *Du, *bg, *bu;
      if (!split(ga, &Dg, &bg) || !split(ua, &Du, &bu)) continue;
      Node *ng_ = Dg->prod, *nu = Du->prod;
      if (ng_->in[0] != nu->in[0] || ng_->in[1]->shape != nu->in[1]->shape ||
          Dg->dt != kBF16 || !Dg->plan_mat || !Du->plan_mat)
        continue;
      GemmPlan gp;
      gp.dot = ng_;
      gp.dot2 = nu;
      gp.epi = EPI_SWIGLU;
      gp.bias = bg;
      gp.bias2 = bu;
      for (Tensor* t : {Dg, Du, yg, yu, g32, u32, ng->out[0], ex, den, sig, act, cv->in[0]})
        t->plan_mat = false;
      hb->plan_mat = true;
      gemm_out[hb] = gp;
      break;
    }
  }
  // 2. bias (+ residual) epilogues of the remaining matmuls
  std::unordered_map<const Node*, size_t> order;
  for (size_t i = 0; i < nodes.size(); ++i) order.emplace(nodes[i], i);
  // y = add(matmul D', bias) of a later matmul D': the sum add(.., y) is
  // left to D''s epilogue, which reads this GEMM's output as its residual
  // (DeepSeekMoE's shared experts, out = E_0(x) + E_1(x))
  auto later_biased_matmul = [&](Tensor* y, size_t here) -> bool {
    if (!y || y->st || !y->prod || y->prod->kind != K_BINARY || y->prod->sub != 0) return false;
    for (Tensor* d : y->prod->in) {
      Tensor* bias;
      if (d->prod && !d->st && d->ext == 0 && d->uses == 1 && plain_matmul(d->prod) &&
          bias_of(y->prod->in[0] == d ? y->prod->in[1] : y->prod->in[0], d->shape, &bias)) {
        auto it = order.find(d->prod);
        return it != order.end() && it->second > here;
      }
    }
    return false;
  };
  for (Node* n : nodes) {
    if (!plain_matmul(n)) continue;
    Tensor* D = n->out[0];
    if (!D->plan_mat || D->ext != 0) continue;  // claimed, or held by the caller
    Tensor* bias;
    Node* ad = bias_add(*this, D, &bias);
    if (!ad) continue;
    Tensor* y = ad->out[0];
    GemmPlan gp;
    gp.dot = n;
    gp.epi = EPI_BIAS;
    gp.bias = bias;
    Tensor* out = y;
    std::vector<Tensor*> inner = {D};
    // residual: add(R, y), add(y, R), or through one reshape of y
    Tensor* r = y;
    Node* c1 = sole_consumer(*this, y);
    if (c1 && c1->kind == K_RESHAPE && c1->out[0]->ext == 0) {
      r = c1->out[0];
      c1 = sole_consumer(*this, r);
    }
    if (c1 && c1->kind == K_BINARY && c1->sub == 0 && c1->in[0] != c1->in[1]) {
      Tensor* R = c1->in[0] == r ? c1->in[1] : c1->in[0];
      if (R->dt == D->dt && R->shape == r->shape && R->shape.numel() == D->numel() &&
          !later_biased_matmul(R, order[n])) {
        gp.epi = EPI_BIAS_RES;
        gp.res = R;
        inner.push_back(y);
        if (r != y) inner.push_back(r);
        out = c1->out[0];
      }
    }
    // rew's relu (maximum with a broadcast zero constant) after an f32 bias add
    if (gp.epi == EPI_BIAS && D->dt == kF32) {
      Node* c2 = sole_consumer(*this, y);
      float v;
      if (c2 && c2->kind == K_BINARY && c2->sub == 4 && c2->in[0] != c2->in[1] &&
          c2->out[0]->shape == y->shape) {
        const int yi = c2->in[0] == y ? 0 : 1;
        if (const_bcast(c2->in[1 - yi], &v)) {
          gp.epi = EPI_BIAS_RELU;
          gp.relu_c = v;
          gp.relu_first = yi == 0;
          inner.push_back(y);
          out = c2->out[0];
        }
      }
    }
    for (Tensor* t : inner) t->plan_mat = false;
    out->plan_mat = true;
    gemm_out[out] = gp;
  }
}

// Kernel arguments of a planned GEMM (all but the output pointer).
bool Lower::gemm_fused_args(Tensor* t, const GemmPlan& p, GemmArgs& g) {
  Tensor *ta, *tb;
  dot_args(p.dot, g, ta, tb);
  if (g.batch != 1 || g.K == 0 || t->numel() != g.M * g.N || t->dt != g.c_dtype) return false;
  auto vec = [&](Tensor* v) -> const void* {
    ensure_mat(v);
    return (v->shape.rank == 1 && v->numel() == g.N) ? v->data() : nullptr;
  };
  g.epi = p.epi;
  g.bias = vec(p.bias);
  if (!g.bias) return false;
  g.relu_c = p.relu_c;
  g.relu_first = p.relu_first ? 1 : 0;
  if (p.epi == EPI_SWIGLU) {
    GemmArgs g2;
    Tensor *ta2, *tb2;
    dot_args(p.dot2, g2, ta2, tb2);
    if (g2.a != g.a || g2.a_sm != g.a_sm || g2.a_sk != g.a_sk || g2.K != g.K || g2.N != g.N ||
        g2.b_sk != g.b_sk || g2.b_sn != g.b_sn)
      return false;
    g.b2 = g2.b;
    g.bias2 = vec(p.bias2);
    if (!g.bias2) return false;
  }
  if (p.epi == EPI_BIAS_RES) {
    Tensor* base;
    int64_t off, st[kMaxRank], ds[kMaxRank];
    operand_strides(p.res, &base, &off, st);
    dense_strides(p.res->shape, ds);
    bool dense = true;
    for (int i = 0; i < p.res->shape.rank; ++i)
      if (p.res->shape.d[i] != 1 && st[i] != ds[i]) dense = false;
    if (!dense) {
      std::vector<int> id(p.res->shape.rank);
      for (int i = 0; i < p.res->shape.rank; ++i) id[i] = i;
      base = emit_permuted_copy(p.res, id);
      off = 0;
    }
    g.res = (const char*)base->data() + off * dt_size(base->dt);
    g.res_sm = g.N;
    g.res_sb = 0;
  }
  if (p.epi == EPI_BIAS_ROPE) {
    const int64_t B = p.rope_B, S = p.rope_S, H = p.rope_H, D = p.rope_D;
    if (g.M != B * S || g.N != H * D) return false;
    int64_t sc[4], sn[4];
    const void *pc, *ps;
    view4(p.rope_cos, 4, &pc, sc);
    view4(p.rope_sin, 4, &ps, sn);
    for (int i = 0; i < 4; ++i)
      if (sc[i] != sn[i]) return false;
    g.rope_cos = (const float*)pc;
    g.rope_sin = (const float*)ps;
    g.rope_S = S;
    g.rope_D = D;
    g.rope_tb = sc[0];
    g.rope_ti = sc[3];
    if (p.rope_t) {  // [B, H, S, D]
      g.rope_th = sc[1];
      g.rope_ts = sc[2];
      g.out_b = H * S * D;
      g.out_h = S * D;
      g.out_s = D;
    } else {  // [B, S, H, D]
      g.rope_ts = sc[1];
      g.rope_th = sc[2];
      g.out_b = S * H * D;
      g.out_s = H * D;
      g.out_h = D;
    }
  }
  g.c_sb = g.M * g.N;
  g.c_sm = g.N;
  return true;
}

static const char* epi_suffix(int epi) {
  switch (epi) {
    case EPI_BIAS: return "+bias";
    case EPI_BIAS_RES: return "+bias+res";
    case EPI_BIAS_ROPE: return "+bias+rope";
    case EPI_BIAS_RELU: return "+bias+relu";
    default: return "";
  }
}

bool Lower::emit_gemm_fused(Tensor* t, const GemmPlan& p) {
  if (p.group >= 0) {
    // the planned siblings (q / k / v of one input, or the SwiGLU pairs of
    // DeepSeekMoE's shared experts) in one launch
    std::vector<Tensor*> outs = {t};
    std::vector<GemmPlan> plans = {p};
    for (Tensor* u : gemm_groups[p.group]) {
      auto it = gemm_out.find(u);
      if (u == t || it == gemm_out.end() || u->st) continue;
      outs.push_back(u);
      plans.push_back(it->second);
    }
    std::vector<GemmArgs> args(outs.size());
    bool ok = outs.size() >= 2 && outs.size() <= (size_t)kMaxSegs;
    for (size_t i = 0; ok && i < outs.size(); ++i)
      ok = gemm_fused_args(outs[i], plans[i], args[i]);
    if (ok) ok = gemm_multi_ok(args.data(), (int)args.size());
    if (ok) {
      int64_t n_all = 0;
      std::string parts;
      for (size_t i = 0; i < outs.size(); ++i) {
        tensor_alloc(outs[i]);
        args[i].c = outs[i]->data();
        n_all += args[i].N;
        parts += std::string(i ? "," : "") + std::to_string(args[i].N) + epi_suffix(args[i].epi);
        if (i) gemm_out.erase(outs[i]);
      }
      Launch L{GemmL{args, true}};
      if (c->profiling) {
        char nm[200];
        std::snprintf(nm, sizeof nm, "%s{%s}[1,%lld,%lld,%lld]",
                      p.epi == EPI_SWIGLU ? "gemm_lds_swiglu" : "gemm_lds_nn", parts.c_str(),
                      (long long)args[0].M, (long long)n_all, (long long)args[0].K);
        L.name = nm;
      }
      L.fused = true;
      run_launch(c, std::move(L));
      return true;
    }
    // otherwise each member is launched on its own
  }
  GemmArgs g;
  if (!gemm_fused_args(t, p, g)) return false;
  if (p.epi == EPI_BIAS_ROPE) {
    if (!gemm_multi_ok(&g, 1)) return false;
  } else if (!gemm_epilogue_ok(g)) {
    return false;
  }
  tensor_alloc(t);
  g.c = t->data();
  Launch L{GemmL{{g}, p.epi == EPI_BIAS_ROPE}};
  if (c->profiling) {
    char nm[160];
    std::snprintf(nm, sizeof nm, "%s%s[%lld,%lld,%lld,%lld]",
                  p.epi == EPI_BIAS_ROPE ? "gemm_lds_nn" : gemm_variant(g), epi_suffix(p.epi),
                  (long long)g.batch, (long long)g.M, (long long)g.N, (long long)g.K);
    L.name = nm;
  }
  L.fused = true;
  run_launch(c, std::move(L));
  return true;
}

// Projections of one input that are all planned as fused GEMMs (the q, k and
// v projections of GroupedQueryAttention.forward, groupedqueryattention.nim)
// become one multi-segment launch.
void Lower::match_gemm_groups() {
  // key: the input seen through reshapes (q, k and v each reshape the same
  // normed tensor), and whether the plan is a SwiGLU pair (DeepSeekMoE's
  // shared experts all read x; the dual kernel takes only SwiGLU segments)
  using Key = std::pair<Tensor*, bool>;
  std::map<Key, std::vector<Tensor*>> by_a;
  std::vector<Key> order;
  for (Node* n : nodes)
    for (Tensor* t : n->out) {
      auto it = gemm_out.find(t);
      if (it == gemm_out.end()) continue;
      const GemmPlan& gp = it->second;
      const bool dual = gp.epi == EPI_SWIGLU;
      if (gp.epi != EPI_BIAS && gp.epi != EPI_BIAS_ROPE && gp.epi != EPI_BIAS_RES && !dual)
        continue;
      Tensor* a = gp.dot->in[0];
      while (a->prod && a->prod->kind == K_RESHAPE && !a->st) a = a->prod->in[0];
      if (gp.dot->in[0]->shape.rank != 2) continue;
      const Key key{a, dual};
      if (!by_a.count(key)) order.push_back(key);
      by_a[key].push_back(t);
    }
  for (const Key& a : order) {
    std::vector<Tensor*>& v = by_a[a];
    for (size_t i = 0; i + 1 < v.size(); i += kMaxSegs) {
      const size_t n = std::min(v.size() - i, (size_t)kMaxSegs);
      if (n < 2) break;
      const int id = (int)gemm_groups.size();
      gemm_groups.emplace_back(v.begin() + i, v.begin() + i + n);
      for (size_t j = i; j < i + n; ++j) gemm_out[v[j]].group = id;
    }
  }
}

// ---------------------------------------------------------------------------
// routed mixture of experts (src/rew/models/deepseek.nim:114-145)
// ---------------------------------------------------------------------------

// Expert id of broadcastTo(scalarI32(e), shape, []) (ops/literal.nim:191-194).
static bool const_i32_bcast(Tensor* t, int* val) {
  if (!t || t->st || !t->prod || t->prod->kind != K_BROADCAST_TO) return false;
  Tensor* s = t->prod->in[0];
  if (s->shape.rank != 0 || s->dt != kI32 || !s->has_host) return false;
  std::memcpy(val, s->host, 4);
  return true;
}

// w = reduceSum(mul(TW, astype(compare(TI, broadcastTo(e), EQ), f32)), [1])
// with TI the index output of a pending topK (distinct ids per row).
static bool routed_weight(Tensor* w, Tensor** tw, Tensor** ti, int* e,
                          std::vector<Tensor*>* inner) {
  Node* rs = chain_node(w, K_REDUCE, 1);
  if (!rs || rs->sub != RED_SUM || !dims_are(rs->l0, {1}) || w->dt != kF32) return false;
  Node* mu = chain_node(rs->in[0], K_BINARY, 1);
  if (!mu || mu->sub != 2) return false;
  for (int ord = 0; ord < 2; ++ord) {
    Tensor* TW = mu->in[ord];
    Node* cv = chain_node(mu->in[1 - ord], K_CONVERT, 1);
    if (!cv || cv->out[0]->dt != kF32 || cv->in[0]->dt != kBool) continue;
    Node* cp = chain_node(cv->in[0], K_COMPARE, 1);
    if (!cp || cp->cmp != 0 /* EQ */) continue;
    for (int o2 = 0; o2 < 2; ++o2) {
      Tensor* TI = cp->in[o2];
      if (!const_i32_bcast(cp->in[1 - o2], e)) continue;
      if (!TI->prod || TI->prod->kind != K_TOPK || TI->prod->out.size() != 2 ||
          TI->prod->out[1] != TI || TI->dt != kI32 || TI->shape.rank != 2)
        continue;
      if (TW->dt != kF32 || TW->shape != TI->shape) continue;
      *tw = TW;
      *ti = TI;
      for (Tensor* t : {w, rs->in[0], mu->in[1 - ord], cv->in[0], cp->in[1 - o2]})
        inner->push_back(t);
      return true;
    }
  }
  return false;
}

// c = astype(mul(astype(Y, f32), broadcastTo(reshape(w, [T, 1]), [T, H], [0, 1])), bf16)
// with Y the planned down projection of a planned SwiGLU of x.
bool match_contribution(Lower& L, Tensor* c, MoeMember* m, Tensor** x, Tensor** ti,
                        Tensor** tw, std::vector<Tensor*>* inner) {
  Node* cb = chain_node(c, K_CONVERT, 1);
  if (!cb || c->dt != kBF16 || cb->in[0]->dt != kF32 || c->shape.rank != 2) return false;
  Node* mu = chain_node(cb->in[0], K_BINARY, 1);
  if (!mu || mu->sub != 2) return false;
  const int64_t T = c->shape.d[0], H = c->shape.d[1];
  for (int ord = 0; ord < 2; ++ord) {
    Node* cy = chain_node(mu->in[ord], K_CONVERT, 1);
    if (!cy || cy->in[0]->dt != kBF16) continue;
    Tensor* Y = cy->in[0];
    auto dit = L.gemm_out.find(Y);
    if (dit == L.gemm_out.end() || dit->second.epi != EPI_BIAS || Y->ext != 0 || Y->uses != 1)
      continue;
    Tensor* hb = dit->second.dot->in[0];
    auto sit = L.gemm_out.find(hb);
    if (sit == L.gemm_out.end() || sit->second.epi != EPI_SWIGLU || hb->ext != 0 ||
        hb->uses != 1)
      continue;
    Node* bw = chain_node(mu->in[1 - ord], K_BROADCAST_TO, 1);
    if (!bw || !dims_are(bw->l1, {0, 1})) continue;
    Node* rw = chain_node(bw->in[0], K_RESHAPE, 1);
    if (!rw || rw->out[0]->shape.rank != 2 || rw->out[0]->shape.d[0] != T ||
        rw->out[0]->shape.d[1] != 1)
      continue;
    std::vector<Tensor*> in2;
    int e;
    if (!routed_weight(rw->in[0], tw, ti, &e, &in2)) continue;
    Tensor* X = sit->second.dot->in[0];
    if (X->dt != kBF16 || X->shape.rank != 2 || X->shape.d[0] != T || X->shape.d[1] != H ||
        (*ti)->shape.d[0] != T || (*ti)->shape.d[1] > kMoeMaxK)
      continue;
    m->e = e;
    m->sw = sit->second;
    m->dn = dit->second;
    *x = X;
    for (Tensor* t : {c, cb->in[0], mu->in[ord], Y, hb, mu->in[1 - ord], bw->in[0]})
      inner->push_back(t);
    inner->insert(inner->end(), in2.begin(), in2.end());
    return true;
  }
  return false;
}

void Lower::match_moe() {
  // running-sum tensor -> the group whose chain currently ends in it
  std::unordered_map<Tensor*, MoePlan> open;
  for (Node* ad : nodes) {
    if (ad->kind != K_BINARY || ad->sub != 0 || ad->out[0]->dt != kBF16) continue;
    Tensor* out = ad->out[0];
    for (int ord = 0; ord < 2; ++ord) {
      Tensor *prev = ad->in[ord], *c = ad->in[1 - ord];
      if (prev == c) continue;
      MoeMember m;
      Tensor *x, *ti, *tw;
      std::vector<Tensor*> inner;
      if (!match_contribution(*this, c, &m, &x, &ti, &tw, &inner)) continue;
      const Tensor* router = ti->prod->in[0];
      if (m.e < 0 || m.e >= router->shape.d[router->shape.rank - 1]) continue;
      MoePlan g;
      auto it = open.find(prev);
      bool extend = it != open.end() && prev->ext == 0 && prev->uses == 1 &&
                    it->second.x == x && it->second.topi == ti && it->second.topw == tw;
      if (extend)
        for (const MoeMember& q : it->second.mem)
          if (q.e == m.e) extend = false;
      if (extend) {
        g = std::move(it->second);
        open.erase(it);
        g.mids.push_back(prev);
      } else {
        g.start = prev;
        g.x = x;
        g.topi = ti;
        g.topw = tw;
        Tensor* src = ti->prod->in[0];
        g.E = (int)src->shape.d[src->shape.rank - 1];
      }
      g.mem.push_back(m);
      g.inner.insert(g.inner.end(), inner.begin(), inner.end());
      open[out] = std::move(g);
      break;
    }
  }
  // A group is claimed only when emit_moe cannot fail on it; otherwise its
  // ops keep their ordinary plans (fused SwiGLU / bias GEMMs, elementwise
  // combine), exactly as in op-by-op mode.
  for (auto& kv : open) {
    MoePlan& g = kv.second;
    if (!moe_lowerable(g)) {
      if (debug_plan())
        std::fprintf(stderr, "[plan] moe: group of %zu experts not lowerable, generic path\n",
                     g.mem.size());
      continue;
    }
    for (Tensor* t : g.inner) {
      t->plan_mat = false;
      gemm_out.erase(t);
    }
    for (Tensor* t : g.mids) t->plan_mat = false;
    if (match_shared(g, g.mids.empty() ? kv.first : g.mids.front())) {
      for (Tensor* t : g.shared_inner) {
        t->plan_mat = false;
        gemm_out.erase(t);
      }
    }
    kv.first->plan_mat = true;
    moe_out[kv.first] = std::move(g);
  }
}

static bool reads_dense(Tensor* w);

// DeepSeekMoE.forward's shared experts (deepseek.nim:123-126): out =
// S_0(x), then out = out + S_i(x), which the GEMM epilogues planned as
// start = down_{n-1}(SwiGLU_{n-1}(x)) + bias with the earlier sum as its
// residual, ..., down_0 with the bias alone.  Every SwiGLU reads the
// group's own x, and every link of the chain (start included) is read by
// the next one only, so the group can compute them itself.  With one
// shared expert the epilogue planning has already taken the first routed
// add (first_sum = start + the first member's contribution) into that
// expert's down GEMM as its residual; the group then takes that plan back
// with the bias epilogue alone.
bool Lower::match_shared(MoePlan& g, Tensor* first_sum) {
  std::vector<MoeMember> sh;
  std::vector<Tensor*> inner;
  const int64_t T = g.x->shape.d[0], H = g.x->shape.d[1];
  const int64_t I = g.mem[0].sw.dot->in[1]->shape.d[1];
  auto weight = [&](Tensor* w, int64_t rows, int64_t cols) {
    return w->dt == kBF16 && w->shape.rank == 2 && w->shape.d[0] == rows &&
           w->shape.d[1] == cols && reads_dense(w);
  };
  auto vec = [&](Tensor* v, int64_t len) { return v && v->dt == kBF16 && v->numel() == len; };
  Tensor* s = g.start;
  Tensor* taken = nullptr;  // the first routed add's plan, taken back
  for (;;) {
    if (s->ext != 0 || s->uses != 1 || s->dt != kBF16 || s->shape != g.x->shape) return false;
    GemmPlan dn;
    auto dit = gemm_out.find(s);
    if (dit != gemm_out.end()) {
      dn = dit->second;
    } else {
      auto fit = sh.empty() ? gemm_out.find(first_sum) : gemm_out.end();
      if (fit == gemm_out.end() || fit->second.epi != EPI_BIAS_RES || !fit->second.dot ||
          !s->prod || s->prod->kind != K_BINARY ||
          (s->prod->in[0] != fit->second.dot->out[0] && s->prod->in[1] != fit->second.dot->out[0]))
        return false;
      dn = fit->second;
      dn.epi = EPI_BIAS;
      dn.res = nullptr;
      taken = first_sum;
    }
    if ((dn.epi != EPI_BIAS && dn.epi != EPI_BIAS_RES) || !dn.dot) return false;
    Tensor* hb = dn.dot->in[0];
    auto sit = gemm_out.find(hb);
    if (sit == gemm_out.end() || sit->second.epi != EPI_SWIGLU || hb->ext != 0 || hb->uses != 1)
      return false;
    const GemmPlan& sw = sit->second;
    if (!sw.dot || !sw.dot2 || sw.dot->in[0] != g.x || sw.dot2->in[0] != g.x) return false;
    if (!weight(sw.dot->in[1], H, I) || !weight(sw.dot2->in[1], H, I) ||
        !weight(dn.dot->in[1], I, H) || !vec(sw.bias, I) || !vec(sw.bias2, I) ||
        !vec(dn.bias, H))
      return false;
    MoeMember m;
    m.e = -1;
    m.sw = sw;
    m.dn = dn;
    sh.insert(sh.begin(), m);
    inner.push_back(s);
    inner.push_back(hb);
    if (dn.epi == EPI_BIAS) break;
    s = dn.res;
    if (!s || (int64_t)sh.size() >= kMoeMaxMembers - (int64_t)g.mem.size()) return false;
  }
  // the down GEMMs run with their epilogues on dense rows (stand-in
  // addresses: the real ones are aligned allocator blocks)
  for (size_t i = 0; i < sh.size(); ++i) {
    GemmArgs d{};
    void* const al = reinterpret_cast<void*>(uintptr_t(4096));
    d.dtype = d.c_dtype = kBF16;
    d.batch = 1;
    d.a = d.b = d.bias = al;
    d.c = al;
    d.M = T;
    d.K = I;
    d.N = H;
    d.a_sm = I;
    d.a_sk = 1;
    d.b_sk = H;
    d.b_sn = 1;
    d.c_sm = H;
    d.c_sb = T * H;
    d.epi = i ? EPI_BIAS_RES : EPI_BIAS;
    if (i) {
      d.res = al;
      d.res_sm = H;
    }
    if (!gemm_epilogue_ok(d)) return false;
  }
  if (taken) gemm_out.erase(taken);  // the group's combine makes that sum
  g.shared = std::move(sh);
  g.shared_inner = std::move(inner);
  return true;
}

// Arguments of the two grouped expert GEMMs over dense [*, H] token rows
// and dense [*, I] hidden rows (operand pointers left null).
static void moe_gemm_args(int64_t T, int64_t H, int64_t I, int64_t R, GemmArgs* gs,
                          GemmArgs* gd) {
  *gs = GemmArgs{};
  *gd = GemmArgs{};
  for (GemmArgs* g : {gs, gd}) {
    g->dtype = kBF16;
    g->c_dtype = kBF16;
    g->batch = 1;
    g->a_sk = 1;
    g->b_sn = 1;
    g->a_sb = 0;
    g->c_sb = 0;
  }
  gs->M = T;
  gs->K = H;
  gs->N = I;
  gs->b_sk = I;
  gs->a_sm = H;
  gs->c_sm = I;
  gs->epi = EPI_SWIGLU;
  gd->M = R;
  gd->K = I;
  gd->N = H;
  gd->b_sk = H;
  gd->a_sm = I;
  gd->c_sm = H;
  gd->epi = EPI_BIAS;
}

// Whether operand_strides(w) reads w as dense row-major storage at offset 0:
// a materialized tensor, a pending non-view result (materialized densely
// when read), a view the planner materializes, or a reshape chain of these.
static bool reads_dense(Tensor* w) {
  while (!w->st && !w->plan_mat && w->prod && w->prod->kind == K_RESHAPE) w = w->prod->in[0];
  return w->st || w->plan_mat || !w->prod || !is_view(w->prod->kind);
}

// Every condition under which emit_moe would refuse the group, checked
// before the group's ops give up their own plans: expert weights dense
// row-major bf16 of the member shapes, bf16 bias vectors, and both grouped
// GEMMs launchable over dense 16-byte-aligned rows (emit_moe copies x and
// the running sum densely when their views are not).
bool Lower::moe_lowerable(const MoePlan& p) {
  if (p.mem.empty() || p.x->shape.rank != 2 || p.topi->shape.rank != 2) return false;
  if ((int64_t)p.mem.size() > kMoeMaxMembers) return false;
  const int64_t T = p.x->shape.d[0], H = p.x->shape.d[1];
  const int64_t k = p.topi->shape.d[1];
  if (k < 1 || k > kMoeMaxK || H % 8 || p.start->dt != kBF16 || p.start->numel() != T * H)
    return false;
  const int64_t I = p.mem[0].sw.dot->in[1]->shape.d[1];
  auto weight = [&](Tensor* w, int64_t rows, int64_t cols) {
    return w->dt == kBF16 && w->shape.rank == 2 && w->shape.d[0] == rows &&
           w->shape.d[1] == cols && reads_dense(w);
  };
  auto vec = [&](Tensor* v, int64_t len) { return v && v->dt == kBF16 && v->numel() == len; };
  for (const MoeMember& m : p.mem) {
    if (!m.sw.dot || !m.sw.dot2 || !m.dn.dot) return false;
    if (!weight(m.sw.dot->in[1], H, I) || !weight(m.sw.dot2->in[1], H, I) ||
        !weight(m.dn.dot->in[1], I, H) || !vec(m.sw.bias, I) || !vec(m.sw.bias2, I) ||
        !vec(m.dn.bias, H))
      return false;
  }
  GemmArgs gs, gd;
  moe_gemm_args(T, H, I, T * k, &gs, &gd);
  // stand-in operand addresses: the real ones are allocator blocks (aligned)
  void* const al = reinterpret_cast<void*>(uintptr_t(4096));
  for (GemmArgs* g : {&gs, &gd}) {
    g->a = g->b = g->b2 = g->bias = g->bias2 = al;
    g->c = al;
  }
  return gemm_grouped_ok(gs) && gemm_grouped_ok(gd);
}

// rows_view, with a dense copy when the rows are not 16-byte aligned with
// a row stride of whole 16-byte chunks (the grouped GEMM and the combine
// read 16-byte vectors).
void Lower::dense_rows(Tensor* x, int64_t n, const void** ptr, int64_t* rs) {
  rows_view(x, n, ptr, rs);
  if (((uintptr_t)*ptr & 15) == 0 && *rs % 8 == 0) return;
  std::vector<int> id(x->shape.rank);
  for (int i = 0; i < x->shape.rank; ++i) id[i] = i;
  Tensor* d = emit_permuted_copy(x, id);
  *ptr = d->data();
  *rs = n;
}

bool Lower::emit_moe(Tensor* t, const MoePlan& p) {
  const int n = (int)p.mem.size(), ns = (int)p.shared.size();
  if (!ns) ensure_mat(p.start);  // (else the group computes it)
  ensure_mat(p.x);
  ensure_mat(p.topi);
  ensure_mat(p.topw);
  const int64_t T = p.x->shape.d[0], H = p.x->shape.d[1];
  const int k = (int)p.topi->shape.d[1];
  const void* xp;
  int64_t x_rs;
  dense_rows(p.x, H, &xp, &x_rs);
  const void* sp = nullptr;
  int64_t s_rs = 0;
  if (!ns) dense_rows(p.start, H, &sp, &s_rs);
  if (p.topi->st == nullptr || p.topw->st == nullptr) return false;

  // member weights: gate/up [H, I], down [I, H], dense row-major.  Only the
  // weights are inspected here: the members' A operands (x and the SwiGLU
  // outputs) are never materialized densely.
  auto weight = [&](Tensor* w, int64_t rows, int64_t cols) -> const void* {
    if (w->dt != kBF16 || w->shape.rank != 2 || w->shape.d[0] != rows || w->shape.d[1] != cols)
      return nullptr;
    Tensor* base;
    int64_t off, st[kMaxRank];
    operand_strides(w, &base, &off, st);
    if (st[1] != 1 || st[0] != cols) return nullptr;
    return (const char*)base->data() + off * 2;
  };
  auto vec = [&](Tensor* v, int64_t len) -> const void* {
    ensure_mat(v);
    if (v->dt != kBF16 || v->numel() != len || !v->st) return nullptr;
    return v->data();
  };
  const int64_t I = p.mem[0].sw.dot->in[1]->shape.d[1];
  // the members' six tables, then the shared experts' (table j of the
  // shared experts at 6 n + j ns)
  std::vector<const void*> ptrs(6 * (size_t)(n + ns));
  std::vector<int32_t> ids(n);
  for (int i = 0; i < n + ns; ++i) {
    const MoeMember& m = i < n ? p.mem[i] : p.shared[i - n];
    if (i < n) ids[i] = m.e;
    const void* q[6] = {weight(m.sw.dot->in[1], H, I), weight(m.sw.dot2->in[1], H, I),
                        vec(m.sw.bias, I), vec(m.sw.bias2, I),
                        weight(m.dn.dot->in[1], I, H), vec(m.dn.bias, H)};
    for (int j = 0; j < 6; ++j) {
      if (!q[j] || ((uintptr_t)q[j] & 15)) return false;
      if (i < n) ptrs[(size_t)j * n + i] = q[j];
      else ptrs[6 * (size_t)n + (size_t)j * ns + (i - n)] = q[j];
    }
  }
  RoutedFfn a;
  a.x = xp;
  a.x_rs = x_rs;
  a.start = sp;
  a.start_rs = s_rs;
  a.topi = (const int32_t*)p.topi->data();
  a.topw = (const float*)p.topw->data();
  a.T = T;
  a.H = H;
  a.I = I;
  a.k = k;
  a.E = p.E;
  a.n = n;
  a.expert = ids.data();
  for (int j = 0; j < 6; ++j) a.ptr[j] = ptrs.data() + (size_t)j * n;
  a.n_shared = ns;
  for (int j = 0; j < 6 && ns; ++j) a.sptr[j] = ptrs.data() + 6 * (size_t)n + (size_t)j * ns;
  tensor_alloc(t);
  a.out = t->data();
  try {
    routed_ffn_check(a);
  } catch (const Error&) {
    // moe_lowerable checked the GEMMs on dense rows: a wider row stride of
    // x is the one thing that can differ here
    if (x_rs == H) throw;
    Tensor* d = emit_permuted_copy(p.x, {0, 1});
    a.x = d->data();
    a.x_rs = H;
    routed_ffn_check(a);
  }
  Shape ws;
  ws.rank = 1;
  ws.d[0] = (int64_t)routed_ffn_scratch_bytes(a);
  Tensor* work = new_tensor(c, kU8, ws);
  work->plan_dead = true;
  tensor_alloc(work);
  MoeL m{a, ids, ptrs, work->data()};
  run_launch(c, Launch{std::move(m)});
  maybe_destroy(work);
  return true;
}

// ---------------------------------------------------------------------------
// row composites: rmsNorm and RoPE chains as single kernels
// ---------------------------------------------------------------------------

static std::vector<int64_t> iota_dims(int n) {
  std::vector<int64_t> v(n);
  for (int i = 0; i < n; ++i) v[i] = i;
  return v;
}

// Registers a matched norm chain: its source x (an astype from bf16 with
// `x_uses` uses, all inside the chain, is folded into the kernel's load),
// its result o (or o's astype to bf16, its only consumer), the chain's
// intermediates (never materialized) and, when x is an embedding lookup
// seen through reshapes, the gather form.  False: x is neither f32 nor such
// an astype.
bool Lower::plan_norm(NormPlan np, Tensor* x, int x_uses, Tensor* o,
                      std::vector<Tensor*>& inner) {
  np.src = x;
  if (!x->st && x->prod && x->prod->kind == K_CONVERT && x->ext == 0 && x->uses == x_uses &&
      x->prod->in[0]->dt == kBF16) {
    np.src = x->prod->in[0];
    inner.push_back(x);
  } else if (x->dt != kF32) {
    return false;
  }
  Tensor* out = o;
  Node* cv = sole_consumer(*this, o);
  if (cv && cv->kind == K_CONVERT && cv->out[0]->dt == kBF16) {
    inner.push_back(o);
    out = cv->out[0];
  }
  for (Tensor* t : inner) t->plan_mat = false;
  out->plan_mat = true;
  norm_out[out] = np;
  Tensor* s = np.src;
  while (s && !s->st && s->prod && s->prod->kind == K_RESHAPE) s = s->prod->in[0];
  if (s && s != np.src && !s->st && s->prod && s->prod->kind == K_INDEX_SELECT)
    gather_norm[s] = out;
  return true;
}

// rew's LayerNorm.forward over the last axis (normalizedShape of rank 1),
// ending in the add node `ao`:
//   mean = divide(reduceSum(x, [r-1]), bcast(n));  c = sub(x, bcast(mean, [0..r-2]))
//   var = divide(reduceSum(mul(c, c), [r-1]), bcast(n))
//   inv = rsqrt(add(var, bcast(eps)));  y = add(mul(bcast(gamma), mul(c, bcast(inv))),
//                                              bcast(beta))
// Each broadcast and intermediate must be used only inside the chain.
bool Lower::match_layernorm(Node* ao) {
  Tensor* o = ao->out[0];
  const int r = o->shape.rank;
  const int64_t n = o->shape.d[r - 1];
  // a [n] f32 vector broadcast along the last axis
  auto vec_bcast = [&](Tensor* t) -> Tensor* {
    if (!t || t->st || !t->prod || t->prod->kind != K_BROADCAST_TO || t->ext != 0 ||
        t->uses != 1 || !dims_are(t->prod->l1, {r - 1}))
      return nullptr;
    Tensor* v = t->prod->in[0];
    return v->shape.rank == 1 && v->shape.d[0] == n && v->dt == kF32 ? v : nullptr;
  };
  // divide(reduceSum(v, [r-1]), bcast(const)) -> v
  auto mean_of = [&](Tensor* t, float* dv, std::vector<Tensor*>& inner) -> Tensor* {
    Node* md = chain_node(t, K_BINARY, 1);
    if (!md || md->sub != 3 || !const_bcast(md->in[1], dv)) return nullptr;
    Node* rs = chain_node(md->in[0], K_REDUCE, 1);
    if (!rs || rs->sub != RED_SUM || !dims_are(rs->l0, {r - 1})) return nullptr;
    inner.push_back(md->in[0]);
    return rs->in[0];
  };
  for (int ord = 0; ord < 2; ++ord) {
    Tensor* beta = vec_bcast(ao->in[1 - ord]);
    Node* gm = chain_node(ao->in[ord], K_BINARY, 1);
    if (!beta || !gm || gm->sub != 2) continue;
    for (int og = 0; og < 2; ++og) {
      Tensor* gamma = vec_bcast(gm->in[og]);
      Node* nm = chain_node(gm->in[1 - og], K_BINARY, 1);
      if (!gamma || !nm || nm->sub != 2) continue;
      Tensor *cen = nm->in[0], *invB = nm->in[1];
      Node* ib = chain_node(invB, K_BROADCAST_TO, 1);
      if (!ib || ib->l1 != iota_dims(r - 1)) continue;
      Node* rq = chain_node(ib->in[0], K_UNARY, 1);
      if (!rq || rq->sub != 22) continue;  // rsqrt
      Node* ve = chain_node(rq->in[0], K_BINARY, 1);
      float eps, dv2, dv1;
      if (!ve || ve->sub != 0 || !const_bcast(ve->in[1], &eps)) continue;
      std::vector<Tensor*> inner = {ao->in[ord], ao->in[1 - ord], gm->in[og], gm->in[1 - og],
                                    invB, ib->in[0], rq->in[0], ve->in[0]};
      Tensor* sq = mean_of(ve->in[0], &dv2, inner);
      Node* sqn = sq ? chain_node(sq, K_BINARY, 1) : nullptr;
      if (!sqn || sqn->sub != 2 || sqn->in[0] != cen || sqn->in[1] != cen) continue;
      // c feeds c * c (twice) and the normalisation
      if (cen->st || !cen->prod || cen->prod->kind != K_BINARY || cen->prod->sub != 1 ||
          cen->ext != 0 || cen->uses != 3)
        continue;
      Tensor *x = cen->prod->in[0], *meanB = cen->prod->in[1];
      Node* mb = chain_node(meanB, K_BROADCAST_TO, 1);
      if (!mb || mb->l1 != iota_dims(r - 1)) continue;
      Tensor* xs = mean_of(mb->in[0], &dv1, inner);
      if (xs != x || x->shape != o->shape) continue;
      inner.insert(inner.end(), {sq, cen, meanB, mb->in[0]});
      NormPlan np;
      np.gamma = gamma;
      np.beta = beta;
      np.eps = eps;
      np.divisor = dv1;
      np.divisor2 = dv2;
      np.layer = true;
      // x feeds the mean's sum and c
      if (plan_norm(np, x, 2, o, inner)) return true;
    }
  }
  return false;
}

void Lower::match_rows() {
  for (Node* mo : nodes) {
    // ---- rmsNorm: mul(bcast(gamma), divide(x, bcast(sqrt(sum(x*x)/n + eps))))
    if (mo->kind == K_BINARY && mo->sub == 2 && mo->out[0]->dt == kF32 &&
        mo->out[0]->shape.rank >= 1 && !mo->out[0]->st) {
      Tensor* o = mo->out[0];
      const int r = o->shape.rank;
      const int64_t n = o->shape.d[r - 1];
      for (int ord = 0; ord < 2; ++ord) {
        Tensor *gB = mo->in[ord], *normed = mo->in[1 - ord];
        if (gB->st || !gB->prod || gB->prod->kind != K_BROADCAST_TO) continue;
        Tensor* gamma = gB->prod->in[0];
        if (!dims_are(gB->prod->l1, {r - 1}) || gamma->shape.rank != 1 ||
            gamma->shape.d[0] != n || gamma->dt != kF32)
          continue;
        Node* dvn = chain_node(normed, K_BINARY, 1);
        if (!dvn || dvn->sub != 3) continue;
        Tensor *x = dvn->in[0], *rmsB = dvn->in[1];
        Node* rb = chain_node(rmsB, K_BROADCAST_TO, 1);
        if (!rb || rb->l1 != iota_dims(r - 1)) continue;
        Node* sq_ = chain_node(rb->in[0], K_UNARY, 1);
        if (!sq_ || sq_->sub != 4) continue;  // sqrt
        Node* ad = chain_node(sq_->in[0], K_BINARY, 1);
        float eps, dv;
        if (!ad || ad->sub != 0 || !const_bcast(ad->in[1], &eps)) continue;
        Node* md = chain_node(ad->in[0], K_BINARY, 1);
        if (!md || md->sub != 3 || !const_bcast(md->in[1], &dv)) continue;
        Node* rs = chain_node(md->in[0], K_REDUCE, 1);
        if (!rs || rs->sub != RED_SUM || !dims_are(rs->l0, {r - 1})) continue;
        Node* sm = chain_node(rs->in[0], K_BINARY, 1);
        if (!sm || sm->sub != 2 || sm->in[0] != x || sm->in[1] != x) continue;
        NormPlan np;
        np.gamma = gamma;
        np.eps = eps;
        np.divisor = dv;
        std::vector<Tensor*> inner = {normed, rmsB, rb->in[0], sq_->in[0], ad->in[0],
                                      md->in[0], rs->in[0]};
        if (plan_norm(np, x, 3, o, inner)) break;
      }
    }
    // ---- LayerNorm: add(mul(bcast(gamma), mul(c, bcast(rsqrt(mean(c*c) + eps)))), bcast(beta)),
    // c = sub(x, bcast(mean(x))), mean(v) = divide(reduceSum(v), n) (norm.nim:41-84,
    // reduce.nim:132-150)
    if (mo->kind == K_BINARY && mo->sub == 0 && mo->out[0]->dt == kF32 &&
        mo->out[0]->shape.rank >= 2 && !mo->out[0]->st)
      match_layernorm(mo);
    // ---- softmax: divide(e, bcast(reduceSum(e))), e = exp(sub(x, bcast(reduceMax(x))))
    // (only where the probabilities are materialized anyway: inside a fused
    // attention they never are)
    if (mo->kind == K_BINARY && mo->sub == 3 && mo->out[0]->dt == kF32 && !mo->out[0]->st &&
        mo->out[0]->plan_mat && mo->out[0]->shape.rank >= 1) {
      Tensor* y = mo->out[0];
      const int r = y->shape.rank;
      Tensor *e = mo->in[0], *sB = mo->in[1];
      Node* en = (!e->st && e->prod && e->prod->kind == K_UNARY && e->prod->sub == 2 &&
                  e->ext == 0 && e->uses == 2) ? e->prod : nullptr;
      Node* sb = chain_node(sB, K_BROADCAST_TO, 1);
      Node* rs = sb ? chain_node(sb->in[0], K_REDUCE, 1) : nullptr;
      Node* sh = en ? chain_node(en->in[0], K_BINARY, 1) : nullptr;
      if (en && rs && sh && sh->sub == 1 && rs->sub == RED_SUM && rs->in[0] == e &&
          dims_are(rs->l0, {r - 1}) && sb->l1 == iota_dims(r - 1)) {
        Tensor* x = sh->in[0];
        Node* mb = chain_node(sh->in[1], K_BROADCAST_TO, 1);
        Node* rm = mb ? chain_node(mb->in[0], K_REDUCE, 1) : nullptr;
        if (rm && rm->sub == RED_MAX && rm->in[0] == x && dims_are(rm->l0, {r - 1}) &&
            mb->l1 == iota_dims(r - 1) && x->dt == kF32 && x->shape == y->shape) {
          // e, its sum and the broadcasts, x - max and the max live only
          // inside the row kernel
          for (Tensor* t : {e, sB, sb->in[0], sh->out[0], sh->in[1], mb->in[0]})
            t->plan_mat = false;
          y->plan_mat = true;
          SoftmaxPlan sp;
          sp.x = x;
          softmax_out[y] = sp;
          continue;
        }
      }
    }
    // ---- RoPE: [astype(] reshape(concat([x0', x1'] as [..., half, 1]), shape) [)]
    if (mo->kind == K_CONCAT && mo->in.size() == 2) {
      Tensor* cc = mo->out[0];
      const int rc = cc->shape.rank;
      if (rc < 3 || mo->i0 != rc - 1 || cc->shape.d[rc - 1] != 2 || cc->ext != 0 ||
          cc->uses != 1)
        continue;
      Node* rsh = sole_consumer(*this, cc);
      if (!rsh || rsh->kind != K_RESHAPE) continue;
      Tensor* R = rsh->out[0];
      const int r = R->shape.rank;
      if (r != rc - 1 || R->shape.d[r - 1] != 2 * cc->shape.d[rc - 2]) continue;
      const int64_t half = cc->shape.d[rc - 2];
      Node* a0 = chain_node(mo->in[0], K_RESHAPE, 1);
      Node* a1 = chain_node(mo->in[1], K_RESHAPE, 1);
      if (!a0 || !a1) continue;
      Node* x0r = chain_node(a0->in[0], K_BINARY, 1);
      Node* x1r = chain_node(a1->in[0], K_BINARY, 1);
      if (!x0r || !x1r || x0r->sub != 1 || x1r->sub != 0) continue;
      Node* m1 = chain_node(x0r->in[0], K_BINARY, 1);
      Node* m2 = chain_node(x0r->in[1], K_BINARY, 1);
      Node* m3 = chain_node(x1r->in[0], K_BINARY, 1);
      Node* m4 = chain_node(x1r->in[1], K_BINARY, 1);
      if (!m1 || !m2 || !m3 || !m4 || m1->sub != 2 || m2->sub != 2 || m3->sub != 2 ||
          m4->sub != 2)
        continue;
      Tensor *cos0 = m1->in[0], *x0F = m1->in[1], *sin0 = m2->in[0], *x1F = m2->in[1];
      if (m3->in[0] != sin0 || m3->in[1] != x0F || m4->in[0] != cos0 || m4->in[1] != x1F)
        continue;
      if (cos0->dt != kF32 || sin0->dt != kF32 || cos0->shape.rank != r ||
          sin0->shape.rank != r)
        continue;
      // x0F / x1F = reshape(slice(reshape(X, [..., half, 2]), [...,0|1], [...,1|2]))
      auto pair_slice = [&](Tensor* f, int which, Tensor** pairs) -> bool {
        Node* fr = chain_node(f, K_RESHAPE, 2);
        if (!fr) return false;
        Node* sl = chain_node(fr->in[0], K_SLICE, 1);
        if (!sl) return false;
        const Shape& P = sl->in[0]->shape;
        if (P.rank != rc) return false;
        for (int i = 0; i < rc; ++i) {
          const int64_t st = i == rc - 1 ? which : 0;
          const int64_t lim = i == rc - 1 ? which + 1 : P.d[i];
          if (sl->l0[i] != st || sl->l1[i] != lim || sl->l2[i] != 1) return false;
        }
        *pairs = sl->in[0];
        return true;
      };
      Tensor *p0, *p1;
      if (!pair_slice(x0F, 0, &p0) || !pair_slice(x1F, 1, &p1) || p0 != p1) continue;
      Node* pr = chain_node(p0, K_RESHAPE, 2);
      if (!pr) continue;
      Tensor* X = pr->in[0];
      if (X->shape != R->shape || X->shape.rank < 2 || X->shape.rank > 4) continue;
      std::vector<Tensor*> inner = {cc, mo->in[0], mo->in[1], a0->in[0], a1->in[0],
                                    x0r->in[0], x0r->in[1], x1r->in[0], x1r->in[1], x0F, x1F,
                                    x0F->prod->in[0], x1F->prod->in[0], p0};
      RopePlan rp;
      rp.cos0 = cos0;
      rp.sin0 = sin0;
      rp.src = X;
      if (!X->st && X->prod && X->prod->kind == K_CONVERT && X->ext == 0 && X->uses == 1 &&
          X->prod->in[0]->dt == kBF16 && X->dt == kF32) {
        rp.src = X->prod->in[0];
        inner.push_back(X);
      } else if (X->dt != kF32) {
        continue;
      }
      if (half % 4) continue;
      Tensor* out = R;
      Node* cv = sole_consumer(*this, R);
      if (cv && cv->kind == K_CONVERT && cv->out[0]->dt == kBF16 && R->dt == kF32) {
        inner.push_back(R);
        out = cv->out[0];
      }
      (void)half;
      for (Tensor* t : inner) t->plan_mat = false;
      out->plan_mat = true;
      if (!fuse_rope(rp, out)) rope_out[out] = rp;
    }
  }
}

// x viewed as rows of n contiguous elements with a uniform row stride.
bool Lower::rows_view(Tensor* x, int64_t n, const void** ptr, int64_t* rs) {
  Tensor* base;
  int64_t off, st[kMaxRank];
  operand_strides(x, &base, &off, st);
  const Shape& S = x->shape;
  const int r = S.rank;
  bool ok = r >= 1 && (S.d[r - 1] == 1 || st[r - 1] == 1);
  int64_t row = r >= 2 ? st[r - 2] : n;
  for (int i = r - 3; i >= 0 && ok; --i)
    if (S.d[i] != 1 && st[i] != st[i + 1] * S.d[i + 1]) ok = false;
  if (r >= 2 && S.d[r - 2] == 1) row = n;
  if (!ok || row < n) {
    std::vector<int> id(r);
    for (int i = 0; i < r; ++i) id[i] = i;
    base = emit_permuted_copy(x, id);
    off = 0;
    row = n;
  }
  *ptr = (const char*)base->data() + off * dt_size(base->dt);
  *rs = row;
  return true;
}

bool Lower::emit_norm(Tensor* t, const NormPlan& p) {
  const int64_t n = t->shape.d[t->shape.rank - 1];
  RowNormArgs a;
  std::memset(&a, 0, sizeof(a));
  rows_view(p.src, n, &a.x, &a.x_rs);
  a.x_dt = p.src->dt;
  a.n = n;
  a.rows = n ? t->numel() / n : 0;
  ensure_mat(p.gamma);
  a.gamma = (const float*)p.gamma->data();
  a.eps = p.eps;
  a.divisor = p.divisor;
  if (p.layer) {
    ensure_mat(p.beta);
    a.layer = 1;
    a.beta = (const float*)p.beta->data();
    a.divisor2 = p.divisor2;
  }
  tensor_alloc(t);
  a.y = t->data();
  a.y_dt = t->dt;
  Launch L{a};
  if (c->profiling)
    L.name = std::string(p.layer ? "layernorm_rows{" : "rmsnorm_rows{") +
             std::to_string(a.rows) + "x" + std::to_string(n) + "}";
  L.fused = true;
  run_launch(c, std::move(L));
  return true;
}

// Strides of v's (rank r <= 4) dims right-aligned into 4 (size-1 dims and
// the missing leading dims get stride 0) over its materialized base.
void Lower::view4(Tensor* v, int r, const void** ptr, int64_t* s) {
  Tensor* base;
  int64_t off, st[kMaxRank];
  operand_strides(v, &base, &off, st);
  for (int i = 0; i < 4; ++i) s[i] = 0;
  for (int i = 0; i < r; ++i) s[4 - r + i] = v->shape.d[i] == 1 ? 0 : st[i];
  *ptr = (const char*)base->data() + off * dt_size(base->dt);
}

// When the rotated tensor is a biased projection seen as heads --
// transpose(reshape(y, [B, S, H, D]), [0, 2, 1, 3]) or reshape(y, [B, S, H, D])
// with y = add(matmul(x, W), bias) planned as EPI_BIAS and used nowhere
// else -- the projection's epilogue rotates and writes `out` directly
// (GroupedQueryAttention.forward with rope: groupedqueryattention.nim).
bool Lower::fuse_rope(const RopePlan& rp, Tensor* out) {
  Tensor* X = rp.src;
  if (X->dt != kBF16 || out->dt != kBF16 || X->shape.rank != 4 || X->st || X->ext != 0 ||
      X->uses != 1)
    return false;
  bool tr = false;
  Tensor* r4 = X;
  if (X->prod && X->prod->kind == K_TRANSPOSE) {
    if (!dims_are(X->prod->l0, {0, 2, 1, 3})) return false;
    r4 = X->prod->in[0];
    tr = true;
    if (r4->st || r4->ext != 0 || r4->uses != 1) return false;
  }
  if (!r4->prod || r4->prod->kind != K_RESHAPE || r4->shape.rank != 4) return false;
  // through a chain of reshapes (the [B * S, N] -> [B, S, N] -> [B, S, H, D]
  // of GroupedQueryAttention.forward), each used only by the next
  Tensor* y = r4->prod->in[0];
  while (!gemm_out.count(y) && y->prod && y->prod->kind == K_RESHAPE && !y->st &&
         y->ext == 0 && y->uses == 1)
    y = y->prod->in[0];
  auto it = gemm_out.find(y);
  if (it == gemm_out.end() || it->second.epi != EPI_BIAS || y->st || y->ext != 0 ||
      y->uses != 1 || y->shape.rank != 2)
    return false;
  const int64_t B = r4->shape.d[0], S = r4->shape.d[1], H = r4->shape.d[2], D = r4->shape.d[3];
  if (y->shape.d[0] != B * S || y->shape.d[1] != H * D || D % 8) return false;
  GemmPlan gp = it->second;
  gp.epi = EPI_BIAS_ROPE;
  gp.rope_cos = rp.cos0;
  gp.rope_sin = rp.sin0;
  gp.rope_t = tr;
  gp.rope_B = B;
  gp.rope_S = S;
  gp.rope_H = H;
  gp.rope_D = D;
  gemm_out.erase(it);
  y->plan_mat = false;
  out->plan_mat = true;
  gemm_out[out] = gp;
  return true;
}

bool Lower::emit_softmax(Tensor* t, const SoftmaxPlan& p) {
  const int64_t n = t->shape.d[t->shape.rank - 1];
  SoftmaxArgs a;
  std::memset(&a, 0, sizeof(a));
  const void* xp;
  rows_view(p.x, n, &xp, &a.x_rs);
  a.x = (const float*)xp;
  a.n = n;
  a.rows = n ? t->numel() / n : 0;
  tensor_alloc(t);
  a.y = (float*)t->data();
  if (!softmax_rows_ok(a)) {
    tensor_drop_storage(t);
    return false;
  }
  Launch L{a};
  if (c->profiling) L.name = "softmax_rows{" + std::to_string(a.rows) + "x" + std::to_string(n) + "}";
  L.fused = true;
  run_launch(c, std::move(L));
  return true;
}

bool Lower::emit_rope(Tensor* t, const RopePlan& p) {
  const Shape& S = t->shape;
  const int r = S.rank;
  RopeArgs a;
  std::memset(&a, 0, sizeof(a));
  int64_t d[4] = {1, 1, 1, 1};
  for (int i = 0; i < r; ++i) d[4 - r + i] = S.d[i];
  a.d0 = d[0];
  a.d1 = d[1];
  a.S = d[2];
  a.half = d[3] / 2;
  if (a.d0 * a.d1 * a.S * (a.half / 4) >= (1ll << 31) || a.half % 4) return false;
  int64_t sx[4], sc[4], ss[4];
  const void *px, *pc, *ps;
  view4(p.src, r, &px, sx);
  view4(p.cos0, r, &pc, sc);
  view4(p.sin0, r, &ps, ss);
  a.x = px;
  a.x_dt = p.src->dt;
  a.x_s0 = sx[0]; a.x_s1 = sx[1]; a.x_ss = sx[2]; a.x_sd = sx[3];
  a.cos = (const float*)pc;
  a.c_s0 = sc[0]; a.c_s1 = sc[1]; a.c_ss = sc[2]; a.c_si = sc[3];
  a.sin = (const float*)ps;
  a.s_s0 = ss[0]; a.s_s1 = ss[1]; a.s_ss = ss[2]; a.s_si = ss[3];
  a.fd_g4 = make_fastdiv((uint32_t)(a.half / 4));
  a.fd_s = make_fastdiv((uint32_t)a.S);
  a.fd_d1 = make_fastdiv((uint32_t)a.d1);
  tensor_alloc(t);
  a.y = t->data();
  a.y_dt = t->dt;
  Launch L{a};
  if (c->profiling) L.name = "rope_pairs{" + std::to_string(t->numel()) + "}";
  L.fused = true;
  run_launch(c, std::move(L));
  return true;
}

// The embedding lookup and the rmsNorm that reads it (LlamaDecoderLayer's
// first norm over Embedding.forward's rows) in one pass: table rows by id
// in, the rows and their norm out.
bool Lower::emit_gather_norm(Node* n, Tensor* t, const NormPlan& p) {
  Tensor *tab = n->in[0], *ix = n->in[1], *G = n->out[0];
  if (t->st || n->i0 != 0 || n->i1 != 0 || tab->shape.rank != 2 || tab->dt != G->dt ||
      G->dt != p.src->dt)
    return false;
  const int64_t nn = t->shape.d[t->shape.rank - 1];
  if (tab->shape.d[1] != nn || G->numel() != ix->numel() * nn || t->numel() != G->numel())
    return false;
  RowNormArgs a;
  std::memset(&a, 0, sizeof(a));
  ensure_mat(tab);
  ensure_mat(ix);
  rows_view(tab, nn, &a.x, &a.x_rs);
  a.x_dt = tab->dt;
  a.n = nn;
  a.rows = ix->numel();
  a.ids = ix->data();
  a.ids_dt = ix->dt;
  a.x_rows = tab->shape.d[0];
  ensure_mat(p.gamma);
  a.gamma = (const float*)p.gamma->data();
  a.eps = p.eps;
  a.divisor = p.divisor;
  if (p.layer) {
    ensure_mat(p.beta);
    a.layer = 1;
    a.beta = (const float*)p.beta->data();
    a.divisor2 = p.divisor2;
  }
  a.y_dt = t->dt;
  a.xout = a.y = reinterpret_cast<void*>(uintptr_t(256));  // allocator blocks are aligned
  if (!rmsnorm_gather_ok(a)) return false;
  tensor_alloc(G);
  tensor_alloc(t);
  a.xout = G->data();
  a.y = t->data();
  Launch L{a};
  if (c->profiling)
    L.name = std::string(p.layer ? "gather_layernorm{" : "gather_rmsnorm{") +
             std::to_string(a.rows) + "x" + std::to_string(nn) + "}";
  L.fused = true;
  run_launch(c, std::move(L));
  return true;
}

void Lower::emit_gather(Node* n) {
  {
    auto gn = gather_norm.find(n->out[0]);
    if (gn != gather_norm.end()) {
      Tensor* t = gn->second;
      gather_norm.erase(gn);
      auto nit = norm_out.find(t);
      if (nit != norm_out.end() && emit_gather_norm(n, t, nit->second)) {
        norm_out.erase(nit);
        return;
      }
    }
  }
  Tensor *src = n->in[0], *ix = n->in[1], *out = n->out[0];
  ensure_mat(src);
  ensure_mat(ix);
  tensor_alloc(out);
  GatherArgs g;
  g.src = src->data();
  g.index = ix->data();
  g.out = out->data();
  g.index_dtype = ix->dt;
  const int dim = (int)n->i0;
  g.n_pre = 1;
  for (int i = 0; i < dim; ++i) g.n_pre *= src->shape.d[i];
  g.src_dim = src->shape.d[dim];
  g.n_idx = ix->numel();
  int64_t post = 1;
  for (int i = dim + 1; i < src->shape.rank; ++i) post *= src->shape.d[i];
  g.row_bytes = post * dt_size(src->dt);
  Launch L{g};
  if (c->profiling) L.name = "gather_rows";
  run_launch(c, std::move(L));
}

// argmax (src/rew/ops/reduce.nim:202-225 semantics) over any dim of a dense
// f32 operand.
void Lower::emit_argmax(Node* n) {
  Tensor *x = n->in[0], *out = n->out[0];
  auto hit = head_out.find(out);
  if (hit != head_out.end()) {
    const HeadPlan hp = hit->second;
    head_out.erase(hit);
    if (emit_class_head(n, hp)) return;
    // outside the fused kernel's limits: the head runs as its own kernels
  }
  ensure_mat(x);
  tensor_alloc(out);
  ArgmaxArgs g;
  g.x = (const float*)x->data();
  g.out = (int32_t*)out->data();
  const int dim = (int)n->i0;
  g.outer = 1;
  g.inner = 1;
  for (int i = 0; i < dim; ++i) g.outer *= x->shape.d[i];
  for (int i = dim + 1; i < x->shape.rank; ++i) g.inner *= x->shape.d[i];
  g.n = x->shape.d[dim];
  if (g.n > INT32_MAX) throw Error(REW_MI355X_ERR_UNSUPPORTED, "argmax: dimension above 2^31");
  Launch L{g};
  if (c->profiling)
    L.name = "argmax{" + std::to_string(g.outer) + "x" + std::to_string(g.n) + "x" +
             std::to_string(g.inner) + "}";
  run_launch(c, std::move(L));
}

// The classifier head: an argmax over dim 1 of a planned softmax of a
// planned Linear (bias epilogue) whose logits and probabilities have no
// other reader.  The plans stay registered, so a head the fused kernel
// cannot take is emitted by them instead.
void Lower::match_class_head() {
  for (Node* n : nodes) {
    if (n->kind != K_ARGMAX || n->i0 != 1) continue;
    Tensor* p = n->in[0];
    if (p->dt != kF32 || p->shape.rank != 2 || p->st || p->ext != 0 || p->uses != 1) continue;
    auto sit = softmax_out.find(p);
    if (sit == softmax_out.end()) continue;
    Tensor* lg = sit->second.x;
    auto lit = gemm_out.find(lg);
    if (lit == gemm_out.end() || lg->st || lg->ext != 0 || lg->uses != 2) continue;
    const GemmPlan& lp = lit->second;
    if (lp.epi != EPI_BIAS || lp.dot2 || lp.group >= 0 || lg->shape != p->shape) continue;
    Tensor *x = lp.dot->in[0], *w = lp.dot->in[1];
    if (x->dt != kF32 || w->dt != kF32 || lg->dt != kF32 || lp.bias->dt != kF32) continue;
    HeadPlan hp;
    hp.x = x;
    hp.w = w;
    hp.b = lp.bias;
    head_out[n->out[0]] = hp;
    lg->plan_mat = false;
    p->plan_mat = false;
  }
}

bool Lower::emit_class_head(Node* n, const HeadPlan& p) {
  Tensor* out = n->out[0];
  const int64_t M = p.x->shape.d[0], K = p.x->shape.d[1], N = p.w->shape.d[1];
  if (p.w->shape.d[0] != K || out->numel() != M) return false;
  // a dense [rows, cols] (or [cols]) f32 operand's address, or null
  auto dense = [&](Tensor* t, int64_t cols) -> const float* {
    Tensor* base;
    int64_t off, st[kMaxRank];
    operand_strides(t, &base, &off, st);
    if (st[t->shape.rank - 1] != 1 || (t->shape.rank == 2 && st[0] != cols)) return nullptr;
    return (const float*)base->data() + off;
  };
  HeadArgs a;
  std::memset(&a, 0, sizeof(a));
  a.M = M;
  a.K = K;
  a.N = N;
  a.x_rs = K;
  a.x = reinterpret_cast<const float*>(uintptr_t(256));  // allocator blocks are aligned
  if (!class_head_ok(a)) return false;
  const void* xp;
  rows_view(p.x, K, &xp, &a.x_rs);
  a.x = (const float*)xp;
  a.w = dense(p.w, N);
  a.b = dense(p.b, N);
  if (!a.w || !a.b || !class_head_ok(a)) return false;
  tensor_alloc(out);
  a.ids = (int32_t*)out->data();
  Launch L{a};
  if (c->profiling)
    L.name = "class_head{" + std::to_string(M) + "x" + std::to_string(K) + "x" +
             std::to_string(N) + "}";
  L.fused = true;
  run_launch(c, std::move(L));
  return true;
}

void Lower::match_router() {
  for (Node* n : nodes) {
    if (n->kind != K_TOPK || n->i2 != 1 || n->out.size() != 2) continue;  // largest first
    Tensor* p = n->in[0];
    if (p->dt != kF32 || p->shape.rank != 2 || p->st || p->ext != 0 || p->uses != 1) continue;
    auto sit = softmax_out.find(p);
    if (sit == softmax_out.end()) continue;
    Tensor* lg = sit->second.x;
    auto lit = gemm_out.find(lg);
    if (lit == gemm_out.end() || lg->st || lg->ext != 0 || lg->uses != 2) continue;
    const GemmPlan& lp = lit->second;
    if (lp.epi != EPI_BIAS || lp.dot2 || lp.group >= 0 || lg->shape != p->shape) continue;
    Tensor *xf = lp.dot->in[0], *w = lp.dot->in[1];
    if (xf->dt != kF32 || w->dt != kF32 || lg->dt != kF32 || lp.bias->dt != kF32 ||
        xf->shape.rank != 2)
      continue;
    RouterPlan rp;
    rp.x = xf;
    bool conv = false;
    if (!xf->st && xf->prod && xf->prod->kind == K_CONVERT && xf->ext == 0 && xf->uses == 1 &&
        xf->prod->in[0]->dt == kBF16) {
      rp.x = xf->prod->in[0];
      conv = true;
    }
    rp.w = w;
    rp.b = lp.bias;
    rp.k = (int)n->i0;
    rp.ids = n->out[1];
    rp.vals = n->out[0];
    // divide(vals, broadcastTo(reduceSum(vals, [1]), vals.shape, [0]))
    Tensor* tv = n->out[0];
    Tensor *denom = nullptr, *dB = nullptr, *tw = nullptr;
    auto ci = cons.find(tv);
    if (!tv->st && tv->ext == 0 && tv->uses == 2 && ci != cons.end() && ci->second.size() == 2) {
      Node *rs = nullptr, *dv = nullptr;
      for (Node* q : ci->second) {
        if (q->kind == K_REDUCE && q->sub == RED_SUM && dims_are(q->l0, {1})) rs = q;
        else if (q->kind == K_BINARY && q->sub == 3 && q->in[0] == tv) dv = q;
      }
      Node* bc = rs ? sole_consumer(*this, rs->out[0]) : nullptr;
      if (bc && dv && bc->kind == K_BROADCAST_TO && dims_are(bc->l1, {0}) &&
          dv->in[1] == bc->out[0] &&
          bc->out[0]->ext == 0 && bc->out[0]->uses == 1 && dv->out[0]->shape == tv->shape) {
        denom = rs->out[0];
        dB = bc->out[0];
        tw = dv->out[0];
      }
    }
    lg->plan_mat = false;
    p->plan_mat = false;
    if (conv) xf->plan_mat = false;
    if (tw) {
      rp.wts = tw;
      rp.vals = nullptr;
      tv->plan_mat = false;
      denom->plan_mat = false;
      dB->plan_mat = false;
      tw->plan_mat = true;
      router_out[tw] = rp;
    } else {
      router_out[tv] = rp;
    }
    router_out[rp.ids] = rp;
  }
}

bool Lower::emit_router(const RouterPlan& p) {
  const int64_t T = p.x->shape.d[0], H = p.x->shape.d[1];
  const int64_t E = p.w->shape.d[1];
  if (p.w->shape.d[0] != H || E > kRouterMaxE) return false;
  auto dense = [&](Tensor* t, int64_t cols) -> const float* {
    Tensor* base;
    int64_t off, st[kMaxRank];
    operand_strides(t, &base, &off, st);
    if (st[t->shape.rank - 1] != 1 || (t->shape.rank == 2 && st[0] != cols)) return nullptr;
    return (const float*)base->data() + off;
  };
  RouterArgs a;
  std::memset(&a, 0, sizeof(a));
  a.x_bf16 = p.x->dt == kBF16 ? 1 : 0;
  a.T = T;
  a.H = H;
  a.E = (int)E;
  a.k = p.k;
  a.x_rs = H;
  a.x = a.w = reinterpret_cast<const float*>(uintptr_t(256));  // allocator blocks are aligned
  if (!moe_router_ok(a)) return false;
  rows_view(p.x, H, &a.x, &a.x_rs);
  a.w = dense(p.w, E);
  a.b = dense(p.b, E);
  if (!a.w || !a.b || !moe_router_ok(a)) return false;
  tensor_alloc(p.ids);
  a.ids = (int32_t*)p.ids->data();
  if (p.wts) {
    tensor_alloc(p.wts);
    a.weights = (float*)p.wts->data();
  }
  if (p.vals) {
    tensor_alloc(p.vals);
    a.vals = (float*)p.vals->data();
  }
  Launch L{a};
  if (c->profiling)
    L.name = "moe_router{" + std::to_string(T) + "x" + std::to_string(H) + "x" +
             std::to_string(E) + ",k" + std::to_string(p.k) + (p.wts ? ",norm" : "") + "}";
  L.fused = true;
  run_launch(c, std::move(L));
  return true;
}

// topK over the last dim (src/rew/ops/sort.nim:36-90 semantics).
void Lower::emit_topk(Node* n) {
  Tensor *x = n->in[0], *vals = n->out[0], *idx = n->out[1];
  ensure_mat(x);
  tensor_alloc(vals);
  tensor_alloc(idx);
  TopkArgs g;
  g.x = (const float*)x->data();
  g.vals = (float*)vals->data();
  g.idx = (int32_t*)idx->data();
  g.cols = x->shape.d[x->shape.rank - 1];
  g.rows = g.cols ? x->numel() / g.cols : 0;
  g.k = (int)n->i0;
  g.largest = (int)n->i2;
  if (g.cols > kTopkMaxCols)
    throw Error(REW_MI355X_ERR_UNSUPPORTED,
                "eager 'topK': last dimension above " + std::to_string(kTopkMaxCols));
  Launch L{g};
  if (c->profiling)
    L.name = "topk{" + std::to_string(g.rows) + "x" + std::to_string(g.cols) + ",k" +
             std::to_string(g.k) + "}";
  run_launch(c, std::move(L));
}

// Row sort over the last dim (the stablehlo.sort form the jit path and the
// sort extension op record).
void Lower::emit_sort(Node* n) {
  SortArgs g;
  std::memset(&g, 0, sizeof g);
  for (Tensor* t : n->in) ensure_mat(t);
  for (Tensor* t : n->out) tensor_alloc(t);
  Tensor* k = n->in[n->i2];
  g.key = k->data();
  g.key_dt = k->dt;
  g.descending = (int)n->i1;
  g.n_ops = (int)n->in.size();
  for (int o = 0; o < g.n_ops; ++o) {
    g.in[o] = n->in[o]->data();
    g.out[o] = n->out[o]->data();
    g.esize[o] = dt_size(n->in[o]->dt);
  }
  g.cols = k->shape.d[k->shape.rank - 1];
  g.rows = g.cols ? k->numel() / g.cols : 0;
  Launch L{g};
  if (c->profiling) L.name = "sort{" + std::to_string(g.rows) + "x" + std::to_string(g.cols) + "}";
  run_launch(c, std::move(L));
}

// pad / dynamicSlice / dynamicUpdateSlice over dense operands: in[0] the
// operand, then the padding value (pad), or the update (dynamicUpdateSlice),
// then the start scalars.
void Lower::emit_window(Node* n) {
  for (Tensor* t : n->in) ensure_mat(t);
  Tensor* out = n->out[0];
  tensor_alloc(out);
  WindowArgs a;
  std::memset(&a, 0, sizeof a);
  Tensor* x = n->in[0];
  a.mode = n->sub;
  a.esize = dt_size(x->dt);
  a.rank = x->shape.rank;
  a.x = x->data();
  a.out = out->data();
  a.total = out->numel();
  const int first_start = n->sub == kWinSlice ? 1 : 2;
  if (n->sub != kWinSlice) a.y = n->in[1]->data();
  for (int d = 0; d < a.rank; ++d) {
    a.out_dims[d] = out->shape.d[d];
    a.x_dims[d] = x->shape.d[d];
    a.y_dims[d] = n->sub == kWinUpdate ? n->in[1]->shape.d[d] : 1;
    if (n->sub == kWinPad) {
      a.lo[d] = n->l0[d];
      a.step[d] = n->l2[d] + 1;
    } else {
      a.start[d] = n->in[first_start + d]->data();
      a.start_dt[d] = n->in[first_start + d]->dt;
    }
  }
  Launch L{a};
  if (c->profiling) L.name = n->name + "{" + std::to_string(a.total) + "}";
  run_launch(c, std::move(L));
}

void Lower::emit_cholesky(Node* n) {
  Tensor* x = n->in[0];
  ensure_mat(x);
  tensor_alloc(n->out[0]);
  CholeskyArgs a;
  std::memset(&a, 0, sizeof a);
  a.x = x->data();
  a.out = n->out[0]->data();
  a.n = x->shape.d[x->shape.rank - 1];
  a.batch = a.n ? x->numel() / (a.n * a.n) : 0;
  a.f64 = x->dt == kF64;
  a.lower = (int)n->i0;
  Launch L{a};
  if (c->profiling)
    L.name = "cholesky{" + std::to_string(a.batch) + "x" + std::to_string(a.n) + "}";
  run_launch(c, std::move(L));
}

void Lower::emit_trisolve(Node* n) {
  Tensor *a = n->in[0], *b = n->in[1];
  ensure_mat(a);
  ensure_mat(b);
  tensor_alloc(n->out[0]);
  TriSolveArgs p;
  std::memset(&p, 0, sizeof p);
  p.a = a->data();
  p.b = b->data();
  p.out = n->out[0]->data();
  p.n = a->shape.d[a->shape.rank - 1];
  p.batch = p.n ? a->numel() / (p.n * p.n) : 0;
  p.m = p.n && p.batch ? b->numel() / (p.batch * p.n) : 0;
  p.f64 = a->dt == kF64;
  p.left = (int)(n->i0 & 1);
  p.lower = (int)((n->i0 >> 1) & 1);
  p.unit = (int)((n->i0 >> 2) & 1);
  p.trans = (int)((n->i0 >> 3) & 1);
  Launch L{p};
  if (c->profiling)
    L.name = "triangular_solve{" + std::to_string(p.batch) + "x" + std::to_string(p.n) + "x" +
             std::to_string(p.m) + "}";
  run_launch(c, std::move(L));
}

void Lower::emit_complex(Node* n) {
  for (Tensor* t : n->in) ensure_mat(t);
  tensor_alloc(n->out[0]);
  ComplexArgs p;
  std::memset(&p, 0, sizeof p);
  p.x = n->in[0]->data();
  p.y = n->in.size() > 1 ? n->in[1]->data() : nullptr;
  p.out = n->out[0]->data();
  p.n = n->out[0]->numel();
  p.mode = (int)n->i0;
  p.esize = (int)n->i1;
  Launch L{p};
  if (c->profiling) L.name = std::string("complex{") + n->name + "}";
  run_launch(c, std::move(L));
}

void Lower::emit_fft1(Node* n) {
  Tensor* x = n->in[0];
  ensure_mat(x);
  tensor_alloc(n->out[0]);
  Fft1Args p;
  std::memset(&p, 0, sizeof p);
  p.x = x->data();
  p.out = n->out[0]->data();
  const int ax = (int)n->i0;
  p.outer = 1;
  p.inner = 1;
  for (int d = 0; d < ax; ++d) p.outer *= x->shape.d[d];
  for (int d = ax + 1; d < x->shape.rank; ++d) p.inner *= x->shape.d[d];
  p.len_in = x->shape.d[ax];
  p.len_out = n->out[0]->shape.d[ax];
  p.n = n->i2;
  p.mode = (int)n->i1;
  p.f64 = x->dt == kF64 || x->dt == kC128;
  Launch L{p};
  if (c->profiling)
    L.name = "fft1{" + std::to_string(p.outer) + "x" + std::to_string(p.len_in) + "x" +
             std::to_string(p.inner) + ",m" + std::to_string(p.mode) + "}";
  run_launch(c, std::move(L));
}

// batch norm: operands in rew's order (inference: x, scale, offset, mean,
// var; training: x, scale, offset; grad: x, scale, mean, var, dy).
void Lower::emit_batchnorm(Node* n) {
  for (Tensor* t : n->in) ensure_mat(t);
  for (Tensor* t : n->out) tensor_alloc(t);
  BatchNormArgs a;
  std::memset(&a, 0, sizeof a);
  Tensor* x = n->in[0];
  a.mode = n->sub;
  a.f64 = x->dt == kF64;
  std::memcpy(&a.eps, &n->i1, sizeof a.eps);
  const int fi = (int)n->i0;
  a.outer = 1;
  a.inner = 1;
  for (int d = 0; d < fi; ++d) a.outer *= x->shape.d[d];
  for (int d = fi + 1; d < x->shape.rank; ++d) a.inner *= x->shape.d[d];
  a.C = x->shape.d[fi];
  a.x = x->data();
  a.scale = n->in[1]->data();
  if (a.mode == kBnInference) {
    a.offset = n->in[2]->data();
    a.mean = n->in[3]->data();
    a.var = n->in[4]->data();
  } else if (a.mode == kBnTraining) {
    a.offset = n->in[2]->data();
  } else {
    a.mean = n->in[2]->data();
    a.var = n->in[3]->data();
    a.dy = n->in[4]->data();
  }
  a.out0 = n->out[0]->data();
  if (n->out.size() == 3) {
    a.out1 = n->out[1]->data();
    a.out2 = n->out[2]->data();
  }
  Launch L{a};
  if (c->profiling) L.name = n->name + "{" + std::to_string(a.outer) + "x" + std::to_string(a.C) +
                             "x" + std::to_string(a.inner) + "}";
  run_launch(c, std::move(L));
}

// stablehlo.gather / stablehlo.scatter: the dimension numbers resolved into
// the per-dimension roles of IndexMapArgs (dense row-major operands).
void Lower::emit_index_map(Node* n) {
  const bool gather = n->kind == K_GATHER;
  Tensor* x = n->in[0];
  Tensor* ix = n->in[1];
  Tensor* src = gather ? x : n->in[2];
  Tensor* out = n->out[0];
  for (Tensor* t : n->in) ensure_mat(t);
  tensor_alloc(out);
  IndexMapArgs g;
  std::memset(&g, 0, sizeof g);
  g.src = src->data();
  g.index = ix->data();
  g.out = out->data();
  g.esize = dt_size(x->dt);
  g.dtype = x->dt;
  g.index_dtype = ix->dt;
  g.op = gather ? 0 : n->sub;
  g.clamp = gather ? 1 : 0;
  const Shape& it = gather ? out->shape : src->shape;  // iteration space
  const Shape& xs = x->shape;
  const Shape& is = ix->shape;
  g.rank_it = it.rank;
  g.rank_x = xs.rank;
  g.total = it.numel();
  int64_t st = 1;
  for (int d = xs.rank - 1; d >= 0; --d) {
    g.dims_x[d] = xs.d[d];
    g.stride_x[d] = st;
    st *= xs.d[d];
  }
  int64_t istride[kMaxRank];
  st = 1;
  for (int d = is.rank - 1; d >= 0; --d) {
    istride[d] = st;
    st *= is.d[d];
  }
  const int ivd = (int)n->i0;
  g.stride_idx_vec = ivd < is.rank ? istride[ivd] : 0;
  std::vector<int> batch_idx_dims;  // index dims other than the index vector dim
  for (int d = 0; d < is.rank; ++d)
    if (d != ivd) batch_idx_dims.push_back(d);
  // window dims of x: not collapsed / inserted (l1) and not batching (l2)
  std::vector<bool> drop(xs.rank, false);
  for (auto d : n->l1) drop[d] = true;
  for (auto d : n->l2) drop[d] = true;
  std::vector<int> win;
  for (int d = 0; d < xs.rank; ++d)
    if (!drop[d]) win.push_back(d);
  std::vector<int> it_of_batch;  // iteration dim of each index batch dim
  size_t wj = 0;
  for (int d = 0; d < it.rank; ++d) {
    g.dims_it[d] = it.d[d];
    if (wj < n->l0.size() && n->l0[wj] == d) {
      g.role[d] = win[wj++];
    } else {
      const int k = (int)it_of_batch.size();
      g.role[d] = -1 - k;
      g.stride_idx_batch[k] = istride[batch_idx_dims[k]];
      it_of_batch.push_back(d);
    }
  }
  g.n_map = (int)n->l4.size();
  for (int j = 0; j < g.n_map; ++j) g.map_x[j] = (int)n->l4[j];
  g.n_bat = (int)n->l2.size();
  for (int i = 0; i < g.n_bat; ++i) {
    g.bat_x[i] = (int)n->l2[i];
    int k = 0;
    while (batch_idx_dims[k] != (int)n->l3[i]) ++k;
    g.bat_it[i] = it_of_batch[k];
  }
  for (int d = 0; d < xs.rank; ++d) g.slice[d] = gather ? n->l5[d] : 0;
  if (!gather)  // the result starts as a copy of the input
    run_launch(c, Launch{FillL{out->data(), x->data(), (size_t)out->nbytes()}});
  Launch L{IndexMapL{g, !gather}};
  if (c->profiling)
    L.name = (gather ? "gather_nd{" : "scatter{") + std::to_string(g.total) + "}";
  run_launch(c, std::move(L));
}

// ---------------------------------------------------------------------------
// flush
// ---------------------------------------------------------------------------

// Steps 2 and 3 of a flush: classification, pattern matching and emission.
static void lower_graph(Ctx* c, Lower& L, const std::string* sig,
                        const std::vector<Tensor*>& leaves, const std::vector<int32_t>& leaf_slot,
                        std::exception_ptr* err) {
  // 2. classification
  std::unordered_map<Tensor*, std::vector<Node*>> consumers;
  for (Node* n : L.nodes)
    for (Tensor* t : n->in) consumers[t].push_back(n);
  // walk consumers through views: (count of expression uses, needs memory)
  std::function<void(Tensor*, int*, bool*)> uses_of = [&](Tensor* t, int* cnt, bool* mem) {
    auto it = consumers.find(t);
    if (it == consumers.end()) return;
    for (Node* q : it->second) {
      if (is_view(q->kind) && q->out[0]->ext == 0) {
        uses_of(q->out[0], cnt, mem);
      } else {
        *cnt += 1;
        if (!takes_expression(q->kind)) *mem = true;
      }
    }
  };
  std::unordered_map<Tensor*, int> cost;
  for (Node* n : L.nodes) {
    for (Tensor* t : n->out) {
      t->plan_mat = false;
      if (!is_ew(n->kind) && !is_view(n->kind)) {
        t->plan_mat = true;
        continue;
      }
      if (t->ext > 0) {
        t->plan_mat = true;
        continue;
      }
      if (is_view(n->kind)) continue;
      int cnt = 0;
      bool mem = false;
      uses_of(t, &cnt, &mem);
      int cst = 1;
      for (Tensor* x : n->in) {
        Tensor* y = x;
        while (y->prod && is_view(y->prod->kind) && !y->plan_mat && !y->st) y = y->prod->in[0];
        if (y->prod && !y->st && !y->plan_mat && is_ew(y->prod->kind)) cst += cost[y];
      }
      cost[t] = cst;
      if (mem || (cnt >= 2 && cst > 2) || cst > 48) t->plan_mat = true;
      if (t->plan_mat) cost[t] = 0;
    }
  }

  // 2b. fused attention: an SDPA chain is emitted as one launch at its PV
  // product; its intermediates are never materialized
  if (c->mode == REW_MI355X_MODE_DEFERRED && !c->no_fusion_patterns) {
    for (Node* n : L.nodes)
      if (n->kind == K_DOT_GENERAL) L.match_flash(n);
    L.cons = consumers;
    L.match_flash_out();
    L.match_gemm_epilogues();
    if (!c->dense_moe) L.match_moe();
    L.match_rows();
    L.match_class_head();
    L.match_router();
    L.match_gemm_groups();
  }

  // 3. emission in creation order (recorded as the graph's plan when
  // `sig` is set)
  if (sig) plan_record_begin(c, L.nodes, leaves, leaf_slot);
  try {
    for (Node* n : L.nodes)
      for (Tensor* t : n->out)
        if (t->plan_mat && !t->st) L.ensure_mat(t);
  } catch (...) {
    *err = std::current_exception();
  }
  for (Tensor* t : L.temps) maybe_destroy(t);
  L.temps.clear();
  if (sig) plan_record_end(c, *sig, !*err);
}

static void flush_graph(Ctx* c, std::vector<Node*>& all);

void flush(Ctx* c) {
  if (c->pending.empty()) return;
  const auto t0 = std::chrono::steady_clock::now();
  std::vector<Node*> all;
  all.swap(c->pending);
  c->stats.flushes++;
  struct Clock {
    Ctx* c;
    std::chrono::steady_clock::time_point t0;
    ~Clock() {
      c->stats.flush_host_ns +=
          std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now() - t0)
              .count();
    }
  } clock{c, t0};
  flush_graph(c, all);
}

static void flush_graph(Ctx* c, std::vector<Node*>& all) {
  // 1. dead-node elimination (reverse creation order)
  for (size_t i = all.size(); i-- > 0;) {
    Node* n = all[i];
    bool dead = true;
    for (Tensor* t : n->out)
      if (t->ext > 0 || t->uses > 0) dead = false;
    if (dead) {
      n->dead = true;
      for (Tensor* t : n->in) t->uses--;
    }
  }
  Lower L(c);
  for (Node* n : all)
    if (!n->dead) L.nodes.push_back(n);

  // 1b. a graph flushed before replays the launches recorded then
  std::string sig;
  std::vector<Tensor*> leaves;
  std::vector<int32_t> leaf_slot;
  FlushPlan* plan = nullptr;
  if (c->plan_cache && !L.nodes.empty()) {
    sig = flush_signature(c, L.nodes, &leaves, &leaf_slot);
    plan = plan_find(c, sig);
  }
  if (c->capture && !sig.empty()) {
    // a jit call recording its module's direct plan: what it needs of this graph
    FlushCapture* cap = c->capture;
    cap->done = true;
    cap->sig = sig;
    cap->leaves = leaves;
    cap->node_meta.resize(L.nodes.size());
    for (size_t i = 0; i < L.nodes.size(); ++i) {
      const Node* n = L.nodes[i];
      for (size_t o = 0; o < n->out.size(); ++o) {
        cap->node_meta[i].emplace_back(n->out[o]->dt, n->out[o]->shape);
        cap->out_ref.emplace(n->out[o], std::make_pair((int32_t)i, (int32_t)o));
      }
    }
  }
  std::exception_ptr err;
  if (plan && plan->ok) {
    c->stats.flush_plan_hits++;
    try {
      plan_replay(c, *plan, L.nodes, leaves);
    } catch (...) {
      err = std::current_exception();
    }
  } else {
    lower_graph(c, L, !sig.empty() && !plan ? &sig : nullptr, leaves, leaf_slot, &err);
  }

  // 4. release: graph references drop, temporaries free
  for (Node* n : all) {
    if (!n->dead)
      for (Tensor* t : n->in) t->uses--;
  }
  std::vector<Tensor*> touched;
  for (Node* n : all) {
    for (Tensor* t : n->in) touched.push_back(t);
    for (Tensor* t : n->out) {
      t->prod = nullptr;
      touched.push_back(t);
    }
  }
  std::sort(touched.begin(), touched.end());
  touched.erase(std::unique(touched.begin(), touched.end()), touched.end());
  for (Tensor* t : touched) {
    t->plan_mat = false;
    maybe_destroy(t);
  }
  for (Node* n : all) delete n;
  if (err) std::rethrow_exception(err);
}

}  // namespace rew
