// Flush plans (the analogue of rew's per-signature executable cache,
// src/rew/eager.nim:1620-1680, one level up: per flushed graph instead of
// per op).  The first flush of a graph is lowered as usual while every
// allocation, alias, release and launch it makes is recorded, with each
// device pointer of a launch stored as (storage slot, byte offset).  A
// later flush whose signature matches replays the record: the same
// allocations in the same order, the launches re-pointed at this flush's
// leaves and new storages.  Lowering depends only on what the signature
// holds, so the replay enqueues exactly what lowering would.  A lowering
// whose record is incomplete (a pointer into memory the flush does not
// own, an event on a tensor outside the flush) is stored as "not
// replayable" and lowered anew each time.
#include "plan.h"

#include <cstring>
#include <deque>
#include <map>
#include <unordered_map>

namespace rew {

namespace {

constexpr size_t kMaxPlans = 64;  // per context, oldest dropped first

// ---- device pointer fields of each launch kind ----------------------------------------
template <class T, class F>
inline void field(F& f, T*& p) {
  const void* v = p;
  f(v);
  p = static_cast<T*>(const_cast<void*>(v));
}

template <class F>
void program_ptrs(vm::Program& P, F& f) {
  for (int i = 0; i < P.n_leaves; ++i) field(f, P.leaf[i].ptr);
  for (int i = 0; i < P.n_outs; ++i) field(f, P.out[i].ptr);
}

template <class F>
struct PtrVisit {
  F& f;
  void operator()(EwL& l) { program_ptrs(l.P, f); }
  void operator()(ReduceL& l) {
    program_ptrs(l.P, f);
    field(f, l.A.out);
    for (int i = 0; i < l.A.n_extra; ++i) field(f, l.A.extra_out[i]);
    for (int i = 0; i < l.A.n_mean; ++i) field(f, l.A.mean_out[i]);
  }
  void operator()(GemmL& l) {
    for (GemmArgs& g : l.g) {
      field(f, g.a);
      field(f, g.b);
      field(f, g.c);
      field(f, g.bias);
      field(f, g.bias2);
      field(f, g.res);
      field(f, g.b2);
      field(f, g.rope_cos);
      field(f, g.rope_sin);
    }
  }
  void operator()(FlashArgs& a) {
    field(f, a.q);
    field(f, a.k);
    field(f, a.v);
    field(f, a.o);
  }
  void operator()(RowNormArgs& a) {
    field(f, a.x);
    field(f, a.gamma);
    field(f, a.beta);
    field(f, a.y);
    field(f, a.ids);
    field(f, a.xout);
  }
  void operator()(SoftmaxArgs& a) {
    field(f, a.x);
    field(f, a.y);
  }
  void operator()(RopeArgs& a) {
    field(f, a.x);
    field(f, a.cos);
    field(f, a.sin);
    field(f, a.y);
  }
  void operator()(GatherArgs& a) {
    field(f, a.src);
    field(f, a.index);
    field(f, a.out);
  }
  void operator()(ArgmaxArgs& a) {
    field(f, a.x);
    field(f, a.out);
  }
  void operator()(TopkArgs& a) {
    field(f, a.x);
    field(f, a.vals);
    field(f, a.idx);
  }
  void operator()(SortArgs& a) {
    field(f, a.key);
    for (int o = 0; o < a.n_ops; ++o) {
      field(f, a.in[o]);
      field(f, a.out[o]);
    }
  }
  void operator()(IndexMapL& l) {
    field(f, l.g.src);
    field(f, l.g.index);
    field(f, l.g.out);
  }
  void operator()(MoeL& l) {
    field(f, l.a.x);
    field(f, l.a.start);
    field(f, l.a.topi);
    field(f, l.a.topw);
    field(f, l.a.out);
    for (const void*& p : l.tab) field(f, p);
    field(f, l.scratch);
  }
  void operator()(FillL& l) {
    field(f, l.dst);
    field(f, l.src);
  }
  void operator()(WindowArgs& a) {
    field(f, a.x);
    field(f, a.y);
    field(f, a.out);
    for (int d = 0; d < a.rank; ++d) field(f, a.start[d]);
  }
  void operator()(CholeskyArgs& a) {
    field(f, a.x);
    field(f, a.out);
  }
  void operator()(ComplexArgs& a) {
    field(f, a.x);
    field(f, a.y);
    field(f, a.out);
  }
  void operator()(Fft1Args& a) {
    field(f, a.x);
    field(f, a.out);
  }
  void operator()(TriSolveArgs& a) {
    field(f, a.a);
    field(f, a.b);
    field(f, a.out);
  }
  void operator()(BatchNormArgs& a) {
    for (const void** p : {&a.x, &a.scale, &a.offset, &a.mean, &a.var, &a.dy}) field(f, *p);
    for (void** p : {&a.out0, &a.out1, &a.out2}) field(f, *p);
  }
  void operator()(HeadArgs& a) {
    field(f, a.x);
    field(f, a.w);
    field(f, a.b);
    field(f, a.probs);
    field(f, a.ids);
  }
  void operator()(RouterArgs& a) {
    field(f, a.x);
    field(f, a.w);
    field(f, a.b);
    field(f, a.ids);
    field(f, a.vals);
    field(f, a.weights);
  }
};

template <class F>
void for_each_ptr(LaunchArgs& a, F& f) {
  std::visit(PtrVisit<F>{f}, a);
}

struct Exec {
  Ctx* c;
  void operator()(EwL& l) { launch_ew(l.P, l.S, l.vec, c->stream); }
  void operator()(ReduceL& l) { launch_reduce(l.P, l.S, l.A, l.vec, c->stream); }
  void operator()(GemmL& l) {
    if (l.multi) launch_gemm_multi(l.g.data(), (int)l.g.size(), c->stream);
    else launch_gemm(l.g[0], c->stream);
  }
  void operator()(FlashArgs& a) { launch_flash(a, c->stream); }
  void operator()(RowNormArgs& a) { launch_rmsnorm_rows(a, c->stream); }
  void operator()(SoftmaxArgs& a) { launch_softmax_rows(a, c->stream); }
  void operator()(RopeArgs& a) { launch_rope(a, c->stream); }
  void operator()(GatherArgs& a) { launch_gather(a, c->stream); }
  void operator()(ArgmaxArgs& a) { launch_argmax(a, c->stream); }
  void operator()(TopkArgs& a) { launch_topk(a, c->stream); }
  void operator()(SortArgs& a) { launch_sort(a, c->stream); }
  void operator()(IndexMapL& l) {
    if (l.scatter) launch_scatter(l.g, c->stream);
    else launch_gather_nd(l.g, c->stream);
  }
  void operator()(MoeL& l) {
    l.a.expert = l.expert.data();
    for (int j = 0; j < 6; ++j) l.a.ptr[j] = l.tab.data() + (size_t)j * l.a.n;
    for (int j = 0; j < 6 && l.a.n_shared; ++j)
      l.a.sptr[j] = l.tab.data() + 6 * (size_t)l.a.n + (size_t)j * l.a.n_shared;
    run_routed_ffn(c, l.a, l.scratch);
  }
  void operator()(WindowArgs& a) { launch_window(a, c->stream); }
  void operator()(CholeskyArgs& a) { launch_cholesky(a, c->stream); }
  void operator()(TriSolveArgs& a) { launch_trisolve(a, c->stream); }
  void operator()(ComplexArgs& a) { launch_complex(a, c->stream); }
  void operator()(Fft1Args& a) { launch_fft1(a, c->stream); }
  void operator()(BatchNormArgs& a) { launch_batchnorm(a, c->stream); }
  void operator()(HeadArgs& a) { launch_class_head(a, c->stream); }
  void operator()(RouterArgs& a) { launch_moe_router(a, c->stream); }
  void operator()(FillL& l) {
    if (l.bytes == 0) return;
    if (l.src)
      REW_HIP(hipMemcpyAsync(l.dst, l.src, l.bytes, hipMemcpyDeviceToDevice, c->stream));
    else
      REW_HIP(hipMemsetAsync(l.dst, 0, l.bytes, c->stream));
  }
};

}  // namespace

// ---- recording ----------------------------------------------------------------------
struct PlanRecorder {
  FlushPlan* plan = nullptr;
  std::unordered_map<const Tensor*, PlanRef> refs;  // leaves, node outputs, temporaries
  // live storages of the flush: start address -> (end address, slot)
  std::map<uintptr_t, std::pair<uintptr_t, int32_t>> live;
  bool ok = true;

  bool find(const Tensor* t, PlanRef* r) const {
    auto it = refs.find(t);
    if (it == refs.end()) return false;
    *r = it->second;
    return true;
  }
  // t's name; a tensor first seen during the lowering is a temporary of it
  PlanRef name(Tensor* t) {
    PlanRef r;
    if (find(t, &r)) return r;
    r.kind = PlanRef::TEMP;
    r.idx = (int32_t)plan->temps.size();
    r.out = 0;
    plan->temps.emplace_back(t->dt, t->shape);
    refs.emplace(t, r);
    return r;
  }
  Reloc resolve(const void* p) {
    if (!p) return {-1, 0};
    const uintptr_t a = (uintptr_t)p;
    auto it = live.upper_bound(a);
    if (it == live.begin()) {
      ok = false;
      return {-1, 0};
    }
    --it;
    if (a >= it->second.first) {
      ok = false;
      return {-1, 0};
    }
    return {it->second.second, (int64_t)(a - it->first)};
  }
};

void plan_note_alloc(Tensor* t) {
  PlanRecorder* r = t->ctx->rec;
  if (!r) return;
  PlanEvent e;
  e.type = PlanEvent::NEW;
  e.a = r->name(t);
  e.id = r->plan->n_slots++;
  const uintptr_t p = (uintptr_t)t->st->ptr;
  r->live[p] = {p + t->st->bytes, e.id};
  r->plan->events.push_back(e);
}

void plan_note_alias(Tensor* t, Tensor* src) {
  PlanRecorder* r = t->ctx->rec;
  if (!r) return;
  PlanEvent e;
  e.type = PlanEvent::ALIAS;
  e.a = r->name(t);
  if (!r->find(src, &e.b)) {
    r->ok = false;
    return;
  }
  r->plan->events.push_back(e);
}

void plan_note_drop(Tensor* t) {
  PlanRecorder* r = t->ctx->rec;
  if (!r) return;
  PlanEvent e;
  e.type = PlanEvent::DROP;
  if (!r->find(t, &e.a)) {
    r->ok = false;
    return;
  }
  r->plan->events.push_back(e);
}

void plan_note_destroy(Tensor* t) {
  PlanRecorder* r = t->ctx->rec;
  if (!r) return;
  PlanEvent e;
  e.type = PlanEvent::DESTROY;
  if (!r->find(t, &e.a) || e.a.kind != PlanRef::TEMP) {
    r->ok = false;
    return;
  }
  r->refs.erase(t);  // the record may be reused for another tensor
  r->plan->events.push_back(e);
}

void plan_note_free(Storage* s) {
  PlanRecorder* r = s->ctx->rec;
  if (!r) return;
  r->live.erase((uintptr_t)s->ptr);
}

void run_launch(Ctx* c, Launch&& L) {
  // the routed-expert chain brackets and counts its own launches; a fill
  // is a copy-engine operation
  const bool kernel = !std::holds_alternative<MoeL>(L.args) &&
                      !std::holds_alternative<FillL>(L.args);
  if (kernel && c->profiling) prof_begin(c, L.name);
  std::visit(Exec{c}, L.args);
  if (kernel) {
    prof_end(c);
    c->stats.kernels_launched++;
    if (L.fused) c->stats.fused_groups++;
  }
  PlanRecorder* r = c->rec;
  if (!r) return;
  std::vector<Reloc> rl;
  auto note = [&](const void*& p) { rl.push_back(r->resolve(p)); };
  for_each_ptr(L.args, note);
  PlanEvent e;
  e.type = PlanEvent::LAUNCH;
  e.id = (int32_t)r->plan->launches.size();
  r->plan->launches.push_back(std::move(L));
  r->plan->relocs.push_back(std::move(rl));
  r->plan->events.push_back(e);
}

// ---- signature ----------------------------------------------------------------------
std::string flush_signature(Ctx* c, const std::vector<Node*>& nodes,
                            std::vector<Tensor*>* leaves, std::vector<int32_t>* leaf_slot) {
  std::string s;
  s.reserve(nodes.size() * 128 + 16);
  auto put = [&](const void* p, size_t n) { s.append(static_cast<const char*>(p), n); };
  auto i32 = [&](int64_t v) {
    const int32_t x = (int32_t)v;
    put(&x, 4);
  };
  auto i64 = [&](int64_t v) { put(&v, 8); };
  auto list = [&](const std::vector<int64_t>& v) {
    i32((int64_t)v.size());
    if (!v.empty()) put(v.data(), v.size() * 8);
  };
  auto shape = [&](const Shape& sh) {
    i32(sh.rank);
    put(sh.d, (size_t)sh.rank * 8);
  };
  i32(c->mode);
  i32((c->no_fusion_patterns ? 1 : 0) | (c->profiling ? 2 : 0) | (c->dense_moe ? 4 : 0));
  std::unordered_map<const Tensor*, std::pair<int32_t, int32_t>> where;
  std::unordered_map<const Tensor*, int32_t> leaf_of;
  std::unordered_map<const Storage*, int32_t> slot_of;
  where.reserve(nodes.size() * 2);
  for (size_t i = 0; i < nodes.size(); ++i) {
    const Node* n = nodes[i];
    i32(n->kind);
    i32(n->sub);
    i32((int64_t)n->name.size());
    put(n->name.data(), n->name.size());
    for (const auto* v : {&n->l0, &n->l1, &n->l2, &n->l3, &n->l4, &n->l5}) list(*v);
    i64(n->i0);
    i64(n->i1);
    i64(n->i2);
    i32(n->dt_attr);
    i32(n->cmp);
    i32((int64_t)n->in.size());
    i32((int64_t)n->out.size());
    for (Tensor* t : n->in) {
      auto w = where.find(t);
      if (w != where.end()) {
        i32(-1);
        i32(w->second.first);
        i32(w->second.second);
        continue;
      }
      auto l = leaf_of.find(t);
      if (l != leaf_of.end()) {
        i32(-2);
        i32(l->second);
        continue;
      }
      // a leaf first used here: what lowering may read of it
      const int32_t li = (int32_t)leaves->size();
      leaf_of.emplace(t, li);
      leaves->push_back(t);
      int32_t slot = -1;
      if (t->st) {
        auto it = slot_of.find(t->st);
        if (it == slot_of.end()) {
          slot = (int32_t)slot_of.size();
          slot_of.emplace(t->st, slot);
        } else {
          slot = it->second;
        }
      }
      leaf_slot->push_back(slot);
      i32(-3);
      i32(t->dt);
      shape(t->shape);
      i32(slot);
      i32(t->st ? (int64_t)((uintptr_t)t->st->ptr & 255) : -1);
      i32(t->prod ? 1 : 0);
      i32(t->has_host ? 1 : 0);
      if (t->has_host) put(t->host, sizeof t->host);
    }
    for (size_t o = 0; o < n->out.size(); ++o) {
      const Tensor* t = n->out[o];
      where.emplace(t, std::make_pair((int32_t)i, (int32_t)o));
      i32(t->dt);
      shape(t->shape);
      i32(t->ext > 0 ? 1 : 0);
    }
  }
  return s;
}

// ---- storage of plans -----------------------------------------------------------------
FlushPlan* plan_find(Ctx* c, const std::string& sig) {
  auto it = c->flush_plans.find(sig);
  return it == c->flush_plans.end() ? nullptr : it->second;
}

void plan_record_begin(Ctx* c, const std::vector<Node*>& nodes,
                       const std::vector<Tensor*>& leaves, const std::vector<int32_t>& leaf_slot) {
  PlanRecorder* r = new PlanRecorder();
  r->plan = new FlushPlan();
  for (size_t i = 0; i < leaves.size(); ++i) {
    Tensor* t = leaves[i];
    r->refs.emplace(t, PlanRef{PlanRef::LEAF, (int32_t)i, 0});
    const int32_t s = leaf_slot[i];
    if (s < 0) continue;
    if ((size_t)s == r->plan->leaf_slot_first.size()) {
      r->plan->leaf_slot_first.push_back((int32_t)i);
      const uintptr_t p = (uintptr_t)t->st->ptr;
      r->live[p] = {p + t->st->bytes, s};
    }
  }
  r->plan->n_slots = (int)r->plan->leaf_slot_first.size();
  for (size_t i = 0; i < nodes.size(); ++i)
    for (size_t o = 0; o < nodes[i]->out.size(); ++o)
      r->refs.emplace(nodes[i]->out[o], PlanRef{PlanRef::NODE, (int32_t)i, (int32_t)o});
  c->rec = r;
}

void plan_record_end(Ctx* c, const std::string& sig, bool keep) {
  PlanRecorder* r = c->rec;
  if (!r) return;
  c->rec = nullptr;
  FlushPlan* p = r->plan;
  p->ok = r->ok;
  delete r;
  if (!keep) {
    delete p;
    return;
  }
  if (!p->ok) {  // kept only to skip recording this graph again
    p->events.clear();
    p->launches.clear();
    p->relocs.clear();
    p->temps.clear();
  }
  while (c->flush_plans.size() >= kMaxPlans && !c->plan_order.empty()) {
    auto it = c->flush_plans.find(c->plan_order.front());
    if (it != c->flush_plans.end()) {
      delete it->second;
      c->flush_plans.erase(it);
    }
    c->plan_order.pop_front();
  }
  auto ins = c->flush_plans.emplace(sig, p);
  if (!ins.second) {  // cannot happen: a stored signature is replayed, not recorded
    delete p;
    return;
  }
  c->plan_order.push_back(sig);
}

void plan_cache_clear(Ctx* c) {
  for (auto& kv : c->flush_plans) delete kv.second;
  c->flush_plans.clear();
  c->plan_order.clear();
}

// ---- replay -----------------------------------------------------------------------------
namespace {

// The events of p over this flush's leaves; node(idx, out) names a node
// output of the recorded graph.
template <class NodeOut>
void replay_events(Ctx* c, const FlushPlan& p, const std::vector<Tensor*>& leaves,
                   NodeOut node) {
  std::vector<uintptr_t> slot((size_t)p.n_slots, 0);
  for (size_t s = 0; s < p.leaf_slot_first.size(); ++s)
    slot[s] = (uintptr_t)leaves[p.leaf_slot_first[s]]->data();
  std::vector<Tensor*> temps(p.temps.size(), nullptr);
  auto get = [&](const PlanRef& r) -> Tensor* {
    switch (r.kind) {
      case PlanRef::LEAF: return leaves[r.idx];
      case PlanRef::NODE: return node(r.idx, r.out);
      default:
        if (!temps[r.idx]) temps[r.idx] = new_tensor(c, p.temps[r.idx].first, p.temps[r.idx].second);
        return temps[r.idx];
    }
  };
  auto release_temps = [&] {
    for (Tensor*& t : temps)
      if (t) {
        maybe_destroy(t);
        t = nullptr;
      }
  };
  try {
    for (const PlanEvent& e : p.events) {
      switch (e.type) {
        case PlanEvent::NEW: {
          Tensor* t = get(e.a);
          if (t->st) throw Error(REW_MI355X_ERR_INVALID, "internal: flush plan out of step");
          tensor_alloc(t);
          slot[e.id] = (uintptr_t)t->data();
          break;
        }
        case PlanEvent::ALIAS: tensor_alias(get(e.a), get(e.b)); break;
        case PlanEvent::DROP: tensor_drop_storage(get(e.a)); break;
        case PlanEvent::DESTROY: {
          Tensor*& t = temps[e.a.idx];
          if (t) {
            maybe_destroy(t);
            t = nullptr;
          }
          break;
        }
        case PlanEvent::LAUNCH: {
          Launch L = p.launches[e.id];
          const std::vector<Reloc>& rl = p.relocs[e.id];
          size_t i = 0;
          auto put = [&](const void*& v) {
            const Reloc& r = rl[i++];
            v = r.slot < 0 ? nullptr : reinterpret_cast<const void*>(slot[r.slot] + r.delta);
          };
          for_each_ptr(L.args, put);
          run_launch(c, std::move(L));
          break;
        }
      }
    }
  } catch (...) {
    release_temps();
    throw;
  }
  release_temps();
}

}  // namespace

void plan_replay(Ctx* c, const FlushPlan& p, const std::vector<Node*>& nodes,
                 const std::vector<Tensor*>& leaves) {
  replay_events(c, p, leaves, [&](int32_t i, int32_t o) { return nodes[i]->out[o]; });
}

std::vector<Tensor*> plan_replay_direct(Ctx* c, const DirectPlan& d,
                                        const std::vector<Tensor*>& leaves) {
  // node outputs exist as plain tensors, made when the plan first names them
  std::vector<std::vector<Tensor*>> made(d.node_meta.size());
  auto node = [&](int32_t i, int32_t o) -> Tensor* {
    std::vector<Tensor*>& v = made[i];
    if (v.empty()) v.assign(d.node_meta[i].size(), nullptr);
    if (!v[o]) v[o] = new_tensor(c, d.node_meta[i][o].first, d.node_meta[i][o].second);
    return v[o];
  };
  auto drop_all = [&] {
    for (auto& v : made)
      for (Tensor*& t : v)
        if (t) {
          maybe_destroy(t);
          t = nullptr;
        }
  };
  std::vector<Tensor*> res;
  try {
    replay_events(c, d.plan, leaves, node);
    for (const auto& r : d.results) {
      Tensor* t = node(r.first, r.second);
      if (!t->st) throw Error(REW_MI355X_ERR_INVALID, "internal: direct plan left a result empty");
      res.push_back(t);
    }
  } catch (...) {
    drop_all();
    throw;
  }
  for (Tensor* t : res) t->ext++;
  drop_all();  // the results keep their owner references
  return res;
}

}  // namespace rew
