// Internal runtime structures of librew_mi355x: tensor records, the
// deferred op graph, the per-device context and its caching allocator.
#pragma once

#include <deque>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "common.h"

namespace rew {

struct Ctx;
struct Node;
struct RoutedFfn;
struct JitModule;
struct FlushPlan;
struct PlanRecorder;
struct FlushCapture;

// A device allocation shared by every tensor that aliases it (a reshape of
// a materialized tensor aliases its source).
struct Storage {
  Ctx* ctx = nullptr;
  void* ptr = nullptr;
  size_t bytes = 0;   // rounded block size
  int refs = 0;
};

// The record behind an opaque rew_mi355x_buf handle.
struct Tensor {
  Ctx* ctx = nullptr;
  int ext = 0;              // owner references held through the ABI
  int uses = 0;             // references from pending graph nodes
  int dt = kF32;
  Shape shape;
  Storage* st = nullptr;    // dense row-major data once materialized
  Node* prod = nullptr;     // pending producer, nullptr once materialized
  int prod_out = 0;         // which output of `prod`
  bool has_host = false;    // small constant whose bytes are known on host
  uint8_t host[16] = {0};
  // planner scratch (valid during one flush)
  int plan_uses = 0;        // remaining consumer launches in this flush
  bool plan_mat = false;    // planner decided to materialize
  bool plan_dead = false;

  int64_t numel() const { return shape.numel(); }
  int64_t nbytes() const { return numel() * dt_size(dt); }
  void* data() const { return st ? st->ptr : nullptr; }
};

// Op kinds (the subset of rew's EagerOpKind this backend implements,
// src/rew/eager.nim:718-764, plus backend extensions argmax/topK/sort/gather/scatter).
enum Kind : int {
  K_BINARY, K_UNARY, K_CONVERT, K_ISFINITE, K_BITCAST, K_RESHAPE,
  K_TRANSPOSE, K_REVERSE, K_BROADCAST_TO, K_BROADCAST, K_SLICE, K_CONCAT,
  K_IOTA, K_COMPARE, K_SELECT, K_CLAMP, K_REDUCE, K_DOT_GENERAL, K_DOT,
  K_INDEX_SELECT, K_ARGMAX, K_TOPK, K_REDUCE_PRECISION, K_PAD, K_SORT, K_GATHER, K_SCATTER,
  K_CONST,     // a scalar whose value the op fixes (getDimensionSize, replicaId, partitionId)
  K_WINDOW,    // pad / dynamicSlice / dynamicUpdateSlice (sub: kWin*)
  K_CHOLESKY,
  K_TRISOLVE,
  K_COMPLEX,
  K_FFT1,
  K_BATCHNORM, // batchNormInference / Training / Grad (sub: kBn*)
  // composite kernels created by the planner (never recorded directly)
  K_COUNT
};

struct Node {
  int kind = 0;
  int sub = 0;              // op-specific selector (binary op, reduce op, ...)
  std::string name;         // rew op name
  std::vector<Tensor*> in;
  std::vector<Tensor*> out;
  // typed attributes
  std::vector<int64_t> l0, l1, l2, l3, l4, l5;
  int64_t i0 = 0, i1 = 0, i2 = 0;
  int dt_attr = -1;
  int cmp = 0;
  int n_in_keep = -1;       // >= 0: only the first n_in_keep operands are read
                            // (the rest only fix static shapes)
  // planner scratch
  bool dead = false;
  bool done = false;
  int order = 0;
};

// Stream-ordered caching allocator.  All work of a context runs on one
// stream, so a block freed after its last consumer was enqueued can be
// handed to the next producer without synchronising.
struct Allocator {
  std::multimap<size_t, void*> free_blocks;
  size_t cached = 0;   // bytes in free_blocks
  size_t in_use = 0;   // bytes handed out
  // most device bytes the allocator may hold (handed out + cached); 0: no
  // limit but the device's (REW_MI355X_MAX_DEVICE_BYTES)
  size_t cap = 0;
  int ordinal = 0;
  void* get(size_t bytes, size_t* rounded);
  void put(void* p, size_t rounded);
  void trim();
  static size_t round(size_t bytes);
};

struct ProfEntry {
  std::string name;
  hipEvent_t start, stop;
};

struct Ctx {
  int ordinal = 0;
  hipStream_t stream = nullptr;
  std::recursive_mutex mu;
  Allocator alloc;
  std::vector<Node*> pending;
  int mode = REW_MI355X_MODE_DEFERRED;
  int flush_threshold = 4096;
  bool no_fusion_patterns = false;  // REW_MI355X_NO_PATTERNS=1: per-op kernels only
  // REW_MI355X_DENSE_MOE=1: DeepSeekMoE's dense expert loop runs as written
  // (every routed expert on every token), not as the routed rewrite, whose
  // results equal the dense chain's only while every expert output is finite
  bool dense_moe = false;
  rew_mi355x_stats stats{};
  int64_t jit_hits_base = 0;  // jit_cache_hits() when the stats were last reset
  int64_t compiled_base = 0, loaded_base = 0;  // program counters at the last reset
  // device copies of small host constants (dtype, shape and bytes as the
  // key): eager tensors are immutable, so a repeated upload of the same
  // scalar (rew's composites upload eps, 1.0, mask values... every call)
  // shares one storage instead of another H2D copy.  Each entry holds one
  // reference on its storage.
  std::unordered_map<std::string, Storage*> const_cache;
  // pinned staging ring for small host->device copies
  uint8_t* ring = nullptr;
  size_t ring_size = 0, ring_pos = 0;
  // profiling
  bool profiling = false;
  std::vector<ProfEntry> prof;
  std::vector<std::pair<std::string, std::pair<int64_t, double>>> prof_summary;
  std::vector<hipEvent_t> event_pool;
  int order_counter = 0;
  // device address of the static scratch array of the allocation-free
  // entry point on this context's device (null, with the reason, if the
  // lookup at init failed)
  void* noalloc_scratch = nullptr;
  std::string noalloc_error;
  // translated jit modules (stablehlo.cpp), keyed by
  // ordinal::name::cacheKey::hash(text)
  std::unordered_map<std::string, JitModule*> jit_modules;
  // recorded lowerings by graph signature (plan.cpp), oldest first in
  // plan_order; `rec` is set while a flush is being recorded
  bool plan_cache = true;  // REW_MI355X_PLAN_CACHE=0 turns replay off
  std::unordered_map<std::string, FlushPlan*> flush_plans;
  std::deque<std::string> plan_order;
  PlanRecorder* rec = nullptr;
  // set by a jit call that records its module's direct plan: the next flush
  // reports its leaves, nodes and signature here
  FlushCapture* capture = nullptr;
  // bumped by rew_mi355x_clear_cache: direct plans of jit modules recorded
  // before the last clear are dropped on their next use
  uint64_t plan_epoch = 0;
};

// ---- runtime services (runtime.cpp) -----------------------------------------
Tensor* new_tensor(Ctx* c, int dt, const Shape& s);
void tensor_alloc(Tensor* t);                 // give t fresh storage
void storage_release(Storage* s);             // drop one reference
void const_cache_clear(Ctx* c);               // release every cached constant
void tensor_alias(Tensor* t, Tensor* src);    // share src's storage
void tensor_drop_storage(Tensor* t);
void maybe_destroy(Tensor* t);                // free when unreferenced
bool tensor_is_live_handle(const Tensor* t);

// Hooks of the flush-plan recorder (plan.cpp): the tensor services above
// report what they do while a lowering is being recorded (ctx->rec set).
void plan_note_alloc(Tensor* t);               // t just received fresh storage
void plan_note_alias(Tensor* t, Tensor* src);  // t now shares src's storage
void plan_note_drop(Tensor* t);                // t is about to drop its storage
void plan_note_destroy(Tensor* t);             // t is about to be deleted
void plan_note_free(Storage* s);               // s is about to return to the allocator

// Stream-ordered copy of a small host table into device memory (through
// the pinned staging ring; `src` may be reused as soon as this returns).
void upload_async(Ctx* c, void* dst, const void* src, size_t bytes);

// A new tensor (one owner reference) holding a copy of `host`; small
// constants share one device copy per distinct (dtype, shape, bytes).
Tensor* upload_tensor(Ctx* c, int dtype, const Shape& s, const void* host);

// Launch bracketing for profiling: call before/after each kernel launch.
void prof_begin(Ctx* c, const std::string& name);
void prof_end(Ctx* c);

// Enqueues the routed-expert FFN `a` (checked with routed_ffn_check) on the
// context's stream, with `scratch` as its working memory (moe_ffn.hip).
void run_routed_ffn(Ctx* c, const RoutedFfn& a, void* scratch);
// With the context's device current: the device address of the static
// scratch array (moe_ffn.hip), or null with *err set.
void* noalloc_scratch_lookup(std::string* err);

// Jit modules (stablehlo.cpp): runs the StableHLO module `text` over `ins`
// (parsing and translating it on first use) and returns its results, one
// owner reference each; jit_module_cache_clear drops every cached module.
std::vector<Tensor*> jit_module_run(Ctx* c, const std::string& name,
                                    const std::string& cache_key, const char* text,
                                    size_t len, const std::vector<Tensor*>& ins);
void jit_module_cache_clear(Ctx* c);

// ABI-edge error plumbing (runtime.cpp): the thread-local message behind
// rew_mi355x_last_error().
void set_last_error(const std::string& msg);

// Runs f, turning exceptions into an ABI status and the last-error message.
template <class F>
int guarded(F&& f) {
  try {
    f();
    set_last_error(std::string());
    return REW_MI355X_OK;
  } catch (const Error& e) {
    set_last_error(e.what());
    return e.code;
  } catch (const std::bad_alloc&) {
    set_last_error("host out of memory");
    return REW_MI355X_ERR_OOM;
  } catch (const std::exception& e) {
    set_last_error(e.what());
    return REW_MI355X_ERR_INVALID;
  }
}

// ---- graph (ops.cpp / lower.cpp) ----------------------------------------------
// Records op `name` (validating and deriving outputs exactly like
// executeEagerOp); returns new tensors with one owner reference each.
std::vector<Tensor*> record_op(Ctx* c, const std::string& name,
                               const std::vector<Tensor*>& ins,
                               const std::vector<std::pair<std::string, std::string>>& attrs);
void flush(Ctx* c);
// record_op in two halves: prepare_node validates the op against its
// operands' dtypes and shapes and returns the node (typed attributes set,
// no operands attached) with its outputs' dtype and shape; commit_node
// attaches operands, creates the outputs (one owner reference each) and
// queues the node.  The jit path prepares a module's nodes once and
// commits copies of them per call.
Node* prepare_node(Ctx* c, const std::string& op, const std::vector<Tensor*>& ins,
                   const std::vector<std::pair<std::string, std::string>>& attrs,
                   std::vector<std::pair<int, Shape>>* outs);
std::vector<Tensor*> commit_node(Ctx* c, Node* n, const std::vector<Tensor*>& ins,
                                 const std::vector<std::pair<int, Shape>>& outs);

}  // namespace rew
