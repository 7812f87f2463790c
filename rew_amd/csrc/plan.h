// Flush plans: the launches and allocations one lowering made, kept per
// graph signature and replayed over new buffers when the same graph is
// flushed again (classification, pattern matching and program building are
// then skipped).
#pragma once

#include <string>
#include <unordered_map>
#include <variant>
#include <vector>

#include "kernels.h"
#include "runtime.h"

namespace rew {

// ---- launches --------------------------------------------------------------------
// The arguments of one enqueued operation of a lowering.  Every device
// pointer a launch reads or writes is a field of these structs, so a
// recorded launch can be re-pointed at another flush's buffers.
struct EwL {
  vm::Program P;
  vm::Space S;
  bool vec;
};
struct ReduceL {
  vm::Program P;
  vm::Space S;
  ReduceArgs A;
  bool vec;
};
struct GemmL {
  std::vector<GemmArgs> g;  // one GEMM, or the segments of a multi-segment launch
  bool multi;
};
struct IndexMapL {
  IndexMapArgs g;
  bool scatter;
};
// The routed experts: RoutedFfn's host tables live here (expert ids, then
// the six per-expert device pointer tables, table j at tab[j * n], and the
// shared experts' after them, table j at tab[6 n + j n_shared]).
struct MoeL {
  RoutedFfn a;
  std::vector<int32_t> expert;
  std::vector<const void*> tab;
  void* scratch;
};
// Stream-ordered fill of `bytes` at dst: a copy of src, or zeros when src
// is null.
struct FillL {
  void* dst;
  const void* src;
  size_t bytes;
};

using LaunchArgs = std::variant<EwL, ReduceL, GemmL, FlashArgs, RowNormArgs, SoftmaxArgs,
                                RopeArgs, GatherArgs, ArgmaxArgs, TopkArgs, SortArgs,
                                IndexMapL, MoeL, FillL, WindowArgs, CholeskyArgs, TriSolveArgs, ComplexArgs, Fft1Args,
                                BatchNormArgs, HeadArgs, RouterArgs>;

struct Launch {
  LaunchArgs args;
  std::string name;    // profile label (built only while profiling)
  bool fused = false;  // counted in fused_groups
};

// Enqueues L on the context's stream inside its profile bracket and counts
// it; while a lowering is being recorded, L is also appended to the
// recording.
void run_launch(Ctx* c, Launch&& L);

// ---- plans -------------------------------------------------------------------------
// A tensor of the flush as the plan names it.
struct PlanRef {
  enum : int8_t { LEAF, NODE, TEMP } kind;
  int32_t idx;  // leaf index / node index / temporary index
  int32_t out;  // output of the node
};

struct PlanEvent {
  enum : int8_t { NEW, ALIAS, DROP, DESTROY, LAUNCH } type;
  PlanRef a{};     // NEW / DROP / DESTROY: the tensor; ALIAS: the new alias
  PlanRef b{};     // ALIAS: the tensor aliased
  int32_t id = 0;  // NEW: storage slot created; LAUNCH: index into launches
};

// A device pointer of a recorded launch: byte `delta` into storage `slot`
// (slot -1: a null pointer).
struct Reloc {
  int32_t slot;
  int64_t delta;
};

struct FlushPlan {
  bool ok = true;  // false: the lowering could not be recorded (lower anew each time)
  int n_slots = 0;
  std::vector<int32_t> leaf_slot_first;  // leaf storage slot -> first leaf holding it
  std::vector<PlanEvent> events;
  std::vector<Launch> launches;
  std::vector<std::vector<Reloc>> relocs;  // per launch, in field-visit order
  std::vector<std::pair<int, Shape>> temps;  // dtype and shape per temporary
};

// Signature of the live nodes of a flush (their kinds, attributes, dtypes,
// shapes, the caller's holds, the wiring between them and what is known of
// every leaf: dtype, shape, host bytes of small constants, which leaves
// share storage).  Fills `leaves` (in first-use order) and `leaf_slot`
// (storage slot per leaf).
std::string flush_signature(Ctx* c, const std::vector<Node*>& nodes,
                            std::vector<Tensor*>* leaves, std::vector<int32_t>* leaf_slot);
// The stored plan for `sig`, or null.
FlushPlan* plan_find(Ctx* c, const std::string& sig);
// Starts recording the lowering of `nodes` into a new plan.
void plan_record_begin(Ctx* c, const std::vector<Node*>& nodes,
                       const std::vector<Tensor*>& leaves, const std::vector<int32_t>& leaf_slot);
// Ends the recording; stores the plan under `sig` when `keep`.
void plan_record_end(Ctx* c, const std::string& sig, bool keep);
// Enqueues plan p's allocations and launches over this flush's tensors.
void plan_replay(Ctx* c, const FlushPlan& p, const std::vector<Node*>& nodes,
                 const std::vector<Tensor*>& leaves);

// What a flush reports to a jit call that records its module's direct plan
// (Ctx::capture): the flush's leaves in signature order, each live node's
// outputs (dtype, shape), where each node output sits as (node, output),
// and the signature under which the flush's plan is stored.
struct FlushCapture {
  bool done = false;
  std::string sig;
  std::vector<Tensor*> leaves;
  std::vector<std::vector<std::pair<int, Shape>>> node_meta;
  std::unordered_map<const Tensor*, std::pair<int32_t, int32_t>> out_ref;
};

// A jit module's lowering replayed without building its graph: the plan of
// the flush that ran the module alone, with each leaf named as a module
// input (>= 0) or constant (-1 - index), each node output's dtype and
// shape, and the module results as (node, output).
struct DirectPlan {
  bool ok = false;  // false: not replayable directly (the graph path runs)
  uint64_t epoch = 0;
  FlushPlan plan;
  std::vector<int32_t> leaf_src;
  std::vector<std::vector<std::pair<int, Shape>>> node_meta;
  std::vector<std::pair<int32_t, int32_t>> results;
};
// Enqueues d's plan over `leaves` (resolved from leaf_src) and returns the
// module results, each holding one owner reference.
std::vector<Tensor*> plan_replay_direct(Ctx* c, const DirectPlan& d,
                                        const std::vector<Tensor*>& leaves);
// Drops every stored plan of the context.
void plan_cache_clear(Ctx* c);

}  // namespace rew
