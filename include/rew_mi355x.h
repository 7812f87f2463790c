/*
 * rew_mi355x.h — C ABI of librew_mi355x.so, the MI355X-native eager backend
 * for rew (bitstormFA/rew v0.2.0).
 *
 * The library replaces the PJRT plugin that rew's eager path drives today.
 * Every entry point below states the reference interface it stands in for
 * (paths relative to the rew repository root).  All calls return an int
 * status (REW_MI355X_OK == 0) and leave a message for
 * rew_mi355x_last_error() on failure; no C++ exception crosses this ABI.
 *
 * Threading: one context per (device ordinal); a context serialises its own
 * calls with a mutex.  The error message is thread-local, like the Nim
 * exception it is turned into.
 *
 * Execution model: rew_mi355x_execute() records the op into the context's
 * deferred op graph and returns immediately with output handles whose
 * shape/dtype are final (derived exactly as eager.nim deriveOutputShapes/
 * DTypes does).  The graph is lowered into fused HIP kernels and launched on
 * the context's stream at the next flush point: rew_mi355x_flush(),
 * rew_mi355x_sync(), rew_mi355x_to_host(), or a pending-graph size limit.
 * rew_mi355x_set_mode(ctx, REW_MI355X_MODE_OP_BY_OP) (or the environment
 * variable REW_MI355X_EAGER_SYNC=1) lowers and launches every op on its own.
 */
#ifndef REW_MI355X_H
#define REW_MI355X_H

#ifndef __HIPCC_RTC__ /* hipRTC (run-time compiled kernels) has these types built in */
#include <stddef.h>
#include <stdint.h>
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define REW_MI355X_ABI_VERSION 3

/* Status codes. */
enum {
  REW_MI355X_OK = 0,
  REW_MI355X_ERR_INVALID = 1,     /* bad argument, shape, dtype or attr      */
  REW_MI355X_ERR_UNSUPPORTED = 2, /* op name / dtype not supported           */
  REW_MI355X_ERR_DEVICE = 3,      /* HIP runtime error                       */
  REW_MI355X_ERR_OOM = 4,         /* device allocation failed                */
  REW_MI355X_ERR_RELEASED = 5     /* use of a handle after its last release  */
};

/* Execution modes (rew_mi355x_set_mode). */
enum {
  REW_MI355X_MODE_DEFERRED = 0, /* record, fuse and launch at flush points */
  REW_MI355X_MODE_OP_BY_OP = 1  /* launch each op as soon as it is recorded */
};

/* Dtype codes follow rew's DType enum order (src/rew/dtype.nim:10-30). */
enum {
  REW_DT_BOOL = 0, REW_DT_INT8 = 1, REW_DT_INT16 = 2, REW_DT_INT32 = 3,
  REW_DT_INT64 = 4, REW_DT_UINT8 = 5, REW_DT_UINT16 = 6, REW_DT_UINT32 = 7,
  REW_DT_UINT64 = 8, REW_DT_FLOAT16 = 9, REW_DT_BFLOAT16 = 10,
  REW_DT_FLOAT32 = 11, REW_DT_FLOAT64 = 12, REW_DT_COMPLEX64 = 13,
  REW_DT_COMPLEX128 = 14, REW_DT_INT4 = 15, REW_DT_UINT4 = 16, REW_DT_NF4 = 17,
  REW_DT_FLOAT8E4M3FN = 18, REW_DT_FLOAT8E5M2 = 19
};

#define REW_MI355X_MAX_RANK 8

typedef struct rew_mi355x_ctx rew_mi355x_ctx; /* one per device ordinal   */
typedef struct rew_mi355x_buf rew_mi355x_buf; /* one per tensor; refcounted */

/* ABI version of the loaded library (compare with REW_MI355X_ABI_VERSION). */
int rew_mi355x_abi_version(void);

/* Message of the last failed call on this thread ("" if none).
 * Replaces: PjrtError text wrapped into EagerError (src/rew/eager.nim:1751-1754). */
const char* rew_mi355x_last_error(void);

/* Number of visible HIP devices.
 * Replaces: PjrtClient.addressableDevices() count (src/rew/eager.nim:175-178). */
int rew_mi355x_device_count(int* out_count);

/* Create (or return the existing) context of device `ordinal`: stream,
 * caching allocator, pinned staging ring, kernel-plan cache.
 * Replaces: ensureClient / loadPlugin (src/rew/eager.nim:119-152,
 * src/rew/pjrt/loader.nim:20-47).  Idempotent per ordinal. */
int rew_mi355x_init(int ordinal, rew_mi355x_ctx** out_ctx);

/* Flush, synchronise and free every cached device block of the context.
 * Handles still alive stay valid until released. */
int rew_mi355x_shutdown(rew_mi355x_ctx* ctx);

/* Copy `nbytes` host bytes into a new device tensor of `dtype`/`shape`.
 * The host buffer may be reused as soon as the call returns
 * (ImmutableUntilTransferDone semantics).  Tensors are immutable, so a
 * tensor of at most 256 bytes whose dtype, shape and bytes match an earlier
 * upload shares that upload's device storage (no copy; the scalars rew's
 * composites upload on every call); rew_mi355x_clear_cache drops them.
 * Replaces: transferToDevice (src/rew/eager.nim:221-235) and through it
 * fromHost[T] / constant (src/rew/eager.nim:360-377, src/rew/ops/literal.nim:56-77). */
int rew_mi355x_from_host(rew_mi355x_ctx* ctx, int dtype, const int64_t* shape,
                         int rank, const void* host, int64_t nbytes,
                         rew_mi355x_buf** out_buf);

/* Blocking copy of a tensor's bytes to host (flushes pending work first).
 * `nbytes` must equal numElements * byteSize(dtype).
 * Replaces: transferToHost / toHost[T] / toHostBytes
 * (src/rew/eager.nim:237-247, 558-595, 635-669). */
int rew_mi355x_to_host(rew_mi355x_buf* buf, void* host, int64_t nbytes);

/* A new tensor of `dtype`/`shape` whose contents are undefined until a
 * caller writes them on the device (through rew_mi355x_buf_device_ptr).
 * Replaces: the uninitialised-buffer slot of the PJRT C API that rew's
 * binding carries (fnClientCreateUninitializedBuffer,
 * src/rew/pjrt/capi.nim:109); the shim's alloc(ctx, bytes, &h). */
int rew_mi355x_alloc(rew_mi355x_ctx* ctx, int dtype, const int64_t* shape, int rank,
                     rew_mi355x_buf** out_buf);

/* Device address of a tensor's storage, valid until its last release.
 * Flushes the tensor's pending producer first.  Only tensors made by
 * rew_mi355x_alloc may be written through it: tensors are otherwise
 * immutable, and small uploads and reshapes share storage.
 * Replaces: PJRT_Buffer_OpaqueDeviceMemoryDataPointer, the slot rew's
 * binding carries (fnBufferOpaqueDeviceMemoryDataPointer,
 * src/rew/pjrt/capi.nim:79). */
int rew_mi355x_buf_device_ptr(rew_mi355x_buf* buf, void** out_ptr);

/* Dtype, rank and shape (up to REW_MI355X_MAX_RANK dims) of a tensor.
 * Replaces: Tensor.dtype / Tensor.shape (src/rew/tensor.nim:42-52). */
int rew_mi355x_buf_meta(const rew_mi355x_buf* buf, int* dtype, int* rank,
                        int64_t* shape);

/* Add one owner reference to a handle. */
int rew_mi355x_retain(rew_mi355x_buf* buf);

/* Drop one owner reference; frees the device memory at the last one.
 * Never fails (errors are swallowed), so it can back a Nim `=destroy`.
 * Replaces: BufferReleaser / pjrtReleaser (src/rew/buffer.nim:33, 69-82;
 * src/rew/eager.nim:113-115; src/rew/pjrt/registry.nim:72-84). */
void rew_mi355x_release(rew_mi355x_buf* buf);

/* Execute one eager op.  `op` is the op name rew's {.rewOp.} procs pass to
 * dispatchEager; `attr_keys`/`attr_vals` are the same stringly-typed attrs
 * in the same wire format ("[1,2]", "@[1, 2]", "float32", "dtInt32",
 * "cpu:0", ...).  On success writes up to `max_outs` new handles (each with
 * one owner reference) and their count.  Errors carry the op name.
 * Replaces: executeEagerOp, the EagerBackend installed by
 * installEagerBackend (src/rew/eager.nim:1717-1772, src/rew/dispatch.nim:47-50, 75-85). */
int rew_mi355x_execute(rew_mi355x_ctx* ctx, const char* op,
                       rew_mi355x_buf* const* operands, int n_operands,
                       const char* const* attr_keys,
                       const char* const* attr_vals, int n_attrs,
                       rew_mi355x_buf** outs, int max_outs, int* n_outs);

/* rew_mi355x_execute that also reports each output's dtype, rank and shape:
 * out_meta[i * (2 + REW_MI355X_MAX_RANK) + {0, 1, 2..}] = dtype, rank, dims.
 * No reference counterpart (rew derives output shapes on the Nim side with
 * deriveOutputShapes, src/rew/eager.nim:1061-1283): a convenience for hosts
 * that would otherwise ask rew_mi355x_buf_meta once per output. */
int rew_mi355x_execute_ex(rew_mi355x_ctx* ctx, const char* op,
                          rew_mi355x_buf* const* operands, int n_operands,
                          const char* const* attr_keys,
                          const char* const* attr_vals, int n_attrs,
                          rew_mi355x_buf** outs, int max_outs, int* n_outs,
                          int64_t* out_meta);

/* Run one jit module: the StableHLO text rew's jit/lazy hand to PJRT
 * (emitText of the traced module with its entry function renamed "main",
 * src/rew/transform/jit.nim:178-185, src/rew/stablehlo/text.nim:1969-2025).
 * The text is parsed and translated once into the graph nodes the eager
 * ops record, cached under ordinal::jit_name::cache_key::hash(text), and
 * instantiated over `inputs` on every call, so its ops join the deferred
 * graph and lower through the same fused kernels.  `text_len` < 0 means
 * NUL-terminated.  Inputs must match the module's argument types;
 * `donate_idx` entries must index `inputs` (the buffers are not reused).
 * Writes one new handle per func.return operand (one owner reference
 * each) and, when `out_meta` is non-null, their dtype/rank/dims as
 * rew_mi355x_execute_ex does.  Modules using an op outside the translated
 * subset fail with REW_MI355X_ERR_UNSUPPORTED naming the op and line.
 * Replaces: executeJit (src/rew/eager.nim:1782-1847): compileWithPersistentCache
 * plus PjrtLoadedExecutable.execute. */
int rew_mi355x_execute_jit(rew_mi355x_ctx* ctx, const char* jit_name,
                           const char* cache_key, const char* module_text,
                           int64_t text_len, rew_mi355x_buf* const* inputs,
                           int n_inputs, const int* donate_idx, int n_donate,
                           rew_mi355x_buf** outs, int max_outs, int* n_outs,
                           int64_t* out_meta);

/* Drop every cached jit module of the context (and its constants).
 * Replaces: clearJitCache (src/rew/eager.nim:1778-1780). */
int rew_mi355x_clear_jit_cache(rew_mi355x_ctx* ctx);

/* Lower and launch every pending op (asynchronous; returns after enqueue).
 * No reference counterpart: the PJRT path executes every op at dispatch
 * (src/rew/eager.nim:1745-1754); this is the deferred-group boundary. */
int rew_mi355x_flush(rew_mi355x_ctx* ctx);

/* Flush, then block until the device has finished all enqueued work.
 * Replaces: the await on PJRT events (src/rew/eager.nim:229-247). */
int rew_mi355x_sync(rew_mi355x_ctx* ctx);

/* REW_MI355X_MODE_DEFERRED or REW_MI355X_MODE_OP_BY_OP.  Switching mode
 * flushes first. */
int rew_mi355x_set_mode(rew_mi355x_ctx* ctx, int mode);

/* Drop the cached small device constants (see rew_mi355x_from_host) and the
 * recorded flush plans (a flushed graph's launches, replayed when the same
 * graph is flushed again); the programs compiled at run time and the
 * caching allocator are kept.
 * Replaces: clearEagerCache (src/rew/eager.nim:1713-1715). */
int rew_mi355x_clear_cache(rew_mi355x_ctx* ctx);

/* Counters of the context since init (or the last reset). */
typedef struct rew_mi355x_stats {
  int64_t ops_recorded;     /* rew_mi355x_execute calls that recorded an op */
  int64_t kernels_launched; /* HIP kernel launches                          */
  int64_t flushes;          /* graph lowerings                              */
  int64_t fused_groups;     /* launches that covered more than one op       */
  int64_t bytes_in_use;     /* device bytes held by live tensors            */
  int64_t bytes_cached;     /* device bytes held by the caching allocator   */
  int64_t plan_cache_hits;  /* launches of a fused program served by its     */
                            /* already compiled kernel (the program cache,  */
                            /* keyed by the program's binary signature; the */
                            /* analogue of rew's executable cache); counted */
                            /* for all contexts of the process since reset  */
  int64_t jit_module_compiles; /* rew_mi355x_execute_jit calls that parsed  */
                               /* and translated a module                   */
  int64_t jit_module_hits;     /* rew_mi355x_execute_jit calls served by a  */
                               /* cached module                             */
  int64_t programs_compiled;   /* fused programs compiled at run time, and  */
  int64_t programs_loaded;     /* those loaded from the persistent cache    */
                               /* (REW_CACHE_DIR; process-wide since reset) */
  int64_t flush_plan_hits;     /* flushes whose graph matched a recorded    */
                               /* lowering and replayed it (no pattern      */
                               /* matching or program building)             */
  int64_t flush_host_ns;       /* host time spent inside flushes: lowering  */
                               /* or replay, plus enqueueing the launches   */
} rew_mi355x_stats;

int rew_mi355x_get_stats(rew_mi355x_ctx* ctx, rew_mi355x_stats* out);
int rew_mi355x_reset_stats(rew_mi355x_ctx* ctx);

/* Kernel timing hooks for the measurement harness.  While profiling is on,
 * every launch is bracketed by HIP events on the context's stream; the
 * per-kernel-name totals are read back after rew_mi355x_sync().
 * Replaces: the PJRT callLocation label "rew:eager:<op>" that external
 * profilers key on (src/rew/eager.nim:1750). */
int rew_mi355x_profile_begin(rew_mi355x_ctx* ctx);
int rew_mi355x_profile_end(rew_mi355x_ctx* ctx);
/* Entry `index` of the last profile: kernel name, launch count and summed
 * device milliseconds.  Returns REW_MI355X_ERR_INVALID past the end. */
int rew_mi355x_profile_entry(rew_mi355x_ctx* ctx, int index, char* name,
                             int name_cap, int64_t* launches, double* total_ms);

/* Native stream of the context (a hipStream_t), for callers that record
 * their own events around the backend's work. */
int rew_mi355x_stream(rew_mi355x_ctx* ctx, void** out_stream);

/* ---- routed mixture-of-experts FFN over caller-owned device rows ---------
 * The routed-expert part of DeepSeekMoE.forward
 * (src/rew/models/deepseek.nim:122-145), given the router's top-k:
 *   out[t] = start[t], then for each of token t's routed experts e in chain
 *   order: out[t] = bf16(out[t] + bf16(f32(E_e(x[t])) * w)),
 *   E_e(x) = down_e(bf16(silu(gate_e(x)) * up_e(x))) with rew's Linear
 *   bias adds and bf16 roundings (src/rew/nn/gated_ffn.nim:46-67),
 * w the token's top-k weight for e.  Exactly the values the backend's
 * deferred graph computes for the dense op chain (its lowering runs these
 * kernels), evaluated only on each expert's routed rows.  All pointers
 * except `expert_ids` and the six weight tables (host arrays of n_experts
 * device pointers) are device addresses; rows are bf16, 16-byte aligned,
 * with strides in elements that are multiples of 8; hidden and ffn are
 * multiples of 8; 1 <= k <= 16; expert ids distinct and in
 * [0, router_width).  Top-k ids outside the chain's experts add nothing.
 * Inputs must be ready on the context's stream (e.g. after
 * rew_mi355x_sync); the work is enqueued on that stream. */
typedef struct rew_mi355x_moe_args {
  const void* x;              /* [tokens, hidden] bf16 tokens                */
  int64_t x_row_stride;
  const void* start;          /* [tokens, hidden] bf16: output before the    */
  int64_t start_row_stride;   /* routed experts (shared experts' sum)        */
  const int32_t* top_ids;     /* [tokens, k] dense                           */
  const float* top_weights;   /* [tokens, k] dense                           */
  int64_t tokens, hidden, ffn;
  int k, router_width, n_experts;
  const int32_t* expert_ids;  /* host [n_experts]: chain order               */
  const void* const* gate_w;  /* host [n_experts] of [hidden, ffn] bf16      */
  const void* const* up_w;    /* host [n_experts] of [hidden, ffn] bf16      */
  const void* const* gate_b;  /* host [n_experts] of [ffn] bf16              */
  const void* const* up_b;    /* host [n_experts] of [ffn] bf16              */
  const void* const* down_w;  /* host [n_experts] of [ffn, hidden] bf16      */
  const void* const* down_b;  /* host [n_experts] of [hidden] bf16           */
  void* out;                  /* [tokens, hidden] bf16, dense                */
} rew_mi355x_moe_args;

/* Enqueues the routed-expert FFN; its working memory (routing tables, the
 * gathered hidden rows and per-slot expert outputs) comes from the
 * context's caching allocator.
 * No reference counterpart: rew reaches this computation only through
 * DeepSeekMoE.forward's op chain (src/rew/models/deepseek.nim:122-145),
 * which rew_mi355x_execute records and lowers to the same kernels; this is
 * the direct form for hosts that already hold the router's top-k. */
int rew_mi355x_moe_routed_ffn(rew_mi355x_ctx* ctx, const rew_mi355x_moe_args* args);

/* rew_mi355x_moe_routed_ffn without any allocation: no hipMalloc / hipFree,
 * no caching-allocator block and no host staging buffer.  Its working memory
 * is a static device array of 64 MiB per GPU (part of this library's code
 * object, held until the process ends); a call needing more (about
 * tokens * k * (hidden + ffn) * 2 bytes) fails with REW_MI355X_ERR_INVALID
 * before anything is launched.  Same arguments and bit-identical results.
 * Every call on one GPU shares that GPU's array, which keeps the last
 * call's contents (no call reads what it has not written first).  Calls
 * are ordered on the context's single stream; work that overlaps a call on
 * the same GPU and uses the array from elsewhere (e.g. a captured copy of
 * these launches replayed on another stream meanwhile) races with it.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory -- code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation. */
int rew_mi355x_moe_routed_ffn_noalloc(rew_mi355x_ctx* ctx, const rew_mi355x_moe_args* args);

/* ---- rew's input generators (host) --------------------------------------
 * Threefry-2x32 with 4 rounds and the Box-Muller / 24-bit uniform samplers,
 * used to build the synthetic inputs every config is quoted on.
 * Replaces: split / foldIn (src/rew/rng.nim:39-80) and uniformF32 /
 * normalF32 (src/rew/nn/init.nim:14-51). */
void rew_mi355x_rng_split(uint32_t key_a, uint32_t key_b, int n,
                          uint32_t* out_pairs /* 2*n */);
void rew_mi355x_rng_fold_in(uint32_t key_a, uint32_t key_b, uint64_t data,
                            uint32_t* out_pair /* 2 */);
void rew_mi355x_rng_uniform_f32(uint32_t key_a, uint32_t key_b, int64_t count,
                                float lo, float hi, float* out);
void rew_mi355x_rng_normal_f32(uint32_t key_a, uint32_t key_b, int64_t count,
                               float mean, float std_dev, float* out);

#ifdef __cplusplus
}
#endif

#endif /* REW_MI355X_H */
