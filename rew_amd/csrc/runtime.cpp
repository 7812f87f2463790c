// ABI entry points of librew_mi355x: contexts, tensors, transfers, the
// eager execute entry, profiling hooks and rew's input generators.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <mutex>
#include <thread>
#include <unordered_set>

#include "kernels.h"
#include "plan.h"
#include "runtime.h"

namespace rew {

// ---- error plumbing -------------------------------------------------------------

static thread_local std::string g_last_error;

void set_last_error(const std::string& msg) { g_last_error = msg; }

// ---- live handle registry ---------------------------------------------------------

static std::mutex g_reg_mu;
static std::unordered_set<const Tensor*> g_live;
static Ctx* g_ctx[64] = {nullptr};
static std::mutex g_ctx_mu;

bool tensor_is_live_handle(const Tensor* t) {
  std::lock_guard<std::mutex> g(g_reg_mu);
  return g_live.count(t) != 0;
}

static Tensor* check_handle(rew_mi355x_buf* b, const char* what) {
  Tensor* t = reinterpret_cast<Tensor*>(b);
  if (!t) invalid(std::string(what) + ": null tensor handle");
  if (!tensor_is_live_handle(t) || t->ext <= 0)
    fail(REW_MI355X_ERR_RELEASED, std::string(what) + ": use of a released tensor handle");
  return t;
}

// ---- allocator --------------------------------------------------------------------

size_t Allocator::round(size_t bytes) {
  if (bytes == 0) bytes = 1;
  if (bytes <= (1u << 20)) return (bytes + 511) & ~(size_t)511;
  return (bytes + (2u << 20) - 1) & ~(size_t)((2u << 20) - 1);
}

void* Allocator::get(size_t bytes, size_t* rounded) {
  const size_t r = round(bytes);
  auto it = free_blocks.lower_bound(r);
  if (it != free_blocks.end() && it->first <= r + r / 4) {
    void* p = it->second;
    *rounded = it->first;
    cached -= it->first;
    free_blocks.erase(it);
    in_use += *rounded;
    return p;
  }
  if (cap && in_use + cached + r > cap) {
    trim();
    if (in_use + r > cap)
      fail(REW_MI355X_ERR_OOM, "device allocation of " + std::to_string(r) +
                                   " bytes failed on mi355x:" + std::to_string(ordinal) +
                                   " (limit REW_MI355X_MAX_DEVICE_BYTES = " +
                                   std::to_string(cap) + ", " + std::to_string(in_use) +
                                   " bytes in use)");
  }
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, r);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    trim();
    e = hipMalloc(&p, r);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      fail(REW_MI355X_ERR_OOM, "device allocation of " + std::to_string(r) +
                                   " bytes failed on mi355x:" + std::to_string(ordinal));
    }
  }
  *rounded = r;
  in_use += r;
  return p;
}

void Allocator::put(void* p, size_t rounded) {
  in_use -= rounded;
  cached += rounded;
  free_blocks.emplace(rounded, p);
}

void Allocator::trim() {
  for (auto& kv : free_blocks) (void)hipFree(kv.second);
  free_blocks.clear();
  cached = 0;
}

// ---- tensors ------------------------------------------------------------------------

Tensor* new_tensor(Ctx* c, int dt, const Shape& s) {
  Tensor* t = new Tensor();
  t->ctx = c;
  t->dt = dt;
  t->shape = s;
  std::lock_guard<std::mutex> g(g_reg_mu);
  g_live.insert(t);
  return t;
}

void tensor_alloc(Tensor* t) {
  if (t->st) return;
  Storage* s = new Storage();
  s->ctx = t->ctx;
  size_t bytes = (size_t)t->nbytes();
  s->ptr = t->ctx->alloc.get(bytes, &s->bytes);
  s->refs = 1;
  t->st = s;
  if (t->ctx->rec) plan_note_alloc(t);
}

void tensor_alias(Tensor* t, Tensor* src) {
  if (t->st) return;
  t->st = src->st;
  t->st->refs++;
  if (t->ctx->rec) plan_note_alias(t, src);
}

void storage_release(Storage* s) {
  if (s && --s->refs == 0) {
    if (s->ctx->rec) plan_note_free(s);
    s->ctx->alloc.put(s->ptr, s->bytes);
    delete s;
  }
}

void const_cache_clear(Ctx* c) {
  for (auto& kv : c->const_cache) storage_release(kv.second);
  c->const_cache.clear();
}

void tensor_drop_storage(Tensor* t) {
  Storage* s = t->st;
  if (!s) return;
  if (t->ctx->rec) plan_note_drop(t);
  t->st = nullptr;
  if (--s->refs == 0) {
    if (s->ctx->rec) plan_note_free(s);
    s->ctx->alloc.put(s->ptr, s->bytes);
    delete s;
  }
}

void maybe_destroy(Tensor* t) {
  if (t->ext > 0 || t->uses > 0 || t->prod) return;
  tensor_drop_storage(t);
  if (t->ctx->rec) plan_note_destroy(t);
  {
    std::lock_guard<std::mutex> g(g_reg_mu);
    g_live.erase(t);
  }
  delete t;
}

// ---- profiling ------------------------------------------------------------------------

static hipEvent_t take_event(Ctx* c) {
  if (!c->event_pool.empty()) {
    hipEvent_t e = c->event_pool.back();
    c->event_pool.pop_back();
    return e;
  }
  hipEvent_t e;
  REW_HIP(hipEventCreate(&e));
  return e;
}

void prof_begin(Ctx* c, const std::string& name) {
  if (!c->profiling) return;
  ProfEntry e;
  e.name = name;
  e.start = take_event(c);
  e.stop = take_event(c);
  REW_HIP(hipEventRecord(e.start, c->stream));
  c->prof.push_back(e);
}

void prof_end(Ctx* c) {
  if (!c->profiling || c->prof.empty()) return;
  REW_HIP(hipEventRecord(c->prof.back().stop, c->stream));
}

static void prof_collect(Ctx* c) {
  REW_HIP(hipStreamSynchronize(c->stream));
  for (auto& e : c->prof) {
    float ms = 0.f;
    REW_HIP(hipEventElapsedTime(&ms, e.start, e.stop));
    bool found = false;
    for (auto& s : c->prof_summary)
      if (s.first == e.name) {
        s.second.first++;
        s.second.second += ms;
        found = true;
      }
    if (!found) c->prof_summary.push_back({e.name, {1, (double)ms}});
    c->event_pool.push_back(e.start);
    c->event_pool.push_back(e.stop);
  }
  c->prof.clear();
}

// ---- transfers -------------------------------------------------------------------------

static void h2d(Ctx* c, void* dst, const void* src, size_t bytes) {
  if (bytes == 0) return;
  if (bytes <= (64u << 10)) {
    if (!c->ring) {
      c->ring_size = 4u << 20;
      REW_HIP(hipHostMalloc((void**)&c->ring, c->ring_size, hipHostMallocDefault));
    }
    if (c->ring_pos + bytes > c->ring_size) {
      // wrap: earlier copies out of the ring must have completed
      REW_HIP(hipStreamSynchronize(c->stream));
      c->ring_pos = 0;
    }
    uint8_t* slot = c->ring + c->ring_pos;
    std::memcpy(slot, src, bytes);
    c->ring_pos = (c->ring_pos + bytes + 255) & ~(size_t)255;
    REW_HIP(hipMemcpyAsync(dst, slot, bytes, hipMemcpyHostToDevice, c->stream));
    return;
  }
  REW_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream));
  REW_HIP(hipStreamSynchronize(c->stream));
}

void upload_async(Ctx* c, void* dst, const void* src, size_t bytes) { h2d(c, dst, src, bytes); }

// A new tensor (one owner reference) holding `host`'s bytes; small
// constants share one device copy per distinct (dtype, shape, bytes).
// The context's device must be current.
Tensor* upload_tensor(Ctx* c, int dtype, const Shape& s, const void* host) {
  Tensor* t = new_tensor(c, dtype, s);
  const int64_t want = s.numel() * dt_size(dtype);
  const int rank = s.rank;
  const int64_t* shape = s.d;
  // small constants: one device copy per distinct (dtype, shape, bytes)
  constexpr int64_t kConstMax = 256;
  std::string key;
  if (want > 0 && want <= kConstMax) {
    key.reserve(16 + 8 * rank + (size_t)want);
    key.append((const char*)&dtype, sizeof dtype);
    key.append((const char*)&rank, sizeof rank);
    key.append((const char*)shape, sizeof(int64_t) * rank);
    key.append((const char*)host, (size_t)want);
    auto hit = c->const_cache.find(key);
    if (hit != c->const_cache.end()) {
      t->st = hit->second;
      t->st->refs++;
    }
  }
  if (!t->st) {
    try {
      tensor_alloc(t);
      h2d(c, t->data(), host, (size_t)want);
    } catch (...) {
      maybe_destroy(t);
      throw;
    }
    if (!key.empty()) {
      if (c->const_cache.size() >= 4096) const_cache_clear(c);
      t->st->refs++;
      c->const_cache.emplace(key, t->st);
    }
  }
  if (want <= 16 && want > 0) {
    t->has_host = true;
    std::memcpy(t->host, host, (size_t)want);
  }
  t->ext = 1;
  return t;
}

}  // namespace rew

using namespace rew;

// ===================================================================================
// C ABI
// ===================================================================================

struct rew_mi355x_ctx {};
struct rew_mi355x_buf {};

static Ctx* as_ctx(rew_mi355x_ctx* c) {
  if (!c) invalid("null context");
  return reinterpret_cast<Ctx*>(c);
}

extern "C" {

int rew_mi355x_abi_version(void) { return REW_MI355X_ABI_VERSION; }

const char* rew_mi355x_last_error(void) { return g_last_error.c_str(); }

int rew_mi355x_device_count(int* out) {
  return guarded([&] {
    if (!out) invalid("null out_count");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      n = 0;
    }
    *out = n;
  });
}

int rew_mi355x_init(int ordinal, rew_mi355x_ctx** out) {
  return guarded([&] {
    if (!out) invalid("null out_ctx");
    if (ordinal < 0 || ordinal >= 64) invalid("device ordinal out of range");
    std::lock_guard<std::mutex> g(g_ctx_mu);
    if (!g_ctx[ordinal]) {
      int n = 0;
      if (hipGetDeviceCount(&n) != hipSuccess || ordinal >= n) {
        (void)hipGetLastError();
        fail(REW_MI355X_ERR_DEVICE, "mi355x:" + std::to_string(ordinal) +
                                        " not present (" + std::to_string(n) +
                                        " HIP device(s) visible)");
      }
      REW_HIP(hipSetDevice(ordinal));
      Ctx* c = new Ctx();
      c->ordinal = ordinal;
      c->alloc.ordinal = ordinal;
      c->jit_hits_base = jit_cache_hits();
      c->compiled_base = jit_programs_compiled();
      c->loaded_base = jit_programs_loaded();
      REW_HIP(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
      init_silu_table(c->stream);
      REW_HIP(hipStreamSynchronize(c->stream));
      // once per device, with the device current
      c->noalloc_scratch = noalloc_scratch_lookup(&c->noalloc_error);
      if (const char* s = std::getenv("REW_MI355X_EAGER_SYNC"))
        if (s[0] == '1') c->mode = REW_MI355X_MODE_OP_BY_OP;
      if (const char* s = std::getenv("REW_MI355X_NO_PATTERNS"))
        if (s[0] == '1') c->no_fusion_patterns = true;
      if (const char* s = std::getenv("REW_MI355X_PLAN_CACHE"))
        if (s[0] == '0') c->plan_cache = false;
      if (const char* s = std::getenv("REW_MI355X_DENSE_MOE"))
        if (s[0] == '1') c->dense_moe = true;
      if (const char* s = std::getenv("REW_MI355X_MAX_DEVICE_BYTES"))
        c->alloc.cap = (size_t)std::strtoull(s, nullptr, 10);
      g_ctx[ordinal] = c;
    }
    *out = reinterpret_cast<rew_mi355x_ctx*>(g_ctx[ordinal]);
  });
}

int rew_mi355x_shutdown(rew_mi355x_ctx* ctx) {
  return guarded([&] {
    Ctx* c = as_ctx(ctx);
    std::lock_guard<std::recursive_mutex> g(c->mu);
    REW_HIP(hipSetDevice(c->ordinal));
    flush(c);
    REW_HIP(hipStreamSynchronize(c->stream));
    jit_module_cache_clear(c);
    plan_cache_clear(c);
    const_cache_clear(c);
    c->alloc.trim();
  });
}


int rew_mi355x_from_host(rew_mi355x_ctx* ctx, int dtype, const int64_t* shape,
                         int rank, const void* host, int64_t nbytes,
                         rew_mi355x_buf** out) {
  return guarded([&] {
    Ctx* c = as_ctx(ctx);
    if (!out) invalid("from_host: null out_buf");
    if (dtype < 0 || dtype >= kNumDT) invalid("from_host: unknown dtype code");
    if (rank < 0 || rank > kMaxRank) invalid("from_host: rank must be in 0..8");
    std::vector<int64_t> v(shape, shape + rank);
    for (auto d : v)
      if (d < 0) invalid("from_host: negative dimension");
    Shape s(v);
    const int64_t want = s.numel() * dt_size(dtype);
    if (nbytes != want)
      invalid("from_host: byte count " + std::to_string(nbytes) + " does not match " +
              dt_enum_name(dtype) + s.str() + " (" + std::to_string(want) + " bytes)");
    if (want > 0 && !host) invalid("from_host: null host pointer");
    std::lock_guard<std::recursive_mutex> g(c->mu);
    REW_HIP(hipSetDevice(c->ordinal));
    Tensor* t = upload_tensor(c, dtype, s, host);
    *out = reinterpret_cast<rew_mi355x_buf*>(t);
  });
}

int rew_mi355x_to_host(rew_mi355x_buf* buf, void* host, int64_t nbytes) {
  return guarded([&] {
    Tensor* t = check_handle(buf, "to_host");
    Ctx* c = t->ctx;
    std::lock_guard<std::recursive_mutex> g(c->mu);
    REW_HIP(hipSetDevice(c->ordinal));
    if (nbytes != t->nbytes())
      invalid("to_host: byte count " + std::to_string(nbytes) + " does not match " +
              dt_enum_name(t->dt) + t->shape.str() + " (" + std::to_string(t->nbytes()) +
              " bytes)");
    if (t->prod) flush(c);
    if (nbytes == 0) return;
    if (!host) invalid("to_host: null host pointer");
    if (!t->st) invalid("to_host: tensor has no data (an earlier flush failed)");
    REW_HIP(hipMemcpyAsync(host, t->data(), (size_t)nbytes, hipMemcpyDeviceToHost,
                           c->stream));
    REW_HIP(hipStreamSynchronize(c->stream));
  });
}

int rew_mi355x_alloc(rew_mi355x_ctx* ctx, int dtype, const int64_t* shape, int rank,
                     rew_mi355x_buf** out) {
  return guarded([&] {
    Ctx* c = as_ctx(ctx);
    if (!out) invalid("alloc: null out_buf");
    if (dtype < 0 || dtype >= kNumDT) invalid("alloc: unknown dtype code");
    if (rank < 0 || rank > kMaxRank) invalid("alloc: rank must be in 0..8");
    if (rank > 0 && !shape) invalid("alloc: null shape");
    std::vector<int64_t> v(shape, shape + rank);
    for (auto d : v)
      if (d < 0) invalid("alloc: negative dimension");
    Shape s(v);
    std::lock_guard<std::recursive_mutex> g(c->mu);
    REW_HIP(hipSetDevice(c->ordinal));
    Tensor* t = new_tensor(c, dtype, s);
    try {
      tensor_alloc(t);
    } catch (...) {
      maybe_destroy(t);
      throw;
    }
    t->ext = 1;
    *out = reinterpret_cast<rew_mi355x_buf*>(t);
  });
}

int rew_mi355x_buf_device_ptr(rew_mi355x_buf* buf, void** out_ptr) {
  return guarded([&] {
    Tensor* t = check_handle(buf, "buf_device_ptr");
    if (!out_ptr) invalid("buf_device_ptr: null out_ptr");
    Ctx* c = t->ctx;
    std::lock_guard<std::recursive_mutex> g(c->mu);
    REW_HIP(hipSetDevice(c->ordinal));
    if (t->prod) flush(c);
    if (!t->st) invalid("buf_device_ptr: tensor has no data (an earlier flush failed)");
    *out_ptr = t->data();
  });
}

int rew_mi355x_buf_meta(const rew_mi355x_buf* buf, int* dtype, int* rank,
                        int64_t* shape) {
  return guarded([&] {
    const Tensor* t = check_handle(const_cast<rew_mi355x_buf*>(buf), "buf_meta");
    if (dtype) *dtype = t->dt;
    if (rank) *rank = t->shape.rank;
    if (shape)
      for (int i = 0; i < t->shape.rank; ++i) shape[i] = t->shape.d[i];
  });
}

int rew_mi355x_retain(rew_mi355x_buf* buf) {
  return guarded([&] {
    Tensor* t = check_handle(buf, "retain");
    std::lock_guard<std::recursive_mutex> g(t->ctx->mu);
    t->ext++;
  });
}

void rew_mi355x_release(rew_mi355x_buf* buf) {
  Tensor* t = reinterpret_cast<Tensor*>(buf);
  if (!t || !tensor_is_live_handle(t) || t->ext <= 0) return;
  try {
    Ctx* c = t->ctx;
    std::lock_guard<std::recursive_mutex> g(c->mu);
    t->ext--;
    maybe_destroy(t);
  } catch (...) {
  }
}

static int execute_impl(rew_mi355x_ctx* ctx, const char* op,
                        rew_mi355x_buf* const* operands, int n_operands,
                        const char* const* keys, const char* const* vals, int n_attrs,
                        rew_mi355x_buf** outs, int max_outs, int* n_outs, int64_t* meta) {
  return guarded([&] {
    Ctx* c = as_ctx(ctx);
    if (!op) invalid("execute: null op name");
    if (n_operands < 0 || (n_operands > 0 && !operands))
      invalid(std::string("eager '") + op + "': bad operand array");
    if (n_attrs < 0 || (n_attrs > 0 && (!keys || !vals)))
      invalid(std::string("eager '") + op + "': bad attr arrays");
    std::vector<Tensor*> ins;
    ins.reserve(n_operands);
    for (int i = 0; i < n_operands; ++i) {
      Tensor* t = reinterpret_cast<Tensor*>(operands[i]);
      if (!t || !tensor_is_live_handle(t) || t->ext <= 0)
        ins.push_back(check_handle(operands[i], (std::string("eager '") + op + "'").c_str()));
      else
        ins.push_back(t);
    }
    std::vector<std::pair<std::string, std::string>> attrs;
    attrs.reserve(n_attrs);
    for (int i = 0; i < n_attrs; ++i) {
      if (!keys[i] || !vals[i]) invalid(std::string("eager '") + op + "': null attr");
      attrs.emplace_back(keys[i], vals[i]);
    }
    std::lock_guard<std::recursive_mutex> g(c->mu);
    REW_HIP(hipSetDevice(c->ordinal));
    std::vector<Tensor*> res = record_op(c, op, ins, attrs);
    if ((int)res.size() > max_outs || !outs) {
      for (Tensor* t : res) {
        t->ext--;
        maybe_destroy(t);
      }
      invalid(std::string("eager '") + op + "': op produces " + std::to_string(res.size()) +
              " output(s), caller has room for " + std::to_string(max_outs));
    }
    for (size_t i = 0; i < res.size(); ++i) {
      outs[i] = reinterpret_cast<rew_mi355x_buf*>(res[i]);
      if (meta) {
        int64_t* m = meta + i * (2 + REW_MI355X_MAX_RANK);
        m[0] = res[i]->dt;
        m[1] = res[i]->shape.rank;
        for (int k = 0; k < res[i]->shape.rank; ++k) m[2 + k] = res[i]->shape.d[k];
      }
    }
    if (n_outs) *n_outs = (int)res.size();
  });
}

int rew_mi355x_execute(rew_mi355x_ctx* ctx, const char* op,
                       rew_mi355x_buf* const* operands, int n_operands,
                       const char* const* keys, const char* const* vals, int n_attrs,
                       rew_mi355x_buf** outs, int max_outs, int* n_outs) {
  return execute_impl(ctx, op, operands, n_operands, keys, vals, n_attrs, outs, max_outs, n_outs,
                      nullptr);
}

int rew_mi355x_execute_ex(rew_mi355x_ctx* ctx, const char* op,
                          rew_mi355x_buf* const* operands, int n_operands,
                          const char* const* keys, const char* const* vals, int n_attrs,
                          rew_mi355x_buf** outs, int max_outs, int* n_outs, int64_t* out_meta) {
  return execute_impl(ctx, op, operands, n_operands, keys, vals, n_attrs, outs, max_outs, n_outs,
                      out_meta);
}

int rew_mi355x_execute_jit(rew_mi355x_ctx* ctx, const char* jit_name, const char* cache_key,
                           const char* module_text, int64_t text_len,
                           rew_mi355x_buf* const* inputs, int n_inputs, const int* donate_idx,
                           int n_donate, rew_mi355x_buf** outs, int max_outs, int* n_outs,
                           int64_t* out_meta) {
  return guarded([&] {
    Ctx* c = as_ctx(ctx);
    const std::string name = jit_name ? jit_name : "";
    const std::string who = "jit '" + name + "'";
    if (!module_text) invalid(who + ": null module text");
    if (n_inputs <= 0 || !inputs) invalid(who + ": zero inputs");
    if (n_donate < 0 || (n_donate > 0 && !donate_idx)) invalid(who + ": bad donation array");
    for (int i = 0; i < n_donate; ++i)
      if (donate_idx[i] < 0 || donate_idx[i] >= n_inputs)
        invalid(who + ": donation index " + std::to_string(donate_idx[i]) + " out of range");
    std::vector<Tensor*> ins;
    ins.reserve(n_inputs);
    for (int i = 0; i < n_inputs; ++i) {
      Tensor* t = check_handle(inputs[i], who.c_str());
      if (t->ctx != c) invalid(who + ": cross-device inputs forbidden");
      ins.push_back(t);
    }
    const size_t len = text_len < 0 ? std::strlen(module_text) : (size_t)text_len;
    std::lock_guard<std::recursive_mutex> g(c->mu);
    REW_HIP(hipSetDevice(c->ordinal));
    std::vector<Tensor*> res =
        jit_module_run(c, name, cache_key ? cache_key : "", module_text, len, ins);
    if ((int)res.size() > max_outs || !outs) {
      for (Tensor* t : res) {
        t->ext--;
        maybe_destroy(t);
      }
      invalid(who + ": module returns " + std::to_string(res.size()) +
              " value(s), caller has room for " + std::to_string(max_outs));
    }
    for (size_t i = 0; i < res.size(); ++i) {
      outs[i] = reinterpret_cast<rew_mi355x_buf*>(res[i]);
      if (out_meta) {
        int64_t* m = out_meta + i * (2 + REW_MI355X_MAX_RANK);
        m[0] = res[i]->dt;
        m[1] = res[i]->shape.rank;
        for (int k = 0; k < res[i]->shape.rank; ++k) m[2 + k] = res[i]->shape.d[k];
      }
    }
    if (n_outs) *n_outs = (int)res.size();
  });
}

int rew_mi355x_clear_jit_cache(rew_mi355x_ctx* ctx) {
  return guarded([&] {
    Ctx* c = as_ctx(ctx);
    std::lock_guard<std::recursive_mutex> g(c->mu);
    REW_HIP(hipSetDevice(c->ordinal));
    jit_module_cache_clear(c);
  });
}

int rew_mi355x_flush(rew_mi355x_ctx* ctx) {
  return guarded([&] {
    Ctx* c = as_ctx(ctx);
    std::lock_guard<std::recursive_mutex> g(c->mu);
    REW_HIP(hipSetDevice(c->ordinal));
    flush(c);
  });
}

int rew_mi355x_sync(rew_mi355x_ctx* ctx) {
  return guarded([&] {
    Ctx* c = as_ctx(ctx);
    std::lock_guard<std::recursive_mutex> g(c->mu);
    REW_HIP(hipSetDevice(c->ordinal));
    flush(c);
    REW_HIP(hipStreamSynchronize(c->stream));
  });
}

int rew_mi355x_set_mode(rew_mi355x_ctx* ctx, int mode) {
  return guarded([&] {
    Ctx* c = as_ctx(ctx);
    if (mode != REW_MI355X_MODE_DEFERRED && mode != REW_MI355X_MODE_OP_BY_OP)
      invalid("set_mode: unknown mode " + std::to_string(mode));
    std::lock_guard<std::recursive_mutex> g(c->mu);
    REW_HIP(hipSetDevice(c->ordinal));
    flush(c);
    c->mode = mode;
  });
}

int rew_mi355x_clear_cache(rew_mi355x_ctx* ctx) {
  return guarded([&] {
    Ctx* c = as_ctx(ctx);
    std::lock_guard<std::recursive_mutex> g(c->mu);
    // The cached small constants are dropped (their storage returns to the
    // allocator once no tensor uses it), and so are the recorded flush plans.
    const_cache_clear(c);
    plan_cache_clear(c);
    c->plan_epoch++;  // and the jit modules' direct plans
  });
}

int rew_mi355x_get_stats(rew_mi355x_ctx* ctx, rew_mi355x_stats* out) {
  return guarded([&] {
    Ctx* c = as_ctx(ctx);
    if (!out) invalid("get_stats: null out");
    std::lock_guard<std::recursive_mutex> g(c->mu);
    c->stats.bytes_in_use = (int64_t)c->alloc.in_use;
    c->stats.bytes_cached = (int64_t)c->alloc.cached;
    c->stats.plan_cache_hits = jit_cache_hits() - c->jit_hits_base;
    c->stats.programs_compiled = jit_programs_compiled() - c->compiled_base;
    c->stats.programs_loaded = jit_programs_loaded() - c->loaded_base;
    *out = c->stats;
  });
}

int rew_mi355x_reset_stats(rew_mi355x_ctx* ctx) {
  return guarded([&] {
    Ctx* c = as_ctx(ctx);
    std::lock_guard<std::recursive_mutex> g(c->mu);
    c->stats = rew_mi355x_stats{};
    c->jit_hits_base = jit_cache_hits();
    c->compiled_base = jit_programs_compiled();
    c->loaded_base = jit_programs_loaded();
  });
}

int rew_mi355x_profile_begin(rew_mi355x_ctx* ctx) {
  return guarded([&] {
    Ctx* c = as_ctx(ctx);
    std::lock_guard<std::recursive_mutex> g(c->mu);
    REW_HIP(hipSetDevice(c->ordinal));
    flush(c);
    prof_collect(c);
    c->prof_summary.clear();
    c->profiling = true;
  });
}

int rew_mi355x_profile_end(rew_mi355x_ctx* ctx) {
  return guarded([&] {
    Ctx* c = as_ctx(ctx);
    std::lock_guard<std::recursive_mutex> g(c->mu);
    REW_HIP(hipSetDevice(c->ordinal));
    flush(c);
    c->profiling = false;
    prof_collect(c);
  });
}

int rew_mi355x_profile_entry(rew_mi355x_ctx* ctx, int index, char* name, int name_cap,
                             int64_t* launches, double* total_ms) {
  return guarded([&] {
    Ctx* c = as_ctx(ctx);
    std::lock_guard<std::recursive_mutex> g(c->mu);
    if (index < 0 || index >= (int)c->prof_summary.size())
      invalid("profile_entry: index past the end");
    auto& e = c->prof_summary[index];
    if (name && name_cap > 0) {
      std::snprintf(name, (size_t)name_cap, "%s", e.first.c_str());
    }
    if (launches) *launches = e.second.first;
    if (total_ms) *total_ms = e.second.second;
  });
}

int rew_mi355x_stream(rew_mi355x_ctx* ctx, void** out) {
  return guarded([&] {
    Ctx* c = as_ctx(ctx);
    if (!out) invalid("stream: null out");
    *out = (void*)c->stream;
  });
}

}  // extern "C"

// ---- rew's generators (src/rew/rng.nim:32-80, src/rew/nn/init.nim:14-51) ------------

static inline uint32_t rotl32(uint32_t x, uint32_t r) { return (x << r) | (x >> (32u - r)); }

// Four-round Threefry-2x32 as rew defines it (src/rew/rng.nim:39-55).
static inline void threefry4(uint32_t k0, uint32_t k1, uint32_t c0, uint32_t c1,
                             uint32_t* o0, uint32_t* o1) {
  static const uint32_t rot[4] = {13u, 15u, 26u, 6u};
  const uint32_t k2 = k0 ^ k1 ^ 0x1BD11BDAu;
  uint32_t x0 = c0 + k0, x1 = c1 + k1;
  for (int r = 0; r < 4; ++r) {
    x0 += x1;
    x1 = rotl32(x1, rot[r]);
    x1 ^= x0;
  }
  *o0 = x0 + k1;
  *o1 = x1 + k2 + 1u;
}

static inline float u32_unit(uint32_t x) { return (float)(x >> 8) * (1.0f / 16777216.0f); }

// Splits [0, n) over the host cores; every index is computed independently,
// so the result does not depend on the thread count.
template <class F>
static void parallel_for(int64_t n, F&& f) {
  unsigned nt = std::thread::hardware_concurrency();
  if (nt == 0) nt = 1;
  if (nt > 32) nt = 32;
  if (n < 65536 || nt == 1) {
    for (int64_t i = 0; i < n; ++i) f(i);
    return;
  }
  std::vector<std::thread> th;
  const int64_t chunk = (n + nt - 1) / nt;
  for (unsigned t = 0; t < nt; ++t) {
    const int64_t b = (int64_t)t * chunk, e = std::min<int64_t>(n, b + chunk);
    if (b >= e) break;
    th.emplace_back([&f, b, e] {
      for (int64_t i = b; i < e; ++i) f(i);
    });
  }
  for (auto& x : th) x.join();
}

extern "C" {

void rew_mi355x_rng_split(uint32_t ka, uint32_t kb, int n, uint32_t* out) {
  for (int i = 0; i < n; ++i) threefry4(ka, kb, (uint32_t)i, 0u, &out[2 * i], &out[2 * i + 1]);
}

void rew_mi355x_rng_fold_in(uint32_t ka, uint32_t kb, uint64_t data, uint32_t* out) {
  threefry4(ka, kb, (uint32_t)(data & 0xffffffffu), (uint32_t)(data >> 32), &out[0], &out[1]);
}

void rew_mi355x_rng_uniform_f32(uint32_t ka, uint32_t kb, int64_t count, float lo,
                                float hi, float* out) {
  const float scale = hi - lo;
  parallel_for(count, [&](int64_t i) {
    uint32_t a, b;
    threefry4(ka, kb, (uint32_t)((uint64_t)i & 0xffffffffu), (uint32_t)((uint64_t)i >> 32), &a, &b);
    out[i] = lo + scale * u32_unit(a);
  });
}

void rew_mi355x_rng_normal_f32(uint32_t ka, uint32_t kb, int64_t count, float mean,
                               float std_dev, float* out) {
  const int64_t pairs = (count + 1) / 2;
  const float two_pi = 2.0f * (float)M_PI;
  parallel_for(pairs, [&](int64_t i) {
    uint32_t a1, b1, a2, b2;
    const uint64_t j1 = (uint64_t)(2 * i), j2 = (uint64_t)(2 * i + 1);
    threefry4(ka, kb, (uint32_t)(j1 & 0xffffffffu), (uint32_t)(j1 >> 32), &a1, &b1);
    threefry4(ka, kb, (uint32_t)(j2 & 0xffffffffu), (uint32_t)(j2 >> 32), &a2, &b2);
    float u1 = u32_unit(a1), u2 = u32_unit(a2);
    float su1 = u1 > 1e-10f ? u1 : 1e-10f;
    float r = sqrtf(-2.0f * logf(su1));
    float th = two_pi * u2;
    out[2 * i] = mean + std_dev * (r * cosf(th));
    if (2 * i + 1 < count) out[2 * i + 1] = mean + std_dev * (r * sinf(th));
  });
}

}  // extern "C"
