// Run-time compiled kernels for fused elementwise programs and reductions.
//
// A vm::Program is interpreted by ew_kernel / reduce_rows_kernel: every
// instruction is decoded per element group, which bounds those kernels by
// instruction issue rather than by HBM.  Here the same program is turned
// into straight-line HIP source -- one statement per instruction, calling
// the interpreter's own op / leaf / store helpers (vm_device.h) with
// compile-time constant arguments, so the semantics are shared, not
// re-implemented -- and compiled once per program signature with hipRTC
// for gfx950.  Tensor addresses are the only run-time arguments, so a plan
// re-used on new buffers hits the cache.  This is the native counterpart of
// rew's per-signature executable cache (src/rew/eager.nim:1557-1680).
//
// REW_MI355X_JIT=0 keeps every program on the interpreter.  A program that
// fails to compile falls back to the interpreter as well (reported once).
#include <dlfcn.h>
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <atomic>
#include <mutex>
#include <sstream>
#include <string>
#include <unordered_map>

#include "kernels.h"
#include "runtime.h"

namespace rew {

namespace {

struct JitFn {
  hipModule_t mod = nullptr;
  hipFunction_t fn = nullptr;
  bool failed = false;
};

std::mutex g_jit_mu;
std::atomic<int64_t> g_jit_hits{0};  // launches served by an already compiled program
std::unordered_map<std::string, JitFn> g_jit;  // key: device ordinal + source

// REW_MI355X_NT=1: nontemporal vector loads / stores in the compiled
// elementwise and reduction kernels
bool stream_nt() {
  static const bool on = [] {
    const char* s = std::getenv("REW_MI355X_NT");
    return s && s[0] == '1';
  }();
  return on;
}

bool jit_enabled() {
  static const bool on = [] {
    const char* s = std::getenv("REW_MI355X_JIT");
    return !(s && s[0] == '0');
  }();
  return on;
}

// REW_MI355X_JIT=strict: a program that fails to compile is an error
// instead of an interpreter fallback (tests use it).
bool jit_strict() {
  static const bool on = [] {
    const char* s = std::getenv("REW_MI355X_JIT");
    return s && std::string(s) == "strict";
  }();
  return on;
}

// Directory of this library's sources: <package>/csrc next to the .so.
std::string src_dir() {
  static const std::string dir = [] {
    Dl_info info;
    if (dladdr((void*)&src_dir, &info) && info.dli_fname) {
      std::string f = info.dli_fname;
      const size_t cut = f.rfind('/');
      if (cut != std::string::npos) return f.substr(0, cut) + "/csrc";
    }
    return std::string("csrc");
  }();
  return dir;
}

// Binary signature of a launch: everything the generated source depends on
// (the program without its pointers, the space, the kind and its constants).
std::string signature(const vm::Program& P, const vm::Space& S, int kind, int V,
                      const ReduceArgs* A) {
  std::string k;
  int dev = 0;
  REW_HIP(hipGetDevice(&dev));
  auto put = [&](const void* p, size_t n) { k.append((const char*)p, n); };
  put(&dev, sizeof dev);
  put(&kind, sizeof kind);
  put(&V, sizeof V);
  put(&P.n_ins, sizeof P.n_ins);
  put(&P.n_leaves, sizeof P.n_leaves);
  put(&P.n_outs, sizeof P.n_outs);
  put(P.ins, sizeof(vm::Ins) * P.n_ins);
  // field by field: struct padding is never part of the key
  for (int i = 0; i < P.n_leaves; ++i) {
    const vm::Leaf& L = P.leaf[i];
    put(&L.dtype, 1);
    put(&L.mode, 1);
    put(&L.vrank, 1);
    put(&L.off, sizeof L.off);
    put(&L.clamp_hi, sizeof L.clamp_hi);
    put(L.stride, sizeof L.stride);
    put(L.vdim, sizeof L.vdim);
  }
  for (int q = 0; q < P.n_outs; ++q) {
    const vm::Out& O = P.out[q];
    put(&O.dtype, 1);
    put(&O.reg, 1);
    put(&O.off, sizeof O.off);
  }
  put(&S.rank, sizeof S.rank);
  put(&S.numel, sizeof S.numel);
  put(S.dim, sizeof(vm::FastDiv) * S.rank);
  if (A) {
    put(&A->op, sizeof A->op);
    put(&A->n_out, sizeof A->n_out);
    put(&A->n_red, sizeof A->n_red);
    put(&A->out_dtype, sizeof A->out_dtype);
    put(&A->n_extra, sizeof A->n_extra);
    put(A->extra_op, sizeof(int) * A->n_extra);
  }
  return k;
}

// Kernel of `key`; `make_src` is called (and the source compiled) only on a
// miss.
template <typename F>
JitFn* get_fn(const std::string& key, F make_src, const char* entry) {
  std::lock_guard<std::mutex> g(g_jit_mu);
  auto it = g_jit.find(key);
  if (it != g_jit.end()) {
    if (it->second.failed) return nullptr;
    g_jit_hits.fetch_add(1, std::memory_order_relaxed);
    return &it->second;
  }
  JitFn& f = g_jit[key];
  const std::string src = make_src();
  hiprtcProgram prog;
  if (hiprtcCreateProgram(&prog, src.c_str(), "rew_jit.hip", 0, nullptr, nullptr) !=
      HIPRTC_SUCCESS) {
    f.failed = true;
    return nullptr;
  }
  const std::string inc = "-I" + src_dir();
  const char* opts[] = {"--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off",
                        inc.c_str(), "-Xclang", "-target-feature", "-Xclang",
                        "-packed-fp32-ops"};
  const hiprtcResult rc = hiprtcCompileProgram(prog, (int)(sizeof opts / sizeof opts[0]), opts);
  if (rc != HIPRTC_SUCCESS) {
    size_t n = 0;
    hiprtcGetProgramLogSize(prog, &n);
    std::string log(n, '\0');
    if (n) hiprtcGetProgramLog(prog, &log[0]);
    if (jit_strict()) {
      hiprtcDestroyProgram(&prog);
      g_jit.erase(key);
      fail(REW_MI355X_ERR_DEVICE, "run-time kernel compile failed: " + log.substr(0, 4000));
    }
    static bool reported = false;
    if (!reported) {
      std::fprintf(stderr, "[rew_mi355x] run-time kernel compile failed (interpreter used): %s\n",
                   log.substr(0, 2000).c_str());
      reported = true;
    }
    hiprtcDestroyProgram(&prog);
    f.failed = true;
    return nullptr;
  }
  size_t n = 0;
  hiprtcGetCodeSize(prog, &n);
  std::string code(n, '\0');
  hiprtcGetCode(prog, &code[0]);
  hiprtcDestroyProgram(&prog);
  if (hipModuleLoadData(&f.mod, code.data()) != hipSuccess ||
      hipModuleGetFunction(&f.fn, f.mod, entry) != hipSuccess) {
    (void)hipGetLastError();
    f.failed = true;
    return nullptr;
  }
  return &f;
}

// ---- source generation ---------------------------------------------------------------

// the interpreter's arity rule (vm_device.h op_arity)
int arity(int op) {
  using namespace vm;
  if (op <= OP_IOTA) return 0;
  if (op >= OP_SELECT && op <= OP_CLAMPU) return 3;
  if ((op >= OP_ADDF && op <= OP_SHRL) || (op >= OP_CMPF && op <= OP_CMPU)) return 2;
  return 1;
}

void put_space(std::ostringstream& o, const vm::Space& S) {
  o << "  Space S; S.rank = " << S.rank << "; S.numel = " << S.numel << "ll;\n";
  for (int k = 0; k < S.rank; ++k)
    o << "  S.dim[" << k << "].d = " << S.dim[k].d << "u; S.dim[" << k << "].m = " << S.dim[k].m
      << "u; S.dim[" << k << "].s = " << S.dim[k].s << "u;\n";
}

void put_leaves(std::ostringstream& o, const vm::Program& P) {
  for (int i = 0; i < P.n_leaves; ++i) {
    const vm::Leaf& L = P.leaf[i];
    o << "  Leaf L" << i << "; L" << i << ".ptr = p" << i << "; L" << i
      << ".dtype = " << (int)L.dtype << "; L" << i << ".mode = " << (int)L.mode << "; L" << i
      << ".vrank = " << (int)L.vrank << "; L" << i << ".off = " << L.off << "; L" << i
      << ".clamp_hi = " << L.clamp_hi << ";\n";
    for (int k = 0; k < vm::kRank; ++k)
      o << "  L" << i << ".stride[" << k << "] = " << L.stride[k] << "; L" << i << ".vdim[" << k
        << "].d = " << L.vdim[k].d << "u; L" << i << ".vdim[" << k << "].m = " << L.vdim[k].m
        << "u; L" << i << ".vdim[" << k << "].s = " << L.vdim[k].s << "u;\n";
  }
}

// Straight-line body: each instruction a fresh array; register numbers of
// the (register-allocated) program map to the latest writer.
void put_body(std::ostringstream& o, const vm::Program& P, int V, const char* sfx,
              std::string* reg_of_out, const char* lin, const char* coord) {
  std::string reg[vm::kMaxRegs];
  for (int pc = 0; pc < P.n_ins; ++pc) {
    const vm::Ins& I = P.ins[pc];
    const std::string d = std::string("v") + std::to_string(pc) + sfx;
    o << "    uint32_t " << d << "[" << V << "];\n";
    const int ar = arity(I.op);
    if (ar == 0) {
      if (I.op == vm::OP_LOAD)
        o << "    leaf_load<" << V << ">(L" << I.imm << ", S.rank, " << coord << ", " << lin << ", "
          << d << ");\n";
      else if (I.op == vm::OP_CONST)
        o << "    for (int j = 0; j < " << V << "; ++j) " << d << "[j] = " << I.imm << "u;\n";
      else
        o << "    leaf_iota<" << V << ">(L" << I.imm << ", S.rank, " << coord << ", " << lin
          << ", " << d << ");\n";
    } else if (ar == 1) {
      o << "    for (int j = 0; j < " << V << "; ++j) " << d << "[j] = op1(" << (int)I.op << ", "
        << reg[I.a] << "[j]);\n";
    } else if (ar == 2) {
      o << "    for (int j = 0; j < " << V << "; ++j) " << d << "[j] = op2(" << (int)I.op << ", "
        << (int)I.aux << ", " << reg[I.a] << "[j], " << reg[I.b] << "[j]);\n";
    } else {
      o << "    for (int j = 0; j < " << V << "; ++j) " << d << "[j] = op3(" << (int)I.op << ", "
        << reg[I.a] << "[j], " << reg[I.b] << "[j], " << reg[I.c] << "[j]);\n";
    }
    reg[I.dst] = d;
  }
  for (int q = 0; q < P.n_outs; ++q) reg_of_out[q] = reg[P.out[q].reg];
}

std::string params(const vm::Program& P, bool outs) {
  std::ostringstream o;
  for (int i = 0; i < P.n_leaves; ++i) o << (i ? ", " : "") << "const void* p" << i;
  if (outs)
    for (int q = 0; q < P.n_outs; ++q) o << (P.n_leaves || q ? ", " : "") << "void* q" << q;
  return o.str();
}

constexpr int kUnroll = 4;  // vectors per thread per grid-stride step

// One V-vector per thread over a grid that covers the whole space: on
// MI355X a full grid of short-lived waves streams HBM faster (6.2 TB/s on a
// 1 GiB copy) than a capped grid of threads looping over several vectors
// (4.7 TB/s).
std::string gen_ew(const vm::Program& P, const vm::Space& S, int V) {
  std::ostringstream o;
  o << "#define REW_VM_NT " << (stream_nt() ? 1 : 0) << "\n#include \"vm_device.h\"\nusing namespace rew::vm;\n";
  o << "extern \"C\" __global__ void __launch_bounds__(256) rew_ew(" << params(P, true) << ") {\n";
  put_space(o, S);
  put_leaves(o, P);
  const int64_t nvec = S.numel / V;
  o << "  const uint32_t t = blockIdx.x * 256u + threadIdx.x;\n";
  o << "  if (t >= " << nvec << "u) return;\n";
  o << "  const uint32_t lin = t * " << V << "u;\n";
  o << "  int32_t c[kRank]; delinearize(S, lin, c);\n";
  std::string outs[vm::kMaxOuts];
  put_body(o, P, V, "", outs, "lin", "c");
  for (int q = 0; q < P.n_outs; ++q)
    o << "  store_vec<" << V << ">(q" << q << ", " << (int)P.out[q].dtype << ", (int64_t)"
      << P.out[q].off << " + lin, " << outs[q] << ");\n";
  o << "}\n";
  return o.str();
}

std::string gen_reduce(const vm::Program& P, const vm::Space& S, const ReduceArgs& A, int V) {
  std::ostringstream o;
  o << "#define REW_VM_NT " << (stream_nt() ? 1 : 0) << "\n#include \"vm_device.h\"\nusing namespace rew::vm;\n";
  o << "__device__ __forceinline__ uint32_t red_init_j(int op) {\n"
       "  switch (op) {\n"
       "    case 0: return as_u(0.0f);\n    case 1: return as_u(-__builtin_inff());\n"
       "    case 2: return as_u(__builtin_inff());\n    case 3: return as_u(1.0f);\n"
       "    case 4: return 1u;\n    case 5: return 0u;\n    case 6: return 0x80000000u;\n"
       "    default: return 0x7fffffffu;\n  }\n}\n";
  o << "__device__ __forceinline__ uint32_t red_op_j(int op, uint32_t a, uint32_t b) {\n"
       "  switch (op) {\n"
       "    case 0: return as_u(as_f(a) + as_f(b));\n"
       "    case 1: return as_u(fmax_prop(as_f(a), as_f(b)));\n"
       "    case 2: return as_u(fmin_prop(as_f(a), as_f(b)));\n"
       "    case 3: return as_u(as_f(a) * as_f(b));\n"
       "    case 4: return (a != 0u) & (b != 0u);\n"
       "    case 5: return (a != 0u) | (b != 0u);\n"
       "    case 6: return (int32_t)a > (int32_t)b ? a : b;\n"
       "    default: return (int32_t)a < (int32_t)b ? a : b;\n  }\n}\n";
  const int n_acc = 1 + A.n_extra;
  o << "extern \"C\" __global__ void __launch_bounds__(256) rew_reduce(" << params(P, false)
    << (P.n_leaves ? ", " : "") << "void* out";
  for (int x = 0; x < A.n_extra; ++x) o << ", void* out" << x + 1;
  o << ") {\n";
  put_space(o, S);
  put_leaves(o, P);
  o << "  const int op = " << A.op << ";\n";
  for (int x = 0; x < A.n_extra; ++x) o << "  const int op" << x + 1 << " = " << A.extra_op[x] << ";\n";
  // one accumulator per op, each updated in the same element order: `stmt`
  // with @ -> the accumulator's suffix and % -> its op
  auto accs = [&](const std::string& stmt) {
    std::string all;
    for (int x = 0; x < n_acc; ++x) {
      std::string t = stmt;
      const std::string suf = x ? std::to_string(x) : "";
      for (size_t p; (p = t.find('@')) != std::string::npos;) t.replace(p, 1, suf);
      for (size_t p; (p = t.find('%')) != std::string::npos;) t.replace(p, 1, "op" + suf);
      all += t;
    }
    return all;
  };
  o << "  const uint32_t n_out = " << A.n_out << "u, n_red = " << A.n_red << "u;\n";
  std::string outs[vm::kMaxOuts];
  if (A.n_red >= 128) {
    // one wave per output; kUnroll V-vectors per lane per step
    o << "  const int lane = threadIdx.x & 63;\n";
    o << "  for (uint32_t r_out = blockIdx.x * 4u + (threadIdx.x >> 6); r_out < n_out; r_out += "
         "gridDim.x * 4u) {\n";
    o << accs("   uint32_t acc@ = red_init_j(%);\n");
    o << "   for (uint32_t r0 = lane * " << V << "u; r0 < n_red; r0 += " << 64 * V * kUnroll
      << "u) {\n";
    for (int u = 0; u < kUnroll; ++u) {
      const std::string sfx = "_" + std::to_string(u);
      o << "    uint32_t r" << sfx << " = r0 + " << u * 64 * V << "u;\n";
      o << "    const bool ok" << sfx << " = r" << sfx << " < n_red;\n";
      o << "    if (!ok" << sfx << ") r" << sfx << " = r0;\n";
      o << "    const uint32_t lin" << sfx << " = r_out * n_red + r" << sfx << ";\n";
      o << "    int32_t c" << sfx << "[kRank]; delinearize(S, lin" << sfx << ", c" << sfx << ");\n";
    }
    for (int u = 0; u < kUnroll; ++u) {
      const std::string sfx = "_" + std::to_string(u);
      put_body(o, P, V, sfx.c_str(), outs, ("lin" + sfx).c_str(), ("c" + sfx).c_str());
      o << "    if (ok" << sfx << ") for (int j = 0; j < " << V << "; ++j) {\n"
        << accs("     acc@ = red_op_j(%, acc@, " + outs[0] + "[j]);\n") << "    }\n";
    }
    o << "   }\n";
    o << "   for (int m = 32; m >= 1; m >>= 1) {\n"
      << accs("    acc@ = red_op_j(%, acc@, __shfl_xor(acc@, m, 64));\n") << "   }\n";
    o << "   if (lane == 0) {\n"
      << accs("    store_scalar(out@, " + std::to_string(A.out_dtype) + ", r_out, acc@);\n")
      << "   }\n";
    o << "  }\n}\n";
  } else {
    o << "  for (uint32_t r_out = blockIdx.x * 256u + threadIdx.x; r_out < n_out; r_out += "
         "gridDim.x * 256u) {\n";
    o << accs("   uint32_t acc@ = red_init_j(%);\n");
    o << "   for (uint32_t r = 0; r < n_red; ++r) {\n";
    o << "    const uint32_t lin = r_out * n_red + r;\n";
    o << "    int32_t c[kRank]; delinearize(S, lin, c);\n";
    put_body(o, P, 1, "", outs, "lin", "c");
    o << accs("    acc@ = red_op_j(%, acc@, " + outs[0] + "[0]);\n");
    o << "   }\n";
    o << accs("   store_scalar(out@, " + std::to_string(A.out_dtype) + ", r_out, acc@);\n");
    o << "  }\n}\n";
  }
  return o.str();
}

bool launch(JitFn* f, const vm::Program& P, const ReduceArgs* A, bool outs, int64_t blocks,
            hipStream_t stream) {
  void* args[vm::kMaxLeaves + vm::kMaxOuts + 4];
  const void* ptrs[vm::kMaxLeaves + vm::kMaxOuts + 4];
  int n = 0;
  for (int i = 0; i < P.n_leaves; ++i) ptrs[n++] = P.leaf[i].ptr;
  if (outs)
    for (int q = 0; q < P.n_outs; ++q) ptrs[n++] = P.out[q].ptr;
  if (A) {
    ptrs[n++] = A->out;
    for (int x = 0; x < A->n_extra; ++x) ptrs[n++] = A->extra_out[x];
  }
  for (int i = 0; i < n; ++i) args[i] = (void*)&ptrs[i];
  REW_HIP(hipModuleLaunchKernel(f->fn, (unsigned)blocks, 1, 1, 256, 1, 1, 0, stream, args,
                                nullptr));
  return true;
}

}  // namespace

bool jit_launch_ew(const vm::Program& P, const vm::Space& S, bool vec, hipStream_t stream) {
  if (!jit_enabled() || S.numel <= 0) return false;
  const int V = vec ? vm::kVec : 1;
  JitFn* f = get_fn(signature(P, S, 0, V, nullptr), [&] { return gen_ew(P, S, V); }, "rew_ew");
  if (!f) return false;
  const int64_t nvec = S.numel / V;
  const int64_t blocks = (nvec + 255) / 256;
  return launch(f, P, nullptr, true, blocks, stream);
}

bool jit_launch_reduce(const vm::Program& P, const vm::Space& S, const ReduceArgs& A, bool vec,
                       hipStream_t stream) {
  if (!jit_enabled() || A.n_out == 0) return false;
  const int V = (A.n_red >= 128 && vec) ? vm::kVec : 1;
  JitFn* f = get_fn(signature(P, S, 1, V, &A), [&] { return gen_reduce(P, S, A, V); },
                    "rew_reduce");
  if (!f) return false;
  int64_t blocks = A.n_red >= 128 ? (A.n_out + 3) / 4 : (A.n_out + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  return launch(f, P, &A, false, blocks, stream);
}

int64_t jit_cache_hits() { return g_jit_hits.load(std::memory_order_relaxed); }

}  // namespace rew
