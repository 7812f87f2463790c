// Device-side interpreter of vm::Program (included by the .hip kernels).
#pragma once

// Compiled both by hipcc (the interpreter kernels) and by hipRTC (the
// kernels generated for fused programs at run time), where the HIP runtime
// headers and the math functions are built in.
#ifndef __HIPCC_RTC__
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <math.h>

#include "../../include/rew_mi355x.h"
#else
#include "rtc_prelude.h"
#endif
#include "vm.h"

namespace rew {
namespace vm {

__device__ __forceinline__ uint32_t fdiv(uint32_t x, const FastDiv& f) {
  // Valid for x < 2^31 (checked on the host for every kernel space).
  return (__umulhi(x, f.m) + x) >> f.s;
}

__device__ __forceinline__ float as_f(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t as_u(float f) { return __float_as_uint(f); }

// f32 -> bf16 bits, round to nearest even; a NaN stays a NaN with its sign,
// its top payload bits and the quiet bit set ((u | 0x400000) >> 16), inf
// stays inf, overflow rounds to inf.  gfx950's v_cvt_pk_bf16_f32 implements
// exactly this rule (checked against the integer formulation on every
// class of input: ties, denormals, infinities, NaN payloads), so it replaces
// the branchy integer code.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t bf16x2_bits(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ uint16_t bf16_bits(float f) {
  return (uint16_t)bf16x2_bits(f, 0.0f);
}

__device__ __forceinline__ float round_bf16(float f) {
  return as_f((uint32_t)bf16_bits(f) << 16);
}

__device__ __forceinline__ float round_f16(float f) {
  return __half2float(__float2half(f));
}

// IEEE 754-2019 maximum/minimum: NaN-propagating (the canonical quiet NaN),
// -0 < +0.  Written as selects: equal operands differ only for +-0, where
// the smaller bit pattern is +0 and the larger -0.  Bitwise | and & keep
// it branch-free (early returns or short-circuit || compiled to a branch per
// element, and the compiler then waited for every load in flight at each).
__device__ __forceinline__ float fmax_prop(float a, float b) {
  const bool take_a = (a > b) | ((a == b) & (as_u(a) <= as_u(b)));
  const float r = take_a ? a : b;
  return ((a != a) | (b != b)) ? __builtin_nanf("") : r;
}
__device__ __forceinline__ float fmin_prop(float a, float b) {
  const bool take_a = (a < b) | ((a == b) & (as_u(a) >= as_u(b)));
  const float r = take_a ? a : b;
  return ((a != a) | (b != b)) ? __builtin_nanf("") : r;
}

// ---- scalar / vector loads and stores in register representation --------

__device__ __forceinline__ uint32_t load_scalar(const void* p, int dt,
                                                int64_t i) {
  switch (dt) {
    case REW_DT_FLOAT32: case REW_DT_INT32: case REW_DT_UINT32:
      return ((const uint32_t*)p)[i];
    case REW_DT_BFLOAT16:
      return (uint32_t)((const uint16_t*)p)[i] << 16;
    case REW_DT_FLOAT16:
      return as_u(__half2float(((const __half*)p)[i]));
    case REW_DT_INT16:
      return (uint32_t)(int32_t)((const int16_t*)p)[i];
    case REW_DT_UINT16:
      return (uint32_t)((const uint16_t*)p)[i];
    case REW_DT_INT8:
      return (uint32_t)(int32_t)((const int8_t*)p)[i];
    default:  // bool, uint8
      return (uint32_t)((const uint8_t*)p)[i];
  }
}

__device__ __forceinline__ void store_scalar(void* p, int dt, int64_t i,
                                             uint32_t v) {
  switch (dt) {
    case REW_DT_FLOAT32: case REW_DT_INT32: case REW_DT_UINT32:
      ((uint32_t*)p)[i] = v; break;
    case REW_DT_BFLOAT16:
      ((uint16_t*)p)[i] = bf16_bits(as_f(v)); break;
    case REW_DT_FLOAT16:
      ((__half*)p)[i] = __float2half(as_f(v)); break;
    case REW_DT_INT16: case REW_DT_UINT16:
      ((uint16_t*)p)[i] = (uint16_t)v; break;
    case REW_DT_BOOL:
      ((uint8_t*)p)[i] = (uint8_t)(v != 0); break;
    default:  // int8, uint8
      ((uint8_t*)p)[i] = (uint8_t)v; break;
  }
}

// Vector loads / stores of the streaming kernels: nontemporal when
// REW_VM_NT is 1 (the run-time compiled kernels choose it per program).
#ifndef REW_VM_NT
#define REW_VM_NT 0
#endif
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
template <typename T>
__device__ __forceinline__ T stream_ld(const T* p) {
  if constexpr (REW_VM_NT) return __builtin_nontemporal_load(p);
  else return *p;
}
template <typename T>
__device__ __forceinline__ void stream_st(T* p, T v) {
  if constexpr (REW_VM_NT) __builtin_nontemporal_store(v, p);
  else *p = v;
}

template <int V>
__device__ __forceinline__ void load_vec(const void* p, int dt, int64_t i,
                                         uint32_t (&d)[V]) {
  if constexpr (V == 4) {
    switch (dt) {
      case REW_DT_FLOAT32: case REW_DT_INT32: case REW_DT_UINT32: {
        const u32x4_t x = stream_ld((const u32x4_t*)((const uint32_t*)p + i));
        d[0] = x.x; d[1] = x.y; d[2] = x.z; d[3] = x.w;
        return;
      }
      case REW_DT_BFLOAT16: {
        const u32x2_t x = stream_ld((const u32x2_t*)((const uint16_t*)p + i));
        d[0] = x.x << 16; d[1] = x.x & 0xffff0000u;
        d[2] = x.y << 16; d[3] = x.y & 0xffff0000u;
        return;
      }
      default: break;
    }
  }
#pragma unroll
  for (int j = 0; j < V; ++j) d[j] = load_scalar(p, dt, i + j);
}

template <int V>
__device__ __forceinline__ void store_vec(void* p, int dt, int64_t i,
                                          const uint32_t (&v)[V]) {
  if constexpr (V == 4) {
    switch (dt) {
      case REW_DT_FLOAT32: case REW_DT_INT32: case REW_DT_UINT32: {
        stream_st((u32x4_t*)((uint32_t*)p + i), (u32x4_t){v[0], v[1], v[2], v[3]});
        return;
      }
      case REW_DT_BFLOAT16: {
        stream_st((u32x2_t*)((uint16_t*)p + i),
                  (u32x2_t){bf16x2_bits(as_f(v[0]), as_f(v[1])),
                            bf16x2_bits(as_f(v[2]), as_f(v[3]))});
        return;
      }
      default: break;
    }
  }
#pragma unroll
  for (int j = 0; j < V; ++j) store_scalar(p, dt, i + j, v[j]);
}

// ---- register file: static indexing only, selected by a uniform switch ----

// Sixteen separately named register vectors: a switch over named members
// keeps every access static, so the file lives in VGPRs (an indexed array
// would be lowered to scratch memory).
template <int V>
struct Regs {
  uint32_t r0[V], r1[V], r2[V], r3[V], r4[V], r5[V], r6[V], r7[V];
  uint32_t r8[V], r9[V], r10[V], r11[V], r12[V], r13[V], r14[V], r15[V];
};

#define REW_VM_CASES(X) \
  X(0) X(1) X(2) X(3) X(4) X(5) X(6) X(7) X(8) X(9) X(10) X(11) X(12) X(13) X(14) X(15)

template <int V>
__device__ __forceinline__ void rget(const Regs<V>& R, int i, uint32_t (&o)[V]) {
  switch (i) {
#define REW_G(k) case k: _Pragma("unroll") for (int j = 0; j < V; ++j) o[j] = R.r##k[j]; break;
    REW_VM_CASES(REW_G)
#undef REW_G
    default: break;
  }
}

template <int V>
__device__ __forceinline__ void rset(Regs<V>& R, int i, const uint32_t (&v)[V]) {
  switch (i) {
#define REW_S(k) case k: _Pragma("unroll") for (int j = 0; j < V; ++j) R.r##k[j] = v[j]; break;
    REW_VM_CASES(REW_S)
#undef REW_S
    default: break;
  }
}

// ---- leaves ----------------------------------------------------------------

// Element offset of element 0 of this lane's vector for a strided leaf.
template <int V>
__device__ __forceinline__ int64_t leaf_base(const Leaf& L, int rank,
                                             const int32_t (&coord)[kRank]) {
  int64_t base = L.off;
#pragma unroll
  for (int k = 0; k < kRank; ++k)
    if (k < rank) base += (int64_t)coord[k] * L.stride[k];
  return base;
}

template <int V>
__device__ __forceinline__ int64_t leaf_virtual(const Leaf& L, uint32_t lin) {
  int64_t a = L.off;
  uint32_t x = lin;
#pragma unroll
  for (int k = kRank - 1; k >= 0; --k) {
    if (k < L.vrank) {
      uint32_t q = fdiv(x, L.vdim[k]);
      a += (int64_t)(x - q * L.vdim[k].d) * L.stride[k];
      x = q;
    }
  }
  return a;
}

template <int V>
__device__ __forceinline__ void leaf_load(const Leaf& L, int rank,
                                          const int32_t (&coord)[kRank],
                                          uint32_t lin, uint32_t (&d)[V]) {
  if (L.mode == LM_VIRTUAL) {
#pragma unroll
    for (int j = 0; j < V; ++j)
      d[j] = load_scalar(L.ptr, L.dtype, leaf_virtual<V>(L, lin + j));
    return;
  }
  int64_t base = leaf_base<V>(L, rank, coord);
  if (L.clamp_hi >= 0) {
    // Branch of a concat evaluated outside its range: any in-bounds value
    // will do, the select that follows discards it.
    int32_t s = L.stride[rank - 1];
#pragma unroll
    for (int j = 0; j < V; ++j) {
      int64_t a = base + (int64_t)j * s;
      a = a < 0 ? 0 : (a > L.clamp_hi ? L.clamp_hi : a);
      d[j] = load_scalar(L.ptr, L.dtype, a);
    }
    return;
  }
  if (L.mode == LM_CONTIG) {
    load_vec<V>(L.ptr, L.dtype, base, d);
  } else if (L.mode == LM_BCAST) {
    uint32_t x = load_scalar(L.ptr, L.dtype, base);
#pragma unroll
    for (int j = 0; j < V; ++j) d[j] = x;
  } else {
    int32_t s = L.stride[rank - 1];
#pragma unroll
    for (int j = 0; j < V; ++j) d[j] = load_scalar(L.ptr, L.dtype, base + (int64_t)j * s);
  }
}

template <int V>
__device__ __forceinline__ void leaf_iota(const Leaf& L, int rank,
                                          const int32_t (&coord)[kRank],
                                          uint32_t lin, uint32_t (&d)[V]) {
  if (L.mode == LM_VIRTUAL) {
#pragma unroll
    for (int j = 0; j < V; ++j) d[j] = (uint32_t)leaf_virtual<V>(L, lin + j);
    return;
  }
  int64_t base = leaf_base<V>(L, rank, coord);
  int32_t s = L.stride[rank - 1];
#pragma unroll
  for (int j = 0; j < V; ++j) d[j] = (uint32_t)(base + (int64_t)j * s);
}

// ---- scalar op semantics ----------------------------------------------------

__device__ __forceinline__ bool cmp_f(float x, float y, int dir) {
  switch (dir) {
    case CMP_EQ: return x == y;
    case CMP_NE: return x != y;
    case CMP_LT: return x < y;
    case CMP_LE: return x <= y;
    case CMP_GT: return x > y;
    default: return x >= y;
  }
}
__device__ __forceinline__ bool cmp_i(int32_t x, int32_t y, int dir) {
  switch (dir) {
    case CMP_EQ: return x == y;
    case CMP_NE: return x != y;
    case CMP_LT: return x < y;
    case CMP_LE: return x <= y;
    case CMP_GT: return x > y;
    default: return x >= y;
  }
}
__device__ __forceinline__ bool cmp_u(uint32_t x, uint32_t y, int dir) {
  switch (dir) {
    case CMP_EQ: return x == y;
    case CMP_NE: return x != y;
    case CMP_LT: return x < y;
    case CMP_LE: return x <= y;
    case CMP_GT: return x > y;
    default: return x >= y;
  }
}

__device__ __forceinline__ uint32_t f2i_sat(float f) {
  if (f != f) return 0;
  if (f >= 2147483647.0f) return 0x7fffffffu;
  if (f <= -2147483648.0f) return 0x80000000u;
  return (uint32_t)(int32_t)f;
}
__device__ __forceinline__ uint32_t f2u_sat(float f) {
  if (f != f || f <= 0.0f) return 0;
  if (f >= 4294967295.0f) return 0xffffffffu;
  return (uint32_t)f;
}

__device__ __forceinline__ uint32_t op1(int op, uint32_t a) {
  float x = as_f(a);
  int32_t i = (int32_t)a;
  switch (op) {
    case OP_NEGF: return a ^ 0x80000000u;
    case OP_ABSF: return a & 0x7fffffffu;
    case OP_EXPF: return as_u(expf(x));
    case OP_LOGF: return as_u(logf(x));
    case OP_SQRTF: return as_u(sqrtf(x));
    case OP_RSQRTF: return as_u(1.0f / sqrtf(x));
    case OP_TANHF: return as_u(tanhf(x));
    case OP_LOGISTICF: return as_u(1.0f / (1.0f + expf(-x)));
    case OP_SINF: return as_u(sinf(x));
    case OP_COSF: return as_u(cosf(x));
    case OP_TANF: return as_u(tanf(x));
    case OP_EXPM1F: return as_u(expm1f(x));
    case OP_LOG1PF: return as_u(log1pf(x));
    case OP_CBRTF: return as_u(cbrtf(x));
    case OP_CEILF: return as_u(ceilf(x));
    case OP_FLOORF: return as_u(floorf(x));
    case OP_SIGNF:
      return (x != x) ? a : as_u(x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : x));
    case OP_ROUNDAFZF: return as_u(roundf(x));
    case OP_ROUNDEVENF: return as_u(rintf(x));
    case OP_ISFINITEF: return (uint32_t)((a & 0x7f800000u) != 0x7f800000u);
    case OP_NEGI: return (uint32_t)(-i);
    case OP_ABSI: return (uint32_t)(i < 0 ? -i : i);
    case OP_NOT: return ~a;
    case OP_NOTB: return a ? 0u : 1u;
    case OP_CLZ: return (uint32_t)__clz(i);
    case OP_POPCNT: return (uint32_t)__popc(a);
    case OP_SIGNI: return (uint32_t)(i > 0 ? 1 : (i < 0 ? -1 : 0));
    case OP_RBF16: return as_u(round_bf16(x));
    case OP_RF16: return as_u(round_f16(x));
    case OP_F2I: return f2i_sat(x);
    case OP_F2U: return f2u_sat(x);
    case OP_I2F: return as_u((float)i);
    case OP_U2F: return as_u((float)a);
    case OP_TOBOOL: return a != 0u;
    case OP_FTOBOOL: return x != 0.0f;
    case OP_SEXT8: return (uint32_t)(int32_t)(int8_t)a;
    case OP_ZEXT8: return a & 0xffu;
    case OP_SEXT16: return (uint32_t)(int32_t)(int16_t)a;
    case OP_ZEXT16: return a & 0xffffu;
    default: return a;
  }
}

__device__ __forceinline__ uint32_t op2(int op, int aux, uint32_t a, uint32_t b) {
  float x = as_f(a), y = as_f(b);
  int32_t i = (int32_t)a, k = (int32_t)b;
  switch (op) {
    case OP_ADDF: return as_u(x + y);
    case OP_SUBF: return as_u(x - y);
    case OP_MULF: return as_u(x * y);
    case OP_DIVF: return as_u(x / y);
    case OP_MAXF: return as_u(fmax_prop(x, y));
    case OP_MINF: return as_u(fmin_prop(x, y));
    case OP_POWF: return as_u(powf(x, y));
    case OP_REMF: return as_u(fmodf(x, y));
    case OP_ATAN2F: return as_u(atan2f(x, y));
    case OP_ADDI: return a + b;
    case OP_SUBI: return a - b;
    case OP_MULI: return a * b;
    case OP_DIVI:
      if (k == 0) return 0xffffffffu;
      if (i == (int32_t)0x80000000 && k == -1) return a;
      return (uint32_t)(i / k);
    case OP_REMI:
      if (k == 0) return a;
      if (i == (int32_t)0x80000000 && k == -1) return 0;
      return (uint32_t)(i % k);
    case OP_MAXI: return (uint32_t)(i > k ? i : k);
    case OP_MINI: return (uint32_t)(i < k ? i : k);
    case OP_DIVU: return b ? a / b : 0xffffffffu;
    case OP_REMU: return b ? a % b : a;
    case OP_MAXU: return a > b ? a : b;
    case OP_MINU: return a < b ? a : b;
    case OP_AND: return a & b;
    case OP_OR: return a | b;
    case OP_XOR: return a ^ b;
    case OP_SHL: return b >= 32u ? 0u : a << b;
    case OP_SHRA: return (uint32_t)(b >= 32u ? (i < 0 ? -1 : 0) : (i >> b));
    case OP_SHRL: return b >= 32u ? 0u : a >> b;
    case OP_CMPF: return cmp_f(x, y, aux);
    case OP_CMPI: return cmp_i(i, k, aux);
    case OP_CMPU: return cmp_u(a, b, aux);
    default: return a;
  }
}

__device__ __forceinline__ uint32_t op3(int op, uint32_t a, uint32_t b, uint32_t c) {
  switch (op) {
    case OP_SELECT: return a ? b : c;
    case OP_CLAMPF: return as_u(fmin_prop(fmax_prop(as_f(b), as_f(a)), as_f(c)));
    case OP_CLAMPI: {
      int32_t lo = (int32_t)a, x = (int32_t)b, hi = (int32_t)c;
      x = x < lo ? lo : x;
      return (uint32_t)(x > hi ? hi : x);
    }
    default: {  // OP_CLAMPU
      uint32_t x = b < a ? a : b;
      return x > c ? c : x;
    }
  }
}

__device__ __forceinline__ int op_arity(int op) {
  if (op <= OP_IOTA) return 0;
  if (op >= OP_SELECT && op <= OP_CLAMPU) return 3;
  if ((op >= OP_ADDF && op <= OP_SHRL) || (op >= OP_CMPF && op <= OP_CMPU)) return 2;
  return 1;
}

// Runs the program for V consecutive elements whose first element has
// kernel coordinates `coord` and kernel linear index `lin`.
template <int V>
__device__ __forceinline__ void run(const Program& P, int rank,
                                    const int32_t (&coord)[kRank], uint32_t lin,
                                    Regs<V>& R) {
  for (int pc = 0; pc < P.n_ins; ++pc) {
    const Ins I = P.ins[pc];
    uint32_t d[V];
    const int ar = op_arity(I.op);
    if (ar == 0) {
      if (I.op == OP_LOAD) {
        leaf_load<V>(P.leaf[I.imm], rank, coord, lin, d);
      } else if (I.op == OP_CONST) {
#pragma unroll
        for (int j = 0; j < V; ++j) d[j] = I.imm;
      } else {
        leaf_iota<V>(P.leaf[I.imm], rank, coord, lin, d);
      }
    } else {
      uint32_t a[V];
      rget<V>(R, I.a, a);
      if (ar == 1) {
#pragma unroll
        for (int j = 0; j < V; ++j) d[j] = op1(I.op, a[j]);
      } else {
        uint32_t b[V];
        rget<V>(R, I.b, b);
        if (ar == 2) {
#pragma unroll
          for (int j = 0; j < V; ++j) d[j] = op2(I.op, I.aux, a[j], b[j]);
        } else {
          uint32_t c[V];
          rget<V>(R, I.c, c);
#pragma unroll
          for (int j = 0; j < V; ++j) d[j] = op3(I.op, a[j], b[j], c[j]);
        }
      }
    }
    rset<V>(R, I.dst, d);
  }
}

// Kernel coordinates of linear index `lin` over `S`.
__device__ __forceinline__ void delinearize(const Space& S, uint32_t lin,
                                            int32_t (&coord)[kRank]) {
  uint32_t x = lin;
#pragma unroll
  for (int k = kRank - 1; k >= 0; --k) {
    if (k < S.rank) {
      uint32_t q = fdiv(x, S.dim[k]);
      coord[k] = (int32_t)(x - q * S.dim[k].d);
      x = q;
    } else {
      coord[k] = 0;
    }
  }
}

}  // namespace vm
}  // namespace rew
