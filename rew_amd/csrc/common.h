// Shared host-side definitions of librew_mi355x: dtypes, shapes, errors.
#pragma once

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include <hip/hip_runtime_api.h>

#include "../../include/rew_mi355x.h"

namespace rew {

constexpr int kMaxRank = REW_MI355X_MAX_RANK;

// Dtype codes mirror rew's DType enum (src/rew/dtype.nim:10-30).
enum DT : int {
  kBool = REW_DT_BOOL, kI8 = REW_DT_INT8, kI16 = REW_DT_INT16,
  kI32 = REW_DT_INT32, kI64 = REW_DT_INT64, kU8 = REW_DT_UINT8,
  kU16 = REW_DT_UINT16, kU32 = REW_DT_UINT32, kU64 = REW_DT_UINT64,
  kF16 = REW_DT_FLOAT16, kBF16 = REW_DT_BFLOAT16, kF32 = REW_DT_FLOAT32,
  kF64 = REW_DT_FLOAT64, kC64 = REW_DT_COMPLEX64, kC128 = REW_DT_COMPLEX128,
  kI4 = REW_DT_INT4, kU4 = REW_DT_UINT4, kNF4 = REW_DT_NF4,
  kF8E4M3 = REW_DT_FLOAT8E4M3FN, kF8E5M2 = REW_DT_FLOAT8E5M2,
  kNumDT = 20
};

// Byte size of one element (src/rew/dtype.nim:32-43).
inline int dt_size(int dt) {
  switch (dt) {
    case kBool: case kI4: case kU4: case kNF4: case kI8: case kU8:
    case kF8E4M3: case kF8E5M2: return 1;
    case kI16: case kU16: case kF16: case kBF16: return 2;
    case kI32: case kU32: case kF32: return 4;
    case kI64: case kU64: case kF64: case kC64: return 8;
    case kC128: return 16;
    default: return 0;
  }
}

// Canonical name ("float32") and enum spelling ("dtFloat32"); rew sends
// either in dtype attrs (src/rew/eager.nim:894-899).
const char* dt_name(int dt);
const char* dt_enum_name(int dt);
int parse_dtype(const std::string& s);  // -1 when unknown

inline bool dt_is_float(int dt) {
  return dt == kF16 || dt == kBF16 || dt == kF32 || dt == kF64;
}
inline bool dt_is_int(int dt) {
  return dt == kI8 || dt == kI16 || dt == kI32 || dt == kI64 || dt == kU8 ||
         dt == kU16 || dt == kU32 || dt == kU64;
}
inline bool dt_is_signed(int dt) {
  return dt == kI8 || dt == kI16 || dt == kI32 || dt == kI64;
}

struct Shape {
  int rank = 0;
  int64_t d[kMaxRank] = {0};
  Shape() = default;
  Shape(const std::vector<int64_t>& v) {
    if ((int)v.size() > kMaxRank) throw std::invalid_argument("rank > 8");
    rank = (int)v.size();
    for (int i = 0; i < rank; ++i) d[i] = v[i];
  }
  int64_t numel() const {
    int64_t n = 1;
    for (int i = 0; i < rank; ++i) n *= d[i];
    return n;
  }
  std::vector<int64_t> vec() const { return std::vector<int64_t>(d, d + rank); }
  bool operator==(const Shape& o) const {
    if (rank != o.rank) return false;
    for (int i = 0; i < rank; ++i)
      if (d[i] != o.d[i]) return false;
    return true;
  }
  bool operator!=(const Shape& o) const { return !(*this == o); }
  std::string str() const;
};

// Internal error carrying an ABI status code; converted at the ABI edge.
struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

[[noreturn]] inline void fail(int code, const std::string& msg) {
  throw Error(code, msg);
}
[[noreturn]] inline void invalid(const std::string& msg) {
  throw Error(REW_MI355X_ERR_INVALID, msg);
}

#define REW_HIP(expr)                                                        \
  do {                                                                       \
    hipError_t e_ = (expr);                                                  \
    if (e_ != hipSuccess)                                                    \
      ::rew::fail(REW_MI355X_ERR_DEVICE, std::string("HIP error '") +        \
                                             hipGetErrorString(e_) +         \
                                             "' in " #expr);                 \
  } while (0)

// Round-to-nearest-even f32 -> bf16 bits with NaN kept quiet; the same
// rule rew's literal path uses for finite values (src/rew/ops/literal.nim:112-116).
inline uint16_t f32_to_bf16_bits(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu))
    return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
inline float bf16_bits_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

}  // namespace rew
