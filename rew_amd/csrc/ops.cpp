// Op table, attribute parsing and output shape/dtype derivation of the
// eager backend.  Mirrors executeEagerOp's front half
// (src/rew/eager.nim:717-1283, 1717-1735): the op name selects a kind,
// string attrs are parsed in rew's wire format, outputs get their final
// shape/dtype at record time, and every error names the op.
#include <algorithm>
#include <cctype>
#include <cstdlib>
#include <cstring>
#include <unordered_map>

#include "kernels.h"
#include "runtime.h"

namespace rew {

// ---- dtype names (src/rew/dtype.nim:58-108) -----------------------------------

static const char* kDtNames[kNumDT] = {
    "bool", "int8", "int16", "int32", "int64", "uint8", "uint16", "uint32",
    "uint64", "float16", "bfloat16", "float32", "float64", "complex64",
    "complex128", "int4", "uint4", "nf4", "float8_e4m3fn", "float8_e5m2"};
static const char* kDtEnum[kNumDT] = {
    "dtBool", "dtInt8", "dtInt16", "dtInt32", "dtInt64", "dtUint8", "dtUint16",
    "dtUint32", "dtUint64", "dtFloat16", "dtBFloat16", "dtFloat32", "dtFloat64",
    "dtComplex64", "dtComplex128", "dtInt4", "dtUint4", "dtNF4",
    "dtFloat8E4M3Fn", "dtFloat8E5M2"};

const char* dt_name(int dt) { return (dt >= 0 && dt < kNumDT) ? kDtNames[dt] : "?"; }
const char* dt_enum_name(int dt) { return (dt >= 0 && dt < kNumDT) ? kDtEnum[dt] : "?"; }

int parse_dtype(const std::string& s) {
  for (int i = 0; i < kNumDT; ++i)
    if (s == kDtNames[i] || s == kDtEnum[i]) return i;
  return -1;
}

std::string Shape::str() const {
  std::string r = "[";
  for (int i = 0; i < rank; ++i) {
    if (i) r += ",";
    r += std::to_string(d[i]);
  }
  return r + "]";
}

// ---- op table -------------------------------------------------------------------

enum BinOp { B_ADD, B_SUB, B_MUL, B_DIV, B_MAX, B_MIN, B_ATAN2, B_POW, B_REM,
             B_AND, B_OR, B_XOR, B_SHL, B_SHRA, B_SHRL };
enum UnOp { U_NEG, U_ABS, U_EXP, U_LOG, U_SQRT, U_TANH, U_CBRT, U_CEIL, U_EXPM1,
            U_FLOOR, U_LOG1P, U_LOGISTIC, U_TAN, U_SIGN, U_ROUNDAFZ, U_ROUNDEVEN,
            U_NOT, U_CLZ, U_POPCNT, U_IDENT, U_SIN, U_COS, U_RSQRT };

struct OpSpec {
  int kind;
  int sub;
};

static const std::unordered_map<std::string, OpSpec>& op_table() {
  static const std::unordered_map<std::string, OpSpec> t = {
      {"add", {K_BINARY, B_ADD}}, {"sub", {K_BINARY, B_SUB}},
      {"mul", {K_BINARY, B_MUL}}, {"divide", {K_BINARY, B_DIV}},
      {"maximum", {K_BINARY, B_MAX}}, {"minimum", {K_BINARY, B_MIN}},
      {"atan2", {K_BINARY, B_ATAN2}}, {"power", {K_BINARY, B_POW}},
      {"remainder", {K_BINARY, B_REM}}, {"bitwiseAnd", {K_BINARY, B_AND}},
      {"bitwiseOr", {K_BINARY, B_OR}}, {"bitwiseXor", {K_BINARY, B_XOR}},
      {"shiftLeft", {K_BINARY, B_SHL}},
      {"shiftRightArithmetic", {K_BINARY, B_SHRA}},
      {"shiftRightLogical", {K_BINARY, B_SHRL}},
      {"neg", {K_UNARY, U_NEG}}, {"abs", {K_UNARY, U_ABS}},
      {"exp", {K_UNARY, U_EXP}}, {"log", {K_UNARY, U_LOG}},
      {"sqrt", {K_UNARY, U_SQRT}}, {"tanh", {K_UNARY, U_TANH}},
      {"cbrt", {K_UNARY, U_CBRT}}, {"ceil", {K_UNARY, U_CEIL}},
      {"expm1", {K_UNARY, U_EXPM1}}, {"floor", {K_UNARY, U_FLOOR}},
      {"log1p", {K_UNARY, U_LOG1P}}, {"logistic", {K_UNARY, U_LOGISTIC}},
      {"tan", {K_UNARY, U_TAN}}, {"sign", {K_UNARY, U_SIGN}},
      {"roundNearestAfz", {K_UNARY, U_ROUNDAFZ}},
      {"roundNearestEven", {K_UNARY, U_ROUNDEVEN}},
      {"bitwiseNot", {K_UNARY, U_NOT}}, {"countLeadingZeros", {K_UNARY, U_CLZ}},
      {"popcnt", {K_UNARY, U_POPCNT}},
      {"optimizationBarrier", {K_UNARY, U_IDENT}},
      {"stopGradient", {K_UNARY, U_IDENT}},
      {"sine", {K_UNARY, U_SIN}}, {"cosine", {K_UNARY, U_COS}},
      {"rsqrt", {K_UNARY, U_RSQRT}},
      {"astype", {K_CONVERT, 0}}, {"isFinite", {K_ISFINITE, 0}},
      {"bitcastConvert", {K_BITCAST, 0}},
      {"reducePrecision", {K_REDUCE_PRECISION, 0}},
      {"reshape", {K_RESHAPE, 0}}, {"transpose", {K_TRANSPOSE, 0}},
      {"reverse", {K_REVERSE, 0}}, {"broadcastTo", {K_BROADCAST_TO, 0}},
      {"broadcast", {K_BROADCAST, 0}}, {"slice", {K_SLICE, 0}},
      {"concat", {K_CONCAT, 0}}, {"iota", {K_IOTA, 0}},
      {"compare", {K_COMPARE, 0}}, {"select", {K_SELECT, 0}},
      {"clamp", {K_CLAMP, 0}},
      {"reduceSum", {K_REDUCE, RED_SUM}}, {"reduceMax", {K_REDUCE, RED_MAX}},
      {"reduceMin", {K_REDUCE, RED_MIN}}, {"reduceProd", {K_REDUCE, RED_PROD}},
      {"all", {K_REDUCE, RED_AND}}, {"any", {K_REDUCE, RED_OR}},
      {"dotGeneral", {K_DOT_GENERAL, 0}}, {"dot", {K_DOT, 0}},
      {"torchIndexSelect", {K_INDEX_SELECT, 0}},
      // backend extensions (no eager counterpart in the reference)
      {"argmax", {K_ARGMAX, 0}}, {"topK", {K_TOPK, 0}}, {"sort", {K_SORT, 0}},
      {"gather", {K_GATHER, 0}}, {"scatter", {K_SCATTER, 0}},
      // eager ops of rew's table outside the configs (src/rew/eager.nim:838-850)
      {"pad", {K_WINDOW, kWinPad}}, {"dynamicSlice", {K_WINDOW, kWinSlice}},
      {"dynamicUpdateSlice", {K_WINDOW, kWinUpdate}}, {"cholesky", {K_CHOLESKY, 0}},
      {"triangularSolve", {K_TRISOLVE, 0}},
      {"complex", {K_COMPLEX, 0}}, {"real", {K_COMPLEX, 1}}, {"imag", {K_COMPLEX, 2}},
      // one axis of rew's fft (recorded by record_fft; not a rew op name)
      {"fft1d", {K_FFT1, 0}},
      {"getDimensionSize", {K_CONST, 0}}, {"replicaId", {K_CONST, 1}},
      {"partitionId", {K_CONST, 1}}, {"setDimensionSize", {K_RESHAPE, 1}},
      {"dynamicReshape", {K_RESHAPE, 2}}, {"dynamicIota", {K_IOTA, 1}},
      {"batchNormInference", {K_BATCHNORM, kBnInference}},
      {"batchNormTraining", {K_BATCHNORM, kBnTraining}},
      {"batchNormGrad", {K_BATCHNORM, kBnGrad}},
  };
  return t;
}

// Op names rew's table knows (src/rew/eager.nim:775-868) that this backend
// does not implement natively.
static bool known_but_unimplemented(const std::string& n) {
  static const char* names[] = {
      "conv2d", "maxPool2d"};
  for (auto* s : names)
    if (n == s) return true;
  return false;
}

// ---- attribute parsing (src/rew/eager.nim:887-983) --------------------------------

using Attrs = std::vector<std::pair<std::string, std::string>>;

static const std::string& find_attr(const Attrs& a, const std::string& key,
                                    const std::string& op) {
  for (auto& kv : a)
    if (kv.first == key) return kv.second;
  invalid("eager '" + op + "': required attr '" + key + "' missing");
}

static std::string strip(const std::string& s) {
  size_t b = 0, e = s.size();
  while (b < e && std::isspace((unsigned char)s[b])) ++b;
  while (e > b && std::isspace((unsigned char)s[e - 1])) --e;
  return s.substr(b, e - b);
}

static int64_t parse_int(const std::string& s0, const std::string& op) {
  std::string s = strip(s0);
  if (s.empty()) invalid("eager '" + op + "': malformed int attr '" + s0 + "'");
  char* end = nullptr;
  long long v = std::strtoll(s.c_str(), &end, 10);
  if (*end != '\0') invalid("eager '" + op + "': malformed int attr '" + s0 + "'");
  return v;
}

// Accepts "[1,2]" (joinInts) and "@[1, 2]" (Nim seq repr).
static std::vector<int64_t> parse_int_list(const std::string& s0,
                                           const std::string& op) {
  std::string t = strip(s0);
  if (!t.empty() && t[0] == '@') t = t.substr(1);
  if (t.size() < 2 || t.front() != '[' || t.back() != ']')
    invalid("eager '" + op + "': malformed int-list attr (expected '[a,b,c]', got '" +
            s0 + "')");
  std::string body = strip(t.substr(1, t.size() - 2));
  std::vector<int64_t> r;
  if (body.empty()) return r;
  size_t p = 0;
  while (p <= body.size()) {
    size_t q = body.find(',', p);
    if (q == std::string::npos) q = body.size();
    r.push_back(parse_int(body.substr(p, q - p), op));
    p = q + 1;
  }
  return r;
}

static int parse_dtype_attr(const std::string& s, const std::string& op) {
  int dt = parse_dtype(strip(s));
  if (dt < 0) invalid("eager '" + op + "': unknown dtype attr '" + s + "'");
  return dt;
}

static int parse_cmp(const std::string& s, const std::string& op) {
  static const char* d[] = {"EQ", "NE", "LT", "LE", "GT", "GE"};
  for (int i = 0; i < 6; ++i)
    if (s == d[i]) return i;
  invalid("eager '" + op + "': invalid comparison_direction '" + s + "'");
}

// ---- helpers ----------------------------------------------------------------------

static void check_axis_list(const std::vector<int64_t>& dims, int rank,
                            const std::string& op, const char* what) {
  std::vector<bool> seen(rank, false);
  for (auto d : dims) {
    if (d < 0 || d >= rank)
      invalid("eager '" + op + "': " + what + " index " + std::to_string(d) +
              " out of range for rank " + std::to_string(rank));
    if (seen[d])
      invalid("eager '" + op + "': " + what + " index " + std::to_string(d) +
              " repeated");
    seen[d] = true;
  }
}

// An int-list attr that may be absent (empty).
static std::vector<int64_t> opt_int_list(const Attrs& a, const std::string& key,
                                         const std::string& op) {
  for (auto& kv : a)
    if (kv.first == key) return parse_int_list(kv.second, op);
  return {};
}

// Shared checks of stablehlo.gather / scatter dimension numbers: returns the
// operand's window dims (those not in `drop1` or `drop2`, in order).
static std::vector<int> window_dims(int rank, const std::vector<int64_t>& drop1,
                                    const std::vector<int64_t>& drop2, const std::string& op,
                                    const char* w1, const char* w2) {
  check_axis_list(drop1, rank, op, w1);
  check_axis_list(drop2, rank, op, w2);
  std::vector<bool> dropped(rank, false);
  for (auto d : drop1) dropped[d] = true;
  for (auto d : drop2) {
    if (dropped[d])
      invalid("eager '" + op + "': dim " + std::to_string(d) + " is both " + w1 + " and " + w2);
    dropped[d] = true;
  }
  std::vector<int> w;
  for (int d = 0; d < rank; ++d)
    if (!dropped[d]) w.push_back(d);
  return w;
}

static void check_sorted_axes(const std::vector<int64_t>& dims, int rank, const std::string& op,
                              const char* what) {
  check_axis_list(dims, rank, op, what);
  for (size_t i = 1; i < dims.size(); ++i)
    if (dims[i] <= dims[i - 1])
      invalid("eager '" + op + "': " + what + " must be sorted ascending");
}

static bool vm_dtype_ok(int dt) {
  switch (dt) {
    case kBool: case kI8: case kI16: case kI32: case kU8: case kU16: case kU32:
    case kF16: case kBF16: case kF32:
      return true;
    default:
      return false;
  }
}

static void require_vm_dtype(int dt, const std::string& op) {
  if (!vm_dtype_ok(dt))
    fail(REW_MI355X_ERR_UNSUPPORTED, "eager '" + op + "': dtype " +
                                         dt_enum_name(dt) +
                                         " not supported by the mi355x backend");
}

static const int64_t kMaxElems = (int64_t)1 << 31;

// ---- record ------------------------------------------------------------------------

Node* prepare_node(Ctx* c, const std::string& op, const std::vector<Tensor*>& ins,
                   const Attrs& attrs, std::vector<std::pair<int, Shape>>* outs_out) {
  auto it = op_table().find(op);
  if (it == op_table().end()) {
    if (known_but_unimplemented(op))
      fail(REW_MI355X_ERR_UNSUPPORTED,
           "eager backend (mi355x): op '" + op + "' is not implemented natively");
    fail(REW_MI355X_ERR_UNSUPPORTED, "eager backend: unsupported op '" + op + "'");
  }
  const OpSpec spec = it->second;
  for (size_t i = 0; i < ins.size(); ++i) {
    if (ins[i]->ctx != c)
      invalid("eager '" + op + "': cross-device operands forbidden");
  }
  auto nin = [&](size_t n) {
    if (ins.size() != n)
      invalid("eager '" + op + "': expected " + std::to_string(n) +
              " operand(s), got " + std::to_string(ins.size()));
  };

  Node* n = new Node();
  n->kind = spec.kind;
  n->sub = spec.sub;
  n->name = op;
  n->in = ins;
  std::vector<std::pair<int, Shape>> outs;  // dtype, shape

  try {
    switch (spec.kind) {
      case K_BINARY: {
        nin(2);
        Tensor *a = ins[0], *b = ins[1];
        if (a->dt != b->dt)
          invalid("eager '" + op + "': dtype mismatch (" + dt_enum_name(a->dt) +
                  " vs " + dt_enum_name(b->dt) + ")");
        if (a->shape != b->shape) invalid("eager '" + op + "': shape mismatch");
        require_vm_dtype(a->dt, op);
        bool fl = dt_is_float(a->dt);
        int s = spec.sub;
        if ((s == B_AND || s == B_OR || s == B_XOR || s == B_SHL || s == B_SHRA ||
             s == B_SHRL) && fl)
          invalid("eager '" + op + "': expected an integer or bool operand");
        if ((s == B_ATAN2 || s == B_POW) && !fl)
          fail(REW_MI355X_ERR_UNSUPPORTED, "eager '" + op + "': integer " + op +
                                               " not supported");
        outs.push_back({a->dt, a->shape});
        break;
      }
      case K_UNARY: {
        nin(1);
        require_vm_dtype(ins[0]->dt, op);
        int s = spec.sub;
        bool fl = dt_is_float(ins[0]->dt);
        bool float_only = !(s == U_NEG || s == U_ABS || s == U_NOT || s == U_CLZ ||
                            s == U_POPCNT || s == U_IDENT || s == U_SIGN);
        if (float_only && !fl)
          invalid("eager '" + op + "': expected a floating-point operand");
        if ((s == U_NOT || s == U_CLZ || s == U_POPCNT) && fl)
          invalid("eager '" + op + "': expected an integer operand");
        outs.push_back({ins[0]->dt, ins[0]->shape});
        break;
      }
      case K_CONVERT: {
        nin(1);
        n->dt_attr = parse_dtype_attr(find_attr(attrs, "dtype", op), op);
        require_vm_dtype(ins[0]->dt, op);
        require_vm_dtype(n->dt_attr, op);
        outs.push_back({n->dt_attr, ins[0]->shape});
        break;
      }
      case K_ISFINITE: {
        nin(1);
        if (!dt_is_float(ins[0]->dt)) invalid("eager 'isFinite': expected float operand");
        require_vm_dtype(ins[0]->dt, op);
        outs.push_back({kBool, ins[0]->shape});
        break;
      }
      case K_REDUCE_PRECISION: {
        nin(1);
        n->i0 = parse_int(find_attr(attrs, "exponent_bits", op), op);
        n->i1 = parse_int(find_attr(attrs, "mantissa_bits", op), op);
        if (ins[0]->dt != kF32 ||
            !((n->i0 == 8 && n->i1 == 7) || (n->i0 == 5 && n->i1 == 10) ||
              (n->i0 == 8 && n->i1 == 23)))
          fail(REW_MI355X_ERR_UNSUPPORTED,
               "eager 'reducePrecision': only float32 to bf16/f16/f32 precision");
        outs.push_back({ins[0]->dt, ins[0]->shape});
        break;
      }
      case K_BITCAST: {
        nin(1);
        n->dt_attr = parse_dtype_attr(find_attr(attrs, "dtype", op), op);
        Shape s(parse_int_list(find_attr(attrs, "output_shape", op), op));
        if (dt_size(n->dt_attr) != dt_size(ins[0]->dt) || s.numel() != ins[0]->numel())
          fail(REW_MI355X_ERR_UNSUPPORTED,
               "eager 'bitcastConvert': only same-width element types");
        n->l0 = s.vec();
        outs.push_back({n->dt_attr, s});
        break;
      }
      case K_RESHAPE: {
        if (spec.sub == 1) {
          // setDimensionSize (src/rew/ops/shape.nim:325-355): shapes are
          // static here, so the result is the operand
          nin(2);
          const int64_t dim = parse_int(find_attr(attrs, "dimension", op), op);
          if (dim < 0 || dim >= ins[0]->shape.rank)
            invalid("eager 'setDimensionSize': dimension out of range");
          if (!dt_is_int(ins[1]->dt) || ins[1]->shape.rank != 0)
            invalid("eager 'setDimensionSize': size must be an integer scalar");
          n->kind = K_RESHAPE;
          n->sub = 0;
          n->n_in_keep = 1;
          n->l0 = ins[0]->shape.vec();
          outs.push_back({ins[0]->dt, ins[0]->shape});
          break;
        }
        if (spec.sub == 2) {
          // dynamicReshape (src/rew/ops/shape.nim:360-393) to its static
          // result_shape; operand 1 (the shape vector) is not read
          nin(2);
          n->l0 = parse_int_list(find_attr(attrs, "result_shape", op), op);
          if (!dt_is_int(ins[1]->dt) || ins[1]->shape.rank != 1 ||
              ins[1]->shape.d[0] != (int64_t)n->l0.size())
            invalid("eager 'dynamicReshape': output_shape must be an integer vector of length " +
                    std::to_string(n->l0.size()));
          n->sub = 0;
          n->n_in_keep = 1;
        } else {
          nin(1);
          n->l0 = parse_int_list(find_attr(attrs, "shape", op), op);
        }
        Shape s(n->l0);
        for (auto d : n->l0)
          if (d < 0) invalid("eager 'reshape': negative dim");
        if (s.numel() != ins[0]->numel())
          invalid("eager 'reshape': element count mismatch");
        outs.push_back({ins[0]->dt, s});
        break;
      }
      case K_TRANSPOSE: {
        nin(1);
        n->l0 = parse_int_list(find_attr(attrs, "permutation", op), op);
        int r = ins[0]->shape.rank;
        if ((int)n->l0.size() != r)
          invalid("eager 'transpose': permutation length does not match rank");
        check_axis_list(n->l0, r, op, "permutation");
        Shape s;
        s.rank = r;
        for (int i = 0; i < r; ++i) s.d[i] = ins[0]->shape.d[n->l0[i]];
        outs.push_back({ins[0]->dt, s});
        break;
      }
      case K_REVERSE: {
        nin(1);
        n->l0 = parse_int_list(find_attr(attrs, "dimensions", op), op);
        check_axis_list(n->l0, ins[0]->shape.rank, op, "dimensions");
        outs.push_back({ins[0]->dt, ins[0]->shape});
        break;
      }
      case K_BROADCAST_TO: {
        nin(1);
        n->l0 = parse_int_list(find_attr(attrs, "output_shape", op), op);
        n->l1 = parse_int_list(find_attr(attrs, "broadcast_dimensions", op), op);
        Shape s(n->l0);
        const Shape& is = ins[0]->shape;
        if ((int)n->l1.size() != is.rank)
          invalid("eager 'broadcastTo': broadcast_dimensions length " +
                  std::to_string(n->l1.size()) + " does not match operand rank " +
                  std::to_string(is.rank));
        check_axis_list(n->l1, s.rank, op, "broadcast_dimensions");
        for (int i = 0; i < is.rank; ++i) {
          int64_t od = s.d[n->l1[i]];
          if (is.d[i] != 1 && is.d[i] != od)
            invalid("eager 'broadcastTo': operand dim " + std::to_string(i) +
                    " (size " + std::to_string(is.d[i]) +
                    ") is not 1 and does not match output dim " +
                    std::to_string(n->l1[i]) + " (size " + std::to_string(od) + ")");
        }
        outs.push_back({ins[0]->dt, s});
        break;
      }
      case K_BROADCAST: {
        nin(1);
        n->l0 = parse_int_list(find_attr(attrs, "broadcast_sizes", op), op);
        std::vector<int64_t> v = n->l0;
        for (int i = 0; i < ins[0]->shape.rank; ++i) v.push_back(ins[0]->shape.d[i]);
        outs.push_back({ins[0]->dt, Shape(v)});
        break;
      }
      case K_SLICE: {
        nin(1);
        n->l0 = parse_int_list(find_attr(attrs, "start_indices", op), op);
        n->l1 = parse_int_list(find_attr(attrs, "limit_indices", op), op);
        n->l2 = parse_int_list(find_attr(attrs, "strides", op), op);
        const Shape& is = ins[0]->shape;
        int r = is.rank;
        if ((int)n->l0.size() != r || (int)n->l1.size() != r || (int)n->l2.size() != r)
          invalid("eager slice: index arrays length must match operand rank " +
                  std::to_string(r));
        Shape s;
        s.rank = r;
        for (int i = 0; i < r; ++i) {
          if (n->l0[i] < 0 || n->l1[i] > is.d[i] || n->l0[i] > n->l1[i] || n->l2[i] <= 0)
            invalid("eager slice: invalid bounds at dim " + std::to_string(i));
          s.d[i] = (n->l1[i] - n->l0[i] + n->l2[i] - 1) / n->l2[i];
        }
        outs.push_back({ins[0]->dt, s});
        break;
      }
      case K_CONCAT: {
        if (ins.empty()) invalid("eager concat: empty input list");
        n->i0 = parse_int(find_attr(attrs, "dimension", op), op);
        Shape s = ins[0]->shape;
        if (n->i0 < 0 || n->i0 >= s.rank)
          invalid("eager concat: dimension " + std::to_string(n->i0) +
                  " out of range for rank " + std::to_string(s.rank));
        for (size_t i = 1; i < ins.size(); ++i) {
          if (ins[i]->dt != ins[0]->dt)
            invalid("eager concat: dtype mismatch at operand #" + std::to_string(i));
          if (ins[i]->shape.rank != s.rank)
            invalid("eager concat: rank mismatch at operand #" + std::to_string(i));
          for (int d = 0; d < s.rank; ++d)
            if (d != n->i0 && ins[i]->shape.d[d] != s.d[d])
              invalid("eager concat: shape mismatch at operand #" + std::to_string(i));
          s.d[n->i0] += ins[i]->shape.d[n->i0];
        }
        require_vm_dtype(ins[0]->dt, op);
        outs.push_back({ins[0]->dt, s});
        break;
      }
      case K_IOTA: {
        if (spec.sub == 1) {
          // dynamicIota (src/rew/ops/shape.nim:442-475) over its static
          // result_shape; operand 0 (the shape vector) is not read
          nin(1);
          n->l0 = parse_int_list(find_attr(attrs, "result_shape", op), op);
          if (!dt_is_int(ins[0]->dt) || ins[0]->shape.rank != 1 ||
              ins[0]->shape.d[0] != (int64_t)n->l0.size())
            invalid("eager 'dynamicIota': output_shape must be an integer vector of length " +
                    std::to_string(n->l0.size()));
          n->sub = 0;
          n->n_in_keep = 0;
        } else {
          nin(0);
          n->l0 = parse_int_list(find_attr(attrs, "shape", op), op);
        }
        n->dt_attr = parse_dtype_attr(find_attr(attrs, "dtype", op), op);
        n->i0 = parse_int(find_attr(attrs, "dimension", op), op);
        for (auto& kv : attrs)
          if (kv.first == "device") {
            std::string d = strip(kv.second);
            size_t colon = d.find(':');
            if (colon != std::string::npos && d.substr(0, colon) == "mi355x" &&
                parse_int(d.substr(colon + 1), op) != c->ordinal)
              invalid("eager 'iota': device attr '" + d +
                      "' does not match this context");
          }
        Shape s(n->l0);
        if (n->i0 < 0 || n->i0 >= s.rank)
          invalid("eager 'iota': dimension out of range");
        if (n->dt_attr == kBool) invalid("eager 'iota': bool dtype is not supported");
        require_vm_dtype(n->dt_attr, op);
        outs.push_back({n->dt_attr, s});
        break;
      }
      case K_COMPARE: {
        nin(2);
        n->cmp = parse_cmp(find_attr(attrs, "comparison_direction", op), op);
        if (ins[0]->dt != ins[1]->dt || ins[0]->shape != ins[1]->shape)
          invalid("eager 'compare': operands must agree on dtype and shape");
        require_vm_dtype(ins[0]->dt, op);
        outs.push_back({kBool, ins[0]->shape});
        break;
      }
      case K_SELECT: {
        nin(3);
        if (ins[0]->dt != kBool) invalid("eager 'select': pred must be bool");
        if (ins[1]->dt != ins[2]->dt || ins[1]->shape != ins[2]->shape)
          invalid("eager 'select': on_true/on_false must agree on dtype and shape");
        if (ins[0]->shape != ins[1]->shape)
          fail(REW_MI355X_ERR_UNSUPPORTED,
               "eager 'select': pred shape must equal the operand shape");
        require_vm_dtype(ins[1]->dt, op);
        outs.push_back({ins[1]->dt, ins[0]->shape});
        break;
      }
      case K_CLAMP: {
        nin(3);
        for (int i : {0, 2}) {
          if (ins[i]->dt != ins[1]->dt) invalid("eager 'clamp': dtype mismatch");
          if (ins[i]->shape.rank != 0 && ins[i]->shape != ins[1]->shape)
            invalid("eager 'clamp': bounds must be scalars or match the operand shape");
        }
        require_vm_dtype(ins[1]->dt, op);
        outs.push_back({ins[1]->dt, ins[1]->shape});
        break;
      }
      case K_REDUCE: {
        nin(1);
        n->l0 = parse_int_list(find_attr(attrs, "dims", op), op);
        const Shape& is = ins[0]->shape;
        check_axis_list(n->l0, is.rank, op, "dims");
        int s = spec.sub;
        if (s == RED_AND || s == RED_OR) {
          if (ins[0]->dt != kBool)
            invalid("eager '" + op + "': expected bool tensor (got " +
                    dt_enum_name(ins[0]->dt) + ")");
        } else if (ins[0]->dt != kF32) {
          // reductionInit (src/rew/eager.nim:1027-1033)
          invalid("eager '" + op + "': v1 supports only float32 (got " +
                  dt_enum_name(ins[0]->dt) + ")");
        }
        std::vector<bool> red(is.rank, false);
        for (auto d : n->l0) red[d] = true;
        std::vector<int64_t> od;
        for (int i = 0; i < is.rank; ++i)
          if (!red[i]) od.push_back(is.d[i]);
        outs.push_back({ins[0]->dt, Shape(od)});
        break;
      }
      case K_ARGMAX: {
        nin(1);
        n->i0 = parse_int(find_attr(attrs, "dimension", op), op);
        const Shape& is = ins[0]->shape;
        if (n->i0 < 0) n->i0 += is.rank;
        if (n->i0 < 0 || n->i0 >= is.rank) invalid("eager 'argmax': dim out of range");
        if (ins[0]->dt != kF32) invalid("eager 'argmax': float32 operand required");
        if (is.d[n->i0] == 0) invalid("eager 'argmax': empty dimension");
        std::vector<int64_t> od;
        for (int i = 0; i < is.rank; ++i)
          if (i != n->i0) od.push_back(is.d[i]);
        outs.push_back({kI32, Shape(od)});
        break;
      }
      case K_TOPK: {
        nin(1);
        n->i0 = parse_int(find_attr(attrs, "k", op), op);
        n->i1 = parse_int(find_attr(attrs, "dimension", op), op);
        n->i2 = 1;
        for (auto& kv : attrs)
          if (kv.first == "largest") n->i2 = (strip(kv.second) == "true" || strip(kv.second) == "1");
        const Shape& is = ins[0]->shape;
        if (n->i1 < 0) n->i1 += is.rank;
        if (is.rank == 0 || n->i1 != is.rank - 1)
          fail(REW_MI355X_ERR_UNSUPPORTED, "eager 'topK': only the last dimension");
        if (n->i0 <= 0 || n->i0 > is.d[n->i1])
          invalid("eager 'topK': k out of range");
        if (n->i0 > 64) fail(REW_MI355X_ERR_UNSUPPORTED, "eager 'topK': k > 64");
        if (is.d[n->i1] > kTopkMaxCols)
          fail(REW_MI355X_ERR_UNSUPPORTED, "eager 'topK': last dimension above 4096");
        if (ins[0]->dt != kF32) invalid("eager 'topK': float32 operand required");
        Shape s = is;
        s.d[n->i1] = n->i0;
        outs.push_back({ins[0]->dt, s});
        outs.push_back({kI32, s});
        break;
      }
      case K_SORT: {
        // stablehlo.sort whose comparator is one compare of the key
        // operand's pair (src/rew/ops/sort.nim:13-33): attrs dimension,
        // comparison_direction (LT/LE ascending, GT/GE descending), key.
        if (ins.empty() || ins.size() > (size_t)kSortMaxOps)
          invalid("eager 'sort': expected 1 to " + std::to_string(kSortMaxOps) + " operands");
        const Shape& is = ins[0]->shape;
        if (is.rank == 0) invalid("eager 'sort': rank-0 operand");
        n->i0 = parse_int(find_attr(attrs, "dimension", op), op);
        if (n->i0 < 0) n->i0 += is.rank;
        if (n->i0 < 0 || n->i0 >= is.rank) invalid("eager 'sort': dimension out of range");
        if (n->i0 != is.rank - 1)
          fail(REW_MI355X_ERR_UNSUPPORTED, "eager 'sort': only the last dimension");
        std::string dir = "LT";
        n->i2 = 0;
        for (auto& kv : attrs) {
          if (kv.first == "comparison_direction") dir = strip(kv.second);
          if (kv.first == "key") n->i2 = parse_int(kv.second, op);
        }
        if (dir == "LT" || dir == "LE") n->i1 = 0;
        else if (dir == "GT" || dir == "GE") n->i1 = 1;
        else invalid("eager 'sort': comparison_direction must be LT, LE, GT or GE");
        if (n->i2 < 0 || n->i2 >= (int64_t)ins.size()) invalid("eager 'sort': key out of range");
        for (Tensor* t : ins) {
          if (t->shape != is) invalid("eager 'sort': all operands must have the same shape");
          const int sz = dt_size(t->dt);
          if (t->dt == kI4 || t->dt == kU4 || t->dt == kNF4 ||
              (sz != 1 && sz != 2 && sz != 4 && sz != 8))
            fail(REW_MI355X_ERR_UNSUPPORTED,
                 std::string("eager 'sort': operand dtype ") + dt_enum_name(t->dt) + " not supported");
          outs.push_back({t->dt, t->shape});
        }
        const int kd = ins[n->i2]->dt;
        if (kd != kF32 && kd != kBF16 && kd != kF16 && kd != kI32 && kd != kI16 &&
            kd != kI8 && kd != kU32 && kd != kU16 && kd != kU8 && kd != kBool)
          fail(REW_MI355X_ERR_UNSUPPORTED,
               std::string("eager 'sort': key dtype ") + dt_enum_name(kd) + " not supported");
        if (is.d[n->i0] > kSortMaxCols)
          fail(REW_MI355X_ERR_UNSUPPORTED, "eager 'sort': dimension above " +
                                               std::to_string(kSortMaxCols));
        break;
      }
      case K_GATHER: {
        // stablehlo.gather (src/rew/ops/gather.nim:10-28): operand, start
        // indices; attrs offset_dims, collapsed_slice_dims,
        // operand_batching_dims, start_indices_batching_dims,
        // start_index_map, index_vector_dim, slice_sizes
        nin(2);
        Tensor *x = ins[0], *ix = ins[1];
        if (!dt_is_int(ix->dt)) invalid("eager 'gather': start indices must be an integer tensor");
        const int sz = dt_size(x->dt);
        if (x->dt == kI4 || x->dt == kU4 || x->dt == kNF4 || (sz != 1 && sz != 2 && sz != 4 && sz != 8))
          fail(REW_MI355X_ERR_UNSUPPORTED,
               std::string("eager 'gather': operand dtype ") + dt_enum_name(x->dt) + " not supported");
        n->l0 = parse_int_list(find_attr(attrs, "offset_dims", op), op);
        n->l1 = parse_int_list(find_attr(attrs, "collapsed_slice_dims", op), op);
        n->l2 = opt_int_list(attrs, "operand_batching_dims", op);
        n->l3 = opt_int_list(attrs, "start_indices_batching_dims", op);
        n->l4 = parse_int_list(find_attr(attrs, "start_index_map", op), op);
        n->l5 = parse_int_list(find_attr(attrs, "slice_sizes", op), op);
        n->i0 = parse_int(find_attr(attrs, "index_vector_dim", op), op);
        const Shape& xs = x->shape;
        const Shape& is = ix->shape;
        if ((int)n->l5.size() != xs.rank) invalid("eager 'gather': slice_sizes must match the operand rank");
        for (int d = 0; d < xs.rank; ++d)
          if (n->l5[d] < 0 || n->l5[d] > xs.d[d])
            invalid("eager 'gather': slice size " + std::to_string(n->l5[d]) +
                    " out of range for operand dim " + std::to_string(d));
        if (n->i0 < 0 || n->i0 > is.rank) invalid("eager 'gather': index_vector_dim out of range");
        const int64_t nvec = n->i0 < is.rank ? is.d[n->i0] : 1;
        if ((int64_t)n->l4.size() != nvec)
          invalid("eager 'gather': start_index_map must have one entry per index vector element");
        check_axis_list(n->l4, xs.rank, op, "start_index_map");
        std::vector<int> win = window_dims(xs.rank, n->l1, n->l2, op, "collapsed_slice_dims",
                                           "operand_batching_dims");
        for (auto d : n->l1)
          if (n->l5[d] > 1) invalid("eager 'gather': a collapsed dim needs slice size 1");
        for (auto d : n->l2)
          if (n->l5[d] > 1) invalid("eager 'gather': a batching dim needs slice size 1");
        if (n->l3.size() != n->l2.size())
          invalid("eager 'gather': operand and start-index batching dims differ in count");
        for (auto d : n->l3)
          if (d < 0 || d >= is.rank || d == n->i0)
            invalid("eager 'gather': start_indices_batching_dims out of range");
        if (win.size() != n->l0.size())
          invalid("eager 'gather': offset_dims must name one result dim per window dim");
        const int out_rank = (int)n->l0.size() + is.rank - (n->i0 < is.rank ? 1 : 0);
        if (out_rank > kMaxRank) fail(REW_MI355X_ERR_UNSUPPORTED, "eager 'gather': result rank above 8");
        check_sorted_axes(n->l0, out_rank, op, "offset_dims");
        std::vector<int64_t> od(out_rank, 0);
        std::vector<bool> is_off(out_rank, false);
        for (size_t j = 0; j < n->l0.size(); ++j) {
          is_off[n->l0[j]] = true;
          od[n->l0[j]] = n->l5[win[j]];
        }
        int bi = 0;
        for (int d = 0; d < out_rank; ++d) {
          if (is_off[d]) continue;
          if (bi == n->i0) ++bi;
          od[d] = is.d[bi++];
        }
        outs.push_back({x->dt, Shape(od)});
        break;
      }
      case K_SCATTER: {
        // stablehlo.scatter (src/rew/ops/scatter.nim:10-39) with one input:
        // input, scatter indices, updates; attrs update_window_dims,
        // inserted_window_dims, input_batching_dims,
        // scatter_indices_batching_dims, scatter_dims_to_operand_dims,
        // index_vector_dim, update_computation (replace / add / maximum /
        // minimum / multiply)
        nin(3);
        Tensor *x = ins[0], *ix = ins[1], *up = ins[2];
        if (!dt_is_int(ix->dt)) invalid("eager 'scatter': scatter indices must be an integer tensor");
        if (up->dt != x->dt) invalid("eager 'scatter': updates dtype differs from the input dtype");
        const std::string uc = strip(find_attr(attrs, "update_computation", op));
        if (uc == "replace") n->sub = kScatterReplace;
        else if (uc == "add") n->sub = kScatterAdd;
        else if (uc == "maximum") n->sub = kScatterMax;
        else if (uc == "minimum") n->sub = kScatterMin;
        else if (uc == "multiply") n->sub = kScatterMul;
        else invalid("eager 'scatter': update_computation must be replace, add, maximum, minimum or multiply");
        const int sz = dt_size(x->dt);
        if (x->dt == kI4 || x->dt == kU4 || x->dt == kNF4 || (sz != 1 && sz != 2 && sz != 4 && sz != 8))
          fail(REW_MI355X_ERR_UNSUPPORTED,
               std::string("eager 'scatter': dtype ") + dt_enum_name(x->dt) + " not supported");
        if (n->sub != kScatterReplace && x->dt != kF32 && x->dt != kI32 && x->dt != kU32 &&
            x->dt != kBF16 && x->dt != kF16)
          fail(REW_MI355X_ERR_UNSUPPORTED, "eager 'scatter': " + uc + " updates of " +
                                               dt_enum_name(x->dt) + " not supported");
        n->l0 = parse_int_list(find_attr(attrs, "update_window_dims", op), op);
        n->l1 = parse_int_list(find_attr(attrs, "inserted_window_dims", op), op);
        n->l2 = opt_int_list(attrs, "input_batching_dims", op);
        n->l3 = opt_int_list(attrs, "scatter_indices_batching_dims", op);
        n->l4 = parse_int_list(find_attr(attrs, "scatter_dims_to_operand_dims", op), op);
        n->i0 = parse_int(find_attr(attrs, "index_vector_dim", op), op);
        const Shape& xs = x->shape;
        const Shape& is = ix->shape;
        const Shape& us = up->shape;
        if (n->i0 < 0 || n->i0 > is.rank) invalid("eager 'scatter': index_vector_dim out of range");
        const int64_t nvec = n->i0 < is.rank ? is.d[n->i0] : 1;
        if ((int64_t)n->l4.size() != nvec)
          invalid("eager 'scatter': scatter_dims_to_operand_dims must have one entry per index "
                  "vector element");
        check_axis_list(n->l4, xs.rank, op, "scatter_dims_to_operand_dims");
        std::vector<int> win = window_dims(xs.rank, n->l1, n->l2, op, "inserted_window_dims",
                                           "input_batching_dims");
        if (n->l3.size() != n->l2.size())
          invalid("eager 'scatter': input and index batching dims differ in count");
        for (auto d : n->l3)
          if (d < 0 || d >= is.rank || d == n->i0)
            invalid("eager 'scatter': scatter_indices_batching_dims out of range");
        if (win.size() != n->l0.size())
          invalid("eager 'scatter': update_window_dims must name one updates dim per window dim");
        if (us.rank != (int)n->l0.size() + is.rank - (n->i0 < is.rank ? 1 : 0))
          invalid("eager 'scatter': updates rank does not match the dimension numbers");
        check_sorted_axes(n->l0, us.rank, op, "update_window_dims");
        std::vector<bool> is_win(us.rank, false);
        for (size_t j = 0; j < n->l0.size(); ++j) {
          is_win[n->l0[j]] = true;
          if (us.d[n->l0[j]] > xs.d[win[j]])
            invalid("eager 'scatter': an update window is larger than the input");
        }
        int bi = 0;
        for (int d = 0; d < us.rank; ++d) {
          if (is_win[d]) continue;
          if (bi == n->i0) ++bi;
          if (us.d[d] != is.d[bi++])
            invalid("eager 'scatter': updates scatter dims do not match the index batch dims");
        }
        outs.push_back({x->dt, xs});
        break;
      }
      case K_CONST: {
        if (spec.sub == 0) {
          // getDimensionSize (src/rew/ops/shape.nim:108-128): int32 scalar
          nin(1);
          n->i0 = parse_int(find_attr(attrs, "dimension", op), op);
          if (n->i0 < 0 || n->i0 >= ins[0]->shape.rank)
            invalid("eager 'getDimensionSize': dimension out of range");
          n->i0 = ins[0]->shape.d[n->i0];
          if (n->i0 > INT32_MAX)
            fail(REW_MI355X_ERR_UNSUPPORTED, "eager 'getDimensionSize': size above INT32_MAX");
          n->n_in_keep = 0;
          outs.push_back({kI32, Shape()});
        } else {
          // replicaId / partitionId (src/rew/ops/distributed.nim:11-35): one
          // replica of one partition, so uint32 0
          nin(0);
          n->i0 = 0;
          outs.push_back({kU32, Shape()});
        }
        break;
      }
      case K_WINDOW: {
        Tensor* x = ins.empty() ? nullptr : ins[0];
        const int sz = x ? dt_size(x->dt) : 0;
        if (x && (x->dt == kI4 || x->dt == kU4 || x->dt == kNF4 ||
                  (sz != 1 && sz != 2 && sz != 4 && sz != 8)))
          fail(REW_MI355X_ERR_UNSUPPORTED,
               std::string("eager '") + op + "': dtype " + dt_enum_name(x->dt) + " not supported");
        auto starts = [&](size_t first) {
          if (ins.size() != first + (size_t)x->shape.rank)
            invalid("eager '" + op + "': start index count " +
                    std::to_string((int64_t)ins.size() - (int64_t)first) +
                    " must match operand rank " + std::to_string(x->shape.rank));
          for (size_t i = first; i < ins.size(); ++i)
            if (!dt_is_int(ins[i]->dt) || ins[i]->shape.rank != 0)
              invalid("eager '" + op + "': start index #" + std::to_string(i - first) +
                      " must be an integer scalar");
        };
        if (spec.sub == kWinPad) {
          // stablehlo.pad (src/rew/ops/shape.nim:139-172, padOutputShape
          // src/rew/stablehlo/ops.nim:807-824)
          nin(2);
          if (ins[1]->dt != x->dt || ins[1]->shape.rank != 0)
            invalid("eager pad: paddingValue must be a scalar of the operand dtype");
          n->l0 = parse_int_list(find_attr(attrs, "edge_padding_low", op), op);
          n->l1 = parse_int_list(find_attr(attrs, "edge_padding_high", op), op);
          n->l2 = parse_int_list(find_attr(attrs, "interior_padding", op), op);
          const Shape& xs = x->shape;
          if ((int)n->l0.size() != xs.rank || (int)n->l1.size() != xs.rank ||
              (int)n->l2.size() != xs.rank)
            invalid("eager pad: pad: padding arrays must match operand rank " +
                    std::to_string(xs.rank));
          Shape s;
          s.rank = xs.rank;
          for (int i = 0; i < xs.rank; ++i) {
            if (n->l2[i] < 0)
              invalid("eager pad: pad: interior padding at dim " + std::to_string(i) +
                      " must be non-negative");
            s.d[i] = xs.d[i] + n->l0[i] + n->l1[i] + std::max<int64_t>(xs.d[i] - 1, 0) * n->l2[i];
            if (s.d[i] < 0)
              invalid("eager pad: pad: result dimension " + std::to_string(i) + " is negative");
          }
          outs.push_back({x->dt, s});
        } else if (spec.sub == kWinSlice) {
          // stablehlo.dynamic_slice (src/rew/ops/shape.nim:213-250)
          if (!x) invalid("eager 'dynamicSlice': expected an operand");
          starts(1);
          n->l0 = parse_int_list(find_attr(attrs, "slice_sizes", op), op);
          if ((int)n->l0.size() != x->shape.rank)
            invalid("eager 'dynamicSlice': slice_sizes length must match operand rank");
          for (int i = 0; i < x->shape.rank; ++i)
            if (n->l0[i] < 0 || n->l0[i] > x->shape.d[i])
              invalid("eager 'dynamicSlice': slice size " + std::to_string(n->l0[i]) +
                      " out of range for dim " + std::to_string(i));
          outs.push_back({x->dt, Shape(n->l0)});
        } else {
          // stablehlo.dynamic_update_slice (src/rew/ops/shape.nim:251-290)
          if (ins.size() < 2) invalid("eager 'dynamicUpdateSlice': expected operand and update");
          Tensor* up = ins[1];
          if (up->dt != x->dt) invalid("eager 'dynamicUpdateSlice': update dtype differs");
          if (up->shape.rank != x->shape.rank)
            invalid("eager 'dynamicUpdateSlice': update rank must match operand rank");
          for (int i = 0; i < x->shape.rank; ++i)
            if (up->shape.d[i] > x->shape.d[i])
              invalid("eager 'dynamicUpdateSlice': update larger than the operand at dim " +
                      std::to_string(i));
          starts(2);
          outs.push_back({x->dt, x->shape});
        }
        break;
      }
      case K_BATCHNORM: {
        // stablehlo.batch_norm_* (src/rew/ops/normalization.nim:40-205; output
        // shapes and dtypes src/rew/eager.nim:1262-1285)
        nin(spec.sub == kBnTraining ? 3 : 5);
        Tensor* x = ins[0];
        if (!dt_is_float(x->dt)) invalid("eager '" + op + "': operand must be floating point");
        if (x->dt != kF32 && x->dt != kF64)
          fail(REW_MI355X_ERR_UNSUPPORTED, "eager '" + op + "': only float32 / float64");
        n->i0 = parse_int(find_attr(attrs, "feature_index", op), op);
        if (n->i0 < 0 || n->i0 >= x->shape.rank)
          invalid("eager '" + op + "': feature_index " + std::to_string(n->i0) +
                  " out of range for rank " + std::to_string(x->shape.rank));
        const std::string es = strip(find_attr(attrs, "epsilon", op));
        char* end = nullptr;
        const double e = std::strtod(es.c_str(), &end);
        if (es.empty() || !end || *end) invalid("eager '" + op + "': malformed epsilon '" + es + "'");
        const double eps = (double)(float)e;  // an f32 attribute
        std::memcpy(&n->i1, &eps, sizeof eps);
        const int64_t C = x->shape.d[n->i0];
        const size_t dy = spec.sub == kBnGrad ? 4 : 0;
        for (size_t i = 1; i < ins.size(); ++i) {
          if (ins[i]->dt != x->dt) invalid("eager '" + op + "': operand dtypes differ");
          if (i == dy) {
            if (!(ins[i]->shape == x->shape)) invalid("eager '" + op + "': gradOutput shape differs");
          } else if (ins[i]->shape.rank != 1 || ins[i]->shape.d[0] != C) {
            invalid("eager '" + op + "': feature operand " + std::to_string(i) +
                    " must have shape [" + std::to_string(C) + "]");
          }
        }
        outs.push_back({x->dt, x->shape});
        if (spec.sub != kBnInference) {
          outs.push_back({x->dt, Shape(std::vector<int64_t>{C})});
          outs.push_back({x->dt, Shape(std::vector<int64_t>{C})});
        }
        break;
      }
      case K_CHOLESKY: {
        // stablehlo.cholesky (src/rew/ops/linalg.nim:177-202)
        nin(1);
        Tensor* x = ins[0];
        if (!dt_is_float(x->dt)) invalid("eager 'cholesky': operand must be floating point");
        if (x->shape.rank < 2 || x->shape.d[x->shape.rank - 1] != x->shape.d[x->shape.rank - 2])
          invalid("eager 'cholesky': innermost matrix dimensions must be square");
        if (x->dt != kF32 && x->dt != kF64)
          fail(REW_MI355X_ERR_UNSUPPORTED, "eager 'cholesky': only float32 / float64");
        if (x->shape.d[x->shape.rank - 1] > kCholMaxN)
          fail(REW_MI355X_ERR_UNSUPPORTED, "eager 'cholesky': matrices above " +
                                               std::to_string(kCholMaxN) + " x " +
                                               std::to_string(kCholMaxN));
        const std::string lw = strip(find_attr(attrs, "lower", op));
        if (lw != "true" && lw != "false") invalid("eager 'cholesky': lower must be true or false");
        n->i0 = lw == "true";
        outs.push_back({x->dt, x->shape});
        break;
      }
      case K_COMPLEX: {
        // complex (src/rew/ops/arith.nim:86-106), real / imag (unary.nim:184-224)
        if (spec.sub == 0) {
          nin(2);
          Tensor *re = ins[0], *im = ins[1];
          if (re->dt != kF32 && re->dt != kF64)
            invalid("eager 'complex': operands must be float32 or float64, got " +
                    std::string(dt_enum_name(re->dt)));
          if (im->dt != re->dt) invalid("eager 'complex': dtype mismatch");
          if (im->shape != re->shape) invalid("eager 'complex': shape mismatch");
          n->i0 = 0;
          n->i1 = dt_size(re->dt);
          outs.push_back({re->dt == kF32 ? (int)kC64 : (int)kC128, re->shape});
        } else {
          nin(1);
          Tensor* x = ins[0];
          const bool cx = x->dt == kC64 || x->dt == kC128;
          if (!cx && !dt_is_float(x->dt))
            invalid("eager '" + op + "': operand must be floating point or complex, got " +
                    dt_enum_name(x->dt));
          if (cx) {
            n->i0 = spec.sub;  // 1 real part, 2 imaginary part
            n->i1 = dt_size(x->dt) / 2;
            outs.push_back({x->dt == kC64 ? (int)kF32 : (int)kF64, x->shape});
          } else {
            n->i0 = spec.sub == 1 ? 3 : 4;  // a real tensor's real part is itself, imag zeros
            n->i1 = dt_size(x->dt);
            outs.push_back({x->dt, x->shape});
          }
        }
        break;
      }
      case K_FFT1: {
        // attrs axis, mode (0 forward, 1 inverse, 2 real to complex, 3 complex to
        // real), n (the transform length along axis)
        nin(1);
        Tensor* x = ins[0];
        const int64_t ax = std::atoll(find_attr(attrs, "axis", op).c_str());
        const int64_t mode = std::atoll(find_attr(attrs, "mode", op).c_str());
        const int64_t len = std::atoll(find_attr(attrs, "n", op).c_str());
        if (ax < 0 || ax >= x->shape.rank || mode < 0 || mode > 3 || len < 0)
          invalid("eager 'fft1d': bad axis / mode / length");
        const bool cx = x->dt == kC64 || x->dt == kC128;
        Shape s = x->shape;
        int odt = x->dt;
        if (mode == 2) {
          if (x->dt != kF32 && x->dt != kF64) invalid("eager 'fft': RFFT operand must be f32 or f64");
          if (x->shape.d[ax] != len) invalid("eager 'fft': RFFT length mismatch");
          s.d[ax] = len / 2 + 1;
          odt = x->dt == kF32 ? (int)kC64 : (int)kC128;
        } else if (mode == 3) {
          if (!cx) invalid("eager 'fft': IRFFT operand must be complex");
          if (x->shape.d[ax] != len / 2 + 1) invalid("eager 'fft': IRFFT length mismatch");
          s.d[ax] = len;
          odt = x->dt == kC64 ? (int)kF32 : (int)kF64;
        } else {
          if (!cx) invalid("eager 'fft': FFT / IFFT operand must be complex");
          if (x->shape.d[ax] != len) invalid("eager 'fft': FFT length mismatch");
        }
        n->i0 = ax;
        n->i1 = mode;
        n->i2 = len;
        outs.push_back({odt, s});
        break;
      }
      case K_TRISOLVE: {
        // stablehlo.triangular_solve (src/rew/ops/linalg.nim:350-376; attrs
        // left_side, lower, unit_diagonal, transpose_a)
        nin(2);
        Tensor *a = ins[0], *b = ins[1];
        if (a->dt != b->dt) invalid("eager 'triangularSolve': dtype mismatch");
        if (!dt_is_float(a->dt)) invalid("eager 'triangularSolve': operands must be floating point");
        const int r = a->shape.rank;
        if (r < 2 || a->shape.d[r - 1] != a->shape.d[r - 2])
          invalid("eager 'triangularSolve': a's innermost matrix dimensions must be square");
        auto flag = [&](const char* k) {
          const std::string v = strip(find_attr(attrs, k, op));
          if (v != "true" && v != "false")
            invalid(std::string("eager 'triangularSolve': ") + k + " must be true or false");
          return v == "true";
        };
        const bool left = flag("left_side"), lower = flag("lower"), unit = flag("unit_diagonal");
        const std::string ta = strip(find_attr(attrs, "transpose_a", op));
        bool trans;
        if (ta == "NO_TRANSPOSE") trans = false;
        else if (ta == "TRANSPOSE" || ta == "ADJOINT") trans = true;  // real operands
        else invalid("eager 'triangularSolve': transpose_a must be NO_TRANSPOSE, TRANSPOSE or "
                     "ADJOINT, got '" + ta + "'");
        const int64_t nn = a->shape.d[r - 1];
        bool ok = b->shape.rank == r;
        for (int k = 0; ok && k < r - 2; ++k) ok = a->shape.d[k] == b->shape.d[k];
        if (ok) ok = left ? b->shape.d[r - 2] == nn : b->shape.d[r - 1] == nn;
        if (!ok)
          invalid("eager 'triangularSolve': b " + b->shape.str() + " does not fit a " +
                  a->shape.str() + (left ? " (left side)" : " (right side)"));
        if (a->dt != kF32 && a->dt != kF64)
          fail(REW_MI355X_ERR_UNSUPPORTED, "eager 'triangularSolve': only float32 / float64");
        if (nn > kCholMaxN)
          fail(REW_MI355X_ERR_UNSUPPORTED, "eager 'triangularSolve': matrices above " +
                                               std::to_string(kCholMaxN) + " x " +
                                               std::to_string(kCholMaxN));
        n->i0 = (left ? 1 : 0) | (lower ? 2 : 0) | (unit ? 4 : 0) | (trans ? 8 : 0);
        outs.push_back({b->dt, b->shape});
        break;
      }
      case K_DOT:
      case K_DOT_GENERAL: {
        nin(2);
        Tensor *a = ins[0], *b = ins[1];
        if (a->dt != b->dt)
          invalid("eager '" + op + "': dtype mismatch (" + dt_enum_name(a->dt) +
                  " vs " + dt_enum_name(b->dt) + ")");
        if (a->dt != kF32 && a->dt != kBF16 && a->dt != kF16)
          fail(REW_MI355X_ERR_UNSUPPORTED,
               "eager '" + op + "': dtype " + dt_enum_name(a->dt) +
                   " not supported by the mi355x backend");
        if (spec.kind == K_DOT) {
          // stablehlo.dot: rank <= 2, contracts lhs last dim with rhs first dim.
          int ra = a->shape.rank, rb = b->shape.rank;
          if (ra < 1 || ra > 2 || rb < 1 || rb > 2)
            invalid("eager dot: operands must be rank 1 or 2");
          n->kind = K_DOT_GENERAL;
          n->l0 = {};
          n->l1 = {};
          n->l2 = {ra - 1};
          n->l3 = {0};
        } else {
          n->l0 = parse_int_list(find_attr(attrs, "lhs_batching", op), op);
          n->l1 = parse_int_list(find_attr(attrs, "rhs_batching", op), op);
          n->l2 = parse_int_list(find_attr(attrs, "lhs_contracting", op), op);
          n->l3 = parse_int_list(find_attr(attrs, "rhs_contracting", op), op);
        }
        const Shape &sa = a->shape, &sb = b->shape;
        if (n->l0.size() != n->l1.size() || n->l2.size() != n->l3.size())
          invalid("eager '" + op + "': batching/contracting lists differ in length");
        std::vector<int64_t> la = n->l0, lb = n->l1;
        la.insert(la.end(), n->l2.begin(), n->l2.end());
        lb.insert(lb.end(), n->l3.begin(), n->l3.end());
        check_axis_list(la, sa.rank, op, "lhs");
        check_axis_list(lb, sb.rank, op, "rhs");
        for (size_t i = 0; i < n->l0.size(); ++i)
          if (sa.d[n->l0[i]] != sb.d[n->l1[i]])
            invalid("eager '" + op + "': batching dim size mismatch");
        for (size_t i = 0; i < n->l2.size(); ++i)
          if (sa.d[n->l2[i]] != sb.d[n->l3[i]])
            invalid("eager '" + op + "': contracting dim size mismatch");
        // dotGeneralShape (src/rew/eager.nim:1000-1014)
        std::vector<bool> ua(sa.rank, false), ub(sb.rank, false);
        for (auto d : la) ua[d] = true;
        for (auto d : lb) ub[d] = true;
        std::vector<int64_t> od;
        for (auto d : n->l0) od.push_back(sa.d[d]);
        for (int i = 0; i < sa.rank; ++i)
          if (!ua[i]) od.push_back(sa.d[i]);
        for (int i = 0; i < sb.rank; ++i)
          if (!ub[i]) od.push_back(sb.d[i]);
        outs.push_back({a->dt, Shape(od)});
        break;
      }
      case K_INDEX_SELECT: {
        nin(2);
        n->i0 = parse_int(find_attr(attrs, "dim", op), op);
        n->i1 = parse_int(find_attr(attrs, "batch_dims", op), op);
        Tensor *a = ins[0], *ix = ins[1];
        if (!dt_is_int(ix->dt))
          invalid("torchIndexSelect: index must be an integer tensor");
        if (n->i1 != 0)
          fail(REW_MI355X_ERR_UNSUPPORTED,
               "eager 'torchIndexSelect': batch_dims > 0 not supported");
        if (n->i0 < 0 || n->i0 >= a->shape.rank)
          invalid("eager torchIndexSelect: dim out of range");
        std::vector<int64_t> od;
        for (int i = 0; i < n->i0; ++i) od.push_back(a->shape.d[i]);
        for (int i = 0; i < ix->shape.rank; ++i) od.push_back(ix->shape.d[i]);
        for (int i = n->i0 + 1; i < a->shape.rank; ++i) od.push_back(a->shape.d[i]);
        outs.push_back({a->dt, Shape(od)});
        break;
      }
      default:
        fail(REW_MI355X_ERR_UNSUPPORTED, "eager backend: unsupported op '" + op + "'");
    }
  } catch (...) {
    delete n;
    throw;
  }

  for (auto& o : outs)
    if (o.second.numel() >= kMaxElems) {
      delete n;
      fail(REW_MI355X_ERR_UNSUPPORTED, "eager '" + op + "': result of " +
                                           std::to_string(o.second.numel()) +
                                           " elements exceeds the 2^31 limit");
    }
  *outs_out = std::move(outs);
  return n;
}

std::vector<Tensor*> commit_node(Ctx* c, Node* n, const std::vector<Tensor*>& ins,
                                 const std::vector<std::pair<int, Shape>>& outs) {
  n->in = ins;
  if (n->n_in_keep >= 0 && (size_t)n->n_in_keep < ins.size()) n->in.resize(n->n_in_keep);
  std::vector<Tensor*> result;
  for (size_t i = 0; i < outs.size(); ++i) {
    Tensor* t = new_tensor(c, outs[i].first, outs[i].second);
    t->prod = n;
    t->prod_out = (int)i;
    t->ext = 1;
    n->out.push_back(t);
    result.push_back(t);
  }
  for (auto* t : n->in) t->uses++;
  n->order = c->order_counter++;
  c->pending.push_back(n);
  c->stats.ops_recorded++;
  if (c->mode == REW_MI355X_MODE_OP_BY_OP ||
      (int)c->pending.size() >= c->flush_threshold)
    flush(c);
  return result;
}

std::vector<Tensor*> record_op(Ctx* c, const std::string& op, const std::vector<Tensor*>& ins,
                               const Attrs& attrs);

static std::string int_list_text(const std::vector<int64_t>& v) {
  std::string s = "[";
  for (size_t i = 0; i < v.size(); ++i) s += (i ? "," : "") + std::to_string(v[i]);
  return s + "]";
}

// rew's einsum / unaryEinsum (src/rew/ops/linalg.nim:378-430; their eager
// attrs einsum_config and output_shape, eager.nim:1495-1502) recorded as
// primitive nodes.  TensorFlow's einsum grammar with an explicit "->",
// letters as labels (no ellipsis, no label repeated within one operand):
//   * labels of one operand that reach neither the other operand nor the
//     output are summed out first (reduceSum);
//   * one dotGeneral then batches the labels both operands and the output
//     hold and contracts those only the operands share;
//   * a transpose puts the dot's [batch, lhs-only, rhs-only] order (or a
//     unary einsum's remaining order) into the output's.
static std::vector<Tensor*> record_einsum(Ctx* c, const std::string& op,
                                          const std::vector<Tensor*>& ins, const Attrs& attrs) {
  const bool unary = op == "unaryEinsum";
  const size_t nin = unary ? 1 : 2;
  if (ins.size() != nin)
    invalid("eager '" + op + "': expected " + std::to_string(nin) + " operand(s), got " +
            std::to_string(ins.size()));
  std::string cfg = find_attr(attrs, "einsum_config", op);
  std::string sp;
  for (char ch : cfg)
    if (ch != ' ') sp.push_back(ch);
  const size_t arrow = sp.find("->");
  if (sp.empty() || arrow == std::string::npos)
    fail(REW_MI355X_ERR_UNSUPPORTED, "eager '" + op + "': config '" + cfg +
                                         "' needs an explicit '->' output");
  if (sp.find("...") != std::string::npos)
    fail(REW_MI355X_ERR_UNSUPPORTED, "eager '" + op + "': ellipsis labels are not supported");
  std::vector<std::string> in_spec;
  {
    const std::string lhs = sp.substr(0, arrow);
    size_t b = 0;
    for (;;) {
      const size_t e = lhs.find(',', b);
      in_spec.push_back(lhs.substr(b, e == std::string::npos ? std::string::npos : e - b));
      if (e == std::string::npos) break;
      b = e + 1;
    }
  }
  const std::string out_spec = sp.substr(arrow + 2);
  if (in_spec.size() != nin)
    invalid("eager '" + op + "': config '" + cfg + "' names " + std::to_string(in_spec.size()) +
            " operand(s)");
  auto check_spec = [&](const std::string& s, const char* what) {
    for (size_t i = 0; i < s.size(); ++i) {
      if (!std::isalpha((unsigned char)s[i]))
        invalid("eager '" + op + "': bad label '" + std::string(1, s[i]) + "' in " + what);
      if (s.find(s[i]) != i)
        fail(REW_MI355X_ERR_UNSUPPORTED, "eager '" + op + "': label '" + std::string(1, s[i]) +
                                             "' repeated in " + what);
    }
  };
  for (size_t i = 0; i < nin; ++i) {
    check_spec(in_spec[i], "an operand");
    if ((int)in_spec[i].size() != ins[i]->shape.rank)
      invalid("eager '" + op + "': operand " + std::to_string(i) + " has rank " +
              std::to_string(ins[i]->shape.rank) + ", config '" + cfg + "' gives it " +
              std::to_string(in_spec[i].size()) + " label(s)");
  }
  check_spec(out_spec, "the output");
  if (!unary && ins[0]->dt != ins[1]->dt)
    invalid(std::string("eager 'einsum': dtype mismatch (") + dt_enum_name(ins[0]->dt) + " vs " +
            dt_enum_name(ins[1]->dt) + ")");
  // label sizes agree across operands
  int64_t size_of[128];
  for (auto& v : size_of) v = -1;
  for (size_t i = 0; i < nin; ++i)
    for (size_t k = 0; k < in_spec[i].size(); ++k) {
      const int ch = (unsigned char)in_spec[i][k];
      const int64_t d = ins[i]->shape.d[k];
      if (size_of[ch] >= 0 && size_of[ch] != d)
        invalid("eager '" + op + "': label '" + std::string(1, (char)ch) + "' sizes " +
                std::to_string(size_of[ch]) + " and " + std::to_string(d));
      size_of[ch] = d;
    }
  for (char ch : out_spec)
    if (size_of[(unsigned char)ch] < 0)
      invalid("eager '" + op + "': output label '" + std::string(1, ch) + "' is in no operand");
  const std::vector<int64_t> want = parse_int_list(find_attr(attrs, "output_shape", op), op);

  std::vector<Tensor*> owned;  // intermediate results (one reference each)
  auto release = [&]() {
    for (Tensor* t : owned) {
      t->ext--;
      maybe_destroy(t);
    }
    owned.clear();
  };
  auto run1 = [&](const std::string& name, const std::vector<Tensor*>& xs,
                  const Attrs& a) -> Tensor* {
    std::vector<Tensor*> r = record_op(c, name, xs, a);
    owned.push_back(r[0]);
    return r[0];
  };
  try {
    std::vector<Tensor*> x(ins.begin(), ins.end());
    std::vector<std::string> lab(in_spec.begin(), in_spec.end());
    for (size_t i = 0; i < nin; ++i) {
      const std::string other = nin == 2 ? lab[1 - i] : std::string();
      std::vector<int64_t> dims;
      std::string keep;
      for (size_t k = 0; k < lab[i].size(); ++k) {
        const char ch = lab[i][k];
        if (out_spec.find(ch) == std::string::npos && other.find(ch) == std::string::npos)
          dims.push_back((int64_t)k);
        else
          keep.push_back(ch);
      }
      if (!dims.empty()) {
        x[i] = run1("reduceSum", {x[i]}, {{"dims", int_list_text(dims)}});
        lab[i] = keep;
      }
    }
    std::string cur;  // labels of the running result, in order
    Tensor* y;
    if (unary) {
      y = x[0];
      cur = lab[0];
    } else {
      std::vector<int64_t> lb, rb, lc, rc;
      std::string batch, lfree, rfree;
      for (size_t k = 0; k < lab[0].size(); ++k) {
        const char ch = lab[0][k];
        const size_t j = lab[1].find(ch);
        if (j == std::string::npos) {
          lfree.push_back(ch);
        } else if (out_spec.find(ch) != std::string::npos) {
          lb.push_back((int64_t)k);
          rb.push_back((int64_t)j);
          batch.push_back(ch);
        } else {
          lc.push_back((int64_t)k);
          rc.push_back((int64_t)j);
        }
      }
      for (char ch : lab[1])
        if (lab[0].find(ch) == std::string::npos) rfree.push_back(ch);
      y = run1("dotGeneral", {x[0], x[1]},
               {{"lhs_batching", int_list_text(lb)}, {"rhs_batching", int_list_text(rb)},
                {"lhs_contracting", int_list_text(lc)}, {"rhs_contracting", int_list_text(rc)}});
      cur = batch + lfree + rfree;
    }
    if (cur.size() != out_spec.size())
      invalid("eager '" + op + "': config '" + cfg + "' leaves labels '" + cur +
              "' for output '" + out_spec + "'");
    std::vector<int64_t> perm;
    bool ident = true;
    for (size_t k = 0; k < out_spec.size(); ++k) {
      const size_t j = cur.find(out_spec[k]);
      perm.push_back((int64_t)j);
      ident = ident && j == k;
    }
    if (!ident) y = run1("transpose", {y}, {{"permutation", int_list_text(perm)}});
    if (y->shape.rank != (int)want.size())
      invalid("eager '" + op + "': output_shape " + int_list_text(want) + " but the config gives " +
              y->shape.str());
    for (int k = 0; k < y->shape.rank; ++k)
      if (y->shape.d[k] != want[k])
        invalid("eager '" + op + "': output_shape " + int_list_text(want) +
                " but the config gives " + y->shape.str());
    y->ext++;  // (an identity unary einsum hands back the operand, one more reference)
    release();
    return {y};
  } catch (...) {
    release();
    throw;
  }
}

// The values of an integer vector operand of length n, read back from the
// device (the pending graph is flushed first, as rew_mi355x_to_host does).
static std::vector<int64_t> read_index_vector(Ctx* c, Tensor* t, const std::string& op,
                                              const char* what, size_t n) {
  if (!dt_is_int(t->dt) || t->shape.rank != 1 || t->shape.d[0] != (int64_t)n)
    invalid("eager '" + op + "': " + what + " must be an integer vector of length " +
            std::to_string(n));
  if (t->prod) flush(c);
  if (!t->st) invalid("eager '" + op + "': " + what + " has no data (an earlier flush failed)");
  std::vector<uint8_t> raw((size_t)t->nbytes());
  if (!raw.empty()) {
    REW_HIP(hipMemcpyAsync(raw.data(), t->data(), raw.size(), hipMemcpyDeviceToHost, c->stream));
    REW_HIP(hipStreamSynchronize(c->stream));
  }
  std::vector<int64_t> v(n);
  const int w = dt_size(t->dt);
  const bool sgn = t->dt == kI8 || t->dt == kI16 || t->dt == kI32 || t->dt == kI64;
  for (size_t i = 0; i < n; ++i) {
    uint64_t u = 0;
    std::memcpy(&u, raw.data() + i * w, (size_t)w);
    if (sgn && w < 8 && (u >> (8 * w - 1)) & 1) u |= ~0ull << (8 * w);
    v[i] = (int64_t)u;
  }
  return v;
}

// The shape-operand ops rew dispatches with a static result_shape
// (src/rew/ops/shape.nim:395-441 dynamicPad, 477-517 realDynamicSlice;
// src/rew/ops/linalg.nim:288-326 dynamicBroadcastInDim) as their static
// forms.  The broadcast's output-dimensions operand only restates the
// result shape and is not read; the padding and slice bounds are read back
// from the device (a synchronising read) and the static pad / slice runs.
static std::vector<Tensor*> record_dynamic_shape_op(Ctx* c, const std::string& op,
                                                    const std::vector<Tensor*>& ins,
                                                    const Attrs& attrs) {
  const std::vector<int64_t> rs = parse_int_list(find_attr(attrs, "result_shape", op), op);
  auto need = [&](size_t n) {
    if (ins.size() != n)
      invalid("eager '" + op + "': expected " + std::to_string(n) + " operand(s), got " +
              std::to_string(ins.size()));
  };
  std::vector<Tensor*> r;
  if (op == "dynamicBroadcastInDim") {
    need(2);
    if (!dt_is_int(ins[1]->dt) || ins[1]->shape.rank != 1 ||
        ins[1]->shape.d[0] != (int64_t)rs.size())
      invalid("eager 'dynamicBroadcastInDim': outputDimensions must be an integer vector of "
              "length " + std::to_string(rs.size()));
    r = record_op(c, "broadcastTo", {ins[0]},
                  {{"output_shape", int_list_text(rs)},
                   {"broadcast_dimensions", find_attr(attrs, "broadcast_dimensions", op)}});
  } else if (op == "dynamicPad") {
    need(5);
    const size_t rank = (size_t)ins[0]->shape.rank;
    const auto lo = read_index_vector(c, ins[2], op, "edgePaddingLow", rank);
    const auto hi = read_index_vector(c, ins[3], op, "edgePaddingHigh", rank);
    const auto in = read_index_vector(c, ins[4], op, "interiorPadding", rank);
    r = record_op(c, "pad", {ins[0], ins[1]},
                  {{"edge_padding_low", int_list_text(lo)}, {"edge_padding_high", int_list_text(hi)},
                   {"interior_padding", int_list_text(in)}});
  } else {  // realDynamicSlice
    need(4);
    const size_t rank = (size_t)ins[0]->shape.rank;
    const auto st = read_index_vector(c, ins[1], op, "startIndices", rank);
    const auto li = read_index_vector(c, ins[2], op, "limitIndices", rank);
    const auto sd = read_index_vector(c, ins[3], op, "strides", rank);
    r = record_op(c, "slice", {ins[0]},
                  {{"start_indices", int_list_text(st)}, {"limit_indices", int_list_text(li)},
                   {"strides", int_list_text(sd)}});
  }
  const Shape& got = r[0]->shape;
  bool ok = got.rank == (int)rs.size();
  for (int k = 0; ok && k < got.rank; ++k) ok = got.d[k] == rs[k];
  if (!ok) {
    const std::string gs = got.str();
    r[0]->ext--;
    maybe_destroy(r[0]);
    invalid("eager '" + op + "': result_shape " + int_list_text(rs) + " but the operands give " +
            gs);
  }
  return r;
}

// rew's fft (src/rew/ops/linalg.nim:328-348; stablehlo.fft with fft_type
// FFT / IFFT / RFFT / IRFFT over the trailing len(fft_length) dims, 1-3) as
// one-axis DFTs: RFFT transforms the last axis real to complex, then the
// others complex; IRFFT the leading ones complex (inverse), then the last one
// complex to real; FFT / IFFT every axis.  Each axis is an exact-length DFT
// summed in double.
static std::vector<Tensor*> record_fft(Ctx* c, const std::vector<Tensor*>& ins,
                                       const Attrs& attrs) {
  if (ins.size() != 1) invalid("eager 'fft': expected 1 operand, got " + std::to_string(ins.size()));
  const std::string ty = strip(find_attr(attrs, "fft_type", "fft"));
  const std::vector<int64_t> len = parse_int_list(find_attr(attrs, "fft_length", "fft"), "fft");
  Tensor* x = ins[0];
  const int r = x->shape.rank;
  if (len.empty() || len.size() > 3)
    invalid("eager 'fft': fftLength must have length 1..3, got " + std::to_string(len.size()));
  if ((int)len.size() > r) invalid("eager 'fft': fftLength rank exceeds operand rank");
  for (int64_t d : len)
    if (d < 0) invalid("eager 'fft': fftLength dimensions must be non-negative");
  const int s0 = r - (int)len.size();
  const bool cx = x->dt == kC64 || x->dt == kC128;
  std::vector<std::pair<int, int>> passes;  // (axis, mode)
  const int last = r - 1;
  if (ty == "FFT" || ty == "IFFT") {
    if (!cx) invalid("eager 'fft': FFT/IFFT operand must be complex, got " + std::string(dt_enum_name(x->dt)));
    for (int a = last; a >= s0; --a) passes.push_back({a, ty == "FFT" ? 0 : 1});
  } else if (ty == "RFFT") {
    if (x->dt != kF32 && x->dt != kF64)
      invalid("eager 'fft': RFFT operand must be float32 or float64, got " + std::string(dt_enum_name(x->dt)));
    passes.push_back({last, 2});
    for (int a = last - 1; a >= s0; --a) passes.push_back({a, 0});
  } else if (ty == "IRFFT") {
    if (!cx) invalid("eager 'fft': IRFFT operand must be complex, got " + std::string(dt_enum_name(x->dt)));
    for (int a = s0; a < last; ++a) passes.push_back({a, 1});
    passes.push_back({last, 3});
  } else {
    invalid("eager 'fft': fft_type must be FFT, IFFT, RFFT or IRFFT, got '" + ty + "'");
  }
  // operand extents: FFT / IFFT / RFFT need the trailing dims equal to
  // fftLength; IRFFT the last one equal to fftLength[-1] / 2 + 1
  for (size_t i = 0; i < len.size(); ++i) {
    const int a = s0 + (int)i;
    const int64_t want = (ty == "IRFFT" && a == last) ? len[i] / 2 + 1 : len[i];
    if (x->shape.d[a] != want)
      invalid("eager 'fft': operand dimension " + std::to_string(a) + " is " +
              std::to_string(x->shape.d[a]) + ", fftLength needs " + std::to_string(want));
  }
  std::vector<Tensor*> owned;
  Tensor* y = x;
  try {
    for (auto& ps : passes) {
      const int64_t n = len[(size_t)(ps.first - s0)];
      std::vector<Tensor*> o = record_op(c, "fft1d", {y},
                                         {{"axis", std::to_string(ps.first)},
                                          {"mode", std::to_string(ps.second)},
                                          {"n", std::to_string(n)}});
      owned.push_back(o[0]);
      y = o[0];
    }
  } catch (...) {
    for (Tensor* t : owned) {
      t->ext--;
      maybe_destroy(t);
    }
    throw;
  }
  y->ext++;
  for (Tensor* t : owned) {
    t->ext--;
    maybe_destroy(t);
  }
  return {y};
}

std::vector<Tensor*> record_op(Ctx* c, const std::string& op,
                               const std::vector<Tensor*>& ins,
                               const Attrs& attrs) {
  if (op == "einsum" || op == "unaryEinsum") return record_einsum(c, op, ins, attrs);
  if (op == "fft") return record_fft(c, ins, attrs);
  if (op == "dynamicPad" || op == "realDynamicSlice" || op == "dynamicBroadcastInDim")
    return record_dynamic_shape_op(c, op, ins, attrs);
  std::vector<std::pair<int, Shape>> outs;
  Node* n = prepare_node(c, op, ins, attrs, &outs);
  return commit_node(c, n, ins, outs);
}

}  // namespace rew
