// Jit execution of rew's StableHLO modules.
//
// rew's jit/lazy trace a function into a StableHLO module and hand its text
// to PJRT (src/rew/transform/jit.nim:216-229 -> executeJit,
// src/rew/eager.nim:1782-1847).  This file is the mi355x side of that call:
//
//   * a parser for the textual form rew's emitter writes
//     (src/rew/stablehlo/text.nim: the pretty forms of the elementwise,
//     reshape/transpose/broadcast_in_dim/slice/concatenate/compare/select/
//     clamp/dot_general/reduce ops and constants, and the quoted generic form
//     "stablehlo.x"(...) ({regions}) {attrs} : (types) -> types used for
//     iota, convert, torch_index_select, sort, gather, scatter, ...);
//   * a translator that turns each op into the graph node the matching eager
//     op records (prepare_node, the same validation and output derivation),
//     with stablehlo.reduce mapped onto reduceSum/Max/Min/Prod by its reducer
//     body, stablehlo.sort onto the row-sort node, stablehlo.gather /
//     scatter onto the general index-map nodes, and the sort+slice pair
//     rew's topK traces (src/rew/ops/sort.nim:36-90) onto one topK node;
//   * a per-context module cache keyed like rew's jitExecCache
//     (ordinal::name::cacheKey::hash(text)), whose entries hold prepared
//     node prototypes and the module's constants on the device, so a call
//     only copies nodes and links them to its inputs.
//
// Nodes join the deferred graph like eager ops, so a lazy batch lowers
// through the same fused kernels (flash attention, GEMM epilogues, routed
// MoE) as the eager op stream and is launched at the next flush.
#include <chrono>
#include <cmath>
#include <cerrno>
#include <cstring>
#include <deque>
#include <memory>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "kernels.h"
#include "plan.h"
#include "runtime.h"

namespace rew {

namespace {

using Attrs = std::vector<std::pair<std::string, std::string>>;

// ---- parsed form ----------------------------------------------------------------

struct Ty {
  int dt = -1;  // -1: a type the backend has no dtype for
  std::vector<int64_t> d;
  std::string text;
};

struct Op {
  std::string name;  // mnemonic without quotes, e.g. "stablehlo.add"
  int line = 0;
  std::vector<int> res;  // value slots defined
  std::vector<int> arg;  // value slots used
  std::vector<Ty> res_ty;
  bool bare_sig = false;  // ": T" signature (result type only)
  // op-specific operands of the pretty forms
  std::vector<int64_t> l0, l1, l2, l3;
  std::string word;             // compare direction
  std::string bytes;            // constant raw bytes
  bool splat = false;           // constant dense<number>
  std::string splat_text;       // the number as written ("1", "-2.5e-3", "0xFF800000")
  Attrs attrs;                  // generic attribute dictionary (raw values)
  std::vector<std::vector<int>> region_args;
  std::vector<std::vector<Op>> regions;
};

struct Func {
  std::string name;
  bool is_private = false;
  std::vector<int> args;
  std::vector<Ty> arg_ty;
  std::vector<Op> ops;
  std::vector<int> ret;
};

[[noreturn]] void unsupported(const std::string& m) { fail(REW_MI355X_ERR_UNSUPPORTED, m); }

int elem_dtype(const std::string& e) {
  static const std::unordered_map<std::string, int> m = {
      {"i1", kBool},   {"i8", kI8},     {"i16", kI16},         {"i32", kI32},
      {"i64", kI64},   {"ui8", kU8},    {"ui16", kU16},        {"ui32", kU32},
      {"ui64", kU64},  {"f16", kF16},   {"bf16", kBF16},       {"f32", kF32},
      {"f64", kF64},   {"i4", kI4},     {"ui4", kU4},          {"f8E4M3FN", kF8E4M3},
      {"f8E5M2", kF8E5M2}, {"complex<f32>", kC64}, {"complex<f64>", kC128}};
  auto it = m.find(e);
  return it == m.end() ? -1 : it->second;
}

class Parser {
 public:
  Parser(const char* s, size_t n, const std::string& who) : s_(s), n_(n), who_(who) {}

  std::vector<Func> module() {
    std::vector<Func> fs;
    expect_word("module");
    ws();
    if (peek('@')) {
      ++p_;
      name_chars();
    }
    if (eat_word("attributes")) skip_balanced('{', '}');
    expect("{");
    for (;;) {
      ws();
      if (eat("}")) break;
      if (eat_word("func.func")) {
        fs.push_back(func());
        continue;
      }
      if (p_ >= n_) err("unterminated module");
      // other top-level ops (sdy.mesh ...): skip the line
      while (p_ < n_ && s_[p_] != '\n') ++p_;
    }
    return fs;
  }

  int slots() const { return next_slot_; }

 private:
  const char* s_;
  size_t n_;
  size_t p_ = 0;
  std::string who_;
  std::unordered_map<std::string, int> names_;
  std::unordered_set<std::string> rew_alias_;  // names registered by rew_result_names
  int next_slot_ = 0;

  int line_at(size_t p) const {
    int l = 1;
    for (size_t i = 0; i < p && i < n_; ++i) l += s_[i] == '\n';
    return l;
  }
  [[noreturn]] void err(const std::string& m) const {
    invalid(who_ + ": StableHLO text line " + std::to_string(line_at(p_)) + ": " + m);
  }
  void ws() {
    while (p_ < n_) {
      const char ch = s_[p_];
      if (ch == ' ' || ch == '\t' || ch == '\n' || ch == '\r') {
        ++p_;
      } else if (ch == '/' && p_ + 1 < n_ && s_[p_ + 1] == '/') {
        while (p_ < n_ && s_[p_] != '\n') ++p_;
      } else {
        break;
      }
    }
  }
  bool peek(char ch) {
    ws();
    return p_ < n_ && s_[p_] == ch;
  }
  bool eat(const char* lit) {
    ws();
    const size_t l = std::strlen(lit);
    if (p_ + l <= n_ && std::memcmp(s_ + p_, lit, l) == 0) {
      p_ += l;
      return true;
    }
    return false;
  }
  static bool ident_char(char ch) {
    return std::isalnum((unsigned char)ch) || ch == '_' || ch == '.' || ch == '$';
  }
  bool eat_word(const char* w) {
    ws();
    const size_t l = std::strlen(w);
    if (p_ + l <= n_ && std::memcmp(s_ + p_, w, l) == 0 &&
        (p_ + l == n_ || !ident_char(s_[p_ + l]))) {
      p_ += l;
      return true;
    }
    return false;
  }
  void expect(const char* lit) {
    if (!eat(lit)) err(std::string("expected '") + lit + "'");
  }
  void expect_word(const char* w) {
    if (!eat_word(w)) err(std::string("expected '") + w + "'");
  }
  std::string name_chars() {
    const size_t b = p_;
    while (p_ < n_ && (ident_char(s_[p_]) ||
                       (s_[p_] == '-' && p_ + 1 < n_ && s_[p_ + 1] != '>')))
      ++p_;
    return std::string(s_ + b, p_ - b);
  }
  std::string word() {
    ws();
    std::string w = name_chars();
    if (w.empty()) err("expected a name");
    return w;
  }
  std::string value_name() {
    ws();
    if (!peek('%')) err("expected an SSA value");
    ++p_;
    std::string nm = name_chars();
    if (nm.empty()) err("empty SSA value name");
    return nm;
  }
  int use_value() {
    std::string nm = value_name();
    if (p_ < n_ && s_[p_] == '#') {  // %r#1: result 1 of a multi-result op
      ++p_;
      nm += "#" + name_chars();
    }
    auto it = names_.find(nm);
    if (it == names_.end()) err("use of undefined value %" + nm);
    return it->second;
  }
  int define(const std::string& nm) {
    if (names_.count(nm) && !rew_alias_.count(nm)) err("redefinition of %" + nm);
    rew_alias_.erase(nm);
    const int s = next_slot_++;
    names_[nm] = s;
    return s;
  }
  // rew's emitter prints a multi-result if / while as `%vN:K = ...` but then
  // names result i by its own id, %v(N+i) (text.nim:995-1001, 1106-1111 with
  // valueRef); those names are registered too, unless the text defines them
  // itself later.
  void rew_result_names(const std::string& base, const std::vector<int>& res) {
    if (base.size() < 2 || base[0] != 'v') return;
    for (size_t i = 1; i < base.size(); ++i)
      if (!std::isdigit((unsigned char)base[i])) return;
    const long long n0 = std::atoll(base.c_str() + 1);
    for (size_t i = 0; i < res.size(); ++i) {
      const std::string nm = "v" + std::to_string(n0 + (long long)i);
      if (names_.count(nm)) continue;
      names_.emplace(nm, res[i]);
      rew_alias_.insert(nm);
    }
  }
  int64_t integer() {
    ws();
    const char* b = s_ + p_;
    char* e = nullptr;
    const long long v = std::strtoll(b, &e, 10);
    if (e == b) err("expected an integer");
    p_ += (size_t)(e - b);
    return (int64_t)v;
  }
  std::vector<int64_t> int_list() {
    std::vector<int64_t> v;
    expect("[");
    if (eat("]")) return v;
    for (;;) {
      v.push_back(integer());
      if (eat("]")) break;
      expect(",");
    }
    return v;
  }
  void skip_balanced(char open, char close) {
    ws();
    if (p_ >= n_ || s_[p_] != open) err(std::string("expected '") + open + "'");
    int depth = 0;
    bool str = false;
    for (; p_ < n_; ++p_) {
      const char ch = s_[p_];
      if (str) {
        if (ch == '\\') ++p_;
        else if (ch == '"') str = false;
        continue;
      }
      if (ch == '"') str = true;
      else if (ch == open) ++depth;
      else if (ch == close && --depth == 0) {
        ++p_;
        return;
      }
    }
    err("unbalanced brackets");
  }

  Ty type() {
    ws();
    Ty t;
    const size_t b = p_;
    if (!eat("tensor<")) {
      if (peek('!') || eat_word("tuple"))
        unsupported(who_ + ": StableHLO text line " + std::to_string(line_at(p_)) +
                    ": only tensor types are supported by the mi355x backend");
      err("expected a tensor type");
    }
    for (;;) {
      ws();
      if (p_ < n_ && std::isdigit((unsigned char)s_[p_])) {
        t.d.push_back(integer());
        if (p_ < n_ && s_[p_] == 'x') {
          ++p_;
          continue;
        }
        err("expected 'x' after a dimension");
      }
      if (p_ < n_ && s_[p_] == '?')
        unsupported(who_ + ": dynamic dimensions are not supported by the mi355x backend");
      break;
    }
    std::string e;
    if (eat("complex<")) {
      e = "complex<" + name_chars() + ">";
      expect(">");
    } else {
      e = name_chars();
    }
    t.dt = elem_dtype(e);
    if (t.dt < 0) err("unknown element type '" + e + "'");
    if (eat(",")) skip_balanced('{', '}');  // encoding attribute
    expect(">");
    ws();
    t.text.assign(s_ + b, p_ - b);
    return t;
  }

  // "(T, T) -> T" or "(T) -> (T, T)" or "T" or "T, T"; returns the
  // result types (bare lists: the last type)
  std::vector<Ty> signature(bool* bare) {
    expect(":");
    std::vector<Ty> out;
    if (eat("(")) {
      if (!eat(")")) {
        for (;;) {
          type();
          if (eat(")")) break;
          expect(",");
        }
      }
      expect("->");
      if (eat("(")) {
        if (!eat(")")) {
          for (;;) {
            out.push_back(type());
            if (eat(")")) break;
            expect(",");
          }
        }
      } else {
        out.push_back(type());
      }
      *bare = false;
      return out;
    }
    std::vector<Ty> all;
    all.push_back(type());
    while (eat(",")) all.push_back(type());
    out.push_back(all.back());
    *bare = true;
    return out;
  }

  // key = value pairs with raw values (balanced up to the next top-level
  // ',' or '}')
  void attr_dict(Attrs* out) {
    expect("{");
    if (eat("}")) return;
    for (;;) {
      std::string k = word();
      expect("=");
      ws();
      const size_t b = p_;
      int depth = 0;
      bool str = false;
      for (; p_ < n_; ++p_) {
        const char ch = s_[p_];
        if (str) {
          if (ch == '\\') ++p_;
          else if (ch == '"') str = false;
          continue;
        }
        if (ch == '"') str = true;
        else if (ch == '<' || ch == '[' || ch == '(' || ch == '{') ++depth;
        else if (ch == '>' || ch == ']' || ch == ')' || ch == '}') {
          if (depth == 0) break;
          if (ch == '>' && p_ > 0 && s_[p_ - 1] == '-') continue;
          --depth;
        } else if (ch == ',' && depth == 0) {
          break;
        }
      }
      std::string v(s_ + b, p_ - b);
      while (!v.empty() && std::isspace((unsigned char)v.back())) v.pop_back();
      out->emplace_back(k, v);
      if (eat("}")) return;
      expect(",");
    }
  }

  // region body: statements up to the closing '}' (consumed)
  void region_body(std::vector<Op>* ops) {
    for (;;) {
      if (eat("}")) return;
      if (p_ >= n_) err("unterminated region");
      std::vector<int> unused;
      bool ended = false;
      stmt(ops, &unused, &ended);
    }
  }

  // '{' opening an attribute dictionary ("{name = ..."), not a body
  bool attr_dict_ahead() {
    if (!peek('{')) return false;
    size_t q = p_ + 1;
    while (q < n_ && std::isspace((unsigned char)s_[q])) ++q;
    const size_t b = q;
    while (q < n_ && (ident_char(s_[q]) || s_[q] == '"')) ++q;
    if (q == b) return false;
    while (q < n_ && (s_[q] == ' ' || s_[q] == '\t')) ++q;
    return q < n_ && s_[q] == '=';
  }

  Func func() {
    Func f;
    if (eat_word("private")) f.is_private = true;
    else eat_word("public");
    expect("@");
    f.name = name_chars();
    expect("(");
    if (!eat(")")) {
      for (;;) {
        f.args.push_back(define(value_name()));
        expect(":");
        f.arg_ty.push_back(type());
        if (peek('{')) skip_balanced('{', '}');  // argument attributes (sdy.sharding)
        if (eat(")")) break;
        expect(",");
      }
    }
    if (eat("->")) {
      if (eat("(")) {
        if (!eat(")")) {
          for (;;) {
            type();
            if (peek('{')) skip_balanced('{', '}');
            if (eat(")")) break;
            expect(",");
          }
        }
      } else {
        type();
        if (attr_dict_ahead()) skip_balanced('{', '}');
      }
    }
    if (eat_word("attributes")) skip_balanced('{', '}');
    expect("{");
    bool ended = false;
    for (;;) {
      if (eat("}")) break;
      if (p_ >= n_) err("unterminated function");
      stmt(&f.ops, &f.ret, &ended);
    }
    if (!ended) err("function @" + f.name + " has no func.return");
    return f;
  }

  void stmt(std::vector<Op>* ops, std::vector<int>* ret, bool* ended) {
    ws();
    const int line = line_at(p_);
    if (eat_word("func.return") || eat_word("return")) {
      ret->clear();
      if (peek('%')) {
        for (;;) {
          ret->push_back(use_value());
          if (!eat(",")) break;
        }
        expect(":");
        type();
        while (eat(",")) type();
      }
      *ended = true;
      return;
    }
    if (eat_word("stablehlo.return") || eat("\"stablehlo.return\"")) {
      Op op;
      op.name = "stablehlo.return";
      op.line = line;
      const bool generic = eat("(");
      if (peek('%')) {
        for (;;) {
          op.arg.push_back(use_value());
          if (!eat(",")) break;
        }
      }
      if (generic) expect(")");
      if (peek(':')) {
        bool bare = false;
        if (generic) {
          expect(":");
          skip_balanced('(', ')');
          expect("->");
          skip_balanced('(', ')');
        } else {
          signature(&bare);
        }
      }
      ops->push_back(std::move(op));
      return;
    }
    // results
    std::vector<std::string> names;
    std::vector<std::pair<std::string, size_t>> groups;  // %nm:K, first index
    for (;;) {
      std::string nm = value_name();
      if (eat(":")) {
        const int64_t k = integer();
        groups.push_back({nm, names.size()});
        for (int64_t i = 0; i < k; ++i) names.push_back(nm + "#" + std::to_string(i));
      } else {
        names.push_back(nm);
      }
      if (!eat(",")) break;
    }
    expect("=");
    Op op;
    op.line = line;
    body(&op);
    if (op.res_ty.size() != names.size())
      err(op.name + " defines " + std::to_string(names.size()) + " value(s) but its type " +
          "lists " + std::to_string(op.res_ty.size()));
    // results are defined after the operands (and region values) were used
    for (auto& nm : names) op.res.push_back(define(nm));
    for (auto& g : groups) {
      std::vector<int> rs;
      for (size_t i = g.second; i < names.size() && names[i].rfind(g.first + "#", 0) == 0; ++i)
        rs.push_back(op.res[i]);
      rew_result_names(g.first, rs);
    }
    ops->push_back(std::move(op));
  }

  void regions(Op* op) {
    for (;;) {
      expect("{");
      std::vector<int> args;
      if (eat("^")) {
        name_chars();
        if (eat("(")) {
          if (!eat(")")) {
            for (;;) {
              args.push_back(define(value_name()));
              expect(":");
              type();
              if (eat(")")) break;
              expect(",");
            }
          }
        }
        expect(":");
      }
      op->region_args.push_back(args);
      op->regions.emplace_back();
      region_body(&op->regions.back());
      if (!eat(",")) break;
    }
  }

  void body(Op* op) {
    ws();
    if (peek('"')) {  // generic form
      ++p_;
      const size_t b = p_;
      while (p_ < n_ && s_[p_] != '"') ++p_;
      if (p_ >= n_) err("unterminated op name");
      op->name.assign(s_ + b, p_ - b);
      ++p_;
      expect("(");
      if (!eat(")")) {
        for (;;) {
          op->arg.push_back(use_value());
          if (eat(")")) break;
          expect(",");
        }
      }
      if (eat("(")) {
        regions(op);
        expect(")");
      }
      if (peek('{')) attr_dict(&op->attrs);
      op->res_ty = signature(&op->bare_sig);
      return;
    }
    op->name = word();
    if (op->name == "stablehlo.constant") {
      expect("dense<");
      ws();
      if (eat("\"0x")) {
        auto hex = [&](char ch) -> int {
          if (ch >= '0' && ch <= '9') return ch - '0';
          if (ch >= 'a' && ch <= 'f') return ch - 'a' + 10;
          if (ch >= 'A' && ch <= 'F') return ch - 'A' + 10;
          err("bad hex digit in a dense constant");
        };
        while (p_ + 1 < n_ && s_[p_] != '"') {
          op->bytes.push_back((char)(hex(s_[p_]) * 16 + hex(s_[p_ + 1])));
          p_ += 2;
        }
        expect("\"");
      } else if (eat_word("true")) {
        op->splat = true;
        op->splat_text = "1";
      } else if (eat_word("false")) {
        op->splat = true;
        op->splat_text = "0";
      } else {
        // a decimal number, or an unquoted hex literal (MLIR's form of a
        // float's bit pattern, e.g. dense<0xFF800000> for -inf)
        size_t len = 0;
        while (p_ + len < n_ && (std::isalnum((unsigned char)s_[p_ + len]) ||
                                 s_[p_ + len] == '.' || s_[p_ + len] == '+' ||
                                 s_[p_ + len] == '-'))
          ++len;
        const std::string tok(s_ + p_, len);
        bool ok = len > 0;
        if (ok && (tok.rfind("0x", 0) == 0 || tok.rfind("0X", 0) == 0)) {
          ok = tok.size() > 2 && tok.size() <= 18 &&
               tok.find_first_not_of("0123456789abcdefABCDEF", 2) == std::string::npos;
        } else if (ok) {
          char* e = nullptr;
          (void)std::strtod(tok.c_str(), &e);
          ok = e == tok.c_str() + tok.size();
        }
        if (!ok)
          unsupported(who_ + ": StableHLO text line " + std::to_string(line_at(p_)) +
                      ": only hex and splat dense constants are supported");
        p_ += len;
        op->splat = true;
        op->splat_text = tok;
      }
      expect(">");
      op->res_ty = signature(&op->bare_sig);
      return;
    }
    if (op->name == "stablehlo.compare") {
      op->word = word();
      expect(",");
      op->arg.push_back(use_value());
      expect(",");
      op->arg.push_back(use_value());
      if (eat(",")) word();  // comparison type
      op->res_ty = signature(&op->bare_sig);
      return;
    }
    if (op->name == "stablehlo.reduce") {
      expect("(");
      op->arg.push_back(use_value());
      expect_word("init");
      expect(":");
      op->arg.push_back(use_value());
      expect(")");
      if (peek(','))
        unsupported(who_ + ": multi-operand stablehlo.reduce is not supported by the mi355x "
                           "backend");
      expect_word("across");
      expect_word("dimensions");
      expect("=");
      op->l0 = int_list();
      op->res_ty = signature(&op->bare_sig);
      expect_word("reducer");
      expect("(");
      std::vector<int> args;
      for (;;) {
        args.push_back(define(value_name()));
        expect(":");
        type();
        if (eat(")")) break;
        expect(",");
      }
      op->region_args.push_back(args);
      expect("{");
      op->regions.emplace_back();
      region_body(&op->regions.back());
      return;
    }
    // pretty op: operands, then keyword attributes, an optional slice
    // range list, then the signature
    for (;;) {
      ws();
      if (peek('%')) {
        op->arg.push_back(use_value());
        if (eat(",")) continue;
        break;
      }
      if (p_ < n_ && std::isalpha((unsigned char)s_[p_])) {
        std::string k = word();
        expect("=");
        if (k == "dims") {
          op->l0 = int_list();
        } else if (k == "batching_dims") {
          op->l0 = int_list();
          expect_word("x");
          op->l1 = int_list();
        } else if (k == "contracting_dims") {
          op->l2 = int_list();
          expect_word("x");
          op->l3 = int_list();
        } else if (k == "dim") {
          op->l0 = {integer()};
        } else {
          err("unknown keyword attribute '" + k + "' of " + op->name);
        }
        if (eat(",")) continue;
        break;
      }
      break;
    }
    if (eat("[")) {  // slice: [start:limit(:stride), ...]
      if (!eat("]")) {
        for (;;) {
          op->l0.push_back(integer());
          expect(":");
          op->l1.push_back(integer());
          op->l2.push_back(eat(":") ? integer() : 1);
          if (eat("]")) break;
          expect(",");
        }
      }
    }
    op->res_ty = signature(&op->bare_sig);
  }
};

// ---- translated form ----------------------------------------------------------------

struct Step;
// A region of a control-flow op: its argument slots, its steps and the
// slots its stablehlo.return hands back.
struct Block {
  std::vector<int> args;
  std::vector<Step> steps;
  std::vector<int> ret;
};
enum StepKind : int { kStepNode = 0, kStepWhile = 1, kStepIf = 2, kStepCase = 3, kStepEager = 4 };
struct Step {
  Node proto;  // prepared node: typed attributes set, no operands
  std::vector<int> in, out;
  std::vector<std::pair<int, Shape>> outs;
  // control flow (kind != kStepNode): `in` holds the op's n_opnd operands
  // (while: the initial carry; if / case: the predicate / branch index),
  // then every slot the regions read from outside them (for liveness)
  int kind = kStepNode;
  int n_opnd = 0;
  std::vector<Block> blocks;
  // kStepEager: the eager op recorded at call time (record_op), for ops the
  // library composes from several nodes or that read operand values
  std::string eager_op;
  Attrs eager_attrs;
};

}  // namespace

struct JitModule {
  std::string name;
  int n_slots = 0;
  std::vector<int> arg_slot;
  std::vector<std::pair<int, Shape>> arg_ty;
  std::vector<std::pair<int, Tensor*>> consts;  // slot, tensor (one reference each)
  std::vector<Step> steps;
  std::vector<int> ret;
  bool has_control = false;  // while / if / case steps (run host-side per call)
  int64_t calls = 0;
  // direct plans (plan.h) by input key, for modules of at least
  // kDirectMinSteps steps called with nothing else pending
  std::unordered_map<std::string, DirectPlan> direct;
};

namespace {

std::string shape_text(const std::vector<int64_t>& d) {
  std::string s = "[";
  for (size_t i = 0; i < d.size(); ++i) s += (i ? "," : "") + std::to_string(d[i]);
  return s + "]";
}

std::string type_text(int dt, const Shape& s) { return dt_enum_name(dt) + s.str(); }

const std::string* attr_raw(const Op& op, const char* key) {
  for (auto& kv : op.attrs)
    if (kv.first == key) return &kv.second;
  return nullptr;
}

// "#stablehlo.gather<offset_dims = [1], ..., index_vector_dim = 1>" (and
// the scatter form) -> "name" -> list; a scalar entry becomes a one-element
// list (src/rew/stablehlo/ops.nim:170-188 renders them).
std::unordered_map<std::string, std::vector<int64_t>> dim_numbers(const std::string& raw,
                                                                  const std::string& who) {
  std::unordered_map<std::string, std::vector<int64_t>> m;
  const size_t lt = raw.find('<'), gt = raw.rfind('>');
  if (lt == std::string::npos || gt == std::string::npos || gt < lt)
    invalid(who + ": malformed dimension numbers '" + raw + "'");
  size_t p = lt + 1;
  while (p < gt) {
    while (p < gt && (raw[p] == ' ' || raw[p] == ',')) ++p;
    const size_t eq = raw.find('=', p);
    if (eq == std::string::npos || eq > gt) break;
    std::string k = raw.substr(p, eq - p);
    while (!k.empty() && k.back() == ' ') k.pop_back();
    p = eq + 1;
    while (p < gt && raw[p] == ' ') ++p;
    std::vector<int64_t> v;
    if (raw[p] == '[') {
      const size_t e = raw.find(']', p);
      if (e == std::string::npos) invalid(who + ": malformed dimension numbers '" + raw + "'");
      std::string body = raw.substr(p + 1, e - p - 1);
      size_t q = 0;
      while (q < body.size()) {
        while (q < body.size() && (body[q] == ' ' || body[q] == ',')) ++q;
        if (q >= body.size()) break;
        char* end = nullptr;
        v.push_back(std::strtoll(body.c_str() + q, &end, 10));
        q = (size_t)(end - body.c_str());
        if (end == body.c_str()) break;
      }
      p = e + 1;
    } else {
      char* end = nullptr;
      v.push_back(std::strtoll(raw.c_str() + p, &end, 10));
      p = (size_t)(end - raw.c_str());
    }
    m[k] = v;
  }
  return m;
}

// "array<i64: 1, 3>" -> {1, 3}
// "array<i64: 1, 2>" or rew's "[1, 2]" (text.nim renderI64Array)
std::vector<int64_t> i64_array(const std::string& raw, const std::string& who) {
  std::string body;
  if (!raw.empty() && raw[0] == '[' && raw.back() == ']') {
    body = raw.substr(1, raw.size() - 2);
  } else {
    const size_t c = raw.find(':'), e = raw.rfind('>');
    if (raw.compare(0, 6, "array<") != 0 || c == std::string::npos || e == std::string::npos)
      invalid(who + ": malformed i64 array '" + raw + "'");
    body = raw.substr(c + 1, e - c - 1);
  }
  std::vector<int64_t> v;
  size_t q = 0;
  while (q < body.size()) {
    while (q < body.size() && (body[q] == ' ' || body[q] == ',')) ++q;
    if (q >= body.size()) break;
    char* end = nullptr;
    v.push_back(std::strtoll(body.c_str() + q, &end, 10));
    if (end == body.c_str() + q) break;
    q = (size_t)(end - body.c_str());
  }
  return v;
}

int64_t attr_int(const Op& op, const char* key, const std::string& who) {
  for (auto& kv : op.attrs)
    if (kv.first == key) {
      const char* b = kv.second.c_str();
      char* e = nullptr;
      const long long v = std::strtoll(b, &e, 10);
      if (e == b) invalid(who + ": attribute " + key + " is not an integer");
      return (int64_t)v;
    }
  invalid(who + ": missing attribute " + key);
}

const char* binary_name(const std::string& m) {
  static const std::unordered_map<std::string, const char*> t = {
      {"stablehlo.add", "add"},         {"stablehlo.subtract", "sub"},
      {"stablehlo.multiply", "mul"},    {"stablehlo.divide", "divide"},
      {"stablehlo.maximum", "maximum"}, {"stablehlo.minimum", "minimum"},
      {"stablehlo.power", "power"},     {"stablehlo.remainder", "remainder"},
      {"stablehlo.atan2", "atan2"},     {"stablehlo.and", "bitwiseAnd"},
      {"stablehlo.or", "bitwiseOr"},    {"stablehlo.xor", "bitwiseXor"},
      {"stablehlo.shift_left", "shiftLeft"},
      {"stablehlo.shift_right_arithmetic", "shiftRightArithmetic"},
      {"stablehlo.shift_right_logical", "shiftRightLogical"}};
  auto it = t.find(m);
  return it == t.end() ? nullptr : it->second;
}

const char* unary_name(const std::string& m) {
  static const std::unordered_map<std::string, const char*> t = {
      {"stablehlo.negate", "neg"},
      {"stablehlo.abs", "abs"},
      {"stablehlo.exponential", "exp"},
      {"stablehlo.log", "log"},
      {"stablehlo.sqrt", "sqrt"},
      {"stablehlo.rsqrt", "rsqrt"},
      {"stablehlo.tanh", "tanh"},
      {"stablehlo.logistic", "logistic"},
      {"stablehlo.sine", "sine"},
      {"stablehlo.cosine", "cosine"},
      {"stablehlo.floor", "floor"},
      {"stablehlo.ceil", "ceil"},
      {"stablehlo.sign", "sign"},
      {"stablehlo.cbrt", "cbrt"},
      {"stablehlo.exponential_minus_one", "expm1"},
      {"stablehlo.log_plus_one", "log1p"},
      {"stablehlo.tan", "tan"},
      {"stablehlo.round_nearest_afz", "roundNearestAfz"},
      {"stablehlo.round_nearest_even", "roundNearestEven"},
      {"stablehlo.not", "bitwiseNot"},
      {"stablehlo.count_leading_zeros", "countLeadingZeros"},
      {"stablehlo.popcnt", "popcnt"},
      {"stablehlo.optimization_barrier", "optimizationBarrier"},
      {"stablehlo.is_finite", "isFinite"}};
  auto it = t.find(m);
  return it == t.end() ? nullptr : it->second;
}

class Translator {
 public:
  Translator(Ctx* c, JitModule* m, const std::string& who) : c_(c), m_(m), who_(who) {}

  void run(const Func& f, int n_parsed_slots) {
    slot_dt_.assign(n_parsed_slots, -1);
    slot_shape_.assign(n_parsed_slots, Shape());
    alias_.assign(n_parsed_slots, -1);
    is_const_.assign(n_parsed_slots, -1);
    def_op_.assign(n_parsed_slots, -1);
    for (size_t i = 0; i < f.ops.size(); ++i)
      for (int r : f.ops[i].res) def_op_[r] = (int)i;
    uses_.assign(n_parsed_slots, {});
    for (size_t i = 0; i < f.ops.size(); ++i) {
      for (int a : f.ops[i].arg) uses_[a].push_back((int)i);
      for (const auto& r : f.ops[i].regions) region_uses(r);
    }
    ret_use_.assign(n_parsed_slots, false);
    for (int r : f.ret) ret_use_[r] = true;
    redirect_.assign(f.ops.size(), -1);

    for (size_t i = 0; i < f.args.size(); ++i) {
      const Ty& t = f.arg_ty[i];
      if (t.dt < 0) unsupported(who_ + ": argument type " + t.text + " not supported");
      set_slot(f.args[i], t.dt, Shape(t.d));
      m_->arg_slot.push_back(f.args[i]);
      m_->arg_ty.push_back({t.dt, Shape(t.d)});
    }
    f_ = &f;
    for (size_t i = 0; i < f.ops.size(); ++i) op(f.ops[i], (int)i);
    for (int r : f.ret) m_->ret.push_back(resolve(r));
    m_->n_slots = (int)slot_dt_.size();
    prune();
  }

  ~Translator() {
    for (Tensor* t : phantoms_) delete t;
  }

 private:
  Ctx* c_;
  JitModule* m_;
  std::string who_;
  const Func* f_ = nullptr;
  std::vector<int> slot_dt_;
  std::vector<Shape> slot_shape_;
  std::vector<int> alias_, is_const_, def_op_, redirect_;
  std::vector<std::vector<int>> uses_;
  std::vector<bool> ret_use_;
  std::vector<Tensor*> phantoms_;
  std::unordered_map<std::string, std::pair<int, int>> topk_;  // (x, k, largest) -> slots

  // uses inside regions count as -1 (no peephole looks into a region)
  void region_uses(const std::vector<Op>& ops) {
    for (const Op& o : ops) {
      for (int a : o.arg)
        if (a >= 0 && a < (int)uses_.size()) uses_[a].push_back(-1);
      for (const auto& r : o.regions) region_uses(r);
    }
  }

  [[noreturn]] void fail_at(const Op& o, const std::string& m, int code = REW_MI355X_ERR_INVALID) {
    fail(code, who_ + ": line " + std::to_string(o.line) + ": " + o.name + ": " + m);
  }

  int resolve(int s) const {
    while (s < (int)alias_.size() && alias_[s] >= 0) s = alias_[s];
    return s;
  }
  void set_slot(int s, int dt, Shape sh) {  // by value: sh may live in slot_shape_
    if (s >= (int)slot_dt_.size()) {
      slot_dt_.resize(s + 1, -1);
      slot_shape_.resize(s + 1);
      alias_.resize(s + 1, -1);
      is_const_.resize(s + 1, -1);
    }
    slot_dt_[s] = dt;
    slot_shape_[s] = sh;
  }
  int new_slot(int dt, const Shape& sh) {
    const int s = (int)slot_dt_.size();
    set_slot(s, dt, sh);
    return s;
  }
  Tensor* phantom(int s) {
    s = resolve(s);
    Tensor* t = new Tensor();
    t->ctx = c_;
    t->dt = slot_dt_[s];
    t->shape = slot_shape_[s];
    phantoms_.push_back(t);
    return t;
  }

  // Prepares eager op `name` over slots `in`; returns its output slots.
  std::vector<int> step(const Op& o, const std::string& name, const std::vector<int>& in,
                        const Attrs& attrs) {
    std::vector<Tensor*> ph;
    std::vector<int> rin;
    for (int s : in) {
      rin.push_back(resolve(s));
      ph.push_back(phantom(s));
    }
    std::vector<std::pair<int, Shape>> outs;
    Node* n = nullptr;
    try {
      n = prepare_node(c_, name, ph, attrs, &outs);
    } catch (const Error& e) {
      fail(e.code, who_ + ": line " + std::to_string(o.line) + ": " + o.name + ": " +
                       e.what());
    }
    Step st;
    st.proto = *n;
    delete n;
    st.proto.in.clear();
    st.proto.out.clear();
    st.in = rin;
    for (auto& od : outs) st.out.push_back(new_slot(od.first, od.second));
    st.outs = outs;
    std::vector<int> res = st.out;
    m_->steps.push_back(std::move(st));
    return res;
  }

  // Binds the op's result slot r to `s` after checking the text's type.
  void bind(const Op& o, size_t r, int s) {
    s = resolve(s);
    const Ty& t = o.res_ty[r];
    if (t.dt != slot_dt_[s] || Shape(t.d) != slot_shape_[s])
      fail_at(o, "result type " + t.text + " but the operands give " +
                     type_text(slot_dt_[s], slot_shape_[s]));
    set_slot(o.res[r], slot_dt_[s], slot_shape_[s]);
    alias_[o.res[r]] = s;
  }

  int one(const Op& o, const std::string& name, const std::vector<int>& in,
          const Attrs& attrs) {
    std::vector<int> r = step(o, name, in, attrs);
    bind(o, 0, r[0]);
    return r[0];
  }

  void need_args(const Op& o, size_t n) {
    if (o.arg.size() != n)
      fail_at(o, "expected " + std::to_string(n) + " operand(s), got " +
                     std::to_string(o.arg.size()));
    if (o.res_ty.size() != 1) fail_at(o, "expected one result");
  }

  // One element of a splat constant of type t, little-endian, into `one`.
  // An unquoted hex literal is the element's bit pattern and must fit it.
  // Integer types take integers only, parsed exactly (no detour through
  // double) and range-checked; float types round the decimal value.
  void splat_element(const Op& o, const Ty& t, uint8_t* one) {
    const std::string& tok = o.splat_text;
    const int size = dt_size(t.dt);
    if (tok.rfind("0x", 0) == 0 || tok.rfind("0X", 0) == 0) {
      if ((int)tok.size() - 2 > 2 * size)
        fail_at(o, "hex constant " + tok + " is wider than " + t.text,
                REW_MI355X_ERR_UNSUPPORTED);
      const uint64_t bits = std::strtoull(tok.c_str() + 2, nullptr, 16);
      std::memcpy(one, &bits, (size_t)size);
      return;
    }
    if (dt_is_int(t.dt)) {
      if (tok.find_first_not_of("0123456789", tok[0] == '-' || tok[0] == '+' ? 1 : 0) !=
              std::string::npos || tok.size() < (tok[0] == '-' || tok[0] == '+' ? 2u : 1u))
        fail_at(o, "integer constant " + tok + " of type " + t.text + " is not an integer",
                REW_MI355X_ERR_UNSUPPORTED);
      const bool neg = tok[0] == '-';
      errno = 0;
      const uint64_t mag = std::strtoull(tok.c_str() + (neg || tok[0] == '+' ? 1 : 0), nullptr, 10);
      const int bits = 8 * size;
      const bool sgn = dt_is_signed(t.dt);
      const uint64_t max_pos = sgn ? (bits == 64 ? (uint64_t)INT64_MAX : (1ull << (bits - 1)) - 1)
                                   : (bits == 64 ? UINT64_MAX : (1ull << bits) - 1);
      const uint64_t max_neg = sgn ? (bits == 64 ? (uint64_t)INT64_MAX + 1 : 1ull << (bits - 1))
                                   : 0;
      if (errno == ERANGE || (neg ? mag > max_neg : mag > max_pos))
        fail_at(o, "integer constant " + tok + " is out of range for " + t.text,
                REW_MI355X_ERR_INVALID);
      const uint64_t u = neg ? (uint64_t)0 - mag : mag;  // two's complement
      std::memcpy(one, &u, (size_t)size);
      return;
    }
    const double v = std::strtod(tok.c_str(), nullptr);
    switch (t.dt) {
      case kF32: { float f = (float)v; std::memcpy(one, &f, 4); break; }
      case kF64: std::memcpy(one, &v, 8); break;
      case kBF16: {
        float f = (float)v;
        uint32_t u;
        std::memcpy(&u, &f, 4);
        const uint16_t h = std::isnan(f) ? (uint16_t)((u >> 16) | 0x40u)
                                         : (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
        std::memcpy(one, &h, 2);
        break;
      }
      case kF16: { _Float16 h = (_Float16)v; std::memcpy(one, &h, 2); break; }
      case kBool: one[0] = v != 0.0; break;
      default:
        fail_at(o, "decimal constant of type " + t.text + " not supported (write its bits "
                   "as hex)", REW_MI355X_ERR_UNSUPPORTED);
    }
  }

  void constant(const Op& o) {
    const Ty& t = o.res_ty.at(0);
    const Shape s(t.d);
    if (t.dt < 0 || t.dt == kC64 || t.dt == kC128 || t.dt == kI4 || t.dt == kU4 || t.dt == kNF4)
      fail_at(o, "constant type " + t.text + " not supported", REW_MI355X_ERR_UNSUPPORTED);
    const int64_t bytes = s.numel() * dt_size(t.dt);
    std::string host;
    if (o.splat) {
      host.resize((size_t)bytes);
      std::vector<uint8_t> one(dt_size(t.dt));
      splat_element(o, t, one.data());
      for (int64_t i = 0; i < s.numel(); ++i)
        std::memcpy(&host[(size_t)(i * one.size())], one.data(), one.size());
    } else {
      if ((int64_t)o.bytes.size() != bytes)
        fail_at(o, "dense data has " + std::to_string(o.bytes.size()) + " bytes, " + t.text +
                       " needs " + std::to_string(bytes));
      host = o.bytes;
    }
    Tensor* k = upload_tensor(c_, t.dt, s, host.data());
    m_->consts.push_back({o.res[0], k});
    set_slot(o.res[0], t.dt, s);
    is_const_[o.res[0]] = (int)m_->consts.size() - 1;
    const_bytes_.emplace(o.res[0], host);
  }
  std::unordered_map<int, std::string> const_bytes_;

  // the reducer / comparator: one op over the region's arguments plus a
  // stablehlo.return of its result
  const Op* single_body(const Op& o, size_t region) {
    const auto& body = o.regions.at(region);
    if (body.size() != 2 || body[1].name != "stablehlo.return" || body[1].arg.size() != 1 ||
        body[0].res.size() != 1 || body[1].arg[0] != body[0].res[0])
      return nullptr;
    return &body[0];
  }

  void reduce(const Op& o) {
    need_args(o, 2);
    const Op* b = single_body(o, 0);
    const auto& ra = o.region_args.at(0);
    static const std::unordered_map<std::string, const char*> red = {
        {"stablehlo.add", "reduceSum"},     {"stablehlo.maximum", "reduceMax"},
        {"stablehlo.minimum", "reduceMin"}, {"stablehlo.multiply", "reduceProd"},
        {"stablehlo.and", "all"},           {"stablehlo.or", "any"}};
    if (!b || ra.size() != 2 || b->arg.size() != 2 || !red.count(b->name) ||
        !((b->arg[0] == ra[0] && b->arg[1] == ra[1]) || (b->arg[0] == ra[1] && b->arg[1] == ra[0])))
      fail_at(o, "only reducers of one add/maximum/minimum/multiply/and/or are supported",
              REW_MI355X_ERR_UNSUPPORTED);
    const int x = o.arg[0], init = resolve(o.arg[1]);
    std::string dims = shape_text(o.l0);
    std::vector<int> r = step(o, red.at(b->name), {x}, {{"dims", dims}});
    // init: the op's identity is dropped; anything else is combined after
    bool identity = false;
    auto cb = const_bytes_.find(init);
    const int dt = slot_dt_[init];
    if (cb != const_bytes_.end() && slot_shape_[init].rank == 0) {
      const std::string& h = cb->second;
      if (dt == kF32) {
        float v;
        uint32_t u;
        std::memcpy(&v, h.data(), 4);
        std::memcpy(&u, h.data(), 4);
        if (b->name == "stablehlo.add") identity = u == 0u;
        else if (b->name == "stablehlo.maximum") identity = std::isinf(v) && v < 0;
        else if (b->name == "stablehlo.minimum") identity = std::isinf(v) && v > 0;
        else if (b->name == "stablehlo.multiply") identity = v == 1.0f;
      } else if (dt == kBool) {
        identity = (b->name == "stablehlo.and") ? h[0] != 0 : h[0] == 0;
      }
    }
    int out = r[0];
    if (!identity) {
      const Shape os = slot_shape_[out];
      std::vector<int64_t> od(os.d, os.d + os.rank);
      int bi = init;
      if (os.rank > 0)
        bi = step(o, "broadcastTo", {init},
                  {{"output_shape", shape_text(od)}, {"broadcast_dimensions", "[]"}})[0];
      out = step(o, binary_name(b->name), {out, bi}, {})[0];
    }
    bind(o, 0, out);
  }

  // (key operand, descending) of a one-compare comparator, or false
  bool comparator(const Op& o, int* key, int* desc) {
    const Op* b = single_body(o, 0);
    const auto& ra = o.region_args.at(0);
    if (!b || b->name != "stablehlo.compare" || b->arg.size() != 2) return false;
    for (size_t j = 0; 2 * j + 1 < ra.size(); ++j) {
      bool fwd = b->arg[0] == ra[2 * j] && b->arg[1] == ra[2 * j + 1];
      bool rev = b->arg[0] == ra[2 * j + 1] && b->arg[1] == ra[2 * j];
      if (!fwd && !rev) continue;
      const std::string& d = b->word;
      int dsc;
      if (d == "LT" || d == "LE") dsc = 0;
      else if (d == "GT" || d == "GE") dsc = 1;
      else return false;
      *key = (int)j;
      *desc = rev ? 1 - dsc : dsc;
      return true;
    }
    return false;
  }

  // k if op `op_index` slices the first k along `dim` (and nothing else)
  // of a value of shape `s`, else -1.
  int64_t head_slice(int op_index, int dim, const Shape& s) {
    const Op& u = f_->ops[op_index];
    if (u.name != "stablehlo.slice" || u.arg.size() != 1) return -1;
    if ((int)u.l0.size() != s.rank) return -1;
    for (int i = 0; i < s.rank; ++i) {
      if (u.l0[i] != 0 || u.l2[i] != 1) return -1;
      if (i != dim && u.l1[i] != s.d[i]) return -1;
    }
    return u.l1[dim];
  }

  // rew's traced topK (src/rew/ops/sort.nim:53-85): sort(x) and sort(x, iota)
  // with a GE/LE comparator on x, each result read only through a slice of
  // the first k along the sort dim.  Both become one topK node.
  bool topk_peephole(const Op& o, int op_index, int dim, int key, int desc) {
    if (key != 0 || o.arg.empty() || o.arg.size() > 2) return false;
    const int x = resolve(o.arg[0]);
    const Shape xs = slot_shape_[x];
    if (slot_dt_[x] != kF32 || dim != xs.rank - 1 || xs.d[dim] > kTopkMaxCols) return false;
    if (o.arg.size() == 2) {
      const int io = def_op_.at(o.arg[1]);
      if (io < 0) return false;
      const Op& iota = f_->ops[io];
      if (iota.name != "stablehlo.iota" || iota.res_ty[0].dt != kI32 ||
          attr_int(iota, "iota_dimension", who_) != dim)
        return false;
    }
    int64_t k = -1;
    for (size_t r = 0; r < o.res.size(); ++r) {
      if (ret_use_[o.res[r]]) return false;
      for (int u : uses_[o.res[r]]) {
        if (u < 0) return false;  // read inside a region
        const int64_t kk = head_slice(u, dim, xs);
        if (kk <= 0 || (k >= 0 && kk != k)) return false;
        k = kk;
      }
    }
    if (k <= 0 || k > 64) return false;
    const std::string tk = std::to_string(x) + ":" + std::to_string(k) + ":" + std::to_string(desc);
    auto it = topk_.find(tk);
    std::pair<int, int> vi;
    if (it != topk_.end()) {
      vi = it->second;
    } else {
      std::vector<int> r = step(o, "topK", {x},
                                {{"k", std::to_string(k)}, {"dimension", std::to_string(dim)},
                                 {"largest", desc ? "true" : "false"}});
      vi = {r[0], r[1]};
      topk_.emplace(tk, vi);
    }
    for (size_t r = 0; r < o.res.size(); ++r)
      for (int u : uses_[o.res[r]]) redirect_[u] = (r == 0) ? vi.first : vi.second;
    (void)op_index;
    return true;
  }

  void sort(const Op& o, int op_index) {
    if (o.arg.empty() || o.res.size() != o.arg.size())
      fail_at(o, "operand/result count mismatch");
    int key = 0, desc = 0;
    if (!comparator(o, &key, &desc))
      fail_at(o, "only comparators of one LT/LE/GT/GE compare of an operand pair are supported",
              REW_MI355X_ERR_UNSUPPORTED);
    const Shape s0 = slot_shape_[resolve(o.arg[0])];
    int64_t dim = attr_int(o, "dimension", who_);
    if (dim < 0) dim += s0.rank;
    if (dim < 0 || dim >= s0.rank) fail_at(o, "dimension out of range");
    if (topk_peephole(o, op_index, (int)dim, key, desc)) return;
    // sort along the last dim; other dims go through a transpose each way
    std::vector<int> in(o.arg.begin(), o.arg.end());
    std::vector<int64_t> perm;
    const bool moved = dim != s0.rank - 1;
    if (moved) {
      for (int i = 0; i < s0.rank; ++i)
        if (i != dim) perm.push_back(i);
      perm.push_back(dim);
      for (int& s : in) s = step(o, "transpose", {s}, {{"permutation", shape_text(perm)}})[0];
    }
    Attrs a = {{"dimension", std::to_string(s0.rank - 1)},
               {"comparison_direction", desc ? "GT" : "LT"},
               {"key", std::to_string(key)}};
    std::vector<int> r = step(o, "sort", in, a);
    if (moved) {
      std::vector<int64_t> inv(perm.size());
      for (size_t i = 0; i < perm.size(); ++i) inv[perm[i]] = (int64_t)i;
      for (int& s : r) s = step(o, "transpose", {s}, {{"permutation", shape_text(inv)}})[0];
    }
    for (size_t i = 0; i < r.size(); ++i) bind(o, i, r[i]);
  }

  static std::string ints(const std::vector<int64_t>& v) { return shape_text(v); }

  void gather(const Op& o) {
    need_args(o, 2);
    const std::string* dn = attr_raw(o, "dimension_numbers");
    const std::string* ss = attr_raw(o, "slice_sizes");
    if (!dn || !ss) fail_at(o, "missing dimension_numbers or slice_sizes");
    auto d = dim_numbers(*dn, who_);
    one(o, "gather", o.arg,
        {{"offset_dims", ints(d["offset_dims"])},
         {"collapsed_slice_dims", ints(d["collapsed_slice_dims"])},
         {"operand_batching_dims", ints(d["operand_batching_dims"])},
         {"start_indices_batching_dims", ints(d["start_indices_batching_dims"])},
         {"start_index_map", ints(d["start_index_map"])},
         {"index_vector_dim", std::to_string(d["index_vector_dim"].empty()
                                                 ? 0 : d["index_vector_dim"][0])},
         {"slice_sizes", ints(i64_array(*ss, who_))}});
  }

  // update computation of a one-input scatter: one op over (current,
  // update), or the update itself (replace)
  std::string scatter_update(const Op& o) {
    const auto& ra = o.region_args.at(0);
    const auto& body = o.regions.at(0);
    if (ra.size() != 2) return "";
    if (body.size() == 1 && body[0].name == "stablehlo.return" && body[0].arg.size() == 1 &&
        body[0].arg[0] == ra[1])
      return "replace";
    const Op* b = single_body(o, 0);
    if (!b || b->arg.size() != 2) return "";
    if (!((b->arg[0] == ra[0] && b->arg[1] == ra[1]) || (b->arg[0] == ra[1] && b->arg[1] == ra[0])))
      return "";
    if (b->name == "stablehlo.add") return "add";
    if (b->name == "stablehlo.maximum") return "maximum";
    if (b->name == "stablehlo.minimum") return "minimum";
    if (b->name == "stablehlo.multiply") return "multiply";
    return "";
  }

  void scatter(const Op& o) {
    if (o.arg.size() != 3 || o.res_ty.size() != 1)
      fail_at(o, "only one-input scatters are supported", REW_MI355X_ERR_UNSUPPORTED);
    const std::string* dn = attr_raw(o, "scatter_dimension_numbers");
    if (!dn) fail_at(o, "missing scatter_dimension_numbers");
    const std::string uc = scatter_update(o);
    if (uc.empty())
      fail_at(o, "only update computations of one add/maximum/minimum/multiply or a plain "
                 "replacement are supported", REW_MI355X_ERR_UNSUPPORTED);
    auto d = dim_numbers(*dn, who_);
    one(o, "scatter", o.arg,
        {{"update_window_dims", ints(d["update_window_dims"])},
         {"inserted_window_dims", ints(d["inserted_window_dims"])},
         {"input_batching_dims", ints(d["input_batching_dims"])},
         {"scatter_indices_batching_dims", ints(d["scatter_indices_batching_dims"])},
         {"scatter_dims_to_operand_dims", ints(d["scatter_dims_to_operand_dims"])},
         {"index_vector_dim", std::to_string(d["index_vector_dim"].empty()
                                                 ? 0 : d["index_vector_dim"][0])},
         {"update_computation", uc}});
  }

  void op(const Op& o, int index) {
    const std::string& n = o.name;
    if (index >= 0 && redirect_[index] >= 0) {  // a slice the topK peephole answers
      bind(o, 0, redirect_[index]);
      return;
    }
    if (const char* b = binary_name(n)) {
      need_args(o, 2);
      one(o, b, o.arg, {});
      return;
    }
    if (const char* u = unary_name(n)) {
      need_args(o, 1);
      one(o, u, o.arg, {});
      return;
    }
    const Ty* rt = o.res_ty.empty() ? nullptr : &o.res_ty[0];
    if (n == "stablehlo.constant") {
      if (!o.arg.empty() || o.res_ty.size() != 1) fail_at(o, "malformed constant");
      constant(o);
    } else if (n == "stablehlo.convert") {
      need_args(o, 1);
      if (rt->dt < 0) fail_at(o, "unsupported result type", REW_MI355X_ERR_UNSUPPORTED);
      one(o, "astype", o.arg, {{"dtype", dt_enum_name(rt->dt)}});
    } else if (n == "stablehlo.bitcast_convert") {
      need_args(o, 1);
      one(o, "bitcastConvert", o.arg,
          {{"dtype", dt_enum_name(rt->dt)}, {"shape", shape_text(rt->d)}});
    } else if (n == "stablehlo.reshape") {
      need_args(o, 1);
      one(o, "reshape", o.arg, {{"shape", shape_text(rt->d)}});
    } else if (n == "stablehlo.transpose") {
      need_args(o, 1);
      one(o, "transpose", o.arg, {{"permutation", shape_text(o.l0)}});
    } else if (n == "stablehlo.reverse") {
      need_args(o, 1);
      one(o, "reverse", o.arg, {{"dimensions", shape_text(o.l0)}});
    } else if (n == "stablehlo.broadcast_in_dim") {
      need_args(o, 1);
      one(o, "broadcastTo", o.arg,
          {{"output_shape", shape_text(rt->d)}, {"broadcast_dimensions", shape_text(o.l0)}});
    } else if (n == "stablehlo.slice") {
      need_args(o, 1);
      one(o, "slice", o.arg,
          {{"start_indices", shape_text(o.l0)}, {"limit_indices", shape_text(o.l1)},
           {"strides", shape_text(o.l2)}});
    } else if (n == "stablehlo.concatenate") {
      if (o.arg.empty() || o.res_ty.size() != 1) fail_at(o, "malformed concatenate");
      if (o.l0.size() != 1) fail_at(o, "missing dim");
      one(o, "concat", o.arg, {{"dimension", std::to_string(o.l0[0])}});
    } else if (n == "stablehlo.iota") {
      if (!o.arg.empty() || o.res_ty.size() != 1) fail_at(o, "malformed iota");
      if (rt->dt < 0) fail_at(o, "unsupported result type", REW_MI355X_ERR_UNSUPPORTED);
      one(o, "iota", {},
          {{"dtype", dt_enum_name(rt->dt)}, {"shape", shape_text(rt->d)},
           {"dimension", std::to_string(attr_int(o, "iota_dimension", who_))}});
    } else if (n == "stablehlo.compare") {
      need_args(o, 2);
      one(o, "compare", o.arg, {{"comparison_direction", o.word}});
    } else if (n == "stablehlo.select") {
      need_args(o, 3);
      one(o, "select", o.arg, {});
    } else if (n == "stablehlo.clamp") {
      need_args(o, 3);
      one(o, "clamp", o.arg, {});
    } else if (n == "stablehlo.dot_general") {
      need_args(o, 2);
      one(o, "dotGeneral", o.arg,
          {{"lhs_batching", shape_text(o.l0)}, {"rhs_batching", shape_text(o.l1)},
           {"lhs_contracting", shape_text(o.l2)}, {"rhs_contracting", shape_text(o.l3)}});
    } else if (n == "stablehlo.dot") {
      need_args(o, 2);
      one(o, "dot", o.arg, {});
    } else if (n == "stablehlo.torch_index_select") {
      need_args(o, 2);
      one(o, "torchIndexSelect", o.arg,
          {{"dim", std::to_string(attr_int(o, "dim", who_))},
           {"batch_dims", std::to_string(attr_int(o, "batch_dims", who_))}});
    } else if (n == "stablehlo.reduce") {
      reduce(o);
    } else if (n == "stablehlo.sort") {
      sort(o, index);
    } else if (n == "stablehlo.pad") {
      // rew's generic form (src/rew/stablehlo/text.nim:589-622)
      need_args(o, 2);
      const std::string* lo = attr_raw(o, "edge_padding_low");
      const std::string* hi = attr_raw(o, "edge_padding_high");
      const std::string* in = attr_raw(o, "interior_padding");
      if (!lo || !hi || !in) fail_at(o, "missing padding attributes");
      one(o, "pad", o.arg,
          {{"edge_padding_low", ints(i64_array(*lo, who_))},
           {"edge_padding_high", ints(i64_array(*hi, who_))},
           {"interior_padding", ints(i64_array(*in, who_))}});
    } else if (n == "stablehlo.dynamic_slice") {
      // (src/rew/stablehlo/text.nim:645-669)
      if (o.arg.size() < 2 || o.res_ty.size() != 1) fail_at(o, "malformed dynamic_slice");
      const std::string* ss = attr_raw(o, "slice_sizes");
      if (!ss) fail_at(o, "missing slice_sizes");
      one(o, "dynamicSlice", o.arg, {{"slice_sizes", ints(i64_array(*ss, who_))}});
    } else if (n == "stablehlo.dynamic_update_slice") {
      // (src/rew/stablehlo/text.nim:671-690)
      if (o.arg.size() < 3 || o.res_ty.size() != 1) fail_at(o, "malformed dynamic_update_slice");
      one(o, "dynamicUpdateSlice", o.arg, {});
    } else if (n == "stablehlo.while" || n == "stablehlo.if" || n == "stablehlo.case") {
      control(o);
    } else if (n == "stablehlo.einsum" || n == "stablehlo.unary_einsum") {
      // (text.nim:1696-1728)
      const std::string* cfg = attr_raw(o, "einsum_config");
      if (!cfg) fail_at(o, "missing einsum_config");
      need_args(o, n == "stablehlo.einsum" ? 2 : 1);
      eager_step(o, n == "stablehlo.einsum" ? "einsum" : "unaryEinsum",
                 {{"einsum_config", unquote(*cfg)}, {"output_shape", shape_text(rt->d)}});
    } else if (n == "stablehlo.triangular_solve") {
      // (text.nim:1645-1695): transpose_a = #stablehlo<transpose KIND>
      need_args(o, 2);
      Attrs at;
      for (const char* k : {"left_side", "lower", "unit_diagonal"}) {
        const std::string* v = attr_raw(o, k);
        if (!v) fail_at(o, std::string("missing ") + k);
        at.push_back({k, *v});
      }
      const std::string* ta = attr_raw(o, "transpose_a");
      if (!ta) fail_at(o, "missing transpose_a");
      std::string kind = unquote(*ta);
      const size_t sp = kind.find_last_of(' ');
      if (sp != std::string::npos) kind = kind.substr(sp + 1);
      while (!kind.empty() && kind.back() == '>') kind.pop_back();
      at.push_back({"transpose_a", kind});
      one(o, "triangularSolve", o.arg, at);
    } else if (n == "stablehlo.complex") {
      need_args(o, 2);
      one(o, "complex", o.arg, {});
    } else if (n == "stablehlo.real" || n == "stablehlo.imag") {
      need_args(o, 1);
      one(o, n == "stablehlo.real" ? "real" : "imag", o.arg, {});
    } else if (n == "stablehlo.fft") {
      // (text.nim emitFftAt): fft_type = #stablehlo<fft_type KIND>, fft_length = [..]
      need_args(o, 1);
      const std::string* ft = attr_raw(o, "fft_type");
      const std::string* fl = attr_raw(o, "fft_length");
      if (!ft || !fl) fail_at(o, "missing fft_type / fft_length");
      std::string kind = unquote(*ft);
      const size_t sp = kind.find_last_of(' ');
      if (sp != std::string::npos) kind = kind.substr(sp + 1);
      while (!kind.empty() && kind.back() == '>') kind.pop_back();
      eager_step(o, "fft", {{"fft_type", kind}, {"fft_length", shape_text(i64_array(*fl, who_))}});
    } else if (n == "stablehlo.dynamic_pad" || n == "stablehlo.real_dynamic_slice") {
      // (text.nim:780-801): the index operands are read when the module runs
      need_args(o, n == "stablehlo.dynamic_pad" ? 5 : 4);
      eager_step(o, n == "stablehlo.dynamic_pad" ? "dynamicPad" : "realDynamicSlice",
                 {{"result_shape", shape_text(rt->d)}});
    } else if (n == "stablehlo.dynamic_broadcast_in_dim") {
      // (text.nim:1575-1610): a broadcast to the static result type
      need_args(o, 2);
      const std::string* bd = attr_raw(o, "broadcast_dimensions");
      if (!bd) fail_at(o, "missing broadcast_dimensions");
      one(o, "broadcastTo", {o.arg[0]},
          {{"output_shape", shape_text(rt->d)},
           {"broadcast_dimensions", shape_text(i64_array(*bd, who_))}});
    } else if (n == "stablehlo.gather") {
      gather(o);
    } else if (n == "stablehlo.scatter") {
      scatter(o);
    } else {
      fail_at(o, "op not supported by the mi355x jit path", REW_MI355X_ERR_UNSUPPORTED);
    }
  }

  static std::string unquote(std::string v) {
    while (!v.empty() && v.back() == ' ') v.pop_back();
    if (v.size() >= 2 && v.front() == '"' && v.back() == '"') v = v.substr(1, v.size() - 2);
    return v;
  }

  // An op the call records through the eager path (record_op), typed by the
  // text's result type.
  void eager_step(const Op& o, const std::string& name, const Attrs& attrs) {
    const Ty& t = o.res_ty[0];
    if (t.dt < 0) fail_at(o, "unsupported result type", REW_MI355X_ERR_UNSUPPORTED);
    Step st;
    st.kind = kStepEager;
    st.eager_op = name;
    st.eager_attrs = attrs;
    for (int a : o.arg) st.in.push_back(resolve(a));
    st.n_opnd = (int)st.in.size();
    set_slot(o.res[0], t.dt, Shape(t.d));
    st.out.push_back(o.res[0]);
    st.outs.push_back({t.dt, Shape(t.d)});
    m_->steps.push_back(std::move(st));
    m_->has_control = true;  // (may read operands back: no direct plan)
  }

  // ---- control flow (src/rew/transform/control.nim: cond / whileLoop / fori
  // trace stablehlo.if and stablehlo.while; the text is text.nim's emitIf /
  // emitWhile).  Each region is translated into a Block over the module's
  // slots; the call runs the regions on the host side (instantiate), reading
  // each predicate back from the device, as PJRT's executable does.

  // The region's ops as a Block whose argument slots carry `types`.
  Block block(const Op& o, size_t r, const std::vector<std::pair<int, Shape>>& types) {
    const auto& args = o.region_args.at(r);
    if (args.size() != types.size())
      fail_at(o, "region " + std::to_string(r) + " takes " + std::to_string(args.size()) +
                     " argument(s), expected " + std::to_string(types.size()));
    Block b;
    for (size_t i = 0; i < args.size(); ++i) {
      set_slot(args[i], types[i].first, types[i].second);
      b.args.push_back(args[i]);
    }
    std::vector<Step> saved;
    saved.swap(m_->steps);
    bool returned = false;
    for (const Op& ro : o.regions[r]) {
      if (returned) fail_at(ro, "op after the region's stablehlo.return");
      if (ro.name == "stablehlo.return") {
        for (int a : ro.arg) b.ret.push_back(resolve(a));
        returned = true;
        continue;
      }
      op(ro, -1);
    }
    b.steps.swap(m_->steps);
    m_->steps.swap(saved);
    if (!returned) fail_at(o, "region " + std::to_string(r) + " has no stablehlo.return");
    return b;
  }

  // The region's results have the types `types`.
  void check_ret(const Op& o, const Block& b, size_t r,
                 const std::vector<std::pair<int, Shape>>& types) {
    if (b.ret.size() != types.size())
      fail_at(o, "region " + std::to_string(r) + " returns " + std::to_string(b.ret.size()) +
                     " value(s), expected " + std::to_string(types.size()));
    for (size_t i = 0; i < types.size(); ++i)
      if (slot_dt_[b.ret[i]] != types[i].first || slot_shape_[b.ret[i]] != types[i].second)
        fail_at(o, "region " + std::to_string(r) + " result " + std::to_string(i) + " is " +
                       type_text(slot_dt_[b.ret[i]], slot_shape_[b.ret[i]]) + ", expected " +
                       type_text(types[i].first, types[i].second));
  }

  // Slots a block reads that it does not define (outer values it captures).
  static void captured(const Block& b, std::vector<int>* out) {
    std::vector<int> defined(b.args.begin(), b.args.end());
    auto is_def = [&](int s) {
      for (int d : defined)
        if (d == s) return true;
      return false;
    };
    auto need = [&](int s) {
      if (is_def(s)) return;
      for (int x : *out)
        if (x == s) return;
      out->push_back(s);
    };
    for (const Step& st : b.steps) {
      for (int s : st.in) need(s);
      for (int s : st.out) defined.push_back(s);
    }
    for (int s : b.ret) need(s);
  }

  void control(const Op& o) {
    const std::string& n = o.name;
    Step st;
    std::vector<std::pair<int, Shape>> res_types;
    for (const Ty& t : o.res_ty) {
      if (t.dt < 0) fail_at(o, "result type " + t.text + " not supported", REW_MI355X_ERR_UNSUPPORTED);
      res_types.push_back({t.dt, Shape(t.d)});
    }
    if (o.res.size() != res_types.size()) fail_at(o, "result count mismatch");
    auto scalar = [&](int s, int dt, const char* what) {
      s = resolve(s);
      if (slot_dt_[s] != dt || slot_shape_[s].rank != 0)
        fail_at(o, std::string(what) + " must be a " + dt_enum_name(dt) + " scalar, got " +
                       type_text(slot_dt_[s], slot_shape_[s]));
    };
    if (n == "stablehlo.while") {
      // "stablehlo.while"(%init...) ({^cond(...): ... return(%pred)}, {^body(...): ...
      // return(%next...)}) (text.nim:1091-1130)
      if (o.arg.empty() || o.regions.size() != 2) fail_at(o, "expected a carry and two regions");
      std::vector<std::pair<int, Shape>> carry;
      for (int a : o.arg) {
        const int s = resolve(a);
        carry.push_back({slot_dt_[s], slot_shape_[s]});
      }
      if (res_types != carry) fail_at(o, "result types differ from the carry's");
      st.kind = kStepWhile;
      st.blocks.push_back(block(o, 0, carry));
      check_ret(o, st.blocks[0], 0, {{kBool, Shape()}});
      st.blocks.push_back(block(o, 1, carry));
      check_ret(o, st.blocks[1], 1, carry);
    } else if (n == "stablehlo.if") {
      // "stablehlo.if"(%pred) ({then ...}, {else ...}) (text.nim:984-1020)
      if (o.arg.size() != 1 || o.regions.size() != 2) fail_at(o, "expected a predicate and two regions");
      scalar(o.arg[0], kBool, "the predicate");
      st.kind = kStepIf;
      for (size_t r = 0; r < 2; ++r) {
        st.blocks.push_back(block(o, r, {}));
        check_ret(o, st.blocks[r], r, res_types);
      }
    } else {
      // "stablehlo.case"(%index) ({branch 0}, ..., {branch N-1})
      if (o.arg.size() != 1 || o.regions.empty()) fail_at(o, "expected an index and regions");
      scalar(o.arg[0], kI32, "the branch index");
      st.kind = kStepCase;
      for (size_t r = 0; r < o.regions.size(); ++r) {
        st.blocks.push_back(block(o, r, {}));
        check_ret(o, st.blocks[r], r, res_types);
      }
    }
    for (int a : o.arg) st.in.push_back(resolve(a));
    st.n_opnd = (int)st.in.size();
    std::vector<int> cap;
    for (const Block& b : st.blocks) captured(b, &cap);
    for (int s : cap) st.in.push_back(s);
    for (size_t i = 0; i < o.res.size(); ++i) {
      set_slot(o.res[i], res_types[i].first, res_types[i].second);
      st.out.push_back(o.res[i]);
    }
    st.outs = res_types;
    m_->steps.push_back(std::move(st));
    m_->has_control = true;
  }

  // Drops steps none of whose outputs reach a func.return.
  void prune() {
    std::vector<bool> live(m_->n_slots, false);
    for (int r : m_->ret) live[r] = true;
    std::vector<Step> kept;
    for (size_t i = m_->steps.size(); i-- > 0;) {
      Step& st = m_->steps[i];
      bool any = false;
      for (int o : st.out) any = any || live[o];
      if (!any) continue;
      for (int s : st.in) live[s] = true;
      kept.push_back(std::move(st));
    }
    m_->steps.assign(std::make_move_iterator(kept.rbegin()),
                     std::make_move_iterator(kept.rend()));
    std::vector<std::pair<int, Tensor*>> consts;
    for (auto& kc : m_->consts) {
      if (live[kc.first]) {
        consts.push_back(kc);
      } else {
        kc.second->ext--;
        maybe_destroy(kc.second);
      }
    }
    m_->consts.swap(consts);
  }
};

uint64_t text_hash(const char* s, size_t n) {
  uint64_t h = 0x243f6a8885a308d3ull ^ (uint64_t)n;
  size_t i = 0;
  for (; i + 8 <= n; i += 8) {
    uint64_t w;
    std::memcpy(&w, s + i, 8);
    h = (h ^ w) * 0x9e3779b97f4a7c15ull;
    h ^= h >> 29;
  }
  uint64_t w = 0;
  std::memcpy(&w, s + i, n - i);
  h = (h ^ w) * 0x9e3779b97f4a7c15ull;
  h ^= h >> 32;
  return h;
}

void destroy_module(JitModule* m) {
  for (auto& kc : m->consts) {
    kc.second->ext--;
    maybe_destroy(kc.second);
  }
  delete m;
}

JitModule* compile_module(Ctx* c, const std::string& who, const char* text, size_t len) {
  Parser p(text, len, who);
  std::vector<Func> fs = p.module();
  const Func* f = nullptr;
  for (auto& x : fs)
    if (x.name == "main") f = &x;
  if (!f) {
    for (auto& x : fs)
      if (!x.is_private) {
        f = &x;
        break;
      }
  }
  if (!f) invalid(who + ": module has no public function");
  for (auto& x : fs)
    if (&x != f)
      unsupported(who + ": modules with more than one function are not supported");
  std::unique_ptr<JitModule> m(new JitModule());
  m->name = who;
  try {
    Translator t(c, m.get(), who);
    t.run(*f, p.slots());
  } catch (...) {
    for (auto& kc : m->consts) {
      kc.second->ext--;
      maybe_destroy(kc.second);
    }
    m->consts.clear();
    throw;
  }
  return m.release();
}

}  // namespace

namespace {

// Modules this large run directly once their plan is recorded: their host
// cost is the graph they would otherwise build and flush on every call.
constexpr size_t kDirectMinSteps = 64;
constexpr size_t kDirectMaxPlans = 8;  // per module, all dropped when exceeded

// What a flush of the module alone may depend on beyond the module itself:
// the context's lowering flags and, per input, which earlier input is the
// same tensor or shares its storage, the address bits alignment checks read
// and the host bytes of small constants (the flush signature's leaf terms).
std::string direct_key(Ctx* c, const std::vector<Tensor*>& ins) {
  std::string k;
  k.reserve(ins.size() * 12 + 4);
  k.push_back((char)((c->no_fusion_patterns ? 1 : 0) | (c->profiling ? 2 : 0) |
                     (c->dense_moe ? 4 : 0)));
  std::unordered_map<const Tensor*, int32_t> first_t;
  std::unordered_map<const Storage*, int32_t> first_s;
  for (size_t i = 0; i < ins.size(); ++i) {
    const Tensor* t = ins[i];
    const int32_t ti = first_t.emplace(t, (int32_t)i).first->second;
    const int32_t si = first_s.emplace(t->st, (int32_t)i).first->second;
    const uint8_t lo = (uint8_t)((uintptr_t)t->st->ptr & 255);
    k.append((const char*)&ti, 4);
    k.append((const char*)&si, 4);
    k.push_back((char)lo);
    k.push_back(t->has_host ? 1 : 0);
    if (t->has_host) k.append((const char*)t->host, sizeof t->host);
  }
  return k;
}

void release_all(std::vector<Tensor*>* ts) {
  for (Tensor* t : *ts) {
    t->ext--;
    maybe_destroy(t);
  }
  ts->clear();
}

// The value of a scalar (bool or i32) result, read back from the device:
// the pending graph is flushed first, as rew_mi355x_to_host does.
int64_t read_scalar(Ctx* c, Tensor* t) {
  if (t->prod) flush(c);
  if (!t->st) invalid("jit: control-flow predicate has no data (an earlier flush failed)");
  int64_t v = 0;
  const size_t n = (size_t)t->nbytes();
  if (n > sizeof v) invalid("jit: control-flow predicate is not a scalar");
  REW_HIP(hipMemcpyAsync(&v, t->data(), n, hipMemcpyDeviceToHost, c->stream));
  REW_HIP(hipStreamSynchronize(c->stream));
  if (t->dt == kBool) return (v & 0xff) != 0;
  return (int64_t)(int32_t)(uint32_t)v;
}

void run_steps(Ctx* c, const std::vector<Step>& steps, std::vector<Tensor*>& v,
               std::vector<Tensor*>& made);

// Runs block b with arguments `args`; returns its results, each with one
// owner reference.  Everything else the block made is released.
std::vector<Tensor*> run_block(Ctx* c, const Block& b, const std::vector<Tensor*>& args,
                               std::vector<Tensor*>& v) {
  for (size_t i = 0; i < args.size(); ++i) v[b.args[i]] = args[i];
  std::vector<Tensor*> made;
  try {
    run_steps(c, b.steps, v, made);
  } catch (...) {
    release_all(&made);
    throw;
  }
  std::vector<Tensor*> res;
  for (int r : b.ret) {
    v[r]->ext++;
    res.push_back(v[r]);
  }
  release_all(&made);
  return res;
}

// A control step (src/rew/transform/control.nim): the chosen region of an
// if / case, or the loop of a while, its predicate read back each turn.
// Results go into v and `made` (one owner reference each).
void run_control(Ctx* c, const Step& st, std::vector<Tensor*>& v, std::vector<Tensor*>& made) {
  std::vector<Tensor*> res;
  if (st.kind == kStepWhile) {
    std::vector<Tensor*> carry;
    for (int i = 0; i < st.n_opnd; ++i) {
      v[st.in[i]]->ext++;
      carry.push_back(v[st.in[i]]);
    }
    try {
      for (;;) {
        std::vector<Tensor*> p = run_block(c, st.blocks[0], carry, v);
        bool go;
        try {
          go = read_scalar(c, p[0]) != 0;
        } catch (...) {
          release_all(&p);
          throw;
        }
        release_all(&p);
        if (!go) break;
        std::vector<Tensor*> next = run_block(c, st.blocks[1], carry, v);
        release_all(&carry);
        carry.swap(next);
      }
    } catch (...) {
      release_all(&carry);
      throw;
    }
    res.swap(carry);
  } else {
    int64_t k = read_scalar(c, v[st.in[0]]);
    const int nb = (int)st.blocks.size();
    if (st.kind == kStepIf) k = k ? 0 : 1;  // then, else
    else if (k < 0 || k >= nb) k = nb - 1;  // stablehlo.case: out of range -> last
    res = run_block(c, st.blocks[(size_t)k], {}, v);
  }
  for (size_t j = 0; j < res.size(); ++j) {
    v[st.out[j]] = res[j];
    made.push_back(res[j]);
  }
}

void run_steps(Ctx* c, const std::vector<Step>& steps, std::vector<Tensor*>& v,
               std::vector<Tensor*>& made) {
  std::vector<Tensor*> in;
  for (const Step& st : steps) {
    if (st.kind == kStepEager) {
      in.clear();
      for (int s : st.in) in.push_back(v[s]);
      std::vector<Tensor*> outs = record_op(c, st.eager_op, in, st.eager_attrs);
      for (size_t j = 0; j < outs.size(); ++j) made.push_back(outs[j]);
      if (outs.size() != st.out.size() || outs[0]->dt != st.outs[0].first ||
          outs[0]->shape != st.outs[0].second)
        invalid("jit: " + st.eager_op + " gives " + type_text(outs[0]->dt, outs[0]->shape) +
                ", the module's type is " + type_text(st.outs[0].first, st.outs[0].second));
      for (size_t j = 0; j < outs.size(); ++j) v[st.out[j]] = outs[j];
      continue;
    }
    if (st.kind != kStepNode) {
      run_control(c, st, v, made);
      continue;
    }
    in.clear();
    for (int s : st.in) in.push_back(v[s]);
    Node* n = new Node(st.proto);
    std::vector<Tensor*> outs = commit_node(c, n, in, st.outs);
    for (size_t j = 0; j < outs.size(); ++j) {
      v[st.out[j]] = outs[j];
      made.push_back(outs[j]);
    }
  }
}

// The module's nodes committed to the pending graph; its results, each
// with one owner reference.
std::vector<Tensor*> instantiate(Ctx* c, JitModule* m, const std::vector<Tensor*>& ins) {
  std::vector<Tensor*> v(m->n_slots, nullptr);
  for (size_t i = 0; i < ins.size(); ++i) v[m->arg_slot[i]] = ins[i];
  for (auto& kc : m->consts) v[kc.first] = kc.second;
  std::vector<Tensor*> made;
  made.reserve(m->steps.size() * 2);
  try {
    run_steps(c, m->steps, v, made);
  } catch (...) {
    release_all(&made);
    throw;
  }
  std::vector<Tensor*> res;
  for (int r : m->ret) {
    Tensor* t = v[r];
    t->ext++;
    res.push_back(t);
  }
  for (Tensor* t : made) {
    t->ext--;
    maybe_destroy(t);
  }
  return res;
}

// The direct plan of a flush that ran module m alone (`cap`), or a plan
// marked not replayable.
DirectPlan make_direct(Ctx* c, JitModule* m, const std::vector<Tensor*>& ins,
                       const std::vector<Tensor*>& res, const FlushCapture& cap) {
  DirectPlan d;
  d.epoch = c->plan_epoch;
  if (!cap.done) return d;
  auto pit = c->flush_plans.find(cap.sig);
  if (pit == c->flush_plans.end() || !pit->second->ok) return d;
  std::unordered_map<const Tensor*, int32_t> src;
  for (size_t i = 0; i < ins.size(); ++i) src.emplace(ins[i], (int32_t)i);
  for (size_t k = 0; k < m->consts.size(); ++k)
    src.emplace(m->consts[k].second, -1 - (int32_t)k);
  for (Tensor* t : cap.leaves) {
    auto it = src.find(t);
    if (it == src.end()) return d;
    d.leaf_src.push_back(it->second);
  }
  for (Tensor* t : res) {
    auto it = cap.out_ref.find(t);
    if (it == cap.out_ref.end()) return d;  // a result that is an input or a constant
    d.results.push_back(it->second);
  }
  d.plan = *pit->second;
  d.node_meta = cap.node_meta;
  d.ok = true;
  return d;
}

}  // namespace

std::vector<Tensor*> jit_module_run(Ctx* c, const std::string& name, const std::string& cache_key,
                             const char* text, size_t len, const std::vector<Tensor*>& ins) {
  const std::string who = "jit '" + name + "'";
  std::string key = std::to_string(c->ordinal) + "::" + name + "::" + cache_key + "::";
  char hx[17];
  std::snprintf(hx, sizeof hx, "%016llx", (unsigned long long)text_hash(text, len));
  key += hx;
  auto it = c->jit_modules.find(key);
  JitModule* m;
  if (it != c->jit_modules.end()) {
    m = it->second;
    c->stats.jit_module_hits++;
  } else {
    m = compile_module(c, who, text, len);
    c->jit_modules.emplace(key, m);
    c->stats.jit_module_compiles++;
  }
  if (ins.size() != m->arg_slot.size())
    invalid(who + ": module takes " + std::to_string(m->arg_slot.size()) + " input(s), got " +
            std::to_string(ins.size()));
  // (a module with control flow flushes inside the call, per predicate)
  bool direct = c->mode == REW_MI355X_MODE_DEFERRED && c->plan_cache && c->pending.empty() &&
                m->steps.size() >= kDirectMinSteps && !m->has_control;
  for (size_t i = 0; i < ins.size(); ++i) {
    if (ins[i]->dt != m->arg_ty[i].first || ins[i]->shape != m->arg_ty[i].second)
      invalid(who + ": input " + std::to_string(i) + " is " + type_text(ins[i]->dt, ins[i]->shape) +
              ", the module expects " + type_text(m->arg_ty[i].first, m->arg_ty[i].second));
    direct = direct && ins[i]->st;
  }
  m->calls++;
  if (!direct) return instantiate(c, m, ins);
  // rew's executeJit runs the module at once (eager.nim:1782-1847): with
  // nothing else pending, the module's graph is flushed here, and later
  // calls with the same input key replay that flush's plan directly
  const std::string dk = direct_key(c, ins);
  auto dit = m->direct.find(dk);
  if (dit != m->direct.end() && dit->second.epoch != c->plan_epoch) {
    m->direct.erase(dit);
    dit = m->direct.end();
  }
  if (dit != m->direct.end()) {
    if (!dit->second.ok) return instantiate(c, m, ins);
    const auto t0 = std::chrono::steady_clock::now();
    std::vector<Tensor*> leaves;
    leaves.reserve(dit->second.leaf_src.size());
    for (int32_t s : dit->second.leaf_src)
      leaves.push_back(s >= 0 ? ins[s] : m->consts[-1 - s].second);
    std::vector<Tensor*> res = plan_replay_direct(c, dit->second, leaves);
    c->stats.flushes++;
    c->stats.flush_plan_hits++;
    c->stats.flush_host_ns += std::chrono::duration_cast<std::chrono::nanoseconds>(
                                  std::chrono::steady_clock::now() - t0).count();
    return res;
  }
  std::vector<Tensor*> res = instantiate(c, m, ins);
  FlushCapture cap;
  c->capture = &cap;
  try {
    flush(c);
  } catch (...) {
    c->capture = nullptr;
    for (Tensor* t : res) {
      t->ext--;
      maybe_destroy(t);
    }
    throw;
  }
  c->capture = nullptr;
  if (m->direct.size() >= kDirectMaxPlans) m->direct.clear();
  m->direct.emplace(dk, make_direct(c, m, ins, res, cap));
  return res;
}

void jit_module_cache_clear(Ctx* c) {
  for (auto& kv : c->jit_modules) destroy_module(kv.second);
  c->jit_modules.clear();
}

}  // namespace rew
