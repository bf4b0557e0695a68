// StableHLO textual-assembly reader.
//
// The reference deserializes the portable artifact with the StableHLO
// library (src/jam/parse.cc:53-63) and walks MLIR objects.  Neither MLIR nor
// StableHLO exists in this image, so jam reads the textual form directly:
// the module/func structure, SSA values, tensor types, attributes, the
// generic op syntax ("stablehlo.op"(...) <{...}> ({...}) {...} : (...) -> ...)
// and the custom pretty syntax JAX prints for the ops of the hot path
// (dot_general, broadcast_in_dim, reduce ... applies / reducer, compare,
// select, iota, transpose, reshape, convert, constant, slice, concatenate,
// call, return).  `loc(...)` annotations and `#loc` alias lines are skipped.
#include <cctype>
#include <cstdlib>
#include <cstring>
#include <sstream>
#include <unordered_map>

#include "jam/ir.h"

namespace mi::jam {

// ------------------------------------------------------------------ dtypes
int DTypeBytes(DType d) {
  switch (d) {
    case DType::kPred: case DType::kI8: case DType::kU8: return 1;
    case DType::kI16: case DType::kU16: case DType::kF16: case DType::kBF16: return 2;
    case DType::kI32: case DType::kU32: case DType::kF32: return 4;
    case DType::kI64: case DType::kU64: case DType::kF64: return 8;
    default: return 0;
  }
}
bool IsFloat(DType d) { return d == DType::kF16 || d == DType::kBF16 || d == DType::kF32 || d == DType::kF64; }
bool IsSigned(DType d) { return d == DType::kI8 || d == DType::kI16 || d == DType::kI32 || d == DType::kI64; }
bool IsUnsigned(DType d) { return d == DType::kU8 || d == DType::kU16 || d == DType::kU32 || d == DType::kU64; }
const char* DTypeName(DType d) {
  switch (d) {
    case DType::kPred: return "i1";
    case DType::kI8: return "i8";
    case DType::kI16: return "i16";
    case DType::kI32: return "i32";
    case DType::kI64: return "i64";
    case DType::kU8: return "ui8";
    case DType::kU16: return "ui16";
    case DType::kU32: return "ui32";
    case DType::kU64: return "ui64";
    case DType::kF16: return "f16";
    case DType::kBF16: return "bf16";
    case DType::kF32: return "f32";
    case DType::kF64: return "f64";
    case DType::kToken: return "token";
    default: return "?";
  }
}
DType ParseElementType(const std::string& s) {
  static const std::unordered_map<std::string, DType> m = {
      {"i1", DType::kPred}, {"i8", DType::kI8}, {"i16", DType::kI16}, {"i32", DType::kI32},
      {"i64", DType::kI64}, {"si8", DType::kI8}, {"si16", DType::kI16}, {"si32", DType::kI32},
      {"si64", DType::kI64}, {"ui8", DType::kU8}, {"ui16", DType::kU16}, {"ui32", DType::kU32},
      {"ui64", DType::kU64}, {"f16", DType::kF16}, {"bf16", DType::kBF16}, {"f32", DType::kF32},
      {"f64", DType::kF64}};
  auto it = m.find(s);
  return it == m.end() ? DType::kInvalid : it->second;
}

std::string TensorType::str() const {
  std::string r = "tensor<";
  for (int64_t d : dims) r += std::to_string(d) + "x";
  return r + DTypeName(dtype) + ">";
}

std::vector<int64_t> Attr::ints() const {
  std::vector<int64_t> r;
  if (kind == kList) {
    for (const Attr& a : list) r.push_back(a.kind == kFloat ? int64_t(a.f) : a.i);
  } else if (kind == kDense) {
    r = ivals;
  } else if (kind == kInt) {
    r.push_back(i);
  }
  return r;
}

bool IsMlirBytecode(const char* data, size_t size) {
  return size >= 4 && data[0] == 'M' && data[1] == 'L' && (unsigned char)data[2] == 0xEF && data[3] == 'R';
}

namespace {

// ------------------------------------------------------------------ lexer
enum class Tok { kEnd, kValue, kSymbol, kBare, kHash, kCaret, kString, kNumber, kPunct, kArrow };

struct Token {
  Tok kind = Tok::kEnd;
  std::string text;
  int line = 1;
};

class Lexer {
 public:
  Lexer(const char* p, size_t n) : p_(p), end_(p + n) {}

  Token next() {
    skip();
    Token t;
    t.line = line_;
    if (p_ >= end_) return t;
    const char c = *p_;
    if (c == '%' || c == '@' || c == '#' || c == '^') {
      const char* s = p_++;
      if (*p_ == '"') {  // quoted symbol
        ++p_;
        while (p_ < end_ && *p_ != '"') ++p_;
        ++p_;
      } else {
        while (p_ < end_ && (isalnum((unsigned char)*p_) || *p_ == '_' || *p_ == '.' || *p_ == '$' ||
                             *p_ == '-' || (c == '%' && *p_ == '#')))
          ++p_;
      }
      t.kind = c == '%' ? Tok::kValue : c == '@' ? Tok::kSymbol : c == '#' ? Tok::kHash : Tok::kCaret;
      t.text.assign(s, p_);
      return t;
    }
    if (c == '"') {
      ++p_;
      std::string s;
      while (p_ < end_ && *p_ != '"') {
        if (*p_ == '\\' && p_ + 1 < end_) {
          s.push_back(*p_++);
        }
        if (*p_ == '\n') ++line_;
        s.push_back(*p_++);
      }
      ++p_;
      t.kind = Tok::kString;
      t.text = s;
      return t;
    }
    if (c == '-' && p_ + 1 < end_ && p_[1] == '>') {
      p_ += 2;
      t.kind = Tok::kArrow;
      t.text = "->";
      return t;
    }
    if (isdigit((unsigned char)c) || ((c == '-' || c == '+') && p_ + 1 < end_ && isdigit((unsigned char)p_[1]))) {
      const char* s = p_++;
      if (c == '0' && p_ < end_ && (*p_ == 'x' || *p_ == 'X')) {
        ++p_;
        while (p_ < end_ && isxdigit((unsigned char)*p_)) ++p_;
      } else {
        while (p_ < end_ && (isdigit((unsigned char)*p_) || *p_ == '.')) ++p_;
        if (p_ < end_ && (*p_ == 'e' || *p_ == 'E') && p_ + 1 < end_ &&
            (isdigit((unsigned char)p_[1]) || p_[1] == '-' || p_[1] == '+')) {
          p_ += 2;
          while (p_ < end_ && isdigit((unsigned char)*p_)) ++p_;
        }
      }
      t.kind = Tok::kNumber;
      t.text.assign(s, p_);
      return t;
    }
    if (isalpha((unsigned char)c) || c == '_') {
      const char* s = p_++;
      while (p_ < end_ && (isalnum((unsigned char)*p_) || *p_ == '_' || *p_ == '.' || *p_ == '$')) ++p_;
      t.kind = Tok::kBare;
      t.text.assign(s, p_);
      return t;
    }
    ++p_;
    t.kind = Tok::kPunct;
    t.text = std::string(1, c);
    return t;
  }

  // raw text up to the '>' that closes an already-consumed '<'
  std::string raw_until_close_angle() {
    int depth = 1;
    const char* s = p_;
    while (p_ < end_) {
      if (*p_ == '"') {  // strings may contain '>'
        ++p_;
        while (p_ < end_ && *p_ != '"') ++p_;
      } else if (*p_ == '<') {
        ++depth;
      } else if (*p_ == '>') {
        if (--depth == 0) break;
      } else if (*p_ == '\n') {
        ++line_;
      }
      ++p_;
    }
    std::string r(s, p_);
    if (p_ < end_) ++p_;
    return r;
  }

  int line() const { return line_; }
  const char* pos() const { return p_; }
  void set_pos(const char* p, int line) { p_ = p; line_ = line; }

 private:
  void skip() {
    for (;;) {
      while (p_ < end_ && isspace((unsigned char)*p_)) {
        if (*p_ == '\n') ++line_;
        ++p_;
      }
      if (p_ + 1 < end_ && p_[0] == '/' && p_[1] == '/') {
        while (p_ < end_ && *p_ != '\n') ++p_;
        continue;
      }
      break;
    }
  }
  const char* p_;
  const char* end_;
  int line_ = 1;
};

// ------------------------------------------------------------------ parser
class Parser {
 public:
  Parser(const char* p, size_t n, Module& m) : lex_(p, n), m_(m) { advance(); }

  bool parse_module(std::string& err) {
    try {
      // optional `module @name attributes {...} {`
      bool wrapped = false;
      while (cur_.kind == Tok::kHash) skip_alias_definition();
      if (is_bare("module")) {
        advance();
        if (cur_.kind == Tok::kSymbol) {
          m_.name = cur_.text.substr(1);
          advance();
        }
        if (is_bare("attributes")) {
          advance();
          parse_attr_dict();
        }
        expect("{");
        wrapped = true;
      }
      for (;;) {
        while (cur_.kind == Tok::kHash) skip_alias_definition();
        if (cur_.kind == Tok::kEnd) break;
        if (wrapped && is_punct("}")) {
          advance();
          wrapped = false;
          continue;
        }
        if (is_bare("func.func") || is_bare("func")) {
          parse_func();
        } else {
          fail("expected func.func, got '" + cur_.text + "'");
        }
      }
      if (m_.funcs.empty()) fail("module has no functions");
      return true;
    } catch (const std::string& e) {
      err = e;
      return false;
    }
  }

 private:
  // -------------------------------------------------------------- helpers
  void advance() { cur_ = lex_.next(); }
  bool is_punct(const char* p) const { return cur_.kind == Tok::kPunct && cur_.text == p; }
  bool is_bare(const char* b) const { return cur_.kind == Tok::kBare && cur_.text == b; }
  [[noreturn]] void fail(const std::string& msg) const {
    throw std::string("jam: parse error at line " + std::to_string(cur_.line) + ": " + msg);
  }
  void expect(const char* p) {
    if (!is_punct(p)) fail(std::string("expected '") + p + "', got '" + cur_.text + "'");
    advance();
  }
  void expect_arrow() {
    if (cur_.kind != Tok::kArrow) fail("expected '->'");
    advance();
  }
  void skip_alias_definition() {  // `#loc1 = loc(...)` or `#map = ...` at top level
    const int line = cur_.line;
    advance();
    while (cur_.kind != Tok::kEnd && cur_.line == line) advance();
  }
  void skip_loc() {  // optional `loc(...)`
    if (is_bare("loc")) {
      advance();
      skip_balanced("(", ")");
    }
  }
  void skip_balanced(const char* open, const char* close) {
    expect(open);
    int depth = 1;
    while (depth > 0) {
      if (cur_.kind == Tok::kEnd) fail("unbalanced brackets");
      if (is_punct(open)) ++depth;
      else if (is_punct(close)) --depth;
      advance();
    }
  }

  // lookahead: is the token after the current one a scalar element type?
  bool next_is_element_type() {
    const char* pos = lex_.pos();
    const int line = lex_.line();
    Token t = lex_.next();
    lex_.set_pos(pos, line);
    return t.kind == Tok::kBare && ParseElementType(t.text) != DType::kInvalid;
  }

  // -------------------------------------------------------------- SSA scope
  int lookup(const std::string& name) {
    std::string base = name, idx;
    auto h = name.find('#');
    if (h != std::string::npos) {
      base = name.substr(0, h);
      idx = name.substr(h + 1);
    }
    auto it = scope_.find(base);
    if (it == scope_.end()) fail("use of undefined value " + name);
    const int k = idx.empty() ? 0 : atoi(idx.c_str());
    if (k >= int(it->second.size())) fail("result index out of range in " + name);
    return it->second[k];
  }
  void define(const std::string& name, std::vector<int> ids) { scope_[name] = std::move(ids); }

  // -------------------------------------------------------------- types
  TensorType parse_type() {
    TensorType t;
    if (is_bare("tensor")) {
      advance();
      if (!is_punct("<")) fail("expected '<' after tensor");
      std::string raw = lex_.raw_until_close_angle();
      advance();
      auto comma = raw.find(',');  // drop encodings
      if (comma != std::string::npos) raw = raw.substr(0, comma);
      std::vector<std::string> parts;
      std::string curp;
      for (char ch : raw) {
        if (isspace((unsigned char)ch)) continue;
        if (ch == 'x' && !curp.empty() && (isdigit((unsigned char)curp[0]) || curp == "?")) {
          parts.push_back(curp);
          curp.clear();
        } else {
          curp.push_back(ch);
        }
      }
      parts.push_back(curp);
      for (size_t i = 0; i + 1 < parts.size(); ++i) {
        if (parts[i] == "?") fail("dynamic shapes are not supported");
        t.dims.push_back(strtoll(parts[i].c_str(), nullptr, 10));
      }
      t.dtype = ParseElementType(parts.back());
      if (t.dtype == DType::kInvalid) fail("unsupported element type '" + parts.back() + "'");
      return t;
    }
    if (cur_.kind == Tok::kPunct && cur_.text == "!") {
      advance();
      if (cur_.kind == Tok::kBare && cur_.text == "stablehlo.token") {
        advance();
        t.dtype = DType::kToken;
        return t;
      }
      fail("unsupported type !" + cur_.text);
    }
    if (cur_.kind == Tok::kBare) {  // scalar element type, e.g. in attributes
      DType d = ParseElementType(cur_.text);
      if (d != DType::kInvalid) {
        advance();
        t.dtype = d;
        return t;
      }
    }
    fail("expected a type, got '" + cur_.text + "'");
  }

  // `(T, T) -> T`, `(T) -> (T, T)`, `T`, or `T, T`
  void parse_signature(std::vector<TensorType>& ins, std::vector<TensorType>& outs) {
    if (is_punct("(")) {
      advance();
      while (!is_punct(")")) {
        ins.push_back(parse_type());
        if (is_punct(",")) advance();
      }
      advance();
      expect_arrow();
      if (is_punct("(")) {
        advance();
        while (!is_punct(")")) {
          outs.push_back(parse_type());
          skip_attr_dict_opt();
          if (is_punct(",")) advance();
        }
        advance();
      } else {
        outs.push_back(parse_type());
      }
      return;
    }
    outs.push_back(parse_type());
    while (is_punct(",")) {
      advance();
      outs.push_back(parse_type());
    }
  }
  void skip_attr_dict_opt() {
    if (is_punct("{")) parse_attr_dict();
  }

  // -------------------------------------------------------------- attributes
  Attr parse_number_attr() {
    Attr a;
    const std::string s = cur_.text;
    advance();
    if (s.size() > 2 && (s[1] == 'x' || s[1] == 'X')) {
      a.kind = Attr::kInt;
      a.i = int64_t(strtoull(s.c_str(), nullptr, 16));
      a.s = s;
    } else if (s.find_first_of(".eE") != std::string::npos) {
      a.kind = Attr::kFloat;
      a.f = strtod(s.c_str(), nullptr);
    } else {
      a.kind = Attr::kInt;
      a.i = strtoll(s.c_str(), nullptr, 10);
    }
    if (is_punct(":") && next_is_element_type()) {  // `1 : i64` typed literal
      advance();
      parse_type();
    }
    return a;
  }

  Attr parse_attr_value(bool typed_dense = true) {
    Attr a;
    if (cur_.kind == Tok::kNumber) return parse_number_attr();
    if (cur_.kind == Tok::kString) {
      a.kind = Attr::kString;
      a.s = cur_.text;
      advance();
      return a;
    }
    if (cur_.kind == Tok::kSymbol) {
      a.kind = Attr::kSymbol;
      a.s = cur_.text.substr(1);
      advance();
      return a;
    }
    if (is_punct("[")) {
      advance();
      a.kind = Attr::kList;
      while (!is_punct("]")) {
        a.list.push_back(parse_attr_value());
        if (is_punct(",")) advance();
      }
      advance();
      return a;
    }
    if (is_punct("{")) return parse_attr_dict();
    if (cur_.kind == Tok::kHash) {
      // #stablehlo<comparison_direction GT>, #stablehlo.gather<k = v, ...>
      const std::string head = cur_.text;
      advance();
      if (!is_punct("<")) {
        a.kind = Attr::kEnum;
        a.s = head;
        return a;
      }
      advance();
      if (cur_.kind == Tok::kBare && (is_bare("comparison_direction") || is_bare("comparison_type") ||
                                      is_bare("precision") || is_bare("rng_algorithm") ||
                                      is_bare("transpose") || is_bare("fft_type") ||
                                      is_bare("rng_distribution"))) {
        advance();
        a.kind = Attr::kEnum;
        a.s = cur_.text;
        advance();
        expect(">");
        return a;
      }
      a.kind = Attr::kDict;
      a.s = head;
      while (!is_punct(">")) {
        if (cur_.kind != Tok::kBare) fail("expected key in " + head);
        std::string k = cur_.text;
        advance();
        expect("=");
        a.dict[k] = parse_attr_value();
        if (is_punct(",")) advance();
      }
      advance();
      return a;
    }
    if (cur_.kind == Tok::kBare) {
      const std::string w = cur_.text;
      if (w == "true" || w == "false") {
        advance();
        a.kind = Attr::kBool;
        a.i = w == "true";
        return a;
      }
      if (w == "dense") {
        advance();
        if (!is_punct("<")) fail("expected '<' after dense");
        a.kind = Attr::kDense;
        a.s = lex_.raw_until_close_angle();
        advance();
        if (typed_dense && is_punct(":")) {  // attribute carries its own type
          advance();
          a.dense_type = parse_type();
        }
        return a;
      }
      if (w == "array") {
        advance();
        if (!is_punct("<")) fail("expected '<' after array");
        std::string raw = lex_.raw_until_close_angle();
        advance();
        a.kind = Attr::kList;
        auto colon = raw.find(':');
        std::string body = colon == std::string::npos ? "" : raw.substr(colon + 1);
        std::stringstream ss(body);
        std::string item;
        while (std::getline(ss, item, ',')) {
          size_t b = item.find_first_not_of(" \t\n");
          if (b == std::string::npos) continue;
          Attr e;
          e.kind = Attr::kInt;
          std::string v = item.substr(b);
          if (v == "true" || v == "false") e.i = v == "true";
          else e.i = strtoll(v.c_str(), nullptr, 10);
          a.list.push_back(e);
        }
        return a;
      }
      if (w == "tensor") {
        a.kind = Attr::kType;
        a.dense_type = parse_type();
        return a;
      }
      ParseElementType(w);
      advance();
      a.kind = Attr::kEnum;  // bare word: DEFAULT, GT, FLOAT, f32, ...
      a.s = w;
      return a;
    }
    fail("unexpected token in attribute: '" + cur_.text + "'");
  }

  Attr parse_attr_dict() {
    Attr a;
    a.kind = Attr::kDict;
    expect("{");
    while (!is_punct("}")) {
      std::string k;
      if (cur_.kind == Tok::kBare || cur_.kind == Tok::kString) k = cur_.text;
      else fail("expected attribute name, got '" + cur_.text + "'");
      advance();
      if (is_punct("=")) {
        advance();
        a.dict[k] = parse_attr_value();
      } else {
        Attr unit;
        unit.kind = Attr::kBool;
        unit.i = 1;
        a.dict[k] = unit;
      }
      if (is_punct(",")) advance();
    }
    advance();
    return a;
  }

  // -------------------------------------------------------------- functions
  void parse_func() {
    advance();  // func.func
    Func f;
    if (is_bare("public") || is_bare("private") || is_bare("nested")) {
      f.is_public = cur_.text == "public";
      advance();
    }
    if (cur_.kind != Tok::kSymbol) fail("expected function name");
    f.name = cur_.text.substr(1);
    if (!f.name.empty() && f.name[0] == '"') f.name = f.name.substr(1, f.name.size() - 2);
    advance();
    scope_.clear();
    expect("(");
    while (!is_punct(")")) {
      if (cur_.kind != Tok::kValue) fail("expected argument name");
      std::string name = cur_.text;
      advance();
      expect(":");
      TensorType t = parse_type();
      int alias = -1;
      bool donor = false;
      if (is_punct("{")) {
        const Attr ad = parse_attr_dict();
        if (const Attr* al = ad.get("tf.aliasing_output")) {
          if (al->kind != Attr::kInt) fail("tf.aliasing_output must be an integer");
          alias = int(al->i);
        }
        if (const Attr* d = ad.get("jax.buffer_donor")) donor = d->kind == Attr::kBool ? d->i != 0 : true;
      }
      skip_loc();
      int id = m_.new_value(t, name);
      define(name, {id});
      f.args.push_back(id);
      f.arg_alias.push_back(alias);
      f.arg_donor.push_back(donor);
      if (is_punct(",")) advance();
    }
    advance();
    if (cur_.kind == Tok::kArrow) {
      advance();
      if (is_punct("(")) {
        advance();
        while (!is_punct(")")) {
          f.result_types.push_back(parse_type());
          skip_attr_dict_opt();
          skip_loc();
          if (is_punct(",")) advance();
        }
        advance();
      } else {
        f.result_types.push_back(parse_type());
      }
    }
    if (is_bare("attributes")) {
      advance();
      parse_attr_dict();
    }
    expect("{");
    parse_block_body(f.body);
    expect("}");
    skip_loc();
    m_.funcs.push_back(std::move(f));
  }

  // ops until the closing '}' of the block (not consumed)
  void parse_block_body(Block& blk) {
    while (!is_punct("}")) {
      if (cur_.kind == Tok::kEnd) fail("unexpected end of input inside a block");
      if (cur_.kind == Tok::kCaret) {  // block label inside a region: ^bb0(%a: T, ...):
        advance();
        if (is_punct("(")) {
          advance();
          while (!is_punct(")")) {
            std::string name = cur_.text;
            advance();
            expect(":");
            TensorType t = parse_type();
            skip_loc();
            int id = m_.new_value(t, name);
            define(name, {id});
            blk.args.push_back(id);
            if (is_punct(",")) advance();
          }
          advance();
        }
        expect(":");
        continue;
      }
      blk.ops.push_back(parse_op());
    }
  }

  // -------------------------------------------------------------- ops
  Op parse_op() {
    Op op;
    op.line = cur_.line;
    std::vector<std::pair<std::string, int>> defs;  // (name, count)
    if (cur_.kind == Tok::kValue) {
      for (;;) {
        std::string name = cur_.text;
        advance();
        int count = 1;
        if (is_punct(":")) {
          advance();
          count = int(strtol(cur_.text.c_str(), nullptr, 10));
          advance();
        }
        defs.push_back({name, count});
        if (is_punct(",")) {
          advance();
          continue;
        }
        break;
      }
      expect("=");
    }
    std::vector<TensorType> in_types, out_types;
    if (cur_.kind == Tok::kString) {
      parse_generic(op, in_types, out_types);
    } else if (cur_.kind == Tok::kBare) {
      parse_pretty(op, in_types, out_types);
    } else {
      fail("expected an operation, got '" + cur_.text + "'");
    }
    skip_loc();
    // results
    int total = 0;
    for (auto& d : defs) total += d.second;
    if (total != int(out_types.size()))
      fail("op " + op.name + " defines " + std::to_string(total) + " values but its type lists " +
           std::to_string(out_types.size()) + " results");
    size_t k = 0;
    for (auto& d : defs) {
      std::vector<int> ids;
      for (int j = 0; j < d.second; ++j) {
        int id = m_.new_value(out_types[k++], d.first);
        ids.push_back(id);
        op.results.push_back(id);
      }
      define(d.first, ids);
    }
    return op;
  }

  void parse_operand_list_until(const char* close, std::vector<int>& out) {
    while (!is_punct(close)) {
      if (cur_.kind != Tok::kValue) fail("expected operand, got '" + cur_.text + "'");
      out.push_back(lookup(cur_.text));
      advance();
      if (is_punct(",")) advance();
    }
    advance();
  }

  void parse_regions(Op& op) {
    // ({ ...block... }, { ... })
    expect("(");
    while (!is_punct(")")) {
      auto r = std::make_shared<Region>();
      expect("{");
      auto saved = scope_;
      r->blocks.emplace_back();
      parse_block_body(r->blocks.back());
      expect("}");
      scope_ = saved;
      op.regions.push_back(r);
      if (is_punct(",")) advance();
    }
    advance();
  }

  void parse_generic(Op& op, std::vector<TensorType>& ins, std::vector<TensorType>& outs) {
    op.name = cur_.text;
    advance();
    expect("(");
    parse_operand_list_until(")", op.operands);
    if (is_punct("<")) {  // properties <{...}>
      advance();
      Attr props = parse_attr_dict();
      for (auto& kv : props.dict) op.attrs[kv.first] = kv.second;
      expect(">");
    }
    if (is_punct("(")) parse_regions(op);
    if (is_punct("{")) {
      Attr d = parse_attr_dict();
      for (auto& kv : d.dict) op.attrs[kv.first] = kv.second;
    }
    expect(":");
    parse_signature(ins, outs);
  }

  void parse_pretty(Op& op, std::vector<TensorType>& ins, std::vector<TensorType>& outs) {
    std::string name = cur_.text;
    advance();
    if (name == "return" || name == "func.return" || name == "stablehlo.return") {
      op.name = "return";
      while (cur_.kind == Tok::kValue) {
        op.operands.push_back(lookup(cur_.text));
        advance();
        if (is_punct(",")) advance();
      }
      if (is_punct(":")) {
        advance();
        std::vector<TensorType> tys;
        tys.push_back(parse_type());
        while (is_punct(",")) {
          advance();
          tys.push_back(parse_type());
        }
      }
      return;
    }
    if (name == "call" || name == "func.call") {
      op.name = "func.call";
      Attr callee;
      callee.kind = Attr::kSymbol;
      callee.s = cur_.text.substr(1);
      op.attrs["callee"] = callee;
      advance();
      expect("(");
      parse_operand_list_until(")", op.operands);
      if (is_punct("{")) parse_attr_dict();
      expect(":");
      parse_signature(ins, outs);
      return;
    }
    // dialect-less names ("add") map to stablehlo
    op.name = name.find('.') == std::string::npos ? "stablehlo." + name : name;
    if (op.name == "stablehlo.reduce") {
      parse_reduce(op, ins, outs);
      return;
    }
    if (op.name == "stablehlo.constant") {
      if (is_punct("{")) {
        Attr d = parse_attr_dict();
        for (auto& kv : d.dict) op.attrs[kv.first] = kv.second;
      }
      op.attrs["value"] = parse_attr_value(/*typed_dense=*/false);
      expect(":");
      parse_signature(ins, outs);
      return;
    }
    if (op.name == "stablehlo.custom_call") {
      Attr target;
      target.kind = Attr::kSymbol;
      target.s = cur_.text.substr(1);
      op.attrs["call_target_name"] = target;
      advance();
      expect("(");
      parse_operand_list_until(")", op.operands);
      if (is_punct("{")) {
        Attr d = parse_attr_dict();
        for (auto& kv : d.dict) op.attrs[kv.first] = kv.second;
      }
      expect(":");
      parse_signature(ins, outs);
      return;
    }
    // generic pretty form: operands, `key = value`, enum words, slice specs
    int enum_index = 0;
    while (!is_punct(":")) {
      if (cur_.kind == Tok::kEnd || is_punct("}")) fail("unterminated operation " + op.name);
      if (cur_.kind == Tok::kValue) {
        op.operands.push_back(lookup(cur_.text));
        advance();
      } else if (is_punct(",")) {
        advance();
      } else if (cur_.kind == Tok::kBare) {
        std::string w = cur_.text;
        advance();
        if (is_punct("=")) {
          advance();
          Attr v = parse_attr_value();
          if (cur_.kind == Tok::kBare && cur_.text == "x") {  // `[0] x [1]` pairs
            advance();
            Attr pair;
            pair.kind = Attr::kList;
            pair.list.push_back(v);
            pair.list.push_back(parse_attr_value());
            v = pair;
          }
          op.attrs[w] = v;
        } else {
          Attr e;
          e.kind = Attr::kEnum;
          e.s = w;
          op.attrs[enum_index++ == 0 ? "enum0" : "enum1"] = e;
        }
      } else if (is_punct("[")) {  // slice spec [a:b(:c), ...]
        advance();
        Attr starts, limits, strides;
        starts.kind = limits.kind = strides.kind = Attr::kList;
        while (!is_punct("]")) {
          Attr s0 = parse_number_attr_plain();
          expect(":");
          Attr l0 = parse_number_attr_plain();
          Attr st;
          st.kind = Attr::kInt;
          st.i = 1;
          if (is_punct(":")) {
            advance();
            st = parse_number_attr_plain();
          }
          starts.list.push_back(s0);
          limits.list.push_back(l0);
          strides.list.push_back(st);
          if (is_punct(",")) advance();
        }
        advance();
        op.attrs["start_indices"] = starts;
        op.attrs["limit_indices"] = limits;
        op.attrs["strides"] = strides;
      } else if (is_punct("{")) {
        Attr d = parse_attr_dict();
        for (auto& kv : d.dict) op.attrs[kv.first] = kv.second;
      } else if (is_punct("(")) {
        parse_regions(op);
      } else {
        fail("unexpected '" + cur_.text + "' in " + op.name);
      }
    }
    advance();  // ':'
    parse_signature(ins, outs);
    if (op.name == "stablehlo.select" && outs.size() == 2) {  // `: tensor<i1>, tensor<f32>`
      outs.erase(outs.begin());
    }
    if (op.name == "stablehlo.optimization_barrier" || op.name == "stablehlo.select" ||
        op.name == "stablehlo.clamp") {
      // `: T` forms list operand types == result types
      if (op.name != "stablehlo.optimization_barrier" && outs.size() > 1) outs.erase(outs.begin(), outs.end() - 1);
    }
    if (is_punct("(") && op.regions.empty()) parse_regions(op);
  }

  Attr parse_number_attr_plain() {
    if (cur_.kind != Tok::kNumber) fail("expected a number");
    Attr a;
    a.kind = Attr::kInt;
    a.i = strtoll(cur_.text.c_str(), nullptr, 10);
    advance();
    return a;
  }

  // stablehlo.reduce(%a init: %b), (%c init: %d) applies OP across dimensions = [..] : sig
  // stablehlo.reduce(%a init: %b) across dimensions = [..] : sig  reducer(...) (...) { body }
  void parse_reduce(Op& op, std::vector<TensorType>& ins, std::vector<TensorType>& outs) {
    std::vector<int> inputs, inits;
    for (;;) {
      expect("(");
      inputs.push_back(lookup(cur_.text));
      advance();
      if (!is_bare("init")) fail("expected 'init:' in reduce");
      advance();
      expect(":");
      inits.push_back(lookup(cur_.text));
      advance();
      expect(")");
      if (is_punct(",")) {
        advance();
        continue;
      }
      break;
    }
    op.operands = inputs;
    op.operands.insert(op.operands.end(), inits.begin(), inits.end());
    std::string applies;
    if (is_bare("applies")) {
      advance();
      applies = cur_.text;
      advance();
    }
    if (!is_bare("across")) fail("expected 'across' in reduce");
    advance();
    if (!is_bare("dimensions")) fail("expected 'dimensions' in reduce");
    advance();
    expect("=");
    op.attrs["dimensions"] = parse_attr_value();
    expect(":");
    parse_signature(ins, outs);
    const size_t n = inputs.size();
    auto region = std::make_shared<Region>();
    region->blocks.emplace_back();
    Block& body = region->blocks.back();
    if (!applies.empty()) {
      // synthesize the body: return applies(acc_i, x_i)
      for (size_t i = 0; i < 2 * n; ++i) {
        TensorType t;
        t.dtype = m_.types[inits[i % n]].dtype;
        body.args.push_back(m_.new_value(t, "%reduce_arg"));
      }
      Op ret;
      ret.name = "return";
      for (size_t i = 0; i < n; ++i) {
        Op b;
        b.name = applies;
        b.operands = {body.args[i], body.args[n + i]};
        TensorType t;
        t.dtype = m_.types[inits[i]].dtype;
        int r = m_.new_value(t, "%reduce_body");
        b.results = {r};
        body.ops.push_back(b);
        ret.operands.push_back(r);
      }
      body.ops.push_back(ret);
    } else {
      if (!is_bare("reducer")) fail("expected 'reducer' block in reduce");
      advance();
      auto saved = scope_;
      std::vector<int> lhs, rhs;
      for (size_t i = 0; i < n; ++i) {
        expect("(");
        for (int side = 0; side < 2; ++side) {
          std::string nm = cur_.text;
          advance();
          expect(":");
          TensorType t = parse_type();
          skip_loc();
          int id = m_.new_value(t, nm);
          define(nm, {id});
          (side == 0 ? lhs : rhs).push_back(id);
          if (is_punct(",")) advance();
        }
        expect(")");
      }
      body.args = lhs;
      body.args.insert(body.args.end(), rhs.begin(), rhs.end());
      expect("{");
      parse_block_body(body);
      expect("}");
      scope_ = saved;
    }
    op.regions.push_back(region);
  }

  Lexer lex_;
  Token cur_;
  Module& m_;
  std::unordered_map<std::string, std::vector<int>> scope_;
};

}  // namespace

std::unique_ptr<Module> ParseText(const char* text, size_t size, std::string& error) {
  auto m = std::make_unique<Module>();
  Parser p(text, size, *m);
  if (!p.parse_module(error)) return nullptr;
  return m;
}

}  // namespace mi::jam
