// Test-only writer of StableHLO portable artifacts, and the check that the
// plugin's compiler reads them back to the same launch plan as the text.
//
// jaxlib serializes a jitted module as a StableHLO portable artifact: MLIR
// bytecode (version 1, producer "StableHLO_v1.0.0") holding VHLO operations
// (the reference reads it with deserializePortableArtifact,
// src/jam/parse.cc:53-63).  Neither MLIR nor jaxlib exists in this
// environment, so this program writes such artifacts itself from a module's
// StableHLO text, by the rules MLIR's bytecode writer follows:
//   - header: magic "ML\xEFR", version varint, producer string;
//   - sections: dialects (vhlo carrying its version 1.0.0 as three varints in
//     a nested section), attributes and types (deduplicated payloads in runs
//     of one dialect, offsets as sizes with the "custom encoding" flag), the
//     IR, and the string table (lengths in reverse order);
//   - IR: one builtin.module whose isolated region holds vhlo.func_v1 ops
//     (isolated), with each region's value count and values numbered block
//     arguments first, then op results; the regions of other ops are not
//     isolated, so their values are numbered after their parent region's;
//   - each op's attributes in a builtin DictionaryAttr (names as builtin
//     StringAttr, sorted), every location the builtin UnknownLoc;
//   - VHLO types by their type codes, VHLO attributes as (code, fields):
//     integer lists as tensor_v1 of i64, integers as integer_v1 (type, APInt),
//     enums and booleans as varints, strings as string-table indices, dense
//     constants as tensor_v1 with the elements' little-endian bytes (one
//     element for a splat; i1 bit-packed, a splat as 0x00 / 0xFF).
// The attribute codes used for VHLO attributes are this writer's; the
// reader decodes attributes by their names and does not depend on them.
//
//   vhlo_writer write <module.mlir> <out.mlirbc>
//   vhlo_writer check <module.mlir>   compiles the text and the artifact
//                                     written from it and compares the two
//                                     launch plans field by field
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iostream>
#include <map>
#include <sstream>
#include <string>
#include <vector>

#include "jam/ir.h"
#include "jam/program.h"

using namespace mi::jam;

namespace {

[[noreturn]] void Die(const std::string& m) {
  std::cerr << "vhlo_writer: " << m << "\n";
  exit(2);
}

// ------------------------------------------------------------------ encoding primitives
void VarInt(std::string& o, uint64_t v) {
  for (int n = 1; n <= 8; ++n) {
    if (n == 8 ? v < (uint64_t(1) << 56) : v < (uint64_t(1) << (7 * n))) {
      const uint64_t x = ((v << 1) | 1) << (n - 1);
      for (int i = 0; i < n; ++i) o.push_back(char((x >> (8 * i)) & 0xFF));
      return;
    }
  }
  o.push_back(0);
  for (int i = 0; i < 8; ++i) o.push_back(char((v >> (8 * i)) & 0xFF));
}
void VarIntFlag(std::string& o, uint64_t v, bool f) { VarInt(o, (v << 1) | (f ? 1 : 0)); }
void SignedVarInt(std::string& o, int64_t v) { VarInt(o, (uint64_t(v) << 1) ^ uint64_t(v >> 63)); }
void Section(std::string& o, int id, const std::string& data) {
  o.push_back(char(id));
  VarInt(o, data.size());
  o += data;
}

// nearest-even rounding of a double to a binary float with `eb` exponent and
// `mb` stored mantissa bits, done on the integer significand
uint64_t RoundToBits(double v, int eb, int mb) {
  uint64_t d;
  memcpy(&d, &v, 8);
  const uint64_t sign = (d >> 63) << (eb + mb);
  const int bias = (1 << (eb - 1)) - 1;
  const uint64_t exp_all = (uint64_t(1) << eb) - 1;
  if (std::isnan(v)) return sign | (exp_all << mb) | (uint64_t(1) << (mb - 1));
  if (std::isinf(v)) return sign | (exp_all << mb);
  if (v == 0) return sign;
  int e = int((d >> 52) & 0x7FF) - 1023;
  uint64_t m = d & ((uint64_t(1) << 52) - 1);
  if (e == -1023) {  // double subnormal: far below any target here
    return sign;
  }
  m |= uint64_t(1) << 52;
  const int emin = 1 - bias;
  int shift = 52 - mb + (e < emin ? emin - e : 0);
  if (shift >= 64) return sign;
  uint64_t q = m >> shift;
  const uint64_t rem = m & ((uint64_t(1) << shift) - 1), half = uint64_t(1) << (shift - 1);
  if (rem > half || (rem == half && (q & 1))) ++q;
  if (e < emin) return sign | q;  // subnormal (q may carry into the smallest normal)
  if (q >> (mb + 1)) {
    q >>= 1;
    ++e;
  }
  if (e > bias) return sign | (exp_all << mb);
  return sign | (uint64_t(e + bias) << mb) | (q & ((uint64_t(1) << mb) - 1));
}


// ------------------------------------------------------------------ attribute / type tables
// Entries are numbered in creation order (an attribute's payload can only
// refer to entries made before it) and deduplicated by (dialect, payload);
// the offset section lists them as runs of one dialect.
struct Entry {
  int dialect;  // 0 builtin, 1 vhlo
  std::string payload;
};

class Tables {
 public:
  std::vector<std::string> strings;
  std::vector<Entry> attrs, types;

  int Str(const std::string& s) {
    auto it = string_ix_.find(s);
    if (it != string_ix_.end()) return it->second;
    strings.push_back(s);
    return string_ix_[s] = int(strings.size()) - 1;
  }
  int Attr(int dialect, const std::string& payload) { return Add(attrs, attr_ix_, dialect, payload); }
  int Type(const std::string& payload) { return Add(types, type_ix_, 1, payload); }

 private:
  static int Add(std::vector<Entry>& v, std::map<std::pair<int, std::string>, int>& ix, int d, const std::string& p) {
    auto key = std::make_pair(d, p);
    auto it = ix.find(key);
    if (it != ix.end()) return it->second;
    v.push_back({d, p});
    return ix[key] = int(v.size()) - 1;
  }
  std::map<std::string, int> string_ix_;
  std::map<std::pair<int, std::string>, int> attr_ix_, type_ix_;
};

// VHLO type codes (the reader's table)
enum : uint64_t {
  kTyBool = 0, kTyBF16 = 2, kTyF16 = 3, kTyF32 = 4, kTyF64 = 5, kTyFunction = 8,
  kTySI16 = 10, kTySI32 = 11, kTySI64 = 13, kTySI8 = 14, kTyUI16 = 15, kTyUI32 = 16, kTyUI64 = 18,
  kTyUI8 = 19, kTyTensor = 20, kTyToken = 22,
};
// this writer's VHLO attribute codes
enum : uint64_t {
  kAtArray = 0, kAtBool = 1, kAtCmpDir = 2, kAtCmpType = 3, kAtDict = 5, kAtInteger = 8, kAtPrecision = 10,
  kAtString = 13, kAtTensor = 14, kAtType = 17,
};
// builtin attribute codes
enum : uint64_t { kBiDictionary = 1, kBiString = 2, kBiUnknownLoc = 15 };

std::string V(uint64_t v) {
  std::string s;
  VarInt(s, v);
  return s;
}

class Writer {
 public:
  explicit Writer(const Module& m) : m_(m) {}

  std::string Write() {
    unknown_loc_ = t_.Attr(0, V(kBiUnknownLoc));
    // op names are numbered in the dialect section's grouped order: making
    // the one builtin name first keeps that order the order of creation
    const int module_name = OpName(0, "module");
    std::map<std::string, int> mattrs;
    mattrs["sym_name"] = t_.Attr(0, V(kBiString) + V(uint64_t(t_.Str(m_.name.empty() ? "jit_module" : m_.name))));
    std::string module_block;
    VarIntFlag(module_block, m_.funcs.size(), false);
    for (const Func& f : m_.funcs) module_block += FuncOp(f);
    std::string ir;
    VarIntFlag(ir, 1, false);  // top block: one op, no arguments
    ir += OpHeader(module_name, Dict(mattrs), {}, {}, true);
    VarIntFlag(ir, 1, true);  // one region, isolated
    VarInt(ir, 1);            // one block
    VarInt(ir, 0);            // no values
    ir += module_block;
    return Assemble(ir);
  }

 private:
  int OpName(int dialect, const std::string& name) {
    auto key = std::make_pair(dialect, name);
    auto it = op_ix_.find(key);
    if (it != op_ix_.end()) return it->second;
    op_names_.push_back(key);
    t_.Str(name);
    return op_ix_[key] = int(op_names_.size()) - 1;
  }

  // ---- types
  int Elem(DType d) {
    uint64_t c;
    switch (d) {
      case DType::kPred: c = kTyBool; break;
      case DType::kBF16: c = kTyBF16; break;
      case DType::kF16: c = kTyF16; break;
      case DType::kF32: c = kTyF32; break;
      case DType::kF64: c = kTyF64; break;
      case DType::kI8: c = kTySI8; break;
      case DType::kI16: c = kTySI16; break;
      case DType::kI32: c = kTySI32; break;
      case DType::kI64: c = kTySI64; break;
      case DType::kU8: c = kTyUI8; break;
      case DType::kU16: c = kTyUI16; break;
      case DType::kU32: c = kTyUI32; break;
      case DType::kU64: c = kTyUI64; break;
      case DType::kToken: c = kTyToken; break;
      default: Die(std::string("no VHLO type for ") + DTypeName(d));
    }
    return t_.Type(V(c));
  }
  int Tensor(const TensorType& t) {
    if (t.dtype == DType::kToken) return Elem(DType::kToken);
    const int e = Elem(t.dtype);
    std::string p = V(kTyTensor);
    VarInt(p, t.dims.size());
    for (int64_t d : t.dims) SignedVarInt(p, d);
    VarInt(p, uint64_t(e));
    return t_.Type(p);
  }
  int FuncType(const std::vector<TensorType>& ins, const std::vector<TensorType>& outs) {
    std::string p = V(kTyFunction);
    VarInt(p, ins.size());
    for (const auto& t : ins) VarInt(p, uint64_t(Tensor(t)));
    VarInt(p, outs.size());
    for (const auto& t : outs) VarInt(p, uint64_t(Tensor(t)));
    return t_.Type(p);
  }

  // ---- VHLO attributes
  int VString(const std::string& s) { return t_.Attr(1, V(kAtString) + V(uint64_t(t_.Str(s)))); }
  int VInt(int64_t v, DType d = DType::kI64) {
    std::string p = V(kAtInteger) + V(uint64_t(Elem(d)));
    const int w = 8 * DTypeBytes(d);
    uint64_t bits = uint64_t(v);
    if (w < 64) bits &= (uint64_t(1) << w) - 1;  // APInt::getLimitedValue is zero-extended
    if (w <= 8) p.push_back(char(bits));
    else SignedVarInt(p, int64_t(bits));
    return t_.Attr(1, p);
  }
  int VBool(bool b) { return t_.Attr(1, V(kAtBool) + V(b ? 1 : 0)); }
  int VEnum(uint64_t code, uint64_t v) { return t_.Attr(1, V(code) + V(v)); }
  int VType(int type) { return t_.Attr(1, V(kAtType) + V(uint64_t(type))); }
  int VArray(const std::vector<int>& elems) {
    std::string p = V(kAtArray) + V(elems.size());
    for (int e : elems) VarInt(p, uint64_t(e));
    return t_.Attr(1, p);
  }
  int VDict(const std::map<std::string, int>& d) {
    std::string p = V(kAtDict) + V(d.size());
    for (const auto& [k, v] : d) {
      VarInt(p, uint64_t(VString(k)));
      VarInt(p, uint64_t(v));
    }
    return t_.Attr(1, p);
  }
  int VTensorRaw(const TensorType& t, const std::string& raw) {
    std::string p = V(kAtTensor) + V(uint64_t(Tensor(t))) + V(raw.size()) + raw;
    return t_.Attr(1, p);
  }
  int VInts(const std::vector<int64_t>& v) {
    TensorType t;
    t.dtype = DType::kI64;
    t.dims = {int64_t(v.size())};
    bool same = v.size() > 1;
    for (int64_t x : v) same = same && x == v[0];
    std::string raw;
    for (size_t k = 0; k < (same ? 1 : v.size()); ++k)
      for (int i = 0; i < 8; ++i) raw.push_back(char((uint64_t(v[k]) >> (8 * i)) & 0xFF));
    return VTensorRaw(t, raw);
  }
  int Dict(const std::map<std::string, int>& d) {  // builtin DictionaryAttr
    std::string p = V(kBiDictionary) + V(d.size());
    for (const auto& [k, v] : d) {
      VarInt(p, uint64_t(t_.Attr(0, V(kBiString) + V(uint64_t(t_.Str(k))))));
      VarInt(p, uint64_t(v));
    }
    return t_.Attr(0, p);
  }

  static std::string PackBools(const std::string& bytes, bool splat) {
    if (splat) return std::string(1, bytes[0] ? '\xFF' : '\0');
    std::string out((bytes.size() + 7) / 8, '\0');
    for (size_t k = 0; k < bytes.size(); ++k)
      if (bytes[k]) out[k / 8] = char(out[k / 8] | (1 << (k % 8)));
    return out;
  }

  // dense<...> text of a constant -> elements' raw bytes (a splat keeps one)
  int VDense(const Attr& a, const TensorType& t) {
    std::string s = a.s;
    const size_t b = s.find_first_not_of(" \n\t"), e = s.find_last_not_of(" \n\t");
    s = b == std::string::npos ? "" : s.substr(b, e - b + 1);
    const size_t w = size_t(DTypeBytes(t.dtype));
    const size_t n = size_t(t.numel());
    std::string elems;  // one byte per i1 element here
    size_t cnt = 0;
    if (s.size() >= 3 && s[0] == '"' && s[1] == '0' && (s[2] == 'x' || s[2] == 'X')) {
      const std::string hex = s.substr(3, s.size() - 4);
      for (size_t i = 0; i + 1 < hex.size(); i += 2) elems.push_back(char(strtoul(hex.substr(i, 2).c_str(), nullptr, 16)));
      cnt = elems.size() / w;
    } else {
      std::vector<std::string> toks;
      std::string tok;
      for (char c : s) {
        if (c == '[' || c == ']' || c == ',' || c == ' ' || c == '\n' || c == '(' || c == ')') {
          if (!tok.empty()) toks.push_back(tok);
          tok.clear();
        } else {
          tok.push_back(c);
        }
      }
      if (!tok.empty()) toks.push_back(tok);
      for (const std::string& x : toks) {
        uint64_t bits = 0;
        if (t.dtype == DType::kPred) {
          bits = x == "true" || x == "1";
        } else if (x.size() > 2 && x[0] == '0' && (x[1] == 'x' || x[1] == 'X')) {
          bits = strtoull(x.c_str(), nullptr, 16);
        } else if (IsFloat(t.dtype)) {
          const double v = x == "inf" || x == "+inf" ? INFINITY
                           : x == "-inf"              ? -INFINITY
                           : x == "nan"               ? NAN
                                                      : strtod(x.c_str(), nullptr);
          if (t.dtype == DType::kBF16) bits = RoundToBits(v, 8, 7);
          else if (t.dtype == DType::kF16) bits = RoundToBits(v, 5, 10);
          else if (t.dtype == DType::kF32) bits = RoundToBits(v, 8, 23);
          else memcpy(&bits, &v, 8);
        } else {
          bits = uint64_t(strtoll(x.c_str(), nullptr, 10));
        }
        for (size_t i = 0; i < w; ++i) elems.push_back(char((bits >> (8 * i)) & 0xFF));
      }
      cnt = toks.size();
    }
    bool same = cnt > 1;
    for (size_t k = 1; same && k < cnt; ++k) same = elems.compare(k * w, w, elems, 0, w) == 0;
    if (cnt != n && !(cnt == 1 && n != 1)) Die("dense constant with " + std::to_string(cnt) + " values for " + t.str());
    const bool splat = n != 1 && (cnt == 1 || same);
    if (t.dtype == DType::kPred) return VTensorRaw(t, n == 1 ? elems.substr(0, 1) : PackBools(elems, splat));
    return VTensorRaw(t, splat ? elems.substr(0, w) : elems);
  }

  static uint64_t Index(const std::vector<std::string>& names, const std::string& s) {
    for (size_t i = 0; i < names.size(); ++i)
      if (names[i] == s) return i;
    Die("unknown enum word " + s);
  }

  // ---- attributes of a StableHLO op (text reader form) in VHLO form
  std::map<std::string, int> OpAttrs(const Op& op, const std::string& base) {
    std::map<std::string, int> out;
    std::map<std::string, bool> used;
    for (const auto& kv : op.attrs) used[kv.first] = false;
    auto take = [&](std::initializer_list<const char*> names) -> const Attr* {
      const Attr* r = nullptr;
      for (const char* n : names) {
        if (const Attr* a = op.attr(n)) {
          used[n] = true;
          if (!r) r = a;
        }
      }
      return r;
    };
    auto ints = [&](std::initializer_list<const char*> names, const char* vname) {
      if (const Attr* a = take(names)) out[vname] = VInts(a->ints());
    };
    auto one = [&](std::initializer_list<const char*> names, const char* vname) {
      if (const Attr* a = take(names)) {
        const auto v = a->ints();
        if (v.size() != 1) Die(std::string("attribute ") + vname + " is not one integer");
        out[vname] = VInt(v[0]);
      }
    };
    auto dims = [&](const Attr* dn, const char* k) {
      const Attr* a = dn ? dn->get(k) : nullptr;
      return a ? a->ints() : std::vector<int64_t>{};
    };
    if (base == "broadcast_in_dim") {
      ints({"dims", "broadcast_dimensions"}, "broadcast_dimensions");
    } else if (base == "transpose") {
      ints({"dims", "permutation"}, "permutation");
    } else if (base == "reduce" || base == "reverse") {
      ints({"dimensions"}, "dimensions");
    } else if (base == "iota") {
      one({"dim", "iota_dimension"}, "iota_dimension");
    } else if (base == "concatenate") {
      one({"dim", "dimension"}, "dimension");
    } else if (base == "slice") {
      ints({"start_indices"}, "start_indices");
      ints({"limit_indices"}, "limit_indices");
      ints({"strides"}, "strides");
    } else if (base == "compare") {
      static const std::vector<std::string> dirs = {"EQ", "NE", "GE", "GT", "LE", "LT"};
      static const std::vector<std::string> cts = {"NOTYPE", "FLOAT", "TOTALORDER", "SIGNED", "UNSIGNED"};
      const Attr* d = take({"comparison_direction", "enum0"});
      const Attr* c = take({"compare_type", "enum1"});
      if (!d) Die("compare without a direction");
      out["comparison_direction"] = VEnum(kAtCmpDir, Index(dirs, d->s));
      out["compare_type"] = VEnum(kAtCmpType, c ? Index(cts, c->s) : 0);
    } else if (base == "constant") {
      const Attr* v = take({"value"});
      if (!v || v->kind != Attr::kDense) Die("constant without a dense value");
      out["value"] = VDense(*v, m_.types[op.results.at(0)]);
    } else if (base == "dot_general") {
      std::vector<int64_t> lb, rb, lc, rc;
      if (const Attr* dn = take({"dot_dimension_numbers"})) {
        lb = dims(dn, "lhs_batching_dimensions");
        rb = dims(dn, "rhs_batching_dimensions");
        lc = dims(dn, "lhs_contracting_dimensions");
        rc = dims(dn, "rhs_contracting_dimensions");
      }
      if (const Attr* b = take({"batching_dims"})) {
        lb = b->list.at(0).ints();
        rb = b->list.at(1).ints();
      }
      if (const Attr* c = take({"contracting_dims"})) {
        lc = c->list.at(0).ints();
        rc = c->list.at(1).ints();
      }
      out["lhs_batching_dimensions"] = VInts(lb);
      out["rhs_batching_dimensions"] = VInts(rb);
      out["lhs_contracting_dimensions"] = VInts(lc);
      out["rhs_contracting_dimensions"] = VInts(rc);
      static const std::vector<std::string> names = {"DEFAULT", "HIGH", "HIGHEST"};
      std::vector<int> prec;
      if (const Attr* p = take({"precision_config", "precision"}))
        for (const Attr& e : p->list) prec.push_back(VEnum(kAtPrecision, Index(names, e.s)));
      out["precision_config"] = VArray(prec);
    } else if (base == "gather") {
      const Attr* dn = take({"dimension_numbers"});
      if (!dn) Die("gather without dimension_numbers");
      out["offset_dims"] = VInts(dims(dn, "offset_dims"));
      out["collapsed_slice_dims"] = VInts(dims(dn, "collapsed_slice_dims"));
      out["start_index_map"] = VInts(dims(dn, "start_index_map"));
      out["index_vector_dim"] = VInt(dims(dn, "index_vector_dim").at(0));
      ints({"slice_sizes"}, "slice_sizes");
      const Attr* s = take({"indices_are_sorted"});
      out["indices_are_sorted"] = VBool(s && s->i);
    } else if (base == "scatter") {
      const Attr* dn = take({"scatter_dimension_numbers"});
      if (!dn) Die("scatter without scatter_dimension_numbers");
      out["update_window_dims"] = VInts(dims(dn, "update_window_dims"));
      out["inserted_window_dims"] = VInts(dims(dn, "inserted_window_dims"));
      out["scatter_dims_to_operand_dims"] = VInts(dims(dn, "scatter_dims_to_operand_dims"));
      out["index_vector_dim"] = VInt(dims(dn, "index_vector_dim").at(0));
      const Attr* s = take({"indices_are_sorted"});
      const Attr* u = take({"unique_indices"});
      out["indices_are_sorted"] = VBool(s && s->i);
      out["unique_indices"] = VBool(u && u->i);
    }
    for (const auto& [k, u] : used)
      if (!u) Die("op stablehlo." + base + ": attribute '" + k + "' has no VHLO form in this writer");
    return out;
  }

  // ---- IR
  std::string OpHeader(int name, int attr_dict, const std::vector<int>& result_types,
                       const std::vector<uint64_t>& operands, bool has_regions) {
    std::string o = V(uint64_t(name));
    uint8_t mask = 0;
    std::string body = V(uint64_t(unknown_loc_));
    if (attr_dict >= 0) {
      mask |= 0x01;
      VarInt(body, uint64_t(attr_dict));
    }
    if (!result_types.empty()) {
      mask |= 0x02;
      VarInt(body, result_types.size());
      for (int t : result_types) VarInt(body, uint64_t(t));
    }
    if (!operands.empty()) {
      mask |= 0x04;
      VarInt(body, operands.size());
      for (uint64_t v : operands) VarInt(body, v);
    }
    if (has_regions) mask |= 0x10;
    o.push_back(char(mask));
    return o + body;
  }

  // value numbers of the region being written (jam value -> number)
  using Numbering = std::map<int, uint64_t>;

  std::string FuncOp(const Func& f) {
    std::map<std::string, int> a;
    a["sym_name"] = VString(f.name);
    a["sym_visibility"] = VString(f.is_public ? "" : "private");
    std::vector<TensorType> ins;
    for (int v : f.args) ins.push_back(m_.types[v]);
    a["function_type"] = VType(FuncType(ins, f.result_types));
    std::vector<int> arg_attrs, res_attrs;
    for (size_t k = 0; k < f.args.size(); ++k) {
      std::map<std::string, int> d;
      if (k < f.arg_alias.size() && f.arg_alias[k] >= 0) d["tf.aliasing_output"] = VInt(f.arg_alias[k], DType::kI32);
      if (k < f.arg_donor.size() && f.arg_donor[k]) d["jax.buffer_donor"] = VBool(true);
      arg_attrs.push_back(VDict(d));
    }
    for (size_t k = 0; k < f.result_types.size(); ++k) res_attrs.push_back(VDict({}));
    a["arg_attrs"] = VArray(arg_attrs);
    a["res_attrs"] = VArray(res_attrs);
    std::string o = OpHeader(OpName(1, "func_v1"), Dict(a), {}, {}, true);
    VarIntFlag(o, 1, true);  // one region, isolated: numbering restarts at 0
    Numbering num;
    o += RegionText(f.body, f.args, num, 0);
    return o;
  }

  // One single-block region whose values start at `first`; nested regions of
  // its ops are numbered from the end of its values.
  std::string RegionText(const Block& blk, const std::vector<int>& args, Numbering num, uint64_t first) {
    uint64_t nvals = args.size();
    for (const Op& op : blk.ops) nvals += op.results.size();
    const uint64_t end = first + nvals;
    std::string r = V(1) + V(nvals);
    VarIntFlag(r, blk.ops.size(), !args.empty());
    uint64_t next = first;
    if (!args.empty()) {
      VarInt(r, args.size());
      for (int v : args) {
        VarInt(r, uint64_t(Tensor(m_.types[v])));  // type
        VarInt(r, uint64_t(unknown_loc_));         // location (written in every version before 4)
        num[v] = next++;
      }
    }
    for (const Op& op : blk.ops) r += OpText(op, num, next, end);
    return r;
  }

  std::string OpText(const Op& op, Numbering& num, uint64_t& next, uint64_t region_end) {
    std::string base;
    std::map<std::string, int> a;
    if (op.name == "return" || op.name == "func.return" || op.name == "stablehlo.return") {
      base = "return";
    } else if (op.name == "func.call") {
      base = "call";
      a["callee"] = VString(op.attr("callee")->s);
    } else if (op.name.compare(0, 10, "stablehlo.") == 0) {
      base = op.name.substr(10);
      a = OpAttrs(op, base);
    } else {
      Die("op " + op.name + " has no VHLO form in this writer");
    }
    std::vector<int> rts;
    for (int v : op.results) rts.push_back(Tensor(m_.types[v]));
    std::vector<uint64_t> ops;
    for (int v : op.operands) {
      auto it = num.find(v);
      if (it == num.end()) Die("operand of " + op.name + " is not defined before it");
      ops.push_back(it->second);
    }
    std::string o = OpHeader(OpName(1, base + "_v1"), a.empty() ? -1 : Dict(a), rts, ops, !op.regions.empty());
    for (int v : op.results) num[v] = next++;
    if (!op.regions.empty()) {
      VarIntFlag(o, op.regions.size(), false);  // not isolated
      for (const auto& reg : op.regions) {
        if (reg->blocks.size() != 1) Die("only single-block regions are written");
        o += RegionText(reg->blocks[0], reg->blocks[0].args, num, region_end);
      }
    }
    return o;
  }

  std::string Assemble(const std::string& ir) {
    std::string out = "ML\xEFR";
    VarInt(out, 1);
    out += "StableHLO_v1.0.0";
    out.push_back(0);
    // dialects: builtin, vhlo (version 1.0.0 as major, minor, patch)
    std::string d = V(2);
    VarIntFlag(d, uint64_t(t_.Str("builtin")), false);
    VarIntFlag(d, uint64_t(t_.Str("vhlo")), true);
    Section(d, 7, V(1) + V(0) + V(0));
    for (int dl = 0; dl < 2; ++dl) {
      std::vector<int> names;
      for (size_t i = 0; i < op_names_.size(); ++i)
        if (op_names_[i].first == dl) names.push_back(int(i));
      if (names.empty()) continue;
      VarInt(d, uint64_t(dl));
      VarInt(d, names.size());
      for (int i : names) VarInt(d, uint64_t(t_.Str(op_names_[size_t(i)].second)));
    }
    std::string data, offs = V(t_.attrs.size()) + V(t_.types.size());
    auto runs = [&](const std::vector<Entry>& v) {
      for (size_t i = 0; i < v.size();) {
        size_t j = i;
        while (j < v.size() && v[j].dialect == v[i].dialect) ++j;
        VarInt(offs, uint64_t(v[i].dialect));
        VarInt(offs, j - i);
        for (size_t k = i; k < j; ++k) {
          VarIntFlag(offs, v[k].payload.size(), true);
          data += v[k].payload;
        }
        i = j;
      }
    };
    runs(t_.attrs);
    runs(t_.types);
    std::string strs = V(t_.strings.size());
    for (size_t i = t_.strings.size(); i-- > 0;) VarInt(strs, t_.strings[i].size() + 1);
    for (const auto& s : t_.strings) {
      strs += s;
      strs.push_back(0);
    }
    Section(out, 1, d);
    Section(out, 3, offs);
    Section(out, 2, data);
    Section(out, 4, ir);
    Section(out, 0, strs);
    return out;
  }

  const Module& m_;
  Tables t_;
  int unknown_loc_ = 0;
  std::vector<std::pair<int, std::string>> op_names_;
  std::map<std::pair<int, std::string>, int> op_ix_;
};

// ------------------------------------------------------------------ plan comparison
std::string BufText(const BufRef& b) {
  return std::to_string(int(b.space)) + ":" + std::to_string(b.index) + "+" + std::to_string(b.offset);
}

std::string Diff(const Program& a, const Program& b) {
  auto tt = [](const std::vector<TensorType>& v) {
    std::string s;
    for (const auto& t : v) s += t.str() + " ";
    return s;
  };
  if (tt(a.inputs) != tt(b.inputs)) return "inputs: " + tt(a.inputs) + "| " + tt(b.inputs);
  if (tt(a.outputs) != tt(b.outputs)) return "outputs: " + tt(a.outputs) + "| " + tt(b.outputs);
  if (a.arena_bytes != b.arena_bytes)
    return "arena " + std::to_string(a.arena_bytes) + " vs " + std::to_string(b.arena_bytes);
  if (a.input_alias != b.input_alias) return "input aliases differ";
  if (a.patterns != b.patterns) return "fused patterns differ";
  if (a.consts.size() != b.consts.size()) return "constant count differs";
  for (size_t k = 0; k < a.consts.size(); ++k)
    if (a.consts[k].type != b.consts[k].type || a.consts[k].bytes != b.consts[k].bytes)
      return "constant " + std::to_string(k) + " (" + a.consts[k].type.str() + ") differs";
  if (a.steps.size() != b.steps.size())
    return "step count " + std::to_string(a.steps.size()) + " vs " + std::to_string(b.steps.size());
  for (size_t k = 0; k < a.steps.size(); ++k) {
    const Step& x = a.steps[k];
    const Step& y = b.steps[k];
    const std::string at = "step " + std::to_string(k) + " (" + StepName(x.kind) + ")";
    if (x.kind != y.kind) return at + ": kind " + StepName(y.kind);
    if (x.bufs.size() != y.bufs.size()) return at + ": buffer count";
    for (size_t i = 0; i < x.bufs.size(); ++i)
      if (BufText(x.bufs[i]) != BufText(y.bufs[i]))
        return at + ": buffer " + std::to_string(i) + " " + BufText(x.bufs[i]) + " vs " + BufText(y.bufs[i]);
    if (x.i != y.i) return at + ": integer parameters";
    if (x.f.size() != y.f.size() || memcmp(x.f.data(), y.f.data(), x.f.size() * sizeof(float)) != 0)
      return at + ": float parameters";
    if (x.prog != y.prog) return at + ": elementwise program";
    if (x.strides != y.strides) return at + ": strides";
    if (x.types != y.types) return at + ": input types";
    if (x.note != y.note) return at + ": note '" + x.note + "' vs '" + y.note + "'";
  }
  return "";
}

std::string ReadFile(const char* path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) Die(std::string("cannot read ") + path);
  std::stringstream ss;
  ss << f.rdbuf();
  return ss.str();
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 3) Die("usage: vhlo_writer write <module.mlir> <out.mlirbc> | check <module.mlir>");
  const std::string mode = argv[1];
  const std::string text = ReadFile(argv[2]);
  std::string err;
  auto m = ParseText(text.data(), text.size(), err);
  if (!m) Die("text does not parse: " + err);
  const std::string art = Writer(*m).Write();
  if (mode == "write") {
    if (argc < 4) Die("write needs an output path");
    std::ofstream o(argv[3], std::ios::binary);
    o.write(art.data(), std::streamsize(art.size()));
    std::cout << art.size() << " bytes\n";
    return o ? 0 : 2;
  }
  if (mode != "check") Die("unknown mode " + mode);
  CompileResult a = Compile(text.data(), text.size());
  if (!a.program) Die("text does not compile: " + a.error);
  CompileResult b = Compile(art.data(), art.size());
  if (!b.program) {
    std::cout << "artifact does not compile: " << b.error << "\n";
    return 1;
  }
  const std::string d = Diff(*a.program, *b.program);
  if (!d.empty()) {
    std::cout << "plans differ: " << d << "\n";
    return 1;
  }
  std::cout << "same plan: " << a.program->steps.size() << " steps, " << a.program->consts.size() << " constants, "
            << art.size() << " artifact bytes\n";
  return 0;
}
