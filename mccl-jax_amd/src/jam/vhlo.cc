// VHLO → jam IR (see vhlo.h).
#include "jam/vhlo.h"

#include <cstring>
#include <map>
#include <set>

namespace mi::jam {
namespace {

using bytecode::Payload;

// VHLO's binary type codes (stablehlo/dialect/VhloBytecode.cpp, TypeCode):
// the V1 types numbered in the order of their C++ names, later types after
// them.  Only the element types, tensors, functions, tuples and tokens are
// carried; the rest are named in errors.
enum TypeCode : uint64_t {
  kBooleanV1 = 0,
  kComplexV1 = 1,
  kFloatBF16V1 = 2,
  kFloatF16V1 = 3,
  kFloatF32V1 = 4,
  kFloatF64V1 = 5,
  kFloatF8E4M3FNV1 = 6,
  kFloatF8E5M2V1 = 7,
  kFunctionV1 = 8,
  kIndexV1 = 9,
  kIntegerSI16V1 = 10,
  kIntegerSI32V1 = 11,
  kIntegerSI4V1 = 12,
  kIntegerSI64V1 = 13,
  kIntegerSI8V1 = 14,
  kIntegerUI16V1 = 15,
  kIntegerUI32V1 = 16,
  kIntegerUI4V1 = 17,
  kIntegerUI64V1 = 18,
  kIntegerUI8V1 = 19,
  kRankedTensorV1 = 20,
  kRankedTensorV1WithEncoding = 21,
  kTokenV1 = 22,
  kTupleV1 = 23,
  kUniformQuantizedV1 = 24,
  kUnrankedTensorV1 = 25,
  kWitnessV1 = 26,
};

struct ElemInfo {
  DType dtype;
  int bits;
  const char* name;
};

// element types by code; dtype kInvalid for those jam does not carry
const std::map<uint64_t, ElemInfo>& ElementCodes() {
  static const std::map<uint64_t, ElemInfo> m = {
      {kBooleanV1, {DType::kPred, 1, "i1"}},
      {kComplexV1, {DType::kInvalid, 0, "complex"}},
      {kFloatBF16V1, {DType::kBF16, 16, "bf16"}},
      {kFloatF16V1, {DType::kF16, 16, "f16"}},
      {kFloatF32V1, {DType::kF32, 32, "f32"}},
      {kFloatF64V1, {DType::kF64, 64, "f64"}},
      {kFloatF8E4M3FNV1, {DType::kInvalid, 8, "f8E4M3FN"}},
      {kFloatF8E5M2V1, {DType::kInvalid, 8, "f8E5M2"}},
      {kIndexV1, {DType::kInvalid, 64, "index"}},
      {kIntegerSI16V1, {DType::kI16, 16, "i16"}},
      {kIntegerSI32V1, {DType::kI32, 32, "i32"}},
      {kIntegerSI4V1, {DType::kInvalid, 4, "i4"}},
      {kIntegerSI64V1, {DType::kI64, 64, "i64"}},
      {kIntegerSI8V1, {DType::kI8, 8, "i8"}},
      {kIntegerUI16V1, {DType::kU16, 16, "ui16"}},
      {kIntegerUI32V1, {DType::kU32, 32, "ui32"}},
      {kIntegerUI4V1, {DType::kInvalid, 4, "ui4"}},
      {kIntegerUI64V1, {DType::kU64, 64, "ui64"}},
      {kIntegerUI8V1, {DType::kU8, 8, "ui8"}},
      {kWitnessV1, {DType::kInvalid, 0, "witness"}},
  };
  return m;
}

constexpr int64_t kDynamicDim = INT64_MIN;  // ShapedType::kDynamic

struct VType {
  enum Kind { kBad, kElem, kTensor, kFunc, kTuple, kToken, kOther } kind = kBad;
  DType dtype = DType::kInvalid;  // element type (kElem, kTensor)
  int bits = 0;                   // element width in bits
  std::string name;               // element / kind name for messages
  std::vector<int64_t> dims;      // kTensor
  std::vector<uint64_t> ins, outs;  // kFunc inputs / results, kTuple elements
};

// Attribute names whose values the lowering reads, by the shape of value
// each one is decoded as.
enum class Want { kInts, kInt, kBool, kString, kDense, kCmpDir, kCmpType, kPrecisions, kSkip };

const std::map<std::string, Want>& KnownAttrs() {
  static const std::map<std::string, Want> m = {
      {"broadcast_dimensions", Want::kInts}, {"permutation", Want::kInts}, {"dimensions", Want::kInts},
      {"start_indices", Want::kInts},        {"limit_indices", Want::kInts}, {"strides", Want::kInts},
      {"slice_sizes", Want::kInts},          {"edge_padding_low", Want::kInts},
      {"edge_padding_high", Want::kInts},    {"interior_padding", Want::kInts},
      {"lhs_batching_dimensions", Want::kInts}, {"rhs_batching_dimensions", Want::kInts},
      {"lhs_contracting_dimensions", Want::kInts}, {"rhs_contracting_dimensions", Want::kInts},
      {"offset_dims", Want::kInts},          {"collapsed_slice_dims", Want::kInts},
      {"start_index_map", Want::kInts},      {"operand_batching_dims", Want::kInts},
      {"start_indices_batching_dims", Want::kInts}, {"update_window_dims", Want::kInts},
      {"inserted_window_dims", Want::kInts}, {"scatter_dims_to_operand_dims", Want::kInts},
      {"input_batching_dims", Want::kInts},  {"scatter_indices_batching_dims", Want::kInts},
      {"iota_dimension", Want::kInt},        {"dimension", Want::kInt}, {"index_vector_dim", Want::kInt},
      {"indices_are_sorted", Want::kBool},   {"unique_indices", Want::kBool},
      {"comparison_direction", Want::kCmpDir}, {"compare_type", Want::kCmpType},
      {"precision_config", Want::kPrecisions}, {"value", Want::kDense},
      {"call_target_name", Want::kString},
  };
  return m;
}

const char* const kCmpDir[] = {"EQ", "NE", "GE", "GT", "LE", "LT"};
const char* const kCmpType[] = {"NOTYPE", "FLOAT", "TOTALORDER", "SIGNED", "UNSIGNED"};
const char* const kPrecision[] = {"DEFAULT", "HIGH", "HIGHEST"};

// which dictionary of the text form an op's flattened dimension numbers go to
const char* Regroup(const std::string& op, const std::string& attr) {
  static const std::set<std::string> dot = {"lhs_batching_dimensions", "rhs_batching_dimensions",
                                            "lhs_contracting_dimensions", "rhs_contracting_dimensions"};
  static const std::set<std::string> gather = {"offset_dims", "collapsed_slice_dims", "start_index_map",
                                               "index_vector_dim", "operand_batching_dims",
                                               "start_indices_batching_dims"};
  static const std::set<std::string> scatter = {"update_window_dims", "inserted_window_dims",
                                                "scatter_dims_to_operand_dims", "index_vector_dim",
                                                "input_batching_dims", "scatter_indices_batching_dims"};
  if (op == "dot_general" && dot.count(attr)) return "dot_dimension_numbers";
  if ((op == "gather" || op == "dynamic_gather") && gather.count(attr)) return "dimension_numbers";
  if (op == "scatter" && scatter.count(attr)) return "scatter_dimension_numbers";
  return nullptr;
}

class Decoder {
 public:
  Decoder(const bytecode::Module& bm, Module& m, std::string& err) : bm_(bm), m_(m), err_(err) {
    types_.resize(bm.types.size());
    type_state_.assign(bm.types.size(), 0);
  }

  bool Run() {
    const auto& top = bm_.top.ops;
    if (top.size() != 1 || bm_.OpFullName(top[0].name) != "builtin.module")
      return Fail("the artifact's top level is not one builtin.module");
    const bytecode::Op& mod = top[0];
    if (mod.regions.size() != 1 || mod.regions[0].blocks.size() != 1)
      return Fail("builtin.module does not hold one block");
    ModuleName(mod);
    const bytecode::Block& body = mod.regions[0].blocks[0];
    // function names first: a call may name a function defined after it
    for (const bytecode::Op& op : body.ops) {
      if (Base(op) != "func") return Fail("module-level operation " + bm_.OpFullName(op.name) + " is not vhlo.func");
      NamedRefs attrs;
      if (!Attrs(op, &attrs)) return false;
      auto it = attrs.find("sym_name");
      std::string name;
      if (it == attrs.end() || !StringOf(it->second, &name)) return Fail("vhlo.func without a readable sym_name");
      func_names_.insert(name);
    }
    PushRegion(mod.regions[0], /*isolated=*/true);
    for (const bytecode::Op& op : body.ops)
      if (!Function(op)) return false;
    PopRegion(mod.regions[0], true);
    return true;
  }

 private:
  using NamedRefs = std::map<std::string, uint64_t>;

  bool Fail(const std::string& what) {
    if (err_.empty()) err_ = "jam: VHLO: " + what;
    return false;
  }

  // ---------------------------------------------------------------- payloads
  const bytecode::Entry& AttrEntry(uint64_t i) const { return bm_.attrs[i]; }
  const std::string& DialectOf(const bytecode::Entry& e) const { return bm_.dialects[size_t(e.dialect)]; }

  // The payload of attribute i after its code; false if i is out of range
  // or the entry is not in a binary encoding.
  bool AttrPayload(uint64_t i, Payload* p, uint64_t* code) {
    if (i >= bm_.attrs.size()) return false;
    const bytecode::Entry& e = bm_.attrs[i];
    if (!e.custom) return false;
    *p = Payload(bm_.attr_type_data.data() + e.offset, e.size);
    return p->VarInt(code);
  }

  // ---------------------------------------------------------------- types
  const VType* Type(uint64_t i) {
    if (i >= types_.size()) {
      Fail("type index " + std::to_string(i) + " out of range");
      return nullptr;
    }
    if (type_state_[i] == 2) return &types_[i];
    if (type_state_[i] == 1) {
      Fail("type " + std::to_string(i) + " refers to itself");
      return nullptr;
    }
    type_state_[i] = 1;
    VType t;
    if (!DecodeType(i, &t)) {
      type_state_[i] = 0;
      return nullptr;
    }
    types_[i] = std::move(t);
    type_state_[i] = 2;
    return &types_[i];
  }

  bool DecodeType(uint64_t i, VType* t) {
    const bytecode::Entry& e = bm_.types[i];
    const std::string where = "type " + std::to_string(i);
    if (!e.custom) return Fail(where + " is in textual form ('" + bm_.EntryText(e) + "'), not VHLO's encoding");
    if (DialectOf(e) != "vhlo") return Fail(where + " is a " + DialectOf(e) + " type, not a VHLO type");
    Payload p(bm_.attr_type_data.data() + e.offset, e.size);
    uint64_t code;
    if (!p.VarInt(&code)) return Fail(where + ": empty payload");
    auto el = ElementCodes().find(code);
    if (el != ElementCodes().end()) {
      t->kind = VType::kElem;
      t->dtype = el->second.dtype;
      t->bits = el->second.bits;
      t->name = el->second.name;
    } else if (code == kRankedTensorV1 || code == kRankedTensorV1WithEncoding) {
      if (code == kRankedTensorV1WithEncoding) {
        uint64_t enc;
        if (!p.VarInt(&enc)) return Fail(where + ": truncated tensor encoding");
        // bounded dynamism: the encoding only matters with dynamic dims,
        // which are refused below
      }
      uint64_t rank;
      if (!p.VarInt(&rank) || rank > p.left()) return Fail(where + ": malformed tensor shape");
      t->dims.resize(rank);
      for (auto& d : t->dims) {
        if (!p.SignedVarInt(&d)) return Fail(where + ": malformed tensor shape");
        if (d == kDynamicDim) return Fail(where + " has a dynamic dimension (only static shapes are compiled)");
        if (d < 0) return Fail(where + " has a negative dimension");
      }
      uint64_t et;
      if (!p.VarInt(&et)) return Fail(where + ": tensor without an element type");
      const VType* elem = Type(et);
      if (!elem) return false;
      if (elem->kind != VType::kElem) return Fail(where + ": tensor element type is not a scalar type");
      t->kind = VType::kTensor;
      t->dtype = elem->dtype;
      t->bits = elem->bits;
      t->name = elem->name;
    } else if (code == kFunctionV1 || code == kTupleV1) {
      auto list = [&](std::vector<uint64_t>* out) {
        uint64_t n;
        if (!p.VarInt(&n) || n > p.left()) return false;
        out->resize(n);
        for (auto& x : *out)
          if (!p.VarInt(&x) || x >= bm_.types.size()) return false;
        return true;
      };
      if (!list(&t->ins) || (code == kFunctionV1 && !list(&t->outs)))
        return Fail(where + ": malformed " + (code == kFunctionV1 ? "function" : "tuple") + " type");
      t->kind = code == kFunctionV1 ? VType::kFunc : VType::kTuple;
      t->name = code == kFunctionV1 ? "function" : "tuple";
    } else if (code == kTokenV1) {
      t->kind = VType::kToken;
      t->dtype = DType::kToken;
      t->name = "token";
    } else {
      static const std::map<uint64_t, const char*> other = {{kUniformQuantizedV1, "quantized tensor element"},
                                                            {kUnrankedTensorV1, "unranked tensor"}};
      auto it = other.find(code);
      return Fail(where + (it != other.end() ? std::string(" is an ") + it->second + " type, which is not compiled"
                                             : " has type code " + std::to_string(code) + ", which is not decoded"));
    }
    if (!p.at_end()) return Fail(where + ": payload longer than its type");
    return true;
  }

  // tensor (or token) type of a value
  bool ValueType(uint64_t i, TensorType* out) {
    const VType* t = Type(i);
    if (!t) return false;
    if (t->kind == VType::kToken) {
      out->dtype = DType::kToken;
      out->dims.clear();
      return true;
    }
    if (t->kind != VType::kTensor) return Fail("a value of " + t->name + " type (values are tensors)");
    if (t->dtype == DType::kInvalid) return Fail("element type " + t->name + " is not supported");
    out->dtype = t->dtype;
    out->dims = t->dims;
    return true;
  }

  // ---------------------------------------------------------------- attributes
  // A string: builtin StringAttr or VHLO StringV1Attr (code, string index),
  // or the textual form "...".
  bool StringOf(uint64_t i, std::string* out) {
    if (i >= bm_.attrs.size()) return false;
    const bytecode::Entry& e = bm_.attrs[i];
    if (!e.custom) {
      const std::string t = bm_.EntryText(e);
      if (t.size() < 2 || t.front() != '"' || t.back() != '"') return false;
      *out = t.substr(1, t.size() - 2);
      return true;
    }
    Payload p(nullptr, 0);
    uint64_t code, s;
    if (!AttrPayload(i, &p, &code) || !p.VarInt(&s) || !p.at_end() || s >= bm_.strings.size()) return false;
    *out = bm_.strings[s];
    return true;
  }

  // A dictionary: builtin DictionaryAttr or VHLO DictionaryV1Attr (code,
  // count, then name and value attribute indices), names being strings.
  bool DictOf(uint64_t i, NamedRefs* out) {
    Payload p(nullptr, 0);
    uint64_t code, n;
    if (!AttrPayload(i, &p, &code) || !p.VarInt(&n) || n > p.left()) return false;
    for (uint64_t k = 0; k < n; ++k) {
      uint64_t key, val;
      std::string name;
      if (!p.VarInt(&key) || !p.VarInt(&val) || val >= bm_.attrs.size() || !StringOf(key, &name)) return false;
      (*out)[name] = val;
    }
    return p.at_end();
  }

  // An array: ArrayV1Attr (code, count, element attribute indices).
  bool ListOf(uint64_t i, std::vector<uint64_t>* out) {
    Payload p(nullptr, 0);
    uint64_t code, n;
    if (!AttrPayload(i, &p, &code) || !p.VarInt(&n) || n > p.left()) return false;
    out->resize(n);
    for (auto& x : *out)
      if (!p.VarInt(&x) || x >= bm_.attrs.size()) return false;
    return p.at_end();
  }

  // IntegerV1Attr: code, integer type, the value as an APInt of its width.
  bool IntOf(uint64_t i, int64_t* out) {
    Payload p(nullptr, 0);
    uint64_t code, ty, bits;
    if (!AttrPayload(i, &p, &code) || !p.VarInt(&ty) || ty >= bm_.types.size()) return false;
    const VType* t = Type(ty);
    if (!t || t->kind != VType::kElem || IsFloat(t->dtype) || t->dtype == DType::kInvalid) return false;
    bool wide = false;
    if (!p.APInt(unsigned(t->bits), &bits, &wide) || wide || !p.at_end()) return false;
    *out = Extend(bits, t->bits, !IsUnsigned(t->dtype) && t->dtype != DType::kPred);
    return true;
  }

  // BooleanV1Attr and the enum attributes: code, varint value.
  bool SmallOf(uint64_t i, uint64_t* out) {
    Payload p(nullptr, 0);
    uint64_t code;
    return AttrPayload(i, &p, &code) && p.VarInt(out) && p.at_end();
  }

  static int64_t Extend(uint64_t bits, int width, bool sign) {
    if (width >= 64) return int64_t(bits);
    bits &= (uint64_t(1) << width) - 1;
    if (sign && (bits >> (width - 1)) & 1) bits |= ~((uint64_t(1) << width) - 1);
    return int64_t(bits);
  }

  // TensorV1Attr: code, tensor type, blob of the elements' little-endian
  // bytes (one element when the tensor is a splat; i1 bit-packed, or one
  // byte 0x00 / 0xFF for a splat).  Yields the elements' bytes, one element
  // per DTypeBytes, expanded from a splat when `expand`.
  bool TensorOf(uint64_t i, uint64_t* type_index, std::vector<uint8_t>* bytes, bool* splat) {
    Payload p(nullptr, 0);
    uint64_t code, ty;
    const uint8_t* data;
    size_t size;
    if (!AttrPayload(i, &p, &code) || !p.VarInt(&ty) || ty >= bm_.types.size()) return false;
    const VType* t = Type(ty);
    if (!t || t->kind != VType::kTensor || t->dtype == DType::kInvalid) return false;
    if (!p.Blob(&data, &size) || !p.at_end()) return false;
    int64_t n = 1;
    for (int64_t d : t->dims) n *= d;
    const size_t w = size_t(DTypeBytes(t->dtype));
    *type_index = ty;
    *splat = false;
    bytes->clear();
    if (t->dtype == DType::kPred) {
      if (size == 1 && (data[0] == 0 || data[0] == 0xFF || n == 1)) {
        bytes->push_back(data[0] ? 1 : 0);
        *splat = n != 1;
      } else if (int64_t(size) == (n + 7) / 8) {
        for (int64_t k = 0; k < n; ++k) bytes->push_back((data[k / 8] >> (k % 8)) & 1);
      } else {
        return false;
      }
      return true;
    }
    if (int64_t(size) == n * int64_t(w)) {
      bytes->assign(data, data + size);
    } else if (size == w && n != 1) {
      bytes->assign(data, data + size);
      *splat = true;
    } else {
      return false;
    }
    return true;
  }

  // Dimension lists: a TensorV1Attr of integers, or an ArrayV1Attr of
  // IntegerV1Attr.
  bool IntsOf(uint64_t i, std::vector<int64_t>* out) {
    uint64_t ty;
    std::vector<uint8_t> raw;
    bool splat;
    if (TensorOf(i, &ty, &raw, &splat)) {
      const VType* t = Type(ty);
      if (t->dims.size() != 1 || IsFloat(t->dtype) || t->dtype == DType::kPred) return false;
      const size_t w = size_t(DTypeBytes(t->dtype));
      out->clear();
      for (int64_t k = 0; k < t->dims[0]; ++k) {
        uint64_t bits = 0;
        memcpy(&bits, raw.data() + (splat ? 0 : size_t(k) * w), w);
        out->push_back(Extend(bits, int(8 * w), !IsUnsigned(t->dtype)));
      }
      return true;
    }
    err_.clear();  // a failed tensor reading is not an error yet
    std::vector<uint64_t> elems;
    if (!ListOf(i, &elems)) return false;
    out->clear();
    for (uint64_t e : elems) {
      int64_t v;
      if (!IntOf(e, &v)) return false;
      out->push_back(v);
    }
    return true;
  }

  bool TypeAttrOf(uint64_t i, uint64_t* type_index) {
    Payload p(nullptr, 0);
    uint64_t code;
    if (!AttrPayload(i, &p, &code) || !p.VarInt(type_index) || !p.at_end()) return false;
    return *type_index < bm_.types.size();
  }

  static Attr IntAttr(int64_t v) {
    Attr a;
    a.kind = Attr::kInt;
    a.i = v;
    return a;
  }
  static Attr IntsAttr(const std::vector<int64_t>& v) {
    Attr a;
    a.kind = Attr::kList;
    for (int64_t x : v) a.list.push_back(IntAttr(x));
    return a;
  }
  static Attr EnumAttr(const char* s) {
    Attr a;
    a.kind = Attr::kEnum;
    a.s = s;
    return a;
  }

  // One known attribute of an op in the text reader's form; false (with the
  // error set) when its payload does not have the shape its name calls for.
  bool Convert(const std::string& op, const std::string& name, uint64_t ref, Want want, const TensorType* result,
               Attr* out) {
    const std::string where = "attribute '" + name + "' of vhlo." + op;
    switch (want) {
      case Want::kInts: {
        std::vector<int64_t> v;
        if (!IntsOf(ref, &v)) return Fail(where + " is not a list of integers");
        *out = IntsAttr(v);
        return true;
      }
      case Want::kInt: {
        int64_t v;
        if (!IntOf(ref, &v)) return Fail(where + " is not an integer");
        *out = IntAttr(v);
        return true;
      }
      case Want::kBool: {
        uint64_t v;
        if (!SmallOf(ref, &v) || v > 1) return Fail(where + " is not a boolean");
        out->kind = Attr::kBool;
        out->i = int64_t(v);
        return true;
      }
      case Want::kString: {
        std::string s;
        if (!StringOf(ref, &s)) return Fail(where + " is not a string");
        out->kind = Attr::kString;
        out->s = s;
        return true;
      }
      case Want::kCmpDir:
      case Want::kCmpType: {
        uint64_t v;
        const size_t n = want == Want::kCmpDir ? 6 : 5;
        if (!SmallOf(ref, &v) || v >= n) return Fail(where + " is not a comparison enum");
        *out = EnumAttr(want == Want::kCmpDir ? kCmpDir[v] : kCmpType[v]);
        return true;
      }
      case Want::kPrecisions: {
        std::vector<uint64_t> elems;
        if (!ListOf(ref, &elems)) return Fail(where + " is not an array");
        out->kind = Attr::kList;
        for (uint64_t e : elems) {
          uint64_t v;
          if (!SmallOf(e, &v) || v > 2) return Fail(where + " holds something other than a precision");
          out->list.push_back(EnumAttr(kPrecision[v]));
        }
        return true;
      }
      case Want::kDense: {
        uint64_t ty;
        std::vector<uint8_t> raw;
        bool splat;
        if (!TensorOf(ref, &ty, &raw, &splat)) return Fail(where + " is not a dense tensor of a carried type");
        TensorType t;
        if (!ValueType(ty, &t)) return false;
        if (result && t != *result)
          return Fail(where + " has type " + t.str() + " but the op returns " + result->str());
        static const char* hex = "0123456789ABCDEF";
        std::string s = "\"0x";
        s.reserve(4 + 2 * raw.size());
        for (uint8_t b : raw) {
          s.push_back(hex[b >> 4]);
          s.push_back(hex[b & 15]);
        }
        s.push_back('"');
        out->kind = Attr::kDense;
        out->s = std::move(s);
        out->dense_type = t;
        return true;
      }
      case Want::kSkip:
        return true;
    }
    return true;
  }

  // ---------------------------------------------------------------- IR
  // "vhlo.add_v1" -> "add"
  std::string Base(const bytecode::Op& op) const {
    const std::string full = bm_.OpFullName(op.name);
    if (full.compare(0, 5, "vhlo.") != 0) return "";
    std::string b = full.substr(5);
    const size_t v = b.rfind("_v");
    if (v != std::string::npos && v + 2 < b.size() &&
        b.find_first_not_of("0123456789", v + 2) == std::string::npos)
      b.resize(v);
    return b;
  }

  bool Attrs(const bytecode::Op& op, NamedRefs* out) {
    if (op.properties >= 0)
      return Fail("vhlo op " + bm_.OpFullName(op.name) +
                  " stores its attributes as properties (bytecode v5+), which are not decoded; "
                  "StableHLO portable artifacts are written as bytecode v1");
    if (op.attr_dict < 0) return true;
    if (!DictOf(uint64_t(op.attr_dict), out))
      return Fail("the attribute dictionary of " + bm_.OpFullName(op.name) + " is malformed");
    return true;
  }

  void ModuleName(const bytecode::Op& mod) {
    NamedRefs attrs;
    if (mod.attr_dict < 0 || !DictOf(uint64_t(mod.attr_dict), &attrs)) return;
    auto it = attrs.find("sym_name");
    std::string s;
    if (it != attrs.end() && StringOf(it->second, &s)) m_.name = s;
  }

  // value numbering (see vhlo.h)
  struct Scope {
    std::vector<int> ids;
    std::vector<size_t> next;
  };
  void PushRegion(const bytecode::Region& r, bool isolated) {
    if (isolated || scopes_.empty()) scopes_.emplace_back();
    Scope& s = scopes_.back();
    s.next.push_back(s.ids.size());
    s.ids.resize(s.ids.size() + size_t(r.num_values), -1);
  }
  void PopRegion(const bytecode::Region& r, bool isolated) {
    Scope& s = scopes_.back();
    s.ids.resize(s.ids.size() - size_t(r.num_values));
    s.next.pop_back();
    if (isolated) scopes_.pop_back();
  }
  bool Define(int id) {
    Scope& s = scopes_.back();
    size_t& n = s.next.back();
    if (n >= s.ids.size()) return Fail("a region defines more values than its header counts");
    s.ids[n++] = id;
    return true;
  }
  bool Use(uint64_t v, int* id) {
    const Scope& s = scopes_.back();
    if (v >= s.ids.size() || s.ids[v] < 0) return Fail("use of value " + std::to_string(v) + " before it is defined");
    *id = s.ids[v];
    return true;
  }

  bool Function(const bytecode::Op& op) {
    NamedRefs attrs;
    if (!Attrs(op, &attrs)) return false;
    jam::Func f;
    StringOf(attrs.at("sym_name"), &f.name);
    auto vis = attrs.find("sym_visibility");
    std::string v;
    if (vis != attrs.end() && StringOf(vis->second, &v)) f.is_public = v != "private" && v != "nested";
    const std::string where = "vhlo.func @" + f.name;
    auto ft = attrs.find("function_type");
    uint64_t fti;
    if (ft == attrs.end() || !TypeAttrOf(ft->second, &fti)) return Fail(where + " has no function_type");
    const VType* fty = Type(fti);
    if (!fty) return false;
    if (fty->kind != VType::kFunc) return Fail(where + ": function_type is not a function type");
    const std::vector<uint64_t> ins = fty->ins, outs = fty->outs;
    for (uint64_t r : outs) {
      TensorType t;
      if (!ValueType(r, &t)) return false;
      f.result_types.push_back(t);
    }
    if (op.regions.size() != 1 || op.regions[0].blocks.size() != 1)
      return Fail(where + " does not have one body block");
    const bytecode::Region& reg = op.regions[0];
    const bytecode::Block& blk = reg.blocks[0];
    if (blk.args.size() != ins.size()) return Fail(where + ": body arguments differ from function_type");
    f.arg_alias.assign(ins.size(), -1);
    f.arg_donor.assign(ins.size(), false);
    auto aa = attrs.find("arg_attrs");
    std::vector<uint64_t> per_arg;
    if (aa != attrs.end() && ListOf(aa->second, &per_arg)) {
      for (size_t k = 0; k < per_arg.size() && k < ins.size(); ++k) {
        NamedRefs d;
        if (!DictOf(per_arg[k], &d)) continue;
        auto al = d.find("tf.aliasing_output");
        int64_t out;
        if (al != d.end()) {
          if (!IntOf(al->second, &out)) return Fail(where + ": tf.aliasing_output is not an integer");
          f.arg_alias[k] = int(out);
        }
        auto dn = d.find("jax.buffer_donor");
        if (dn != d.end()) {
          uint64_t b = 1;
          f.arg_donor[k] = !SmallOf(dn->second, &b) || b != 0;
        }
      }
    }
    PushRegion(reg, op.isolated);
    for (size_t k = 0; k < blk.args.size(); ++k) {
      if (blk.args[k].type != ins[k]) {
        TensorType a, b;
        if (!ValueType(blk.args[k].type, &a) || !ValueType(ins[k], &b)) return false;
        if (a != b) return Fail(where + ": argument " + std::to_string(k) + " type differs from function_type");
      }
      TensorType t;
      if (!ValueType(blk.args[k].type, &t)) return false;
      const int id = m_.new_value(t, "%arg" + std::to_string(k));
      if (!Define(id)) return false;
      f.args.push_back(id);
    }
    for (const bytecode::Op& o : blk.ops)
      if (!Operation(o, f.body, /*in_func=*/true)) return false;
    PopRegion(reg, op.isolated);
    m_.funcs.push_back(std::move(f));
    return true;
  }

  bool Operation(const bytecode::Op& bop, Block& into, bool in_func) {
    const std::string base = Base(bop);
    const std::string full = bm_.OpFullName(bop.name);
    if (base.empty()) return Fail("operation " + full + " is not a VHLO operation");
    if (base == "func") return Fail("nested vhlo.func");
    NamedRefs attrs;
    if (!Attrs(bop, &attrs)) return false;
    Op op;
    if (base == "return") {
      op.name = "return";
    } else if (base == "call") {
      op.name = "func.call";
    } else {
      op.name = "stablehlo." + base;
    }
    for (uint64_t v : bop.operands) {
      int id;
      if (!Use(v, &id)) return false;
      op.operands.push_back(id);
    }
    std::vector<TensorType> result_types;
    for (uint64_t t : bop.result_types) {
      TensorType tt;
      if (!ValueType(t, &tt)) return false;
      result_types.push_back(tt);
    }
    if (base == "call") {
      auto it = attrs.find("callee");
      if (it == attrs.end()) return Fail("vhlo.call without a callee");
      std::string callee;
      if (!Callee(it->second, &callee)) return Fail("vhlo.call names no function of the module");
      Attr a;
      a.kind = Attr::kSymbol;
      a.s = callee;
      op.attrs["callee"] = a;
    } else {
      const TensorType* r0 = result_types.empty() ? nullptr : &result_types[0];
      for (const auto& [name, ref] : attrs) {
        auto k = KnownAttrs().find(name);
        if (k == KnownAttrs().end()) continue;  // not read by the lowering
        Attr a;
        if (!Convert(base, name, ref, k->second, r0, &a)) return false;
        if (const char* group = Regroup(base, name)) {
          Attr& g = op.attrs[group];
          g.kind = Attr::kDict;
          g.dict[name] = a;
        } else {
          op.attrs[name] = a;
        }
      }
      for (const char* batch : {"operand_batching_dims", "start_indices_batching_dims", "input_batching_dims",
                                "scatter_indices_batching_dims"}) {
        const char* group = Regroup(base, batch);
        const Attr* g = group ? op.attr(group) : nullptr;
        const Attr* b = g ? g->get(batch) : nullptr;
        if (b && !b->list.empty()) return Fail("vhlo." + base + " with batching dimensions is not compiled");
      }
      if (!CheckCompareType(op)) return false;
    }
    // results are defined before the op's regions are read
    for (const TensorType& t : result_types) {
      const int id = m_.new_value(t);
      if (!Define(id)) return false;
      op.results.push_back(id);
    }
    for (const bytecode::Region& r : bop.regions) {
      auto region = std::make_shared<Region>();
      PushRegion(r, bop.isolated);
      for (const bytecode::Block& b : r.blocks) {
        region->blocks.emplace_back();
        Block& nb = region->blocks.back();
        for (const bytecode::BlockArg& a : b.args) {
          TensorType t;
          if (!ValueType(a.type, &t)) return false;
          const int id = m_.new_value(t);
          if (!Define(id)) return false;
          nb.args.push_back(id);
        }
        for (const bytecode::Op& o : b.ops)
          if (!Operation(o, nb, false)) return false;
      }
      PopRegion(r, bop.isolated);
      op.regions.push_back(region);
    }
    (void)in_func;
    into.ops.push_back(std::move(op));
    return true;
  }

  // vhlo.call's callee: a string attribute naming the function, or a
  // symbol reference attribute holding that string.
  bool Callee(uint64_t ref, std::string* out) {
    std::string s;
    if (StringOf(ref, &s) && func_names_.count(s)) {
      *out = s;
      return true;
    }
    Payload p(nullptr, 0);
    uint64_t code, inner;
    if (AttrPayload(ref, &p, &code) && p.VarInt(&inner) && p.at_end() && StringOf(inner, &s) &&
        func_names_.count(s)) {
      *out = s;
      return true;
    }
    return false;
  }

  // compare_type must agree with the operands' element type: a check that
  // the element type codes were read as the writer meant them
  bool CheckCompareType(const Op& op) {
    if (op.name != "stablehlo.compare" || op.operands.empty()) return true;
    const Attr* ct = op.attr("compare_type");
    if (!ct) return true;
    const DType d = m_.types[op.operands[0]].dtype;
    bool ok = true;
    if (ct->s == "FLOAT" || ct->s == "TOTALORDER") ok = IsFloat(d);
    else if (ct->s == "SIGNED") ok = IsSigned(d);
    else if (ct->s == "UNSIGNED") ok = IsUnsigned(d) || d == DType::kPred;
    if (!ok)
      return Fail("compare_type " + ct->s + " on " + DTypeName(d) +
                  " operands: the element type codes of this artifact are not the ones this reader knows");
    return true;
  }

  const bytecode::Module& bm_;
  Module& m_;
  std::string& err_;
  std::vector<VType> types_;
  std::vector<uint8_t> type_state_;  // 0 unread, 1 reading, 2 done
  std::vector<Scope> scopes_;
  std::set<std::string> func_names_;
};

}  // namespace

std::unique_ptr<Module> FromVhlo(const bytecode::Module& bm, std::string& error) {
  error.clear();
  bool has_vhlo = false;
  for (const std::string& d : bm.dialects) has_vhlo |= d == "vhlo";
  if (!has_vhlo) {
    error = "jam: VHLO: the bytecode holds no vhlo dialect (not a StableHLO portable artifact)";
    return nullptr;
  }
  auto m = std::make_unique<Module>();
  Decoder d(bm, *m, error);
  if (!d.Run()) {
    if (error.empty()) error = "jam: VHLO: malformed artifact";
    return nullptr;
  }
  return m;
}

}  // namespace mi::jam
