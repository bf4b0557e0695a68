// jam IR: the in-memory form of a StableHLO module.
//
// The reference hands StableHLO to MLIR and walks mlir::Operation objects
// (src/jam/lower.mm:208-314).  This image has no MLIR/StableHLO libraries,
// so jam carries its own small SSA IR: values are integer ids with a tensor
// type, ops are (name, operands, results, attributes, regions).  Attributes
// keep only what the lowering needs (ints, int lists, floats, enums, dense
// element lists, nested dictionaries).
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace mi::jam {

// Element types (values equal PJRT_Buffer_Type / mk_dtype numbering).
enum class DType : int {
  kInvalid = 0, kPred = 1, kI8 = 2, kI16 = 3, kI32 = 4, kI64 = 5,
  kU8 = 6, kU16 = 7, kU32 = 8, kU64 = 9, kF16 = 10, kF32 = 11, kF64 = 12, kBF16 = 13,
  kToken = 23,
};

int DTypeBytes(DType d);
bool IsFloat(DType d);
bool IsSigned(DType d);
bool IsUnsigned(DType d);
const char* DTypeName(DType d);
DType ParseElementType(const std::string& s);  // "f32", "bf16", "i1", "ui8", ... (kInvalid if unknown)

struct TensorType {
  DType dtype = DType::kInvalid;
  std::vector<int64_t> dims;
  int64_t numel() const {
    int64_t n = 1;
    for (int64_t d : dims) n *= d;
    return n;
  }
  size_t bytes() const { return size_t(numel()) * size_t(DTypeBytes(dtype)); }
  int rank() const { return int(dims.size()); }
  bool operator==(const TensorType& o) const { return dtype == o.dtype && dims == o.dims; }
  bool operator!=(const TensorType& o) const { return !(*this == o); }
  std::string str() const;
};

struct Attr {
  enum Kind { kNone, kInt, kFloat, kBool, kString, kEnum, kList, kDense, kDict, kSymbol, kType };
  Kind kind = kNone;
  int64_t i = 0;
  double f = 0;
  std::string s;                        // string / enum word / symbol / type text
  std::vector<Attr> list;               // kList elements
  std::map<std::string, Attr> dict;     // kDict entries (also #stablehlo.xxx<...> params)
  // kDense: element values (ints for integer/pred types, doubles for floats)
  TensorType dense_type;
  bool splat = false;
  std::vector<double> fvals;
  std::vector<int64_t> ivals;

  std::vector<int64_t> ints() const;    // kList of kInt (or kDense ints) -> int vector
  const Attr* get(const std::string& k) const {
    auto it = dict.find(k);
    return it == dict.end() ? nullptr : &it->second;
  }
};

struct Region;

struct Op {
  std::string name;             // e.g. "stablehlo.add", "func.return", "func.call"
  std::vector<int> operands;    // value ids
  std::vector<int> results;     // value ids
  std::map<std::string, Attr> attrs;
  std::vector<std::shared_ptr<Region>> regions;
  int line = 0;                 // source line for diagnostics
  const Attr* attr(const std::string& k) const {
    auto it = attrs.find(k);
    return it == attrs.end() ? nullptr : &it->second;
  }
};

struct Block {
  std::vector<int> args;        // value ids of block arguments
  std::vector<Op> ops;
};

struct Region {
  std::vector<Block> blocks;
};

struct Func {
  std::string name;
  bool is_public = true;
  std::vector<int> args;
  // per argument: `tf.aliasing_output = k` (the output a donated argument may
  // share memory with; -1 none) and `jax.buffer_donor` (donated, output
  // chosen by type)
  std::vector<int> arg_alias;
  std::vector<bool> arg_donor;
  std::vector<TensorType> result_types;
  Block body;
};

struct Module {
  std::string name;
  std::vector<Func> funcs;
  std::vector<TensorType> types;  // indexed by value id
  std::vector<std::string> value_names;

  int new_value(const TensorType& t, const std::string& name = "") {
    types.push_back(t);
    value_names.push_back(name);
    return int(types.size()) - 1;
  }
  const Func* find(const std::string& fname) const {
    for (const auto& f : funcs)
      if (f.name == fname) return &f;
    return nullptr;
  }
};

// Parse StableHLO / MLIR textual assembly.  Returns nullptr and sets `error`
// on failure (message prefixed "jam: ").
std::unique_ptr<Module> ParseText(const char* text, size_t size, std::string& error);

// True when the buffer starts with the MLIR bytecode magic "ML\xEFR".
bool IsMlirBytecode(const char* data, size_t size);

}  // namespace mi::jam
