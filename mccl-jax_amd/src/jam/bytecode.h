// Reader of the MLIR bytecode container, the on-wire form of a StableHLO
// portable artifact (what jaxlib hands to PJRT_Client_Compile).
//
// The reference deserializes artifacts with the MLIR libraries
// (src/jam/parse.cc:53-63, mlir::stablehlo::deserializePortableArtifact) and
// then runs its passes on the resulting module.  This build has no MLIR, so
// this file implements the container format itself, as MLIR's bytecode
// format documentation specifies it (mlir/docs/BytecodeFormat.md):
//   magic "ML\xEFR", version varint, producer (NUL-terminated string), then
//   sections {id | aligned << 7, length varint, [alignment varint, 0xCB
//   padding], data}.
// Sections read here: strings (0), dialects with their versions (1, with
// nested 7), attribute/type offsets (3) over the attribute/type data (2), the
// IR (4, nested for isolated regions from version 2), properties (8, skipped
// per entry), resources (5/6, kept as raw ranges).  Numbers are prefix
// varints (the count of trailing zero bits of the first byte, plus one, is
// the byte count; a zero first byte means eight raw bytes follow), flags ride
// in the low bit.
//
// What the reader yields is the operation tree: op names (dialect + name),
// attribute-dictionary / type / value references and the regions, blocks and
// block arguments, plus each attribute's and type's entry (dialect, bytes,
// whether it is a dialect-specific binary encoding or the textual form).
// Turning VHLO's binary attribute and type encodings into jam IR is done by
// vhlo.cc on top of this tree.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace mi::jam::bytecode {

struct OpName {
  int dialect = 0;
  std::string name;  // without the dialect prefix
  bool registered = true;
};

struct Entry {  // one attribute or type
  int dialect = 0;
  size_t offset = 0, size = 0;  // within the attribute/type section data
  bool custom = false;          // dialect binary encoding; else NUL-terminated text
};

struct Region;

struct Op {
  uint64_t name = 0;                 // index into Module::op_names
  uint8_t mask = 0;
  uint64_t location = 0;             // attribute index
  int64_t attr_dict = -1;            // attribute index, -1 when absent
  int64_t properties = -1;           // properties index, -1 when absent
  std::vector<uint64_t> result_types;  // type indices
  std::vector<uint64_t> operands;      // value numbers
  std::vector<uint64_t> successors;    // block numbers
  bool isolated = false;
  std::vector<Region> regions;
};

struct BlockArg {
  uint64_t type = 0;
  int64_t location = -1;  // -1: unknown location (elided from version 4)
};

struct Block {
  std::vector<BlockArg> args;
  std::vector<Op> ops;
};

struct Region {
  uint64_t num_values = 0;
  std::vector<Block> blocks;
};

struct Module {
  uint64_t version = 0;
  std::string producer;
  std::vector<std::string> strings;
  std::vector<std::string> dialects;
  std::vector<std::vector<uint8_t>> dialect_versions;  // raw version payload, empty when none
  std::vector<OpName> op_names;
  std::vector<Entry> attrs, types;
  std::vector<uint8_t> attr_type_data;
  Block top;  // the top-level block (normally one builtin.module op)

  std::string OpFullName(uint64_t i) const;
  // The text of an attribute or type stored in textual form ("" if custom).
  std::string EntryText(const Entry& e) const;
  // Counts of every op name in the tree, in first-seen order: "name x n, ...".
  std::string OpHistogram() const;
  // Dialect version payloads decoded as varints, e.g. "vhlo 1.9.3" (the VHLO
  // dialect writes major, minor, patch).
  std::string DialectVersionText(size_t d) const;
};

// Parses a whole bytecode buffer.  On failure returns false and sets *error to
// a message naming the offset and what was malformed.
bool Read(const uint8_t* data, size_t size, Module* out, std::string* error);

// Reader of one attribute or type payload in a dialect's binary encoding:
// the primitives MLIR's DialectBytecodeReader offers (varints, zigzag signed
// varints, blobs, APInts of a known width).  Every method returns false at
// the end of the payload.
class Payload {
 public:
  Payload(const uint8_t* p, size_t n) : p_(p), end_(p + n) {}
  bool at_end() const { return p_ == end_; }
  size_t left() const { return size_t(end_ - p_); }
  bool Byte(uint8_t* v);
  bool VarInt(uint64_t* v);
  bool SignedVarInt(int64_t* v);  // zigzag: (u >> 1) ^ -(u & 1)
  bool Blob(const uint8_t** data, size_t* size);  // varint length, then the bytes
  // An APInt of `width` bits: one raw byte up to 8 bits, a signed varint up
  // to 64 bits, else a word count and that many signed-varint words (only
  // the low word is kept; *wide is set when higher words are non-zero).
  bool APInt(unsigned width, uint64_t* bits, bool* wide = nullptr);

 private:
  const uint8_t* p_;
  const uint8_t* end_;
};

}  // namespace mi::jam::bytecode
