// MLIR bytecode container reader (see bytecode.h for the format summary).
#include "jam/bytecode.h"

#include <cstring>
#include <map>

namespace mi::jam::bytecode {
namespace {

// Section ids and op-encoding bits of the MLIR bytecode format.
enum SectionId : uint8_t {
  kString = 0,
  kDialect = 1,
  kAttrType = 2,
  kAttrTypeOffset = 3,
  kIR = 4,
  kResource = 5,
  kResourceOffset = 6,
  kDialectVersions = 7,
  kProperties = 8,
  kNumSections = 9,
};
enum OpMask : uint8_t {
  kHasAttrs = 0x01,
  kHasResults = 0x02,
  kHasOperands = 0x04,
  kHasSuccessors = 0x08,
  kHasInlineRegions = 0x10,
  kHasUseListOrders = 0x20,
  kHasProperties = 0x40,
};
// Format versions that change the layout.
constexpr uint64_t kVersionDialectVersioning = 1;
constexpr uint64_t kVersionLazyLoading = 2;
constexpr uint64_t kVersionUseListOrdering = 3;
constexpr uint64_t kVersionElideUnknownArgLoc = 4;
constexpr uint64_t kVersionNativeProperties = 5;
constexpr uint64_t kVersionNewest = 6;
constexpr uint8_t kAlignmentByte = 0xCB;
constexpr int kMaxDepth = 256;

class Cursor {
 public:
  Cursor(const uint8_t* base, const uint8_t* p, const uint8_t* end, std::string* err)
      : base_(base), p_(p), end_(end), err_(err) {}

  size_t offset() const { return size_t(p_ - base_); }
  size_t left() const { return size_t(end_ - p_); }
  bool at_end() const { return p_ == end_; }

  bool Fail(const std::string& what) {
    if (err_->empty()) *err_ = what + " at byte " + std::to_string(offset());
    return false;
  }
  bool Byte(uint8_t* v) {
    if (p_ == end_) return Fail("unexpected end of data reading a byte");
    *v = *p_++;
    return true;
  }
  bool Bytes(size_t n, const uint8_t** out) {
    if (left() < n) return Fail("unexpected end of data reading " + std::to_string(n) + " bytes");
    *out = p_;
    p_ += n;
    return true;
  }
  // Prefix varint: trailing zero bits of the first byte + 1 = byte count;
  // value = little-endian bytes >> byte count; first byte 0 -> 8 raw bytes.
  bool VarInt(uint64_t* v) {
    uint8_t first = 0;
    if (!Byte(&first)) return false;
    if (first & 1) {
      *v = first >> 1;
      return true;
    }
    if (first == 0) {
      const uint8_t* b;
      if (!Bytes(8, &b)) return false;
      uint64_t x = 0;
      for (int i = 7; i >= 0; --i) x = (x << 8) | b[i];
      *v = x;
      return true;
    }
    const int n = __builtin_ctz(first) + 1;  // 2 .. 8 bytes in all
    const uint8_t* b;
    if (!Bytes(size_t(n - 1), &b)) return false;
    uint64_t x = first;
    for (int i = 0; i < n - 1; ++i) x |= uint64_t(b[i]) << (8 * (i + 1));
    *v = x >> n;
    return true;
  }
  bool VarIntFlag(uint64_t* v, bool* flag) {
    uint64_t x;
    if (!VarInt(&x)) return false;
    *flag = x & 1;
    *v = x >> 1;
    return true;
  }
  // A count of items that each take at least one byte.
  bool Count(uint64_t* n, const char* what) {
    if (!VarInt(n)) return false;
    if (*n > left()) return Fail(std::string("implausible ") + what + " count " + std::to_string(*n));
    return true;
  }
  bool CString(std::string* s) {
    const uint8_t* q = static_cast<const uint8_t*>(memchr(p_, 0, left()));
    if (!q) return Fail("unterminated string");
    s->assign(reinterpret_cast<const char*>(p_), size_t(q - p_));
    p_ = q + 1;
    return true;
  }
  // A section header and body: {id | aligned << 7, length, [alignment,
  // padding]}; *body covers the data.
  bool Section(uint8_t* id, Cursor* body) {
    uint8_t code = 0;
    uint64_t len;
    if (!Byte(&code) || !VarInt(&len)) return false;
    *id = code & 0x7F;
    if (code & 0x80) {
      uint64_t align;
      if (!VarInt(&align)) return false;
      if (align == 0 || (align & (align - 1)) != 0 || align > 4096)
        return Fail("section alignment " + std::to_string(align) + " is not a power of two <= 4096");
      while (offset() % align != 0) {
        uint8_t pad = 0;
        if (!Byte(&pad)) return false;
        if (pad != kAlignmentByte) return Fail("section padding byte is not 0xCB");
      }
    }
    const uint8_t* d;
    if (!Bytes(size_t(len), &d)) return false;
    *body = Cursor(base_, d, d + len, err_);
    return true;
  }

 private:
  const uint8_t* base_;
  const uint8_t* p_;
  const uint8_t* end_;
  std::string* err_;
};

class Reader {
 public:
  Reader(Module* m, std::string* err) : m_(m), err_(err) {}

  bool Run(const uint8_t* data, size_t size) {
    Cursor c(data, data, data + size, err_);
    const uint8_t* magic;
    if (!c.Bytes(4, &magic) || memcmp(magic, "ML\xEFR", 4) != 0) return c.Fail("not MLIR bytecode (bad magic)");
    if (!c.VarInt(&m_->version)) return false;
    if (m_->version > kVersionNewest)
      return c.Fail("bytecode version " + std::to_string(m_->version) + " is newer than this reader (<= " +
                    std::to_string(kVersionNewest) + ")");
    if (!c.CString(&m_->producer)) return false;
    std::vector<bool> seen(kNumSections, false);
    std::vector<Cursor> sec(kNumSections, Cursor(data, data, data, err_));
    while (!c.at_end()) {
      uint8_t id;
      Cursor body(data, data, data, err_);
      if (!c.Section(&id, &body)) return false;
      if (id >= kNumSections || id == kDialectVersions)
        return c.Fail("unexpected top-level section id " + std::to_string(id));
      if (seen[id]) return c.Fail("duplicate section id " + std::to_string(id));
      seen[id] = true;
      sec[id] = body;
    }
    for (uint8_t id : {kString, kDialect, kAttrType, kAttrTypeOffset, kIR})
      if (!seen[id]) return c.Fail("missing section id " + std::to_string(id));
    if (!Strings(sec[kString]) || !Dialects(sec[kDialect]) || !AttrTypes(sec[kAttrTypeOffset], sec[kAttrType]))
      return false;
    if (seen[kProperties] && !Properties(sec[kProperties])) return false;
    return Ir(sec[kIR]);
  }

 private:
  bool String(Cursor& c, uint64_t i, std::string* out) {
    if (i >= m_->strings.size()) return c.Fail("string index " + std::to_string(i) + " out of range");
    *out = m_->strings[i];
    return true;
  }

  bool Strings(Cursor c) {
    uint64_t n;
    if (!c.Count(&n, "string")) return false;
    std::vector<uint64_t> len(n);
    for (uint64_t i = 0; i < n; ++i)  // lengths come in reverse order
      if (!c.VarInt(&len[n - 1 - i])) return false;
    m_->strings.resize(n);
    for (uint64_t i = 0; i < n; ++i) {
      const uint8_t* b;
      if (len[i] == 0) return c.Fail("string length 0 (lengths include the NUL)");
      if (!c.Bytes(size_t(len[i]), &b)) return false;
      if (b[len[i] - 1] != 0) return c.Fail("string " + std::to_string(i) + " is not NUL-terminated");
      m_->strings[i].assign(reinterpret_cast<const char*>(b), size_t(len[i] - 1));
    }
    return c.at_end() || c.Fail("trailing bytes in the string section");
  }

  bool Dialects(Cursor c) {
    uint64_t n;
    if (!c.Count(&n, "dialect")) return false;
    m_->dialects.resize(n);
    m_->dialect_versions.resize(n);
    for (uint64_t i = 0; i < n; ++i) {
      uint64_t name;
      bool versioned = false;
      if (m_->version < kVersionDialectVersioning) {
        if (!c.VarInt(&name)) return false;
      } else if (!c.VarIntFlag(&name, &versioned)) {
        return false;
      }
      if (!String(c, name, &m_->dialects[i])) return false;
      if (versioned) {
        uint8_t id;
        Cursor body(nullptr, nullptr, nullptr, err_);
        if (!c.Section(&id, &body)) return false;
        if (id != kDialectVersions) return c.Fail("dialect version payload has section id " + std::to_string(id));
        const size_t nbytes = body.left();
        const uint8_t* b;
        if (!body.Bytes(nbytes, &b)) return false;
        m_->dialect_versions[i].assign(b, b + nbytes);
      }
    }
    uint64_t total = 0;
    const bool counted = m_->version >= kVersionElideUnknownArgLoc;
    if (counted && !c.Count(&total, "op name")) return false;
    while (counted ? m_->op_names.size() < total : !c.at_end()) {
      uint64_t d, k;
      if (!c.VarInt(&d) || !c.Count(&k, "op name")) return false;
      if (d >= n) return c.Fail("op name group names dialect " + std::to_string(d) + " of " + std::to_string(n));
      for (uint64_t j = 0; j < k; ++j) {
        OpName on;
        on.dialect = int(d);
        uint64_t s;
        if (m_->version >= kVersionNativeProperties) {
          if (!c.VarIntFlag(&s, &on.registered)) return false;
        } else if (!c.VarInt(&s)) {
          return false;
        }
        if (!String(c, s, &on.name)) return false;
        m_->op_names.push_back(std::move(on));
      }
    }
    return c.at_end() || c.Fail("trailing bytes in the dialect section");
  }
  bool AttrTypes(Cursor c, Cursor data) {
    uint64_t na, nt;
    if (!c.Count(&na, "attribute") || !c.Count(&nt, "type")) return false;
    const uint8_t* raw;
    const size_t data_size = data.left();
    if (!data.Bytes(data_size, &raw)) return false;
    m_->attr_type_data.assign(raw, raw + data_size);
    size_t at = 0;
    auto groups = [&](uint64_t want, std::vector<Entry>& out) {
      while (out.size() < want) {
        uint64_t d, k;
        if (!c.VarInt(&d) || !c.Count(&k, "attribute/type")) return false;
        if (d >= m_->dialects.size()) return c.Fail("attribute/type group names dialect " + std::to_string(d));
        if (out.size() + k > want) return c.Fail("attribute/type group overruns its count");
        for (uint64_t j = 0; j < k; ++j) {
          Entry e;
          e.dialect = int(d);
          uint64_t sz;
          if (!c.VarIntFlag(&sz, &e.custom)) return false;
          if (sz > data_size - at) return c.Fail("attribute/type entry runs past its section");
          e.offset = at;
          e.size = size_t(sz);
          at += size_t(sz);
          out.push_back(e);
        }
      }
      return true;
    };
    if (!groups(na, m_->attrs) || !groups(nt, m_->types)) return false;
    if (at != data_size) return c.Fail("attribute/type entries do not cover their section");
    return c.at_end() || c.Fail("trailing bytes in the attribute/type offset section");
  }

  bool Properties(Cursor c) {
    uint64_t n;
    if (!c.Count(&n, "property")) return false;
    for (uint64_t i = 0; i < n; ++i) {  // each: byte size, then the op-specific encoding
      uint64_t sz;
      const uint8_t* b;
      if (!c.VarInt(&sz) || !c.Bytes(size_t(sz), &b)) return false;
    }
    num_properties_ = n;
    return c.at_end() || c.Fail("trailing bytes in the properties section");
  }

  bool Ir(Cursor c) {
    if (!Block(c, &m_->top, 0)) return false;
    return c.at_end() || c.Fail("trailing bytes in the IR section");
  }

  bool SkipUseLists(Cursor& c, uint64_t range) {
    uint64_t n = 1;
    if (range != 1 && !c.Count(&n, "use-list order")) return false;
    for (uint64_t i = 0; i < n; ++i) {
      uint64_t idx, k;
      bool pairs;
      if (range != 1 && !c.VarInt(&idx)) return false;
      if (!c.VarIntFlag(&k, &pairs)) return false;
      if (k > c.left()) return c.Fail("implausible use-list length");
      for (uint64_t j = 0; j < k; ++j)
        if (!c.VarInt(&idx)) return false;
    }
    return true;
  }

  bool Block(Cursor& c, bytecode::Block* b, int depth) {
    uint64_t nops;
    bool has_args;
    if (!c.VarIntFlag(&nops, &has_args)) return false;
    if (nops > c.left()) return c.Fail("implausible operation count " + std::to_string(nops));
    if (has_args) {
      uint64_t na;
      if (!c.Count(&na, "block argument")) return false;
      b->args.resize(na);
      for (auto& a : b->args) {
        if (m_->version >= kVersionElideUnknownArgLoc) {
          bool has_loc;
          uint64_t loc;
          if (!c.VarIntFlag(&a.type, &has_loc)) return false;
          if (has_loc) {
            if (!c.VarInt(&loc)) return false;
            a.location = int64_t(loc);
          }
        } else {
          uint64_t loc;
          if (!c.VarInt(&a.type) || !c.VarInt(&loc)) return false;
          a.location = int64_t(loc);
        }
        if (a.type >= m_->types.size()) return c.Fail("block argument type index out of range");
      }
      if (m_->version >= kVersionUseListOrdering) {
        uint8_t mask = 0;
        if (!c.Byte(&mask)) return false;
        if (mask & ~kHasUseListOrders) return c.Fail("unknown block-argument encoding bits");
        if ((mask & kHasUseListOrders) && !SkipUseLists(c, na)) return false;
      }
    }
    b->ops.resize(nops);
    for (auto& op : b->ops)
      if (!Op(c, &op, depth)) return false;
    return true;
  }

  bool Region(Cursor& c, bytecode::Region* r, int depth) {
    uint64_t nb;
    if (!c.Count(&nb, "block")) return false;
    if (nb == 0) return true;
    if (!c.VarInt(&r->num_values)) return false;
    r->blocks.resize(nb);
    for (auto& b : r->blocks)
      if (!Block(c, &b, depth)) return false;
    return true;
  }

  bool Op(Cursor& c, bytecode::Op* op, int depth) {
    if (depth > kMaxDepth) return c.Fail("regions nested deeper than " + std::to_string(kMaxDepth));
    if (!c.VarInt(&op->name)) return false;
    if (op->name >= m_->op_names.size()) return c.Fail("operation name index out of range");
    if (!c.Byte(&op->mask) || !c.VarInt(&op->location)) return false;
    if (op->mask & 0x80) return c.Fail("unknown operation encoding bit");
    uint64_t v;
    if (op->mask & kHasAttrs) {
      if (!c.VarInt(&v)) return false;
      if (v >= m_->attrs.size()) return c.Fail("attribute dictionary index out of range");
      op->attr_dict = int64_t(v);
    }
    if (op->mask & kHasProperties) {
      if (m_->version < kVersionNativeProperties) return c.Fail("properties in a version < 5 stream");
      if (!c.VarInt(&v)) return false;
      if (v >= num_properties_) return c.Fail("properties index out of range");
      op->properties = int64_t(v);
    }
    auto list = [&](std::vector<uint64_t>& out, const char* what) {
      uint64_t n;
      if (!c.Count(&n, what)) return false;
      out.resize(n);
      for (auto& x : out)
        if (!c.VarInt(&x)) return false;
      return true;
    };
    if ((op->mask & kHasResults) && !list(op->result_types, "result")) return false;
    for (uint64_t t : op->result_types)
      if (t >= m_->types.size()) return c.Fail("result type index out of range");
    if ((op->mask & kHasOperands) && !list(op->operands, "operand")) return false;
    if ((op->mask & kHasSuccessors) && !list(op->successors, "successor")) return false;
    if (op->mask & kHasUseListOrders) {
      if (m_->version < kVersionUseListOrdering) return c.Fail("use-list orders in a version < 3 stream");
      if (!SkipUseLists(c, op->result_types.size())) return false;
    }
    if (op->mask & kHasInlineRegions) {
      uint64_t nr;
      if (!c.VarIntFlag(&nr, &op->isolated)) return false;
      if (nr > c.left()) return c.Fail("implausible region count");
      op->regions.resize(nr);
      if (op->isolated && m_->version >= kVersionLazyLoading) {
        uint8_t id;
        Cursor body(nullptr, nullptr, nullptr, err_);
        if (!c.Section(&id, &body)) return false;
        if (id != kIR) return c.Fail("isolated regions are not in an IR section");
        for (auto& r : op->regions)
          if (!Region(body, &r, depth + 1)) return false;
        if (!body.at_end()) return body.Fail("trailing bytes after isolated regions");
      } else {
        for (auto& r : op->regions)
          if (!Region(c, &r, depth + 1)) return false;
      }
    }
    return true;
  }

  Module* m_;
  std::string* err_;
  uint64_t num_properties_ = 0;
};

void Walk(const Block& b, const Module& m, std::vector<std::pair<std::string, int>>& hist,
          std::map<std::string, size_t>& where) {
  for (const Op& op : b.ops) {
    const std::string n = m.OpFullName(op.name);
    auto it = where.find(n);
    if (it == where.end()) {
      where[n] = hist.size();
      hist.emplace_back(n, 1);
    } else {
      ++hist[it->second].second;
    }
    for (const Region& r : op.regions)
      for (const Block& blk : r.blocks) Walk(blk, m, hist, where);
  }
}

}  // namespace

std::string Module::OpFullName(uint64_t i) const {
  if (i >= op_names.size()) return "?";
  const OpName& o = op_names[i];
  const std::string& d = size_t(o.dialect) < dialects.size() ? dialects[size_t(o.dialect)] : std::string("?");
  return d + "." + o.name;
}

std::string Module::EntryText(const Entry& e) const {
  if (e.custom || e.size == 0 || e.offset + e.size > attr_type_data.size()) return "";
  const char* p = reinterpret_cast<const char*>(attr_type_data.data() + e.offset);
  return std::string(p, strnlen(p, e.size));
}

std::string Module::OpHistogram() const {
  std::vector<std::pair<std::string, int>> hist;
  std::map<std::string, size_t> where;
  Walk(top, *this, hist, where);
  std::string s;
  for (const auto& [n, k] : hist) s += (s.empty() ? "" : ", ") + n + " x" + std::to_string(k);
  return s;
}

std::string Module::DialectVersionText(size_t d) const {
  if (d >= dialects.size()) return "";
  std::string s = dialects[d];
  const auto& v = dialect_versions[d];
  if (v.empty()) return s;
  std::string err;
  Cursor c(v.data(), v.data(), v.data() + v.size(), &err);
  std::string nums;
  while (!c.at_end()) {
    uint64_t x;
    if (!c.VarInt(&x)) return s + " (unparsed version)";
    nums += (nums.empty() ? "" : ".") + std::to_string(x);
  }
  return s + " " + nums;
}

bool Payload::Byte(uint8_t* v) {
  if (p_ == end_) return false;
  *v = *p_++;
  return true;
}

bool Payload::VarInt(uint64_t* v) {
  uint8_t first = 0;
  if (!Byte(&first)) return false;
  if (first & 1) {
    *v = first >> 1;
    return true;
  }
  if (first == 0) {
    if (left() < 8) return false;
    uint64_t x = 0;
    for (int i = 7; i >= 0; --i) x = (x << 8) | p_[i];
    p_ += 8;
    *v = x;
    return true;
  }
  const int n = __builtin_ctz(first) + 1;
  if (left() < size_t(n - 1)) return false;
  uint64_t x = first;
  for (int i = 0; i < n - 1; ++i) x |= uint64_t(p_[i]) << (8 * (i + 1));
  p_ += n - 1;
  *v = x >> n;
  return true;
}

bool Payload::SignedVarInt(int64_t* v) {
  uint64_t u;
  if (!VarInt(&u)) return false;
  *v = int64_t((u >> 1) ^ (~(u & 1) + 1));
  return true;
}

bool Payload::Blob(const uint8_t** data, size_t* size) {
  uint64_t n;
  if (!VarInt(&n) || n > left()) return false;
  *data = p_;
  *size = size_t(n);
  p_ += n;
  return true;
}

bool Payload::APInt(unsigned width, uint64_t* bits, bool* wide) {
  if (wide) *wide = false;
  if (width <= 8) {
    uint8_t b;
    if (!Byte(&b)) return false;
    *bits = b;
    return true;
  }
  if (width <= 64) {
    int64_t x;
    if (!SignedVarInt(&x)) return false;
    *bits = uint64_t(x);
    return true;
  }
  uint64_t words;
  if (!VarInt(&words) || words > left()) return false;
  *bits = 0;
  for (uint64_t w = 0; w < words; ++w) {
    int64_t x;
    if (!SignedVarInt(&x)) return false;
    if (w == 0) *bits = uint64_t(x);
    else if (x != 0 && wide) *wide = true;
  }
  return true;
}

bool Read(const uint8_t* data, size_t size, Module* out, std::string* error) {
  error->clear();
  *out = Module();
  Reader r(out, error);
  if (r.Run(data, size)) return true;
  if (error->empty()) *error = "malformed MLIR bytecode";
  return false;
}

}  // namespace mi::jam::bytecode
