// .animapk (ANMA v1) pack reader: AnimapkFile (AnimaXS/Runtime/Animapk/AnimapkFile.swift:
// 15-185), AnimapkHeader.parse (AnimapkHeader.swift:25-68), the tensor_meta JSON
// (AnimapkTensor.swift:90-173), CRC-32 (Crc32.swift:6-29), AnimapkRangeBuilder and the
// DiT locators (AnimapkRangeLocator.swift:38-261) and DiTQuantizedWeightFactory.makeMatrix
// (LinearExecutor.swift:467-518).  Host-only C++: the file is mapped read-only with mmap
// and never copied; weight templates hold offsets into an execution range so that the
// range can be copied to the device (or streamed through a WeightStreamer slot) as one
// contiguous block.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <set>
#include <string>
#include <unordered_map>
#include <vector>

#include "anima_hip.h"
#include "pack.hpp"
#include "status.hpp"

namespace anima {
namespace {

// ---------------------------------------------------------------------------
// A small JSON reader: objects, arrays, strings (with escapes and \u code points),
// numbers (integers kept exact in 64 bits), true / false / null.
// ---------------------------------------------------------------------------
struct JValue {
  enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
  bool b = false;
  bool is_int = false;   // an integer literal (no fraction or exponent)
  bool negative = false;
  uint64_t u = 0;        // magnitude of an integer literal
  double d = 0.0;
  std::string s;
  std::vector<JValue> a;
  std::vector<std::pair<std::string, JValue>> o;

  const JValue* get(const char* key) const {
    const JValue* found = nullptr;
    for (const auto& kv : o)
      if (kv.first == key) found = &kv.second;  // the last duplicate wins
    return found;
  }
};

class JsonParser {
 public:
  JsonParser(const char* p, size_t n) : p_(p), end_(p + n) {}
  JValue parse() {
    JValue v = value(0);
    ws();
    if (p_ != end_) err("trailing characters after the top-level value");
    return v;
  }

 private:
  const char* p_;
  const char* end_;

  [[noreturn]] void err(const std::string& what) { fail(ANIMA_E_FORMAT, "failed to decode architecture JSON: " + what); }
  void ws() {
    while (p_ != end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
  }
  bool lit(const char* w) {
    const size_t n = std::strlen(w);
    if ((size_t)(end_ - p_) >= n && std::memcmp(p_, w, n) == 0) {
      p_ += n;
      return true;
    }
    return false;
  }
  JValue value(int depth) {
    if (depth > 64) err("nesting too deep");
    ws();
    if (p_ == end_) err("unexpected end of input");
    JValue v;
    const char c = *p_;
    if (c == '{') {
      v.kind = JValue::OBJ;
      ++p_;
      ws();
      if (p_ != end_ && *p_ == '}') {
        ++p_;
        return v;
      }
      for (;;) {
        ws();
        if (p_ == end_ || *p_ != '"') err("expected an object key");
        std::string k = str();
        ws();
        if (p_ == end_ || *p_ != ':') err("expected ':'");
        ++p_;
        v.o.emplace_back(std::move(k), value(depth + 1));
        ws();
        if (p_ != end_ && *p_ == ',') {
          ++p_;
          continue;
        }
        if (p_ != end_ && *p_ == '}') {
          ++p_;
          return v;
        }
        err("expected ',' or '}'");
      }
    }
    if (c == '[') {
      v.kind = JValue::ARR;
      ++p_;
      ws();
      if (p_ != end_ && *p_ == ']') {
        ++p_;
        return v;
      }
      for (;;) {
        v.a.push_back(value(depth + 1));
        ws();
        if (p_ != end_ && *p_ == ',') {
          ++p_;
          continue;
        }
        if (p_ != end_ && *p_ == ']') {
          ++p_;
          return v;
        }
        err("expected ',' or ']'");
      }
    }
    if (c == '"') {
      v.kind = JValue::STR;
      v.s = str();
      return v;
    }
    if (lit("true")) {
      v.kind = JValue::BOOL;
      v.b = true;
      return v;
    }
    if (lit("false")) {
      v.kind = JValue::BOOL;
      return v;
    }
    if (lit("null")) return v;
    if (c == '-' || (c >= '0' && c <= '9')) return number();
    err(std::string("unexpected character '") + c + "'");
  }
  static void utf8(std::string& out, uint32_t cp) {
    if (cp < 0x80) {
      out += (char)cp;
    } else if (cp < 0x800) {
      out += (char)(0xC0 | (cp >> 6));
      out += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      out += (char)(0xE0 | (cp >> 12));
      out += (char)(0x80 | ((cp >> 6) & 0x3F));
      out += (char)(0x80 | (cp & 0x3F));
    } else {
      out += (char)(0xF0 | (cp >> 18));
      out += (char)(0x80 | ((cp >> 12) & 0x3F));
      out += (char)(0x80 | ((cp >> 6) & 0x3F));
      out += (char)(0x80 | (cp & 0x3F));
    }
  }
  uint32_t hex4() {
    if (end_ - p_ < 4) err("truncated \\u escape");
    uint32_t v = 0;
    for (int i = 0; i < 4; ++i) {
      const char h = *p_++;
      v <<= 4;
      if (h >= '0' && h <= '9') v |= (uint32_t)(h - '0');
      else if (h >= 'a' && h <= 'f') v |= (uint32_t)(h - 'a' + 10);
      else if (h >= 'A' && h <= 'F') v |= (uint32_t)(h - 'A' + 10);
      else err("bad \\u escape");
    }
    return v;
  }
  std::string str() {
    ++p_;  // opening quote
    std::string out;
    for (;;) {
      if (p_ == end_) err("unterminated string");
      const char c = *p_++;
      if (c == '"') return out;
      if ((unsigned char)c < 0x20) err("control character in a string");
      if (c != '\\') {
        out += c;
        continue;
      }
      if (p_ == end_) err("unterminated escape");
      const char e = *p_++;
      switch (e) {
        case '"': out += '"'; break;
        case '\\': out += '\\'; break;
        case '/': out += '/'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          uint32_t cp = hex4();
          if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
            if (end_ - p_ < 6 || p_[0] != '\\' || p_[1] != 'u') err("unpaired surrogate");
            p_ += 2;
            const uint32_t lo = hex4();
            if (lo < 0xDC00 || lo >= 0xE000) err("unpaired surrogate");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          utf8(out, cp);
          break;
        }
        default: err("bad escape");
      }
    }
  }
  JValue number() {
    JValue v;
    v.kind = JValue::NUM;
    const char* start = p_;
    if (*p_ == '-') {
      v.negative = true;
      ++p_;
    }
    if (p_ == end_ || !(*p_ >= '0' && *p_ <= '9')) err("bad number");
    bool overflow = false;
    uint64_t mag = 0;
    while (p_ != end_ && *p_ >= '0' && *p_ <= '9') {
      const uint64_t dgt = (uint64_t)(*p_ - '0');
      if (mag > (UINT64_MAX - dgt) / 10) overflow = true;
      mag = mag * 10 + dgt;
      ++p_;
    }
    bool frac = false;
    if (p_ != end_ && *p_ == '.') {
      frac = true;
      ++p_;
      if (p_ == end_ || !(*p_ >= '0' && *p_ <= '9')) err("bad number");
      while (p_ != end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    if (p_ != end_ && (*p_ == 'e' || *p_ == 'E')) {
      frac = true;
      ++p_;
      if (p_ != end_ && (*p_ == '+' || *p_ == '-')) ++p_;
      if (p_ == end_ || !(*p_ >= '0' && *p_ <= '9')) err("bad number");
      while (p_ != end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    v.is_int = !frac && !overflow;
    v.u = mag;
    v.d = std::strtod(std::string(start, p_).c_str(), nullptr);
    return v;
  }
};

// ---------------------------------------------------------------------------
// CRC-32 of zlib (ISO-HDLC): reflected polynomial 0xEDB88320, initial value and
// final XOR 0xFFFFFFFF, one table lookup per byte.
// ---------------------------------------------------------------------------
struct CrcTable {
  uint32_t t[256];
  CrcTable() {
    for (uint32_t i = 0; i < 256; ++i) {
      uint32_t c = i;
      for (int k = 0; k < 8; ++k) c = (c & 1u) ? (0xEDB88320u ^ (c >> 1)) : (c >> 1);
      t[i] = c;
    }
  }
};

uint32_t crc32(const uint8_t* p, size_t n) {
  static const CrcTable table;
  uint32_t c = 0xFFFFFFFFu;
  for (size_t i = 0; i < n; ++i) c = table.t[(c ^ p[i]) & 0xFFu] ^ (c >> 8);
  return c ^ 0xFFFFFFFFu;
}

constexpr uint64_t kAlign = 16384;

uint64_t add_checked(uint64_t a, uint64_t b, const std::string& label) {
  uint64_t r;
  if (__builtin_add_overflow(a, b, &r)) fail(ANIMA_E_FORMAT, "byte offset overflow for " + label);
  return r;
}

uint64_t mul_checked(uint64_t a, uint64_t b, const std::string& label) {
  uint64_t r;
  if (__builtin_mul_overflow(a, b, &r)) fail(ANIMA_E_FORMAT, "byte length overflow for " + label);
  return r;
}

}  // namespace

// One tensor_meta entry, with the optional fields as the reference decodes them.
struct PackTensor {
  std::string name, logical_dtype, storage_dtype, qformat;
  bool has_qformat = false;
  std::vector<int64_t> shape;
  int storage = ANIMA_STORAGE_FP32;
  bool has_crc = false;
  uint32_t crc = 0;
  int64_t block_index = -1;
  uint64_t blob_offset = 0, blob_size = 0, data_offset = 0, data_size = 0;
  bool has_scale_offset = false, has_scale_size = false, has_zero_offset = false, has_zero_size = false;
  uint64_t scale_offset = 0, scale_size = 0, zero_offset = 0, zero_size = 0;
};

// A span relative to an execution range.
struct Span {
  uint64_t offset = 0, length = 0;
  bool present = false;
};

struct TensorSpans {
  const PackTensor* tensor;
  Span blob, data, scale, zero;
};

struct ExecRange {
  int64_t logical_index = 0;
  uint64_t file_offset = 0, length = 0;
  std::vector<TensorSpans> tensors;
};

}  // namespace anima

using namespace anima;

struct anima_pack {
  int fd = -1;
  const uint8_t* map = nullptr;
  size_t size = 0;
  anima_pack_info info{};
  std::string component_name, quant_scheme;
  bool has_scheme = false;
  std::vector<PackTensor> tensors;
  std::unordered_map<std::string, size_t> by_name;

  ~anima_pack() {
    if (map) munmap(const_cast<uint8_t*>(map), size);
    if (fd >= 0) close(fd);
  }
};

namespace anima {
namespace {

uint16_t le16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
uint32_t le32(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }
uint64_t le64(const uint8_t* p) {
  uint64_t v = 0;
  for (int i = 0; i < 8; ++i) v |= (uint64_t)p[i] << (8 * i);
  return v;
}

// --- JSON field access (Codable semantics: a missing required key or a wrong type is an error)
[[noreturn]] void json_err(const std::string& what) { fail(ANIMA_E_FORMAT, "failed to decode architecture JSON: " + what); }

uint64_t json_u64(const JValue& v, const std::string& key) {
  if (v.kind != JValue::NUM || !v.is_int || v.negative) json_err(key + " is not an unsigned integer");
  return v.u;
}

int64_t json_i64(const JValue& v, const std::string& key) {
  if (v.kind != JValue::NUM || !v.is_int || v.u > (uint64_t)INT64_MAX) json_err(key + " is not an integer");
  return v.negative ? -(int64_t)v.u : (int64_t)v.u;
}

const JValue& need(const JValue& obj, const char* key, const std::string& where) {
  const JValue* v = obj.get(key);
  if (!v) json_err("missing key '" + std::string(key) + "' in " + where);
  return *v;
}

// Optional key: absent or null both decode to "absent".
const JValue* opt(const JValue& obj, const char* key) {
  const JValue* v = obj.get(key);
  return (v && v->kind != JValue::NUL) ? v : nullptr;
}

std::string need_str(const JValue& obj, const char* key, const std::string& where) {
  const JValue& v = need(obj, key, where);
  if (v.kind != JValue::STR) json_err(std::string(key) + " in " + where + " is not a string");
  return v.s;
}

int storage_code(const std::string& s) {
  if (s == "w4") return ANIMA_STORAGE_W4;
  if (s == "w8") return ANIMA_STORAGE_W8;
  if (s == "fp16") return ANIMA_STORAGE_FP16;
  return ANIMA_STORAGE_FP32;  // "fp32" and unknown values (AnimapkTensor.storage falls back to fp32)
}

PackTensor decode_tensor(const JValue& t, size_t index) {
  const std::string where = "tensor_meta[" + std::to_string(index) + "]";
  if (t.kind != JValue::OBJ) json_err(where + " is not an object");
  PackTensor r;
  r.name = need_str(t, "name", where);
  const JValue& shape = need(t, "shape", where);
  if (shape.kind != JValue::ARR) json_err("shape of " + r.name + " is not an array");
  // anima_pack_tensor carries at most 8 dimensions; a longer shape is refused here rather
  // than cut off where it is handed out.
  if (shape.a.size() > 8) json_err("shape of " + r.name + " has more than 8 dimensions");
  for (const JValue& d : shape.a) r.shape.push_back(json_i64(d, "shape of " + r.name));
  r.logical_dtype = need_str(t, "logical_dtype", where);
  r.storage_dtype = need_str(t, "storage_dtype", where);
  r.storage = storage_code(r.storage_dtype);
  if (const JValue* v = opt(t, "crc32")) {
    const uint64_t c = json_u64(*v, "crc32");
    if (c > 0xFFFFFFFFull) json_err("crc32 of " + r.name + " exceeds 32 bits");
    r.has_crc = true;
    r.crc = (uint32_t)c;
  }
  if (const JValue* v = opt(t, "block_index")) r.block_index = json_i64(*v, "block_index");
  if (const JValue* v = opt(t, "execution_index")) (void)json_i64(*v, "execution_index");
  r.blob_offset = json_u64(need(t, "blob_offset", where), "blob_offset");
  r.blob_size = json_u64(need(t, "blob_size", where), "blob_size");
  if (const JValue* v = opt(t, "data_offset")) r.data_offset = json_u64(*v, "data_offset");
  r.data_size = json_u64(need(t, "data_size", where), "data_size");
  if (const JValue* v = opt(t, "scale_offset")) { r.has_scale_offset = true; r.scale_offset = json_u64(*v, "scale_offset"); }
  if (const JValue* v = opt(t, "scale_size")) { r.has_scale_size = true; r.scale_size = json_u64(*v, "scale_size"); }
  if (const JValue* v = opt(t, "zero_offset")) { r.has_zero_offset = true; r.zero_offset = json_u64(*v, "zero_offset"); }
  if (const JValue* v = opt(t, "zero_size")) { r.has_zero_size = true; r.zero_size = json_u64(*v, "zero_size"); }
  if (const JValue* v = opt(t, "quantization_format")) {
    if (v->kind != JValue::STR) json_err("quantization_format of " + r.name + " is not a string");
    r.has_qformat = true;
    r.qformat = v->s;
  }
  if (const JValue* v = opt(t, "blob_sha256"))
    if (v->kind != JValue::STR) json_err("blob_sha256 of " + r.name + " is not a string");
  return r;
}

// AnimapkFile.validateTensor (AnimapkFile.swift:91-107), with every end checked for
// overflow.
void validate_tensor(const PackTensor& t, uint64_t file_bytes) {
  uint64_t end;
  if (__builtin_add_overflow(t.blob_offset, t.blob_size, &end) || end > file_bytes)
    fail(ANIMA_E_FORMAT, "blob " + t.name + " out of file bounds");
  if (t.blob_offset % kAlign != 0)
    fail(ANIMA_E_FORMAT, "blob " + t.name + " offset " + std::to_string(t.blob_offset) + " not 16 KB aligned");
  if (__builtin_add_overflow(t.data_offset, t.data_size, &end) || end > t.blob_size)
    fail(ANIMA_E_FORMAT, "blob " + t.name + " data region out of blob bounds");
  if (t.has_scale_offset && t.has_scale_size &&
      (__builtin_add_overflow(t.scale_offset, t.scale_size, &end) || end > t.blob_size))
    fail(ANIMA_E_FORMAT, "blob " + t.name + " scale region out of blob bounds");
  if (t.has_zero_offset && t.has_zero_size &&
      (__builtin_add_overflow(t.zero_offset, t.zero_size, &end) || end > t.blob_size))
    fail(ANIMA_E_FORMAT, "blob " + t.name + " zero region out of blob bounds");
}

void load(anima_pack& pk, const char* path) {
  pk.fd = open(path, O_RDONLY | O_CLOEXEC);
  if (pk.fd < 0) fail(ANIMA_E_IO, std::string("cannot open ") + path + ": " + std::strerror(errno));
  struct stat st;
  if (fstat(pk.fd, &st) != 0) fail(ANIMA_E_IO, std::string("cannot stat ") + path + ": " + std::strerror(errno));
  const uint64_t bytes = (uint64_t)st.st_size;
  // AnimapkHeader.parse (AnimapkHeader.swift:25-68)
  if (bytes < 256)
    fail(ANIMA_E_FORMAT, "file smaller than 256-byte header (" + std::to_string(bytes) + " bytes)");
  void* m = mmap(nullptr, (size_t)bytes, PROT_READ, MAP_PRIVATE, pk.fd, 0);
  if (m == MAP_FAILED) fail(ANIMA_E_IO, std::string("cannot map ") + path + ": " + std::strerror(errno));
  pk.map = static_cast<const uint8_t*>(m);
  pk.size = (size_t)bytes;
  const uint8_t* h = pk.map;
  if (!(h[0] == 0x41 && h[1] == 0x4E && h[2] == 0x4D && h[3] == 0x41))
    fail(ANIMA_E_FORMAT, "bad magic (expected 'ANMA')");
  anima_pack_info& info = pk.info;
  info.version = le16(h + 0x04);
  info.component = le16(h + 0x06);
  info.alignment = le32(h + 0x08);
  const uint64_t tensor_count = le64(h + 0x0C), json_offset = le64(h + 0x14), json_size = le64(h + 0x1C),
                 table_offset = le64(h + 0x24), table_bytes = le64(h + 0x2C), payload_offset = le64(h + 0x34),
                 file_size = le64(h + 0x3C);
  info.record_size = (int32_t)le32(h + 0x44);
  if (info.version != 1)
    fail(ANIMA_E_FORMAT, "unsupported ANMA version " + std::to_string(info.version) + " (expected 1)");
  if (info.alignment != (int64_t)kAlign)
    fail(ANIMA_E_FORMAT, "unexpected alignment " + std::to_string(info.alignment) + " (expected 16384)");
  if (le32(h + 0x44) != 128)
    fail(ANIMA_E_FORMAT, "unexpected record size " + std::to_string(le32(h + 0x44)) + " (expected 128)");
  // AnimapkFile.validateHeader (AnimapkFile.swift:72-89)
  if (file_size != bytes)
    fail(ANIMA_E_FORMAT, "declared file size " + std::to_string(file_size) + " != actual " + std::to_string(bytes));
  uint64_t end;
  if (__builtin_add_overflow(json_offset, json_size, &end) || end > file_size)
    fail(ANIMA_E_FORMAT, "JSON section out of file bounds");
  if (__builtin_add_overflow(table_offset, table_bytes, &end) || end > file_size)
    fail(ANIMA_E_FORMAT, "table section out of file bounds");
  if (payload_offset > file_size) fail(ANIMA_E_FORMAT, "payload offset out of file bounds");
  if (tensor_count > (uint64_t)INT64_MAX || file_size > (uint64_t)INT64_MAX)
    fail(ANIMA_E_FORMAT, "header count or size exceeds int64");
  info.tensor_count = (int64_t)tensor_count;
  info.json_offset = (int64_t)json_offset;
  info.json_size = (int64_t)json_size;
  info.table_offset = (int64_t)table_offset;
  info.table_bytes = (int64_t)table_bytes;
  info.payload_offset = (int64_t)payload_offset;
  info.file_size = (int64_t)file_size;

  // Architecture JSON (authoritative names, shapes and offsets)
  JsonParser parser(reinterpret_cast<const char*>(pk.map + json_offset), (size_t)json_size);
  const JValue env = parser.parse();
  if (env.kind != JValue::OBJ) json_err("the envelope is not an object");
  pk.component_name = need_str(env, "component", "the envelope");
  info.quant_group = -1;
  if (const JValue* q = opt(env, "quant")) {
    if (q->kind != JValue::OBJ) json_err("quant is not an object");
    if (const JValue* s = opt(*q, "scheme")) {
      if (s->kind != JValue::STR) json_err("quant.scheme is not a string");
      pk.has_scheme = true;
      pk.quant_scheme = s->s;
    }
    if (const JValue* g = opt(*q, "group")) {
      const int64_t gv = json_i64(*g, "quant.group");
      info.quant_group = (gv >= INT32_MIN && gv <= INT32_MAX) ? (int32_t)gv : -1;
    }
  }
  if (const JValue* sh = opt(env, "source_hashes"))
    if (sh->kind != JValue::OBJ) json_err("source_hashes is not an object");
  const JValue& meta = need(env, "tensor_meta", "the envelope");
  if (meta.kind != JValue::ARR) json_err("tensor_meta is not an array");
  pk.tensors.reserve(meta.a.size());
  for (size_t i = 0; i < meta.a.size(); ++i) pk.tensors.push_back(decode_tensor(meta.a[i], i));
  for (size_t i = 0; i < pk.tensors.size(); ++i) pk.by_name[pk.tensors[i].name] = i;
  info.component_name = pk.component_name.c_str();
  info.quant_scheme = pk.has_scheme ? pk.quant_scheme.c_str() : nullptr;
  if (pk.tensors.size() != tensor_count)
    fail(ANIMA_E_FORMAT, "JSON tensor_meta count " + std::to_string(pk.tensors.size()) + " != header tensor_count " +
                             std::to_string(tensor_count));
  for (const PackTensor& t : pk.tensors) validate_tensor(t, file_size);

  // AnimapkFile.validateTableCrossMatch (AnimapkFile.swift:110-135): the set of the binary
  // table's blob offsets (u64 at record byte 96) equals the JSON's.
  if (table_bytes % 128 != 0) fail(ANIMA_E_FORMAT, "table bytes not a multiple of record size");
  const uint64_t records = table_bytes / 128;
  if (records != tensor_count)
    fail(ANIMA_E_FORMAT, "table record count " + std::to_string(records) + " != tensor_count " +
                             std::to_string(tensor_count));
  std::set<uint64_t> table_offsets, json_offsets;
  for (uint64_t r = 0; r < records; ++r) table_offsets.insert(le64(pk.map + table_offset + r * 128 + 96));
  for (const PackTensor& t : pk.tensors) json_offsets.insert(t.blob_offset);
  if (table_offsets.size() != json_offsets.size())
    fail(ANIMA_E_FORMAT, "table blob_offsets (" + std::to_string(table_offsets.size()) + ") != JSON blob_offsets (" +
                             std::to_string(json_offsets.size()) + ")");
  for (uint64_t off : table_offsets)
    if (!json_offsets.count(off))
      fail(ANIMA_E_FORMAT, "table blob_offset " + std::to_string(off) + " missing from JSON tensor_meta");
}

void to_c(const PackTensor& t, anima_pack_tensor& o) {
  std::memset(&o, 0, sizeof o);
  o.name = t.name.c_str();
  o.storage = t.storage;
  o.rank = (int32_t)t.shape.size();  // <= 8, checked when the JSON is decoded
  for (int i = 0; i < o.rank; ++i) o.shape[i] = t.shape[i];
  o.blob_offset = (int64_t)t.blob_offset;
  o.blob_size = (int64_t)t.blob_size;
  o.data_offset = (int64_t)t.data_offset;
  o.data_size = (int64_t)t.data_size;
  const bool scale = t.has_scale_offset && t.has_scale_size, zero = t.has_zero_offset && t.has_zero_size;
  o.scale_offset = scale ? (int64_t)t.scale_offset : -1;
  o.scale_size = scale ? (int64_t)t.scale_size : -1;
  o.zero_offset = zero ? (int64_t)t.zero_offset : -1;
  o.zero_size = zero ? (int64_t)t.zero_size : -1;
  o.block_index = t.block_index;
  o.crc32 = t.crc;
  o.has_crc32 = t.has_crc ? 1 : 0;
  o.logical_dtype = t.logical_dtype.c_str();
  o.quantization_format = t.has_qformat ? t.qformat.c_str() : nullptr;
}

// --- AnimapkRangeBuilder (AnimapkRangeLocator.swift:38-154)
Span relative(uint64_t abs_off, uint64_t len, uint64_t start, uint64_t end, const std::string& label) {
  const uint64_t abs_end = add_checked(abs_off, len, label);
  if (abs_off < start || abs_end > end) fail(ANIMA_E_FORMAT, label + " lies outside its execution range");
  return Span{abs_off - start, len, true};
}

Span optional_span(bool has_off, uint64_t off, bool has_len, uint64_t len, const PackTensor& t, uint64_t start,
                   uint64_t end, const char* label) {
  if (!has_off && !has_len) return Span{};
  if (!(has_off && has_len)) fail(ANIMA_E_FORMAT, t.name + " has incomplete " + label + " metadata");
  const uint64_t abs = add_checked(t.blob_offset, off, t.name + " " + label);
  return relative(abs, len, start, end, t.name + " " + label);
}

ExecRange execution_range(const std::vector<const PackTensor*>& all, const std::string& prefix, int64_t logical) {
  std::vector<const PackTensor*> members;
  for (const PackTensor* t : all)
    if (t->name.compare(0, prefix.size(), prefix) == 0) members.push_back(t);
  if (members.empty()) fail(ANIMA_E_FORMAT, "no tensors found for " + prefix);
  uint64_t start = UINT64_MAX, end = 0;
  for (const PackTensor* t : members) start = std::min(start, t->blob_offset);
  end = start;
  for (const PackTensor* t : members) end = std::max(end, add_checked(t->blob_offset, t->blob_size, t->name));
  std::stable_sort(members.begin(), members.end(),
                   [](const PackTensor* a, const PackTensor* b) { return a->blob_offset < b->blob_offset; });
  ExecRange r;
  r.logical_index = logical;
  r.file_offset = start;
  r.length = end - start;
  for (const PackTensor* t : members) {
    if (t->blob_offset % kAlign != 0) fail(ANIMA_E_FORMAT, "blob " + t->name + " is not 16 KB aligned");
    TensorSpans s;
    s.tensor = t;
    s.blob = relative(t->blob_offset, t->blob_size, start, end, t->name + " blob");
    s.data = relative(add_checked(t->blob_offset, t->data_offset, t->name + " data"), t->data_size, start, end,
                      t->name + " data");
    s.scale = optional_span(t->has_scale_offset, t->scale_offset, t->has_scale_size, t->scale_size, *t, start, end,
                            "scale");
    s.zero = optional_span(t->has_zero_offset, t->zero_offset, t->has_zero_size, t->zero_size, *t, start, end, "zero");
    r.tensors.push_back(s);
  }
  return r;
}

std::vector<const PackTensor*> all_of(const anima_pack& pk) {
  std::vector<const PackTensor*> v;
  v.reserve(pk.tensors.size());
  for (const PackTensor& t : pk.tensors) v.push_back(&t);
  return v;
}

void range_to_c(const anima_pack& pk, const ExecRange& r, anima_pack_range& o) {
  o.logical_index = r.logical_index;
  o.file_offset = (int64_t)r.file_offset;
  o.length = (int64_t)r.length;
  o.tensor_count = (int64_t)r.tensors.size();
  o.host = pk.map + r.file_offset;
}

// --- DiTQuantizedWeightFactory.makeMatrix (LinearExecutor.swift:467-518): a template
// whose buffers are the range (ptr NULL = offset 0) and whose offsets are the tensor's.
constexpr int64_t kGroup = 64;

anima_qweight make_matrix(const TensorSpans& item, const ExecRange& r, int64_t rows, int64_t cols,
                          const std::string& label) {
  const PackTensor& t = *item.tensor;
  if (!(t.storage == ANIMA_STORAGE_W4 || t.storage == ANIMA_STORAGE_W8 || t.storage == ANIMA_STORAGE_FP16))
    fail(ANIMA_E_FORMAT, label + " must be W4, W8, or FP16");
  if (!(t.shape.size() == 2 && t.shape[0] == rows && t.shape[1] == cols))
    fail(ANIMA_E_INVALID_SHAPE, label + " shape mismatch");
  anima_qweight q{};
  q.storage = t.storage;
  q.rows = rows;
  q.columns = cols;
  const anima_buffer range_buf{nullptr, (int64_t)r.length};
  q.packed = q.scale = q.zero = range_buf;
  if (t.storage == ANIMA_STORAGE_FP16) {
    if (item.data.length != mul_checked(mul_checked((uint64_t)rows, (uint64_t)cols, label), 2, label))
      fail(ANIMA_E_FORMAT, label + " FP16 layout mismatch");
    q.packed_offset = q.scale_offset = q.zero_offset = (int64_t)item.data.offset;
    q.packed_row_stride = cols;
    return q;
  }
  if (!item.scale.present || !item.zero.present) fail(ANIMA_E_FORMAT, label + " missing scale/zero");
  const int64_t stride = t.storage == ANIMA_STORAGE_W4 ? (cols + 1) / 2 : cols;
  const int64_t groups = (cols + kGroup - 1) / kGroup;
  const uint64_t expect_data = mul_checked((uint64_t)rows, (uint64_t)stride, label);
  const uint64_t expect_params = mul_checked(mul_checked((uint64_t)rows, (uint64_t)groups, label), 2, label);
  if (item.data.length != expect_data || item.scale.length != expect_params || item.zero.length != expect_params)
    fail(ANIMA_E_FORMAT, label + " quantized layout mismatch");
  q.packed_offset = (int64_t)item.data.offset;
  q.scale_offset = (int64_t)item.scale.offset;
  q.zero_offset = (int64_t)item.zero.offset;
  q.packed_row_stride = stride;
  return q;
}

// fp16 vector of `n` values: the norm weights.
anima_buffer make_vector(const TensorSpans* item, int64_t n, const std::string& message) {
  if (!item || !(item->tensor->shape.size() == 1 && item->tensor->shape[0] == n) ||
      item->tensor->storage != ANIMA_STORAGE_FP16 || item->data.length != (uint64_t)(2 * n))
    fail(ANIMA_E_FORMAT, message);
  return anima_buffer{reinterpret_cast<void*>((uintptr_t)item->data.offset), 2 * n};
}

std::map<std::string, const TensorSpans*> by_suffix(const ExecRange& r, const std::string& prefix) {
  std::map<std::string, const TensorSpans*> m;
  for (const TensorSpans& s : r.tensors) m[s.tensor->name.substr(prefix.size())] = &s;
  return m;
}

}  // namespace

// Template rebasing shared with the streamed forward (a template pointer holds a byte
// offset from the start of its range).
anima_buffer rebase_buffer(const anima_buffer& t, char* base, int64_t range_bytes, const char* what) {
  const uintptr_t off = reinterpret_cast<uintptr_t>(t.ptr);
  if (off > (uintptr_t)range_bytes)
    fail(ANIMA_E_OUT_OF_BOUNDS, std::string("streamed ") + what + " offset lies outside its block range");
  return anima_buffer{base + off, range_bytes - (int64_t)off};
}

anima_qweight rebase_qweight(const anima_qweight& t, char* base, int64_t range_bytes, const char* what) {
  anima_qweight q = t;
  q.packed = rebase_buffer(t.packed, base, range_bytes, what);
  q.scale = rebase_buffer(t.scale, base, range_bytes, what);
  q.zero = rebase_buffer(t.zero, base, range_bytes, what);
  return q;
}

anima_dit_block_weights rebase_block(const anima_dit_block_weights& t, char* base, int64_t range_bytes) {
  anima_dit_block_weights w = t;
  anima_qweight* dst[] = {&w.self_q, &w.self_k, &w.self_v, &w.self_o, &w.cross_q, &w.cross_k, &w.cross_v, &w.cross_o,
                          &w.mlp1, &w.mlp2, &w.mod_self_w1, &w.mod_self_w2, &w.mod_cross_w1, &w.mod_cross_w2,
                          &w.mod_mlp_w1, &w.mod_mlp_w2};
  for (anima_qweight* q : dst) *q = rebase_qweight(*q, base, range_bytes, "weight");
  w.self_q_norm = rebase_buffer(t.self_q_norm, base, range_bytes, "norm weight");
  w.self_k_norm = rebase_buffer(t.self_k_norm, base, range_bytes, "norm weight");
  w.cross_q_norm = rebase_buffer(t.cross_q_norm, base, range_bytes, "norm weight");
  w.cross_k_norm = rebase_buffer(t.cross_k_norm, base, range_bytes, "norm weight");
  return w;
}

}  // namespace anima

template <class T>
static T* need_handle(T* p, const char* what) {
  if (!p) fail(ANIMA_E_INVALID_ARGUMENT, std::string(what) + " handle is null");
  return p;
}

extern "C" {

anima_status anima_pack_open(const char* path, anima_pack** out) {
  return guarded([&] {
    need_handle(out, "pack output");
    *out = nullptr;
    if (!path) fail(ANIMA_E_INVALID_ARGUMENT, "pack path is null");
    std::unique_ptr<anima_pack> pk(new anima_pack());
    load(*pk, path);
    *out = pk.release();
  });
}

anima_status anima_pack_close(anima_pack* pack) {
  return guarded([&] { delete pack; });
}

anima_status anima_pack_get_info(const anima_pack* pack, anima_pack_info* out) {
  return guarded([&] { *need_handle(out, "output") = need_handle(pack, "pack")->info; });
}

anima_status anima_pack_tensor_at(const anima_pack* pack, int64_t index, anima_pack_tensor* out) {
  return guarded([&] {
    const anima_pack& pk = *need_handle(pack, "pack");
    need_handle(out, "output");
    if (index < 0 || index >= (int64_t)pk.tensors.size()) fail(ANIMA_E_INVALID_ARGUMENT, "tensor index out of range");
    to_c(pk.tensors[(size_t)index], *out);
  });
}

anima_status anima_pack_find(const anima_pack* pack, const char* name, anima_pack_tensor* out) {
  return guarded([&] {
    const anima_pack& pk = *need_handle(pack, "pack");
    need_handle(out, "output");
    if (!name) fail(ANIMA_E_INVALID_ARGUMENT, "tensor name is null");
    auto it = pk.by_name.find(name);
    if (it == pk.by_name.end()) fail(ANIMA_E_INVALID_ARGUMENT, std::string("missing tensor ") + name);
    to_c(pk.tensors[it->second], *out);
  });
}

anima_status anima_pack_crc32_mismatch_count(const anima_pack* pack, int64_t* out) {
  return guarded([&] {
    const anima_pack& pk = *need_handle(pack, "pack");
    need_handle(out, "output");
    int64_t bad = 0;
    for (const PackTensor& t : pk.tensors)
      if (t.has_crc && crc32(pk.map + t.blob_offset + t.data_offset, (size_t)t.data_size) != t.crc) ++bad;
    *out = bad;
  });
}

anima_status anima_pack_bytes(const anima_pack* pack, int64_t offset, int64_t length, const void** out) {
  return guarded([&] {
    const anima_pack& pk = *need_handle(pack, "pack");
    need_handle(out, "output");
    int64_t end;
    if (offset < 0 || length < 0 || __builtin_add_overflow(offset, length, &end) || end > (int64_t)pk.size)
      fail(ANIMA_E_OUT_OF_BOUNDS, "mmap byte range " + std::to_string(offset) + "..<" + std::to_string(offset + length) +
                                      " is out of bounds");
    *out = pk.map + offset;
  });
}

anima_status anima_pack_execution_ranges(const anima_pack* pack, const char* prefix, int64_t count,
                                         anima_pack_range* out) {
  return guarded([&] {
    const anima_pack& pk = *need_handle(pack, "pack");
    if (!prefix) fail(ANIMA_E_INVALID_ARGUMENT, "range prefix is null");
    if (count < 0) fail(ANIMA_E_INVALID_ARGUMENT, "range count must be >= 0");
    if (count > 0) need_handle(out, "output");
    const auto all = all_of(pk);
    std::vector<ExecRange> ranges;
    for (int64_t i = 0; i < count; ++i)
      ranges.push_back(execution_range(all, std::string(prefix) + std::to_string(i) + ".", i));
    std::vector<const ExecRange*> phys;
    for (const ExecRange& r : ranges) phys.push_back(&r);
    std::sort(phys.begin(), phys.end(),
              [](const ExecRange* a, const ExecRange* b) { return a->file_offset < b->file_offset; });
    for (size_t i = 0; i + 1 < phys.size(); ++i)
      if (phys[i]->file_offset + phys[i]->length > phys[i + 1]->file_offset)
        fail(ANIMA_E_FORMAT, "execution ranges " + std::to_string(phys[i]->logical_index) + " and " +
                                 std::to_string(phys[i + 1]->logical_index) + " overlap");
    for (int64_t i = 0; i < count; ++i) range_to_c(pk, ranges[(size_t)i], out[i]);
  });
}

anima_status anima_pack_dit_block(const anima_pack* pack, int64_t block, anima_dit_block_weights* tmpl,
                                  anima_pack_range* range) {
  return guarded([&] {
    const anima_pack& pk = *need_handle(pack, "pack");
    need_handle(tmpl, "template output");
    if (block < 0) fail(ANIMA_E_INVALID_ARGUMENT, "DiT block index " + std::to_string(block) + " is out of range");
    const std::string prefix = "model.diffusion_model.blocks." + std::to_string(block) + ".";
    const ExecRange r = execution_range(all_of(pk), prefix, block);
    const auto spans = by_suffix(r, prefix);
    auto matrix = [&](const char* name, int64_t rows, int64_t cols) {
      auto it = spans.find(name);
      if (it == spans.end()) fail(ANIMA_E_FORMAT, "missing DiT matrix " + prefix + name);
      return make_matrix(*it->second, r, rows, cols, "DiT " + prefix + name);
    };
    auto norm = [&](const char* name) {
      auto it = spans.find(name);
      return make_vector(it == spans.end() ? nullptr : it->second, 128, "invalid DiT norm " + prefix + name);
    };
    anima_dit_block_weights w{};
    w.mod_self_w1 = matrix("adaln_modulation_self_attn.1.weight", 256, 2048);
    w.mod_self_w2 = matrix("adaln_modulation_self_attn.2.weight", 6144, 256);
    w.mod_cross_w1 = matrix("adaln_modulation_cross_attn.1.weight", 256, 2048);
    w.mod_cross_w2 = matrix("adaln_modulation_cross_attn.2.weight", 6144, 256);
    w.mod_mlp_w1 = matrix("adaln_modulation_mlp.1.weight", 256, 2048);
    w.mod_mlp_w2 = matrix("adaln_modulation_mlp.2.weight", 6144, 256);
    w.self_q = matrix("self_attn.q_proj.weight", 2048, 2048);
    w.self_k = matrix("self_attn.k_proj.weight", 2048, 2048);
    w.self_v = matrix("self_attn.v_proj.weight", 2048, 2048);
    w.self_o = matrix("self_attn.output_proj.weight", 2048, 2048);
    w.cross_q = matrix("cross_attn.q_proj.weight", 2048, 2048);
    w.cross_k = matrix("cross_attn.k_proj.weight", 2048, 1024);
    w.cross_v = matrix("cross_attn.v_proj.weight", 2048, 1024);
    w.cross_o = matrix("cross_attn.output_proj.weight", 2048, 2048);
    w.mlp1 = matrix("mlp.layer1.weight", 8192, 2048);
    w.mlp2 = matrix("mlp.layer2.weight", 2048, 8192);
    w.self_q_norm = norm("self_attn.q_norm.weight");
    w.self_k_norm = norm("self_attn.k_norm.weight");
    w.cross_q_norm = norm("cross_attn.q_norm.weight");
    w.cross_k_norm = norm("cross_attn.k_norm.weight");
    if (spans.size() != 20) fail(ANIMA_E_FORMAT, "DiT block must contain exactly 20 tensors");
    *tmpl = w;
    if (range) range_to_c(pk, r, *range);
  });
}

anima_status anima_pack_dit_prepare(const anima_pack* pack, int64_t dim, anima_dit_prepare_weights* tmpl,
                                    anima_pack_range* range) {
  return guarded([&] {
    const anima_pack& pk = *need_handle(pack, "pack");
    need_handle(tmpl, "template output");
    if (dim <= 0) fail(ANIMA_E_INVALID_SHAPE, "DiT preparation hidden width must be positive");
    if (pk.info.quant_group != 64) fail(ANIMA_E_FORMAT, "DiT preparation requires quant group 64");
    const std::string p = "model.diffusion_model.";
    const std::set<std::string> names = {p + "t_embedder.1.linear_1.weight", p + "t_embedder.1.linear_2.weight",
                                         p + "t_embedding_norm.weight", p + "x_embedder.proj.1.weight"};
    std::vector<const PackTensor*> chosen;
    for (const PackTensor& t : pk.tensors)
      if (names.count(t.name)) chosen.push_back(&t);
    const ExecRange r = execution_range(chosen, p, -2);
    std::set<std::string> got;
    for (const TensorSpans& s : r.tensors) got.insert(s.tensor->name);
    if (got != names) fail(ANIMA_E_FORMAT, "DiT preparation range is incomplete");
    const auto spans = by_suffix(r, p);
    auto matrix = [&](const char* name, int64_t rows, int64_t cols) {
      return make_matrix(*spans.at(name), r, rows, cols, std::string("DiT preparation ") + name);
    };
    anima_dit_prepare_weights w{};
    w.x_embed = matrix("x_embedder.proj.1.weight", dim, 68);
    w.t_embed1 = matrix("t_embedder.1.linear_1.weight", dim, dim);
    w.t_embed2 = matrix("t_embedder.1.linear_2.weight", 3 * dim, dim);
    w.t_norm = make_vector(spans.at("t_embedding_norm.weight"), dim, "invalid DiT preparation norm/range");
    if (r.tensors.size() != 4) fail(ANIMA_E_FORMAT, "invalid DiT preparation norm/range");
    *tmpl = w;
    if (range) range_to_c(pk, r, *range);
  });
}

anima_status anima_pack_dit_final(const anima_pack* pack, int64_t dim, anima_dit_final_weights* tmpl,
                                  anima_pack_range* range) {
  return guarded([&] {
    const anima_pack& pk = *need_handle(pack, "pack");
    need_handle(tmpl, "template output");
    if (dim <= 0) fail(ANIMA_E_INVALID_SHAPE, "DiT final-layer hidden width must be positive");
    const std::string prefix = "model.diffusion_model.final_layer.";
    const ExecRange r = execution_range(all_of(pk), prefix, -1);
    if (r.tensors.size() != 3) fail(ANIMA_E_FORMAT, "DiT final layer must contain exactly 3 tensors");
    std::map<std::string, const TensorSpans*> spans;
    for (const TensorSpans& s : r.tensors)
      if (!spans.emplace(s.tensor->name.substr(prefix.size()), &s).second)
        fail(ANIMA_E_FORMAT, "duplicate DiT final tensor " + s.tensor->name.substr(prefix.size()));
    auto item = [&](const char* name) -> const TensorSpans& {
      auto it = spans.find(name);
      if (it == spans.end()) fail(ANIMA_E_FORMAT, std::string("missing DiT final matrix ") + name);
      return *it->second;
    };
    const TensorSpans& m1 = item("adaln_modulation.1.weight");
    const int64_t lora = m1.tensor->shape.size() == 2 ? m1.tensor->shape[0] : -1;
    if (lora <= 0) fail(ANIMA_E_INVALID_SHAPE, "DiT final adaln_modulation.1.weight shape mismatch");
    anima_dit_final_weights w{};
    w.mod_w1 = make_matrix(m1, r, lora, dim, "DiT final adaln_modulation.1.weight");
    w.mod_w2 = make_matrix(item("adaln_modulation.2.weight"), r, 2 * dim, lora, "DiT final adaln_modulation.2.weight");
    w.proj = make_matrix(item("linear.weight"), r, 64, dim, "DiT final linear.weight");
    *tmpl = w;
    if (range) range_to_c(pk, r, *range);
  });
}

anima_status anima_dit_block_weights_rebase(const anima_dit_block_weights* tmpl, void* base, int64_t range_bytes,
                                            anima_dit_block_weights* out) {
  return guarded([&] {
    need_handle(tmpl, "template");
    need_handle(out, "output");
    if (!base || range_bytes < 0) fail(ANIMA_E_INVALID_ARGUMENT, "rebase needs a base pointer and a range size");
    *out = rebase_block(*tmpl, static_cast<char*>(base), range_bytes);
  });
}

anima_status anima_dit_prepare_weights_rebase(const anima_dit_prepare_weights* tmpl, void* base,
                                              int64_t range_bytes, anima_dit_prepare_weights* out) {
  return guarded([&] {
    need_handle(tmpl, "template");
    need_handle(out, "output");
    if (!base || range_bytes < 0) fail(ANIMA_E_INVALID_ARGUMENT, "rebase needs a base pointer and a range size");
    char* b = static_cast<char*>(base);
    anima_dit_prepare_weights w = *tmpl;
    w.x_embed = rebase_qweight(tmpl->x_embed, b, range_bytes, "weight");
    w.t_embed1 = rebase_qweight(tmpl->t_embed1, b, range_bytes, "weight");
    w.t_embed2 = rebase_qweight(tmpl->t_embed2, b, range_bytes, "weight");
    w.t_norm = rebase_buffer(tmpl->t_norm, b, range_bytes, "norm weight");
    *out = w;
  });
}

anima_status anima_dit_final_weights_rebase(const anima_dit_final_weights* tmpl, void* base, int64_t range_bytes,
                                            anima_dit_final_weights* out) {
  return guarded([&] {
    need_handle(tmpl, "template");
    need_handle(out, "output");
    if (!base || range_bytes < 0) fail(ANIMA_E_INVALID_ARGUMENT, "rebase needs a base pointer and a range size");
    char* b = static_cast<char*>(base);
    anima_dit_final_weights w = *tmpl;
    w.mod_w1 = rebase_qweight(tmpl->mod_w1, b, range_bytes, "weight");
    w.mod_w2 = rebase_qweight(tmpl->mod_w2, b, range_bytes, "weight");
    w.proj = rebase_qweight(tmpl->proj, b, range_bytes, "weight");
    *out = w;
  });
}

}  // extern "C"
