// Reader of MLL packages and the plan classifier that binds them to the
// fused encoder.
//
// The container is what the reference writes through m31labs.dev/mll v0.1.0
// (artifact/eos/mll.go:112-330 for modules, runtime/weight_file.go:122-229
// for weight files). That module is not vendored; the framing below was read
// off the packages the reference ships and is checked against their BLAKE3
// section digests:
//   header   24 bytes: "MLL\0", version 1.0 (bytes 0x00 0x01), profile byte,
//            reserved byte, u64 file size, u64 section count
//   section  64-byte directory entries from offset 24: tag[4], u64 offset,
//            u64 size, BLAKE3 digest[32] of the body, u16 flags (1 required,
//            2 skippable, 0x10 aligned, 0x20 schemaless), u16 schema
//            version, 8 reserved zero bytes
//   STRG     u64 count (the implicit "" at index 0 included), then count - 1
//            strings as u32 length + bytes
//   TNSR     u32 count, then per tensor: u32 name index, u8 dtype, u32 rank,
//            u64 dims[rank], u64 offset and u64 size of the payload (relative
//            to the section body), u32 reserved zero
//   XMTA     JSON metadata (MLLMetadata, artifact/eos/mll.go:24-34): the
//            artifact (params, steps, kernels), json_files, logical dtypes
//            and the Q8/Q4 tensor_scales
//   XKBI     offline kernel images: never read, hashed or decoded here.
// Packed Q8 payloads are int8 codes and packed Q4 payloads offset-binary
// nibbles, low nibble first, each with one per-tensor scale (dequantized =
// code * scale; decodeTensorEntry, runtime/weight_file.go:305-415).
#include <algorithm>
#include <array>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <string>
#include <utility>
#include <vector>

#include "eoship_internal.h"

using eoship::set_err;

namespace {

// ----------------------------------------------------------------- BLAKE3
// Hash mode of BLAKE3 as its specification defines it (1 KiB chunks of
// 64-byte blocks, seven rounds of the G function, a binary tree of chaining
// values merged as chunks complete, ROOT on the last compression).
namespace b3 {

constexpr uint32_t kIV[8] = {0x6A09E667u, 0xBB67AE85u, 0x3C6EF372u, 0xA54FF53Au,
                             0x510E527Fu, 0x9B05688Cu, 0x1F83D9ABu, 0x5BE0CD19u};
constexpr int kPerm[16] = {2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8};
enum : uint32_t { kChunkStart = 1, kChunkEnd = 2, kParent = 4, kRoot = 8 };
using Cv = std::array<uint32_t, 8>;

inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

inline void g(uint32_t* s, int a, int b, int c, int d, uint32_t x, uint32_t y) {
  s[a] = s[a] + s[b] + x;
  s[d] = rotr(s[d] ^ s[a], 16);
  s[c] = s[c] + s[d];
  s[b] = rotr(s[b] ^ s[c], 12);
  s[a] = s[a] + s[b] + y;
  s[d] = rotr(s[d] ^ s[a], 8);
  s[c] = s[c] + s[d];
  s[b] = rotr(s[b] ^ s[c], 7);
}

// First 8 output words of the compression function.
Cv compress(const Cv& cv, const uint8_t block[64], uint64_t counter, uint32_t blen,
            uint32_t flags) {
  uint32_t m[16];
  for (int i = 0; i < 16; ++i)
    m[i] = (uint32_t)block[4 * i] | (uint32_t)block[4 * i + 1] << 8 |
           (uint32_t)block[4 * i + 2] << 16 | (uint32_t)block[4 * i + 3] << 24;
  uint32_t s[16] = {cv[0],  cv[1],  cv[2],  cv[3],  cv[4],  cv[5],
                    cv[6],  cv[7],  kIV[0], kIV[1], kIV[2], kIV[3],
                    (uint32_t)counter, (uint32_t)(counter >> 32), blen, flags};
  for (int r = 0; r < 7; ++r) {
    g(s, 0, 4, 8, 12, m[0], m[1]);
    g(s, 1, 5, 9, 13, m[2], m[3]);
    g(s, 2, 6, 10, 14, m[4], m[5]);
    g(s, 3, 7, 11, 15, m[6], m[7]);
    g(s, 0, 5, 10, 15, m[8], m[9]);
    g(s, 1, 6, 11, 12, m[10], m[11]);
    g(s, 2, 7, 8, 13, m[12], m[13]);
    g(s, 3, 4, 9, 14, m[14], m[15]);
    if (r < 6) {
      uint32_t t[16];
      for (int i = 0; i < 16; ++i) t[i] = m[kPerm[i]];
      std::memcpy(m, t, sizeof(m));
    }
  }
  Cv out;
  for (int i = 0; i < 8; ++i) out[i] = s[i] ^ s[i + 8];
  return out;
}

Cv iv() {
  Cv c;
  for (int i = 0; i < 8; ++i) c[i] = kIV[i];
  return c;
}

// Chaining value of one chunk (len <= 1024); `root` puts ROOT on its last
// block (a message of a single chunk).
Cv chunk(const uint8_t* p, size_t len, uint64_t index, bool root) {
  Cv cv = iv();
  const size_t nblocks = len == 0 ? 1 : (len + 63) / 64;
  for (size_t b = 0; b < nblocks; ++b) {
    uint8_t block[64] = {0};
    const size_t n = std::min<size_t>(64, len - std::min(len, b * 64));
    if (n > 0) std::memcpy(block, p + b * 64, n);
    uint32_t flags = (b == 0 ? kChunkStart : 0u) | (b + 1 == nblocks ? kChunkEnd : 0u);
    if (root && b + 1 == nblocks) flags |= kRoot;
    cv = compress(cv, block, index, (uint32_t)n, flags);
  }
  return cv;
}

Cv parent(const Cv& l, const Cv& r, bool root) {
  uint8_t block[64];
  for (int i = 0; i < 8; ++i)
    for (int j = 0; j < 4; ++j) {
      block[4 * i + j] = (uint8_t)(l[i] >> (8 * j));
      block[32 + 4 * i + j] = (uint8_t)(r[i] >> (8 * j));
    }
  return compress(iv(), block, 0, 64, kParent | (root ? kRoot : 0u));
}

void hash(const uint8_t* p, size_t len, uint8_t out[32]) {
  const size_t nchunks = len == 0 ? 1 : (len + 1023) / 1024;
  Cv cv;
  if (nchunks == 1) {
    cv = chunk(p, len, 0, true);
  } else {
    std::vector<Cv> stack;
    for (size_t i = 0; i + 1 < nchunks; ++i) {
      Cv c = chunk(p + i * 1024, 1024, i, false);
      // A completed subtree merges while the chunk count has trailing zeros.
      for (uint64_t total = i + 1; (total & 1) == 0; total >>= 1) {
        c = parent(stack.back(), c, false);
        stack.pop_back();
      }
      stack.push_back(c);
    }
    cv = chunk(p + (nchunks - 1) * 1024, len - (nchunks - 1) * 1024, nchunks - 1, false);
    while (stack.size() > 1) {
      cv = parent(stack.back(), cv, false);
      stack.pop_back();
    }
    cv = parent(stack.back(), cv, true);
  }
  for (int i = 0; i < 8; ++i)
    for (int j = 0; j < 4; ++j) out[4 * i + j] = (uint8_t)(cv[i] >> (8 * j));
}

}  // namespace b3

// ------------------------------------------------------------------- JSON
// A small DOM: objects keep their members in file order.
struct Json {
  enum Kind { kNull, kBool, kNum, kStr, kArr, kObj } kind = kNull;
  bool b = false;
  double num = 0.0;
  std::string str;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;

  const Json* get(const char* key) const {
    if (kind != kObj) return nullptr;
    for (const auto& kv : obj)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
  const std::string* get_str(const char* key) const {
    const Json* v = get(key);
    return v != nullptr && v->kind == kStr ? &v->str : nullptr;
  }
  std::string str_or(const char* key, const char* dflt) const {
    const std::string* s = get_str(key);
    return s != nullptr ? *s : std::string(dflt);
  }
};

class JsonParser {
 public:
  JsonParser(const char* p, size_t n) : p_(p), end_(p + n) {}
  bool parse(Json* out, std::string* err) {
    if (!value(out, 0)) {
      *err = err_;
      return false;
    }
    ws();
    if (p_ != end_) {
      *err = "trailing bytes after the JSON value";
      return false;
    }
    return true;
  }

 private:
  const char* p_;
  const char* end_;
  std::string err_;

  bool fail(const char* what) {
    if (err_.empty()) err_ = what;
    return false;
  }
  void ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
  }
  bool lit(const char* s) {
    const size_t n = std::strlen(s);
    if ((size_t)(end_ - p_) < n || std::memcmp(p_, s, n) != 0) return fail("invalid literal");
    p_ += n;
    return true;
  }
  static void utf8(uint32_t c, std::string* s) {
    if (c < 0x80) {
      s->push_back((char)c);
    } else if (c < 0x800) {
      s->push_back((char)(0xC0 | (c >> 6)));
      s->push_back((char)(0x80 | (c & 0x3F)));
    } else if (c < 0x10000) {
      s->push_back((char)(0xE0 | (c >> 12)));
      s->push_back((char)(0x80 | ((c >> 6) & 0x3F)));
      s->push_back((char)(0x80 | (c & 0x3F)));
    } else {
      s->push_back((char)(0xF0 | (c >> 18)));
      s->push_back((char)(0x80 | ((c >> 12) & 0x3F)));
      s->push_back((char)(0x80 | ((c >> 6) & 0x3F)));
      s->push_back((char)(0x80 | (c & 0x3F)));
    }
  }
  bool hex4(uint32_t* v) {
    if (end_ - p_ < 4) return fail("short \\u escape");
    uint32_t r = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = *p_++;
      r <<= 4;
      if (c >= '0' && c <= '9') r |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') r |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') r |= (uint32_t)(c - 'A' + 10);
      else return fail("bad \\u escape");
    }
    *v = r;
    return true;
  }
  bool string(std::string* s) {
    ++p_;  // opening quote
    while (true) {
      if (p_ >= end_) return fail("unterminated string");
      const unsigned char c = (unsigned char)*p_++;
      if (c == '"') return true;
      if (c < 0x20) return fail("control character in string");
      if (c != '\\') {
        s->push_back((char)c);
        continue;
      }
      if (p_ >= end_) return fail("unterminated escape");
      const char e = *p_++;
      switch (e) {
        case '"': s->push_back('"'); break;
        case '\\': s->push_back('\\'); break;
        case '/': s->push_back('/'); break;
        case 'b': s->push_back('\b'); break;
        case 'f': s->push_back('\f'); break;
        case 'n': s->push_back('\n'); break;
        case 'r': s->push_back('\r'); break;
        case 't': s->push_back('\t'); break;
        case 'u': {
          uint32_t c1 = 0;
          if (!hex4(&c1)) return false;
          if (c1 >= 0xD800 && c1 < 0xDC00 && end_ - p_ >= 6 && p_[0] == '\\' && p_[1] == 'u') {
            const char* save = p_;
            p_ += 2;
            uint32_t c2 = 0;
            if (!hex4(&c2)) return false;
            if (c2 >= 0xDC00 && c2 < 0xE000) {
              c1 = 0x10000 + ((c1 - 0xD800) << 10) + (c2 - 0xDC00);
            } else {
              p_ = save;
            }
          }
          utf8(c1, s);
          break;
        }
        default:
          return fail("bad escape");
      }
    }
  }
  bool number(Json* out) {
    const char* s = p_;
    if (p_ < end_ && *p_ == '-') ++p_;
    if (p_ >= end_) return fail("bad number");
    if (*p_ == '0') {
      ++p_;
    } else if (*p_ >= '1' && *p_ <= '9') {
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    } else {
      return fail("bad number");
    }
    if (p_ < end_ && *p_ == '.') {
      ++p_;
      if (p_ >= end_ || *p_ < '0' || *p_ > '9') return fail("bad fraction");
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
      ++p_;
      if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
      if (p_ >= end_ || *p_ < '0' || *p_ > '9') return fail("bad exponent");
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    out->kind = Json::kNum;
    out->str.assign(s, p_);
    out->num = std::strtod(out->str.c_str(), nullptr);
    return true;
  }
  bool value(Json* out, int depth) {
    if (depth > 200) return fail("JSON nested too deeply");
    ws();
    if (p_ >= end_) return fail("unexpected end of JSON");
    const char c = *p_;
    if (c == '{') {
      ++p_;
      out->kind = Json::kObj;
      ws();
      if (p_ < end_ && *p_ == '}') {
        ++p_;
        return true;
      }
      while (true) {
        ws();
        if (p_ >= end_ || *p_ != '"') return fail("expected a member name");
        std::string key;
        if (!string(&key)) return false;
        ws();
        if (p_ >= end_ || *p_ != ':') return fail("expected ':'");
        ++p_;
        out->obj.emplace_back(std::move(key), Json());
        if (!value(&out->obj.back().second, depth + 1)) return false;
        ws();
        if (p_ < end_ && *p_ == ',') {
          ++p_;
          continue;
        }
        if (p_ < end_ && *p_ == '}') {
          ++p_;
          return true;
        }
        return fail("expected ',' or '}'");
      }
    }
    if (c == '[') {
      ++p_;
      out->kind = Json::kArr;
      ws();
      if (p_ < end_ && *p_ == ']') {
        ++p_;
        return true;
      }
      while (true) {
        out->arr.emplace_back();
        if (!value(&out->arr.back(), depth + 1)) return false;
        ws();
        if (p_ < end_ && *p_ == ',') {
          ++p_;
          continue;
        }
        if (p_ < end_ && *p_ == ']') {
          ++p_;
          return true;
        }
        return fail("expected ',' or ']'");
      }
    }
    if (c == '"') {
      out->kind = Json::kStr;
      return string(&out->str);
    }
    if (c == 't') {
      out->kind = Json::kBool;
      out->b = true;
      return lit("true");
    }
    if (c == 'f') {
      out->kind = Json::kBool;
      return lit("false");
    }
    if (c == 'n') return lit("null");
    return number(out);
  }
};

// ---------------------------------------------------------------- container

uint64_t rd64(const uint8_t* p) {
  uint64_t v = 0;
  for (int i = 7; i >= 0; --i) v = v << 8 | p[i];
  return v;
}
uint32_t rd32(const uint8_t* p) {
  return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}
uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | p[1] << 8); }

constexpr uint8_t kDTypeQ8 = 13;  // the only storage dtype code the shipped packages use

struct Section {
  char tag[5] = {0};
  uint64_t off = 0, size = 0;
  uint16_t flags = 0, schema = 0;
  bool verified = false;
};

struct Tensor {
  std::string name;
  int code = 0;  // storage dtype code of the TNSR entry
  int kind = 0;  // EOSHIP_MLL_*
  std::vector<int64_t> dims;
  int64_t elements = 0;
  uint64_t off = 0, size = 0;  // payload, relative to the file
  float scale = 0.f;
  bool has_scale = false;
  std::string logical;
};

bool known_tag(const char* t) {
  static const char* kTags[] = {"HEAD", "STRG", "DIMS", "TYPE", "PARM", "ENTR", "BUFF",
                                "KRNL", "MEMP", "TNSR", "SCHM", "XMTA", "XKBI", "XTOK"};
  for (const char* k : kTags)
    if (std::memcmp(k, t, 4) == 0) return true;
  return false;
}

}  // namespace

struct EosHipMll {
  std::vector<uint8_t> bytes;
  int profile = 0;
  std::vector<Section> sections;
  std::vector<std::string> strings;
  std::vector<Tensor> tensors;
  bool has_meta = false;
  Json meta;  // the XMTA document
  std::string xmta_text;

  const Section* section(const char* tag) const {
    for (const Section& s : sections)
      if (std::memcmp(s.tag, tag, 4) == 0) return &s;
    return nullptr;
  }
  const Tensor* tensor(const std::string& name) const {
    for (const Tensor& t : tensors)
      if (t.name == name) return &t;
    return nullptr;
  }
};

namespace {

int parse_container(EosHipMll* m, char** err) {
  const char* what = "eoship_mll_open";
  const uint8_t* d = m->bytes.data();
  const size_t n = m->bytes.size();
  if (n < 24 || std::memcmp(d, "MLL\0", 4) != 0) return set_err(err, "%s: not an MLL file", what);
  if (d[4] != 0x00 || d[5] != 0x01)
    return set_err(err, "%s: MLL version %u.%u is not supported (want 1.0)", what, d[5], d[4]);
  m->profile = d[6];
  if (rd64(d + 8) != (uint64_t)n)
    return set_err(err, "%s: header says %llu bytes, the file has %zu", what,
                   (unsigned long long)rd64(d + 8), n);
  const uint64_t count = rd64(d + 16);
  if (count > 4096 || 24 + 64 * count > n)
    return set_err(err, "%s: section directory (%llu entries) exceeds the file", what,
                   (unsigned long long)count);
  const uint64_t body0 = 24 + 64 * count;
  for (uint64_t i = 0; i < count; ++i) {
    const uint8_t* e = d + 24 + 64 * i;
    Section s;
    std::memcpy(s.tag, e, 4);
    s.off = rd64(e + 4);
    s.size = rd64(e + 12);
    s.flags = rd16(e + 52);
    s.schema = rd16(e + 54);
    for (int j = 56; j < 64; ++j)
      if (e[j] != 0) return set_err(err, "%s: section %.4s has non-zero reserved bytes", what, s.tag);
    if (s.off < body0 || s.off > n || s.size > n - s.off)
      return set_err(err, "%s: section %.4s [%llu, +%llu) lies outside the file", what, s.tag,
                     (unsigned long long)s.off, (unsigned long long)s.size);
    for (const Section& o : m->sections)
      if (std::memcmp(o.tag, s.tag, 4) == 0)
        return set_err(err, "%s: duplicate section %.4s", what, s.tag);
    if (!known_tag(s.tag) && (s.flags & 1) != 0)
      return set_err(err, "%s: required section %.4s is not supported", what, s.tag);
    // XKBI (offline kernel images) is skipped without reading its bytes.
    if (std::memcmp(s.tag, "XKBI", 4) != 0) {
      uint8_t digest[32];
      b3::hash(d + s.off, (size_t)s.size, digest);
      if (std::memcmp(digest, e + 20, 32) != 0)
        return set_err(err, "%s: section %.4s fails its BLAKE3 digest", what, s.tag);
      s.verified = true;
    }
    m->sections.push_back(s);
  }
  // Bodies may not overlap.
  std::vector<std::pair<uint64_t, uint64_t>> spans;
  for (const Section& s : m->sections) spans.emplace_back(s.off, s.size);
  std::sort(spans.begin(), spans.end());
  for (size_t i = 1; i < spans.size(); ++i)
    if (spans[i - 1].first + spans[i - 1].second > spans[i].first)
      return set_err(err, "%s: section bodies overlap", what);
  return 0;
}

int parse_strings(EosHipMll* m, char** err) {
  const Section* s = m->section("STRG");
  if (s == nullptr) return set_err(err, "eoship_mll_open: missing STRG section");
  const uint8_t* p = m->bytes.data() + s->off;
  const uint64_t n = s->size;
  if (n < 8) return set_err(err, "eoship_mll_open: STRG section too short");
  const uint64_t count = rd64(p);
  if (count == 0 || count > n) return set_err(err, "eoship_mll_open: bad STRG count");
  m->strings.reserve((size_t)count);
  m->strings.emplace_back();
  uint64_t q = 8;
  for (uint64_t i = 1; i < count; ++i) {
    if (n - q < 4) return set_err(err, "eoship_mll_open: STRG entry %llu truncated", (unsigned long long)i);
    const uint32_t len = rd32(p + q);
    q += 4;
    if (n - q < len) return set_err(err, "eoship_mll_open: STRG entry %llu truncated", (unsigned long long)i);
    m->strings.emplace_back(reinterpret_cast<const char*>(p + q), len);
    q += len;
  }
  if (q != n) return set_err(err, "eoship_mll_open: %llu stray bytes after the STRG entries", (unsigned long long)(n - q));
  return 0;
}

// MLLMetadata.Validate (artifact/eos/mll.go:62-103).
int parse_meta(EosHipMll* m, char** err) {
  const char* what = "eoship_mll_open";
  const Section* s = m->section("XMTA");
  if (s == nullptr) return 0;
  m->xmta_text.assign(reinterpret_cast<const char*>(m->bytes.data() + s->off), (size_t)s->size);
  std::string perr;
  JsonParser jp(m->xmta_text.data(), m->xmta_text.size());
  if (!jp.parse(&m->meta, &perr)) return set_err(err, "%s: XMTA metadata: %s", what, perr.c_str());
  const Json& j = m->meta;
  if (j.kind != Json::kObj) return set_err(err, "%s: XMTA metadata is not an object", what);
  const std::string* ver = j.get_str("version");
  if (ver == nullptr || ver->empty()) return set_err(err, "%s: MLL metadata version is required", what);
  if (*ver != "manta/mll/v0alpha1")
    return set_err(err, "%s: MLL metadata version \"%s\" is not supported, want \"manta/mll/v0alpha1\"",
                   what, ver->c_str());
  const std::string* mn = j.get_str("module_name");
  const std::string* mv = j.get_str("module_version");
  if (mn == nullptr || mn->empty()) return set_err(err, "%s: MLL metadata module_name is required", what);
  if (mv == nullptr || mv->empty()) return set_err(err, "%s: MLL metadata module_version is required", what);
  const Json* art = j.get("artifact");
  if (art == nullptr || art->kind != Json::kObj)
    return set_err(err, "%s: MLL metadata artifact must be valid JSON", what);
  if (const Json* lt = j.get("logical_tensor_dtypes")) {
    if (lt->kind != Json::kObj) return set_err(err, "%s: logical_tensor_dtypes must be an object", what);
    for (const auto& kv : lt->obj)
      if (kv.first.empty() || kv.second.kind != Json::kStr || kv.second.str.empty())
        return set_err(err, "%s: MLL metadata logical tensor dtype for \"%s\" is required", what,
                       kv.first.c_str());
  }
  if (const Json* ts = j.get("tensor_scales")) {
    if (ts->kind != Json::kObj) return set_err(err, "%s: tensor_scales must be an object", what);
    for (const auto& kv : ts->obj) {
      // Go decodes these as float32; the metadata writes each one's shortest
      // float32 digits, so rounding through double gives the same value.
      const float sc = (float)kv.second.num;
      if (kv.first.empty() || kv.second.kind != Json::kNum || std::isnan(sc) || std::isinf(sc) ||
          sc < 0.f)
        return set_err(err, "%s: MLL metadata tensor scale for \"%s\" must be finite and non-negative",
                       what, kv.first.c_str());
    }
  }
  m->has_meta = true;
  return 0;
}

int parse_tensors(EosHipMll* m, char** err) {
  const char* what = "eoship_mll_open";
  const Section* s = m->section("TNSR");
  if (s == nullptr) return set_err(err, "%s: missing TNSR section", what);
  const uint8_t* p = m->bytes.data() + s->off;
  const uint64_t n = s->size;
  if (n < 4) return set_err(err, "%s: TNSR section too short", what);
  const uint32_t count = rd32(p);
  uint64_t q = 4;
  const Json* logical = m->has_meta ? m->meta.get("logical_tensor_dtypes") : nullptr;
  const Json* scales = m->has_meta ? m->meta.get("tensor_scales") : nullptr;
  for (uint32_t i = 0; i < count; ++i) {
    if (n - q < 9) return set_err(err, "%s: TNSR entry %u truncated", what, i);
    Tensor t;
    const uint32_t name = rd32(p + q);
    t.code = p[q + 4];
    const uint32_t rank = rd32(p + q + 5);
    q += 9;
    if (rank > 8 || n - q < 8ull * rank + 20) return set_err(err, "%s: TNSR entry %u truncated", what, i);
    if (name >= m->strings.size() || m->strings[name].empty())
      return set_err(err, "%s: weight tensor missing name for index %u", what, name);
    t.name = m->strings[name];
    t.elements = 1;
    for (uint32_t r = 0; r < rank; ++r) {
      const uint64_t dim = rd64(p + q + 8ull * r);
      if (dim == 0 || dim > (1ull << 40) || (uint64_t)t.elements > (1ull << 40) / dim)
        return set_err(err, "%s: tensor \"%s\" has a bad shape", what, t.name.c_str());
      t.dims.push_back((int64_t)dim);
      t.elements *= (int64_t)dim;
    }
    q += 8ull * rank;
    const uint64_t off = rd64(p + q), size = rd64(p + q + 8);
    const uint32_t reserved = rd32(p + q + 16);
    q += 20;
    if (reserved != 0)
      return set_err(err, "%s: tensor \"%s\" has an unsupported entry field (%u)", what,
                     t.name.c_str(), reserved);
    if (off > n || size > n - off)
      return set_err(err, "%s: tensor \"%s\" payload lies outside TNSR", what, t.name.c_str());
    t.off = s->off + off;
    t.size = size;
    if (logical != nullptr)
      if (const std::string* l = logical->get_str(t.name.c_str())) t.logical = *l;
    if (scales != nullptr)
      if (const Json* v = scales->get(t.name.c_str())) {
        t.scale = (float)v->num;
        t.has_scale = true;
      }
    // Storage kind: the Q8 code, else the logical dtype with the payload
    // size it implies (packed q4 is (n + 1) / 2 bytes, values 4 bytes each).
    const uint64_t e = (uint64_t)t.elements;
    if (t.code == kDTypeQ8) {
      if (size != e)
        return set_err(err, "%s: q8 tensor \"%s\" data length %llu does not match %llu elements",
                       what, t.name.c_str(), (unsigned long long)size, (unsigned long long)e);
      t.kind = EOSHIP_MLL_Q8;
    } else if (t.logical == "q4" && size == (e + 1) / 2) {
      t.kind = EOSHIP_MLL_Q4;
    } else if ((t.logical == "f32" || t.logical == "q8" || t.logical == "q4") && size == 4 * e) {
      t.kind = EOSHIP_MLL_F32;
    } else if (t.logical == "f16" && size == 2 * e) {
      t.kind = EOSHIP_MLL_F16;
    } else if (t.logical == "i32" && size == 4 * e) {
      t.kind = EOSHIP_MLL_I32;
    } else if (t.logical == "i64" && size == 8 * e) {
      t.kind = EOSHIP_MLL_I64;
    } else {
      return set_err(err, "%s: tensor \"%s\": storage dtype %d with logical dtype \"%s\" and %llu bytes is not supported",
                     what, t.name.c_str(), t.code, t.logical.c_str(), (unsigned long long)size);
    }
    // Packed payloads without a scale must be all zero codes
    // (requireAllZeroPackedPayload, runtime/weight_file.go:417-440).
    if ((t.kind == EOSHIP_MLL_Q8 || t.kind == EOSHIP_MLL_Q4) && !(t.scale > 0.f)) {
      const uint8_t* b = m->bytes.data() + t.off;
      bool zero = true;
      if (t.kind == EOSHIP_MLL_Q8) {
        for (uint64_t k = 0; k < size && zero; ++k) zero = b[k] == 0;
      } else {
        for (uint64_t k = 0; k < e && zero; ++k) zero = ((b[k / 2] >> (4 * (k & 1))) & 0xF) == 8;
      }
      if (!zero)
        return set_err(err, "%s: tensor \"%s\": packed payload has non-zero codes but no dequantization scale (missing tensor_scales metadata)",
                       what, t.name.c_str());
    }
    for (const Tensor& o : m->tensors)
      if (o.name == t.name) return set_err(err, "%s: duplicate tensor \"%s\"", what, t.name.c_str());
    m->tensors.push_back(std::move(t));
  }
  return 0;
}

// ------------------------------------------------------------ plan matching

// The op class of a launch_kernel step's kernel (classifyCUDAKernel,
// runtime/backends/cuda/native_linux.go:3783-3803, keeps the first body op):
// the body must be exactly that op followed by return.
std::string kernel_op(const Json& art, const std::string& kernel, const Json** op_out) {
  const Json* ks = art.get("kernels");
  if (ks == nullptr || ks->kind != Json::kArr) return "";
  for (const Json& k : ks->arr) {
    if (k.str_or("name", "") != kernel) continue;
    const Json* body = k.get("body");
    if (body == nullptr || body->kind != Json::kArr || body->arr.size() != 2) return "";
    if (body->arr[1].str_or("op", "") != "return") return "";
    if (op_out != nullptr) *op_out = &body->arr[0];
    return body->arr[0].str_or("op", "");
  }
  return "";
}

// Symbolic values of the family-(a) encoder graph, tracked through the steps.
struct Sym {
  enum Kind {
    kNone, kTokens, kMask, kParam, kEmbQ, kX, kLin, kLinT, kScores, kProbs, kMixed, kAtt, kRes1,
    kH1, kUp, kAct, kDown, kRes2, kNorm, kPooled
  } kind = kNone;
  int layer = 0;
  std::string a, b, c;  // parameter names the value depends on
};

struct LayerParams {
  std::string q, k, v, o, up, down;
};

struct PlanResult {
  EosHipMllPlan plan{};
  std::string token_param;
  std::vector<LayerParams> layers;
  // BERT family: the bert_embedder step's inputs (ids, mask, types, the five
  // embedding tensors, 16 per layer in the reference's order).
  std::vector<std::string> bert_inputs;
};

int plan_fail(char** err, const std::string& entry, size_t step, const char* fmt, const char* a = "",
              const char* b = "") {
  char msg[512];
  std::snprintf(msg, sizeof(msg), fmt, a, b);
  return set_err(err, "eoship_mll_classify: entry \"%s\" not handled at step %zu: %s", entry.c_str(),
                 step, msg);
}

// Copies a name into a fixed plan field; false when it does not fit (the
// classifiers refuse such names, so a plan never names a truncated value).
bool copy_name(char* dst, size_t cap, const std::string& s) {
  std::snprintf(dst, cap, "%s", s.c_str());
  return s.size() < cap;
}

// Go's strconv.Atoi: an optional sign and decimal digits, nothing else.
bool go_atoi(const std::string& s, long long* out) {
  size_t i = 0;
  if (i < s.size() && (s[i] == '+' || s[i] == '-')) ++i;
  if (i == s.size()) return false;
  for (size_t j = i; j < s.size(); ++j)
    if (s[j] < '0' || s[j] > '9') return false;
  if (s.size() - i > 18) return false;
  *out = std::strtoll(s.c_str(), nullptr, 10);
  return true;
}

// The bert_embedder step (one fused step of BERT embeddings, every encoder
// layer, pooling and L2, runtime/backend/bert_embedder_ops.go:10-197; the
// module the pretrained-BERT importer emits, runtime/pretrained_bert_importer.go:
// 901-1009): attributes as bertEmbedderConfigFromAttrs reads them, 8 + 16 L
// inputs (input_ids, attention_mask, token_type_ids entry inputs, then the
// five embedding tensors and 16 tensors per layer, all params), the one
// output returned. Shapes are those BERTEmbedderReferenceWithPooling and
// BERTEncoderLayerReference accept, and the fused encoder's own limits.
int classify_bert(const EosHipMll* m, const Json& art, const std::string& entry, const Json& ep,
                  PlanResult* out, char** err) {
  auto fail = [&](size_t step, const std::string& msg) {
    return plan_fail(err, entry, step, "%s", msg.c_str());
  };
  const Json* steps = art.get("steps");
  const Json* bstep = nullptr;
  size_t bi = 0, nsteps = 0;
  std::string result;
  bool returned = false;
  for (size_t i = 0; i < steps->arr.size(); ++i) {
    const Json& st = steps->arr[i];
    if (st.str_or("entry", "") != entry) continue;
    ++nsteps;
    const std::string kind = st.str_or("kind", "");
    if (returned) return fail(i, "steps after return");
    if (kind == "bert_embedder") {
      if (bstep != nullptr) return fail(i, "a second bert_embedder step");
      bstep = &st;
      bi = i;
      const Json* o = st.get("outputs");
      if (o == nullptr || o->kind != Json::kArr || o->arr.size() != 1)
        return fail(i, "bert_embedder step expects 1 output");
      result = o->arr[0].str;
    } else if (kind == "return") {
      const Json* o = st.get("outputs");
      if (bstep == nullptr || o == nullptr || o->kind != Json::kArr || o->arr.size() != 1 ||
          o->arr[0].str != result)
        return fail(i, "return of something other than the bert_embedder output");
      returned = true;
    } else {
      return fail(i, "step kind \"" + kind + "\" beside a bert_embedder step");
    }
  }
  if (!returned) return set_err(err, "eoship_mll_classify: entry \"%s\" has no return step", entry.c_str());
  // Attributes (bertEmbedderConfigFromAttrs, bert_embedder_ops.go:35-77).
  long long layers = 1, heads = 1;
  double eps = 1e-12;
  std::string act = "gelu", pooling = "masked_mean";
  if (const Json* at = bstep->get("attributes")) {
    if (at->kind != Json::kObj) return fail(bi, "attributes are not an object");
    for (const auto& kv : at->obj) {
      if (kv.second.kind != Json::kStr) return fail(bi, "attribute \"" + kv.first + "\" is not a string");
      const std::string& v = kv.second.str;
      if (v.empty()) continue;
      if (kv.first == "num_hidden_layers") {
        if (!go_atoi(v, &layers) || layers <= 0)
          return fail(bi, "bert_embedder num_hidden_layers \"" + v + "\" is invalid");
      } else if (kv.first == "num_attention_heads") {
        if (!go_atoi(v, &heads) || heads <= 0)
          return fail(bi, "bert_embedder num_attention_heads \"" + v + "\" is invalid");
      } else if (kv.first == "epsilon") {
        char* end = nullptr;
        eps = std::strtod(v.c_str(), &end);
        if (end == v.c_str() || *end != 0) return fail(bi, "bert_embedder epsilon \"" + v + "\" is invalid");
        if (eps < 0) return fail(bi, "bert_embedder epsilon must be non-negative");
        if (!std::isfinite(eps)) return fail(bi, "bert_embedder epsilon is not finite");
      } else if (kv.first == "hidden_act") {
        act = v;
      } else if (kv.first == "pooling") {
        pooling = v;
      }
    }
  }
  if (act != "gelu")
    return fail(bi, "bert_embedder unsupported hidden_act \"" + act + "\"; only gelu is supported");
  if (pooling != "masked_mean" && pooling != "cls")
    return fail(bi, "bert_embedder unsupported pooling \"" + pooling +
                        "\"; supported values are masked_mean and cls");
  std::vector<std::string> in;
  if (const Json* a = bstep->get("inputs"))
    for (const Json& x : a->arr) in.push_back(x.str);
  if (layers > 4096 || (long long)in.size() != 8 + 16 * layers) {
    char msg[160];
    std::snprintf(msg, sizeof(msg), "bert_embedder expects %lld tensors for %lld layers, got %zu",
                  8 + 16 * layers, layers, in.size());
    return fail(bi, msg);
  }
  // input_ids, attention_mask, token_type_ids: the entry's i32 [B, T] inputs.
  const Json* eins = ep.get("inputs");
  for (int k = 0; k < 3; ++k) {
    const Json* found = nullptr;
    if (eins != nullptr && eins->kind == Json::kArr)
      for (const Json& e : eins->arr)
        if (e.str_or("name", "") == in[k]) found = &e;
    const Json* ty = found != nullptr ? found->get("type") : nullptr;
    const Json* tt = ty != nullptr ? ty->get("tensor") : nullptr;
    const Json* shape = tt != nullptr ? tt->get("shape") : nullptr;
    if (tt == nullptr || tt->str_or("dtype", "") != "i32" || shape == nullptr ||
        shape->kind != Json::kArr || shape->arr.size() != 2)
      return fail(bi, "bert_embedder input \"" + in[k] + "\" is not an i32 [B, T] entry input");
  }
  // Tensors: the payload of every other input, of the shape the reference
  // validates (validateBERTEmbeddingTables, validateBERTLayerNormParam, the
  // per-layer checks of BERTEncoderLayerReference).
  auto tensor = [&](const std::string& n, const Tensor** t) -> bool {
    *t = m->tensor(n);
    return *t != nullptr && ((*t)->kind == EOSHIP_MLL_F32 || (*t)->kind == EOSHIP_MLL_F16 ||
                             (*t)->kind == EOSHIP_MLL_Q8 || (*t)->kind == EOSHIP_MLL_Q4);
  };
  const Tensor *tok = nullptr, *pos = nullptr, *typ = nullptr, *g = nullptr, *be = nullptr;
  if (!tensor(in[3], &tok) || !tensor(in[4], &pos) || !tensor(in[5], &typ) || !tensor(in[6], &g) ||
      !tensor(in[7], &be))
    return fail(bi, "an embedding tensor is missing or not f32, f16, q8 or q4");
  if (tok->dims.size() != 2 || pos->dims.size() != 2 || typ->dims.size() != 2)
    return fail(bi, "embedding tables must be rank 2");
  const int64_t H = tok->dims[1];
  if (pos->dims[1] != H || typ->dims[1] != H)
    return fail(bi, "embedding tables differ in width");
  if (g->dims.size() != 1 || g->dims[0] != H || be->dims.size() != 1 || be->dims[0] != H)
    return fail(bi, "embedding layernorm parameters must be [hidden]");
  if (H % heads != 0) return fail(bi, "hidden size is not a multiple of num_attention_heads");
  int64_t F = -1;
  for (long long l = 0; l < layers; ++l) {
    const std::string* w = &in[8 + 16 * l];
    const Tensor* t[16];
    for (int k = 0; k < 16; ++k)
      if (!tensor(w[k], &t[k])) return fail(bi, "layer tensor \"" + w[k] + "\" is missing or not f32, f16, q8 or q4");
    if (F < 0 && t[10]->dims.size() == 2) F = t[10]->dims[0];
    auto is = [](const Tensor* x, int64_t a, int64_t b) {
      return b < 0 ? (x->dims.size() == 1 && x->dims[0] == a)
                   : (x->dims.size() == 2 && x->dims[0] == a && x->dims[1] == b);
    };
    const bool ok = is(t[0], H, H) && is(t[1], H, -1) && is(t[2], H, H) && is(t[3], H, -1) &&
                    is(t[4], H, H) && is(t[5], H, -1) && is(t[6], H, H) && is(t[7], H, -1) &&
                    is(t[8], H, -1) && is(t[9], H, -1) && is(t[10], F, H) && is(t[11], F, -1) &&
                    is(t[12], H, F) && is(t[13], H, -1) && is(t[14], H, -1) && is(t[15], H, -1);
    if (!ok) {
      char msg[96];
      std::snprintf(msg, sizeof(msg), "layer %lld tensor shapes do not match hidden %lld", l,
                    (long long)H);
      return fail(bi, msg);
    }
  }
  // What the encoder binds: the MFMA kernels' shapes, or the general-shape
  // (f32) kernels' (hidden a multiple of 8 up to 1024, head dim up to 64,
  // intermediate up to 16384).
  const int64_t hd = H / heads;
  const bool mfma_shape = (H == 128 || H == 256 || H == 384 || H == 512 || H == 768) &&
                          (hd == 32 || hd == 64 || hd == 128 || hd == 256) && F > 0 &&
                          F % 128 == 0;
  const bool general_shape = H >= 8 && H <= 1024 && H % 8 == 0 && hd <= 64 && F > 0 &&
                             F <= 16384;
  if ((!mfma_shape && !general_shape) || tok->dims[0] > (1ll << 30) || pos->dims[0] > 65536 ||
      typ->dims[0] > 65536) {
    char msg[200];
    std::snprintf(msg, sizeof(msg),
                  "hidden %lld, head dim %lld, intermediate %lld outside the encoder (hidden "
                  "128/256/384/512/768 with head dim 32/64/128/256 and intermediate a multiple of "
                  "128, or hidden a multiple of 8 up to 1024 with head dim up to 64)",
                  (long long)H, (long long)hd, (long long)F);
    return fail(bi, msg);
  }
  PlanResult r;
  EosHipMllPlan& p = r.plan;
  p.route = EOSHIP_PLAN_BERT_EMBEDDER;
  p.layers = (int32_t)layers;
  p.distinct_layers = (int32_t)layers;
  p.model_dim = (int32_t)H;
  p.heads = (int32_t)heads;
  p.hidden_dim = (int32_t)F;
  p.vocab = (int32_t)tok->dims[0];
  p.max_sequence = (int32_t)pos->dims[0];
  p.output_dim = (int32_t)H;
  p.batched = 1;
  p.steps = (int32_t)nsteps;
  p.pooling = pooling == "cls" ? 1 : 0;
  p.ln_eps = eps;
  p.type_vocab = (int32_t)typ->dims[0];
  bool quantize = false;
  for (long long l = 0; l < layers; ++l)
    for (int k : {0, 2, 4, 6, 10, 12}) {
      const Tensor* t = m->tensor(in[8 + 16 * l + k]);
      quantize = quantize || t->kind == EOSHIP_MLL_F32 || t->kind == EOSHIP_MLL_F16;
    }
  p.weights_quantized = quantize ? 1 : 0;
  if (!copy_name(p.entry, sizeof(p.entry), entry) ||
      !copy_name(p.token_input, sizeof(p.token_input), in[0]) ||
      !copy_name(p.mask_input, sizeof(p.mask_input), in[1]) ||
      !copy_name(p.type_input, sizeof(p.type_input), in[2]) ||
      !copy_name(p.output_name, sizeof(p.output_name), result))
    return set_err(err, "eoship_mll_classify: an entry, input or output name of %zu bytes or more",
                   sizeof(p.entry));
  r.bert_inputs = in;
  *out = std::move(r);
  return 0;
}

int classify(const EosHipMll* m, const char* entry_name, PlanResult* out, char** err) {
  if (!m->has_meta) return set_err(err, "eoship_mll_classify: the package has no XMTA metadata");
  const Json& art = *m->meta.get("artifact");
  const Json* files = m->meta.get("json_files");
  const Json* man = files != nullptr ? files->get("embedding_manifest") : nullptr;
  std::string entry;
  if (entry_name != nullptr && entry_name[0] != 0) {
    entry = entry_name;
  } else if (man != nullptr) {
    entry = man->str_or("batch_entry", "");
    if (entry.empty()) entry = man->str_or("pooled_entry", "");
  }
  const Json* eps = art.get("entry_points");
  if (entry.empty() && eps != nullptr && eps->kind == Json::kArr && eps->arr.size() == 1)
    entry = eps->arr[0].str_or("name", "");
  if (entry.empty())
    return set_err(err, "eoship_mll_classify: no entry named and no embedding_manifest entry");
  const Json* ep = nullptr;
  if (eps != nullptr && eps->kind == Json::kArr)
    for (const Json& e : eps->arr)
      if (e.str_or("name", "") == entry) ep = &e;
  if (ep == nullptr) return set_err(err, "eoship_mll_classify: unknown entrypoint \"%s\"", entry.c_str());
  if (const Json* all = art.get("steps"))
    if (all->kind == Json::kArr)
      for (const Json& st : all->arr)
        if (st.str_or("entry", "") == entry && st.str_or("kind", "") == "bert_embedder")
          return classify_bert(m, art, entry, *ep, out, err);
  const Json* ins = ep->get("inputs");
  const Json* outs = ep->get("outputs");
  if (ins == nullptr || ins->kind != Json::kArr || ins->arr.size() != 2 || outs == nullptr ||
      outs->kind != Json::kArr || outs->arr.size() != 1)
    return set_err(err, "eoship_mll_classify: entry \"%s\" not handled: want inputs (tokens, mask) and one output",
                   entry.c_str());
  std::string tok_in = man != nullptr ? man->str_or("token_input", "") : "";
  std::string mask_in = man != nullptr ? man->str_or("mask_input", "") : "";
  if (tok_in.empty()) tok_in = ins->arr[0].str_or("name", "");
  if (mask_in.empty()) mask_in = ins->arr[1].str_or("name", "");
  int batched = -1;
  for (const Json& in : ins->arr) {
    const Json* ty = in.get("type");
    const Json* tt = ty != nullptr ? ty->get("tensor") : nullptr;
    const Json* shape = tt != nullptr ? tt->get("shape") : nullptr;
    if (tt == nullptr || tt->str_or("dtype", "") != "i32" || shape == nullptr ||
        shape->kind != Json::kArr || shape->arr.empty() || shape->arr.size() > 2)
      return set_err(err, "eoship_mll_classify: entry \"%s\" input \"%s\" is not an i32 [T] or [B, T] tensor",
                     entry.c_str(), in.str_or("name", "").c_str());
    const int b = shape->arr.size() == 2 ? 1 : 0;
    if (batched >= 0 && batched != b)
      return set_err(err, "eoship_mll_classify: entry \"%s\" inputs differ in rank", entry.c_str());
    batched = b;
    const std::string nm = in.str_or("name", "");
    if (nm != tok_in && nm != mask_in)
      return set_err(err, "eoship_mll_classify: entry \"%s\" input \"%s\" is neither tokens nor mask",
                     entry.c_str(), nm.c_str());
  }
  std::vector<std::pair<std::string, Sym>> env;
  auto find = [&](const std::string& n) -> Sym* {
    for (auto& kv : env)
      if (kv.first == n) return &kv.second;
    return nullptr;
  };
  auto set = [&](const std::string& n, const Sym& s) {
    if (Sym* o = find(n)) *o = s;
    else env.emplace_back(n, s);
  };
  {
    Sym t;
    t.kind = Sym::kTokens;
    set(tok_in, t);
    Sym mk;
    mk.kind = Sym::kMask;
    set(mask_in, mk);
  }
  auto is_param = [&](const std::string& n) {
    const Json* ps = art.get("params");
    if (ps == nullptr || ps->kind != Json::kArr) return false;
    for (const Json& p : ps->arr)
      if (p.str_or("name", "") == n) return true;
    return false;
  };
  auto value = [&](const std::string& n) -> Sym {
    if (Sym* s = find(n)) return *s;
    Sym p;
    if (is_param(n)) {
      p.kind = Sym::kParam;
      p.a = n;
    }
    return p;
  };
  PlanResult r;
  int layer = 0;
  bool scaled = false, key_masked = false, have_scale_form = false, have_mask_form = false;
  std::string result_name;
  size_t nsteps = 0;
  const Json* steps = art.get("steps");
  if (steps == nullptr || steps->kind != Json::kArr)
    return set_err(err, "eoship_mll_classify: the artifact has no steps");
  bool returned = false;
  for (size_t i = 0; i < steps->arr.size(); ++i) {
    const Json& st = steps->arr[i];
    if (st.str_or("entry", "") != entry) continue;
    ++nsteps;
    if (returned) return plan_fail(err, entry, i, "steps after return");
    const std::string kind = st.str_or("kind", "");
    std::vector<std::string> in, outn;
    if (const Json* a = st.get("inputs"))
      for (const Json& x : a->arr) in.push_back(x.str);
    if (const Json* a = st.get("outputs"))
      for (const Json& x : a->arr) outn.push_back(x.str);
    const Json* attrs = st.get("attributes");
    const bool no_attrs = attrs == nullptr || (attrs->kind == Json::kObj && attrs->obj.empty());
    if (kind == "return") {
      if (outn.size() != 1 || value(outn[0]).kind != Sym::kPooled)
        return plan_fail(err, entry, i, "return of something other than the pooled embedding");
      result_name = outn[0];
      returned = true;
      continue;
    }
    if (outn.size() != 1) return plan_fail(err, entry, i, "%s step with %s outputs", kind.c_str(), "several");
    Sym o;
    std::vector<Sym> v;
    for (const std::string& x : in) v.push_back(value(x));
    if (kind == "gather") {
      // The compiler marks the [B, T] token gather mode "shared".
      const bool shared = attrs != nullptr && attrs->kind == Json::kObj &&
                          attrs->obj.size() == 1 && attrs->str_or("mode", "") == "shared";
      if (v.size() != 2 || v[0].kind != Sym::kParam || v[1].kind != Sym::kTokens ||
          !(no_attrs || shared))
        return plan_fail(err, entry, i, "gather of something other than (param, tokens)");
      o.kind = Sym::kEmbQ;
      o.a = v[0].a;
    } else if (kind == "dequant") {
      if (v.size() != 1 || !no_attrs) return plan_fail(err, entry, i, "dequant with %s inputs", "several");
      if (v[0].kind == Sym::kParam) {
        o = v[0];  // a dtype relabel (tensor_ops.go:225-237)
      } else if (v[0].kind == Sym::kEmbQ) {
        if (layer != 0 || !r.token_param.empty())
          return plan_fail(err, entry, i, "a second token embedding");
        r.token_param = v[0].a;
        o.kind = Sym::kX;
        o.layer = 0;
      } else {
        return plan_fail(err, entry, i, "dequant of an intermediate value");
      }
    } else if (kind == "transpose") {
      if (v.size() != 1 || v[0].kind != Sym::kLin || !no_attrs)
        return plan_fail(err, entry, i, "transpose of something other than a projection");
      o = v[0];
      o.kind = Sym::kLinT;
    } else if (kind == "matmul") {
      if (v.size() != 2) return plan_fail(err, entry, i, "matmul with %s inputs", "other than 2");
      std::string sc;
      if (!no_attrs) {
        if (attrs->kind != Json::kObj || attrs->obj.size() != 1 || attrs->get_str("scale") == nullptr)
          return plan_fail(err, entry, i, "matmul attributes other than scale");
        sc = *attrs->get_str("scale");
        if (sc == "none") sc.clear();
      }
      const Sym &x = v[0], &w = v[1];
      if (!sc.empty() && !(x.kind == Sym::kLin && w.kind == Sym::kLinT))
        return plan_fail(err, entry, i, "a scaled matmul outside the attention scores");
      if (x.kind == Sym::kX && w.kind == Sym::kParam && x.layer == layer) {
        o.kind = Sym::kLin;
        o.layer = layer;
        o.a = w.a;
      } else if (x.kind == Sym::kLin && w.kind == Sym::kLinT && x.layer == layer && w.layer == layer) {
        if (sc.empty()) {
          if (have_scale_form && scaled) return plan_fail(err, entry, i, "layers differ in score scaling");
          scaled = false;
        } else if (sc == "rsqrt_rhs_rows") {
          if (have_scale_form && !scaled) return plan_fail(err, entry, i, "layers differ in score scaling");
          scaled = true;  // 1/sqrt(rows of kT) = 1/sqrt(D) (tensor_ops.go:1291-1304)
        } else {
          return plan_fail(err, entry, i, "matmul scale \"%s\" not handled", sc.c_str());
        }
        have_scale_form = true;
        o.kind = Sym::kScores;
        o.layer = layer;
        o.a = x.a;
        o.b = w.a;
      } else if (x.kind == Sym::kProbs && w.kind == Sym::kLin && x.layer == layer && w.layer == layer) {
        o = x;
        o.kind = Sym::kMixed;
        o.c = w.a;
      } else if (x.kind == Sym::kMixed && w.kind == Sym::kParam) {
        if (r.layers.size() != (size_t)layer) return plan_fail(err, entry, i, "layer bookkeeping");
        LayerParams lp;
        lp.q = x.a;
        lp.k = x.b;
        lp.v = x.c;
        lp.o = w.a;
        r.layers.push_back(lp);
        o.kind = Sym::kAtt;
        o.layer = layer;
      } else if (x.kind == Sym::kH1 && w.kind == Sym::kParam && x.layer == layer) {
        r.layers[(size_t)layer].up = w.a;
        o.kind = Sym::kUp;
        o.layer = layer;
      } else if (x.kind == Sym::kAct && w.kind == Sym::kParam && x.layer == layer) {
        r.layers[(size_t)layer].down = w.a;
        o.kind = Sym::kDown;
        o.layer = layer;
      } else {
        return plan_fail(err, entry, i, "matmul of operands outside the encoder graph (%s x %s)",
                         in[0].c_str(), in[1].c_str());
      }
      if (o.kind == Sym::kLin && (r.layers.size() > (size_t)layer))
        return plan_fail(err, entry, i, "projection after the layer's attention");
    } else if (kind == "launch_kernel") {
      const Json* op = nullptr;
      const std::string cls = kernel_op(art, st.str_or("kernel", ""), &op);
      const Json* oattrs = op != nullptr ? op->get("attributes") : nullptr;
      if (cls == "softmax") {
        if (v.size() != 1 || v[0].kind != Sym::kScores || v[0].layer != layer)
          return plan_fail(err, entry, i, "softmax of something other than the scores");
        if (oattrs != nullptr && oattrs->kind == Json::kObj) {
          const std::string ax = oattrs->str_or("axis", "-1");
          if (ax != "-1") return plan_fail(err, entry, i, "softmax over axis %s", ax.c_str());
        }
        if (have_mask_form && key_masked) return plan_fail(err, entry, i, "layers differ in key masking");
        have_mask_form = true;
        key_masked = false;
        o = v[0];
        o.kind = Sym::kProbs;
      } else if (cls == "masked_softmax") {
        if (v.size() != 2 || v[0].kind != Sym::kScores || v[1].kind != Sym::kMask || v[0].layer != layer)
          return plan_fail(err, entry, i, "masked_softmax of something other than (scores, mask)");
        if (have_mask_form && !key_masked) return plan_fail(err, entry, i, "layers differ in key masking");
        have_mask_form = true;
        key_masked = true;
        o = v[0];
        o.kind = Sym::kProbs;
      } else if (cls == "binary_add") {
        if (oattrs != nullptr && oattrs->kind == Json::kObj && oattrs->str_or("operator", "+") != "+")
          return plan_fail(err, entry, i, "binary_add with another operator");
        if (v.size() != 2) return plan_fail(err, entry, i, "binary_add with %s inputs", "other than 2");
        // f32 addition commutes: either operand order is the same sum.
        auto pair_is = [&](Sym::Kind a, Sym::Kind b) {
          return (v[0].kind == a && v[1].kind == b) || (v[0].kind == b && v[1].kind == a);
        };
        if (pair_is(Sym::kAtt, Sym::kX) && v[0].layer == layer && v[1].layer == layer) {
          o.kind = Sym::kRes1;
        } else if (pair_is(Sym::kDown, Sym::kH1) && v[0].layer == layer && v[1].layer == layer) {
          o.kind = Sym::kRes2;
        } else {
          return plan_fail(err, entry, i, "residual add of operands outside the encoder graph");
        }
        o.layer = layer;
      } else if (cls == "layernorm") {
        if (v.size() != 1 || v[0].layer != layer ||
            (v[0].kind != Sym::kRes1 && v[0].kind != Sym::kRes2))
          return plan_fail(err, entry, i, "layernorm of something other than a residual sum");
        if (v[0].kind == Sym::kRes1) {
          o.kind = Sym::kH1;
          o.layer = layer;
        } else {
          ++layer;
          o.kind = Sym::kX;
          o.layer = layer;
        }
      } else if (cls == "gelu") {
        if (v.size() != 1 || v[0].kind != Sym::kUp || v[0].layer != layer)
          return plan_fail(err, entry, i, "gelu of something other than the FFN up projection");
        o.kind = Sym::kAct;
        o.layer = layer;
      } else if (cls == "normalize") {
        if (v.size() != 1 || v[0].kind != Sym::kX || v[0].layer != layer || layer == 0)
          return plan_fail(err, entry, i, "normalize of something other than the last layer's output");
        o.kind = Sym::kNorm;
      } else if (cls == "mean_pool") {
        if (v.size() != 2 || v[0].kind != Sym::kNorm || v[1].kind != Sym::kMask)
          return plan_fail(err, entry, i, "mean_pool of something other than (normalized, mask)");
        o.kind = Sym::kPooled;
      } else {
        return plan_fail(err, entry, i, "kernel \"%s\" (op class \"%s\") not handled",
                         st.str_or("kernel", "").c_str(), cls.c_str());
      }
    } else {
      return plan_fail(err, entry, i, "step kind \"%s\" not handled", kind.c_str());
    }
    set(outn[0], o);
  }
  if (!returned) return set_err(err, "eoship_mll_classify: entry \"%s\" has no return step", entry.c_str());
  if (layer == 0 || r.token_param.empty() || (size_t)layer != r.layers.size())
    return set_err(err, "eoship_mll_classify: entry \"%s\" has no complete encoder layer", entry.c_str());
  // Shapes from the payloads.
  const Tensor* tok = m->tensor(r.token_param);
  if (tok == nullptr || tok->dims.size() != 2)
    return set_err(err, "eoship_mll_classify: token embedding \"%s\" missing or not rank 2",
                   r.token_param.c_str());
  const int64_t V = tok->dims[0], D = tok->dims[1];
  int64_t F = -1;
  auto check = [&](const std::string& name, int64_t rows, int64_t cols, char** e) {
    const Tensor* t = m->tensor(name);
    if (t == nullptr) return set_err(e, "eoship_mll_classify: weight \"%s\" has no payload", name.c_str());
    if (t->dims.size() != 2 || t->dims[0] != rows || (cols >= 0 && t->dims[1] != cols))
      return set_err(e, "eoship_mll_classify: weight \"%s\" has shape [%lld, %lld], want [%lld, %lld]",
                     name.c_str(), (long long)(t->dims.size() > 0 ? t->dims[0] : 0),
                     (long long)(t->dims.size() > 1 ? t->dims[1] : 0), (long long)rows, (long long)cols);
    if (t->kind != EOSHIP_MLL_Q8 && t->kind != EOSHIP_MLL_Q4)
      return set_err(e, "eoship_mll_classify: weight \"%s\" is not packed q8/q4 (the fused encoder binds int8 codes)",
                     name.c_str());
    return 0;
  };
  if (check(r.token_param, V, D, err)) return 1;
  for (const LayerParams& lp : r.layers) {
    if (lp.up.empty() || lp.down.empty())
      return set_err(err, "eoship_mll_classify: entry \"%s\" has a layer without its FFN", entry.c_str());
    const Tensor* up = m->tensor(lp.up);
    if (up == nullptr || up->dims.size() != 2)
      return set_err(err, "eoship_mll_classify: weight \"%s\" missing", lp.up.c_str());
    if (F < 0) F = up->dims[1];
    if (check(lp.q, D, D, err) || check(lp.k, D, D, err) || check(lp.v, D, D, err) ||
        check(lp.o, D, D, err) || check(lp.up, D, F, err) || check(lp.down, F, D, err))
      return 1;
  }
  EosHipMllPlan& p = r.plan;
  p.route = EOSHIP_PLAN_COMPACT_EMBEDDER;
  p.layers = (int32_t)r.layers.size();
  p.model_dim = (int32_t)D;
  p.heads = 1;
  p.hidden_dim = (int32_t)F;
  p.vocab = (int32_t)V;
  p.max_sequence = 0;
  if (man != nullptr)
    if (const Json* tk = man->get("tokenizer"))
      if (const Json* ms = tk->get("max_sequence")) {
        // A finite integer in 1..8192 (it sizes the bind-time RoPE table).
        const double v = ms->num;
        if (ms->kind != Json::kNum || !(v >= 1.0 && v <= 8192.0) || v != std::floor(v))
          return set_err(err, "eoship_mll_classify: tokenizer.max_sequence must be an integer in "
                              "1..8192");
        p.max_sequence = (int32_t)v;
      }
  if (p.max_sequence <= 0) p.max_sequence = 512;
  p.output_dim = (int32_t)D;
  p.batched = batched;
  p.steps = (int32_t)nsteps;
  int distinct = 0;
  for (size_t l = 0; l < r.layers.size(); ++l) {
    bool seen = false;
    for (size_t j = 0; j < l; ++j) {
      const LayerParams &a = r.layers[l], &b = r.layers[j];
      seen = seen || (a.q == b.q && a.k == b.k && a.v == b.v && a.o == b.o && a.up == b.up &&
                      a.down == b.down);
    }
    distinct += seen ? 0 : 1;
  }
  p.distinct_layers = distinct;
  p.options.rope = 0;
  p.options.role = 0;
  p.options.scaled_scores = scaled ? 1 : 0;
  p.options.attend_padding = key_masked ? 0 : 1;
  if (!copy_name(p.entry, sizeof(p.entry), entry) ||
      !copy_name(p.token_input, sizeof(p.token_input), tok_in) ||
      !copy_name(p.mask_input, sizeof(p.mask_input), mask_in) ||
      !copy_name(p.output_name, sizeof(p.output_name), result_name))
    return set_err(err, "eoship_mll_classify: an entry, input or output name of %zu bytes or more",
                   sizeof(p.entry));
  *out = std::move(r);
  return 0;
}

// int8 codes of a packed Q8 or Q4 payload (Q4: nibble - 8).
std::vector<int8_t> codes_of(const EosHipMll* m, const Tensor& t) {
  std::vector<int8_t> c((size_t)t.elements);
  const uint8_t* b = m->bytes.data() + t.off;
  if (t.kind == EOSHIP_MLL_Q8) {
    std::memcpy(c.data(), b, c.size());
  } else {
    for (size_t k = 0; k < c.size(); ++k) c[k] = (int8_t)(((b[k / 2] >> (4 * (k & 1))) & 0xF) - 8);
  }
  return c;
}

// Retrieval plans: score step, topk, gathers, pack_candidates, return.
int classify_retrieval(const EosHipMll* m, const char* entry_name, EosHipRetrievalPlan* out,
                       char** err) {
  const char* what = "eoship_mll_classify_retrieval";
  if (!m->has_meta) return set_err(err, "%s: the package has no XMTA metadata", what);
  const Json& art = *m->meta.get("artifact");
  const Json* eps = art.get("entry_points");
  const Json* ep = nullptr;
  std::string entry = entry_name != nullptr ? entry_name : "";
  if (eps != nullptr && eps->kind == Json::kArr) {
    if (entry.empty() && eps->arr.size() == 1) entry = eps->arr[0].str_or("name", "");
    for (const Json& e : eps->arr)
      if (e.str_or("name", "") == entry) ep = &e;
  }
  if (ep == nullptr) return set_err(err, "%s: unknown entrypoint \"%s\"", what, entry.c_str());
  struct In {
    std::string name, dtype;
    size_t rank;
  };
  std::vector<In> inputs;
  if (const Json* ins = ep->get("inputs"))
    for (const Json& in : ins->arr) {
      const Json* ty = in.get("type");
      const Json* tt = ty != nullptr ? ty->get("tensor") : nullptr;
      const Json* shape = tt != nullptr ? tt->get("shape") : nullptr;
      inputs.push_back({in.str_or("name", ""), tt != nullptr ? tt->str_or("dtype", "") : "",
                        shape != nullptr && shape->kind == Json::kArr ? shape->arr.size() : 0});
    }
  auto input = [&](const std::string& n) -> const In* {
    for (const In& i : inputs)
      if (i.name == n) return &i;
    return nullptr;
  };
  auto is_param = [&](const std::string& n) {
    const Json* ps = art.get("params");
    if (ps == nullptr || ps->kind != Json::kArr) return false;
    for (const Json& p : ps->arr)
      if (p.str_or("name", "") == n) return true;
    return false;
  };
  enum Kind { kNone, kQuery, kDocs, kIds, kScores, kIdx, kTopIds, kTopScores, kTopDocs, kPack };
  std::vector<std::pair<std::string, int>> env;
  auto kind_of = [&](const std::string& n) {
    for (auto& kv : env)
      if (kv.first == n) return kv.second;
    return (int)kNone;
  };
  EosHipRetrievalPlan p{};
  std::string query, docs, ids;
  const Json* steps = art.get("steps");
  if (steps == nullptr || steps->kind != Json::kArr)
    return set_err(err, "%s: the artifact has no steps", what);
  bool returned = false, have_score = false, packed = false;
  int nsteps = 0;
  auto fail = [&](size_t i, const std::string& msg) {
    return set_err(err, "%s: entry \"%s\" not handled at step %zu: %s", what, entry.c_str(), i,
                   msg.c_str());
  };
  for (size_t i = 0; i < steps->arr.size(); ++i) {
    const Json& st = steps->arr[i];
    if (st.str_or("entry", "") != entry) continue;
    ++nsteps;
    if (returned) return fail(i, "steps after return");
    const std::string kind = st.str_or("kind", "");
    std::vector<std::string> in, outn;
    if (const Json* a = st.get("inputs"))
      for (const Json& x : a->arr) in.push_back(x.str);
    if (const Json* a = st.get("outputs"))
      for (const Json& x : a->arr) outn.push_back(x.str);
    const Json* attrs = st.get("attributes");
    if (kind == "return") {
      if (outn.empty() || outn.size() > 8) return fail(i, "return of no or too many values");
      for (const std::string& o : outn) {
        const int k = kind_of(o);
        static const int kMap[] = {0, 0, 0, 0, EOSHIP_RET_SCORES, EOSHIP_RET_TOP_INDEX,
                                   EOSHIP_RET_TOP_IDS, EOSHIP_RET_TOP_SCORES, EOSHIP_RET_TOP_DOCS,
                                   EOSHIP_RET_PACK};
        if (kMap[k] == 0) return fail(i, "return of \"" + o + "\", not a plan result");
        p.outputs[p.n_outputs++] = kMap[k];
      }
      returned = true;
      continue;
    }
    if (outn.size() != 1) return fail(i, kind + " step without one output");
    int o = kNone;
    if (kind == "launch_kernel") {
      const std::string cls = kernel_op(art, st.str_or("kernel", ""), nullptr);
      const int op = cls == "dot" ? EOSHIP_SCORE_DOT
                     : cls == "cosine" ? EOSHIP_SCORE_COSINE
                     : cls == "l2_distance" ? EOSHIP_SCORE_L2 : 0;
      if (op == 0) return fail(i, "kernel op class \"" + cls + "\" not handled");
      if (have_score) return fail(i, "a second score step");
      if (in.size() != 2) return fail(i, "score step without (query, documents)");
      const In* qi = input(in[0]);
      if (qi == nullptr || (qi->rank != 1 && qi->rank != 2)) return fail(i, "query is not a [D] or [Q, D] input");
      const In* di = input(in[1]);
      const bool dparam = di == nullptr && is_param(in[1]);
      if (!dparam && (di == nullptr || di->rank != qi->rank + 1))
        return fail(i, "documents are not a [N, D] or [Q, N, D] input or param");
      if (dparam && qi->rank != 1) return fail(i, "param documents with batched queries");
      query = in[0];
      docs = in[1];
      p.op = op;
      p.batched = qi->rank == 2 ? 1 : 0;
      p.docs_param = dparam ? 1 : 0;
      env.emplace_back(query, (int)kQuery);
      env.emplace_back(docs, (int)kDocs);
      have_score = true;
      o = kScores;
    } else if (kind == "topk") {
      if (in.size() != 1 || kind_of(in[0]) != kScores) return fail(i, "topk of something other than the scores");
      const std::string* kk = attrs != nullptr ? attrs->get_str("k") : nullptr;
      char* end = nullptr;
      const long k = kk != nullptr ? std::strtol(kk->c_str(), &end, 10) : 0;
      if (kk == nullptr || end == kk->c_str() || *end != 0 || k <= 0 || k > 8192)
        return fail(i, "topk limit missing or outside 1..8192");
      if (p.k != 0) return fail(i, "a second topk");
      p.k = (int32_t)k;
      o = kIdx;
    } else if (kind == "gather") {
      if (in.size() != 2 || kind_of(in[1]) != kIdx) return fail(i, "gather not indexed by the topk");
      if (attrs != nullptr && attrs->kind == Json::kObj && !attrs->obj.empty()) {
        const std::string mode = attrs->str_or("mode", "");
        if (attrs->obj.size() != 1 || mode != "batched" || !p.batched)
          return fail(i, "gather attributes other than the batched mode of batched plans");
      }
      const int src = kind_of(in[0]);
      if (src == kScores) {
        o = kTopScores;
      } else if (src == kDocs) {
        o = kTopDocs;
      } else if (src == kNone && input(in[0]) != nullptr && input(in[0])->dtype == "i64" &&
                 (ids.empty() || ids == in[0])) {
        ids = in[0];
        env.emplace_back(ids, (int)kIds);
        o = kTopIds;
      } else {
        return fail(i, "gather of \"" + in[0] + "\", not the scores, documents or i64 candidate ids");
      }
    } else if (kind == "pack_candidates") {
      if (in.size() != 3 || kind_of(in[0]) != kTopIds || kind_of(in[1]) != kTopScores ||
          kind_of(in[2]) != kTopDocs)
        return fail(i, "pack_candidates of something other than (ids, scores, docs) at the topk");
      packed = true;
      o = kPack;
    } else {
      return fail(i, "step kind \"" + kind + "\" not handled");
    }
    env.emplace_back(outn[0], o);
  }
  (void)packed;
  if (!returned) return set_err(err, "%s: entry \"%s\" has no return step", what, entry.c_str());
  if (!have_score) return set_err(err, "%s: entry \"%s\" has no score step", what, entry.c_str());
  p.has_candidate_ids = ids.empty() ? 0 : 1;
  if (p.docs_param) {
    const Tensor* t = m->tensor(docs);
    if (t == nullptr || t->dims.size() != 2)
      return set_err(err, "%s: document param \"%s\" has no [N, D] payload", what, docs.c_str());
    if (t->kind != EOSHIP_MLL_Q4 && t->kind != EOSHIP_MLL_Q8 && t->kind != EOSHIP_MLL_F32)
      return set_err(err, "%s: document param \"%s\" is not q4, q8 or f32", what, docs.c_str());
    if (t->dims[1] > 4096) return set_err(err, "%s: documents wider than 4096", what);
    p.docs_rows = t->dims[0];
    p.dim = (int32_t)t->dims[1];
    p.docs_q4 = t->kind == EOSHIP_MLL_Q4 ? 1 : 0;
  }
  p.steps = nsteps;
  if (!copy_name(p.entry, sizeof(p.entry), entry) ||
      !copy_name(p.query_input, sizeof(p.query_input), query) ||
      !copy_name(p.docs_input, sizeof(p.docs_input), docs) ||
      !copy_name(p.ids_input, sizeof(p.ids_input), ids))
    return set_err(err, "%s: an entry, input or param name of %zu bytes or more", what,
                   sizeof(p.entry));
  *out = p;
  return 0;
}

}  // namespace

extern "C" {

int eoship_mll_open(const uint8_t* data, uint64_t bytes, EosHipMll** out, char** err) {
  if (data == nullptr || out == nullptr) return set_err(err, "eoship_mll_open: NULL argument");
  *out = nullptr;
  auto* m = new EosHipMll();
  m->bytes.assign(data, data + bytes);
  if (parse_container(m, err) || parse_strings(m, err) || parse_meta(m, err) ||
      parse_tensors(m, err)) {
    delete m;
    return 1;
  }
  *out = m;
  return 0;
}

void eoship_mll_close(EosHipMll* m) { delete m; }

int eoship_mll_info(const EosHipMll* m, EosHipMllInfo* info, char** err) {
  if (m == nullptr || info == nullptr) return set_err(err, "eoship_mll_info: NULL argument");
  std::memset(info, 0, sizeof(*info));
  info->profile = m->profile;
  info->sections = (int32_t)m->sections.size();
  info->strings = (int64_t)m->strings.size();
  info->tensors = (int64_t)m->tensors.size();
  info->has_metadata = m->has_meta ? 1 : 0;
  if (m->has_meta) {
    copy_name(info->module_name, sizeof(info->module_name), m->meta.str_or("module_name", ""));
    copy_name(info->module_version, sizeof(info->module_version), m->meta.str_or("module_version", ""));
  }
  return 0;
}

int eoship_mll_section(const EosHipMll* m, const char* tag, const uint8_t** body, uint64_t* size,
                       char** err) {
  if (m == nullptr || tag == nullptr || body == nullptr || size == nullptr)
    return set_err(err, "eoship_mll_section: NULL argument");
  if (std::strlen(tag) != 4) return set_err(err, "eoship_mll_section: a tag has 4 characters");
  if (std::memcmp(tag, "XKBI", 4) == 0)
    return set_err(err, "eoship_mll_section: XKBI (offline kernel images) is never read");
  const Section* s = m->section(tag);
  if (s == nullptr) return set_err(err, "eoship_mll_section: no %s section", tag);
  *body = m->bytes.data() + s->off;
  *size = s->size;
  return 0;
}

int eoship_mll_tensor(const EosHipMll* m, int64_t index, const char* name, EosHipMllTensor* out,
                      char** err) {
  if (m == nullptr || out == nullptr) return set_err(err, "eoship_mll_tensor: NULL argument");
  const Tensor* t = nullptr;
  if (name != nullptr) {
    t = m->tensor(name);
    if (t == nullptr) return set_err(err, "eoship_mll_tensor: no tensor \"%s\"", name);
  } else {
    if (index < 0 || index >= (int64_t)m->tensors.size())
      return set_err(err, "eoship_mll_tensor: index %lld out of range", (long long)index);
    t = &m->tensors[(size_t)index];
  }
  std::memset(out, 0, sizeof(*out));
  out->name = t->name.c_str();
  out->kind = t->kind;
  out->storage_dtype = t->code;
  out->rank = (int32_t)t->dims.size();
  for (size_t r = 0; r < t->dims.size(); ++r) out->dims[r] = t->dims[r];
  out->elements = t->elements;
  out->data = m->bytes.data() + t->off;
  out->bytes = t->size;
  out->scale = t->scale;
  return 0;
}

int eoship_mll_classify(const EosHipMll* m, const char* entry, EosHipMllPlan* plan, char** err) {
  if (m == nullptr || plan == nullptr) return set_err(err, "eoship_mll_classify: NULL argument");
  PlanResult r;
  if (classify(m, entry, &r, err) != 0) return 1;
  *plan = r.plan;
  return 0;
}

}  // extern "C"

namespace {

float half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu, f = h & 0x3ffu;
  uint32_t bits;
  if (e == 0x1f) {
    bits = sign | 0x7f800000u | (f << 13);
  } else if (e != 0) {
    bits = sign | ((e + 112u) << 23) | (f << 13);
  } else if (f == 0) {
    bits = sign;
  } else {  // subnormal: f * 2^-24, exact in f32
    const float v = (float)f * 5.9604644775390625e-8f;
    std::memcpy(&bits, &v, 4);
    bits |= sign;
  }
  float out;
  std::memcpy(&out, &bits, 4);
  return out;
}

// f32 values of a tensor as the reference decodes it (q8: code * scale, q4:
// (nibble - 8) * scale, runtime/weight_file.go:315-351).
std::vector<float> values_of(const EosHipMll* m, const Tensor& t) {
  std::vector<float> v((size_t)t.elements);
  const uint8_t* b = m->bytes.data() + t.off;
  if (t.kind == EOSHIP_MLL_F32) {
    std::memcpy(v.data(), b, v.size() * 4);
  } else if (t.kind == EOSHIP_MLL_F16) {
    for (size_t i = 0; i < v.size(); ++i) {
      uint16_t h;
      std::memcpy(&h, b + 2 * i, 2);
      v[i] = half_to_float(h);
    }
  } else {
    const std::vector<int8_t> c = codes_of(m, t);
    const float sc = t.scale > 0.f ? t.scale : 0.f;
    for (size_t i = 0; i < v.size(); ++i) v[i] = (float)c[i] * sc;
  }
  return v;
}

// int8 codes [rows][cols] with one scale per row: a q8/q4 payload keeps its
// codes and per-tensor scale; f32/f16 values are quantized per row (output
// channel): scale = max|w| / 127, code = rint(w / scale) clamped to +-127.
void codes_per_row(const EosHipMll* m, const Tensor& t, std::vector<int8_t>* codes,
                   std::vector<float>* scales) {
  const int64_t rows = t.dims[0], cols = t.dims[1];
  if (t.kind == EOSHIP_MLL_Q8 || t.kind == EOSHIP_MLL_Q4) {
    *codes = codes_of(m, t);
    scales->assign((size_t)rows, t.scale > 0.f ? t.scale : 0.f);
    return;
  }
  const std::vector<float> v = values_of(m, t);
  codes->assign((size_t)(rows * cols), 0);
  scales->assign((size_t)rows, 0.f);
  for (int64_t r = 0; r < rows; ++r) {
    const float* w = v.data() + r * cols;
    float mx = 0.f;
    for (int64_t c = 0; c < cols; ++c) mx = std::max(mx, std::fabs(w[c]));
    const float sc = mx > 0.f ? mx / 127.0f : 0.f;
    (*scales)[(size_t)r] = sc;
    if (sc == 0.f) continue;
    for (int64_t c = 0; c < cols; ++c) {
      const float q = std::nearbyint(w[c] / sc);
      (*codes)[(size_t)(r * cols + c)] = (int8_t)std::max(-127.f, std::min(127.f, q));
    }
  }
}

// Binds a classified bert_embedder plan to the fused BERT encoder.
int bind_bert(EosHipRuntime* rt, const EosHipMll* m, const PlanResult& r, EosHipEncoder** out,
              char** err) {
  const EosHipMllPlan& p = r.plan;
  const std::vector<std::string>& in = r.bert_inputs;
  const int H = p.model_dim, F = p.hidden_dim;
  auto vals = [&](const std::string& n) { return values_of(m, *m->tensor(n)); };
  const std::vector<float> tok = vals(in[3]), pos = vals(in[4]), typ = vals(in[5]),
                           eg = vals(in[6]), eb = vals(in[7]);
  struct Layer {
    std::vector<int8_t> qkv, o, w1, w2;
    std::vector<float> sqkv, bqkv, so, bo, g1, b1, s1, bb1, s2, bb2, g2, b2;
  };
  std::vector<Layer> ls((size_t)p.layers);
  std::vector<EosHipEncoderLayer> desc_layers((size_t)p.layers);
  for (int l = 0; l < p.layers; ++l) {
    const std::string* w = &in[8 + 16 * (size_t)l];
    Layer& L = ls[(size_t)l];
    // Q, K, V stacked into one [3H][H] projection (rows: q, then k, then v).
    for (int part = 0; part < 3; ++part) {
      std::vector<int8_t> c;
      std::vector<float> sc;
      codes_per_row(m, *m->tensor(w[2 * part]), &c, &sc);
      L.qkv.insert(L.qkv.end(), c.begin(), c.end());
      L.sqkv.insert(L.sqkv.end(), sc.begin(), sc.end());
      const std::vector<float> bias = vals(w[2 * part + 1]);
      L.bqkv.insert(L.bqkv.end(), bias.begin(), bias.end());
    }
    codes_per_row(m, *m->tensor(w[6]), &L.o, &L.so);
    L.bo = vals(w[7]);
    L.g1 = vals(w[8]);
    L.b1 = vals(w[9]);
    codes_per_row(m, *m->tensor(w[10]), &L.w1, &L.s1);
    L.bb1 = vals(w[11]);
    codes_per_row(m, *m->tensor(w[12]), &L.w2, &L.s2);
    L.bb2 = vals(w[13]);
    L.g2 = vals(w[14]);
    L.b2 = vals(w[15]);
    EosHipEncoderLayer& d = desc_layers[(size_t)l];
    d.w_qkv = L.qkv.data();
    d.s_qkv = L.sqkv.data();
    d.b_qkv = L.bqkv.data();
    d.w_o = L.o.data();
    d.s_o = L.so.data();
    d.b_o = L.bo.data();
    d.ln1_gamma = L.g1.data();
    d.ln1_beta = L.b1.data();
    d.w_1 = L.w1.data();
    d.s_1 = L.s1.data();
    d.b_1 = L.bb1.data();
    d.w_2 = L.w2.data();
    d.s_2 = L.s2.data();
    d.b_2 = L.bb2.data();
    d.ln2_gamma = L.g2.data();
    d.ln2_beta = L.b2.data();
  }
  (void)F;
  EosHipEncoderDesc desc{};
  desc.layers = p.layers;
  desc.hidden = H;
  desc.heads = p.heads;
  desc.intermediate = p.hidden_dim;
  desc.vocab = p.vocab;
  desc.max_positions = p.max_sequence;
  desc.type_vocab = p.type_vocab;
  desc.ln_eps = (float)p.ln_eps;
  desc.gelu = 1;  // hidden_act "gelu": exactGELU, the erf form
  if (eoship_encoder_bind(rt, &desc, tok.data(), pos.data(), typ.data(), eg.data(), eb.data(),
                          desc_layers.data(), out, err) != 0)
    return 1;
  if (eoship_encoder_set_pooling(rt, *out, p.pooling, err) != 0) {
    eoship_encoder_release(*out, nullptr);
    *out = nullptr;
    return 1;
  }
  return 0;
}

}  // namespace

extern "C" {

int eoship_encoder_bind_mll(EosHipRuntime* rt, const EosHipMll* m, const char* entry,
                            int32_t attend_padding, EosHipEncoder** out, EosHipMllPlan* plan,
                            char** err) {
  if (rt == nullptr || m == nullptr || out == nullptr)
    return set_err(err, "eoship_encoder_bind_mll: NULL argument");
  *out = nullptr;
  if (attend_padding < -1 || attend_padding > 1)
    return set_err(err, "eoship_encoder_bind_mll: attend_padding must be -1, 0 or 1");
  PlanResult r;
  if (classify(m, entry, &r, err) != 0) return 1;
  if (r.plan.route == EOSHIP_PLAN_BERT_EMBEDDER) {
    if (attend_padding == 1)
      return set_err(err, "eoship_encoder_bind_mll: attend_padding 1 applies to the compact "
                          "family (BERT attention is masked)");
    if (bind_bert(rt, m, r, out, err) != 0) return 1;
    if (plan != nullptr) *plan = r.plan;
    return 0;
  }
  EosHipCompactOptions opts = r.plan.options;
  if (attend_padding >= 0) opts.attend_padding = attend_padding;
  EosHipCompactDesc desc{};
  desc.layers = r.plan.layers;
  desc.model_dim = r.plan.model_dim;
  desc.heads = r.plan.heads;
  desc.hidden_dim = r.plan.hidden_dim;
  desc.vocab = r.plan.vocab;
  desc.max_sequence = r.plan.max_sequence;
  desc.output_dim = r.plan.output_dim;
  // int8 codes of every weight (q4 unpacked) with its per-tensor scale.
  std::vector<std::vector<int8_t>> keep;
  auto codes = [&](const std::string& name, float* scale) -> const int8_t* {
    const Tensor* t = m->tensor(name);
    *scale = t->scale > 0.f ? t->scale : 0.f;
    keep.push_back(codes_of(m, *t));
    return keep.back().data();
  };
  keep.reserve(1 + 6 * r.layers.size());
  float s_tok = 0.f;
  const int8_t* tok = codes(r.token_param, &s_tok);
  std::vector<EosHipCompactLayer> layers(r.layers.size());
  // Tied layers pass the same buffers, so the bind shares their device copies.
  for (size_t l = 0; l < r.layers.size(); ++l) {
    const LayerParams& lp = r.layers[l];
    size_t tied = l;
    for (size_t j = 0; j < l && tied == l; ++j) {
      const LayerParams& o = r.layers[j];
      if (o.q == lp.q && o.k == lp.k && o.v == lp.v && o.o == lp.o && o.up == lp.up &&
          o.down == lp.down)
        tied = j;
    }
    if (tied != l) {
      layers[l] = layers[tied];
      continue;
    }
    EosHipCompactLayer& L = layers[l];
    L.attn_q = codes(lp.q, &L.s_q);
    L.attn_k = codes(lp.k, &L.s_k);
    L.attn_v = codes(lp.v, &L.s_v);
    L.attn_o = codes(lp.o, &L.s_o);
    L.ffn_up = codes(lp.up, &L.s_up);
    L.ffn_down = codes(lp.down, &L.s_down);
  }
  if (eoship_encoder_bind_compact_opts(rt, &desc, &opts, tok, s_tok, nullptr, 0.f, layers.data(),
                                       nullptr, 0.f, out, err) != 0)
    return 1;
  if (plan != nullptr) {
    *plan = r.plan;
    plan->options = opts;
  }
  return 0;
}

int eoship_mll_classify_retrieval(const EosHipMll* m, const char* entry,
                                  EosHipRetrievalPlan* plan, char** err) {
  if (m == nullptr || plan == nullptr)
    return set_err(err, "eoship_mll_classify_retrieval: NULL argument");
  return classify_retrieval(m, entry, plan, err);
}

int eoship_retrieval_bind_mll(EosHipRuntime* rt, const EosHipMll* m, const char* entry,
                              EosHipRetrieval** out, EosHipRetrievalPlan* plan, char** err) {
  const char* what = "eoship_retrieval_bind_mll";
  if (rt == nullptr || m == nullptr || out == nullptr) return set_err(err, "%s: NULL argument", what);
  *out = nullptr;
  EosHipRetrievalPlan p{};
  if (classify_retrieval(m, entry, &p, err) != 0) return 1;
  auto* r = new EosHipRetrieval();
  r->rt = rt;
  r->plan = p;
  r->spec.op = p.op;
  r->spec.k = p.k;
  r->spec.batched = p.batched;
  r->has_ids = p.has_candidate_ids != 0;
  if (p.docs_param) {
    const Tensor* t = m->tensor(p.docs_input);
    if (t == nullptr) {
      delete r;
      return set_err(err, "%s: document param \"%s\" has no payload", what, p.docs_input);
    }
    r->docs_param = true;
    r->rows = p.docs_rows;
    r->dim = p.dim;
    const uint8_t* b = m->bytes.data() + t->off;
    void* dev = nullptr;
    hipError_t e = hipSuccess;
    if (t->kind == EOSHIP_MLL_Q4) {
      // Packed nibbles stay packed; the kernels decode (nibble - 8) * scale.
      r->spec.docs_q4 = 1;
      r->spec.docs_scale = t->scale > 0.f ? t->scale : 0.f;
      if (rt->alloc(t->size, &dev, err) != 0) {
        delete r;
        return 1;
      }
      r->docs_q4 = static_cast<uint8_t*>(dev);
      e = rt->copy_sync(dev, b, t->size, hipMemcpyHostToDevice);
    } else {
      // q8 codes dequantized as the reference decodes them (f32 code * scale).
      std::vector<float> v((size_t)t->elements);
      if (t->kind == EOSHIP_MLL_Q8) {
        const float sc = t->scale > 0.f ? t->scale : 0.f;
        for (size_t i = 0; i < v.size(); ++i) v[i] = (float)(int8_t)b[i] * sc;
      } else {
        std::memcpy(v.data(), b, v.size() * 4);
      }
      if (rt->alloc(v.size() * 4, &dev, err) != 0) {
        delete r;
        return 1;
      }
      r->docs_f32 = static_cast<float*>(dev);
      e = rt->copy_sync(dev, v.data(), v.size() * 4, hipMemcpyHostToDevice);
    }
    if (e != hipSuccess) {
      if (r->docs_f32) (void)hipFree(r->docs_f32);
      if (r->docs_q4) (void)hipFree(r->docs_q4);
      delete r;
      return eoship::hip_err(err, "hipMemcpy(retrieval documents)", e);
    }
  }
  *out = r;
  if (plan != nullptr) *plan = p;
  return 0;
}

// BLAKE3 of a buffer (the digest the container stores per section).
int eoship_blake3(const uint8_t* data, uint64_t bytes, uint8_t* digest32, char** err) {
  if ((data == nullptr && bytes != 0) || digest32 == nullptr)
    return set_err(err, "eoship_blake3: NULL argument");
  static const uint8_t kEmpty = 0;
  b3::hash(data != nullptr ? data : &kEmpty, (size_t)bytes, digest32);
  return 0;
}

}  // extern "C"
