// Strict safetensors header reader (see safetensors.h).
#include "safetensors.h"

#include <sys/stat.h>

#include <algorithm>
#include <cctype>
#include <cstdint>
#include <cstring>
#include <fstream>
#include <memory>
#include <set>
#include <stdexcept>

namespace hb {
namespace {

[[noreturn]] void bad(const std::string& why) { throw std::invalid_argument("safetensors: " + why); }

// A JSON value: enough of RFC 8259 for a safetensors header (objects with
// unique keys, arrays, strings, numbers, literals), nesting bounded.
struct Json {
  enum Kind { kNull, kBool, kNumber, kString, kArray, kObject } kind = kNull;
  bool boolean = false;
  bool integer = false;  // the number has no fraction or exponent
  uint64_t uvalue = 0;   // its value when integer and non-negative
  bool negative = false;
  std::string text;
  std::vector<Json> items;
  std::vector<std::pair<std::string, Json>> fields;
};

class Reader {
 public:
  explicit Reader(const std::string& s) : s_(s) {}

  Json document() {
    Json v = value(0);
    ws();
    if (i_ != s_.size()) bad("trailing bytes after the header object");
    return v;
  }

 private:
  const std::string& s_;
  size_t i_ = 0;

  void ws() {
    while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\t' || s_[i_] == '\n' || s_[i_] == '\r')) ++i_;
  }
  char peek() {
    ws();
    if (i_ >= s_.size()) bad("truncated header JSON");
    return s_[i_];
  }
  void expect(char c) {
    if (peek() != c) bad(std::string("expected '") + c + "' in the header JSON");
    ++i_;
  }

  static void utf8(std::string& out, uint32_t cp) {
    if (cp < 0x80) {
      out += char(cp);
    } else if (cp < 0x800) {
      out += char(0xC0 | (cp >> 6));
      out += char(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      out += char(0xE0 | (cp >> 12));
      out += char(0x80 | ((cp >> 6) & 0x3F));
      out += char(0x80 | (cp & 0x3F));
    } else {
      out += char(0xF0 | (cp >> 18));
      out += char(0x80 | ((cp >> 12) & 0x3F));
      out += char(0x80 | ((cp >> 6) & 0x3F));
      out += char(0x80 | (cp & 0x3F));
    }
  }
  uint32_t hex4() {
    if (i_ + 4 > s_.size()) bad("truncated \\u escape");
    uint32_t v = 0;
    for (int k = 0; k < 4; ++k) {
      const char c = s_[i_++];
      v <<= 4;
      if (c >= '0' && c <= '9')
        v |= uint32_t(c - '0');
      else if (c >= 'a' && c <= 'f')
        v |= uint32_t(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F')
        v |= uint32_t(c - 'A' + 10);
      else
        bad("bad \\u escape");
    }
    return v;
  }
  std::string string() {
    expect('"');
    std::string out;
    for (;;) {
      if (i_ >= s_.size()) bad("unterminated string");
      const char c = s_[i_++];
      if (c == '"') return out;
      if (static_cast<unsigned char>(c) < 0x20) bad("control character in a string");
      if (c != '\\') {
        out += c;
        continue;
      }
      if (i_ >= s_.size()) bad("unterminated escape");
      const char e = s_[i_++];
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
          if (cp >= 0xD800 && cp < 0xDC00) {
            if (i_ + 2 > s_.size() || s_[i_] != '\\' || s_[i_ + 1] != 'u') bad("unpaired surrogate");
            i_ += 2;
            const uint32_t lo = hex4();
            if (lo < 0xDC00 || lo >= 0xE000) bad("unpaired surrogate");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          } else if (cp >= 0xDC00 && cp < 0xE000) {
            bad("unpaired surrogate");
          }
          utf8(out, cp);
          break;
        }
        default: bad("bad escape");
      }
    }
  }
  Json number() {
    Json v;
    v.kind = Json::kNumber;
    v.integer = true;
    if (s_[i_] == '-') {
      v.negative = true;
      ++i_;
    }
    if (i_ >= s_.size() || !std::isdigit(static_cast<unsigned char>(s_[i_]))) bad("bad number");
    if (s_[i_] == '0' && i_ + 1 < s_.size() && std::isdigit(static_cast<unsigned char>(s_[i_ + 1])))
      bad("leading zero in a number");
    bool overflow = false;
    while (i_ < s_.size() && std::isdigit(static_cast<unsigned char>(s_[i_]))) {
      const uint64_t d = uint64_t(s_[i_++] - '0');
      if (v.uvalue > (UINT64_MAX - d) / 10) overflow = true;
      v.uvalue = v.uvalue * 10 + d;
    }
    if (i_ < s_.size() && s_[i_] == '.') {
      v.integer = false;
      ++i_;
      if (i_ >= s_.size() || !std::isdigit(static_cast<unsigned char>(s_[i_]))) bad("bad fraction");
      while (i_ < s_.size() && std::isdigit(static_cast<unsigned char>(s_[i_]))) ++i_;
    }
    if (i_ < s_.size() && (s_[i_] == 'e' || s_[i_] == 'E')) {
      v.integer = false;
      ++i_;
      if (i_ < s_.size() && (s_[i_] == '+' || s_[i_] == '-')) ++i_;
      if (i_ >= s_.size() || !std::isdigit(static_cast<unsigned char>(s_[i_]))) bad("bad exponent");
      while (i_ < s_.size() && std::isdigit(static_cast<unsigned char>(s_[i_]))) ++i_;
    }
    if (overflow) v.integer = false;  // not usable as a size
    return v;
  }
  void literal(const char* word) {
    const size_t n = std::strlen(word);
    if (s_.compare(i_, n, word) != 0) bad("bad literal");
    i_ += n;
  }
  Json value(int depth) {
    if (depth > 16) bad("header nested too deeply");
    const char c = peek();
    Json v;
    if (c == '{') {
      ++i_;
      v.kind = Json::kObject;
      std::set<std::string> keys;
      if (peek() == '}') {
        ++i_;
        return v;
      }
      for (;;) {
        std::string k = string();
        if (!keys.insert(k).second) bad("duplicate key \"" + k + "\"");
        expect(':');
        v.fields.emplace_back(std::move(k), value(depth + 1));
        const char d = peek();
        ++i_;
        if (d == '}') return v;
        if (d != ',') bad("expected ',' or '}'");
      }
    }
    if (c == '[') {
      ++i_;
      v.kind = Json::kArray;
      if (peek() == ']') {
        ++i_;
        return v;
      }
      for (;;) {
        v.items.push_back(value(depth + 1));
        const char d = peek();
        ++i_;
        if (d == ']') return v;
        if (d != ',') bad("expected ',' or ']'");
      }
    }
    if (c == '"') {
      v.kind = Json::kString;
      v.text = string();
      return v;
    }
    if (c == 't' || c == 'f') {
      v.kind = Json::kBool;
      v.boolean = c == 't';
      literal(c == 't' ? "true" : "false");
      return v;
    }
    if (c == 'n') {
      literal("null");
      return v;
    }
    if (c == '-' || std::isdigit(static_cast<unsigned char>(c))) return number();
    bad("unexpected character in the header JSON");
  }
};

const Json* field(const Json& obj, const char* key) {
  for (const auto& [k, v] : obj.fields)
    if (k == key) return &v;
  return nullptr;
}

uint64_t size_value(const Json& v, const char* what) {
  if (v.kind != Json::kNumber || !v.integer || v.negative) bad(std::string(what) + " must be a non-negative integer");
  return v.uvalue;
}

}  // namespace

std::vector<SafeTensor> parse_safetensors_header(const std::string& json, uint64_t payload_bytes) {
  const Json doc = Reader(json).document();
  if (doc.kind != Json::kObject) bad("header is not a JSON object");
  std::vector<SafeTensor> out;
  for (const auto& [name, v] : doc.fields) {
    if (name == "__metadata__") {
      if (v.kind != Json::kObject) bad("__metadata__ must be an object");
      continue;
    }
    if (name.empty()) bad("empty tensor name");
    if (v.kind != Json::kObject) bad("tensor \"" + name + "\" is not an object");
    const Json* dt = field(v, "dtype");
    const Json* sh = field(v, "shape");
    const Json* off = field(v, "data_offsets");
    if (!dt || !sh || !off) bad("tensor \"" + name + "\" lacks dtype, shape or data_offsets");
    if (v.fields.size() != 3) bad("tensor \"" + name + "\" has unknown fields");
    SafeTensor t;
    t.name = name;
    if (dt->kind != Json::kString) bad("dtype must be a string");
    static const char* kNames[] = {"F32", "I32", "U32", "F16", "BF16"};
    static const uint64_t kItem[] = {4, 4, 4, 2, 2};
    t.dtype = -1;
    for (int k = 0; k < 5; ++k)
      if (dt->text == kNames[k]) t.dtype = k;
    if (t.dtype < 0) bad("tensor \"" + name + "\": unsupported dtype " + dt->text);
    if (sh->kind != Json::kArray || sh->items.empty() || sh->items.size() > 4)
      bad("tensor \"" + name + "\": shape rank outside 1..4");
    uint64_t bytes = kItem[t.dtype];
    for (const Json& d : sh->items) {
      const uint64_t n = size_value(d, "shape dimension");
      if (n == 0 || n > uint64_t(INT32_MAX)) bad("tensor \"" + name + "\": shape dimension outside 1..2^31-1");
      if (bytes > UINT64_MAX / n) bad("tensor \"" + name + "\": size overflow");
      bytes *= n;
      t.shape.push_back(int32_t(n));
    }
    if (off->kind != Json::kArray || off->items.size() != 2) bad("data_offsets must be two integers");
    t.begin = size_value(off->items[0], "data offset");
    t.end = size_value(off->items[1], "data offset");
    if (t.begin > t.end || t.end - t.begin != bytes)
      bad("tensor \"" + name + "\": data_offsets do not span its shape");
    if (t.end > payload_bytes) bad("tensor \"" + name + "\": data_offsets outside the payload");
    out.push_back(std::move(t));
  }
  std::vector<std::pair<uint64_t, uint64_t>> ranges;
  for (const SafeTensor& t : out) ranges.emplace_back(t.begin, t.end);
  std::sort(ranges.begin(), ranges.end());
  for (size_t k = 1; k < ranges.size(); ++k)
    if (ranges[k - 1].second > ranges[k].first) bad("overlapping tensor data");
  return out;
}

SafeFile read_safetensors_header(const std::string& path) {
  struct stat st {};
  if (lstat(path.c_str(), &st) != 0) bad("cannot stat " + path);
  if (!S_ISREG(st.st_mode)) bad("not a regular file: " + path);
  const uint64_t size = uint64_t(st.st_size);
  std::ifstream f(path, std::ios::binary);
  if (!f) bad("cannot open " + path);
  unsigned char len8[8];
  if (size < 8 || !f.read(reinterpret_cast<char*>(len8), 8)) bad("file shorter than its header length");
  uint64_t n = 0;
  for (int k = 7; k >= 0; --k) n = (n << 8) | len8[k];
  if (n < 2 || n > 8ull * 1024 * 1024 || n > size - 8) bad("header length outside 2 B..8 MiB or past the file end");
  std::string json(size_t(n), '\0');
  if (!f.read(json.data(), std::streamsize(n))) bad("truncated header");
  SafeFile out;
  out.payload = 8 + n;
  out.tensors = parse_safetensors_header(json, size - out.payload);
  return out;
}

}  // namespace hb
