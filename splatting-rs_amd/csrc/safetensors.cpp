#include "safetensors.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdint>
#include <cstring>

#include "errors.h"

namespace splat {

namespace {

// A JSON subset parser sufficient for safetensors headers: objects, arrays, strings,
// integers (and skipping of floats / booleans / null inside __metadata__).
struct Json {
  const char* p;
  const char* end;
  int depth = 0;  // nesting of the value being skipped (a crafted header must not exhaust the stack)

  [[noreturn]] void fail(const char* what) { throw Error(IO_ERROR, std::string("safetensors header: ") + what); }
  void ws() {
    while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
  }
  bool peek(char c) {
    ws();
    return p < end && *p == c;
  }
  void expect(char c) {
    ws();
    if (p >= end || *p != c) fail("unexpected character");
    ++p;
  }
  std::string str() {
    expect('"');
    std::string s;
    while (p < end && *p != '"') {
      if (*p == '\\') {
        ++p;
        if (p >= end) fail("bad escape");
        char c = *p;
        if (c == 'u') {
          if (end - p < 5) fail("bad \\u escape");
          unsigned v = 0;
          for (int i = 1; i <= 4; ++i) {
            const char h = p[i], l = char(h | 32);
            if (h >= '0' && h <= '9') v = v * 16 + unsigned(h - '0');
            else if (l >= 'a' && l <= 'f') v = v * 16 + unsigned(l - 'a' + 10);
            else fail("bad \\u escape");
          }
          p += 4;
          if (v < 0x80) s += char(v);
          else if (v < 0x800) { s += char(0xC0 | (v >> 6)); s += char(0x80 | (v & 0x3F)); }
          else { s += char(0xE0 | (v >> 12)); s += char(0x80 | ((v >> 6) & 0x3F)); s += char(0x80 | (v & 0x3F)); }
        } else {
          s += c == 'n' ? '\n' : c == 't' ? '\t' : c == 'r' ? '\r' : c == 'b' ? '\b' : c == 'f' ? '\f' : c;
        }
        ++p;
      } else {
        s += *p++;
      }
    }
    expect('"');
    return s;
  }
  int64_t integer() {
    ws();
    bool neg = false;
    if (p < end && *p == '-') { neg = true; ++p; }
    if (p >= end || *p < '0' || *p > '9') fail("expected an integer");
    int64_t v = 0;
    while (p < end && *p >= '0' && *p <= '9') {
      const int digit = *p++ - '0';
      if (v > (INT64_MAX - digit) / 10) fail("integer out of range");
      v = v * 10 + digit;
    }
    return neg ? -v : v;
  }
  void skip_value() {
    ws();
    if (p >= end) fail("truncated");
    if (*p == '{' || *p == '[') {
      if (++depth > 64) fail("nested too deeply");
      skip_container();
      --depth;
      return;
    }
    if (*p == '"') { str(); return; }
    while (p < end && *p != ',' && *p != '}' && *p != ']') ++p;
  }
  void skip_container() {
    if (*p == '{') {
      ++p;
      if (peek('}')) { ++p; return; }
      do { str(); expect(':'); skip_value(); } while (peek(',') && ++p);
      expect('}');
      return;
    }
    if (*p == '[') {
      ++p;
      if (peek(']')) { ++p; return; }
      do { skip_value(); } while (peek(',') && ++p);
      expect(']');
    }
  }
  std::vector<int64_t> int_array() {
    std::vector<int64_t> v;
    expect('[');
    if (peek(']')) { ++p; return v; }
    do { v.push_back(integer()); } while (peek(',') && ++p);
    expect(']');
    return v;
  }
};

size_t dtype_bytes(const std::string& dt) {
  if (dt == "F32" || dt == "I32" || dt == "U32") return 4;
  if (dt == "BF16" || dt == "F16" || dt == "I16" || dt == "U16") return 2;
  if (dt == "F64" || dt == "I64" || dt == "U64") return 8;
  if (dt == "U8" || dt == "I8" || dt == "BOOL") return 1;
  return 0;
}

float bf16_to_f32(uint16_t h) {
  const uint32_t u = uint32_t(h) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// The element count of a header shape, or -1 if a dimension is negative or the byte size of the
// tensor (count times `elem` bytes) does not fit in int64_t.
int64_t checked_numel(const std::vector<int64_t>& shape, size_t elem) {
  int64_t n = 1;
  for (int64_t s : shape)
    if (s < 0 || __builtin_mul_overflow(n, s, &n)) return -1;
  int64_t bytes;
  if (__builtin_mul_overflow(n, int64_t(elem), &bytes)) return -1;
  return n;
}

float half_to_f32(uint16_t h) {
  const uint32_t sign = uint32_t(h & 0x8000) << 16;
  uint32_t exp = (h >> 10) & 0x1f, man = h & 0x3ff, u;
  if (exp == 0) {
    if (man == 0) u = sign;
    else {
      exp = 127 - 15 + 1;
      while (!(man & 0x400)) { man <<= 1; --exp; }
      u = sign | (exp << 23) | ((man & 0x3ff) << 13);
    }
  } else if (exp == 31) {
    u = sign | 0x7f800000u | (man << 13);
  } else {
    u = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

}  // namespace

std::string shape_str(const std::vector<int64_t>& s) {
  std::string r = "[";
  for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
  return r + "]";
}

SafeTensors::~SafeTensors() {
  if (map_) munmap(map_, map_len_);
}

void SafeTensors::open_file(const std::string& path) {
  int fd = ::open(path.c_str(), O_RDONLY);
  SPLAT_CHECK(fd >= 0, IO_ERROR, "cannot open " + path);
  struct stat sb;
  if (fstat(fd, &sb) != 0) {
    ::close(fd);
    throw Error(IO_ERROR, "cannot stat " + path);
  }
  map_len_ = size_t(sb.st_size);
  map_ = map_len_ ? mmap(nullptr, map_len_, PROT_READ, MAP_PRIVATE, fd, 0) : nullptr;
  ::close(fd);
  if (map_ == MAP_FAILED) {
    map_ = nullptr;
    throw Error(IO_ERROR, "cannot map " + path);
  }
  parse(static_cast<const uint8_t*>(map_), map_len_);
}

void SafeTensors::open_bytes(const uint8_t* bytes, size_t len) {
  owned_.assign(bytes, bytes + len);
  parse(owned_.data(), owned_.size());
}

void SafeTensors::parse(const uint8_t* base, size_t len) {
  SPLAT_CHECK(len >= 8, IO_ERROR, "safetensors: file too short");
  uint64_t hlen = 0;
  std::memcpy(&hlen, base, 8);
  SPLAT_CHECK(hlen <= len - 8, IO_ERROR, "safetensors: header length past the end");
  const uint8_t* data = base + 8 + hlen;
  const size_t data_len = len - 8 - hlen;
  Json j{reinterpret_cast<const char*>(base + 8), reinterpret_cast<const char*>(base + 8 + hlen)};
  j.expect('{');
  if (j.peek('}')) return;
  do {
    std::string name = j.str();
    j.expect(':');
    if (name == "__metadata__") {
      j.skip_value();
      continue;
    }
    StTensor t;
    std::vector<int64_t> offs;
    j.expect('{');
    do {
      std::string key = j.str();
      j.expect(':');
      if (key == "dtype") t.dtype = j.str();
      else if (key == "shape") t.shape = j.int_array();
      else if (key == "data_offsets") offs = j.int_array();
      else j.skip_value();
    } while (j.peek(',') && ++j.p);
    j.expect('}');
    SPLAT_CHECK(offs.size() == 2 && offs[0] >= 0 && offs[0] <= offs[1] && size_t(offs[1]) <= data_len, IO_ERROR,
                "safetensors: bad data_offsets for " + name);
    const size_t eb = dtype_bytes(t.dtype);
    SPLAT_CHECK(eb != 0, IO_ERROR, "safetensors: unsupported dtype " + t.dtype + " for " + name);
    const int64_t n = checked_numel(t.shape, eb);
    SPLAT_CHECK(n >= 0, IO_ERROR, "safetensors: bad shape " + shape_str(t.shape) + " for " + name);
    SPLAT_CHECK(uint64_t(offs[1] - offs[0]) == uint64_t(n) * eb, IO_ERROR, "safetensors: size mismatch for " + name);
    t.data = data + offs[0];
    t.nbytes = size_t(offs[1] - offs[0]);
    tensors_[name] = std::move(t);
  } while (j.peek(',') && ++j.p);
  j.expect('}');
}

const StTensor& SafeTensors::get(const std::string& name) const {
  auto it = tensors_.find(name);
  if (it == tensors_.end()) throw Error(MISSING_KEY, "missing tensor " + name);
  return it->second;
}

std::vector<float> SafeTensors::f32(const std::string& name, const std::vector<int64_t>& shape) const {
  const StTensor& t = get(name);
  SPLAT_CHECK(t.shape == shape, SHAPE_MISMATCH,
              "tensor " + name + " has shape " + shape_str(t.shape) + ", expected " + shape_str(shape));
  const size_t n = size_t(t.numel());
  std::vector<float> out(n);
  if (t.dtype == "F32") {
    std::memcpy(out.data(), t.data, n * 4);
  } else if (t.dtype == "BF16") {
    for (size_t i = 0; i < n; ++i) {
      uint16_t v;
      std::memcpy(&v, t.data + 2 * i, 2);
      out[i] = bf16_to_f32(v);
    }
  } else if (t.dtype == "F16") {
    for (size_t i = 0; i < n; ++i) {
      uint16_t v;
      std::memcpy(&v, t.data + 2 * i, 2);
      out[i] = half_to_f32(v);
    }
  } else if (t.dtype == "F64") {
    for (size_t i = 0; i < n; ++i) {
      double v;
      std::memcpy(&v, t.data + 8 * i, 8);
      out[i] = float(v);
    }
  } else {
    throw Error(SHAPE_MISMATCH, "tensor " + name + " has non-float dtype " + t.dtype);
  }
  return out;
}

}  // namespace splat
