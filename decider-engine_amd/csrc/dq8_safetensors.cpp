// safetensors reader: the header checks of read_tensors (decider-engine
// src/weights.rs:298-365) with the metadata rules of the safetensors crate
// 0.8.0, and Data::read / Data::into_f32 (weights.rs:147-195, 83-90) on host
// memory.  Host code only; the device load path is dq8_st_load_weights in
// dq8_api.hip.
#include <errno.h>
#include <fcntl.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <map>
#include <new>

#include "../../include/dq8.h"
#include "dq8_internal.h"
#include "dq8_st.h"

namespace {

constexpr uint64_t kMaxHeader = 16u << 20;  // weights.rs:308
constexpr int kMaxDepth = 128;              // serde_json's nesting limit

// Element bits of the safetensors dtypes (safetensors 0.8.0 Dtype), 0 if unknown.
int dtype_bits(const std::string& d) {
  static const std::map<std::string, int> bits = {
      {"BOOL", 8},  {"F4", 4},   {"F6_E2M3", 6}, {"F6_E3M2", 6}, {"U8", 8},   {"I8", 8},   {"F8_E5M2", 8},
      {"F8_E4M3", 8}, {"F8_E8M0", 8}, {"I16", 16}, {"U16", 16},   {"F16", 16}, {"BF16", 16}, {"I32", 32},
      {"U32", 32},  {"F32", 32}, {"C64", 64},    {"F64", 64},    {"I64", 64}, {"U64", 64}};
  auto it = bits.find(d);
  return it == bits.end() ? 0 : it->second;
}

// A JSON reader for the header, accepting what serde_json accepts for this
// schema: UTF-8 text, string escapes (including surrogate pairs), no control
// characters in strings, integers without sign, fraction, exponent or leading
// zeros where sizes are expected, any JSON value for fields it ignores, and
// surrounding whitespace.
struct Json {
  const unsigned char* p;
  const unsigned char* end;

  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool take(char c) {
    ws();
    if (p < end && *p == (unsigned char)c) {
      ++p;
      return true;
    }
    return false;
  }
  bool peek(char c) {
    ws();
    return p < end && *p == (unsigned char)c;
  }
  static void put_utf8(std::string& s, uint32_t c) {
    if (c < 0x80) {
      s += (char)c;
    } else if (c < 0x800) {
      s += (char)(0xC0 | (c >> 6));
      s += (char)(0x80 | (c & 0x3F));
    } else if (c < 0x10000) {
      s += (char)(0xE0 | (c >> 12));
      s += (char)(0x80 | ((c >> 6) & 0x3F));
      s += (char)(0x80 | (c & 0x3F));
    } else {
      s += (char)(0xF0 | (c >> 18));
      s += (char)(0x80 | ((c >> 12) & 0x3F));
      s += (char)(0x80 | ((c >> 6) & 0x3F));
      s += (char)(0x80 | (c & 0x3F));
    }
  }
  bool hex4(uint32_t& v) {
    if (end - p < 4) return false;
    v = 0;
    for (int i = 0; i < 4; ++i) {
      const unsigned char c = p[i];
      v <<= 4;
      if (c >= '0' && c <= '9') v |= c - '0';
      else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
      else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
      else return false;
    }
    p += 4;
    return true;
  }
  // One well-formed UTF-8 sequence starting at p (not ASCII).
  bool utf8(std::string& s) {
    const unsigned char c = *p;
    int n;
    uint32_t cp, min;
    if (c >= 0xC2 && c <= 0xDF) n = 1, cp = c & 0x1F, min = 0x80;
    else if (c >= 0xE0 && c <= 0xEF) n = 2, cp = c & 0x0F, min = 0x800;
    else if (c >= 0xF0 && c <= 0xF4) n = 3, cp = c & 0x07, min = 0x10000;
    else return false;
    if (end - p < n + 1) return false;
    for (int i = 1; i <= n; ++i) {
      if ((p[i] & 0xC0) != 0x80) return false;
      cp = (cp << 6) | (p[i] & 0x3F);
    }
    if (cp < min || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return false;
    s.append((const char*)p, n + 1);
    p += n + 1;
    return true;
  }
  bool string(std::string& s) {
    s.clear();
    if (!take('"')) return false;
    while (p < end) {
      const unsigned char c = *p;
      if (c == '"') {
        ++p;
        return true;
      }
      if (c < 0x20) return false;
      if (c >= 0x80) {
        if (!utf8(s)) return false;
        continue;
      }
      ++p;
      if (c != '\\') {
        s += (char)c;
        continue;
      }
      if (p >= end) return false;
      const unsigned char e = *p++;
      switch (e) {
        case '"': s += '"'; break;
        case '\\': s += '\\'; break;
        case '/': s += '/'; break;
        case 'b': s += '\b'; break;
        case 'f': s += '\f'; break;
        case 'n': s += '\n'; break;
        case 'r': s += '\r'; break;
        case 't': s += '\t'; break;
        case 'u': {
          uint32_t u;
          if (!hex4(u)) return false;
          if (u >= 0xDC00 && u <= 0xDFFF) return false;  // lone trailing surrogate
          if (u >= 0xD800 && u <= 0xDBFF) {
            uint32_t lo;
            if (end - p < 2 || p[0] != '\\' || p[1] != 'u') return false;
            p += 2;
            if (!hex4(lo) || lo < 0xDC00 || lo > 0xDFFF) return false;
            u = 0x10000 + ((u - 0xD800) << 10) + (lo - 0xDC00);
          }
          put_utf8(s, u);
          break;
        }
        default: return false;
      }
    }
    return false;
  }
  // A non-negative integer that fits 64 bits (a usize field).
  bool uint(uint64_t& v) {
    ws();
    if (p >= end || *p < '0' || *p > '9') return false;
    if (*p == '0' && p + 1 < end && p[1] >= '0' && p[1] <= '9') return false;  // leading zero
    v = 0;
    while (p < end && *p >= '0' && *p <= '9') {
      const uint64_t d = *p - '0';
      if (v > (UINT64_MAX - d) / 10) return false;
      v = v * 10 + d;
      ++p;
    }
    // a fraction or an exponent makes it a float, which a usize field rejects
    return !(p < end && (*p == '.' || *p == 'e' || *p == 'E'));
  }
  bool number() {
    ws();
    if (p < end && *p == '-') ++p;
    if (p >= end) return false;
    if (*p == '0') {
      ++p;
    } else if (*p >= '1' && *p <= '9') {
      while (p < end && *p >= '0' && *p <= '9') ++p;
    } else {
      return false;
    }
    if (p < end && *p == '.') {
      ++p;
      if (p >= end || *p < '0' || *p > '9') return false;
      while (p < end && *p >= '0' && *p <= '9') ++p;
    }
    if (p < end && (*p == 'e' || *p == 'E')) {
      ++p;
      if (p < end && (*p == '+' || *p == '-')) ++p;
      if (p >= end || *p < '0' || *p > '9') return false;
      while (p < end && *p >= '0' && *p <= '9') ++p;
    }
    return true;
  }
  bool word(const char* w) {
    ws();
    const size_t n = strlen(w);
    if ((size_t)(end - p) < n || memcmp(p, w, n) != 0) return false;
    p += n;
    return true;
  }
  // Any JSON value (fields the schema ignores).
  bool skip(int depth) {
    if (depth > kMaxDepth) return false;
    ws();
    if (p >= end) return false;
    std::string tmp;
    switch (*p) {
      case '"': return string(tmp);
      case '{': {
        ++p;
        if (take('}')) return true;
        do {
          if (!string(tmp) || !take(':') || !skip(depth + 1)) return false;
        } while (take(','));
        return take('}');
      }
      case '[': {
        ++p;
        if (take(']')) return true;
        do {
          if (!skip(depth + 1)) return false;
        } while (take(','));
        return take(']');
      }
      case 't': return word("true");
      case 'f': return word("false");
      case 'n': return word("null");
      default: return number();
    }
  }
  bool uint_array(std::vector<uint64_t>& out) {
    out.clear();
    if (!take('[')) return false;
    if (take(']')) return true;
    do {
      uint64_t v;
      if (!uint(v)) return false;
      out.push_back(v);
    } while (take(','));
    return take(']');
  }
  // TensorInfo {dtype, shape, data_offsets}; other fields are ignored, a
  // repeated or missing field is an error.
  bool tensor(dq8_st_tensor& t) {
    if (!take('{')) return false;
    bool has_dtype = false, has_shape = false, has_offsets = false;
    std::string key;
    if (!take('}')) {
      do {
        if (!string(key) || !take(':')) return false;
        if (key == "dtype") {
          if (has_dtype || !string(t.dtype)) return false;
          t.bits = dtype_bits(t.dtype);
          if (t.bits == 0) return false;
          has_dtype = true;
        } else if (key == "shape") {
          std::vector<uint64_t> v;
          if (has_shape || !uint_array(v)) return false;
          t.shape.assign(v.begin(), v.end());
          has_shape = true;
        } else if (key == "data_offsets") {
          std::vector<uint64_t> v;
          if (has_offsets || !uint_array(v) || v.size() != 2) return false;
          t.begin = v[0];
          t.end = v[1];
          has_offsets = true;
        } else if (!skip(2)) {
          return false;
        }
      } while (take(','));
      if (!take('}')) return false;
    }
    return has_dtype && has_shape && has_offsets;
  }
  // "__metadata__": null or an object of strings.
  bool metadata() {
    if (word("null")) return true;
    if (!take('{')) return false;
    if (take('}')) return true;
    std::string k, v;
    do {
      if (!string(k) || !take(':') || !string(v)) return false;
    } while (take(','));
    return take('}');
  }
};

// Header text -> tensors in file order, validated as safetensors'
// Metadata::validate: sorted by data_offsets, they must tile [0, data_len)
// exactly, each spanning its shape's bytes.
bool parse_header(const unsigned char* text, size_t size, std::vector<dq8_st_tensor>& out) {
  Json j{text, text + size};
  std::map<std::string, dq8_st_tensor> byname;  // a repeated name keeps its last entry
  if (!j.take('{')) return false;
  if (!j.take('}')) {
    std::string key;
    do {
      if (!j.string(key) || !j.take(':')) return false;
      if (key == "__metadata__") {
        if (!j.metadata()) return false;
        continue;
      }
      dq8_st_tensor t;
      if (!j.tensor(t)) return false;
      t.name = key;
      byname[key] = std::move(t);
    } while (j.take(','));
    if (!j.take('}')) return false;
  }
  j.ws();
  if (j.p != j.end) return false;
  out.clear();
  for (auto& kv : byname) out.push_back(std::move(kv.second));
  std::stable_sort(out.begin(), out.end(), [](const dq8_st_tensor& a, const dq8_st_tensor& b) {
    return a.begin != b.begin ? a.begin < b.begin : a.end < b.end;
  });
  uint64_t start = 0;
  for (const dq8_st_tensor& t : out) {
    if (t.begin != start || t.end < t.begin) return false;
    start = t.end;
    uint64_t elements = 1;
    for (size_t d : t.shape) {
      if (d != 0 && elements > UINT64_MAX / d) return false;
      elements *= d;
    }
    if (elements > UINT64_MAX / (uint64_t)t.bits) return false;
    const uint64_t bits = elements * (uint64_t)t.bits;
    if (bits % 8 != 0) return false;
    if (t.end - t.begin != bits / 8) return false;
  }
  return true;
}

float half_to_f32(uint16_t v) {
  // weights.rs:367-382: exact for every finite half.
  const int e = (v >> 10) & 31, m = v & 1023;
  float r;
  if (e == 0) r = std::ldexp((float)m, -24);
  else if (e == 31) r = m == 0 ? INFINITY : NAN;
  else r = std::ldexp((float)(1024 + m), e - 25);
  return (v & 0x8000) ? -r : r;
}

size_t element_bytes(int code) { return code == dq8::kDtypeF32 ? 4 : 2; }

}  // namespace

namespace dq8 {

int st_dtype_code(const std::string& dtype) {
  if (dtype == "F32") return kDtypeF32;
  if (dtype == "BF16") return kDtypeBF16;
  if (dtype == "F16") return kDtypeF16;
  return -1;
}

bool st_pread(const dq8_st* st, void* dst, size_t count, uint64_t at) {
  char* d = static_cast<char*>(dst);
  while (count > 0) {
    const ssize_t got = pread(st->fd, d, count, (off_t)at);
    if (got < 0 && errno == EINTR) continue;
    if (got <= 0) return false;
    d += got;
    count -= (size_t)got;
    at += (uint64_t)got;
  }
  return true;
}

bool st_all_finite(int code, const void* data, size_t bytes) {
  if (code == kDtypeF32) {
    const unsigned char* b = static_cast<const unsigned char*>(data);
    for (size_t i = 0; i + 4 <= bytes; i += 4) {
      uint32_t u;
      memcpy(&u, b + i, 4);
      if ((u & 0x7F800000u) == 0x7F800000u) return false;
    }
    return true;
  }
  const uint16_t mask = code == kDtypeBF16 ? 0x7F80 : 0x7C00;
  const unsigned char* b = static_cast<const unsigned char*>(data);
  for (size_t i = 0; i + 2 <= bytes; i += 2) {
    uint16_t u;
    memcpy(&u, b + i, 2);
    if ((u & mask) == mask) return false;
  }
  return true;
}

}  // namespace dq8

extern "C" {

dq8_status dq8_st_open(const char* path, dq8_st** out) {
  if (!path || !out) return DQ8_ERR_ARG;
  *out = nullptr;
  const int fd = open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) return DQ8_ERR_IO;
  dq8_st* st = new (std::nothrow) dq8_st();
  if (!st) {
    close(fd);
    return DQ8_ERR_NOMEM;
  }
  st->fd = fd;
  dq8_status status = DQ8_OK;
  struct stat sb;
  unsigned char size8[8];
  uint64_t header = 0;
  if (fstat(fd, &sb) != 0) {
    status = DQ8_ERR_IO;
  } else {
    st->length = (uint64_t)sb.st_size;
    // weights.rs:306-311: an 8-byte size, a header of at most 16 MiB inside the file
    if (st->length < 8) status = DQ8_ERR_FORMAT;
    else if (!dq8::st_pread(st, size8, 8, 0)) status = DQ8_ERR_IO;
  }
  if (status == DQ8_OK) {
    for (int i = 7; i >= 0; --i) header = (header << 8) | size8[i];
    if (header > kMaxHeader || header + 8 > st->length) status = DQ8_ERR_FORMAT;
  }
  if (status == DQ8_OK) {
    std::vector<unsigned char> text(header);
    if (header && !dq8::st_pread(st, text.data(), header, 8)) status = DQ8_ERR_IO;
    else if (!parse_header(text.data(), header, st->tensors)) status = DQ8_ERR_FORMAT;
  }
  if (status == DQ8_OK) {
    // weights.rs:314-317: the data section ends exactly at the end of the file
    st->data_start = header + 8;
    const uint64_t data_len = st->tensors.empty() ? 0 : st->tensors.back().end;
    if (data_len > UINT64_MAX - st->data_start || st->data_start + data_len != st->length) status = DQ8_ERR_FORMAT;
  }
  if (status != DQ8_OK) {
    close(fd);
    delete st;
    return status;
  }
  *out = st;
  return DQ8_OK;
}

dq8_status dq8_st_close(dq8_st* st) {
  if (!st) return DQ8_ERR_ARG;
  if (st->fd >= 0) close(st->fd);
  delete st;
  return DQ8_OK;
}

dq8_status dq8_st_count(const dq8_st* st, size_t* count) {
  if (!st || !count) return DQ8_ERR_ARG;
  *count = st->tensors.size();
  return DQ8_OK;
}

dq8_status dq8_st_info(const dq8_st* st, size_t i, const char** name, const char** dtype, size_t* ndim,
                       const size_t** shape, size_t* bytes) {
  if (!st || i >= st->tensors.size()) return DQ8_ERR_ARG;
  const dq8_st_tensor& t = st->tensors[i];
  if (name) *name = t.name.c_str();
  if (dtype) *dtype = t.dtype.c_str();
  if (ndim) *ndim = t.shape.size();
  if (shape) *shape = t.shape.data();
  if (bytes) *bytes = (size_t)(t.end - t.begin);
  return DQ8_OK;
}

dq8_status dq8_st_find(const dq8_st* st, const char* name, size_t* index) {
  if (!st || !name || !index) return DQ8_ERR_ARG;
  for (size_t i = 0; i < st->tensors.size(); ++i)
    if (st->tensors[i].name == name) {
      *index = i;
      return DQ8_OK;
    }
  return DQ8_ERR_ARG;
}

dq8_status dq8_st_read_host(const dq8_st* st, size_t i, void* dst, size_t bytes) {
  if (!st || i >= st->tensors.size() || (!dst && bytes)) return DQ8_ERR_ARG;
  const dq8_st_tensor& t = st->tensors[i];
  const int code = dq8::st_dtype_code(t.dtype);
  if (code < 0) return DQ8_ERR_FORMAT;  // "unsupported weight dtype"
  if (bytes != t.end - t.begin) return DQ8_ERR_SHAPE;
  if (bytes && !dq8::st_pread(st, dst, bytes, st->data_start + t.begin)) return DQ8_ERR_IO;
  return dq8::st_all_finite(code, dst, bytes) ? DQ8_OK : DQ8_ERR_NONFINITE;
}

dq8_status dq8_st_read_f32_host(const dq8_st* st, size_t i, float* dst, size_t count) {
  if (!st || i >= st->tensors.size() || (!dst && count)) return DQ8_ERR_ARG;
  const dq8_st_tensor& t = st->tensors[i];
  const int code = dq8::st_dtype_code(t.dtype);
  if (code < 0) return DQ8_ERR_FORMAT;
  const size_t es = element_bytes(code);
  if (count != (t.end - t.begin) / es) return DQ8_ERR_SHAPE;
  // A bounded transfer buffer, as Data::read (weights.rs:161-163).
  std::vector<unsigned char> buf(std::min<size_t>(count * es, 1u << 20));
  size_t done = 0;
  while (done < count) {
    const size_t n = std::min(count - done, buf.size() / es);
    if (!dq8::st_pread(st, buf.data(), n * es, st->data_start + t.begin + done * es)) return DQ8_ERR_IO;
    if (!dq8::st_all_finite(code, buf.data(), n * es)) return DQ8_ERR_NONFINITE;
    for (size_t j = 0; j < n; ++j) {
      if (code == dq8::kDtypeF32) {
        memcpy(&dst[done + j], &buf[4 * j], 4);
      } else {
        uint16_t h;
        memcpy(&h, &buf[2 * j], 2);
        dst[done + j] = code == dq8::kDtypeBF16 ? [](uint16_t b) {
          const uint32_t u = (uint32_t)b << 16;
          float f;
          memcpy(&f, &u, 4);
          return f;
        }(h) : half_to_f32(h);
      }
    }
    done += n;
  }
  return DQ8_OK;
}

}  // extern "C"
