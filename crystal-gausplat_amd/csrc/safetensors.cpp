// Safetensors checkpoint ingestion: the format reader of SafetensorsLoader
// (src/mastr/weights.cr:30-290) and the name mapping of WeightLoader
// (src/mastr/weight_loader.cr:43-123), feeding a MASt3R context.
//
// Format: u64 little-endian header length, a JSON header mapping tensor names
// to {"dtype", "shape", "data_offsets": [begin, end]} (offsets relative to the
// data section that follows the header; "__metadata__" is skipped), then the
// raw little-endian data. F32 is copied, F16 converted exactly (IEEE binary16
// -> binary32, subnormals included), BF16 widened by a 16-bit shift -- the
// three dtypes the reference converts (src/mastr/weights.cr:168-175).
// Unlike the reference, the fused attention qkv weights stay fused (the
// kernels consume them that way), and convolution / ConvTranspose weights are
// re-laid for the kernels when the context places them.
#include <fcntl.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <map>
#include <string>
#include <vector>

#include "../../include/gs_hip.h"
#include "internal.h"

namespace gs {
namespace {

struct TensorEntry {
  std::string name, dtype;
  std::vector<int64_t> shape;
  int64_t begin = 0, end = 0;
};

// Minimal JSON reader for the safetensors header: objects, arrays, strings,
// integers, true / false / null. Values other than the tensor records are
// skipped.
struct Json {
  const char* p;
  const char* e;
  std::string err;

  void ws() {
    while (p < e && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
  }
  bool lit(char c) {
    ws();
    if (p < e && *p == c) {
      ++p;
      return true;
    }
    return false;
  }
  bool str(std::string& out) {
    ws();
    if (p >= e || *p != '"') return fail("expected string");
    ++p;
    out.clear();
    while (p < e && *p != '"') {
      if (*p == '\\') {
        ++p;
        if (p >= e) return fail("bad escape");
        const char c = *p++;
        switch (c) {
          case 'n': out += '\n'; break;
          case 't': out += '\t'; break;
          case 'r': out += '\r'; break;
          case 'b': out += '\b'; break;
          case 'f': out += '\f'; break;
          case 'u': {  // keep ASCII, replace the rest (names are ASCII)
            if (e - p < 4) return fail("bad \\u escape");
            unsigned v = 0;
            for (int i = 0; i < 4; ++i) {
              const char h = *p++;
              v = v * 16 + (unsigned)(h >= '0' && h <= '9' ? h - '0'
                                      : h >= 'a' && h <= 'f' ? h - 'a' + 10
                                      : h >= 'A' && h <= 'F' ? h - 'A' + 10 : 0);
            }
            out += v < 128 ? (char)v : '?';
            break;
          }
          default: out += c;
        }
      } else {
        out += *p++;
      }
    }
    if (p >= e) return fail("unterminated string");
    ++p;
    return true;
  }
  bool integer(int64_t& v) {
    ws();
    const char* s = p;
    bool neg = false;
    if (p < e && *p == '-') {
      neg = true;
      ++p;
    }
    if (p >= e || *p < '0' || *p > '9') return fail("expected integer");
    v = 0;
    while (p < e && *p >= '0' && *p <= '9') {
      if (v > (INT64_MAX - 9) / 10) return fail("integer overflow");
      v = v * 10 + (*p++ - '0');
    }
    if (p < e && (*p == '.' || *p == 'e' || *p == 'E')) {
      p = s;
      return fail("expected integer");
    }
    if (neg) v = -v;
    return true;
  }
  bool skip() {  // any value
    ws();
    if (p >= e) return fail("unexpected end");
    if (*p == '"') {
      std::string t;
      return str(t);
    }
    if (*p == '{') {
      ++p;
      if (lit('}')) return true;
      do {
        std::string k;
        if (!str(k) || !lit(':') || !skip()) return false;
      } while (lit(','));
      return lit('}') || fail("expected }");
    }
    if (*p == '[') {
      ++p;
      if (lit(']')) return true;
      do {
        if (!skip()) return false;
      } while (lit(','));
      return lit(']') || fail("expected ]");
    }
    const char* s = p;
    while (p < e && *p != ',' && *p != '}' && *p != ']' && *p != ' ' && *p != '\n') ++p;
    return p > s || fail("bad value");
  }
  bool int_array(std::vector<int64_t>& out) {
    out.clear();
    if (!lit('[')) return fail("expected [");
    if (lit(']')) return true;
    do {
      int64_t v;
      if (!integer(v)) return false;
      out.push_back(v);
    } while (lit(','));
    return lit(']') || fail("expected ]");
  }
  bool fail(const char* m) {
    if (err.empty()) err = m;
    return false;
  }
};

int parse_header(const char* h, size_t n, std::vector<TensorEntry>& out) {
  Json j{h, h + n, ""};
  out.clear();
  if (!j.lit('{')) {
    set_error("safetensors: header is not a JSON object");
    return -1;
  }
  if (j.lit('}')) return 0;
  do {
    std::string key;
    if (!j.str(key) || !j.lit(':')) break;
    if (key == "__metadata__") {
      if (!j.skip()) break;
      continue;
    }
    TensorEntry t;
    t.name = key;
    if (!j.lit('{')) {
      j.fail("expected tensor record");
      break;
    }
    std::vector<int64_t> offs;
    bool have_dtype = false, have_shape = false, have_offs = false;
    if (!j.lit('}')) {
      do {
        std::string f;
        if (!j.str(f) || !j.lit(':')) break;
        if (f == "dtype") {
          have_dtype = j.str(t.dtype);
        } else if (f == "shape") {
          have_shape = j.int_array(t.shape);
        } else if (f == "data_offsets") {
          have_offs = j.int_array(offs);
        } else if (!j.skip()) {
          break;
        }
      } while (j.lit(','));
      if (!j.lit('}')) j.fail("expected } after tensor record");
    }
    if (!j.err.empty()) break;
    if (!have_dtype || !have_shape || !have_offs || offs.size() != 2) {
      set_error("safetensors: incomplete record for " + key);
      return -1;
    }
    t.begin = offs[0];
    t.end = offs[1];
    out.push_back(t);
  } while (j.lit(','));
  if (!j.err.empty() || !j.lit('}')) {
    set_error("safetensors: bad header JSON (" + (j.err.empty() ? std::string("trailing data") : j.err) +
              ")");
    return -1;
  }
  return 0;
}

int64_t elem_size(const std::string& dt) {
  if (dt == "F32" || dt == "I32" || dt == "U32") return 4;
  if (dt == "F16" || dt == "BF16" || dt == "I16" || dt == "U16") return 2;
  if (dt == "F64" || dt == "I64" || dt == "U64") return 8;
  if (dt == "I8" || dt == "U8" || dt == "BOOL" || dt == "F8_E4M3" || dt == "F8_E5M2") return 1;
  return 0;
}

float half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t exp = (h >> 10) & 0x1f, man = h & 0x3ff;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {  // subnormal: normalise
      int e = -1;
      do {
        ++e;
        man <<= 1;
      } while ((man & 0x400) == 0);
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ff) << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

// A read-only mapping of one safetensors file with its parsed header.
struct File {
  int fd = -1;
  const uint8_t* map = nullptr;
  size_t size = 0;
  int64_t data_off = 0;
  std::vector<TensorEntry> tensors;

  ~File() {
    if (map) munmap((void*)map, size);
    if (fd >= 0) close(fd);
  }

  int open_file(const char* path) {
    fd = ::open(path, O_RDONLY);
    if (fd < 0) {
      set_error(std::string("safetensors: cannot open ") + path);
      return -1;
    }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 8) {
      set_error("safetensors: file too small");
      return -1;
    }
    size = (size_t)st.st_size;
    void* m = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (m == MAP_FAILED) {
      set_error("safetensors: mmap failed");
      return -1;
    }
    map = (const uint8_t*)m;
    uint64_t hl = 0;
    for (int i = 0; i < 8; ++i) hl |= (uint64_t)map[i] << (8 * i);
    if (hl > size - 8) {
      set_error("safetensors: header length exceeds the file");
      return -1;
    }
    data_off = 8 + (int64_t)hl;
    if (parse_header((const char*)map + 8, (size_t)hl, tensors)) return -1;
    const int64_t data_size = (int64_t)size - data_off;
    for (auto& t : tensors) {
      int64_t n = 1;
      for (int64_t d : t.shape) {
        if (d < 0) {
          set_error("safetensors: negative dimension in " + t.name);
          return -1;
        }
        if (__builtin_mul_overflow(n, d, &n)) {  // a crafted shape must not wrap
          set_error("safetensors: element count of " + t.name + " overflows");
          return -1;
        }
      }
      const int64_t es = elem_size(t.dtype);
      if (es == 0) {
        set_error("safetensors: unknown dtype " + t.dtype + " for " + t.name);
        return -1;
      }
      int64_t nbytes = 0;
      if (__builtin_mul_overflow(n, es, &nbytes)) {
        set_error("safetensors: byte size of " + t.name + " overflows");
        return -1;
      }
      if (t.begin < 0 || t.end < t.begin || t.end > data_size || t.end - t.begin != nbytes) {
        set_error("safetensors: data offsets of " + t.name + " do not match its shape");
        return -1;
      }
    }
    return 0;
  }

  const TensorEntry* find(const std::string& name) const {
    for (auto& t : tensors)
      if (t.name == name) return &t;
    return nullptr;
  }

  int64_t numel(const TensorEntry& t) const {
    int64_t n = 1;
    for (int64_t d : t.shape) n *= d;
    return n;
  }

  // Convert to fp32 (F32, F16, BF16 only).
  int read_f32(const TensorEntry& t, float* out) const {
    const uint8_t* src = map + data_off + t.begin;
    const int64_t n = numel(t);
    if (t.dtype == "F32") {
      memcpy(out, src, (size_t)n * 4);
    } else if (t.dtype == "F16") {
      for (int64_t i = 0; i < n; ++i) {
        uint16_t h;
        memcpy(&h, src + 2 * i, 2);
        out[i] = half_to_float(h);
      }
    } else if (t.dtype == "BF16") {
      for (int64_t i = 0; i < n; ++i) {
        uint16_t h;
        memcpy(&h, src + 2 * i, 2);
        const uint32_t bits = (uint32_t)h << 16;
        memcpy(&out[i], &bits, 4);
      }
    } else {
      set_error("safetensors: unsupported dtype " + t.dtype + " for " + t.name);
      return -1;
    }
    return 0;
  }
};

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" {

int32_t gs_safetensors_count(const char* path) {
  GS_REQUIRE(path, "safetensors: null path");
  File f;
  if (f.open_file(path)) return -1;
  return (int32_t)f.tensors.size();
}

int32_t gs_safetensors_info(const char* path, int32_t i, char* name_out, int32_t name_cap,
                            char* dtype_out, int64_t shape_out[8], int32_t* ndim_out) {
  GS_REQUIRE(path, "safetensors: null path");
  File f;
  if (f.open_file(path)) return -1;
  GS_REQUIRE(i >= 0 && i < (int32_t)f.tensors.size(), "safetensors: index out of range");
  const TensorEntry& t = f.tensors[i];
  GS_REQUIRE(t.shape.size() <= 8, "safetensors: more than 8 dimensions");
  if (name_out && name_cap > 0) {
    strncpy(name_out, t.name.c_str(), name_cap - 1);
    name_out[name_cap - 1] = 0;
  }
  if (dtype_out) {
    strncpy(dtype_out, t.dtype.c_str(), 7);
    dtype_out[7] = 0;
  }
  if (shape_out)
    for (size_t d = 0; d < 8; ++d) shape_out[d] = d < t.shape.size() ? t.shape[d] : 0;
  if (ndim_out) *ndim_out = (int32_t)t.shape.size();
  return 0;
}

int32_t gs_safetensors_read_f32(const char* path, const char* name, float* host_out, int64_t n) {
  GS_REQUIRE(path && name && host_out, "safetensors: null argument");
  File f;
  if (f.open_file(path)) return -1;
  const TensorEntry* t = f.find(name);
  GS_REQUIRE(t, std::string("safetensors: no tensor ") + name);
  GS_REQUIRE(f.numel(*t) == n, std::string("safetensors: numel mismatch for ") + name);
  return f.read_f32(*t, host_out);
}

int32_t gs_hip_mastr_load_safetensors(void* ctx, const char* path, int32_t* n_loaded,
                                      int32_t* n_unexpected, int32_t* n_missing) {
  GS_REQUIRE(ctx && path, "load_safetensors: null argument");
  File f;
  if (f.open_file(path)) return -1;
  const gs_mastr_config cfg = *mastr_ctx_config(ctx);
  int rc = 0;
  const int32_t nw = gs_mastr_weight_count(&cfg);
  std::map<std::string, std::vector<int64_t>> want;  // inventory name -> shape
  char name[256];
  int64_t shp[4];
  int32_t kind;
  for (int32_t i = 0; i < nw; ++i) {
    gs_mastr_weight_info(&cfg, i, name, sizeof(name), shp, &kind);
    std::vector<int64_t> v;
    for (int d = 0; d < 4 && shp[d]; ++d) v.push_back(shp[d]);
    want[name] = v;
  }
  int32_t loaded = 0, unexpected = 0;
  std::vector<float> buf;
  for (const TensorEntry& t : f.tensors) {
    auto it = want.find(t.name);
    if (it == want.end()) {
      ++unexpected;
      continue;
    }
    if (t.shape != it->second) {
      std::string a, b;
      for (int64_t d : t.shape) a += std::to_string(d) + ",";
      for (int64_t d : it->second) b += std::to_string(d) + ",";
      set_error("load_safetensors: shape of " + t.name + " is [" + a + "], expected [" + b + "]");
      return -1;
    }
    const int64_t n = f.numel(t);
    buf.resize((size_t)n);
    if (f.read_f32(t, buf.data())) return -1;
    rc = gs_hip_mastr_set_weight(ctx, t.name.c_str(), buf.data(), n);
    if (rc) return rc;
    ++loaded;
    want.erase(it);
  }
  if (n_loaded) *n_loaded = loaded;
  if (n_unexpected) *n_unexpected = unexpected;
  if (n_missing) *n_missing = (int32_t)want.size();
  return 0;
}

}  // extern "C"
