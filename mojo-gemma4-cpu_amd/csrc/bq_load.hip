// bq_load.hip -- the on-disk -> device path for butterquant weights:
// safetensors shards (safetensors/parser.mojo) located by tensor name across
// shards (modeling/loader.mojo:151-186), validated against the expected
// quantized member shapes (loader.mojo:52-96; members from
// quant/manifest.mojo:69-199: the int8 codes "<name>" and the f32 scales
// "<name>.scale"), copied to the device and re-tiled to tile16x64 straight
// from the row-major on-disk codes (quant/quantizer.mojo:1028-1036), where
// the reference would pack VNNI tiles and colsums.
//
// The file is memory-mapped; the header is parsed with the reference's
// validation rules (header size bound, required fields, supported dtypes,
// byte size = dtype size x numel, offsets inside the payload, no
// overlapping ranges, no duplicate names, payload fully indexed, nothing
// after the root object).
#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/bq_api.h"
#include "bq_kernels.hpp"

namespace {

int lfail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  const int r = bq::api_failv(code, fmt, ap);
  va_end(ap);
  return r;
}

struct TensorMeta {
  int dtype;
  std::vector<int64_t> shape;
  uint64_t start, end;
};

// dtype tags of safetensors/parser.mojo:19-54 and their byte sizes
struct DtypeTag {
  const char* tag;
  int code;
  int bytes;
};
constexpr DtypeTag kDtypes[] = {
    {"BOOL", BQ_DT_BOOL, 1}, {"U8", BQ_DT_U8, 1},      {"I8", BQ_DT_I8, 1},
    {"I16", BQ_DT_I16, 2},   {"U16", BQ_DT_U16, 2},    {"F16", BQ_DT_F16, 2},
    {"BF16", BQ_DT_BF16, 2}, {"I32", BQ_DT_I32, 4},    {"U32", BQ_DT_U32, 4},
    {"F32", BQ_DT_F32, 4},   {"F64", BQ_DT_F64, 8},    {"F8_E4M3", BQ_DT_F8_E4M3, 1},
    {"F8_E4M3FN", BQ_DT_F8_E4M3, 1}, {"F8_E5M2", BQ_DT_F8_E5M2, 1}, {"I64", BQ_DT_I64, 8},
    {"U64", BQ_DT_U64, 8},
};

int dtype_bytes(int code) {
  for (const auto& d : kDtypes)
    if (d.code == code) return d.bytes;
  return 0;
}

// A small JSON reader for the header: objects, arrays, strings, unsigned
// integers; other scalars are skipped.
struct Json {
  const char* p;
  const char* e;
  bool ok = true;
  std::string err;

  void fail(const char* m) {
    if (ok) err = m;
    ok = false;
  }
  void ws() {
    while (p < e && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
  }
  bool eat(char c) {
    ws();
    if (p < e && *p == c) {
      ++p;
      return true;
    }
    return false;
  }
  std::string str() {
    ws();
    std::string s;
    if (p >= e || *p != '"') {
      fail("expected a string");
      return s;
    }
    ++p;
    while (p < e && *p != '"') {
      if (*p == '\\') {
        if (++p >= e) break;
        switch (*p) {
          case 'n': s += '\n'; break;
          case 't': s += '\t'; break;
          case 'r': s += '\r'; break;
          case 'b': s += '\b'; break;
          case 'f': s += '\f'; break;
          case 'u': {  // keep the escape's code point as UTF-8 (BMP only)
            if (e - p < 5) { fail("bad \\u escape"); return s; }
            unsigned v = 0;
            for (int i = 1; i <= 4; ++i) {
              const char c = p[i];
              v = v * 16 + (c >= '0' && c <= '9' ? c - '0' : c >= 'a' && c <= 'f' ? c - 'a' + 10
                                                         : c >= 'A' && c <= 'F' ? c - 'A' + 10 : 0);
            }
            if (v < 0x80) s += (char)v;
            else if (v < 0x800) { s += (char)(0xC0 | (v >> 6)); s += (char)(0x80 | (v & 63)); }
            else { s += (char)(0xE0 | (v >> 12)); s += (char)(0x80 | ((v >> 6) & 63)); s += (char)(0x80 | (v & 63)); }
            p += 4;
            break;
          }
          default: s += *p;
        }
        ++p;
      } else {
        s += *p++;
      }
    }
    if (p >= e) {
      fail("unterminated string");
      return s;
    }
    ++p;
    return s;
  }
  uint64_t uint() {
    ws();
    if (p >= e || *p < '0' || *p > '9') {
      fail("expected an unsigned integer");
      return 0;
    }
    uint64_t v = 0;
    while (p < e && *p >= '0' && *p <= '9') {
      const uint64_t d = (uint64_t)(*p++ - '0');
      if (v > (UINT64_MAX - d) / 10) {
        fail("integer overflow");
        return 0;
      }
      v = v * 10 + d;
    }
    return v;
  }
  void skip() {  // any value
    ws();
    if (p >= e) { fail("unexpected end"); return; }
    if (*p == '"') { str(); return; }
    if (*p == '{' || *p == '[') {
      const char close = *p == '{' ? '}' : ']';
      const bool obj = *p == '{';
      ++p;
      if (eat(close)) return;
      while (ok) {
        if (obj) {
          str();
          if (!eat(':')) { fail("expected ':'"); return; }
        }
        skip();
        if (eat(',')) continue;
        if (eat(close)) return;
        fail("expected ',' or a closing bracket");
      }
      return;
    }
    while (p < e && *p != ',' && *p != '}' && *p != ']' && *p != ' ' && *p != '\n') ++p;
  }
};

}  // namespace

struct bq_st_file {
  std::string path;
  int fd = -1;
  const uint8_t* map = nullptr;
  size_t len = 0;
  size_t data_offset = 0;
  std::unordered_map<std::string, TensorMeta> tensors;
};

namespace {

int parse_header(bq_st_file* f, const char* h, size_t hlen, uint64_t payload) {
  Json j{h, h + hlen};
  if (!j.eat('{')) return lfail(BQ_ERR_INVALID, "%s: expected '{' at start", f->path.c_str());
  std::vector<std::pair<uint64_t, uint64_t>> ranges;
  uint64_t indexed = 0;
  if (!j.eat('}')) {
    while (j.ok) {
      const std::string key = j.str();
      if (!j.eat(':')) j.fail("expected ':'");
      if (!j.ok) break;
      if (key == "__metadata__") {
        j.skip();
      } else {
        if (f->tensors.count(key)) return lfail(BQ_ERR_INVALID, "%s: duplicate tensor name %s", f->path.c_str(), key.c_str());
        TensorMeta m{-1, {}, 0, 0};
        bool has_off = false, has_dt = false, has_shape = false;
        if (!j.eat('{')) { j.fail("expected '{' for tensor"); break; }
        if (j.eat('}')) return lfail(BQ_ERR_INVALID, "%s: empty tensor object", f->path.c_str());
        while (j.ok) {
          const std::string k = j.str();
          if (!j.eat(':')) { j.fail("expected ':'"); break; }
          if (k == "data_offsets") {
            if (!j.eat('[')) { j.fail("expected '[' for offsets"); break; }
            m.start = j.uint();
            if (!j.eat(',')) { j.fail("expected two offsets"); break; }
            m.end = j.uint();
            if (!j.eat(']')) { j.fail("expected ']' after offsets"); break; }
            has_off = true;
          } else if (k == "dtype") {
            const std::string t = j.str();
            for (const auto& d : kDtypes)
              if (t == d.tag) m.dtype = d.code;
            has_dt = true;
          } else if (k == "shape") {
            if (!j.eat('[')) { j.fail("expected '[' for shape"); break; }
            if (!j.eat(']')) {
              while (j.ok) {
                const uint64_t v = j.uint();
                if (v > (uint64_t)INT64_MAX) { j.fail("shape dimension too large"); break; }
                m.shape.push_back((int64_t)v);
                if (j.eat(',')) continue;
                if (j.eat(']')) break;
                j.fail("expected ',' or ']' in shape");
              }
            }
            has_shape = true;
          } else {
            j.skip();
          }
          if (j.eat(',')) continue;
          if (j.eat('}')) break;
          j.fail("expected ',' or '}' in tensor");
        }
        if (!j.ok) break;
        if (!has_off || !has_dt || !has_shape)
          return lfail(BQ_ERR_INVALID, "%s: tensor %s missing required fields (dtype, shape, data_offsets)", f->path.c_str(), key.c_str());
        if (m.dtype < 0) return lfail(BQ_ERR_INVALID, "%s: tensor %s: unsupported dtype", f->path.c_str(), key.c_str());
        if (m.end < m.start) return lfail(BQ_ERR_INVALID, "%s: tensor %s: invalid offsets", f->path.c_str(), key.c_str());
        if (m.end > payload) return lfail(BQ_ERR_INVALID, "%s: tensor %s: offsets exceed the payload", f->path.c_str(), key.c_str());
        uint64_t n = (uint64_t)dtype_bytes(m.dtype);
        for (int64_t d : m.shape) {
          if (d != 0 && n > UINT64_MAX / (uint64_t)d) return lfail(BQ_ERR_INVALID, "%s: tensor %s: byte size overflow", f->path.c_str(), key.c_str());
          n *= (uint64_t)d;
        }
        if (m.end - m.start != n)
          return lfail(BQ_ERR_INVALID, "%s: tensor %s: byte size does not match dtype and shape", f->path.c_str(), key.c_str());
        for (const auto& r : ranges)
          if (m.start < r.second && m.end > r.first)
            return lfail(BQ_ERR_INVALID, "%s: tensor %s: overlapping data offsets", f->path.c_str(), key.c_str());
        ranges.emplace_back(m.start, m.end);
        indexed += n;
        f->tensors.emplace(key, std::move(m));
      }
      if (j.eat(',')) continue;
      if (j.eat('}')) break;
      j.fail("expected ',' or '}' at the root");
    }
  } else if (payload > 0) {
    return lfail(BQ_ERR_INVALID, "%s: payload bytes are not indexed by tensor metadata", f->path.c_str());
  }
  if (!j.ok) return lfail(BQ_ERR_INVALID, "%s: parse error at byte %zu: %s", f->path.c_str(), (size_t)(j.p - h), j.err.c_str());
  j.ws();
  if (j.p != j.e) return lfail(BQ_ERR_INVALID, "%s: trailing content after the root object", f->path.c_str());
  if (indexed != payload) return lfail(BQ_ERR_INVALID, "%s: payload bytes are not fully indexed by tensor metadata", f->path.c_str());
  return BQ_OK;
}

const TensorMeta* find(const bq_st_file* const* files, int n, const char* name, int* which) {
  for (int i = 0; i < n; ++i) {
    auto it = files[i]->tensors.find(name);
    if (it != files[i]->tensors.end()) {
      *which = i;
      return &it->second;
    }
  }
  return nullptr;
}

// loader.mojo:52-96: the dtype must match; a 1-D shape must hold rows*cols
// elements, a 2-D one be [rows, cols], a 3-D one [a, b, cols] with a*b = rows
int validate(const char* name, const TensorMeta& m, int dtype, int64_t rows, int64_t cols) {
  if (m.dtype != dtype) return lfail(BQ_ERR_SHAPE, "dtype mismatch for %s", name);
  const auto& s = m.shape;
  bool ok;
  if (s.size() == 1) ok = s[0] == rows * cols;
  else if (s.size() == 2) ok = s[0] == rows && s[1] == cols;
  else if (s.size() == 3) ok = s[0] * s[1] == rows && s[2] == cols;
  else return lfail(BQ_ERR_SHAPE, "unexpected rank for %s: %zu", name, s.size());
  if (!ok) return lfail(BQ_ERR_SHAPE, "shape mismatch for %s (expected %lld x %lld)", name, (long long)rows, (long long)cols);
  return BQ_OK;
}

}  // namespace

extern "C" {

int bq_st_open(const char* path, bq_st_file** out) {
  if (!path || !out) return lfail(BQ_ERR_INVALID, "bq_st_open: null pointer");
  *out = nullptr;
  const int fd = open(path, O_RDONLY);
  if (fd < 0) return lfail(BQ_ERR_INVALID, "%s: %s", path, strerror(errno));
  struct stat st;
  if (fstat(fd, &st) != 0) {
    close(fd);
    return lfail(BQ_ERR_INVALID, "%s: %s", path, strerror(errno));
  }
  const size_t len = (size_t)st.st_size;
  if (len < 8) {
    close(fd);
    return lfail(BQ_ERR_INVALID, "%s: file too small", path);
  }
  void* m = mmap(nullptr, len, PROT_READ, MAP_SHARED, fd, 0);
  if (m == MAP_FAILED) {
    close(fd);
    return lfail(BQ_ERR_INVALID, "%s: mmap: %s", path, strerror(errno));
  }
  auto* f = new bq_st_file();
  f->path = path;
  f->fd = fd;
  f->map = static_cast<const uint8_t*>(m);
  f->len = len;
  uint64_t hlen = 0;
  for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | f->map[i];  // little-endian u64
  int rc = BQ_OK;
  if (hlen > 100ull * 1024 * 1024) rc = lfail(BQ_ERR_INVALID, "%s: header too large", path);
  else if (hlen > len - 8) rc = lfail(BQ_ERR_INVALID, "%s: header length exceeds file", path);
  else {
    f->data_offset = 8 + (size_t)hlen;
    rc = parse_header(f, reinterpret_cast<const char*>(f->map + 8), (size_t)hlen,
                      (uint64_t)(len - f->data_offset));
  }
  if (rc != BQ_OK) {
    bq_st_close(f);
    return rc;
  }
  *out = f;
  return BQ_OK;
}

void bq_st_close(bq_st_file* f) {
  if (!f) return;
  if (f->map) munmap(const_cast<uint8_t*>(f->map), f->len);
  if (f->fd >= 0) close(f->fd);
  delete f;
}

int bq_st_num_tensors(const bq_st_file* f) { return f ? (int)f->tensors.size() : 0; }

int bq_st_tensor_info(const bq_st_file* f, const char* name, int* dtype, int* ndim,
                      int64_t* shape, size_t* nbytes, const void** host_data) {
  if (!f || !name) return lfail(BQ_ERR_INVALID, "bq_st_tensor_info: null pointer");
  auto it = f->tensors.find(name);
  if (it == f->tensors.end()) return lfail(BQ_ERR_INVALID, "missing tensor: %s", name);
  const TensorMeta& m = it->second;
  if (m.shape.size() > 8) return lfail(BQ_ERR_UNSUPPORTED, "%s: rank %zu > 8", name, m.shape.size());
  if (dtype) *dtype = m.dtype;
  if (ndim) *ndim = (int)m.shape.size();
  if (shape)
    for (size_t i = 0; i < m.shape.size(); ++i) shape[i] = m.shape[i];
  if (nbytes) *nbytes = (size_t)(m.end - m.start);
  if (host_data) *host_data = f->map + f->data_offset + m.start;
  return BQ_OK;
}

int bq_load_quantized(const bq_st_file* const* files, int n_files, const char* name, int n_rows,
                      int k, int scale_cols, int8_t* w_tiled, float* scales, int8_t* staging,
                      size_t staging_bytes, void* stream) {
  if (!files || n_files <= 0 || !name || !w_tiled || !scales || !staging)
    return lfail(BQ_ERR_INVALID, "bq_load_quantized: null pointer");
  for (int i = 0; i < n_files; ++i)
    if (!files[i]) return lfail(BQ_ERR_INVALID, "bq_load_quantized: null file %d", i);
  if (n_rows <= 0 || n_rows % 16 || k <= 0 || k % 64 || scale_cols <= 0)
    return lfail(BQ_ERR_SHAPE, "bq_load_quantized: need n_rows %% 16 == 0, k %% 64 == 0, scale_cols > 0");
  const size_t strip = (size_t)16 * (size_t)k;
  if (staging_bytes < strip)
    return lfail(BQ_ERR_SHAPE, "bq_load_quantized: staging %zu < one 16-row strip (%zu bytes)", staging_bytes, strip);
  if ((reinterpret_cast<uintptr_t>(w_tiled) | reinterpret_cast<uintptr_t>(staging)) & 15u)
    return lfail(BQ_ERR_INVALID, "bq_load_quantized: w_tiled and staging must be 16-byte aligned");
  int wi = 0, si = 0;
  const TensorMeta* wm = find(files, n_files, name, &wi);
  if (!wm) return lfail(BQ_ERR_INVALID, "missing tensor: %s", name);
  int rc = validate(name, *wm, BQ_DT_I8, n_rows, k);
  if (rc) return rc;
  const std::string sname = std::string(name) + ".scale";  // quant/manifest.mojo:10
  const TensorMeta* sm = find(files, n_files, sname.c_str(), &si);
  if (!sm) return lfail(BQ_ERR_INVALID, "missing tensor: %s", sname.c_str());
  if (scale_cols == 1 && sm->shape.size() == 1) {
    if (sm->dtype != BQ_DT_F32 || sm->shape[0] != n_rows)
      return lfail(BQ_ERR_SHAPE, "dtype or shape mismatch for %s", sname.c_str());
  } else if ((rc = validate(sname.c_str(), *sm, BQ_DT_F32, n_rows, scale_cols))) {
    return rc;
  }
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const uint8_t* wsrc = files[wi]->map + files[wi]->data_offset + wm->start;
  const uint8_t* ssrc = files[si]->map + files[si]->data_offset + sm->start;
  hipError_t e = hipMemcpyAsync(scales, ssrc, (size_t)n_rows * scale_cols * 4, hipMemcpyHostToDevice, st);
  if (e != hipSuccess) return lfail(BQ_ERR_HIP, "bq_load_quantized: scales copy: %s", hipGetErrorString(e));
  // whole 16-row strips per chunk: a strip of the row-major codes maps to one
  // contiguous run of the tiled layout (strip s at s * 16 * k)
  const int rows_per_chunk = (int)(staging_bytes / strip) * 16;
  for (int r0 = 0; r0 < n_rows; r0 += rows_per_chunk) {
    const int rows = n_rows - r0 < rows_per_chunk ? n_rows - r0 : rows_per_chunk;
    e = hipMemcpyAsync(staging, wsrc + (size_t)r0 * k, (size_t)rows * k, hipMemcpyHostToDevice, st);
    if (e != hipSuccess) return lfail(BQ_ERR_HIP, "bq_load_quantized: codes copy: %s", hipGetErrorString(e));
    e = bq::launch_retile(staging, BQ_LAYOUT_ROWMAJOR, w_tiled + (size_t)r0 * k, rows, k, st);
    if (e != hipSuccess) return lfail(BQ_ERR_HIP, "bq_load_quantized: retile: %s", hipGetErrorString(e));
  }
  return BQ_OK;
}

}  // extern "C"
