// dq_gguf.cpp -- GGUF files to device weights: the host side of loading a model.
//
// Opens a GGUF v2 / v3 file read-only with mmap and parses its header, metadata
// and tensor directory, checking every length and offset against the mapping
// (a malformed file gives DQ_CORRUPT, never an access past the end), as
// dynalm's reader does (dynalm/src/loader/gguf/gguf.cpp:248-343). The first part
// of a model split by gguf-split (NAME-00001-of-0000N.gguf, keys split.no /
// split.count / split.tensors.count) opens every part
// (dynalm/src/loader/gguf/gguf_model.cpp:291-331). Tensors of the four weight
// types upload straight from the mapping into the GPU's row-group layout.
//
// The reference's GPU device maps file pages into device address space
// (dynacore/src/gpu/ggml_device_internal.h:295-320) because its kernels read GGUF
// blocks as they lie; the kernels here read the repacked 64-row planes, so every
// weight is copied once (the pages are not held after the upload).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdio>
#include <cstring>
#include <limits>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/dynaq.h"
#include "dq_internal.h"

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF", little-endian
constexpr uint64_t kDefaultAlignment = 32;
constexpr int kMaxDims = 4;
constexpr int kMaxArrayDepth = 2;
constexpr uint64_t kMaxParts = 512;

// GGUF metadata value types (the GGUF format's numbering).
enum VType : uint32_t { kU8, kI8, kU16, kI16, kU32, kI32, kF32, kBool, kStr, kArr, kU64, kI64, kF64 };

size_t scalar_bytes(uint32_t t) {
  switch (t) {
    case kU8: case kI8: case kBool: return 1;
    case kU16: case kI16: return 2;
    case kU32: case kI32: case kF32: return 4;
    case kU64: case kI64: case kF64: return 8;
    default: return 0;
  }
}

// Block geometry of the ggml tensor types (values per block, bytes per block),
// known for every type so that the extents of tensors this library does not run
// are still checked. Zero entries are ids with no type.
struct Geometry {
  uint32_t elems, bytes;
};
Geometry ggml_geometry(uint32_t id) {
  static const Geometry kTable[] = {
      {1, 4},      {1, 2},      {32, 18},    {32, 20},  {0, 0},     {0, 0},     {32, 22},  {32, 24},  // 0-7
      {32, 34},    {32, 36},    {256, 84},   {256, 110}, {256, 144}, {256, 176}, {256, 210}, {256, 292},  // 8-15
      {256, 66},   {256, 74},   {256, 98},   {256, 50}, {32, 18},   {256, 110}, {256, 82}, {256, 136},  // 16-23
      {1, 1},      {1, 2},      {1, 4},      {1, 8},    {1, 8},     {256, 56},  {1, 2},    {0, 0},  // 24-31
      {0, 0},      {0, 0},      {256, 54},   {256, 66}, {0, 0},     {0, 0},     {0, 0},    {32, 17},  // 32-39
  };
  return id < sizeof(kTable) / sizeof(kTable[0]) ? kTable[id] : Geometry{0, 0};
}

// GGUF tensor type id -> dq_dtype of the weight types the kernels run (-1 otherwise).
int dtype_of(uint32_t ggml_type) {
  switch (ggml_type) {
    case 2: return DQ_Q4_0;
    case 8: return DQ_Q8_0;
    case 12: return DQ_Q4_K;
    case 14: return DQ_Q6_K;
    default: return -1;
  }
}

struct Value {
  uint32_t type = kU8;
  uint64_t u = 0;    // unsigned integers and bool
  int64_t i = 0;     // signed integers
  double f = 0.0;    // floats
  const char* s = nullptr;  // string bytes (not NUL-terminated) / array elements
  uint64_t len = 0;         // string length / array count
  uint32_t elem = 0;        // array element type
};

struct Tensor {
  std::string name;
  uint32_t ggml_type = 0;
  int n_dims = 0;
  int64_t dims[kMaxDims] = {0, 0, 0, 0};  // outermost first
  uint64_t offset = 0;                    // absolute offset in its part
  uint64_t nbytes = 0;
  int part = 0;
};

struct Part {
  std::string path;
  const uint8_t* base = nullptr;
  size_t size = 0;
  uint32_t version = 0;
  uint64_t alignment = kDefaultAlignment;
  uint64_t data_offset = 0;
  std::vector<std::pair<std::string, Value>> kvs;
  std::unordered_map<std::string, size_t> kv_index;
  std::vector<Tensor> tensors;
};

// Little-endian cursor over [p, end) that never reads past end.
class Cursor {
 public:
  Cursor(const uint8_t* begin, size_t size) : begin_(begin), p_(begin), end_(begin + size) {}
  size_t offset() const { return (size_t)(p_ - begin_); }
  size_t left() const { return (size_t)(end_ - p_); }
  template <typename T>
  bool get(T& v) {
    if (left() < sizeof(T)) return false;
    std::memcpy(&v, p_, sizeof(T));
    p_ += sizeof(T);
    return true;
  }
  bool skip(uint64_t n) {
    if (n > left()) return false;
    p_ += n;
    return true;
  }
  bool str(const char*& s, uint64_t& n) {
    if (!get(n) || n > left()) return false;
    s = reinterpret_cast<const char*>(p_);
    p_ += n;
    return true;
  }
  const uint8_t* here() const { return p_; }

 private:
  const uint8_t* begin_;
  const uint8_t* p_;
  const uint8_t* end_;
};

int corrupt(const Part& p, const Cursor& c, const char* what) {
  return dq::set_error(DQ_CORRUPT, "GGUF %s: %s at offset %zu", p.path.c_str(), what, c.offset());
}

bool type_ok(uint32_t t) { return t <= kF64; }

// Walks `count` encoded elements of type t (arrays nest at most kMaxArrayDepth deep).
bool skip_elems(Cursor& c, uint32_t t, uint64_t count, int depth) {
  if (t == kStr) {
    for (uint64_t i = 0; i < count; ++i) {
      const char* s;
      uint64_t n;
      if (!c.str(s, n)) return false;
    }
    return true;
  }
  if (t == kArr) {
    if (depth >= kMaxArrayDepth) return false;
    for (uint64_t i = 0; i < count; ++i) {
      uint32_t et;
      uint64_t n;
      if (!c.get(et) || !c.get(n) || !type_ok(et) || !skip_elems(c, et, n, depth + 1)) return false;
    }
    return true;
  }
  const size_t b = scalar_bytes(t);
  return b != 0 && count <= c.left() / b && c.skip(count * b);
}

bool read_value(Cursor& c, uint32_t t, Value& v) {
  v.type = t;
  switch (t) {
    case kU8: { uint8_t x; if (!c.get(x)) return false; v.u = x; return true; }
    case kI8: { int8_t x; if (!c.get(x)) return false; v.i = x; return true; }
    case kU16: { uint16_t x; if (!c.get(x)) return false; v.u = x; return true; }
    case kI16: { int16_t x; if (!c.get(x)) return false; v.i = x; return true; }
    case kU32: { uint32_t x; if (!c.get(x)) return false; v.u = x; return true; }
    case kI32: { int32_t x; if (!c.get(x)) return false; v.i = x; return true; }
    case kU64: { uint64_t x; if (!c.get(x)) return false; v.u = x; return true; }
    case kI64: { int64_t x; if (!c.get(x)) return false; v.i = x; return true; }
    case kF32: { float x; if (!c.get(x)) return false; v.f = x; return true; }
    case kF64: { double x; if (!c.get(x)) return false; v.f = x; return true; }
    case kBool: { uint8_t x; if (!c.get(x) || x > 1) return false; v.u = x; return true; }
    case kStr: return c.str(v.s, v.len);
    case kArr: {
      if (!c.get(v.elem) || !c.get(v.len) || !type_ok(v.elem)) return false;
      v.s = reinterpret_cast<const char*>(c.here());
      return skip_elems(c, v.elem, v.len, 1);
    }
    default: return false;
  }
}

bool is_int(uint32_t t) { return t == kU8 || t == kI8 || t == kU16 || t == kI16 || t == kU32 || t == kI32 || t == kU64 || t == kI64; }
bool is_signed(uint32_t t) { return t == kI8 || t == kI16 || t == kI32 || t == kI64; }

int map_file(const std::string& path, Part& p) {
  p.path = path;
  const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) {
    const int err = errno;
    return dq::set_error(err == ENOENT ? DQ_NOT_FOUND : DQ_IO_ERROR, "GGUF %s: %s", path.c_str(), std::strerror(err));
  }
  struct stat st;
  if (::fstat(fd, &st) != 0) {
    const int err = errno;
    ::close(fd);
    return dq::set_error(DQ_IO_ERROR, "GGUF %s: %s", path.c_str(), std::strerror(err));
  }
  p.size = (size_t)st.st_size;
  if (p.size < 24) {
    ::close(fd);
    return dq::set_error(DQ_CORRUPT, "GGUF %s: not a GGUF file (%zu bytes)", path.c_str(), p.size);
  }
  void* m = ::mmap(nullptr, p.size, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (m == MAP_FAILED) return dq::set_error(DQ_IO_ERROR, "GGUF %s: mmap: %s", path.c_str(), std::strerror(errno));
  p.base = static_cast<const uint8_t*>(m);
  return DQ_OK;
}

int parse(Part& p) {
  Cursor c(p.base, p.size);
  uint32_t magic;
  if (!c.get(magic) || magic != kMagic) return dq::set_error(DQ_CORRUPT, "GGUF %s: bad magic", p.path.c_str());
  if (!c.get(p.version)) return corrupt(p, c, "truncated header");
  if (p.version < 2 || p.version > 3) {
    return dq::set_error(DQ_UNSUPPORTED, "GGUF %s: version %u (2 and 3 are supported)", p.path.c_str(), p.version);
  }
  uint64_t n_tensors, n_kv;
  if (!c.get(n_tensors) || !c.get(n_kv)) return corrupt(p, c, "truncated header");
  // a key/value takes at least 12 bytes and a tensor entry at least 28
  if (n_kv > c.left() / 12 || n_tensors > c.left() / 28) return corrupt(p, c, "implausible tensor / key counts");
  p.kvs.reserve((size_t)n_kv);
  for (uint64_t i = 0; i < n_kv; ++i) {
    const char* ks;
    uint64_t kn;
    uint32_t t;
    if (!c.str(ks, kn) || !c.get(t)) return corrupt(p, c, "truncated metadata key");
    if (!type_ok(t)) return corrupt(p, c, "unknown metadata value type");
    Value v;
    if (!read_value(c, t, v)) return corrupt(p, c, "truncated or invalid metadata value");
    std::string key(ks, (size_t)kn);
    if (!p.kv_index.emplace(key, p.kvs.size()).second) {
      return dq::set_error(DQ_CORRUPT, "GGUF %s: duplicate metadata key '%s'", p.path.c_str(), key.c_str());
    }
    p.kvs.emplace_back(std::move(key), v);
  }
  if (auto it = p.kv_index.find("general.alignment"); it != p.kv_index.end()) {
    const Value& a = p.kvs[it->second].second;
    const uint64_t al = is_signed(a.type) ? (uint64_t)a.i : a.u;
    if (!is_int(a.type) || (is_signed(a.type) && a.i <= 0) || al == 0 || (al & (al - 1)) != 0) {
      return dq::set_error(DQ_CORRUPT, "GGUF %s: general.alignment must be a power of two", p.path.c_str());
    }
    p.alignment = al;
  }
  std::unordered_map<std::string, size_t> names;
  p.tensors.reserve((size_t)n_tensors);
  for (uint64_t i = 0; i < n_tensors; ++i) {
    Tensor t;
    const char* ns;
    uint64_t nn;
    uint32_t nd;
    if (!c.str(ns, nn) || !c.get(nd)) return corrupt(p, c, "truncated tensor entry");
    t.name.assign(ns, (size_t)nn);
    if (nd == 0 || nd > (uint32_t)kMaxDims) {
      return dq::set_error(DQ_CORRUPT, "GGUF %s: tensor '%s' has %u dims", p.path.c_str(), t.name.c_str(), nd);
    }
    t.n_dims = (int)nd;
    uint64_t numel = 1;
    for (uint32_t d = 0; d < nd; ++d) {
      uint64_t ne;
      if (!c.get(ne)) return corrupt(p, c, "truncated tensor dims");
      if (ne > (uint64_t)std::numeric_limits<int64_t>::max() ||
          (ne != 0 && numel > std::numeric_limits<uint64_t>::max() / ne)) {
        return corrupt(p, c, "tensor dims overflow");
      }
      numel *= ne;
      t.dims[nd - 1 - d] = (int64_t)ne;  // GGUF lists the innermost dim first
    }
    if (!c.get(t.ggml_type) || !c.get(t.offset)) return corrupt(p, c, "truncated tensor entry");
    const Geometry g = ggml_geometry(t.ggml_type);
    if (g.elems == 0) {
      return dq::set_error(DQ_UNSUPPORTED, "GGUF %s: tensor '%s' has unknown ggml type %u", p.path.c_str(),
                           t.name.c_str(), t.ggml_type);
    }
    if ((uint64_t)t.dims[nd - 1] % g.elems != 0) {
      return dq::set_error(DQ_CORRUPT, "GGUF %s: tensor '%s' row is not a whole number of blocks", p.path.c_str(),
                           t.name.c_str());
    }
    t.nbytes = numel / g.elems * g.bytes;
    if (!names.emplace(t.name, p.tensors.size()).second) {
      return dq::set_error(DQ_CORRUPT, "GGUF %s: duplicate tensor '%s'", p.path.c_str(), t.name.c_str());
    }
    p.tensors.push_back(std::move(t));
  }
  // tensor data starts at the first alignment boundary after the directory
  p.data_offset = ((uint64_t)c.offset() + p.alignment - 1) / p.alignment * p.alignment;
  for (Tensor& t : p.tensors) {
    if (t.offset % p.alignment != 0) {
      return dq::set_error(DQ_CORRUPT, "GGUF %s: tensor '%s' data is misaligned", p.path.c_str(), t.name.c_str());
    }
    if (p.data_offset > p.size || t.offset > p.size - p.data_offset || t.nbytes > p.size - p.data_offset - t.offset) {
      return dq::set_error(DQ_CORRUPT, "GGUF %s: tensor '%s' extends past the end of the file", p.path.c_str(),
                           t.name.c_str());
    }
    t.offset += p.data_offset;
  }
  return DQ_OK;
}

const Value* find_kv(const Part& p, const char* key) {
  auto it = p.kv_index.find(key);
  return it == p.kv_index.end() ? nullptr : &p.kvs[it->second].second;
}

bool get_u(const Part& p, const char* key, uint64_t& out) {
  const Value* v = find_kv(p, key);
  if (v == nullptr || !is_int(v->type) || (is_signed(v->type) && v->i < 0)) return false;
  out = is_signed(v->type) ? (uint64_t)v->i : v->u;
  return true;
}

}  // namespace

struct dq_gguf {
  std::vector<Part> parts;
  std::vector<Tensor> tensors;  // all parts, in part order
  std::unordered_map<std::string, int64_t> index;
  ~dq_gguf() {
    for (Part& p : parts)
      if (p.base != nullptr) ::munmap(const_cast<uint8_t*>(p.base), p.size);
  }
};

namespace {

int open_part(const std::string& path, Part& p) {
  if (int rc = map_file(path, p); rc != DQ_OK) return rc;
  return parse(p);
}

}  // namespace

extern "C" {

int dq_gguf_open(const char* path, dq_gguf** out) {
  if (path == nullptr || out == nullptr) return dq::set_error(DQ_INVALID_ARGUMENT, "null argument");
  *out = nullptr;
  auto* g = new (std::nothrow) dq_gguf();
  if (g == nullptr) return dq::set_error(DQ_OUT_OF_MEMORY, "host allocation failed");
  g->parts.emplace_back();
  int rc = open_part(path, g->parts[0]);
  uint64_t count = 1;
  if (rc == DQ_OK && get_u(g->parts[0], "split.count", count) && count > 1) {
    uint64_t no = 0;
    const std::string p0 = path;
    char tail[48];
    std::snprintf(tail, sizeof tail, "-%05d-of-%05d.gguf", 1, (int)(count > kMaxParts ? 0 : count));
    const size_t tl = std::strlen(tail);
    if (count > kMaxParts) {
      rc = dq::set_error(DQ_CORRUPT, "GGUF %s: split.count %llu is out of range", path, (unsigned long long)count);
    } else if (!get_u(g->parts[0], "split.no", no) || no != 0) {
      rc = dq::set_error(DQ_INVALID_ARGUMENT, "GGUF %s is not the first part of its split model (open ...%s)", path, tail);
    } else if (p0.size() < tl || p0.compare(p0.size() - tl, tl, tail) != 0) {
      rc = dq::set_error(DQ_INVALID_ARGUMENT, "split model %s: expected a name ending in %s", path, tail);
    } else {
      const std::string prefix = p0.substr(0, p0.size() - tl);
      for (uint64_t i = 1; i < count && rc == DQ_OK; ++i) {
        std::snprintf(tail, sizeof tail, "-%05d-of-%05d.gguf", (int)(i + 1), (int)count);
        g->parts.emplace_back();
        Part& part = g->parts.back();
        rc = open_part(prefix + tail, part);
        uint64_t pno = 0, pcount = 0;
        if (rc == DQ_OK && (!get_u(part, "split.no", pno) || pno != i || !get_u(part, "split.count", pcount) ||
                            pcount != count)) {
          rc = dq::set_error(DQ_CORRUPT, "split model: %s is not part %llu of %llu", part.path.c_str(),
                             (unsigned long long)(i + 1), (unsigned long long)count);
        }
      }
    }
  }
  if (rc == DQ_OK) {
    for (size_t pi = 0; pi < g->parts.size() && rc == DQ_OK; ++pi) {
      for (Tensor& t : g->parts[pi].tensors) {
        t.part = (int)pi;
        if (!g->index.emplace(t.name, (int64_t)g->tensors.size()).second) {
          rc = dq::set_error(DQ_CORRUPT, "GGUF %s: tensor '%s' appears in two parts", path, t.name.c_str());
          break;
        }
        g->tensors.push_back(t);
      }
    }
    uint64_t want = 0;
    if (rc == DQ_OK && g->parts.size() > 1 && get_u(g->parts[0], "split.tensors.count", want) &&
        want != g->tensors.size()) {
      rc = dq::set_error(DQ_CORRUPT, "split model %s: the parts hold %zu tensors, the first part lists %llu", path,
                         g->tensors.size(), (unsigned long long)want);
    }
  }
  if (rc != DQ_OK) {
    delete g;
    return rc;
  }
  *out = g;
  return DQ_OK;
}

int dq_gguf_close(dq_gguf* g) {
  delete g;
  return DQ_OK;
}

int dq_gguf_info(const dq_gguf* g, uint32_t* version, uint64_t* alignment, int64_t* n_tensors, int64_t* n_parts) {
  if (g == nullptr) return dq::set_error(DQ_INVALID_ARGUMENT, "null handle");
  if (version) *version = g->parts[0].version;
  if (alignment) *alignment = g->parts[0].alignment;
  if (n_tensors) *n_tensors = (int64_t)g->tensors.size();
  if (n_parts) *n_parts = (int64_t)g->parts.size();
  return DQ_OK;
}

int64_t dq_gguf_find_tensor(const dq_gguf* g, const char* name) {
  if (g == nullptr || name == nullptr) return -1;
  auto it = g->index.find(name);
  return it == g->index.end() ? -1 : it->second;
}

int dq_gguf_tensor_info(const dq_gguf* g, int64_t i, dq_gguf_tensor* out) {
  if (g == nullptr || out == nullptr) return dq::set_error(DQ_INVALID_ARGUMENT, "null argument");
  if (i < 0 || i >= (int64_t)g->tensors.size()) {
    return dq::set_error(DQ_INVALID_ARGUMENT, "tensor index %lld outside [0, %zu)", (long long)i, g->tensors.size());
  }
  const Tensor& t = g->tensors[(size_t)i];
  out->name = t.name.c_str();
  out->ggml_type = t.ggml_type;
  out->dtype = dtype_of(t.ggml_type);
  out->n_dims = t.n_dims;
  for (int d = 0; d < kMaxDims; ++d) out->dims[d] = d < t.n_dims ? t.dims[d] : 0;
  out->offset = t.offset;
  out->nbytes = t.nbytes;
  out->part = t.part;
  out->data = g->parts[(size_t)t.part].base + t.offset;
  return DQ_OK;
}

int dq_gguf_get_uint(const dq_gguf* g, const char* key, uint64_t* out) {
  if (g == nullptr || key == nullptr || out == nullptr) return dq::set_error(DQ_INVALID_ARGUMENT, "null argument");
  const Value* v = find_kv(g->parts[0], key);
  if (v == nullptr) return dq::set_error(DQ_NOT_FOUND, "GGUF key '%s' not found", key);
  if (!is_int(v->type) || (is_signed(v->type) && v->i < 0)) {
    return dq::set_error(DQ_INVALID_ARGUMENT, "GGUF key '%s' is not a non-negative integer", key);
  }
  *out = is_signed(v->type) ? (uint64_t)v->i : v->u;
  return DQ_OK;
}

int dq_gguf_get_string(const dq_gguf* g, const char* key, const char** str, int64_t* len) {
  if (g == nullptr || key == nullptr || str == nullptr || len == nullptr) {
    return dq::set_error(DQ_INVALID_ARGUMENT, "null argument");
  }
  const Value* v = find_kv(g->parts[0], key);
  if (v == nullptr) return dq::set_error(DQ_NOT_FOUND, "GGUF key '%s' not found", key);
  if (v->type != kStr) return dq::set_error(DQ_INVALID_ARGUMENT, "GGUF key '%s' is not a string", key);
  *str = v->s;
  *len = (int64_t)v->len;
  return DQ_OK;
}

int dq_gguf_upload_weight(const dq_gguf* g, int64_t i, void* stream, dq_weight** out) {
  if (out == nullptr) return dq::set_error(DQ_INVALID_ARGUMENT, "null argument");
  *out = nullptr;
  dq_gguf_tensor t;
  if (int rc = dq_gguf_tensor_info(g, i, &t); rc != DQ_OK) return rc;
  if (t.dtype < 0) {
    return dq::set_error(DQ_UNSUPPORTED, "tensor '%s': ggml type %u is not a weight type of this library", t.name,
                         t.ggml_type);
  }
  if (t.n_dims < 2) return dq::set_error(DQ_INVALID_ARGUMENT, "tensor '%s' is not a matrix", t.name);
  int64_t n = 1;
  for (int d = 0; d + 1 < t.n_dims; ++d) n *= t.dims[d];  // outer dims (experts x rows) as rows
  const int64_t k = t.dims[t.n_dims - 1];
  const int64_t rb = dq_row_bytes(t.dtype, k);
  if (rb <= 0 || (uint64_t)(n * rb) != t.nbytes) {
    return dq::set_error(DQ_CORRUPT, "tensor '%s': %llu bytes for %lld rows of %lld values", t.name,
                         (unsigned long long)t.nbytes, (long long)n, (long long)k);
  }
  return dq_weight_upload(t.dtype, t.data, n, k, rb, stream, out);
}

}  // extern "C"
