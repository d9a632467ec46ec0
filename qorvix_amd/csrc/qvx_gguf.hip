// qvx_gguf.hip -- GGUF file reader and weight upload of libqvx.so (host code only; declared in
// include/qvx.h, qvx_gguf_*).
//
// Parses the public GGUF container (versions 1-3: header, metadata key/value table, tensor table,
// aligned tensor-data section) from a read-only memory map or a caller's buffer, with the checks of
// the reference's GgufFile::parse (gguf/src/gguf_file.cpp:95-180): bad magic, unsupported version,
// unknown or nested metadata value types, truncation, array lengths that cannot fit, rank > 8,
// element-count overflow, element counts that are not whole blocks, tensor offsets that are not
// aligned, and tensor extents past the data section (checked when the buffer carries it).  Tensor
// data is only located; qvx_gguf_upload copies a tensor's raw blocks to the device, where the
// GEMV / GEMM entry points read them as they are (no repack).
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <limits>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/qvx.h"
#include "qvx_common.hpp"

namespace {

constexpr uint32_t kGgufMagic = 0x46554747u;  // "GGUF" little-endian
constexpr uint32_t kDefaultAlign = 32u;
constexpr uint32_t kMaxRank = 8u;

// Metadata value type tags of the format (0..12).
enum MetaTag : uint32_t {
  M_U8 = 0, M_I8 = 1, M_U16 = 2, M_I16 = 3, M_U32 = 4, M_I32 = 5, M_F32 = 6,
  M_BOOL = 7, M_STR = 8, M_ARR = 9, M_U64 = 10, M_I64 = 11, M_F64 = 12,
};

struct ParseError {
  std::string msg;
};

// One metadata value: a scalar (kept as the widest integer / double it fits), a string, or an
// array of scalars or strings of one element type.
struct Value {
  uint32_t tag = M_U8;
  uint32_t elem = M_U8;  // array element type
  bool is_int = false, is_signed = false, is_float = false;
  uint64_t u = 0;
  int64_t i = 0;
  double f = 0.0;
  std::string s;
  std::vector<Value> arr;
};

struct Tensor {
  std::string name;
  std::vector<uint64_t> dims;
  uint32_t type = 0;
  uint64_t offset = 0, n_elements = 0, n_bytes = 0;
};

class Reader {
 public:
  Reader(const uint8_t* p, size_t n) : p_(p), n_(n) {}
  size_t pos() const { return pos_; }
  size_t remaining() const { return n_ - pos_; }
  template <typename T>
  T get() {
    need(sizeof(T));
    T v;
    std::memcpy(&v, p_ + pos_, sizeof(T));
    pos_ += sizeof(T);
    return v;
  }
  std::string str(bool wide) {
    const uint64_t len = wide ? get<uint64_t>() : get<uint32_t>();
    need(len);
    std::string s(reinterpret_cast<const char*>(p_ + pos_), (size_t)len);
    pos_ += (size_t)len;
    return s;
  }

 private:
  void need(uint64_t k) {
    if (k > remaining()) throw ParseError{"truncated GGUF data at byte " + std::to_string(pos_)};
  }
  const uint8_t* p_;
  size_t n_, pos_ = 0;
};

Value scalar(Reader& r, uint32_t tag, bool wide) {
  Value v;
  v.tag = tag;
  switch (tag) {
    case M_U8: v.is_int = true; v.u = r.get<uint8_t>(); v.i = (int64_t)v.u; break;
    case M_I8: v.is_int = v.is_signed = true; v.i = r.get<int8_t>(); v.u = (uint64_t)v.i; break;
    case M_U16: v.is_int = true; v.u = r.get<uint16_t>(); v.i = (int64_t)v.u; break;
    case M_I16: v.is_int = v.is_signed = true; v.i = r.get<int16_t>(); v.u = (uint64_t)v.i; break;
    case M_U32: v.is_int = true; v.u = r.get<uint32_t>(); v.i = (int64_t)v.u; break;
    case M_I32: v.is_int = v.is_signed = true; v.i = r.get<int32_t>(); v.u = (uint64_t)v.i; break;
    case M_U64: v.is_int = true; v.u = r.get<uint64_t>(); v.i = (int64_t)v.u; break;
    case M_I64: v.is_int = v.is_signed = true; v.i = r.get<int64_t>(); v.u = (uint64_t)v.i; break;
    case M_F32: v.is_float = true; v.f = r.get<float>(); break;
    case M_F64: v.is_float = true; v.f = r.get<double>(); break;
    case M_BOOL: v.u = r.get<uint8_t>() != 0 ? 1u : 0u; v.i = (int64_t)v.u; break;
    case M_STR: v.s = r.str(wide); break;
    case M_ARR: throw ParseError{"nested arrays are not permitted in GGUF metadata"};
    default: throw ParseError{"unknown metadata value type " + std::to_string(tag)};
  }
  return v;
}

// Fewest bytes one array element of `tag` occupies (to refuse impossible lengths up front).
uint64_t min_elem_bytes(uint32_t tag, bool wide) {
  switch (tag) {
    case M_U8: case M_I8: case M_BOOL: return 1;
    case M_U16: case M_I16: return 2;
    case M_U32: case M_I32: case M_F32: return 4;
    case M_U64: case M_I64: case M_F64: return 8;
    case M_STR: return wide ? 8 : 4;
    default: return 0;
  }
}

Value value(Reader& r, uint32_t tag, bool wide) {
  if (tag != M_ARR) return scalar(r, tag, wide);
  Value v;
  v.tag = M_ARR;
  v.elem = r.get<uint32_t>();
  if (v.elem == M_ARR) throw ParseError{"nested arrays are not permitted in GGUF metadata"};
  if (v.elem > M_F64) throw ParseError{"unknown metadata value type " + std::to_string(v.elem)};
  const uint64_t len = wide ? r.get<uint64_t>() : r.get<uint32_t>();
  const uint64_t mb = min_elem_bytes(v.elem, wide);
  if (mb > 0 && len > r.remaining() / mb)
    throw ParseError{"array length " + std::to_string(len) + " exceeds remaining buffer"};
  v.arr.reserve((size_t)len);
  for (uint64_t k = 0; k < len; ++k) v.arr.push_back(scalar(r, v.elem, wide));
  return v;
}

}  // namespace

// A parsed GGUF file (include/qvx.h, qvx_gguf_*).
struct qvx_gguf {
  uint32_t version = 0, alignment = kDefaultAlign;
  uint64_t tensor_count = 0, meta_count = 0, data_offset = 0;
  std::vector<std::pair<std::string, Value>> meta;
  std::unordered_map<std::string, size_t> meta_index;
  std::vector<Tensor> tensors;
  std::unordered_map<std::string, size_t> tensor_index;
  const uint8_t* base = nullptr;  // the mapping or the caller's buffer
  size_t size = 0;
  void* map = nullptr;            // owned mapping (open), else null
  size_t map_size = 0;

  const Value* find(const char* key) const {
    if (!key) return nullptr;
    auto it = meta_index.find(key);
    return it == meta_index.end() ? nullptr : &meta[it->second].second;
  }

  void parse() {
    Reader r(base, size);
    if (r.get<uint32_t>() != kGgufMagic) throw ParseError{"not a GGUF file (bad magic)"};
    version = r.get<uint32_t>();
    if (version < 1 || version > 3) throw ParseError{"unsupported GGUF version " + std::to_string(version)};
    const bool wide = version >= 2;  // v2 and v3: 64-bit counts, lengths and dimensions
    tensor_count = wide ? r.get<uint64_t>() : r.get<uint32_t>();
    meta_count = wide ? r.get<uint64_t>() : r.get<uint32_t>();
    for (uint64_t k = 0; k < meta_count; ++k) {
      std::string key = r.str(wide);
      const uint32_t tag = r.get<uint32_t>();
      Value v = value(r, tag, wide);
      meta_index[key] = meta.size();
      meta.emplace_back(std::move(key), std::move(v));
    }
    if (const Value* a = find("general.alignment"); a && (a->is_int || a->tag == M_BOOL)) {
      alignment = (uint32_t)a->u;
      if (alignment == 0) alignment = kDefaultAlign;
    }
    for (uint64_t k = 0; k < tensor_count; ++k) {
      Tensor t;
      t.name = r.str(wide);
      const uint32_t nd = r.get<uint32_t>();
      if (nd > kMaxRank)
        throw ParseError{"tensor '" + t.name + "' has implausible rank " + std::to_string(nd)};
      for (uint32_t d = 0; d < nd; ++d) t.dims.push_back(wide ? r.get<uint64_t>() : r.get<uint32_t>());
      t.type = r.get<uint32_t>();
      t.offset = r.get<uint64_t>();
      uint64_t n = 1;
      for (uint64_t d : t.dims) {
        if (d == 0) {
          n = 0;
          break;
        }
        if (n > std::numeric_limits<uint64_t>::max() / d)
          throw ParseError{"tensor '" + t.name + "' element count overflows uint64"};
        n *= d;
      }
      t.n_elements = n;
      if (const qvx::TypeInfo* ti = qvx::type_info(t.type)) {
        if (ti->block > 1 && n % ti->block != 0)
          throw ParseError{"tensor '" + t.name + "' element count " + std::to_string(n) +
                           " is not a multiple of block size " + std::to_string(ti->block)};
        t.n_bytes = n / ti->block * ti->bytes;
      }
      if (t.offset % alignment != 0)
        throw ParseError{"tensor '" + t.name + "' offset " + std::to_string(t.offset) + " is not aligned to " +
                         std::to_string(alignment)};
      tensor_index[t.name] = tensors.size();
      tensors.push_back(std::move(t));
    }
    const uint64_t p = r.pos();
    data_offset = (p + alignment - 1) / alignment * alignment;
    if (size > data_offset) {  // the buffer carries the data section: every extent must fit in it
      const uint64_t avail = size - data_offset;
      for (const Tensor& t : tensors)
        if (t.n_bytes && (t.offset > avail || t.n_bytes > avail - t.offset))
          throw ParseError{"tensor '" + t.name + "' data extent exceeds the tensor-data section"};
    }
  }

  ~qvx_gguf() {
    if (map) munmap(map, map_size);
  }
};

namespace {

thread_local std::string g_gguf_error;

int fail(qvx_gguf* f, int code, std::string msg) {
  delete f;
  g_gguf_error = std::move(msg);
  return code;
}

const Tensor* tensor_at(const qvx_gguf* f, int64_t i) {
  if (!f || i < 0 || (uint64_t)i >= f->tensors.size()) return nullptr;
  return &f->tensors[(size_t)i];
}

}  // namespace

#pragma GCC visibility push(default)
extern "C" {

int qvx_gguf_parse(const void* data, size_t size, qvx_gguf** out) {
  if (!out) return QVX_E_NULL;
  *out = nullptr;
  if (!data && size) return QVX_E_NULL;
  auto* f = new (std::nothrow) qvx_gguf;
  if (!f) return QVX_E_HIP;
  f->base = static_cast<const uint8_t*>(data);
  f->size = size;
  try {
    f->parse();
  } catch (const ParseError& e) {
    return fail(f, QVX_E_FORMAT, e.msg);
  } catch (const std::bad_alloc&) {
    return fail(f, QVX_E_FORMAT, "GGUF table too large to hold");
  }
  g_gguf_error.clear();
  *out = f;
  return QVX_OK;
}

int qvx_gguf_open(const char* path, qvx_gguf** out) {
  if (!out || !path) return QVX_E_NULL;
  *out = nullptr;
  const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) {
    g_gguf_error = std::string("cannot open '") + path + "': " + std::strerror(errno);
    return QVX_E_IO;
  }
  struct stat st {};
  if (fstat(fd, &st) != 0 || st.st_size <= 0) {
    g_gguf_error = std::string("cannot map '") + path + "': empty or unreadable";
    ::close(fd);
    return QVX_E_IO;
  }
  void* m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (m == MAP_FAILED) {
    g_gguf_error = std::string("cannot map '") + path + "': " + std::strerror(errno);
    return QVX_E_IO;
  }
  auto* f = new (std::nothrow) qvx_gguf;
  if (!f) {
    munmap(m, (size_t)st.st_size);
    return QVX_E_HIP;
  }
  f->map = m;
  f->map_size = (size_t)st.st_size;
  f->base = static_cast<const uint8_t*>(m);
  f->size = (size_t)st.st_size;
  try {
    f->parse();
  } catch (const ParseError& e) {
    return fail(f, QVX_E_FORMAT, e.msg);
  } catch (const std::bad_alloc&) {
    return fail(f, QVX_E_FORMAT, "GGUF table too large to hold");
  }
  g_gguf_error.clear();
  *out = f;
  return QVX_OK;
}

void qvx_gguf_close(qvx_gguf* f) { delete f; }

const char* qvx_gguf_last_error(void) { return g_gguf_error.c_str(); }

uint32_t qvx_gguf_version(const qvx_gguf* f) { return f ? f->version : 0; }
uint32_t qvx_gguf_alignment(const qvx_gguf* f) { return f ? f->alignment : 0; }
uint64_t qvx_gguf_data_offset(const qvx_gguf* f) { return f ? f->data_offset : 0; }
int64_t qvx_gguf_tensor_count(const qvx_gguf* f) { return f ? (int64_t)f->tensors.size() : 0; }
int64_t qvx_gguf_meta_count(const qvx_gguf* f) { return f ? (int64_t)f->meta.size() : 0; }

int64_t qvx_gguf_find_tensor(const qvx_gguf* f, const char* name) {
  if (!f || !name) return -1;
  auto it = f->tensor_index.find(name);
  return it == f->tensor_index.end() ? -1 : (int64_t)it->second;
}

int qvx_gguf_tensor_info(const qvx_gguf* f, int64_t i, const char** name, uint32_t* type, uint32_t* n_dims,
                         uint64_t* dims, uint64_t* offset, uint64_t* n_elements, uint64_t* n_bytes) {
  const Tensor* t = tensor_at(f, i);
  if (!t) return QVX_E_RANGE;
  if (name) *name = t->name.c_str();
  if (type) *type = t->type;
  if (n_dims) *n_dims = (uint32_t)t->dims.size();
  if (dims)
    for (size_t d = 0; d < kMaxRank; ++d) dims[d] = d < t->dims.size() ? t->dims[d] : 0;
  if (offset) *offset = t->offset;
  if (n_elements) *n_elements = t->n_elements;
  if (n_bytes) *n_bytes = t->n_bytes;
  return QVX_OK;
}

const void* qvx_gguf_tensor_data(const qvx_gguf* f, int64_t i) {
  const Tensor* t = tensor_at(f, i);
  if (!t || f->data_offset + t->offset + t->n_bytes > f->size || (t->n_bytes == 0 && t->n_elements != 0)) return nullptr;
  return f->base + f->data_offset + t->offset;
}

int qvx_gguf_upload(const qvx_gguf* f, int64_t i, void* d_dst, size_t dst_bytes, void* stream) {
  const Tensor* t = tensor_at(f, i);
  if (!t) return QVX_E_RANGE;
  if (t->n_bytes == 0 && t->n_elements != 0) return QVX_E_TYPE;  // a type whose size is unknown
  const void* src = qvx_gguf_tensor_data(f, i);
  if (!src) return QVX_E_RANGE;  // the buffer does not carry this tensor's data
  if (!d_dst) return QVX_E_NULL;
  if (dst_bytes < t->n_bytes) return QVX_E_RANGE;
  if (t->n_bytes == 0) return QVX_OK;
  if (hipMemcpyAsync(d_dst, src, (size_t)t->n_bytes, hipMemcpyHostToDevice, static_cast<hipStream_t>(stream)) !=
      hipSuccess) {
    (void)hipGetLastError();
    return QVX_E_HIP;
  }
  return QVX_OK;
}

const char* qvx_gguf_meta_key(const qvx_gguf* f, int64_t i) {
  if (!f || i < 0 || (uint64_t)i >= f->meta.size()) return nullptr;
  return f->meta[(size_t)i].first.c_str();
}

int qvx_gguf_meta_type(const qvx_gguf* f, const char* key, uint32_t* type, uint32_t* elem_type, uint64_t* count) {
  const Value* v = f ? f->find(key) : nullptr;
  if (!v) return QVX_E_RANGE;
  if (type) *type = v->tag;
  if (elem_type) *elem_type = v->tag == M_ARR ? v->elem : v->tag;
  if (count) *count = v->tag == M_ARR ? (uint64_t)v->arr.size() : 1;
  return QVX_OK;
}

// Element `index` of `key` (index 0 for a scalar): the widening rules of the reference's
// GgufValue accessors (gguf/src/gguf_types.cpp:82-120): integers and bools widen to u64 / i64,
// every number but a bool to f64, strings only as strings.  Wrong category -> QVX_E_TYPE.
static const Value* meta_elem(const qvx_gguf* f, const char* key, uint64_t index) {
  const Value* v = f ? f->find(key) : nullptr;
  if (!v) return nullptr;
  if (v->tag == M_ARR) return index < v->arr.size() ? &v->arr[(size_t)index] : nullptr;
  return index == 0 ? v : nullptr;
}

int qvx_gguf_meta_u64(const qvx_gguf* f, const char* key, uint64_t index, uint64_t* out) {
  const Value* v = meta_elem(f, key, index);
  if (!v) return QVX_E_RANGE;
  if (!(v->is_int || v->tag == M_BOOL)) return QVX_E_TYPE;
  if (out) *out = v->u;
  return QVX_OK;
}

int qvx_gguf_meta_i64(const qvx_gguf* f, const char* key, uint64_t index, int64_t* out) {
  const Value* v = meta_elem(f, key, index);
  if (!v) return QVX_E_RANGE;
  if (!(v->is_int || v->tag == M_BOOL)) return QVX_E_TYPE;
  if (out) *out = v->i;
  return QVX_OK;
}

int qvx_gguf_meta_f64(const qvx_gguf* f, const char* key, uint64_t index, double* out) {
  const Value* v = meta_elem(f, key, index);
  if (!v) return QVX_E_RANGE;
  if (!(v->is_int || v->is_float)) return QVX_E_TYPE;
  if (out) *out = v->is_float ? v->f : v->is_signed ? (double)v->i : (double)v->u;
  return QVX_OK;
}

int qvx_gguf_meta_bool(const qvx_gguf* f, const char* key, uint64_t index, int* out) {
  const Value* v = meta_elem(f, key, index);
  if (!v) return QVX_E_RANGE;
  if (v->tag != M_BOOL) return QVX_E_TYPE;
  if (out) *out = v->u ? 1 : 0;
  return QVX_OK;
}

int qvx_gguf_meta_string(const qvx_gguf* f, const char* key, uint64_t index, const char** out, size_t* len) {
  const Value* v = meta_elem(f, key, index);
  if (!v) return QVX_E_RANGE;
  if (v->tag != M_STR) return QVX_E_TYPE;
  if (out) *out = v->s.data();
  if (len) *len = v->s.size();
  return QVX_OK;
}

}  // extern "C"
#pragma GCC visibility pop
