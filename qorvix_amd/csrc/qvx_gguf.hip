// qvx_gguf.hip -- GGUF container reader and weight upload of libqvx.so (host code only; declared in
// include/qvx.h, qvx_gguf_*).  Written from the public GGUF format description (ggml's docs/gguf.md):
//
//   file   := magic "GGUF" | u32 version | count tensors | count kvs | kv * | tensor_info * |
//             padding to ALIGN | tensor data
//   kv     := string key | u32 value_type | value
//   value  := scalar | string | u32 elem_type, count n, value * n        (value_type 9: array)
//   tensor_info := string name | u32 n_dims | dim * n_dims | u32 ggml_type | u64 offset
//   string := count len | len bytes (no terminator)
//   count / dim: u32 in version 1, u64 from version 2 on; all numbers little-endian.
//
// The index is built in one pass without copying the data: every metadata entry records its value
// type and where its payload starts in the buffer, and values are decoded when asked for (string
// arrays also record where each element starts).  So the buffer -- the read-only mapping of
// qvx_gguf_open, or the caller's buffer of qvx_gguf_parse -- must stay valid while the handle lives,
// which the mapping does by construction.  Tensor data is only located; qvx_gguf_upload copies a
// tensor's raw blocks to the device, where the GEMV / GEMM entry points read them as they are.
//
// Where each check comes from:
//  * magic, version 1..3, 32-bit counts in version 1 -- the format's header definition;
//  * every read inside the buffer; metadata value types 0..12; at most 4 dimensions per tensor
//    (the format's GGML_MAX_DIMS); tensor offsets a multiple of the alignment; the alignment
//    (general.alignment, default 32) a u32 power of two; unique keys and tensor names -- the
//    format description and the ggml reader that defines it;
//  * a row length (dims[0]) that is a whole number of blocks for a block-quantised type -- the
//    GGUF block layout, whose rows are stored as whole blocks;
//  * every tensor's bytes inside the file -- a GGUF file carries the data its tensor table
//    describes;
//  * element counts and byte extents computed without overflow -- this reader's own arithmetic.
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

#include "../../include/qvx.h"
#include "qvx_common.hpp"

namespace {

constexpr uint8_t kMagic[4] = {'G', 'G', 'U', 'F'};
constexpr uint32_t kAlignDefault = 32;
constexpr uint32_t kRankMax = 4;          // GGML_MAX_DIMS
constexpr size_t kKeyMax = 65535;         // metadata keys are at most 2^16 - 1 bytes
constexpr int kNestMax = 8;               // deepest array-of-array this reader walks

// Value types of the format.
enum : uint32_t {
  V_U8 = 0, V_I8, V_U16, V_I16, V_U32, V_I32, V_F32, V_BOOL, V_STRING, V_ARRAY, V_U64, V_I64, V_F64,
  V_COUNT
};

// Bytes of one fixed-size value, 0 for strings and arrays.
constexpr uint32_t fixed_size(uint32_t t) {
  return t == V_U8 || t == V_I8 || t == V_BOOL ? 1
         : t == V_U16 || t == V_I16          ? 2
         : t == V_U32 || t == V_I32 || t == V_F32 ? 4
         : t == V_U64 || t == V_I64 || t == V_F64 ? 8
                                                   : 0;
}

// A bounded little-endian reader over [data, data + size).  Every failed read leaves `bad` set and a
// message naming the field; later reads are no-ops, so a parse checks once per record.
struct Cursor {
  const uint8_t* data;
  size_t size;
  size_t at = 0;
  bool bad = false;
  std::string why;

  bool fail(std::string msg) {
    if (!bad) {
      bad = true;
      why = std::move(msg);
    }
    return false;
  }
  bool skip(uint64_t n, const char* what) {
    if (bad) return false;
    if (n > size - at) return fail(std::string("file ends inside ") + what + " (byte " + std::to_string(at) + ")");
    at += (size_t)n;
    return true;
  }
  template <typename T>
  T num(const char* what) {
    T v{};
    const size_t here = at;
    if (skip(sizeof(T), what)) std::memcpy(&v, data + here, sizeof(T));
    return v;
  }
  // u32 in version 1, u64 after
  uint64_t count(bool wide, const char* what) { return wide ? num<uint64_t>(what) : num<uint32_t>(what); }
  // a string: returns its view (empty on failure)
  std::string_view text(bool wide, const char* what) {
    const uint64_t n = count(wide, what);
    const size_t here = at;
    if (!skip(n, what)) return {};
    return std::string_view(reinterpret_cast<const char*>(data + here), (size_t)n);
  }
};

// Metadata entry: where its value sits in the buffer.
struct Entry {
  std::string key;
  uint32_t type = 0;   // value type
  uint32_t elem = 0;   // element type of an array (== type for a scalar)
  uint64_t count = 1;  // elements of an array (1 for a scalar)
  size_t pos = 0;      // first byte of the scalar / of the first array element
  std::vector<size_t> items;  // string arrays: start of each element
};

struct TensorRec {
  std::string name;
  uint32_t rank = 0;
  uint64_t dims[kRankMax] = {0, 0, 0, 0};
  uint32_t type = 0;
  uint64_t offset = 0, elements = 0, bytes = 0;
  bool sized = false;  // the type's block size is known (bytes is meaningful)
};

// Walks (does not store) one value of type t, nested arrays included, and records an array's
// element positions when they are strings.
bool walk_value(Cursor& c, bool wide, uint32_t t, int depth, Entry* top) {
  if (t >= V_COUNT) return c.fail("metadata value type " + std::to_string(t) + " is not defined by the format");
  if (uint32_t sz = fixed_size(t)) return c.skip(sz, "a metadata value");
  if (t == V_STRING) {
    c.text(wide, "a metadata string");
    return !c.bad;
  }
  // array
  if (depth >= kNestMax) return c.fail("metadata arrays nested deeper than " + std::to_string(kNestMax));
  const uint32_t et = c.num<uint32_t>("an array element type");
  const uint64_t n = c.count(wide, "an array length");
  if (c.bad) return false;
  if (et >= V_COUNT) return c.fail("array element type " + std::to_string(et) + " is not defined by the format");
  if (top) {
    top->elem = et;
    top->count = n;
    top->pos = c.at;
  }
  if (uint32_t sz = fixed_size(et)) {
    if (n > (c.size - c.at) / sz) return c.fail("array of " + std::to_string(n) + " elements runs past the end of the file");
    return c.skip(n * sz, "an array");
  }
  // strings and arrays take at least one length field each
  const uint64_t least = wide ? 8 : 4;
  if (n > (c.size - c.at) / least) return c.fail("array of " + std::to_string(n) + " elements runs past the end of the file");
  if (top && et == V_STRING) top->items.reserve((size_t)n);
  for (uint64_t k = 0; k < n && !c.bad; ++k) {
    if (top && et == V_STRING) top->items.push_back(c.at);
    walk_value(c, wide, et, depth + 1, nullptr);
  }
  return !c.bad;
}

// a * b, false on overflow
bool mul_ok(uint64_t a, uint64_t b, uint64_t* out) {
  if (a != 0 && b > UINT64_MAX / a) return false;
  *out = a * b;
  return true;
}

}  // namespace

// The index of one GGUF file (include/qvx.h, qvx_gguf_*).
struct qvx_gguf {
  const uint8_t* bytes = nullptr;  // the mapping or the caller's buffer
  size_t size = 0;
  void* mapping = nullptr;         // owned by the handle when opened from a file
  size_t mapping_size = 0;
  uint32_t version = 0, align = kAlignDefault;
  uint64_t data_start = 0;
  std::vector<Entry> entries;
  std::unordered_map<std::string_view, size_t> by_key;   // views into entries[i].key
  std::vector<TensorRec> tensors;
  std::unordered_map<std::string_view, size_t> by_name;  // views into tensors[i].name

  ~qvx_gguf() {
    if (mapping) munmap(mapping, mapping_size);
  }

  const Entry* entry(const char* key) const {
    if (!key) return nullptr;
    auto it = by_key.find(std::string_view(key));
    return it == by_key.end() ? nullptr : &entries[it->second];
  }

  // Builds the index; returns "" or what is wrong.
  std::string index() {
    Cursor c{bytes, size};
    uint8_t magic[4] = {0, 0, 0, 0};
    if (size >= 4) std::memcpy(magic, bytes, 4);
    if (std::memcmp(magic, kMagic, 4) != 0) {
      if (magic[0] == 'F' && magic[1] == 'U' && magic[2] == 'G' && magic[3] == 'G')
        return "byte-swapped GGUF magic: big-endian files are not supported";
      return "no GGUF magic at the start of the data";
    }
    c.at = 4;
    version = c.num<uint32_t>("the version");
    if (c.bad) return c.why;
    if (version < 1 || version > 3) return "GGUF version " + std::to_string(version) + " is not one of 1, 2, 3";
    const bool wide = version >= 2;
    const uint64_t n_tensors = c.count(wide, "the tensor count");
    const uint64_t n_kv = c.count(wide, "the metadata count");
    if (c.bad) return c.why;
    // each key/value takes at least a length and a type; each tensor record at least name length,
    // rank, type and offset -- bounds before any reservation
    if (n_kv > size / (wide ? 12 : 8)) return "metadata count " + std::to_string(n_kv) + " cannot fit in the file";
    if (n_tensors > size / (wide ? 24 : 20)) return "tensor count " + std::to_string(n_tensors) + " cannot fit in the file";

    entries.reserve((size_t)n_kv);
    for (uint64_t k = 0; k < n_kv; ++k) {
      Entry e;
      const std::string_view key = c.text(wide, "a metadata key");
      const uint32_t t = c.num<uint32_t>("a metadata value type");
      if (c.bad) return c.why;
      if (key.size() > kKeyMax) return "metadata key of " + std::to_string(key.size()) + " bytes (longer than 65535)";
      e.key.assign(key);
      e.type = e.elem = t;
      e.pos = c.at;
      if (!walk_value(c, wide, t, 0, &e)) return c.why + " (key '" + e.key + "')";
      entries.push_back(std::move(e));
    }
    for (size_t i = 0; i < entries.size(); ++i)
      if (!by_key.emplace(std::string_view(entries[i].key), i).second)
        return "metadata key '" + entries[i].key + "' appears twice";

    if (const Entry* a = entry("general.alignment")) {
      if (a->type != V_U32) return "general.alignment must be a u32";
      uint32_t v = 0;
      std::memcpy(&v, bytes + a->pos, 4);
      if (v == 0 || (v & (v - 1)) != 0) return "general.alignment " + std::to_string(v) + " is not a power of two";
      align = v;
    }

    tensors.reserve((size_t)n_tensors);
    for (uint64_t k = 0; k < n_tensors; ++k) {
      TensorRec t;
      const std::string_view name = c.text(wide, "a tensor name");
      t.rank = c.num<uint32_t>("a tensor rank");
      if (c.bad) return c.why;
      t.name.assign(name);
      if (t.rank > kRankMax)
        return "tensor '" + t.name + "': " + std::to_string(t.rank) + " dimensions (the format allows up to 4)";
      for (uint32_t d = 0; d < t.rank; ++d) t.dims[d] = c.count(wide, "tensor dimensions");
      t.type = c.num<uint32_t>("a tensor type");
      t.offset = c.num<uint64_t>("a tensor offset");
      if (c.bad) return c.why;
      uint64_t n = 1;
      for (uint32_t d = 0; d < t.rank; ++d)
        if (!mul_ok(n, t.dims[d], &n)) return "tensor '" + t.name + "': element count does not fit in 64 bits";
      t.elements = n;
      if (const qvx::TypeInfo* ti = qvx::type_info(t.type)) {
        const uint64_t row = t.rank ? t.dims[0] : 1;
        if (row % ti->block != 0)
          return "tensor '" + t.name + "': rows of " + std::to_string(row) + " elements are not whole blocks of " +
                 std::to_string(ti->block);
        if (!mul_ok(n / ti->block, ti->bytes, &t.bytes)) return "tensor '" + t.name + "': byte size does not fit in 64 bits";
        t.sized = true;
      }
      if (t.offset % align != 0)
        return "tensor '" + t.name + "': offset " + std::to_string(t.offset) + " is not a multiple of the alignment " +
               std::to_string(align);
      tensors.push_back(std::move(t));
    }
    for (size_t i = 0; i < tensors.size(); ++i)
      if (!by_name.emplace(std::string_view(tensors[i].name), i).second)
        return "tensor name '" + tensors[i].name + "' appears twice";

    // data section: the next multiple of the alignment after the tables
    const uint64_t end_of_tables = c.at;
    data_start = end_of_tables + (align - end_of_tables % align) % align;
    const uint64_t room = size >= data_start ? size - data_start : 0;
    for (const TensorRec& t : tensors) {
      if (!t.sized || t.bytes == 0) continue;
      if (size < data_start || t.offset > room || t.bytes > room - t.offset)
        return "tensor '" + t.name + "': bytes [" + std::to_string(t.offset) + ", +" + std::to_string(t.bytes) +
               ") lie outside the file's data section of " + std::to_string(room) + " bytes";
    }
    return {};
  }

  const TensorRec* tensor(int64_t i) const {
    return i >= 0 && (uint64_t)i < tensors.size() ? &tensors[(size_t)i] : nullptr;
  }
};

namespace {

thread_local std::string g_last_error;

int finish(qvx_gguf* f, qvx_gguf** out) {
  std::string why;
  try {
    why = f->index();
  } catch (const std::bad_alloc&) {
    why = "not enough host memory for the GGUF index";
  }
  if (!why.empty()) {
    delete f;
    g_last_error = std::move(why);
    return QVX_E_FORMAT;
  }
  g_last_error.clear();
  *out = f;
  return QVX_OK;
}

// Element `index` of `key` as (type, position), or false when absent / out of range / nested.
bool locate(const qvx_gguf* f, const char* key, uint64_t index, uint32_t* type, size_t* pos) {
  const Entry* e = f ? f->entry(key) : nullptr;
  if (!e) return false;
  if (e->type != V_ARRAY) {
    if (index != 0) return false;
    *type = e->type;
    *pos = e->pos;
    return true;
  }
  if (index >= e->count) return false;
  *type = e->elem;
  if (uint32_t sz = fixed_size(e->elem)) {
    *pos = e->pos + (size_t)index * sz;
    return true;
  }
  if (e->elem == V_STRING) {
    *pos = e->items[(size_t)index];
    return true;
  }
  *pos = 0;  // an array of arrays: present, but no scalar to give
  return true;
}

// The integer of a fixed-size integer / bool value at pos, as u64 (bit pattern) and i64.
bool read_int(const qvx_gguf* f, uint32_t t, size_t pos, uint64_t* u, int64_t* i) {
  const uint8_t* p = f->bytes + pos;
  switch (t) {
    case V_U8: case V_BOOL: { uint8_t v; std::memcpy(&v, p, 1); *u = v; *i = v; return true; }
    case V_I8: { int8_t v; std::memcpy(&v, p, 1); *i = v; *u = (uint64_t)*i; return true; }
    case V_U16: { uint16_t v; std::memcpy(&v, p, 2); *u = v; *i = v; return true; }
    case V_I16: { int16_t v; std::memcpy(&v, p, 2); *i = v; *u = (uint64_t)*i; return true; }
    case V_U32: { uint32_t v; std::memcpy(&v, p, 4); *u = v; *i = v; return true; }
    case V_I32: { int32_t v; std::memcpy(&v, p, 4); *i = v; *u = (uint64_t)*i; return true; }
    case V_U64: { uint64_t v; std::memcpy(&v, p, 8); *u = v; *i = (int64_t)v; return true; }
    case V_I64: { int64_t v; std::memcpy(&v, p, 8); *i = v; *u = (uint64_t)v; return true; }
    default: return false;
  }
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
  f->bytes = static_cast<const uint8_t*>(data);
  f->size = size;
  return finish(f, out);
}

int qvx_gguf_open(const char* path, qvx_gguf** out) {
  if (!out || !path) return QVX_E_NULL;
  *out = nullptr;
  const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) {
    g_last_error = std::string("cannot open '") + path + "': " + std::strerror(errno);
    return QVX_E_IO;
  }
  struct stat st {};
  if (fstat(fd, &st) != 0 || st.st_size <= 0) {
    g_last_error = std::string("cannot map '") + path + "': empty or not a regular file";
    ::close(fd);
    return QVX_E_IO;
  }
  void* m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
  const int map_err = errno;
  ::close(fd);
  if (m == MAP_FAILED) {
    g_last_error = std::string("cannot map '") + path + "': " + std::strerror(map_err);
    return QVX_E_IO;
  }
  auto* f = new (std::nothrow) qvx_gguf;
  if (!f) {
    munmap(m, (size_t)st.st_size);
    return QVX_E_HIP;
  }
  f->mapping = m;
  f->mapping_size = (size_t)st.st_size;
  f->bytes = static_cast<const uint8_t*>(m);
  f->size = (size_t)st.st_size;
  return finish(f, out);
}

void qvx_gguf_close(qvx_gguf* f) { delete f; }

const char* qvx_gguf_last_error(void) { return g_last_error.c_str(); }

uint32_t qvx_gguf_version(const qvx_gguf* f) { return f ? f->version : 0; }
uint32_t qvx_gguf_alignment(const qvx_gguf* f) { return f ? f->align : 0; }
uint64_t qvx_gguf_data_offset(const qvx_gguf* f) { return f ? f->data_start : 0; }
int64_t qvx_gguf_tensor_count(const qvx_gguf* f) { return f ? (int64_t)f->tensors.size() : 0; }
int64_t qvx_gguf_meta_count(const qvx_gguf* f) { return f ? (int64_t)f->entries.size() : 0; }

int64_t qvx_gguf_find_tensor(const qvx_gguf* f, const char* name) {
  if (!f || !name) return -1;
  auto it = f->by_name.find(std::string_view(name));
  return it == f->by_name.end() ? -1 : (int64_t)it->second;
}

int qvx_gguf_tensor_info(const qvx_gguf* f, int64_t i, const char** name, uint32_t* type, uint32_t* n_dims,
                         uint64_t* dims, uint64_t* offset, uint64_t* n_elements, uint64_t* n_bytes) {
  const TensorRec* t = f ? f->tensor(i) : nullptr;
  if (!t) return QVX_E_RANGE;
  if (name) *name = t->name.c_str();
  if (type) *type = t->type;
  if (n_dims) *n_dims = t->rank;
  if (dims)  // 8 slots, zeros past the rank
    for (uint32_t d = 0; d < 8; ++d) dims[d] = d < t->rank ? t->dims[d] : 0;
  if (offset) *offset = t->offset;
  if (n_elements) *n_elements = t->elements;
  if (n_bytes) *n_bytes = t->sized ? t->bytes : 0;
  return QVX_OK;
}

const void* qvx_gguf_tensor_data(const qvx_gguf* f, int64_t i) {
  const TensorRec* t = f ? f->tensor(i) : nullptr;
  if (!t || !t->sized) return nullptr;
  // the index checked the extent against the buffer; recheck without overflow anyway
  if (f->size < f->data_start || t->offset > f->size - f->data_start ||
      t->bytes > f->size - f->data_start - t->offset)
    return nullptr;
  return f->bytes + f->data_start + t->offset;
}

int qvx_gguf_upload(const qvx_gguf* f, int64_t i, void* d_dst, size_t dst_bytes, void* stream) {
  const TensorRec* t = f ? f->tensor(i) : nullptr;
  if (!t) return QVX_E_RANGE;
  if (!t->sized) return QVX_E_TYPE;  // a type id whose block size this engine does not know
  const void* src = qvx_gguf_tensor_data(f, i);
  if (!src) return QVX_E_RANGE;
  if (!d_dst) return QVX_E_NULL;
  if (dst_bytes < t->bytes) return QVX_E_RANGE;
  if (t->bytes == 0) return QVX_OK;
  if (hipMemcpyAsync(d_dst, src, (size_t)t->bytes, hipMemcpyHostToDevice, static_cast<hipStream_t>(stream)) !=
      hipSuccess) {
    (void)hipGetLastError();
    return QVX_E_HIP;
  }
  return QVX_OK;
}

const char* qvx_gguf_meta_key(const qvx_gguf* f, int64_t i) {
  if (!f || i < 0 || (uint64_t)i >= f->entries.size()) return nullptr;
  return f->entries[(size_t)i].key.c_str();
}

int qvx_gguf_meta_type(const qvx_gguf* f, const char* key, uint32_t* type, uint32_t* elem_type, uint64_t* count) {
  const Entry* e = f ? f->entry(key) : nullptr;
  if (!e) return QVX_E_RANGE;
  if (type) *type = e->type;
  if (elem_type) *elem_type = e->elem;
  if (count) *count = e->count;
  return QVX_OK;
}

// Typed element access.  Integers and bools widen to u64 / i64; every number but a bool converts
// to f64; strings come back as (pointer, length) into the buffer.  A value of another category
// (and an element of an array of arrays) -> QVX_E_TYPE.
int qvx_gguf_meta_u64(const qvx_gguf* f, const char* key, uint64_t index, uint64_t* out) {
  uint32_t t;
  size_t pos;
  if (!locate(f, key, index, &t, &pos)) return QVX_E_RANGE;
  uint64_t u;
  int64_t i;
  if (!read_int(f, t, pos, &u, &i)) return QVX_E_TYPE;
  if (out) *out = u;
  return QVX_OK;
}

int qvx_gguf_meta_i64(const qvx_gguf* f, const char* key, uint64_t index, int64_t* out) {
  uint32_t t;
  size_t pos;
  if (!locate(f, key, index, &t, &pos)) return QVX_E_RANGE;
  uint64_t u;
  int64_t i;
  if (!read_int(f, t, pos, &u, &i)) return QVX_E_TYPE;
  if (out) *out = i;
  return QVX_OK;
}

int qvx_gguf_meta_f64(const qvx_gguf* f, const char* key, uint64_t index, double* out) {
  uint32_t t;
  size_t pos;
  if (!locate(f, key, index, &t, &pos)) return QVX_E_RANGE;
  double v;
  if (t == V_F32) {
    float x;
    std::memcpy(&x, f->bytes + pos, 4);
    v = x;
  } else if (t == V_F64) {
    std::memcpy(&v, f->bytes + pos, 8);
  } else {
    uint64_t u;
    int64_t i;
    if (t == V_BOOL || !read_int(f, t, pos, &u, &i)) return QVX_E_TYPE;
    v = (t == V_I8 || t == V_I16 || t == V_I32 || t == V_I64) ? (double)i : (double)u;
  }
  if (out) *out = v;
  return QVX_OK;
}

int qvx_gguf_meta_bool(const qvx_gguf* f, const char* key, uint64_t index, int* out) {
  uint32_t t;
  size_t pos;
  if (!locate(f, key, index, &t, &pos)) return QVX_E_RANGE;
  if (t != V_BOOL) return QVX_E_TYPE;
  if (out) *out = f->bytes[pos] != 0 ? 1 : 0;
  return QVX_OK;
}

int qvx_gguf_meta_string(const qvx_gguf* f, const char* key, uint64_t index, const char** out, size_t* len) {
  uint32_t t;
  size_t pos;
  if (!locate(f, key, index, &t, &pos)) return QVX_E_RANGE;
  if (t != V_STRING) return QVX_E_TYPE;
  Cursor c{f->bytes, f->size, pos};
  const std::string_view s = c.text(f->version >= 2, "a metadata string");
  if (c.bad) return QVX_E_FORMAT;  // cannot happen for an indexed string
  if (out) *out = s.data();
  if (len) *len = s.size();
  return QVX_OK;
}

}  // extern "C"
#pragma GCC visibility pop
