// gguf.cpp -- the GGUF v2/v3 reader of the load path (host C++; exported by
// the C ABI as btf_hip_gguf_*).
//
// Behaviour of the reference's reader bd::Gguf
// (ref/bonsai-decoder/include/bd/gguf.hpp:49-85, src/gguf.cpp:73-147): the
// file is memory-mapped read-only and parsed in one pass; every metadata
// value (scalars of each kind, strings, arrays) and every tensor info is
// kept; tensor data stay in the mapping (no copy). The layout:
//   "GGUF", u32 version (2 or 3), u64 n_tensors, u64 n_kv,
//   n_kv x (string key, u32 type, value), n_tensors x (string name,
//   u32 n_dims, n_dims x u64 ne, u32 ggml type, u64 offset),
//   padding to `general.alignment` (default 32), the data section.
// A string is a u64 length and its bytes. The same checks as the reference
// reject a file (bad magic or version, implausible counts, over-long strings
// or arrays, an alignment that is not a power of two, a tensor with 0 or more
// than 4 dimensions, an unknown ggml type, a row that is not whole blocks, a
// tensor offset off the alignment, a tensor past the end of the file unless
// only the header is read, truncation anywhere). Numeric values keep both an
// integer and a double form: integers convert exactly to double, floats
// truncate towards zero to integer, booleans are 0 or 1.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/btf/hip_abi.h"
#include "common.h"

namespace btfhip {

// ggml type id -> (elements per block, bytes per block); 0 = unknown. The
// sizes are the ggml formats' (the reference's bd::type_info,
// ref/bonsai-decoder/src/types.cpp:13-34).
struct GgmlSize {
  int block, bytes;
};
static GgmlSize ggml_size(uint32_t t) {
  switch (t) {
    case 0: return {1, 4};       // F32
    case 1: return {1, 2};       // F16
    case 2: return {32, 18};     // Q4_0
    case 3: return {32, 20};     // Q4_1
    case 6: return {32, 22};     // Q5_0
    case 7: return {32, 24};     // Q5_1
    case 8: return {32, 34};     // Q8_0
    case 12: return {256, 144};  // Q4_K
    case 13: return {256, 176};  // Q5_K
    case 14: return {256, 210};  // Q6_K
    case 26: return {1, 4};      // I32
    case 30: return {1, 2};      // BF16
    case 34: return {256, 54};   // TQ1_0
    case 35: return {256, 66};   // TQ2_0
    case 42: return {64, 18};    // Q2_0
    case 142: return {128, 34};  // PQ2_0
    case 143: return {128, 28};  // PTQ1_0
    default: return {0, 0};
  }
}

enum : uint32_t {
  kU8 = 0, kI8, kU16, kI16, kU32, kI32, kF32, kBool, kString, kArray, kU64, kI64, kF64,
};

struct GgufKv {
  std::string key;
  uint32_t type = 0, arr_type = 0;
  // one element per scalar, len elements per array: integer and double forms
  // for numbers, bytes for strings
  std::vector<int64_t> iv;
  std::vector<double> fv;
  std::vector<std::string> sv;
  uint64_t len() const { return type == kArray ? (arr_type == kString ? sv.size() : iv.size()) : 1; }
};

struct GgufTensorInfo {
  std::string name;
  int n_dims = 0;
  int64_t ne[4] = {1, 1, 1, 1};
  uint32_t type = 0;
  uint64_t offset = 0, bytes = 0;
  const uint8_t* data = nullptr;
};

struct Gguf {
  int fd = -1;
  void* map = nullptr;
  size_t size = 0;
  uint32_t version = 0;
  uint64_t alignment = 32;
  uint64_t data_offset = 0;
  bool header_only = false;
  std::vector<GgufKv> kv;
  std::unordered_map<std::string, int64_t> kv_index;  // last entry of each key
  std::vector<GgufTensorInfo> tensors;
  std::unordered_map<std::string, int64_t> tensor_index;
  ~Gguf() {
    if (map && map != MAP_FAILED) munmap(map, size);
    if (fd >= 0) close(fd);
  }
};

namespace {

// Bounds-checked little-endian cursor over the mapping.
struct Cursor {
  const uint8_t* base;
  size_t size, pos = 0;
  void need(size_t n) const {
    if (n > size || pos > size - n) throw std::runtime_error("gguf: truncated at byte " + std::to_string(pos));
  }
  template <class T>
  T take() {
    need(sizeof(T));
    T v;
    std::memcpy(&v, base + pos, sizeof(T));
    pos += sizeof(T);
    return v;
  }
  std::string string() {
    const uint64_t n = take<uint64_t>();
    if (n > (1ull << 30)) throw std::runtime_error("gguf: string too long at byte " + std::to_string(pos));
    need((size_t)n);
    std::string s(reinterpret_cast<const char*>(base + pos), (size_t)n);
    pos += (size_t)n;
    return s;
  }
};

// One value of scalar type t appended to kv's element lists.
void read_value(Cursor& c, uint32_t t, GgufKv& kv) {
  int64_t i = 0;
  double f = 0.0;
  switch (t) {
    case kU8: i = c.take<uint8_t>(); break;
    case kI8: i = c.take<int8_t>(); break;
    case kU16: i = c.take<uint16_t>(); break;
    case kI16: i = c.take<int16_t>(); break;
    case kU32: i = c.take<uint32_t>(); break;
    case kI32: i = c.take<int32_t>(); break;
    case kU64: i = (int64_t)c.take<uint64_t>(); break;
    case kI64: i = c.take<int64_t>(); break;
    case kBool: i = c.take<uint8_t>() != 0; break;
    case kF32: f = c.take<float>(); break;
    case kF64: f = c.take<double>(); break;
    case kString: kv.sv.push_back(c.string()); return;
    default: throw std::runtime_error("gguf: bad value type " + std::to_string(t));
  }
  if (t == kF32 || t == kF64)
    i = (int64_t)f;
  else
    f = (double)i;
  kv.iv.push_back(i);
  kv.fv.push_back(f);
}

void parse(Gguf& g) {
  Cursor c{static_cast<const uint8_t*>(g.map), g.size};
  c.need(4);
  if (std::memcmp(c.base, "GGUF", 4) != 0) throw std::runtime_error("gguf: bad magic");
  c.pos = 4;
  g.version = c.take<uint32_t>();
  if (g.version != 2 && g.version != 3) throw std::runtime_error("gguf: unsupported version " + std::to_string(g.version));
  const uint64_t n_tensors = c.take<uint64_t>(), n_kv = c.take<uint64_t>();
  if (n_tensors > (1u << 24) || n_kv > (1u << 24)) throw std::runtime_error("gguf: implausible counts");
  g.kv.reserve((size_t)n_kv);
  for (uint64_t k = 0; k < n_kv; ++k) {
    GgufKv v;
    v.key = c.string();
    v.type = c.take<uint32_t>();
    if (v.type == kArray) {
      v.arr_type = c.take<uint32_t>();
      const uint64_t n = c.take<uint64_t>();
      if (n > (1ull << 32)) throw std::runtime_error("gguf: array too large: " + v.key);
      for (uint64_t j = 0; j < n; ++j) read_value(c, v.arr_type, v);
    } else {
      read_value(c, v.type, v);
    }
    if (v.key == "general.alignment") {
      const int64_t a = v.type == kString || v.type == kArray ? 0 : v.iv[0];
      if (a <= 0 || (a & (a - 1))) throw std::runtime_error("gguf: bad alignment");
      g.alignment = (uint64_t)a;
    }
    g.kv_index[v.key] = (int64_t)g.kv.size();
    g.kv.push_back(std::move(v));
  }
  // A key present more than once keeps every position but resolves to the
  // value of its last entry, at every position (the reference keeps one
  // value per key).
  for (size_t k = 0; k < g.kv.size(); ++k) {
    const size_t last = (size_t)g.kv_index[g.kv[k].key];
    if (last != k) {
      g.kv[k].type = g.kv[last].type;
      g.kv[k].arr_type = g.kv[last].arr_type;
      g.kv[k].iv = g.kv[last].iv;
      g.kv[k].fv = g.kv[last].fv;
      g.kv[k].sv = g.kv[last].sv;
    }
  }
  g.tensors.resize((size_t)n_tensors);
  for (uint64_t k = 0; k < n_tensors; ++k) {
    GgufTensorInfo& t = g.tensors[(size_t)k];
    t.name = c.string();
    const uint32_t nd = c.take<uint32_t>();
    if (nd < 1 || nd > 4) throw std::runtime_error("gguf: bad n_dims for " + t.name);
    t.n_dims = (int)nd;
    int64_t n = 1;
    for (uint32_t d = 0; d < nd; ++d) {
      t.ne[d] = (int64_t)c.take<uint64_t>();
      n *= t.ne[d];
    }
    t.type = c.take<uint32_t>();
    t.offset = c.take<uint64_t>();
    if (t.offset % g.alignment) throw std::runtime_error("gguf: misaligned " + t.name);
    const GgmlSize z = ggml_size(t.type);
    if (!z.block) throw std::runtime_error("gguf: unknown ggml type " + std::to_string(t.type) + " for " + t.name);
    if (t.ne[0] % z.block) throw std::runtime_error("gguf: row not whole blocks: " + t.name);
    t.bytes = (uint64_t)(n / z.block) * (uint64_t)z.bytes;
    g.tensor_index[t.name] = (int64_t)k;
  }
  g.data_offset = (c.pos + g.alignment - 1) / g.alignment * g.alignment;
  for (GgufTensorInfo& t : g.tensors) {
    const uint64_t end = g.data_offset + t.offset + t.bytes;
    if (end <= g.size)
      t.data = static_cast<const uint8_t*>(g.map) + g.data_offset + t.offset;
    else if (!g.header_only)
      throw std::runtime_error("gguf: tensor past end of file: " + t.name);
  }
}

int gguf_err(const std::exception& e) { return fail(BTF_ERR_ARGS, e.what()); }

}  // namespace

}  // namespace btfhip

using btfhip::Gguf;
using btfhip::fail;

extern "C" {

int btf_hip_gguf_open(const char* path, int header_only, btf_gguf_t* out) {
  if (!path || !out) return fail(BTF_ERR_ARGS, "gguf: null argument");
  *out = nullptr;
  std::unique_ptr<Gguf> g(new Gguf());
  g->header_only = header_only != 0;
  g->fd = open(path, O_RDONLY | O_CLOEXEC);
  if (g->fd < 0) return fail(BTF_ERR_ARGS, std::string("gguf: cannot open ") + path);
  struct stat st;
  if (fstat(g->fd, &st) != 0) return fail(BTF_ERR_ARGS, std::string("gguf: cannot stat ") + path);
  g->size = (size_t)st.st_size;
  if (g->size == 0) return fail(BTF_ERR_ARGS, "gguf: truncated at byte 0");
  g->map = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
  if (g->map == MAP_FAILED) {
    g->map = nullptr;
    return fail(BTF_ERR_ARGS, std::string("gguf: cannot map ") + path);
  }
  try {
    btfhip::parse(*g);
  } catch (const std::exception& e) {
    return btfhip::gguf_err(e);
  }
  *out = g.release();
  return BTF_OK;
}

int btf_hip_gguf_close(btf_gguf_t h) {
  delete static_cast<Gguf*>(h);
  return BTF_OK;
}

int btf_hip_gguf_info(btf_gguf_t h, btf_gguf_header* out) {
  const Gguf* g = static_cast<const Gguf*>(h);
  if (!g || !out) return fail(BTF_ERR_ARGS, "gguf: null argument");
  out->version = g->version;
  out->alignment = g->alignment;
  out->data_offset = g->data_offset;
  out->file_bytes = g->size;
  out->n_tensors = (int64_t)g->tensors.size();
  out->n_kv = (int64_t)g->kv.size();
  return BTF_OK;
}

int btf_hip_gguf_tensor(btf_gguf_t h, int64_t index, btf_gguf_tensor* out) {
  const Gguf* g = static_cast<const Gguf*>(h);
  if (!g || !out) return fail(BTF_ERR_ARGS, "gguf: null argument");
  if (index < 0 || index >= (int64_t)g->tensors.size()) return fail(BTF_ERR_ARGS, "gguf: tensor index out of range");
  const btfhip::GgufTensorInfo& t = g->tensors[(size_t)index];
  out->name = t.name.c_str();
  out->n_dims = t.n_dims;
  for (int d = 0; d < 4; ++d) out->ne[d] = t.ne[d];
  out->type = t.type;
  out->offset = t.offset;
  out->bytes = t.bytes;
  out->data = t.data;
  return BTF_OK;
}

int64_t btf_hip_gguf_find_tensor(btf_gguf_t h, const char* name) {
  const Gguf* g = static_cast<const Gguf*>(h);
  if (!g || !name) return -1;
  auto it = g->tensor_index.find(name);
  return it == g->tensor_index.end() ? -1 : it->second;
}

int btf_hip_gguf_kv(btf_gguf_t h, int64_t index, btf_gguf_kv* out) {
  const Gguf* g = static_cast<const Gguf*>(h);
  if (!g || !out) return fail(BTF_ERR_ARGS, "gguf: null argument");
  if (index < 0 || index >= (int64_t)g->kv.size()) return fail(BTF_ERR_ARGS, "gguf: key index out of range");
  const btfhip::GgufKv& v = g->kv[(size_t)index];
  out->key = v.key.c_str();
  out->key_len = v.key.size();
  out->type = v.type;
  out->arr_type = v.arr_type;
  out->len = v.len();
  return BTF_OK;
}

int64_t btf_hip_gguf_find_kv(btf_gguf_t h, const char* key) {
  const Gguf* g = static_cast<const Gguf*>(h);
  if (!g || !key) return -1;
  auto it = g->kv_index.find(key);
  return it == g->kv_index.end() ? -1 : it->second;
}

// Element `elem` of a numeric value (0 for a scalar).
int btf_hip_gguf_kv_num(btf_gguf_t h, int64_t index, uint64_t elem, int64_t* i, double* f) {
  const Gguf* g = static_cast<const Gguf*>(h);
  if (!g) return fail(BTF_ERR_ARGS, "gguf: null argument");
  if (index < 0 || index >= (int64_t)g->kv.size()) return fail(BTF_ERR_ARGS, "gguf: key index out of range");
  const btfhip::GgufKv& v = g->kv[(size_t)index];
  if (elem >= v.iv.size()) return fail(BTF_ERR_ARGS, "gguf: " + v.key + " has no numeric element " + std::to_string(elem));
  if (i) *i = v.iv[(size_t)elem];
  if (f) *f = v.fv[(size_t)elem];
  return BTF_OK;
}

int btf_hip_gguf_kv_str(btf_gguf_t h, int64_t index, uint64_t elem, const char** s, uint64_t* len) {
  const Gguf* g = static_cast<const Gguf*>(h);
  if (!g || !s || !len) return fail(BTF_ERR_ARGS, "gguf: null argument");
  if (index < 0 || index >= (int64_t)g->kv.size()) return fail(BTF_ERR_ARGS, "gguf: key index out of range");
  const btfhip::GgufKv& v = g->kv[(size_t)index];
  if (elem >= v.sv.size()) return fail(BTF_ERR_ARGS, "gguf: " + v.key + " has no string element " + std::to_string(elem));
  *s = v.sv[(size_t)elem].data();
  *len = v.sv[(size_t)elem].size();
  return BTF_OK;
}

int64_t btf_hip_ggml_row_bytes(uint32_t type, int64_t n) {
  const btfhip::GgmlSize z = btfhip::ggml_size(type);
  if (!z.block || n < 0 || n % z.block) return -1;
  return n / z.block * z.bytes;
}

}  // extern "C"
