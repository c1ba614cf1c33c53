// GGUF reader (declared in include/mlxr_gguf.h): header, metadata and tensor infos of a
// .gguf file parsed from a read-only memory map, and the upload of quantized weights into
// the packed device layout.
//
// Follows the file format the reference reads in daemon/registry/gguf_parser.cpp
// (read_header :318-337, read_string :339-352, read_metadata_value :354-426,
// read_metadata :428-446, read_tensor_infos :448-491, data offset :306-313) and the
// mmap view of core/runtime/mmap_loader.cpp:102-199 (WILLNEED advice before an upload as
// advise(), :243-278), with the fixes listed in the header
// (GGUF block sizes, general.alignment, bounds-checked reads).
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/mlxr_gguf.h"
#include "../../include/mlxr_qgemm.h"
#include "qgemm_internal.h"

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF"
constexpr uint64_t kMaxString = 1ull << 30;

struct Value {
  uint32_t type = 0;
  uint64_t u = 0;  // integer / bool bits (sign-extended for signed types)
  double f = 0.0;
  uint64_t str_off = 0, len = 0;  // string: bytes at str_off; array: element count
  uint32_t elem_type = 0;
  uint64_t arr_off = 0;                // array: offset of the first element
  std::vector<uint64_t> str_elems;     // array of strings: offset of each element's length
};

struct Tensor {
  std::string name;
  uint32_t n_dims = 0;
  uint64_t dims[4] = {1, 1, 1, 1};
  uint32_t type = 0;
  uint64_t offset = 0, size = 0;
  bool size_known = false;
};

// Bytes per block and elements per block of the ggml types (ggml's type traits).
bool type_traits(uint32_t t, uint64_t* block_elems, uint64_t* block_bytes) {
  uint64_t be = 1, bb = 0;
  switch (t) {
    case MLXR_GGML_F32: bb = 4; break;
    case MLXR_GGML_F16: bb = 2; break;
    case MLXR_GGML_BF16: bb = 2; break;
    case MLXR_GGML_F64: bb = 8; break;
    case MLXR_GGML_I8: bb = 1; break;
    case MLXR_GGML_I16: bb = 2; break;
    case MLXR_GGML_I32: bb = 4; break;
    case MLXR_GGML_I64: bb = 8; break;
    case MLXR_GGML_Q4_0: be = 32; bb = 18; break;
    case MLXR_GGML_Q4_1: be = 32; bb = 20; break;
    case MLXR_GGML_Q5_0: be = 32; bb = 22; break;
    case MLXR_GGML_Q5_1: be = 32; bb = 24; break;
    case MLXR_GGML_Q8_0: be = 32; bb = 34; break;
    case MLXR_GGML_Q8_1: be = 32; bb = 36; break;
    case MLXR_GGML_Q2_K: be = 256; bb = 84; break;
    case MLXR_GGML_Q3_K: be = 256; bb = 110; break;
    case MLXR_GGML_Q4_K: be = 256; bb = 144; break;
    case MLXR_GGML_Q5_K: be = 256; bb = 176; break;
    case MLXR_GGML_Q6_K: be = 256; bb = 210; break;
    case MLXR_GGML_Q8_K: be = 256; bb = 292; break;
    default: return false;
  }
  *block_elems = be;
  *block_bytes = bb;
  return true;
}

size_t scalar_bytes(uint32_t t) {
  switch (t) {
    case MLXR_GGUF_UINT8: case MLXR_GGUF_INT8: case MLXR_GGUF_BOOL: return 1;
    case MLXR_GGUF_UINT16: case MLXR_GGUF_INT16: return 2;
    case MLXR_GGUF_UINT32: case MLXR_GGUF_INT32: case MLXR_GGUF_FLOAT32: return 4;
    case MLXR_GGUF_UINT64: case MLXR_GGUF_INT64: case MLXR_GGUF_FLOAT64: return 8;
    default: return 0;
  }
}

// Little-endian cursor over [base, base + size); every read is bounds-checked.
struct Reader {
  const uint8_t* base;
  uint64_t size, pos = 0;
  std::string err;
  bool need(uint64_t n, const char* what) {
    if (n > size - pos) {
      if (err.empty()) err = std::string("truncated file while reading ") + what;
      return false;
    }
    return true;
  }
  template <typename T>
  bool get(T* v, const char* what) {
    if (!need(sizeof(T), what)) return false;
    memcpy(v, base + pos, sizeof(T));
    pos += sizeof(T);
    return true;
  }
  // GGUF v1 stores lengths and counts as u32, v2+ as u64
  bool count(uint32_t version, uint64_t* v, const char* what) {
    if (version == 1) {
      uint32_t c;
      if (!get(&c, what)) return false;
      *v = c;
      return true;
    }
    return get(v, what);
  }
  bool string(uint32_t version, uint64_t* off, uint64_t* len, const char* what) {
    if (!count(version, len, what)) return false;
    if (*len > kMaxString) {
      err = std::string("invalid string length while reading ") + what;
      return false;
    }
    if (!need(*len, what)) return false;
    *off = pos;
    pos += *len;
    return true;
  }
};

}  // namespace

struct mlxr_gguf {
  const uint8_t* bytes = nullptr;
  uint64_t size = 0;
  void* map = nullptr;  // owned mapping (mlxr_gguf_open), unmapped on close
  mlxr_gguf_header hdr{};
  std::vector<std::string> keys;
  std::vector<Value> values;
  std::unordered_map<std::string, size_t> key_index;
  std::vector<Tensor> tensors;
  std::unordered_map<std::string, size_t> tensor_index;
};

namespace {

using mlxr::set_error;

bool read_value(Reader& r, uint32_t version, uint32_t type, Value& v, int depth) {
  v.type = type;
  const size_t sb = scalar_bytes(type);
  if (sb) {
    if (!r.need(sb, "metadata value")) return false;
    const uint8_t* p = r.base + r.pos;
    switch (type) {
      case MLXR_GGUF_UINT8: v.u = p[0]; break;
      case MLXR_GGUF_BOOL: v.u = p[0] != 0; break;
      case MLXR_GGUF_INT8: v.u = (uint64_t)(int64_t)(int8_t)p[0]; break;
      case MLXR_GGUF_UINT16: { uint16_t x; memcpy(&x, p, 2); v.u = x; break; }
      case MLXR_GGUF_INT16: { int16_t x; memcpy(&x, p, 2); v.u = (uint64_t)(int64_t)x; break; }
      case MLXR_GGUF_UINT32: { uint32_t x; memcpy(&x, p, 4); v.u = x; break; }
      case MLXR_GGUF_INT32: { int32_t x; memcpy(&x, p, 4); v.u = (uint64_t)(int64_t)x; break; }
      case MLXR_GGUF_UINT64: case MLXR_GGUF_INT64: memcpy(&v.u, p, 8); break;
      case MLXR_GGUF_FLOAT32: { float x; memcpy(&x, p, 4); v.f = x; break; }
      case MLXR_GGUF_FLOAT64: memcpy(&v.f, p, 8); break;
    }
    r.pos += sb;
    return true;
  }
  if (type == MLXR_GGUF_STRING) return r.string(version, &v.str_off, &v.len, "metadata string");
  if (type != MLXR_GGUF_ARRAY) {
    r.err = "unknown metadata type " + std::to_string(type);
    return false;
  }
  if (depth > 8) {
    r.err = "metadata arrays nested too deeply";
    return false;
  }
  if (!r.get(&v.elem_type, "array type") || !r.count(version, &v.len, "array length")) return false;
  v.arr_off = r.pos;
  const size_t eb = scalar_bytes(v.elem_type);
  if (eb) {
    if (v.len > (r.size - r.pos) / eb) {
      r.err = "truncated file while reading array data";
      return false;
    }
    r.pos += v.len * eb;
    return true;
  }
  if (v.elem_type == MLXR_GGUF_STRING) {
    if (v.len > (r.size - r.pos) / (version == 1 ? 4 : 8)) {
      r.err = "truncated file while reading a string array";
      return false;
    }
    v.str_elems.reserve(v.len);
    for (uint64_t j = 0; j < v.len; ++j) {
      v.str_elems.push_back(r.pos);
      uint64_t off, len;
      if (!r.string(version, &off, &len, "string array element")) return false;
    }
    return true;
  }
  for (uint64_t j = 0; j < v.len; ++j) {  // arrays of arrays: walked, not exposed
    Value inner;
    if (!read_value(r, version, v.elem_type, inner, depth + 1)) return false;
  }
  return true;
}

int parse(mlxr_gguf* g) {
  Reader r{g->bytes, g->size};
  mlxr_gguf_header& h = g->hdr;
  h.file_size = g->size;
  if (!r.get(&h.magic, "magic")) return set_error(MLXR_E_INVALID, "GGUF: %s", r.err.c_str());
  if (h.magic != kMagic) return set_error(MLXR_E_INVALID, "Invalid GGUF magic number 0x%08x", h.magic);
  if (!r.get(&h.version, "version")) return set_error(MLXR_E_INVALID, "GGUF: %s", r.err.c_str());
  if (h.version < 1 || h.version > 3) return set_error(MLXR_E_INVALID, "Unsupported GGUF version: %u", h.version);
  if (!r.count(h.version, &h.tensor_count, "tensor count") ||
      !r.count(h.version, &h.metadata_kv_count, "metadata count"))
    return set_error(MLXR_E_INVALID, "GGUF: %s", r.err.c_str());
  // every key-value pair and tensor info takes at least 12 bytes
  if (h.metadata_kv_count > g->size / 12 || h.tensor_count > g->size / 12)
    return set_error(MLXR_E_INVALID, "GGUF: implausible counts (%llu tensors, %llu keys) for a %llu-byte file",
                     (unsigned long long)h.tensor_count, (unsigned long long)h.metadata_kv_count,
                     (unsigned long long)g->size);
  h.alignment = 32;
  g->keys.reserve(h.metadata_kv_count);
  g->values.reserve(h.metadata_kv_count);
  for (uint64_t i = 0; i < h.metadata_kv_count; ++i) {
    uint64_t off, len;
    uint32_t type;
    Value v;
    if (!r.string(h.version, &off, &len, "metadata key") || !r.get(&type, "metadata type") ||
        !read_value(r, h.version, type, v, 0))
      return set_error(MLXR_E_INVALID, "GGUF metadata entry %llu: %s", (unsigned long long)i, r.err.c_str());
    std::string key((const char*)g->bytes + off, len);
    g->key_index[key] = g->keys.size();  // a repeated key: the last one wins
    g->keys.push_back(std::move(key));
    g->values.push_back(std::move(v));
  }
  auto it = g->key_index.find("general.alignment");
  if (it != g->key_index.end()) {
    const Value& v = g->values[it->second];
    const bool is_int = v.type == MLXR_GGUF_UINT32 || v.type == MLXR_GGUF_UINT64 || v.type == MLXR_GGUF_INT32 ||
                        v.type == MLXR_GGUF_UINT16 || v.type == MLXR_GGUF_UINT8;
    if (!is_int || v.u == 0 || (v.u & (v.u - 1)) != 0)
      return set_error(MLXR_E_INVALID, "GGUF: general.alignment must be a power of two");
    h.alignment = v.u;
  }
  g->tensors.reserve(h.tensor_count);
  for (uint64_t i = 0; i < h.tensor_count; ++i) {
    Tensor t;
    uint64_t off, len;
    if (!r.string(h.version, &off, &len, "tensor name") || !r.get(&t.n_dims, "tensor rank"))
      return set_error(MLXR_E_INVALID, "GGUF tensor info %llu: %s", (unsigned long long)i, r.err.c_str());
    t.name.assign((const char*)g->bytes + off, len);
    if (t.n_dims < 1 || t.n_dims > 4)
      return set_error(MLXR_E_INVALID, "GGUF tensor %s: rank %u outside 1..4", t.name.c_str(), t.n_dims);
    uint64_t n = 1;
    for (uint32_t d = 0; d < t.n_dims; ++d) {
      if (!r.count(h.version, &t.dims[d], "tensor dims"))
        return set_error(MLXR_E_INVALID, "GGUF tensor %s: %s", t.name.c_str(), r.err.c_str());
      if (t.dims[d] != 0 && n > (~0ull) / t.dims[d])
        return set_error(MLXR_E_INVALID, "GGUF tensor %s: element count overflows", t.name.c_str());
      n *= t.dims[d];
    }
    if (!r.get(&t.type, "tensor type") || !r.get(&t.offset, "tensor offset"))
      return set_error(MLXR_E_INVALID, "GGUF tensor %s: %s", t.name.c_str(), r.err.c_str());
    uint64_t be, bb;
    if (type_traits(t.type, &be, &bb) && n % be == 0 && n / be <= (~0ull) / bb) {
      t.size = n / be * bb;
      t.size_known = true;
    }
    g->tensor_index.emplace(t.name, g->tensors.size());  // first tensor of a name wins
    g->tensors.push_back(std::move(t));
  }
  h.data_offset = (r.pos + h.alignment - 1) / h.alignment * h.alignment;
  return MLXR_OK;
}

int finish_open(mlxr_gguf* g, mlxr_gguf** out) {
  const int rc = parse(g);
  if (rc) {
    mlxr_gguf_close(g);
    return rc;
  }
  *out = g;
  return MLXR_OK;
}

}  // namespace

extern "C" {

int mlxr_gguf_open(const char* path, mlxr_gguf** out) {
  if (!path || !out) return set_error(MLXR_E_INVALID, "null argument");
  *out = nullptr;
  const int fd = open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) return set_error(MLXR_E_INVALID, "Failed to open file: %s", path);
  struct stat st;
  if (fstat(fd, &st) != 0 || st.st_size <= 0) {
    close(fd);
    return set_error(MLXR_E_INVALID, "Failed to open file: %s (empty or unreadable)", path);
  }
  void* m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (m == MAP_FAILED) return set_error(MLXR_E_INVALID, "mmap of %s failed", path);
  mlxr_gguf* g = new mlxr_gguf;
  g->map = m;
  g->bytes = (const uint8_t*)m;
  g->size = (uint64_t)st.st_size;
  return finish_open(g, out);
}

int mlxr_gguf_open_memory(const void* bytes, size_t size, mlxr_gguf** out) {
  if (!bytes || !out) return set_error(MLXR_E_INVALID, "null argument");
  *out = nullptr;
  mlxr_gguf* g = new mlxr_gguf;
  g->bytes = (const uint8_t*)bytes;
  g->size = size;
  return finish_open(g, out);
}

void mlxr_gguf_close(mlxr_gguf* g) {
  if (!g) return;
  if (g->map) munmap(g->map, (size_t)g->size);
  delete g;
}

int mlxr_gguf_get_header(const mlxr_gguf* g, mlxr_gguf_header* out) {
  if (!g || !out) return set_error(MLXR_E_INVALID, "null argument");
  *out = g->hdr;
  return MLXR_OK;
}

int mlxr_gguf_get_tensor(const mlxr_gguf* g, uint64_t i, mlxr_gguf_tensor_info* out) {
  if (!g || !out) return set_error(MLXR_E_INVALID, "null argument");
  if (i >= g->tensors.size()) return set_error(MLXR_E_INVALID, "tensor index %llu out of range", (unsigned long long)i);
  const Tensor& t = g->tensors[i];
  out->name = t.name.c_str();
  out->n_dims = t.n_dims;
  for (int d = 0; d < 4; ++d) out->dims[d] = t.dims[d];
  out->type = t.type;
  out->offset = t.offset;
  out->file_offset = g->hdr.data_offset + t.offset;
  out->size = t.size;
  const bool in_file = t.size_known && t.offset <= g->size && g->hdr.data_offset <= g->size - t.offset &&
                       t.size <= g->size - g->hdr.data_offset - t.offset;
  out->data = in_file ? g->bytes + g->hdr.data_offset + t.offset : nullptr;
  return MLXR_OK;
}

int64_t mlxr_gguf_find_tensor(const mlxr_gguf* g, const char* name) {
  if (!g || !name) return -1;
  auto it = g->tensor_index.find(name);
  return it == g->tensor_index.end() ? -1 : (int64_t)it->second;
}

static void fill_value(const mlxr_gguf* g, const Value& v, mlxr_gguf_value* out) {
  memset(out, 0, sizeof(*out));
  out->type = v.type;
  if (v.type == MLXR_GGUF_FLOAT32 || v.type == MLXR_GGUF_FLOAT64) out->v.f64 = v.f;
  else out->v.u64 = v.u;
  if (v.type == MLXR_GGUF_STRING) {
    out->str = (const char*)g->bytes + v.str_off;
    out->len = v.len;
  } else if (v.type == MLXR_GGUF_ARRAY) {
    out->len = v.len;
    out->elem_type = v.elem_type;
    out->data = scalar_bytes(v.elem_type) ? g->bytes + v.arr_off : nullptr;
  }
}

int mlxr_gguf_get_key(const mlxr_gguf* g, uint64_t i, const char** key, mlxr_gguf_value* out) {
  if (!g || !key || !out) return set_error(MLXR_E_INVALID, "null argument");
  if (i >= g->keys.size()) return set_error(MLXR_E_INVALID, "metadata index %llu out of range", (unsigned long long)i);
  *key = g->keys[i].c_str();
  fill_value(g, g->values[i], out);
  return MLXR_OK;
}

int mlxr_gguf_get_value(const mlxr_gguf* g, const char* key, mlxr_gguf_value* out) {
  if (!g || !key || !out) return set_error(MLXR_E_INVALID, "null argument");
  auto it = g->key_index.find(key);
  if (it == g->key_index.end()) return set_error(MLXR_E_INVALID, "no metadata key %s", key);
  fill_value(g, g->values[it->second], out);
  return MLXR_OK;
}

int mlxr_gguf_get_array_string(const mlxr_gguf* g, const char* key, uint64_t j, const char** s, uint64_t* len) {
  if (!g || !key || !s || !len) return set_error(MLXR_E_INVALID, "null argument");
  auto it = g->key_index.find(key);
  if (it == g->key_index.end()) return set_error(MLXR_E_INVALID, "no metadata key %s", key);
  const Value& v = g->values[it->second];
  if (v.type != MLXR_GGUF_ARRAY || v.elem_type != MLXR_GGUF_STRING)
    return set_error(MLXR_E_INVALID, "metadata %s is not an array of strings", key);
  if (j >= v.str_elems.size()) return set_error(MLXR_E_INVALID, "index %llu out of range", (unsigned long long)j);
  const uint64_t p = v.str_elems[j];
  uint64_t n;
  if (g->hdr.version == 1) {
    uint32_t c;
    memcpy(&c, g->bytes + p, 4);
    n = c;
    *s = (const char*)g->bytes + p + 4;
  } else {
    memcpy(&n, g->bytes + p, 8);
    *s = (const char*)g->bytes + p + 8;
  }
  *len = n;
  return MLXR_OK;
}

int mlxr_gguf_type_bytes(uint32_t ggml_type, uint64_t n, uint64_t* bytes) {
  if (!bytes) return set_error(MLXR_E_INVALID, "null argument");
  uint64_t be, bb;
  if (!type_traits(ggml_type, &be, &bb)) return set_error(MLXR_E_UNSUPPORTED, "unknown ggml type %u", ggml_type);
  if (n % be != 0)
    return set_error(MLXR_E_SHAPE, "%llu elements are not whole %s blocks of %llu", (unsigned long long)n,
                     mlxr_gguf_type_name(ggml_type), (unsigned long long)be);
  *bytes = n / be * bb;
  return MLXR_OK;
}

int mlxr_gguf_block_size(uint32_t ggml_type) {
  uint64_t be, bb;
  return type_traits(ggml_type, &be, &bb) ? (int)be : 1;
}

const char* mlxr_gguf_type_name(uint32_t t) {
  switch (t) {
    case MLXR_GGML_F32: return "F32";
    case MLXR_GGML_F16: return "F16";
    case MLXR_GGML_BF16: return "BF16";
    case MLXR_GGML_F64: return "F64";
    case MLXR_GGML_Q4_0: return "Q4_0";
    case MLXR_GGML_Q4_1: return "Q4_1";
    case MLXR_GGML_Q5_0: return "Q5_0";
    case MLXR_GGML_Q5_1: return "Q5_1";
    case MLXR_GGML_Q8_0: return "Q8_0";
    case MLXR_GGML_Q8_1: return "Q8_1";
    case MLXR_GGML_Q2_K: return "Q2_K";
    case MLXR_GGML_Q3_K: return "Q3_K";
    case MLXR_GGML_Q4_K: return "Q4_K";
    case MLXR_GGML_Q5_K: return "Q5_K";
    case MLXR_GGML_Q6_K: return "Q6_K";
    case MLXR_GGML_Q8_K: return "Q8_K";
    case MLXR_GGML_I8: return "I8";
    case MLXR_GGML_I16: return "I16";
    case MLXR_GGML_I32: return "I32";
    case MLXR_GGML_I64: return "I64";
    default: return "UNKNOWN";
  }
}

int mlxr_gguf_quant_type(uint32_t ggml_type) {
  switch (ggml_type) {
    case MLXR_GGML_Q4_0: return MLXR_Q4_0;
    case MLXR_GGML_Q4_1: return MLXR_Q4_1;
    case MLXR_GGML_Q8_0: return MLXR_Q8_0;
    case MLXR_GGML_Q4_K: return MLXR_Q4_K;
    case MLXR_GGML_Q5_K: return MLXR_Q5_K;
    case MLXR_GGML_Q6_K: return MLXR_Q6_K;
    default:
      return set_error(MLXR_E_UNSUPPORTED, "ggml type %s has no quantized matmul", mlxr_gguf_type_name(ggml_type));
  }
}

int mlxr_gguf_upload(const mlxr_gguf* g, uint64_t i, void* packed_dev, void* stream) {
  mlxr_gguf_tensor_info t;
  int rc = mlxr_gguf_get_tensor(g, i, &t);
  if (rc) return rc;
  const int qt = mlxr_gguf_quant_type(t.type);
  if (qt < 0) return qt;
  if (t.n_dims != 2 || t.dims[0] > 0x7fffffffull || t.dims[1] > 0x7fffffffull)
    return set_error(MLXR_E_SHAPE, "tensor %s is not a 2-D weight with dims below 2^31", t.name);
  if (!t.data)
    return set_error(MLXR_E_INVALID, "tensor %s: data range [%llu, +%llu) is outside the %llu-byte file", t.name,
                     (unsigned long long)t.file_offset, (unsigned long long)t.size,
                     (unsigned long long)g->hdr.file_size);
  if (g->map) {
    // the pack reads the tensor once, front to back: ask for its pages ahead of the copy
    // (as the reference's WILLNEED advice on a mapped region; advisory, errors ignored)
    const uintptr_t pg = (uintptr_t)sysconf(_SC_PAGESIZE);
    const uintptr_t a = (uintptr_t)t.data & ~(pg - 1);
    const uintptr_t e = ((uintptr_t)t.data + (uintptr_t)t.size + pg - 1) & ~(pg - 1);
    (void)madvise((void*)a, (size_t)(e - a), MADV_WILLNEED);
  }
  return mlxr_qgemm_pack(qt, (int)t.dims[1], (int)t.dims[0], t.data, packed_dev, stream);
}

}  // extern "C"
