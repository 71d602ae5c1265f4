// nx_gguf.hip — GGUF model files (host code): parser and the quantized-
// resident MoE expert loader.
//
// Parsing follows GgufReader::parse_file / parse_from_bytes
// (src/gguf/mod.rs:869-876, 1091-1310): the file is memory-mapped; magic
// "GGUF", version 2 or 3, u64 tensor and key/value counts, the key/value
// pairs, then the tensor table (u64 name length, name, u32 dims, u64 dims
// innermost first, u32 type, u64 offset).  Tensor data starts at the end of
// the table rounded up to general.alignment (a U32 or U64 value, default 32).
// Error messages are the reference's.  Where the reference indexes past the
// end of a truncated metadata value (a panic there), this parser returns
// "Unexpected EOF reading metadata value".  Array values keep the
// reference's handling: I32, F32 and String arrays are read, other element
// types are skipped as 12 + 4 * length bytes.
//
// The expert loader keeps the payloads quantized: each expert matrix goes
// from the mapping into the resident layout through nx_experts_load, with no
// f32 copy and no element cap (the reference dequantizes every tensor to f32
// at load and skips tensors above 10M elements, src/engine/mod.rs:600-612).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "nx_internal.hpp"

namespace {

// GgufValueType ids (src/gguf/mod.rs:329-345)
enum ValType {
  V_U8 = 0, V_I8 = 1, V_U16 = 2, V_I16 = 3, V_U32 = 4, V_I32 = 5, V_F32 = 6, V_BOOL = 7,
  V_STRING = 8, V_ARRAY = 9, V_U64 = 10, V_I64 = 11, V_F64 = 12
};

struct Value {
  int type = -1;   // ValType of a scalar or string; V_ARRAY for arrays
  int elem = -1;   // element type of an array (as stored: I32, F32, String, or skipped)
  uint64_t u = 0;  // unsigned integer or raw bits
  int64_t i = 0;
  double f = 0;
  std::string s;
  size_t count = 0;  // array length (0 for skipped element types)
};

// Bytes of n elements of GGUF type `id`, or -1 for an id the reference does
// not know (GgufDataType::from_id and bytes_per_element, src/gguf/mod.rs:153-293).
int64_t type_bytes(uint32_t id, uint64_t n) {
  auto blocks = [&](uint64_t block, uint64_t size) { return (int64_t)((n + block - 1) / block * size); };
  switch (id) {
    case 0: case 47: return (int64_t)(n * 4);          // F32, TF32
    case 1: case 28: return (int64_t)(n * 2);          // F16, BF16
    case 16: return (int64_t)n;                        // I8
    case 17: return (int64_t)(n * 2);                  // I16
    case 18: return (int64_t)(n * 4);                  // I32
    case 19: case 20: return (int64_t)(n * 8);         // I64, F64
    case 2: case 36: case 37: return blocks(32, 18);   // Q4_0 (+ 4x4, 8x8)
    case 3: return blocks(32, 20);                     // Q4_1
    case 6: return blocks(32, 22);                     // Q5_0
    case 7: return blocks(32, 24);                     // Q5_1
    case 8: return blocks(32, 34);                     // Q8_0
    case 9: return blocks(32, 36);                     // Q8_1
    case 10: return blocks(256, 84);                   // Q2_K
    case 11: return blocks(256, 110);                  // Q3_K
    case 12: return blocks(256, 144);                  // Q4_K
    case 13: return blocks(256, 176);                  // Q5_K
    case 14: return blocks(256, 210);                  // Q6_K
    case 15: return blocks(256, 292);                  // Q8_K
    case 38: return blocks(256, 324);                  // Q9_K
    case 25: case 31: return blocks(256, 32);          // IQ1_S, IQ1_N
    case 21: case 22: case 34: case 23: return blocks(256, 64);  // IQ2_XXS/XS/S, Q2_S
    case 24: case 27: return blocks(256, 96);          // IQ3_XXS, IQ3_S
    case 26: case 30: case 41: case 42: return (int64_t)((n + 1) / 2);  // IQ4_NL/XS, F4E2M1(x2)
    case 43: case 44: case 45: case 46: return (int64_t)n;  // F8 types
    case 39: case 40: return (int64_t)n;               // I8x4, I8x8
    default: return -1;
  }
}

}  // namespace

struct nx_gguf {
  int fd = -1;
  const uint8_t *data = nullptr;
  size_t len = 0;
  uint32_t version = 0;
  uint64_t tensor_count = 0, kv_count = 0;
  size_t alignment = 32;
  uint64_t data_offset = 0;
  std::map<std::string, Value> meta;
  struct Tensor {
    std::string name;
    uint32_t type = 0;
    std::vector<uint64_t> dims;
    uint64_t offset = 0;  // relative to the data section
    uint64_t elements() const {
      uint64_t n = 1;
      for (uint64_t d : dims) n *= d;
      return n;
    }
  };
  std::vector<Tensor> tensors;
};

namespace {

using nx::fail;

struct Cursor {
  const uint8_t *d;
  size_t len, pos;
  bool has(size_t n) const { return n <= len && pos <= len - n; }
  uint32_t u32() { uint32_t v; std::memcpy(&v, d + pos, 4); pos += 4; return v; }
  uint64_t u64() { uint64_t v; std::memcpy(&v, d + pos, 8); pos += 8; return v; }
};

const char *EOF_VALUE = "Unexpected EOF reading metadata value";

// UTF-8 well-formedness (the reference's std::str::from_utf8)
bool utf8_ok(const uint8_t *p, size_t n) {
  size_t i = 0;
  while (i < n) {
    const uint8_t c = p[i];
    size_t k;
    uint8_t lo = 0x80, hi = 0xBF;  // bounds of the second byte
    if (c < 0x80) {
      k = 0;
    } else if (c >= 0xC2 && c <= 0xDF) {
      k = 1;
    } else if (c >= 0xE0 && c <= 0xEF) {
      k = 2;
      if (c == 0xE0) lo = 0xA0;
      if (c == 0xED) hi = 0x9F;
    } else if (c >= 0xF0 && c <= 0xF4) {
      k = 3;
      if (c == 0xF0) lo = 0x90;
      if (c == 0xF4) hi = 0x8F;
    } else {
      return false;
    }
    if (k > n - 1 - i) return false;
    for (size_t j = 1; j <= k; ++j) {
      const uint8_t b = p[i + j];
      if (j == 1 ? (b < lo || b > hi) : (b & 0xC0) != 0x80) return false;
    }
    i += k + 1;
  }
  return true;
}

// one metadata value (GgufReader::read_value_from_bytes, src/gguf/mod.rs:1312-1533)
int read_value(Cursor &c, uint32_t type, Value &v) {
  v.type = (int)type;
  auto need = [&](size_t n) { return c.has(n) ? 0 : fail(NX_ERR_TRUNCATED, EOF_VALUE); };
  switch (type) {
    case V_BOOL: case V_U8: case V_I8: {
      NX_TRY(need(1));
      const uint8_t b = c.d[c.pos++];
      v.u = type == V_BOOL ? (b != 0) : b;
      v.i = type == V_I8 ? (int8_t)b : (int64_t)v.u;
      return NX_OK;
    }
    case V_U16: case V_I16: {
      NX_TRY(need(2));
      uint16_t h;
      std::memcpy(&h, c.d + c.pos, 2);
      c.pos += 2;
      v.u = h;
      v.i = type == V_I16 ? (int16_t)h : (int64_t)h;
      return NX_OK;
    }
    case V_U32: case V_I32: case V_F32: {
      NX_TRY(need(4));
      const uint32_t w = c.u32();
      v.u = w;
      v.i = type == V_I32 ? (int32_t)w : (int64_t)w;
      float f;
      std::memcpy(&f, &w, 4);
      v.f = f;
      return NX_OK;
    }
    case V_U64: case V_I64: case V_F64: {
      NX_TRY(need(8));
      const uint64_t w = c.u64();
      v.u = w;
      v.i = (int64_t)w;
      double f;
      std::memcpy(&f, &w, 8);
      v.f = f;
      return NX_OK;
    }
    case V_STRING: {
      NX_TRY(need(8));
      const uint64_t n = c.u64();
      NX_TRY(need(n));
      if (!utf8_ok(c.d + c.pos, n)) return fail(NX_ERR_SHAPE, "invalid utf-8 in a metadata string");
      v.s.assign((const char *)c.d + c.pos, n);
      c.pos += n;
      return NX_OK;
    }
    case V_ARRAY: {
      NX_TRY(need(12));
      const uint32_t et = c.u32();
      if (et > 12) return fail(NX_ERR_SHAPE, "Unknown array type");
      const uint64_t n = c.u64();
      v.elem = (int)et;
      if (et == V_I32 || et == V_F32) {
        if (n > (c.len - c.pos) / 4) return fail(NX_ERR_TRUNCATED, EOF_VALUE);
        c.pos += 4 * n;
        v.count = n;
      } else if (et == V_STRING) {
        for (uint64_t k = 0; k < n; ++k) {
          NX_TRY(need(8));
          const uint64_t sl = c.u64();
          NX_TRY(need(sl));
          if (!utf8_ok(c.d + c.pos, sl))
            return fail(NX_ERR_SHAPE, "invalid utf-8 in a metadata string");
          c.pos += sl;
        }
        v.count = n;
      } else {
        // other element types: skipped as 4 bytes each, value an empty array
        if (n > (c.len - c.pos) / 4) return fail(NX_ERR_TRUNCATED, EOF_VALUE);
        c.pos += 4 * n;
        v.count = 0;
      }
      return NX_OK;
    }
    default:
      return fail(NX_ERR_SHAPE, "Unknown value type: " + std::to_string(type));
  }
}

int parse(nx_gguf *g) {
  Cursor c{g->data, g->len, 0};
  if (g->len < 8 || std::memcmp(g->data, "GGUF", 4) != 0)
    return fail(NX_ERR_SHAPE, "Invalid GGUF magic");
  c.pos = 4;
  g->version = c.u32();
  if (g->version != 2 && g->version != 3)
    return fail(NX_ERR_UNSUPPORTED, "Unsupported GGUF version: " + std::to_string(g->version));
  if (!c.has(8)) return fail(NX_ERR_TRUNCATED, "Unexpected EOF reading tensor count");
  g->tensor_count = c.u64();
  if (!c.has(8)) return fail(NX_ERR_TRUNCATED, "Unexpected EOF reading kv count");
  g->kv_count = c.u64();
  for (uint64_t k = 0; k < g->kv_count; ++k) {
    if (!c.has(8)) return fail(NX_ERR_TRUNCATED, "Unexpected EOF reading metadata key length");
    const uint64_t kl = c.u64();
    if (!c.has(kl)) return fail(NX_ERR_TRUNCATED, "Key string exceeds file bounds");
    if (!utf8_ok(c.d + c.pos, kl)) return fail(NX_ERR_SHAPE, "invalid utf-8 in a metadata key");
    std::string key((const char *)c.d + c.pos, kl);
    c.pos += kl;
    if (!c.has(4)) return fail(NX_ERR_TRUNCATED, "Unexpected EOF reading value type");
    const uint32_t type = c.u32();
    if (type > 12) return fail(NX_ERR_SHAPE, "Unknown value type: " + std::to_string(type));
    Value v;
    NX_TRY(read_value(c, type, v));
    g->meta[key] = v;  // a repeated key keeps the last value, as a HashMap insert does
  }
  for (uint64_t t = 0; t < g->tensor_count; ++t) {
    if (!c.has(8)) return fail(NX_ERR_TRUNCATED, "Unexpected EOF reading tensor name length");
    const uint64_t nl = c.u64();
    if (!c.has(nl)) return fail(NX_ERR_TRUNCATED, "Tensor name exceeds file bounds");
    if (!utf8_ok(c.d + c.pos, nl)) return fail(NX_ERR_SHAPE, "invalid utf-8 in a tensor name");
    nx_gguf::Tensor ti;
    ti.name.assign((const char *)c.d + c.pos, nl);
    c.pos += nl;
    if (!c.has(4)) return fail(NX_ERR_TRUNCATED, "Unexpected EOF reading dims");
    const uint32_t nd = c.u32();
    for (uint32_t d = 0; d < nd; ++d) {
      if (!c.has(8)) return fail(NX_ERR_TRUNCATED, "Unexpected EOF reading shape");
      ti.dims.push_back(c.u64());
    }
    if (!c.has(4)) return fail(NX_ERR_TRUNCATED, "Unexpected EOF reading data type");
    ti.type = c.u32();
    if (type_bytes(ti.type, 0) < 0)
      return fail(NX_ERR_SHAPE, "Unknown data type: " + std::to_string(ti.type));
    if (!c.has(8)) return fail(NX_ERR_TRUNCATED, "Unexpected EOF reading tensor offset");
    ti.offset = c.u64();
    g->tensors.push_back(std::move(ti));
  }
  size_t align = 32;
  auto it = g->meta.find("general.alignment");
  if (it != g->meta.end() && (it->second.type == V_U32 || it->second.type == V_U64))
    align = (size_t)it->second.u;
  if (align == 0) align = 1;
  g->alignment = align;
  g->data_offset = (c.pos + align - 1) / align * align;
  return NX_OK;
}

const nx_gguf::Tensor *find(const nx_gguf *g, const std::string &name, size_t *index = nullptr) {
  for (size_t i = 0; i < g->tensors.size(); ++i)
    if (g->tensors[i].name == name) {
      if (index) *index = i;
      return &g->tensors[i];
    }
  return nullptr;
}

// payload of a tensor inside the mapping
int tensor_payload(const nx_gguf *g, const nx_gguf::Tensor &t, const uint8_t **p, uint64_t *bytes) {
  const int64_t b = type_bytes(t.type, t.elements());
  const uint64_t start = g->data_offset + t.offset;
  if (b < 0 || start > g->len || (uint64_t)b > g->len - start)
    return fail(NX_ERR_TRUNCATED, "tensor " + t.name + " extends past the end of the file");
  *p = g->data + start;
  *bytes = (uint64_t)b;
  return NX_OK;
}

}  // namespace

extern "C" {

int nx_gguf_open(const char *path, nx_gguf **out) {
  nx::clear_error();
  if (!path || !out) return fail(NX_ERR_INVALID_ARG, "null argument");
  *out = nullptr;
  const int fd = ::open(path, O_RDONLY);
  if (fd < 0) return fail(NX_ERR_IO, std::string(std::strerror(errno)) + ": " + path);
  struct stat st;
  if (fstat(fd, &st) != 0) {
    const int e = errno;
    ::close(fd);
    return fail(NX_ERR_IO, std::string(std::strerror(e)) + ": " + path);
  }
  nx_gguf *g = new nx_gguf;
  g->fd = fd;
  g->len = (size_t)st.st_size;
  if (g->len > 0) {
    void *m = mmap(nullptr, g->len, PROT_READ, MAP_PRIVATE, fd, 0);
    if (m == MAP_FAILED) {
      const int e = errno;
      ::close(fd);
      delete g;
      return fail(NX_ERR_IO, std::string("mmap: ") + std::strerror(e));
    }
    g->data = (const uint8_t *)m;
  }
  const int rc = parse(g);
  if (rc) {
    nx_gguf_close(g);
    return rc;
  }
  *out = g;
  return NX_OK;
}

int nx_gguf_close(nx_gguf *g) {
  if (!g) return NX_OK;
  if (g->data) munmap((void *)g->data, g->len);
  if (g->fd >= 0) ::close(g->fd);
  delete g;
  return NX_OK;
}

int nx_gguf_info(const nx_gguf *g, uint32_t *version, size_t *tensor_count, size_t *kv_count,
                 size_t *alignment, uint64_t *data_offset) {
  if (!g) return fail(NX_ERR_INVALID_ARG, "null GGUF handle");
  if (version) *version = g->version;
  if (tensor_count) *tensor_count = g->tensors.size();
  if (kv_count) *kv_count = g->meta.size();
  if (alignment) *alignment = g->alignment;
  if (data_offset) *data_offset = g->data_offset;
  return NX_OK;
}

int nx_gguf_tensor(const nx_gguf *g, size_t index, char *name, size_t name_cap, uint32_t *type,
                   uint32_t *n_dims, uint64_t *dims, size_t dims_cap, uint64_t *offset,
                   uint64_t *bytes) {
  if (!g) return fail(NX_ERR_INVALID_ARG, "null GGUF handle");
  if (index >= g->tensors.size()) return fail(NX_ERR_INVALID_ARG, "tensor index out of range");
  const auto &t = g->tensors[index];
  if (name && name_cap) {
    const size_t n = std::min(name_cap - 1, t.name.size());
    std::memcpy(name, t.name.data(), n);
    name[n] = 0;
  }
  if (type) *type = t.type;
  if (n_dims) *n_dims = (uint32_t)t.dims.size();
  if (dims)
    for (size_t d = 0; d < t.dims.size() && d < dims_cap; ++d) dims[d] = t.dims[d];
  if (offset) *offset = g->data_offset + t.offset;
  if (bytes) *bytes = (uint64_t)std::max<int64_t>(0, type_bytes(t.type, t.elements()));
  return NX_OK;
}

int nx_gguf_find_tensor(const nx_gguf *g, const char *name, size_t *index) {
  if (!g || !name) return fail(NX_ERR_INVALID_ARG, "null argument");
  size_t i = 0;
  if (!find(g, name, &i)) return fail(NX_ERR_NOT_FOUND, std::string("Missing tensor: ") + name);
  if (index) *index = i;
  return NX_OK;
}

int nx_gguf_tensor_data(const nx_gguf *g, size_t index, const void **data, uint64_t *bytes) {
  if (!g || !data) return fail(NX_ERR_INVALID_ARG, "null argument");
  if (index >= g->tensors.size()) return fail(NX_ERR_INVALID_ARG, "tensor index out of range");
  const uint8_t *p;
  uint64_t b;
  NX_TRY(tensor_payload(g, g->tensors[index], &p, &b));
  *data = p;
  if (bytes) *bytes = b;
  return NX_OK;
}

// ModelMetadata::get_usize (src/gguf/mod.rs:512-521): U64, U32, or a
// non-negative I64 / I32
int nx_gguf_meta_usize(const nx_gguf *g, const char *key, uint64_t *value) {
  if (!g || !key || !value) return fail(NX_ERR_INVALID_ARG, "null argument");
  auto it = g->meta.find(key);
  if (it != g->meta.end()) {
    const Value &v = it->second;
    if (v.type == V_U64 || v.type == V_U32) {
      *value = v.u;
      return NX_OK;
    }
    if ((v.type == V_I64 || v.type == V_I32) && v.i >= 0) {
      *value = (uint64_t)v.i;
      return NX_OK;
    }
  }
  return fail(NX_ERR_NOT_FOUND, std::string("no unsigned metadata value ") + key);
}

// ModelMetadata::get_f32: an F32 value
int nx_gguf_meta_f32(const nx_gguf *g, const char *key, float *value) {
  if (!g || !key || !value) return fail(NX_ERR_INVALID_ARG, "null argument");
  auto it = g->meta.find(key);
  if (it == g->meta.end() || it->second.type != V_F32)
    return fail(NX_ERR_NOT_FOUND, std::string("no f32 metadata value ") + key);
  *value = (float)it->second.f;
  return NX_OK;
}

// ModelMetadata::get_str: a String value; *len gets its length in bytes
int nx_gguf_meta_str(const nx_gguf *g, const char *key, char *buf, size_t cap, size_t *len) {
  if (!g || !key) return fail(NX_ERR_INVALID_ARG, "null argument");
  auto it = g->meta.find(key);
  if (it == g->meta.end() || it->second.type != V_STRING)
    return fail(NX_ERR_NOT_FOUND, std::string("no string metadata value ") + key);
  const std::string &s = it->second.s;
  if (len) *len = s.size();
  if (buf && cap) {
    const size_t n = std::min(cap - 1, s.size());
    std::memcpy(buf, s.data(), n);
    buf[n] = 0;
  }
  return NX_OK;
}

}  // extern "C"

// ------------------------------------------------------------ MoE experts
namespace {

// Q4_K code bytes from upstream ggml's order (per 64 elements j: 32 bytes,
// low nibbles = elements 64j .. 64j+31, high nibbles = 64j+32 .. 64j+63) to
// the reference's (element i < 128: low nibble of byte i; i >= 128: high
// nibble of byte i - 128; src/quant/mod.rs:833-841).  Scales are shared.
void q4k_ggml_to_reference(const uint8_t *src, uint8_t *dst, size_t blocks) {
  for (size_t b = 0; b < blocks; ++b) {
    const uint8_t *s = src + b * 144;
    uint8_t *d = dst + b * 144;
    std::memcpy(d, s, 16);
    uint8_t code[256];
    for (int i = 0; i < 256; ++i) {
      const int j = i / 64, l = i % 64;
      const uint8_t byte = s[16 + 32 * j + (l % 32)];
      code[i] = l < 32 ? (byte & 15) : (byte >> 4);
    }
    for (int i = 0; i < 128; ++i) d[16 + i] = (uint8_t)(code[i] | (code[i + 128] << 4));
  }
}

struct RoleTensor {
  const nx_gguf::Tensor *t = nullptr;
  bool merged = false;  // one 3-D tensor for all experts
};

// the names a block's expert matrices go by (cf. the reference's
// layer_tensor_names, src/engine/mod.rs:727-746, which has none for MoE)
std::vector<std::string> expert_names(int layer, int role, int expert) {
  static const char *gguf_role[3] = {"ffn_gate", "ffn_up", "ffn_down"};
  static const char *hf_mixtral[3] = {"w1", "w3", "w2"};
  static const char *hf_proj[3] = {"gate_proj", "up_proj", "down_proj"};
  const std::string L = std::to_string(layer), e = std::to_string(expert);
  if (expert == NX_EXPERT_SHARED)
    return {"blk." + L + "." + gguf_role[role] + "_shexp.weight",
            "model.layers." + L + ".mlp.shared_experts." + hf_proj[role] + ".weight",
            "model.layers." + L + ".mlp.shared_expert." + hf_proj[role] + ".weight"};
  return {"blk." + L + "." + gguf_role[role] + "." + e + ".weight",
          "model.layers." + L + ".block_sparse_moe.experts." + e + "." + hf_mixtral[role] + ".weight",
          "model.layers." + L + ".mlp.experts." + e + "." + hf_proj[role] + ".weight"};
}

const nx_gguf::Tensor *find_any(const nx_gguf *g, const std::vector<std::string> &names) {
  for (const auto &n : names)
    if (const auto *t = find(g, n)) return t;
  return nullptr;
}

bool supported_fmt(uint32_t type) {
  return type == NX_FMT_F32 || type == NX_FMT_Q4_0 || type == NX_FMT_Q8_0 || type == NX_FMT_Q4_K ||
         type == NX_FMT_Q2_K || type == NX_FMT_F16 || type == NX_FMT_BF16;
}

// expert tensors of block `layer`: merged blk.L.ffn_{gate,up,down}_exps
// (dims [cols, rows, E]) or one 2-D tensor per expert
int moe_layout(const nx_gguf *g, int layer, RoleTensor role[3], int *E, int *H, int *F,
               uint32_t *fmt, const nx_gguf::Tensor *shared[3], int *Fs) {
  static const char *merged[3] = {"ffn_gate_exps", "ffn_up_exps", "ffn_down_exps"};
  const std::string L = std::to_string(layer);
  int e_count = -1;
  for (int r = 0; r < 3; ++r) {
    role[r] = {};
    if (const auto *t = find(g, "blk." + L + "." + merged[r] + ".weight")) {
      if (t->dims.size() != 3)
        return fail(NX_ERR_SHAPE, "merged expert tensor " + t->name + " is not 3-D");
      role[r] = {t, true};
    } else if (const auto *t0 = find_any(g, expert_names(layer, r, 0))) {
      role[r] = {t0, false};
    } else {
      return fail(NX_ERR_NOT_FOUND, "Missing tensor: blk." + L + "." + merged[r] + ".weight or blk." +
                                        L + "." + (r == 0 ? "ffn_gate" : r == 1 ? "ffn_up" : "ffn_down") +
                                        ".0.weight");
    }
  }
  // per-expert naming: count experts 0, 1, ... present for all three roles
  int n_sep = 0;
  if (!role[0].merged || !role[1].merged || !role[2].merged) {
    while (find_any(g, expert_names(layer, 0, n_sep)) && find_any(g, expert_names(layer, 1, n_sep)) &&
           find_any(g, expert_names(layer, 2, n_sep)))
      ++n_sep;
  }
  // shapes: gate/up [H cols, F rows], down [F cols, H rows]; a file may
  // declare any number of dims, so check before reading them
  for (int r = 0; r < 3; ++r)
    if (role[r].t->dims.size() < 2)
      return fail(NX_ERR_SHAPE, "expert tensor " + role[r].t->name + " has fewer than 2 dims");
  const auto &tg = *role[0].t, &tu = *role[1].t, &td = *role[2].t;
  const uint64_t h = tg.dims[0], f = tg.dims[1];
  for (int r = 0; r < 3; ++r) {
    const auto &t = *role[r].t;
    if (t.type != tg.type)
      return fail(NX_ERR_SHAPE, "expert tensors of block " + L + " mix types");
    const int ecount = role[r].merged ? (int)t.dims[2] : n_sep;
    if (e_count < 0) e_count = ecount;
    if (ecount != e_count)
      return fail(NX_ERR_SHAPE, "expert counts of block " + L + " differ between roles");
  }
  if (tu.dims.size() < 2 || td.dims.size() < 2 || tu.dims[0] != h || tu.dims[1] != f ||
      td.dims[0] != f || td.dims[1] != h)
    return fail(NX_ERR_SHAPE, "expert matrix shapes of block " + L + " are inconsistent");
  if (!supported_fmt(tg.type))
    return fail(NX_ERR_UNSUPPORTED, "expert tensor type " + std::to_string(tg.type) +
                                        " is not resident-capable (F32, F16, BF16, Q4_0, Q8_0, Q4_K, Q2_K)");
  if (e_count <= 0 || h > 0x7FFFFFFF || f > 0x7FFFFFFF)
    return fail(NX_ERR_SHAPE, "no experts in block " + L);
  *E = e_count;
  *H = (int)h;
  *F = (int)f;
  *fmt = tg.type;
  *Fs = 0;
  for (int r = 0; r < 3; ++r) shared[r] = find_any(g, expert_names(layer, r, NX_EXPERT_SHARED));
  if (shared[0] || shared[1] || shared[2]) {
    if (!shared[0] || !shared[1] || !shared[2])
      return fail(NX_ERR_SHAPE, "shared expert of block " + L + " is incomplete");
    const uint64_t fs = shared[0]->dims.size() > 1 ? shared[0]->dims[1] : 0;
    for (int r = 0; r < 3; ++r) {
      const auto &t = *shared[r];
      const bool ok = t.dims.size() == 2 && t.type == tg.type &&
                      (r < 2 ? (t.dims[0] == h && t.dims[1] == fs) : (t.dims[0] == fs && t.dims[1] == h));
      if (!ok) return fail(NX_ERR_SHAPE, "shared expert shapes of block " + L + " are inconsistent");
    }
    *Fs = (int)fs;
  }
  return NX_OK;
}

}  // namespace

extern "C" {

int nx_gguf_moe_info(const nx_gguf *g, int layer, int *fmt, int *num_experts, int *hidden,
                     int *ff_dim, int *shared_ff_dim) {
  if (!g) return fail(NX_ERR_INVALID_ARG, "null GGUF handle");
  RoleTensor role[3];
  const nx_gguf::Tensor *shared[3];
  int E, H, F, Fs;
  uint32_t f;
  NX_TRY(moe_layout(g, layer, role, &E, &H, &F, &f, shared, &Fs));
  if (fmt) *fmt = (int)f;
  if (num_experts) *num_experts = E;
  if (hidden) *hidden = H;
  if (ff_dim) *ff_dim = F;
  if (shared_ff_dim) *shared_ff_dim = Fs;
  return NX_OK;
}

int nx_q4k_from_ggml(const void *src, void *dst, size_t blocks) {
  if (blocks && (!src || !dst)) return fail(NX_ERR_INVALID_ARG, "null buffer");
  q4k_ggml_to_reference((const uint8_t *)src, (uint8_t *)dst, blocks);
  return NX_OK;
}

int nx_experts_load_gguf(nx_ctx *ctx, const nx_gguf *g, int layer, int q4k_order,
                         nx_experts **out) {
  if (!ctx || !g || !out) return fail(NX_ERR_INVALID_ARG, "null argument");
  if (q4k_order != NX_Q4K_REFERENCE && q4k_order != NX_Q4K_GGML)
    return fail(NX_ERR_INVALID_ARG, "unknown Q4_K code order");
  *out = nullptr;
  RoleTensor role[3];
  const nx_gguf::Tensor *shared[3];
  int E, H, F, Fs;
  uint32_t fmt;
  NX_TRY(moe_layout(g, layer, role, &E, &H, &F, &fmt, shared, &Fs));
  nx_experts *ex = nullptr;
  NX_TRY(nx_experts_create(ctx, (int)fmt, E, H, F, &ex));
  auto give_up = [&](int rc) {
    nx_experts_destroy(ex);
    return rc;
  };
  if (Fs) {
    const int rc = nx_experts_add_shared(ctx, ex, Fs);
    if (rc) return give_up(rc);
  }
  std::vector<uint8_t> conv;
  auto load = [&](int expert, int r, const uint8_t *p, uint64_t bytes) -> int {
    if (fmt == NX_FMT_Q4_K && q4k_order == NX_Q4K_GGML) {
      conv.resize(bytes);
      q4k_ggml_to_reference(p, conv.data(), bytes / 144);
      p = conv.data();
    }
    return nx_experts_load(ctx, ex, expert, r, p, bytes, 0);
  };
  for (int r = 0; r < 3; ++r) {
    const int rows = r < 2 ? F : H, cols = r < 2 ? H : F;
    const int64_t per_expert = type_bytes(fmt, (uint64_t)rows * (uint64_t)cols);
    if (role[r].merged) {
      const uint8_t *p;
      uint64_t bytes;
      int rc = tensor_payload(g, *role[r].t, &p, &bytes);
      if (rc) return give_up(rc);
      for (int e = 0; e < E && !rc; ++e) rc = load(e, r, p + (uint64_t)e * per_expert, per_expert);
      if (rc) return give_up(rc);
    } else {
      for (int e = 0; e < E; ++e) {
        const auto *t = find_any(g, expert_names(layer, r, e));
        if (t->dims.size() != 2 || t->dims[0] != (uint64_t)cols || t->dims[1] != (uint64_t)rows ||
            t->type != fmt)
          return give_up(fail(NX_ERR_SHAPE, "expert tensor " + t->name + " has another shape"));
        const uint8_t *p;
        uint64_t bytes;
        int rc = tensor_payload(g, *t, &p, &bytes);
        if (!rc) rc = load(e, r, p, bytes);
        if (rc) return give_up(rc);
      }
    }
    if (Fs) {
      const uint8_t *p;
      uint64_t bytes;
      int rc = tensor_payload(g, *shared[r], &p, &bytes);
      if (!rc) rc = load(NX_EXPERT_SHARED, r, p, bytes);
      if (rc) return give_up(rc);
    }
  }
  *out = ex;
  return NX_OK;
}

int nx_matrix_load_gguf(nx_ctx *ctx, const nx_gguf *g, const char *name, int q4k_order,
                        nx_matrix **out) {
  if (!ctx || !g || !name || !out) return fail(NX_ERR_INVALID_ARG, "null argument");
  if (q4k_order != NX_Q4K_REFERENCE && q4k_order != NX_Q4K_GGML)
    return fail(NX_ERR_INVALID_ARG, "unknown Q4_K code order");
  *out = nullptr;
  const nx_gguf::Tensor *t = find(g, name);
  if (!t) return fail(NX_ERR_NOT_FOUND, std::string("Missing tensor: ") + name);
  if (!supported_fmt(t->type))
    return fail(NX_ERR_UNSUPPORTED, "tensor type " + std::to_string(t->type) +
                                        " is not resident-capable (F32, F16, BF16, Q4_0, Q8_0, Q4_K, Q2_K)");
  // dims innermost first: a row is dims[0] long, the rest count rows
  if (t->dims.empty()) return fail(NX_ERR_SHAPE, "tensor " + t->name + " has no dimensions");
  uint64_t rows = 1;
  for (size_t i = 1; i < t->dims.size(); ++i) rows *= t->dims[i];
  const uint64_t cols = t->dims[0];
  if (rows == 0 || cols == 0 || rows > 0x7FFFFFFF || cols > 0x7FFFFFFF)
    return fail(NX_ERR_SHAPE, "tensor " + t->name + " is not a usable matrix");
  const uint8_t *p;
  uint64_t bytes;
  NX_TRY(tensor_payload(g, *t, &p, &bytes));
  nx_matrix *m = nullptr;
  NX_TRY(nx_matrix_create(ctx, (int)t->type, (int)rows, (int)cols, &m));
  std::vector<uint8_t> conv;
  if (t->type == NX_FMT_Q4_K && q4k_order == NX_Q4K_GGML) {
    conv.resize(bytes);
    q4k_ggml_to_reference(p, conv.data(), bytes / 144);
    p = conv.data();
  }
  const int rc = nx_matrix_load(ctx, m, p, bytes, 0);
  if (rc) {
    nx_matrix_destroy(m);
    return rc;
  }
  *out = m;
  return NX_OK;
}

}  // extern "C"
