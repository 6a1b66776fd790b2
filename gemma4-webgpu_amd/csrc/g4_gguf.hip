// g4_gguf.hip — native GGUF v2/v3 reader (host code) and raw tensor upload.
//
// The reference parses the whole file in JavaScript (src/gguf.ts:75-101:
// magic, version, tensor and key/value counts, typed key/value metadata,
// tensor infos, data section aligned to 32) and dequantizes every tensor to
// f16 before upload (src/engine.ts:570-593). This reader memory-maps the file,
// parses only the header (every read bounds-checked against the mapping),
// and uploads a tensor's GGUF bytes unchanged, which is the weight format the
// matvecs take; float tensors (norm weights, rope_freqs) can be uploaded as
// f16 instead, rounded to nearest even.
#include "g4_internal.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" little-endian
enum : uint32_t {
  T_U8 = 0, T_I8 = 1, T_U16 = 2, T_I16 = 3, T_U32 = 4, T_I32 = 5, T_F32 = 6, T_BOOL = 7,
  T_STR = 8, T_ARR = 9, T_U64 = 10, T_I64 = 11, T_F64 = 12
};

uint32_t scalar_size(uint32_t t) {
  switch (t) {
    case T_U8: case T_I8: case T_BOOL: return 1;
    case T_U16: case T_I16: return 2;
    case T_U32: case T_I32: case T_F32: return 4;
    case T_U64: case T_I64: case T_F64: return 8;
    default: return 0;
  }
}

// Bytes of a tensor of `n` elements (src/gguf.ts:385-395) in *bytes; 0 for
// a type the reference does not load. False when the size does not fit 64
// bits (a file whose dims describe more bytes than any file holds).
bool type_bytes(uint32_t type, uint64_t n, uint64_t* bytes) {
  uint64_t per = 0;  // bytes per element of the unblocked types
  switch (type) {
    case 0: per = 4; break;   // F32
    case 1: per = 2; break;   // F16
    case 30: per = 2; break;  // BF16
    // block types: n / block x block bytes stays below n
    case 8: *bytes = n % 32 ? 0 : n / 32 * 34; return true;      // Q8_0
    case 12: *bytes = n % 256 ? 0 : n / 256 * 144; return true;  // Q4_K
    case 13: *bytes = n % 256 ? 0 : n / 256 * 176; return true;  // Q5_K
    case 14: *bytes = n % 256 ? 0 : n / 256 * 210; return true;  // Q6_K
    default: *bytes = 0; return true;
  }
  if (n > UINT64_MAX / per) return false;
  *bytes = n * per;
  return true;
}

struct Kv {
  std::string key;
  uint32_t type = 0, arr_type = 0;
  uint64_t count = 1;                 // elements (1 for a scalar)
  size_t off = 0;                     // file offset of the value (of an array's first element)
  std::vector<size_t> str_off;        // string arrays: offset of each element's length field
};

struct Tensor {
  std::string name;
  uint32_t n_dims = 0, type = 0;
  uint64_t dims[4] = {1, 1, 1, 1};
  uint64_t offset = 0, nbytes = 0;
};

struct Reader {
  const uint8_t* p;
  size_t size, pos = 0;
  bool ok = true;
  const char* err = nullptr;
  bool need(size_t n) {
    if (!ok) return false;
    if (n > size - pos) {
      ok = false;
      err = "truncated";
      return false;
    }
    return true;
  }
  template <class T>
  T get() {
    T v{};
    if (need(sizeof(T))) {
      std::memcpy(&v, p + pos, sizeof(T));
      pos += sizeof(T);
    }
    return v;
  }
  bool skip(size_t n) {
    if (!need(n)) return false;
    pos += n;
    return true;
  }
  std::string str() {
    const uint64_t n = get<uint64_t>();
    if (!ok || n > size - pos) {
      ok = false;
      err = "truncated string";
      return {};
    }
    std::string s((const char*)p + pos, (size_t)n);
    pos += (size_t)n;
    return s;
  }
};

// f32 -> f16 bits, round to nearest even (overflow to inf, NaN kept quiet).
uint16_t f16_rne(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // rounds to >= 65520: inf
  if (ax < 0x38800000u) {                                     // below 2^-14: f16 subnormal or zero
    if (ax < 0x33000000u) return (uint16_t)sign;               // below 2^-25 (half the least subnormal)
    const uint32_t e = ax >> 23, m = (ax & 0x7fffffu) | 0x800000u;
    const uint32_t sh = 126u - e;  // 14..24: m >> sh is the subnormal mantissa
    uint32_t h = m >> sh;
    const uint32_t rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1u);
    if (rem > half || (rem == half && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
  }
  uint32_t h = ((ax >> 13) - (112u << 10));  // rebias exponent 127 -> 15
  const uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;  // may carry into the exponent: still exact
  return (uint16_t)(sign | h);
}

// Skips one value of type t (recording string-array element offsets in kv).
bool skip_value(Reader& r, uint32_t t, Kv* kv, int depth) {
  if (t == T_STR) {
    const uint64_t n = r.get<uint64_t>();
    return r.ok && r.skip((size_t)std::min<uint64_t>(n, r.size));
  }
  if (t == T_ARR) {
    if (depth >= 8) return r.ok = false, r.err = "arrays nested deeper than 8", false;
    if (depth > 0) {  // nested arrays: allowed by the format, not used by the reference's keys
      const uint32_t et = r.get<uint32_t>();
      const uint64_t n = r.get<uint64_t>();
      for (uint64_t i = 0; r.ok && i < n; ++i) skip_value(r, et, nullptr, depth + 1);
      return r.ok;
    }
    kv->arr_type = r.get<uint32_t>();
    kv->count = r.get<uint64_t>();
    kv->off = r.pos;
    if (!r.ok) return false;
    if (kv->arr_type == T_STR) {
      if (kv->count > (r.size - r.pos) / 8) return r.ok = false, r.err = "array count past the file", false;
      kv->str_off.reserve((size_t)kv->count);
      for (uint64_t i = 0; r.ok && i < kv->count; ++i) {
        kv->str_off.push_back(r.pos);
        skip_value(r, T_STR, nullptr, depth + 1);
      }
      return r.ok;
    }
    if (kv->arr_type == T_ARR) {
      for (uint64_t i = 0; r.ok && i < kv->count; ++i) skip_value(r, T_ARR, nullptr, depth + 1);
      return r.ok;
    }
    const uint32_t es = scalar_size(kv->arr_type);
    if (!es) return r.ok = false, r.err = "unknown array element type", false;
    if (kv->count > (r.size - r.pos) / es) return r.ok = false, r.err = "truncated array", false;
    return r.skip((size_t)(kv->count * es));
  }
  const uint32_t s = scalar_size(t);
  if (!s) return r.ok = false, r.err = "unknown value type", false;
  return r.skip(s);
}

}  // namespace

struct g4_gguf {
  const uint8_t* base = nullptr;
  size_t size = 0;
  int fd = -1;
  bool mapped = false;
  uint32_t version = 0, alignment = 32;
  uint64_t data_offset = 0;
  std::vector<Kv> kvs;
  std::vector<Tensor> tensors;
  std::unordered_map<std::string, uint64_t> kv_index, tensor_index;
};

namespace {

int parse(g4_gguf* g) {
  Reader r{g->base, g->size};
  const uint32_t magic = r.get<uint32_t>();
  G4_REQUIRE(r.ok && magic == kMagic, "g4_gguf: not a GGUF file (magic 0x%08x)", magic);
  g->version = r.get<uint32_t>();
  G4_REQUIRE(r.ok && (g->version == 2 || g->version == 3), "g4_gguf: version %u not supported (2 or 3)",
             g->version);
  const uint64_t nt = r.get<uint64_t>(), nkv = r.get<uint64_t>();
  G4_REQUIRE(r.ok && nt <= g->size / 24 && nkv <= g->size / 12, "g4_gguf: tensor/key counts past the file");
  g->kvs.resize((size_t)nkv);
  for (uint64_t i = 0; i < nkv; ++i) {
    Kv& kv = g->kvs[(size_t)i];
    kv.key = r.str();
    kv.type = r.get<uint32_t>();
    kv.off = r.pos;
    skip_value(r, kv.type, &kv, 0);
    G4_REQUIRE(r.ok, "g4_gguf: key/value %llu (%s): %s", (unsigned long long)i, kv.key.c_str(),
               r.err ? r.err : "truncated");
    g->kv_index[kv.key] = i;
  }
  auto ai = g->kv_index.find("general.alignment");
  if (ai != g->kv_index.end() && g->kvs[(size_t)ai->second].type == T_U32) {
    uint32_t a = 0;
    std::memcpy(&a, g->base + g->kvs[(size_t)ai->second].off, 4);
    G4_REQUIRE(a > 0 && (a & (a - 1)) == 0, "g4_gguf: general.alignment %u is not a power of two", a);
    g->alignment = a;
  }
  g->tensors.resize((size_t)nt);
  for (uint64_t i = 0; i < nt; ++i) {
    Tensor& t = g->tensors[(size_t)i];
    t.name = r.str();
    t.n_dims = r.get<uint32_t>();
    G4_REQUIRE(r.ok && t.n_dims >= 1 && t.n_dims <= 4, "g4_gguf: tensor %llu: %u dims (1..4)",
               (unsigned long long)i, t.n_dims);
    uint64_t n = 1;
    for (uint32_t d = 0; d < t.n_dims; ++d) {
      t.dims[d] = r.get<uint64_t>();
      G4_REQUIRE(r.ok && t.dims[d] > 0 && n <= UINT64_MAX / t.dims[d], "g4_gguf: tensor %s: bad dims",
                 t.name.c_str());
      n *= t.dims[d];
    }
    t.type = r.get<uint32_t>();
    t.offset = r.get<uint64_t>();
    G4_REQUIRE(r.ok, "g4_gguf: tensor info %llu truncated", (unsigned long long)i);
    G4_REQUIRE(type_bytes(t.type, n, &t.nbytes), "g4_gguf: tensor %s: %llu elements of type %u overflow 64-bit bytes",
               t.name.c_str(), (unsigned long long)n, t.type);
    g->tensor_index[t.name] = i;
  }
  g->data_offset = (r.pos + g->alignment - 1) / g->alignment * g->alignment;
  for (const Tensor& t : g->tensors) {
    G4_REQUIRE(t.offset % g->alignment == 0, "g4_gguf: tensor %s at offset %llu is not %u-aligned", t.name.c_str(),
               (unsigned long long)t.offset, g->alignment);
    G4_REQUIRE(!t.nbytes || (g->data_offset <= g->size && t.offset <= g->size - g->data_offset &&
                             t.nbytes <= g->size - g->data_offset - t.offset),
               "g4_gguf: tensor %s data past the end of the file", t.name.c_str());
  }
  return G4_OK;
}

int check_kv(const g4_gguf* g, uint64_t index, const char* fn) {
  G4_REQUIRE(g, "%s: null handle", fn);
  G4_REQUIRE(index < g->kvs.size(), "%s: key index %llu >= %zu", fn, (unsigned long long)index, g->kvs.size());
  return G4_OK;
}

}  // namespace

extern "C" {

int g4_gguf_open_memory(const void* data, size_t bytes, g4_gguf** out) {
  G4_REQUIRE(data && out, "g4_gguf_open_memory: null argument");
  auto* g = new g4_gguf();
  g->base = (const uint8_t*)data;
  g->size = bytes;
  const int rc = parse(g);
  if (rc) {
    delete g;
    return rc;
  }
  *out = g;
  return G4_OK;
}

int g4_gguf_open(const char* path, g4_gguf** out) {
  G4_REQUIRE(path && out, "g4_gguf_open: null argument");
  const int fd = ::open(path, O_RDONLY);
  G4_REQUIRE(fd >= 0, "g4_gguf_open: cannot open %s", path);
  struct stat st {};
  if (fstat(fd, &st) != 0 || st.st_size <= 0) {
    ::close(fd);
    return g4::set_error(G4_ERR_INVALID, "g4_gguf_open: %s is empty or unreadable", path);
  }
  void* m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
  if (m == MAP_FAILED) {
    ::close(fd);
    return g4::set_error(G4_ERR_INVALID, "g4_gguf_open: cannot map %s", path);
  }
  auto* g = new g4_gguf();
  g->base = (const uint8_t*)m;
  g->size = (size_t)st.st_size;
  g->fd = fd;
  g->mapped = true;
  const int rc = parse(g);
  if (rc) {
    g4_gguf_close(g);
    return rc;
  }
  *out = g;
  return G4_OK;
}

int g4_gguf_close(g4_gguf* g) {
  if (!g) return G4_OK;
  if (g->mapped) munmap((void*)g->base, g->size);
  if (g->fd >= 0) ::close(g->fd);
  delete g;
  return G4_OK;
}

int g4_gguf_info(const g4_gguf* g, uint32_t* version, uint64_t* tensor_count, uint64_t* kv_count,
                 uint64_t* data_offset, uint32_t* alignment) {
  G4_REQUIRE(g, "g4_gguf_info: null handle");
  if (version) *version = g->version;
  if (tensor_count) *tensor_count = g->tensors.size();
  if (kv_count) *kv_count = g->kvs.size();
  if (data_offset) *data_offset = g->data_offset;
  if (alignment) *alignment = g->alignment;
  return G4_OK;
}

int g4_gguf_find_key(const g4_gguf* g, const char* key, int64_t* index) {
  G4_REQUIRE(g && key && index, "g4_gguf_find_key: null argument");
  auto it = g->kv_index.find(key);
  *index = it == g->kv_index.end() ? -1 : (int64_t)it->second;
  return G4_OK;
}

int g4_gguf_kv(const g4_gguf* g, uint64_t index, const char** key, uint32_t* type, uint32_t* arr_type,
               uint64_t* count) {
  int rc = check_kv(g, index, __func__);
  if (rc) return rc;
  const Kv& kv = g->kvs[(size_t)index];
  if (key) *key = kv.key.c_str();
  if (type) *type = kv.type;
  if (arr_type) *arr_type = kv.type == T_ARR ? kv.arr_type : 0u;
  if (count) *count = kv.type == T_ARR ? kv.count : 1u;
  return G4_OK;
}

int g4_gguf_kv_number(const g4_gguf* g, uint64_t index, uint64_t element, double* f, int64_t* i, uint64_t* u) {
  int rc = check_kv(g, index, __func__);
  if (rc) return rc;
  const Kv& kv = g->kvs[(size_t)index];
  const uint32_t t = kv.type == T_ARR ? kv.arr_type : kv.type;
  const uint64_t count = kv.type == T_ARR ? kv.count : 1u;
  const uint32_t es = scalar_size(t);
  G4_REQUIRE(es, "g4_gguf_kv_number: %s is not numeric", kv.key.c_str());
  G4_REQUIRE(element < count, "g4_gguf_kv_number: %s element %llu >= %llu", kv.key.c_str(),
             (unsigned long long)element, (unsigned long long)count);
  const uint8_t* p = g->base + kv.off + (size_t)element * es;
  double fv = 0;
  int64_t iv = 0;
  uint64_t uv = 0;
  switch (t) {
    case T_U8: case T_BOOL: uv = p[0]; iv = (int64_t)uv; fv = (double)uv; break;
    case T_I8: { int8_t v; std::memcpy(&v, p, 1); iv = v; uv = (uint64_t)v; fv = v; break; }
    case T_U16: { uint16_t v; std::memcpy(&v, p, 2); uv = v; iv = v; fv = v; break; }
    case T_I16: { int16_t v; std::memcpy(&v, p, 2); iv = v; uv = (uint64_t)v; fv = v; break; }
    case T_U32: { uint32_t v; std::memcpy(&v, p, 4); uv = v; iv = v; fv = v; break; }
    case T_I32: { int32_t v; std::memcpy(&v, p, 4); iv = v; uv = (uint64_t)v; fv = v; break; }
    case T_F32: { float v; std::memcpy(&v, p, 4); fv = v; iv = (int64_t)v; uv = (uint64_t)iv; break; }
    case T_U64: { uint64_t v; std::memcpy(&v, p, 8); uv = v; iv = (int64_t)v; fv = (double)v; break; }
    case T_I64: { int64_t v; std::memcpy(&v, p, 8); iv = v; uv = (uint64_t)v; fv = (double)v; break; }
    case T_F64: { double v; std::memcpy(&v, p, 8); fv = v; iv = (int64_t)v; uv = (uint64_t)iv; break; }
    default: break;
  }
  if (f) *f = fv;
  if (i) *i = iv;
  if (u) *u = uv;
  return G4_OK;
}

int g4_gguf_kv_string(const g4_gguf* g, uint64_t index, uint64_t element, const char** s, uint64_t* len) {
  int rc = check_kv(g, index, __func__);
  if (rc) return rc;
  const Kv& kv = g->kvs[(size_t)index];
  size_t off;
  if (kv.type == T_STR) {
    G4_REQUIRE(element == 0, "g4_gguf_kv_string: %s is a single string", kv.key.c_str());
    off = kv.off;
  } else {
    G4_REQUIRE(kv.type == T_ARR && kv.arr_type == T_STR, "g4_gguf_kv_string: %s is not a string",
               kv.key.c_str());
    G4_REQUIRE(element < kv.str_off.size(), "g4_gguf_kv_string: %s element %llu >= %zu", kv.key.c_str(),
               (unsigned long long)element, kv.str_off.size());
    off = kv.str_off[(size_t)element];
  }
  uint64_t n = 0;
  std::memcpy(&n, g->base + off, 8);
  if (s) *s = (const char*)g->base + off + 8;  // not NUL-terminated: use len
  if (len) *len = n;
  return G4_OK;
}

int g4_gguf_find_tensor(const g4_gguf* g, const char* name, int64_t* index) {
  G4_REQUIRE(g && name && index, "g4_gguf_find_tensor: null argument");
  auto it = g->tensor_index.find(name);
  *index = it == g->tensor_index.end() ? -1 : (int64_t)it->second;
  return G4_OK;
}

int g4_gguf_tensor(const g4_gguf* g, uint64_t index, const char** name, uint32_t* n_dims, uint64_t* dims,
                   uint32_t* type, uint64_t* offset, uint64_t* nbytes) {
  G4_REQUIRE(g, "g4_gguf_tensor: null handle");
  G4_REQUIRE(index < g->tensors.size(), "g4_gguf_tensor: index %llu >= %zu", (unsigned long long)index,
             g->tensors.size());
  const Tensor& t = g->tensors[(size_t)index];
  if (name) *name = t.name.c_str();
  if (n_dims) *n_dims = t.n_dims;
  if (dims)
    for (int d = 0; d < 4; ++d) dims[d] = t.dims[d];
  if (type) *type = t.type;
  if (offset) *offset = t.offset;
  if (nbytes) *nbytes = t.nbytes;
  return G4_OK;
}

int g4_gguf_tensor_data(const g4_gguf* g, uint64_t index, const void** data) {
  G4_REQUIRE(g && data, "g4_gguf_tensor_data: null argument");
  G4_REQUIRE(index < g->tensors.size(), "g4_gguf_tensor_data: index %llu >= %zu", (unsigned long long)index,
             g->tensors.size());
  const Tensor& t = g->tensors[(size_t)index];
  G4_REQUIRE(t.nbytes, "g4_gguf_tensor_data: %s has type %u, whose size is not known", t.name.c_str(), t.type);
  *data = g->base + g->data_offset + t.offset;
  return G4_OK;
}

int g4_gguf_upload(g4_ctx* ctx, const g4_gguf* g, uint64_t index, void* dst, size_t dst_bytes) {
  G4_ENTER(ctx);
  const void* src = nullptr;
  int rc = g4_gguf_tensor_data(g, index, &src);
  if (rc) return rc;
  const Tensor& t = g->tensors[(size_t)index];
  G4_REQUIRE(dst && dst_bytes >= t.nbytes, "g4_gguf_upload: %s needs %llu bytes, destination has %zu",
             t.name.c_str(), (unsigned long long)t.nbytes, dst_bytes);
  return g4_upload(ctx, dst, src, (size_t)t.nbytes, 0);
}

int g4_gguf_upload_f16(g4_ctx* ctx, const g4_gguf* g, uint64_t index, uint16_t* dst, size_t dst_elems) {
  G4_ENTER(ctx);
  const void* src = nullptr;
  int rc = g4_gguf_tensor_data(g, index, &src);
  if (rc) return rc;
  const Tensor& t = g->tensors[(size_t)index];
  G4_REQUIRE(t.type == 0 || t.type == 1 || t.type == 30,
             "g4_gguf_upload_f16: %s has type %u (F32, F16 or BF16 only)", t.name.c_str(), t.type);
  const uint64_t n = t.nbytes / (t.type == 0 ? 4u : 2u);
  G4_REQUIRE(dst && dst_elems >= n, "g4_gguf_upload_f16: %s has %llu elements, destination %zu", t.name.c_str(),
             (unsigned long long)n, dst_elems);
  if (t.type == 1) return g4_upload(ctx, dst, src, (size_t)n * 2, 0);
  constexpr uint64_t kChunk = 1u << 20;
  std::vector<uint16_t> h((size_t)std::min<uint64_t>(n, kChunk));
  for (uint64_t e0 = 0; e0 < n; e0 += kChunk) {
    const uint64_t m = std::min<uint64_t>(kChunk, n - e0);
    for (uint64_t e = 0; e < m; ++e) {
      float v;
      if (t.type == 0) {
        std::memcpy(&v, (const uint8_t*)src + (e0 + e) * 4, 4);
      } else {  // BF16: the high half of an f32 (src/gguf.ts:143-150)
        uint16_t b;
        std::memcpy(&b, (const uint8_t*)src + (e0 + e) * 2, 2);
        const uint32_t u = (uint32_t)b << 16;
        std::memcpy(&v, &u, 4);
      }
      h[(size_t)e] = f16_rne(v);
    }
    rc = g4_upload(ctx, dst, h.data(), (size_t)m * 2, (size_t)e0 * 2);
    if (rc) return rc;
  }
  return G4_OK;
}

}  // extern "C"
