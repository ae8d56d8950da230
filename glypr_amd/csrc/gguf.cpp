// gguf.cpp — GGUF v3 reader (host side) and the model loader built on it.
//
// The reference reads GGUF through candle's gguf_file::Content::read
// (lib.rs:180-186, model.rs:235) and builds its config from the
// gemma-embedding2.* metadata (config.rs:79-189).  This reader follows the
// published GGUF v3 layout:
//   header   : magic "GGUF", u32 version (2 or 3), u64 tensor count,
//              u64 metadata count
//   metadata : { string key, u32 value type, value }*
//   tensors  : { string name, u32 n_dims, u64 ne[n_dims], u32 ggml type,
//                u64 offset }*
//   data     : starts at the next multiple of general.alignment (default
//              32); each tensor at data + offset.
// Strings are u64 length + bytes; arrays are u32 element type + u64 count +
// elements.  ne[0] is the innermost dimension: a [out, in] weight has
// ne = {in, out}.  The file is memory-mapped read-only; every read is bounds
// checked, so a truncated or corrupt file fails with an error, never a fault.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <map>
#include <new>
#include <string>
#include <vector>
#include <vector>

#include "host_common.hpp"
#include "internal.hpp"

namespace glypr {
namespace {

enum GgufType : uint32_t {
  T_U8 = 0, T_I8 = 1, T_U16 = 2, T_I16 = 3, T_U32 = 4, T_I32 = 5, T_F32 = 6, T_BOOL = 7,
  T_STR = 8, T_ARR = 9, T_U64 = 10, T_I64 = 11, T_F64 = 12
};

// A metadata value.  Arrays are not materialised: the parser checks their
// bounds and keeps the element type, the count and where the elements start,
// and get_array_u64 decodes one element on demand (string arrays such as the
// tokenizer's 262144 tokens cost no host memory).
struct GgufValue {
  uint32_t type = 0;
  uint64_t u = 0;   // unsigned integers and bool
  int64_t i = 0;    // signed integers
  double f = 0.0;   // floats
  std::string s;
  uint32_t arr_type = 0;
  uint64_t arr_len = 0;
  const uint8_t* arr_data = nullptr;
};

// Byte size of a fixed-size GGUF value type, 0 for strings and arrays.
size_t scalar_size(uint32_t t) {
  switch (t) {
    case T_U8: case T_I8: case T_BOOL: return 1;
    case T_U16: case T_I16: return 2;
    case T_U32: case T_I32: case T_F32: return 4;
    case T_U64: case T_I64: case T_F64: return 8;
    default: return 0;
  }
}

struct GgufTensor {
  std::string name;
  uint32_t type = 0;
  uint32_t n_dims = 0;
  int64_t ne[4] = {1, 1, 1, 1};
  uint64_t offset = 0;
  const uint8_t* data = nullptr;
  int64_t nbytes = -1;   // -1: unknown ggml type
};

// (elements per block, bytes per block) of the ggml types; {0, 0} = unknown.
void ggml_type_size(uint32_t t, int64_t* blk, int64_t* bytes) {
  static const int64_t tab[][2] = {
      {1, 4},     {1, 2},    {32, 18},  {32, 20},  {0, 0},    {0, 0},     {32, 22},
      {32, 24},   {32, 34},  {32, 36},  {256, 84}, {256, 110}, {256, 144}, {256, 176},
      {256, 210}, {256, 292}};
  *blk = 0;
  *bytes = 0;
  if (t < sizeof(tab) / sizeof(tab[0])) {
    *blk = tab[t][0];
    *bytes = tab[t][1];
  } else if (t == 24) {   // I8
    *blk = 1; *bytes = 1;
  } else if (t == 25 || t == 30) {   // I16, BF16
    *blk = 1; *bytes = 2;
  } else if (t == 26) {   // I32
    *blk = 1; *bytes = 4;
  } else if (t == 27 || t == 28) {   // I64, F64
    *blk = 1; *bytes = 8;
  }
}

// IEEE binary16 -> binary32, exact (normals, subnormals, infinities, NaNs).
float half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000) << 16;
  uint32_t exp = (h >> 10) & 0x1F, man = h & 0x3FF, bits;
  if (exp == 0x1F) {
    bits = sign | 0x7F800000u | (man << 13);
  } else if (exp != 0) {
    bits = sign | ((exp + 112) << 23) | (man << 13);
  } else if (man == 0) {
    bits = sign;
  } else {   // subnormal: normalise
    int e = 113;
    while ((man & 0x400) == 0) {
      man <<= 1;
      e--;
    }
    bits = sign | ((uint32_t)e << 23) | ((man & 0x3FF) << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

// binary32 -> bfloat16, round to nearest even; NaNs stay (quiet) NaNs.
uint16_t float_to_bf16_rne(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

struct Cursor {
  const uint8_t* p;
  const uint8_t* end;
  bool ok = true;
  bool take(void* dst, size_t n) {
    if (!ok || (size_t)(end - p) < n) return ok = false;
    memcpy(dst, p, n);
    p += n;
    return true;
  }
  template <class T>
  T get() {
    T v{};
    take(&v, sizeof(T));
    return v;
  }
  std::string str() {
    const uint64_t n = get<uint64_t>();
    if (!ok || n > (uint64_t)(end - p)) {
      ok = false;
      return std::string();
    }
    std::string s((const char*)p, (size_t)n);
    p += n;
    return s;
  }
};

bool read_value(Cursor& c, uint32_t type, GgufValue& v, int depth) {
  v.type = type;
  switch (type) {
    case T_U8: v.u = c.get<uint8_t>(); break;
    case T_I8: v.i = c.get<int8_t>(); break;
    case T_U16: v.u = c.get<uint16_t>(); break;
    case T_I16: v.i = c.get<int16_t>(); break;
    case T_U32: v.u = c.get<uint32_t>(); break;
    case T_I32: v.i = c.get<int32_t>(); break;
    case T_F32: v.f = c.get<float>(); break;
    case T_BOOL: v.u = c.get<uint8_t>() != 0; break;
    case T_STR: v.s = c.str(); break;
    case T_U64: v.u = c.get<uint64_t>(); break;
    case T_I64: v.i = c.get<int64_t>(); break;
    case T_F64: v.f = c.get<double>(); break;
    case T_ARR: {
      if (depth > 0) return false;   // nested arrays do not occur in GGUF files
      v.arr_type = c.get<uint32_t>();
      const uint64_t n = c.get<uint64_t>();
      if (!c.ok) return false;
      const size_t remaining = (size_t)(c.end - c.p);
      v.arr_len = n;
      v.arr_data = c.p;
      const size_t es = scalar_size(v.arr_type);
      if (es > 0) {
        if (n > remaining / es) return false;
        c.p += n * es;
      } else if (v.arr_type == T_STR) {
        if (n > remaining / 8) return false;   // each string takes >= 8 bytes
        for (uint64_t k = 0; k < n; k++) {
          const uint64_t len = c.get<uint64_t>();
          if (!c.ok || len > (uint64_t)(c.end - c.p)) return false;
          c.p += len;
        }
      } else {
        return false;
      }
      break;
    }
    default:
      return false;
  }
  return c.ok;
}

bool as_u64(const GgufValue& v, uint64_t* out) {
  switch (v.type) {
    case T_U8: case T_U16: case T_U32: case T_U64: case T_BOOL: *out = v.u; return true;
    case T_I8: case T_I16: case T_I32: case T_I64:
      if (v.i < 0) return false;
      *out = (uint64_t)v.i;
      return true;
    default: return false;
  }
}

bool as_f64(const GgufValue& v, double* out) {
  uint64_t u;
  if (v.type == T_F32 || v.type == T_F64) { *out = v.f; return true; }
  if (v.type == T_I8 || v.type == T_I16 || v.type == T_I32 || v.type == T_I64) {
    *out = (double)v.i;
    return true;
  }
  if (as_u64(v, &u)) { *out = (double)u; return true; }
  return false;
}

// Element i of a fixed-size-typed array (bounds already checked by the parser).
bool array_elem(const GgufValue& a, uint64_t i, GgufValue* out) {
  const size_t es = scalar_size(a.arr_type);
  if (es == 0 || i >= a.arr_len) return false;
  Cursor c{a.arr_data + i * es, a.arr_data + (i + 1) * es};
  return read_value(c, a.arr_type, *out, 1);
}

}  // namespace
}  // namespace glypr

struct glypr_gguf {
  void* map = nullptr;
  size_t size = 0;
  uint32_t version = 0;
  uint32_t alignment = 32;
  std::map<std::string, glypr::GgufValue> kv;
  std::vector<glypr::GgufTensor> tensors;
  std::map<std::string, size_t> by_name;
};

using namespace glypr;

namespace {

int parse(glypr_gguf* g) {
  Cursor c{(const uint8_t*)g->map, (const uint8_t*)g->map + g->size};
  const uint32_t magic = c.get<uint32_t>();
  GLYPR_CHECK(c.ok && magic == 0x46554747u, GLYPR_ERR_SHAPE, "not a GGUF file (bad magic)");
  g->version = c.get<uint32_t>();
  GLYPR_CHECK(c.ok && (g->version == 2 || g->version == 3), GLYPR_ERR_UNSUPPORTED,
              "GGUF version %u (2 and 3 are supported)", g->version);
  const uint64_t n_tensors = c.get<uint64_t>();
  const uint64_t n_kv = c.get<uint64_t>();
  GLYPR_CHECK(c.ok && n_tensors < (1u << 24) && n_kv < (1u << 24), GLYPR_ERR_SHAPE,
              "GGUF header counts are corrupt");
  for (uint64_t k = 0; k < n_kv; k++) {
    std::string key = c.str();
    const uint32_t type = c.get<uint32_t>();
    GgufValue v;
    GLYPR_CHECK(c.ok && read_value(c, type, v, 0), GLYPR_ERR_SHAPE,
                "GGUF metadata entry %llu is truncated or has an unknown type",
                (unsigned long long)k);
    g->kv[key] = std::move(v);
  }
  auto al = g->kv.find("general.alignment");
  if (al != g->kv.end()) {
    uint64_t a = 0;
    GLYPR_CHECK(as_u64(al->second, &a) && a > 0 && (a & (a - 1)) == 0 && a <= 4096,
                GLYPR_ERR_SHAPE, "general.alignment must be a power of two <= 4096");
    g->alignment = (uint32_t)a;
  }
  g->tensors.resize((size_t)n_tensors);
  for (uint64_t k = 0; k < n_tensors; k++) {
    GgufTensor& t = g->tensors[(size_t)k];
    t.name = c.str();
    t.n_dims = c.get<uint32_t>();
    GLYPR_CHECK(c.ok && t.n_dims >= 1 && t.n_dims <= 4, GLYPR_ERR_SHAPE,
                "tensor %llu: bad dimension count", (unsigned long long)k);
    for (uint32_t d = 0; d < t.n_dims; d++) {
      const uint64_t ne = c.get<uint64_t>();
      GLYPR_CHECK(c.ok && ne >= 1 && ne < (1ull << 40), GLYPR_ERR_SHAPE,
                  "tensor '%s': bad dimension", t.name.c_str());
      t.ne[d] = (int64_t)ne;
    }
    t.type = c.get<uint32_t>();
    t.offset = c.get<uint64_t>();
    GLYPR_CHECK(c.ok, GLYPR_ERR_SHAPE, "tensor table is truncated");
    GLYPR_CHECK(t.offset % g->alignment == 0, GLYPR_ERR_SHAPE,
                "tensor '%s': offset %llu is not aligned to %u", t.name.c_str(),
                (unsigned long long)t.offset, g->alignment);
    GLYPR_CHECK(g->by_name.count(t.name) == 0, GLYPR_ERR_SHAPE, "tensor '%s' appears twice",
                t.name.c_str());
    g->by_name[t.name] = (size_t)k;
  }
  const size_t header = (size_t)(c.p - (const uint8_t*)g->map);
  const size_t data0 = (header + g->alignment - 1) / g->alignment * g->alignment;
  for (GgufTensor& t : g->tensors) {
    int64_t blk, bytes;
    ggml_type_size(t.type, &blk, &bytes);
    int64_t n = 1;
    bool ovf = false;
    for (int d = 0; d < 4; d++) ovf = ovf || __builtin_mul_overflow(n, t.ne[d], &n);
    GLYPR_CHECK(!ovf, GLYPR_ERR_SHAPE, "tensor '%s': element count overflows", t.name.c_str());
    if (blk > 0) {
      GLYPR_CHECK(t.ne[0] % blk == 0, GLYPR_ERR_SHAPE,
                  "tensor '%s': ne[0] = %lld is not a multiple of the type's block %lld",
                  t.name.c_str(), (long long)t.ne[0], (long long)blk);
      GLYPR_CHECK(!__builtin_mul_overflow(n / blk, bytes, &t.nbytes), GLYPR_ERR_SHAPE,
                  "tensor '%s': byte count overflows", t.name.c_str());
      GLYPR_CHECK(data0 <= g->size && t.offset <= g->size - data0 &&
                      (uint64_t)t.nbytes <= g->size - data0 - t.offset,
                  GLYPR_ERR_SHAPE, "tensor '%s' runs past the end of the file",
                  t.name.c_str());
      t.data = (const uint8_t*)g->map + data0 + t.offset;
    }
  }
  return GLYPR_OK;
}

const GgufValue* find_kv(const glypr_gguf* g, const char* key) {
  if (!g || !key) return nullptr;
  auto it = g->kv.find(key);
  return it == g->kv.end() ? nullptr : &it->second;
}

}  // namespace

extern "C" {

static int gguf_open_impl(const char* path, glypr_gguf** out);
static int model_load_gguf_impl(glypr_hip_ctx* ctx, const char* path, glypr_model** out);

// std::bad_alloc (metadata strings, maps) and any other exception end as a
// status here: none may cross the C ABI.
int glypr_gguf_open(const char* path, glypr_gguf** out) {
  clear_error();
  try {
    return gguf_open_impl(path, out);
  } catch (const std::bad_alloc&) {
    return set_error(GLYPR_ERR_OOM, "host allocation failed while parsing the GGUF file");
  } catch (...) {
    return set_error(GLYPR_ERR_SHAPE, "GGUF parse failed");
  }
}

int glypr_hip_model_load_gguf(glypr_hip_ctx* ctx, const char* path, glypr_model** out) {
  clear_error();
  try {
    return model_load_gguf_impl(ctx, path, out);
  } catch (const std::bad_alloc&) {
    return set_error(GLYPR_ERR_OOM, "host allocation failed while loading the model");
  } catch (...) {
    return set_error(GLYPR_ERR_SHAPE, "model load failed");
  }
}

}  // extern "C"

static int gguf_open_impl(const char* path, glypr_gguf** out) {
  GLYPR_CHECK(path != nullptr && out != nullptr, GLYPR_ERR_INVALID_ARG, "path or out is NULL");
  *out = nullptr;
  const int fd = open(path, O_RDONLY);
  GLYPR_CHECK(fd >= 0, GLYPR_ERR_INVALID_ARG, "cannot open '%s'", path);
  struct stat st;
  if (fstat(fd, &st) != 0 || st.st_size < 24) {
    close(fd);
    return set_error(GLYPR_ERR_SHAPE, "'%s' is too short for a GGUF header", path);
  }
  void* map = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  GLYPR_CHECK(map != MAP_FAILED, GLYPR_ERR_INVALID_ARG, "cannot map '%s'", path);
  glypr_gguf* g = new (std::nothrow) glypr_gguf();
  if (!g) {
    munmap(map, (size_t)st.st_size);
    return set_error(GLYPR_ERR_OOM, "host allocation failed");
  }
  g->map = map;
  g->size = (size_t)st.st_size;
  int rc;
  try {
    rc = parse(g);
  } catch (...) {
    munmap(g->map, g->size);
    delete g;
    throw;
  }
  if (rc != GLYPR_OK) {
    munmap(g->map, g->size);
    delete g;
    return rc;
  }
  *out = g;
  return GLYPR_OK;
}

extern "C" {

int glypr_gguf_close(glypr_gguf* g) {
  clear_error();
  if (!g) return GLYPR_OK;
  munmap(g->map, g->size);
  delete g;
  return GLYPR_OK;
}

int glypr_gguf_version(const glypr_gguf* g, uint32_t* version, uint32_t* alignment) {
  clear_error();
  GLYPR_CHECK(g && version && alignment, GLYPR_ERR_INVALID_ARG, "NULL argument");
  *version = g->version;
  *alignment = g->alignment;
  return GLYPR_OK;
}

int glypr_gguf_tensor_count(const glypr_gguf* g, int64_t* n) {
  clear_error();
  GLYPR_CHECK(g && n, GLYPR_ERR_INVALID_ARG, "NULL argument");
  *n = (int64_t)g->tensors.size();
  return GLYPR_OK;
}

int glypr_gguf_tensor_info(const glypr_gguf* g, int64_t i, const char** name, int* type,
                           int* n_dims, int64_t* ne, const void** data, int64_t* nbytes) {
  clear_error();
  GLYPR_CHECK(g && name && type && n_dims && ne && data && nbytes, GLYPR_ERR_INVALID_ARG,
              "NULL argument");
  GLYPR_CHECK(i >= 0 && i < (int64_t)g->tensors.size(), GLYPR_ERR_RANGE,
              "tensor index %lld out of range", (long long)i);
  const GgufTensor& t = g->tensors[(size_t)i];
  *name = t.name.c_str();
  *type = (int)t.type;
  *n_dims = (int)t.n_dims;
  for (int d = 0; d < 4; d++) ne[d] = t.ne[d];
  *data = t.data;
  *nbytes = t.nbytes;
  return GLYPR_OK;
}

int glypr_gguf_find_tensor(const glypr_gguf* g, const char* name, int64_t* index) {
  clear_error();
  GLYPR_CHECK(g && name && index, GLYPR_ERR_INVALID_ARG, "NULL argument");
  auto it = g->by_name.find(name);
  GLYPR_CHECK(it != g->by_name.end(), GLYPR_ERR_NOT_FOUND, "no tensor '%s'", name);
  *index = (int64_t)it->second;
  return GLYPR_OK;
}

int glypr_gguf_get_u64(const glypr_gguf* g, const char* key, uint64_t* out) {
  clear_error();
  GLYPR_CHECK(g && key && out, GLYPR_ERR_INVALID_ARG, "NULL argument");
  const GgufValue* v = find_kv(g, key);
  GLYPR_CHECK(v != nullptr, GLYPR_ERR_NOT_FOUND, "no metadata key '%s'", key);
  GLYPR_CHECK(as_u64(*v, out), GLYPR_ERR_UNSUPPORTED, "'%s' is not a non-negative integer", key);
  return GLYPR_OK;
}

int glypr_gguf_get_f64(const glypr_gguf* g, const char* key, double* out) {
  clear_error();
  GLYPR_CHECK(g && key && out, GLYPR_ERR_INVALID_ARG, "NULL argument");
  const GgufValue* v = find_kv(g, key);
  GLYPR_CHECK(v != nullptr, GLYPR_ERR_NOT_FOUND, "no metadata key '%s'", key);
  GLYPR_CHECK(as_f64(*v, out), GLYPR_ERR_UNSUPPORTED, "'%s' is not a number", key);
  return GLYPR_OK;
}

int glypr_gguf_get_str(const glypr_gguf* g, const char* key, const char** out) {
  clear_error();
  GLYPR_CHECK(g && key && out, GLYPR_ERR_INVALID_ARG, "NULL argument");
  const GgufValue* v = find_kv(g, key);
  GLYPR_CHECK(v != nullptr, GLYPR_ERR_NOT_FOUND, "no metadata key '%s'", key);
  GLYPR_CHECK(v->type == T_STR, GLYPR_ERR_UNSUPPORTED, "'%s' is not a string", key);
  *out = v->s.c_str();
  return GLYPR_OK;
}

int glypr_gguf_get_array(const glypr_gguf* g, const char* key, int* elem_type, int64_t* len) {
  clear_error();
  GLYPR_CHECK(g && key && elem_type && len, GLYPR_ERR_INVALID_ARG, "NULL argument");
  const GgufValue* v = find_kv(g, key);
  GLYPR_CHECK(v != nullptr, GLYPR_ERR_NOT_FOUND, "no metadata key '%s'", key);
  GLYPR_CHECK(v->type == T_ARR, GLYPR_ERR_UNSUPPORTED, "'%s' is not an array", key);
  *elem_type = (int)v->arr_type;
  *len = (int64_t)v->arr_len;
  return GLYPR_OK;
}

int glypr_gguf_get_array_u64(const glypr_gguf* g, const char* key, int64_t i, uint64_t* out) {
  clear_error();
  GLYPR_CHECK(g && key && out, GLYPR_ERR_INVALID_ARG, "NULL argument");
  const GgufValue* v = find_kv(g, key);
  GLYPR_CHECK(v != nullptr, GLYPR_ERR_NOT_FOUND, "no metadata key '%s'", key);
  GLYPR_CHECK(v->type == T_ARR, GLYPR_ERR_UNSUPPORTED, "'%s' is not an array", key);
  GLYPR_CHECK(i >= 0 && (uint64_t)i < v->arr_len, GLYPR_ERR_RANGE,
              "index %lld out of range for '%s'", (long long)i, key);
  GgufValue e;
  GLYPR_CHECK(array_elem(*v, (uint64_t)i, &e) && as_u64(e, out), GLYPR_ERR_UNSUPPORTED,
              "'%s'[%lld] is not a non-negative integer", key, (long long)i);
  return GLYPR_OK;
}

// EmbeddingGemma2Model::from_gguf_content (model.rs:244-488) with the config of
// TextConfig::from_gguf_metadata (config.rs:79-189): per-layer head dims and kv
// heads as get_head_dim / get_num_kv_heads give them, the Per-Layer-Embedding
// block and the embedding projection when the file has their tensors.
static int model_load_gguf_impl(glypr_hip_ctx* ctx, const char* path, glypr_model** out) {
  GLYPR_CHECK(path != nullptr && out != nullptr, GLYPR_ERR_INVALID_ARG, "path or out is NULL");
  *out = nullptr;
  RET_IF(check_ctx(ctx));
  glypr_gguf* g = nullptr;
  RET_IF(glypr_gguf_open(path, &g));
  struct Closer {
    glypr_gguf* g;
    ~Closer() { glypr_gguf_close(g); }
  } closer{g};

  const char* P = "gemma-embedding2.";
  auto key = [&](const char* k) { return std::string(P) + k; };
  auto req_u = [&](const char* k, uint64_t* v) -> int {
    const int rc = glypr_gguf_get_u64(g, key(k).c_str(), v);
    if (rc == GLYPR_ERR_NOT_FOUND) return set_error(rc, "GGUF is missing %s%s", P, k);
    return rc;
  };
  auto opt_u = [&](const char* k, uint64_t dflt) -> uint64_t {
    uint64_t v;
    return glypr_gguf_get_u64(g, key(k).c_str(), &v) == GLYPR_OK ? v : dflt;
  };
  auto opt_f = [&](const char* k, double dflt) -> double {
    double v;
    return glypr_gguf_get_f64(g, key(k).c_str(), &v) == GLYPR_OK ? v : dflt;
  };
  uint64_t layers, hidden, ffn, heads;
  RET_IF(req_u("block_count", &layers));
  RET_IF(req_u("embedding_length", &hidden));
  RET_IF(req_u("feed_forward_length", &ffn));
  RET_IF(req_u("attention.head_count", &heads));
  const uint64_t head_dim = opt_u("attention.key_length_swa", 256);
  const uint64_t full_head_dim = opt_u("attention.key_length", 512);   // config.rs:149-150
  // head_count_kv (config.rs:142-168): only an array counts.  Its first entry
  // is every sliding layer's value (2 without one); a full layer i takes entry
  // i (1 without one).  A scalar is ignored, as in the reference.
  int et;
  int64_t kv_len = 0;
  const std::string kvk = key("attention.head_count_kv");
  const bool kv_arr = glypr_gguf_get_array(g, kvk.c_str(), &et, &kv_len) == GLYPR_OK;
  uint64_t kv_heads = 2;
  if (kv_arr && kv_len > 0) RET_IF(glypr_gguf_get_array_u64(g, kvk.c_str(), 0, &kv_heads));
  clear_error();

  // layer_types (config.rs:117-140): sliding_window_pattern, an array of
  // bools (true = sliding), when the file has one; else layer i is full iff
  // (i+1) % 6 == 0.  The pattern must cover every block.
  GLYPR_CHECK(layers > 0 && layers < (1u << 20), GLYPR_ERR_SHAPE, "block_count %llu",
              (unsigned long long)layers);
  std::vector<uint8_t> layer_full((size_t)layers);
  int pat_et = 0;
  int64_t pat_len = 0;
  const std::string patk = key("attention.sliding_window_pattern");
  const bool has_pat = glypr_gguf_get_array(g, patk.c_str(), &pat_et, &pat_len) == GLYPR_OK;
  clear_error();
  if (has_pat) {
    GLYPR_CHECK(pat_et == T_BOOL, GLYPR_ERR_UNSUPPORTED,
                "Invalid boolean in sliding_window_pattern (element type %d)", pat_et);
    GLYPR_CHECK(pat_len >= (int64_t)layers, GLYPR_ERR_SHAPE,
                "sliding_window_pattern has %lld entries for %llu blocks", (long long)pat_len,
                (unsigned long long)layers);
  }
  uint64_t full_kv = 0;   // the full layers' kv heads (0: no full layer)
  for (uint64_t i = 0; i < layers; i++) {
    bool full = (i + 1) % 6 == 0;
    if (has_pat) {
      uint64_t sliding = 0;
      RET_IF(glypr_gguf_get_array_u64(g, patk.c_str(), (int64_t)i, &sliding));
      full = sliding == 0;
    }
    layer_full[(size_t)i] = full ? 1 : 0;
    if (!full) continue;
    uint64_t kvi = 1;
    if (kv_arr && kv_len > (int64_t)i) RET_IF(glypr_gguf_get_array_u64(g, kvk.c_str(), (int64_t)i, &kvi));
    GLYPR_CHECK(full_kv == 0 || kvi == full_kv, GLYPR_ERR_UNSUPPORTED,
                "full-attention layers with differing kv heads (%llu and %llu) are not "
                "supported", (unsigned long long)full_kv, (unsigned long long)kvi);
    full_kv = kvi;
  }
  GLYPR_CHECK(kv_heads > 0 && kv_heads < (1u << 20) && full_kv < (1u << 20) &&
                  head_dim > 0 && head_dim < (1u << 20) && full_head_dim < (1u << 20),
              GLYPR_ERR_SHAPE, "attention geometry in the metadata is corrupt");

  int64_t ti;
  RET_IF(glypr_gguf_find_tensor(g, "token_embd.weight", &ti));
  const GgufTensor& emb = g->tensors[(size_t)ti];
  glypr_model_config cfg{};
  cfg.hidden = (int64_t)hidden;
  cfg.ffn = (int64_t)ffn;
  cfg.n_heads = (int64_t)heads;
  cfg.n_kv_heads = (int64_t)kv_heads;
  cfg.head_dim = (int64_t)head_dim;
  cfg.full_head_dim = full_kv ? (int64_t)full_head_dim : 0;
  cfg.full_n_kv_heads = (int64_t)full_kv;
  cfg.max_seq_len = 0;   // DEFAULT_MAX_SEQ_LEN
  cfg.n_layers = (int64_t)layers;
  cfg.vocab = emb.ne[1];
  cfg.sliding_window = 512;   // config.rs:191
  cfg.eps = (float)opt_f("attention.layer_norm_rms_epsilon", 1e-6);
  cfg.rope_theta_sliding = opt_f("rope.freq_base_swa", 10000.0);
  cfg.rope_theta_full = opt_f("rope.freq_base", 1000000.0);
  cfg.layer_types = layer_full.data();
  clear_error();
  // TextPLE (model.rs:257-275) and the embedding projection (model.rs:472-473)
  // when the file has them
  int64_t pi = -1, oi = -1;
  const bool has_ple = glypr_gguf_find_tensor(g, "per_layer_model_proj.weight", &pi) == GLYPR_OK;
  const bool has_out = glypr_gguf_find_tensor(g, "output.weight", &oi) == GLYPR_OK;
  clear_error();
  // hidden_size_per_layer_input, 512 without the key (config.rs:100-102)
  cfg.ple_dim = has_ple ? (int64_t)opt_u("embedding_length_per_layer_input", 512) : 0;
  clear_error();
  cfg.out_dim = has_out ? g->tensors[(size_t)oi].ne[1] : 0;

  glypr_model* m = nullptr;
  RET_IF(glypr_hip_model_create(ctx, &cfg, &m));
  struct Dropper {   // frees the model if a load step throws
    glypr_model** m;
    ~Dropper() {
      if (*m) glypr_hip_model_destroy(*m);
    }
  } dropper{&m};
  // LinearOp::from_gguf_tensor (linear.rs:36-78): a layer projection stored as
  // F32, F16 or BF16 becomes a dense Linear; here the dense bf16 arm, its rows
  // rounded to bf16 (nearest even; exact for BF16, narrower than the
  // reference's f32 Linear for F32 and F16).  Norms and scalars are F32, the
  // token table, PLE and output projections Q8_0.
  std::vector<uint16_t> bf;
  auto load = [&](const std::string& name, bool projection) -> int {
    int64_t idx;
    RET_IF(glypr_gguf_find_tensor(g, name.c_str(), &idx));
    const GgufTensor& t = g->tensors[(size_t)idx];
    GLYPR_CHECK(t.n_dims <= 2, GLYPR_ERR_SHAPE, "tensor '%s' has %u dimensions", name.c_str(),
                t.n_dims);
    if (t.type == 8 || (t.type == 0 && !projection))
      return glypr_hip_model_set_tensor(m, name.c_str(), t.data, t.ne[1], t.ne[0],
                                        t.type == 8 ? 1 : 0);
    GLYPR_CHECK(projection && (t.type == 0 || t.type == 1 || t.type == 30),
                GLYPR_ERR_UNSUPPORTED,
                "tensor '%s' has ggml type %u (Q8_0, and F32 / F16 / BF16 layer projections, "
                "are supported)", name.c_str(), t.type);
    const int64_t n = t.ne[0] * t.ne[1];
    bf.resize((size_t)n);
    for (int64_t i = 0; i < n; i++) {
      if (t.type == 30) {
        bf[(size_t)i] = reinterpret_cast<const uint16_t*>(t.data)[i];
        continue;
      }
      float f;
      if (t.type == 0) memcpy(&f, t.data + 4 * i, 4);
      else f = half_to_float(reinterpret_cast<const uint16_t*>(t.data)[i]);
      bf[(size_t)i] = float_to_bf16_rne(f);
    }
    return glypr_hip_model_set_tensor(m, name.c_str(), bf.data(), t.ne[1], t.ne[0], 2);
  };
  int rc = load("token_embd.weight", false);
  if (rc == GLYPR_OK) rc = load("output_norm.weight", false);
  static const char* kLayer[] = {"attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate",
                                 "ffn_up", "ffn_down", "attn_norm", "post_attention_norm",
                                 "ffn_norm", "post_ffw_norm", "attn_q_norm", "attn_k_norm"};
  static const char* kPle[] = {"inp_gate", "proj", "post_norm", "layer_output_scale"};
  for (uint64_t i = 0; rc == GLYPR_OK && i < layers; i++) {
    for (int j = 0; j < (int)(sizeof(kLayer) / sizeof(kLayer[0])); j++) {
      rc = load("blk." + std::to_string(i) + "." + kLayer[j] + ".weight", j < 7);
      if (rc != GLYPR_OK) break;
    }
    for (const char* nm : kPle) {
      if (rc != GLYPR_OK || !has_ple) break;
      rc = load("blk." + std::to_string(i) + "." + nm + ".weight", false);
    }
  }
  if (rc == GLYPR_OK && has_ple) rc = load("per_layer_model_proj.weight", false);
  if (rc == GLYPR_OK && has_ple) rc = load("per_layer_proj_norm.weight", false);
  if (rc == GLYPR_OK && has_out) rc = load("output.weight", false);
  if (rc == GLYPR_OK) rc = glypr_hip_model_finalize(m);
  if (rc != GLYPR_OK) {
    std::string msg = glypr_hip_last_error();
    glypr_hip_model_destroy(m);
    m = nullptr;
    return set_error(rc, "%s", msg.c_str());
  }
  *out = m;
  m = nullptr;
  return GLYPR_OK;
}

}  // extern "C"
