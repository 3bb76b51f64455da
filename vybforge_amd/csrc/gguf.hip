// GGUF reader and one-buffer packed-slab residency (host code).
//
// The GGUF container (v2 / v3, little-endian): "GGUF", u32 version, u64 n_tensors, u64 n_kv;
// n_kv metadata pairs (string key, u32 value type, value); n_tensors tensor infos (string name,
// u32 n_dims, u64 dims[n_dims], u32 ggml type, u64 offset); then the tensor data. Strings are a
// u64 byte length and the bytes. Value types: 0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32,
// 7 bool, 8 string, 9 array (u32 element type, u64 count, elements), 10 u64, 11 i64, 12 f64.
// In the GGUF specification a tensor's offset is relative to the data section, which starts at
// the end of the tensor infos rounded up to general.alignment (default 32); the reference's
// own fixture writer stores absolute file offsets instead (native/gguf/mk_fixture.vyb), so the
// raw offset field is kept and the loader takes the convention as an argument.
// Replaces the reference's Vyb readers (native/gguf/parse_gguf.vyb, read_real_meta.vyb) and
// the resident-slab upload of ridge_decode.vyb:1-3.
#include "common.h"

#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <vector>

namespace vybdq {

struct GgufValue {
  int type = -1;
  int64_t i = 0;       // integer and bool types
  double f = 0.0;      // f32 / f64
  std::string s;       // string
  int arr_type = -1;   // array element type
  int64_t arr_len = 0;
};

struct GgufTensor {
  std::string name;
  std::vector<int64_t> dims;
  int type = 0;
  uint64_t offset = 0;  // the raw offset field
};

struct GgufFile {
  std::string path;
  uint32_t version = 0;
  uint64_t file_size = 0;
  std::vector<std::pair<std::string, GgufValue>> kv;
  std::vector<GgufTensor> tensors;
  uint64_t info_end = 0, alignment = 32, data_base = 0;
};

// (weights per block, bytes per block) of a ggml type; {0, 0} when unknown
struct TypeSize { int64_t blk, bytes; };
static TypeSize ggml_type_size(int t) {
  switch (t) {
    case 0: return {1, 4};      case 1: return {1, 2};      case 2: return {32, 18};   case 3: return {32, 20};
    case 6: return {32, 22};    case 7: return {32, 24};    case 8: return {32, 34};   case 9: return {32, 36};
    case 10: return {256, 84};  case 11: return {256, 110}; case 12: return {256, 144}; case 13: return {256, 176};
    case 14: return {256, 210}; case 15: return {256, 292}; case 16: return {256, 66};  case 17: return {256, 74};
    case 18: return {256, 98};  case 19: return {256, 50};  case 20: return {32, 18};  case 21: return {256, 110};
    case 22: return {256, 82};  case 23: return {256, 136}; case 24: return {1, 1};    case 25: return {1, 2};
    case 26: return {1, 4};     case 27: return {1, 8};     case 28: return {1, 8};    case 29: return {256, 56};
    case 30: return {1, 2};
    default: return {0, 0};
  }
}

class Reader {
 public:
  Reader(FILE *f, uint64_t size) : f_(f), size_(size) {}
  bool ok() const { return ok_; }
  uint64_t pos() const { return pos_; }
  bool bytes(void *dst, uint64_t n) {
    if (!ok_ || n > size_ - pos_) return ok_ = false;
    if (n && fread(dst, 1, n, f_) != n) return ok_ = false;
    pos_ += n;
    return true;
  }
  template <typename T> T get() {
    T v{};
    bytes(&v, sizeof(T));
    return v;
  }
  std::string str() {
    const uint64_t n = get<uint64_t>();
    if (!ok_ || n > size_ - pos_) { ok_ = false; return {}; }
    std::string s(n, '\0');
    bytes(&s[0], n);
    return s;
  }
  bool skip(uint64_t n) {
    if (!ok_ || n > size_ - pos_) return ok_ = false;
    if (fseeko(f_, static_cast<off_t>(n), SEEK_CUR) != 0) return ok_ = false;
    pos_ += n;
    return true;
  }

 private:
  FILE *f_;
  uint64_t size_, pos_ = 0;
  bool ok_ = true;
};

static int scalar_bytes(int t) {
  switch (t) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: return 8;
    default: return 0;
  }
}

static bool read_scalar(Reader &r, int t, GgufValue &v) {
  switch (t) {
    case 0: v.i = r.get<uint8_t>(); break;
    case 1: v.i = r.get<int8_t>(); break;
    case 2: v.i = r.get<uint16_t>(); break;
    case 3: v.i = r.get<int16_t>(); break;
    case 4: v.i = r.get<uint32_t>(); break;
    case 5: v.i = r.get<int32_t>(); break;
    case 6: v.f = r.get<float>(); break;
    case 7: v.i = r.get<uint8_t>() != 0; break;
    case 10: v.i = static_cast<int64_t>(r.get<uint64_t>()); break;
    case 11: v.i = r.get<int64_t>(); break;
    case 12: v.f = r.get<double>(); break;
    default: return false;
  }
  return r.ok();
}

// skips one array element of type t (strings and nested arrays included)
static bool skip_value(Reader &r, int t, int depth) {
  if (t == 8) { const uint64_t n = r.get<uint64_t>(); return r.skip(n); }
  if (t == 9) {
    if (depth > 8) return false;
    const int et = static_cast<int>(r.get<uint32_t>());
    const uint64_t n = r.get<uint64_t>();
    if (!r.ok()) return false;
    const int sb = scalar_bytes(et);
    if (sb) return n <= UINT64_MAX / sb && r.skip(n * sb);
    for (uint64_t k = 0; k < n; ++k)
      if (!skip_value(r, et, depth + 1)) return false;
    return true;
  }
  const int sb = scalar_bytes(t);
  return sb && r.skip(sb);
}

static int parse(const char *path, GgufFile &g) {
  FILE *f = fopen(path, "rb");
  if (!f) return set_error(VYBDQ_ERR_ARG, std::string("gguf: cannot open ") + path);
  std::unique_ptr<FILE, int (*)(FILE *)> guard(f, fclose);
  if (fseeko(f, 0, SEEK_END) != 0) return set_error(VYBDQ_ERR_ARG, "gguf: cannot seek");
  g.file_size = static_cast<uint64_t>(ftello(f));
  fseeko(f, 0, SEEK_SET);
  g.path = path;
  Reader r(f, g.file_size);
  char magic[4];
  if (!r.bytes(magic, 4) || memcmp(magic, "GGUF", 4) != 0) return set_error(VYBDQ_ERR_ARG, "gguf: bad magic");
  g.version = r.get<uint32_t>();
  if (g.version < 2 || g.version > 3) return set_error(VYBDQ_ERR_ARG, "gguf: unsupported version");
  const uint64_t nt = r.get<uint64_t>(), nkv = r.get<uint64_t>();
  // every metadata pair takes at least 13 bytes (key length, type, one value byte) and every tensor
  // info 24 (name length, n_dims, type, offset): counts beyond what the file can hold are corrupt
  const uint64_t rest = g.file_size - r.pos();
  if (!r.ok() || nkv > rest / 13 || nt > rest / 24) return set_error(VYBDQ_ERR_ARG, "gguf: bad counts");
  for (uint64_t k = 0; k < nkv; ++k) {
    std::string key = r.str();
    GgufValue v;
    v.type = static_cast<int>(r.get<uint32_t>());
    if (!r.ok()) return set_error(VYBDQ_ERR_ARG, "gguf: truncated metadata");
    if (v.type == 8) {
      v.s = r.str();
    } else if (v.type == 9) {
      v.arr_type = static_cast<int>(r.get<uint32_t>());
      v.arr_len = static_cast<int64_t>(r.get<uint64_t>());
      if (!r.ok() || v.arr_len < 0) return set_error(VYBDQ_ERR_ARG, "gguf: bad array");
      const int sb = scalar_bytes(v.arr_type);
      if (sb) {
        if (static_cast<uint64_t>(v.arr_len) > UINT64_MAX / sb || !r.skip(static_cast<uint64_t>(v.arr_len) * sb))
          return set_error(VYBDQ_ERR_ARG, "gguf: truncated array");
      } else {
        for (int64_t e = 0; e < v.arr_len; ++e)
          if (!skip_value(r, v.arr_type, 1)) return set_error(VYBDQ_ERR_ARG, "gguf: bad array element");
      }
    } else if (!read_scalar(r, v.type, v)) {
      return set_error(VYBDQ_ERR_ARG, "gguf: bad metadata value type");
    }
    if (!r.ok()) return set_error(VYBDQ_ERR_ARG, "gguf: truncated metadata");
    if (key == "general.alignment" && (v.type == 4 || v.type == 10 || v.type == 5 || v.type == 11)) {
      if (v.i <= 0 || (v.i & (v.i - 1))) return set_error(VYBDQ_ERR_ARG, "gguf: alignment not a power of two");
      g.alignment = static_cast<uint64_t>(v.i);
    }
    g.kv.emplace_back(std::move(key), std::move(v));
  }
  g.tensors.resize(nt);
  for (uint64_t t = 0; t < nt; ++t) {
    GgufTensor &ti = g.tensors[t];
    ti.name = r.str();
    const uint32_t nd = r.get<uint32_t>();
    if (!r.ok() || nd > 8) return set_error(VYBDQ_ERR_ARG, "gguf: bad tensor info");
    ti.dims.resize(nd);
    for (uint32_t d = 0; d < nd; ++d) ti.dims[d] = static_cast<int64_t>(r.get<uint64_t>());
    ti.type = static_cast<int>(r.get<uint32_t>());
    ti.offset = r.get<uint64_t>();
    if (!r.ok()) return set_error(VYBDQ_ERR_ARG, "gguf: truncated tensor info");
  }
  g.info_end = r.pos();
  g.data_base = (g.info_end + g.alignment - 1) / g.alignment * g.alignment;
  return VYBDQ_OK;
}

static std::mutex g_mu;
static std::vector<std::shared_ptr<GgufFile>> g_files;  // handle h -> g_files[h - 1]

// The file of handle h, shared: a concurrent vybdq_gguf_close only drops the table's reference.
static std::shared_ptr<GgufFile> lookup(int64_t h) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (h < 1 || h > static_cast<int64_t>(g_files.size())) return nullptr;
  return g_files[h - 1];
}

static int64_t tensor_bytes(const GgufTensor &t) {
  const TypeSize ts = ggml_type_size(t.type);
  if (!ts.blk) return -1;
  int64_t n = 1;
  for (int64_t d : t.dims) {
    if (d < 0 || (d && n > INT64_MAX / d)) return -1;
    n *= d;
  }
  if (n % ts.blk || n / ts.blk > INT64_MAX / ts.bytes) return -1;
  return n / ts.blk * ts.bytes;
}

static int64_t copy_str(const std::string &s, char *buf, int64_t cap) {
  if (buf && cap > 0) {
    const int64_t n = static_cast<int64_t>(s.size()) < cap - 1 ? static_cast<int64_t>(s.size()) : cap - 1;
    memcpy(buf, s.data(), n);
    buf[n] = '\0';
  }
  return static_cast<int64_t>(s.size());
}

}  // namespace vybdq

using namespace vybdq;

#define GGUF_GET(h, g)                                                     \
  const std::shared_ptr<GgufFile> g = lookup(h);                           \
  if (!g) return set_error(VYBDQ_ERR_ARG, "gguf: unknown handle")
#define GGUF_TENSOR(g, i)                                                  \
  if (i < 0 || i >= static_cast<int64_t>(g->tensors.size()))               \
    return set_error(VYBDQ_ERR_ARG, "gguf: tensor index out of range")
#define GGUF_KV(g, i)                                                      \
  if (i < 0 || i >= static_cast<int64_t>(g->kv.size()))                    \
    return set_error(VYBDQ_ERR_ARG, "gguf: metadata index out of range")

extern "C" int64_t vybdq_gguf_open(const char *path) {
  VYBDQ_REQUIRE(path, VYBDQ_ERR_ARG, "null path");
  try {  // no exception crosses the C boundary (allocation failures on corrupt counts included)
    auto g = std::make_shared<GgufFile>();
    const int rc = parse(path, *g);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    g_files.push_back(std::move(g));
    return static_cast<int64_t>(g_files.size());
  } catch (const std::exception &e) {
    return set_error(VYBDQ_ERR_ARG, std::string("gguf: ") + e.what());
  }
}

extern "C" int vybdq_gguf_close(int64_t h) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (h < 1 || h > static_cast<int64_t>(g_files.size()) || !g_files[h - 1])
    return set_error(VYBDQ_ERR_ARG, "gguf: unknown handle");
  g_files[h - 1].reset();
  return VYBDQ_OK;
}

extern "C" int64_t vybdq_gguf_info(int64_t h, int what) {
  GGUF_GET(h, g);
  switch (what) {
    case 0: return g->version;
    case 1: return static_cast<int64_t>(g->tensors.size());
    case 2: return static_cast<int64_t>(g->kv.size());
    case 3: return static_cast<int64_t>(g->alignment);
    case 4: return static_cast<int64_t>(g->info_end);
    case 5: return static_cast<int64_t>(g->data_base);
    case 6: return static_cast<int64_t>(g->file_size);
    default: return set_error(VYBDQ_ERR_ARG, "gguf: unknown info field");
  }
}

extern "C" int64_t vybdq_gguf_find_tensor(int64_t h, const char *name) {
  GGUF_GET(h, g);
  VYBDQ_REQUIRE(name, VYBDQ_ERR_ARG, "null name");
  for (size_t i = 0; i < g->tensors.size(); ++i)
    if (g->tensors[i].name == name) return static_cast<int64_t>(i);
  return -1;
}

extern "C" int64_t vybdq_gguf_tensor_name(int64_t h, int64_t i, char *buf, int64_t cap) {
  GGUF_GET(h, g);
  GGUF_TENSOR(g, i);
  return copy_str(g->tensors[i].name, buf, cap);
}

// what: 0 ggml type, 1 n_dims, 2 + d dims[d], -1 raw offset field, -2 bytes (-1: unknown type)
extern "C" int64_t vybdq_gguf_tensor_field(int64_t h, int64_t i, int what) {
  GGUF_GET(h, g);
  GGUF_TENSOR(g, i);
  const GgufTensor &t = g->tensors[i];
  if (what == 0) return t.type;
  if (what == 1) return static_cast<int64_t>(t.dims.size());
  if (what == -1) return static_cast<int64_t>(t.offset);
  if (what == -2) return tensor_bytes(t);
  if (what >= 2 && what - 2 < static_cast<int>(t.dims.size())) return t.dims[what - 2];
  return set_error(VYBDQ_ERR_ARG, "gguf: unknown tensor field");
}

extern "C" int64_t vybdq_gguf_find_kv(int64_t h, const char *key) {
  GGUF_GET(h, g);
  VYBDQ_REQUIRE(key, VYBDQ_ERR_ARG, "null key");
  for (size_t i = 0; i < g->kv.size(); ++i)
    if (g->kv[i].first == key) return static_cast<int64_t>(i);
  return -1;
}

extern "C" int64_t vybdq_gguf_kv_key(int64_t h, int64_t i, char *buf, int64_t cap) {
  GGUF_GET(h, g);
  GGUF_KV(g, i);
  return copy_str(g->kv[i].first, buf, cap);
}

// what: 0 value type, 1 integer value (integer and bool types), 2 array element type,
// 3 array length
extern "C" int64_t vybdq_gguf_kv_field(int64_t h, int64_t i, int what) {
  GGUF_GET(h, g);
  GGUF_KV(g, i);
  const GgufValue &v = g->kv[i].second;
  switch (what) {
    case 0: return v.type;
    case 1:
      if (v.type == 6 || v.type == 8 || v.type == 9 || v.type == 12) return set_error(VYBDQ_ERR_ARG, "gguf: not an integer value");
      return v.i;
    case 2: return v.arr_type;
    case 3: return v.arr_len;
    default: return set_error(VYBDQ_ERR_ARG, "gguf: unknown metadata field");
  }
}

extern "C" double vybdq_gguf_kv_float(int64_t h, int64_t i) {
  const std::shared_ptr<GgufFile> g = lookup(h);
  if (!g || i < 0 || i >= static_cast<int64_t>(g->kv.size())) return 0.0;
  const GgufValue &v = g->kv[i].second;
  return (v.type == 6 || v.type == 12) ? v.f : static_cast<double>(v.i);
}

extern "C" int64_t vybdq_gguf_kv_string(int64_t h, int64_t i, char *buf, int64_t cap) {
  GGUF_GET(h, g);
  GGUF_KV(g, i);
  if (g->kv[i].second.type != 8) return set_error(VYBDQ_ERR_ARG, "gguf: not a string value");
  return copy_str(g->kv[i].second.s, buf, cap);
}

// Slab layout: tensors in index order, each at an offset rounded up to `align` (a power of two).
extern "C" int64_t vybdq_gguf_slab_offset(int64_t h, int64_t i, int64_t align) {
  GGUF_GET(h, g);
  VYBDQ_REQUIRE(align > 0 && !(align & (align - 1)), VYBDQ_ERR_ARG, "align must be a power of two");
  VYBDQ_REQUIRE(i >= 0 && i <= static_cast<int64_t>(g->tensors.size()), VYBDQ_ERR_ARG, "tensor index out of range");
  int64_t off = 0;
  for (int64_t k = 0; k < i; ++k) {
    const int64_t b = tensor_bytes(g->tensors[k]);
    if (b < 0) return set_error(VYBDQ_ERR_SHAPE, "gguf: tensor of unknown type or shape: " + g->tensors[k].name);
    off = (off + b + align - 1) / align * align;
  }
  return off;
}

extern "C" int64_t vybdq_gguf_slab_bytes(int64_t h, int64_t align) {
  GGUF_GET(h, g);
  return vybdq_gguf_slab_offset(h, static_cast<int64_t>(g->tensors.size()), align);
}

// Absolute file position of tensor i's data: absolute = 1 takes the offset field as a file
// offset (the reference fixture's convention), else data_base + offset (the GGUF convention).
static int tensor_span(const GgufFile &g, int64_t i, int absolute, uint64_t &pos, int64_t &n) {
  n = tensor_bytes(g.tensors[i]);
  if (n < 0) return set_error(VYBDQ_ERR_SHAPE, "gguf: tensor of unknown type or shape: " + g.tensors[i].name);
  pos = absolute ? g.tensors[i].offset : g.data_base + g.tensors[i].offset;
  if (pos < g.tensors[i].offset || pos > g.file_size || static_cast<uint64_t>(n) > g.file_size - pos)
    return set_error(VYBDQ_ERR_SHAPE, "gguf: tensor data past the end of the file: " + g.tensors[i].name);
  return VYBDQ_OK;
}

extern "C" int64_t vybdq_gguf_read_tensor(int64_t h, int64_t i, int absolute, void *dst, int64_t cap) {
  GGUF_GET(h, g);
  GGUF_TENSOR(g, i);
  uint64_t pos;
  int64_t n;
  const int rc = tensor_span(*g, i, absolute, pos, n);
  if (rc) return rc;
  VYBDQ_REQUIRE(dst && cap >= n, VYBDQ_ERR_ARG, "destination missing or too small");
  FILE *f = fopen(g->path.c_str(), "rb");
  if (!f) return set_error(VYBDQ_ERR_ARG, "gguf: cannot reopen " + g->path);
  std::unique_ptr<FILE, int (*)(FILE *)> guard(f, fclose);
  if (fseeko(f, static_cast<off_t>(pos), SEEK_SET) != 0 || fread(dst, 1, n, f) != static_cast<size_t>(n))
    return set_error(VYBDQ_ERR_ARG, "gguf: read failed");
  return n;
}

// Copies every tensor's bytes into the device slab (dev_bytes >= vybdq_gguf_slab_bytes), through
// a host buffer in 64 MB pieces, ordered on `stream`; returns when the last copy has finished.
extern "C" int vybdq_gguf_load_slab(int64_t h, uint64_t dev, int64_t dev_bytes, int64_t align, int absolute,
                                    uint64_t stream) {
  GGUF_GET(h, g);
  VYBDQ_REQUIRE(dev, VYBDQ_ERR_ARG, "null device buffer");
  const int64_t need = vybdq_gguf_slab_bytes(h, align);
  if (need < 0) return static_cast<int>(need);
  VYBDQ_REQUIRE(dev_bytes >= need, VYBDQ_ERR_WORKSPACE, "device slab smaller than vybdq_gguf_slab_bytes");
  FILE *f = fopen(g->path.c_str(), "rb");
  if (!f) return set_error(VYBDQ_ERR_ARG, "gguf: cannot reopen " + g->path);
  std::unique_ptr<FILE, int (*)(FILE *)> guard(f, fclose);
  constexpr int64_t kChunk = 64 << 20;
  std::vector<char> buf;
  hipStream_t s = as_stream(stream);
  int64_t off = 0;
  for (size_t i = 0; i < g->tensors.size(); ++i) {
    uint64_t pos;
    int64_t n;
    const int rc = tensor_span(*g, static_cast<int64_t>(i), absolute, pos, n);
    if (rc) return rc;
    if (fseeko(f, static_cast<off_t>(pos), SEEK_SET) != 0) return set_error(VYBDQ_ERR_ARG, "gguf: seek failed");
    for (int64_t done = 0; done < n;) {
      const int64_t m = n - done < kChunk ? n - done : kChunk;
      try {
        buf.resize(static_cast<size_t>(m));
      } catch (const std::exception &ex) {
        return set_error(VYBDQ_ERR_ARG, std::string("gguf: host buffer: ") + ex.what());
      }
      if (fread(buf.data(), 1, m, f) != static_cast<size_t>(m)) return set_error(VYBDQ_ERR_ARG, "gguf: read failed");
      hipError_t e = hipMemcpyAsync(reinterpret_cast<char *>(dev) + off + done, buf.data(), m, hipMemcpyHostToDevice, s);
      if (e == hipSuccess) e = hipStreamSynchronize(s);  // the host buffer is reused
      if (e != hipSuccess) return set_error(VYBDQ_ERR_HIP, std::string("gguf: copy to the slab: ") + hipGetErrorString(e));
      done += m;
    }
    off = (off + n + align - 1) / align * align;
  }
  return VYBDQ_OK;
}
