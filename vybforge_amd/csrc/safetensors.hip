// safetensors container reader, sharded-checkpoint index and device upload (host code).
//
// Container: u64 little-endian N, then N bytes of UTF-8 JSON, then the raw tensor bytes. The
// JSON is one object: every key but "__metadata__" names a tensor whose value is
// {"dtype": "<name>", "shape": [d0, ...], "data_offsets": [begin, end]} with [begin, end) relative
// to the first byte after the header (8 + N); "__metadata__" maps strings to strings. Trailing
// whitespace after the object pads the header. A sharded checkpoint adds
// model.safetensors.index.json: {"metadata": {...}, "weight_map": {"<tensor>": "<shard file>"}}.
// Replaces the reference's readers: native/torchload/safetensors.vyb (container and dtype table,
// safetensors.vyb:8-19 and 48-66) and native/glm53/gx.vyb (name -> shard through the index,
// gx.vyb:1-16). The EXL3 tensors of one linear layer (<prefix>.trellis / .suh / .svh / .mcg,
// native/glm53/loader.py:20-29) are resolved by name through these entry points.
#include "common.h"

#include <cerrno>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

namespace vybdq {

// ---- minimal JSON (the subset a header or an index needs, strict about syntax) ----------------

struct JsonVal {
  enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
  bool b = false;
  bool is_int = false;
  int64_t i = 0;
  double num = 0.0;
  std::string s;
  std::vector<JsonVal> arr;
  std::vector<std::pair<std::string, JsonVal>> obj;
};

class JsonParser {
 public:
  JsonParser(const char *p, size_t n) : p_(p), n_(n) {}
  bool parse_top(JsonVal &v) {
    ws();
    if (!value(v, 0)) return false;
    ws();
    if (pos_ != n_) return fail("trailing characters after the JSON value");
    return true;
  }
  const std::string &error() const { return err_; }

 private:
  const char *p_;
  size_t n_, pos_ = 0;
  std::string err_;

  bool fail(const std::string &m) {
    if (err_.empty()) err_ = m + " at byte " + std::to_string(pos_);
    return false;
  }
  void ws() {
    while (pos_ < n_ && (p_[pos_] == ' ' || p_[pos_] == '\t' || p_[pos_] == '\n' || p_[pos_] == '\r')) ++pos_;
  }
  bool lit(const char *w) {
    const size_t l = strlen(w);
    if (n_ - pos_ < l || memcmp(p_ + pos_, w, l) != 0) return fail("bad literal");
    pos_ += l;
    return true;
  }
  static void put_utf8(std::string &o, uint32_t c) {
    if (c < 0x80) {
      o += static_cast<char>(c);
    } else if (c < 0x800) {
      o += static_cast<char>(0xC0 | (c >> 6));
      o += static_cast<char>(0x80 | (c & 0x3F));
    } else if (c < 0x10000) {
      o += static_cast<char>(0xE0 | (c >> 12));
      o += static_cast<char>(0x80 | ((c >> 6) & 0x3F));
      o += static_cast<char>(0x80 | (c & 0x3F));
    } else {
      o += static_cast<char>(0xF0 | (c >> 18));
      o += static_cast<char>(0x80 | ((c >> 12) & 0x3F));
      o += static_cast<char>(0x80 | ((c >> 6) & 0x3F));
      o += static_cast<char>(0x80 | (c & 0x3F));
    }
  }
  bool hex4(uint32_t &c) {
    if (n_ - pos_ < 4) return fail("short \\u escape");
    c = 0;
    for (int k = 0; k < 4; ++k) {
      const char h = p_[pos_++];
      c <<= 4;
      if (h >= '0' && h <= '9') c |= h - '0';
      else if (h >= 'a' && h <= 'f') c |= h - 'a' + 10;
      else if (h >= 'A' && h <= 'F') c |= h - 'A' + 10;
      else return fail("bad hex digit in \\u escape");
    }
    return true;
  }
  bool str(std::string &o) {
    if (pos_ >= n_ || p_[pos_] != '"') return fail("expected a string");
    ++pos_;
    while (true) {
      if (pos_ >= n_) return fail("unterminated string");
      const unsigned char ch = static_cast<unsigned char>(p_[pos_++]);
      if (ch == '"') return true;
      if (ch < 0x20) return fail("control character in a string");
      if (ch != '\\') {
        o += static_cast<char>(ch);
        continue;
      }
      if (pos_ >= n_) return fail("unterminated escape");
      const char e = p_[pos_++];
      switch (e) {
        case '"': o += '"'; break;
        case '\\': o += '\\'; break;
        case '/': o += '/'; break;
        case 'b': o += '\b'; break;
        case 'f': o += '\f'; break;
        case 'n': o += '\n'; break;
        case 'r': o += '\r'; break;
        case 't': o += '\t'; break;
        case 'u': {
          uint32_t c;
          if (!hex4(c)) return false;
          if (c >= 0xD800 && c < 0xDC00) {  // high surrogate: a low one must follow
            uint32_t lo;
            if (n_ - pos_ < 2 || p_[pos_] != '\\' || p_[pos_ + 1] != 'u') return fail("lone high surrogate");
            pos_ += 2;
            if (!hex4(lo)) return false;
            if (lo < 0xDC00 || lo >= 0xE000) return fail("bad low surrogate");
            c = 0x10000 + ((c - 0xD800) << 10) + (lo - 0xDC00);
          } else if (c >= 0xDC00 && c < 0xE000) {
            return fail("lone low surrogate");
          }
          put_utf8(o, c);
          break;
        }
        default: return fail("bad escape");
      }
    }
  }
  bool number(JsonVal &v) {
    const size_t b = pos_;
    if (pos_ < n_ && p_[pos_] == '-') ++pos_;
    if (pos_ >= n_ || !(p_[pos_] >= '0' && p_[pos_] <= '9')) return fail("bad number");
    if (p_[pos_] == '0') ++pos_;
    else while (pos_ < n_ && p_[pos_] >= '0' && p_[pos_] <= '9') ++pos_;
    bool integral = true;
    if (pos_ < n_ && p_[pos_] == '.') {
      integral = false;
      ++pos_;
      if (pos_ >= n_ || !(p_[pos_] >= '0' && p_[pos_] <= '9')) return fail("bad fraction");
      while (pos_ < n_ && p_[pos_] >= '0' && p_[pos_] <= '9') ++pos_;
    }
    if (pos_ < n_ && (p_[pos_] == 'e' || p_[pos_] == 'E')) {
      integral = false;
      ++pos_;
      if (pos_ < n_ && (p_[pos_] == '+' || p_[pos_] == '-')) ++pos_;
      if (pos_ >= n_ || !(p_[pos_] >= '0' && p_[pos_] <= '9')) return fail("bad exponent");
      while (pos_ < n_ && p_[pos_] >= '0' && p_[pos_] <= '9') ++pos_;
    }
    const std::string t(p_ + b, pos_ - b);
    v.kind = JsonVal::NUM;
    v.num = strtod(t.c_str(), nullptr);
    if (integral) {
      errno = 0;
      char *end = nullptr;
      const long long x = strtoll(t.c_str(), &end, 10);
      v.is_int = errno == 0 && end && *end == '\0';
      v.i = x;
    }
    return true;
  }
  bool value(JsonVal &v, int depth) {
    if (depth > 64) return fail("JSON nested too deeply");
    ws();
    if (pos_ >= n_) return fail("unexpected end of JSON");
    const char c = p_[pos_];
    if (c == '{') {
      v.kind = JsonVal::OBJ;
      ++pos_;
      ws();
      if (pos_ < n_ && p_[pos_] == '}') { ++pos_; return true; }
      while (true) {
        ws();
        std::string k;
        if (!str(k)) return false;
        ws();
        if (pos_ >= n_ || p_[pos_] != ':') return fail("expected ':'");
        ++pos_;
        v.obj.emplace_back(std::move(k), JsonVal());
        if (!value(v.obj.back().second, depth + 1)) return false;
        ws();
        if (pos_ < n_ && p_[pos_] == ',') { ++pos_; continue; }
        if (pos_ < n_ && p_[pos_] == '}') { ++pos_; return true; }
        return fail("expected ',' or '}'");
      }
    }
    if (c == '[') {
      v.kind = JsonVal::ARR;
      ++pos_;
      ws();
      if (pos_ < n_ && p_[pos_] == ']') { ++pos_; return true; }
      while (true) {
        v.arr.emplace_back();
        if (!value(v.arr.back(), depth + 1)) return false;
        ws();
        if (pos_ < n_ && p_[pos_] == ',') { ++pos_; continue; }
        if (pos_ < n_ && p_[pos_] == ']') { ++pos_; return true; }
        return fail("expected ',' or ']'");
      }
    }
    if (c == '"') { v.kind = JsonVal::STR; return str(v.s); }
    if (c == 't') { v.kind = JsonVal::BOOL; v.b = true; return lit("true"); }
    if (c == 'f') { v.kind = JsonVal::BOOL; v.b = false; return lit("false"); }
    if (c == 'n') { v.kind = JsonVal::NUL; return lit("null"); }
    return number(v);
  }
};

// ---- safetensors files ------------------------------------------------------------------------

// element size of a safetensors dtype spelling; 0 = not sized here (the tensor is listed, and its
// byte range is still checked against the data region, but no shape x size check applies)
static int st_dtype_size(const std::string &d) {
  static const std::pair<const char *, int> k[] = {
      {"F64", 8}, {"I64", 8}, {"U64", 8}, {"F32", 4}, {"I32", 4}, {"U32", 4}, {"F16", 2}, {"BF16", 2},
      {"I16", 2}, {"U16", 2}, {"I8", 1}, {"U8", 1}, {"BOOL", 1}, {"F8_E4M3", 1}, {"F8_E5M2", 1}};
  for (const auto &e : k)
    if (d == e.first) return e.second;
  return 0;
}

struct StTensor {
  std::string name, dtype;
  std::vector<int64_t> shape;
  uint64_t begin = 0, end = 0;  // relative to data_base
};

struct StFile {
  std::string path;
  uint64_t file_size = 0, header_len = 0, data_base = 0;
  std::vector<StTensor> tensors;
  std::unordered_map<std::string, int64_t> by_name;
  std::vector<std::pair<std::string, std::string>> meta;
};

struct StIndex {
  std::vector<std::pair<std::string, std::string>> map;  // tensor -> shard file, file order
  std::unordered_map<std::string, int64_t> by_name;
};

static constexpr uint64_t kMaxHeader = 100ull << 20;  // the limit of the safetensors library

static int parse_st(const std::string &path, StFile &out) {
  FILE *f = fopen(path.c_str(), "rb");
  if (!f) return set_error(VYBDQ_ERR_ARG, "safetensors: cannot open " + path);
  std::unique_ptr<FILE, int (*)(FILE *)> guard(f, fclose);
  if (fseeko(f, 0, SEEK_END) != 0) return set_error(VYBDQ_ERR_ARG, "safetensors: seek failed");
  out.file_size = static_cast<uint64_t>(ftello(f));
  fseeko(f, 0, SEEK_SET);
  unsigned char lb[8];
  if (out.file_size < 8 || fread(lb, 1, 8, f) != 8) return set_error(VYBDQ_ERR_SHAPE, "safetensors: file shorter than 8 bytes");
  uint64_t n = 0;
  for (int k = 7; k >= 0; --k) n = (n << 8) | lb[k];
  if (n > kMaxHeader) return set_error(VYBDQ_ERR_SHAPE, "safetensors: header length over 100 MB");
  if (n > out.file_size - 8) return set_error(VYBDQ_ERR_SHAPE, "safetensors: header runs past the end of the file");
  std::string hdr(static_cast<size_t>(n), '\0');
  if (n && fread(&hdr[0], 1, n, f) != n) return set_error(VYBDQ_ERR_ARG, "safetensors: header read failed");
  out.header_len = n;
  out.data_base = 8 + n;
  const uint64_t data_size = out.file_size - out.data_base;
  if (n == 0 || hdr[0] != '{') return set_error(VYBDQ_ERR_SHAPE, "safetensors: header is not a JSON object");
  JsonVal root;
  JsonParser jp(hdr.data(), hdr.size());
  if (!jp.parse_top(root)) return set_error(VYBDQ_ERR_SHAPE, "safetensors: header JSON: " + jp.error());
  for (auto &kv : root.obj) {
    if (kv.first == "__metadata__") {
      if (kv.second.kind != JsonVal::OBJ) return set_error(VYBDQ_ERR_SHAPE, "safetensors: __metadata__ is not an object");
      for (auto &m : kv.second.obj) {
        if (m.second.kind != JsonVal::STR)
          return set_error(VYBDQ_ERR_SHAPE, "safetensors: __metadata__ value of '" + m.first + "' is not a string");
        out.meta.emplace_back(m.first, m.second.s);
      }
      continue;
    }
    const JsonVal &t = kv.second;
    if (t.kind != JsonVal::OBJ) return set_error(VYBDQ_ERR_SHAPE, "safetensors: entry '" + kv.first + "' is not an object");
    StTensor st;
    st.name = kv.first;
    bool has_dt = false, has_shape = false, has_off = false;
    for (auto &f2 : t.obj) {
      if (f2.first == "dtype") {
        if (f2.second.kind != JsonVal::STR) return set_error(VYBDQ_ERR_SHAPE, "safetensors: dtype of '" + st.name + "'");
        st.dtype = f2.second.s;
        has_dt = true;
      } else if (f2.first == "shape") {
        if (f2.second.kind != JsonVal::ARR) return set_error(VYBDQ_ERR_SHAPE, "safetensors: shape of '" + st.name + "'");
        for (auto &d : f2.second.arr) {
          if (d.kind != JsonVal::NUM || !d.is_int || d.i < 0)
            return set_error(VYBDQ_ERR_SHAPE, "safetensors: shape of '" + st.name + "' is not non-negative integers");
          st.shape.push_back(d.i);
        }
        has_shape = true;
      } else if (f2.first == "data_offsets") {
        const JsonVal &o = f2.second;
        if (o.kind != JsonVal::ARR || o.arr.size() != 2 || o.arr[0].kind != JsonVal::NUM || o.arr[1].kind != JsonVal::NUM ||
            !o.arr[0].is_int || !o.arr[1].is_int || o.arr[0].i < 0 || o.arr[1].i < o.arr[0].i)
          return set_error(VYBDQ_ERR_SHAPE, "safetensors: data_offsets of '" + st.name + "' must be [begin, end], begin <= end");
        st.begin = static_cast<uint64_t>(o.arr[0].i);
        st.end = static_cast<uint64_t>(o.arr[1].i);
        has_off = true;
      }
    }
    if (!has_dt || !has_shape || !has_off)
      return set_error(VYBDQ_ERR_SHAPE, "safetensors: entry '" + st.name + "' lacks dtype, shape or data_offsets");
    if (st.end > data_size) return set_error(VYBDQ_ERR_SHAPE, "safetensors: data of '" + st.name + "' past the end of the file");
    const int es = st_dtype_size(st.dtype);
    if (es) {
      uint64_t numel = 1;
      for (int64_t d : st.shape) {
        if (d && numel > UINT64_MAX / static_cast<uint64_t>(d)) return set_error(VYBDQ_ERR_SHAPE, "safetensors: shape overflow");
        numel *= static_cast<uint64_t>(d);
      }
      if (numel > UINT64_MAX / es || numel * es != st.end - st.begin)
        return set_error(VYBDQ_ERR_SHAPE, "safetensors: byte range of '" + st.name + "' does not match its shape and dtype");
    }
    if (!out.by_name.emplace(st.name, static_cast<int64_t>(out.tensors.size())).second)
      return set_error(VYBDQ_ERR_SHAPE, "safetensors: duplicate tensor '" + st.name + "'");
    out.tensors.push_back(std::move(st));
  }
  return VYBDQ_OK;
}

static int parse_index(const std::string &path, StIndex &out) {
  FILE *f = fopen(path.c_str(), "rb");
  if (!f) return set_error(VYBDQ_ERR_ARG, "safetensors index: cannot open " + path);
  std::unique_ptr<FILE, int (*)(FILE *)> guard(f, fclose);
  std::string text;
  char buf[1 << 16];
  size_t m;
  while ((m = fread(buf, 1, sizeof buf, f)) > 0) text.append(buf, m);
  JsonVal root;
  JsonParser jp(text.data(), text.size());
  if (!jp.parse_top(root) || root.kind != JsonVal::OBJ)
    return set_error(VYBDQ_ERR_SHAPE, "safetensors index: " + (jp.error().empty() ? std::string("not a JSON object") : jp.error()));
  for (auto &kv : root.obj) {
    if (kv.first != "weight_map") continue;
    if (kv.second.kind != JsonVal::OBJ) return set_error(VYBDQ_ERR_SHAPE, "safetensors index: weight_map is not an object");
    for (auto &e : kv.second.obj) {
      if (e.second.kind != JsonVal::STR) return set_error(VYBDQ_ERR_SHAPE, "safetensors index: shard of '" + e.first + "' is not a string");
      if (!out.by_name.emplace(e.first, static_cast<int64_t>(out.map.size())).second)
        return set_error(VYBDQ_ERR_SHAPE, "safetensors index: duplicate tensor '" + e.first + "'");
      out.map.emplace_back(e.first, e.second.s);
    }
    return VYBDQ_OK;
  }
  return set_error(VYBDQ_ERR_SHAPE, "safetensors index: no weight_map");
}

static std::mutex st_mu;
static std::vector<std::unique_ptr<StFile>> st_files;     // handle h -> st_files[h - 1]
static std::vector<std::unique_ptr<StIndex>> st_indexes;  // handle h -> st_indexes[h - 1]

static StFile *st_lookup(int64_t h) {
  std::lock_guard<std::mutex> lk(st_mu);
  if (h < 1 || h > static_cast<int64_t>(st_files.size())) return nullptr;
  return st_files[h - 1].get();
}
static StIndex *idx_lookup(int64_t h) {
  std::lock_guard<std::mutex> lk(st_mu);
  if (h < 1 || h > static_cast<int64_t>(st_indexes.size())) return nullptr;
  return st_indexes[h - 1].get();
}

static int64_t st_copy_str(const std::string &s, char *buf, int64_t cap) {
  if (buf && cap > 0) {
    const int64_t n = static_cast<int64_t>(s.size()) < cap - 1 ? static_cast<int64_t>(s.size()) : cap - 1;
    memcpy(buf, s.data(), n);
    buf[n] = '\0';
  }
  return static_cast<int64_t>(s.size());
}

}  // namespace vybdq

using namespace vybdq;

#define ST_GET(h, g)                                                        \
  StFile *g = st_lookup(h);                                                 \
  if (!g) return set_error(VYBDQ_ERR_ARG, "safetensors: unknown handle")
#define ST_TENSOR(g, i)                                                     \
  if (i < 0 || i >= static_cast<int64_t>(g->tensors.size()))               \
    return set_error(VYBDQ_ERR_ARG, "safetensors: tensor index out of range")

extern "C" int64_t vybdq_st_open(const char *path) {
  VYBDQ_REQUIRE(path, VYBDQ_ERR_ARG, "null path");
  std::unique_ptr<StFile> g(new StFile);
  g->path = path;
  const int rc = parse_st(g->path, *g);
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(st_mu);
  st_files.push_back(std::move(g));
  return static_cast<int64_t>(st_files.size());
}

extern "C" int vybdq_st_close(int64_t h) {
  std::lock_guard<std::mutex> lk(st_mu);
  if (h < 1 || h > static_cast<int64_t>(st_files.size()) || !st_files[h - 1])
    return set_error(VYBDQ_ERR_ARG, "safetensors: unknown handle");
  st_files[h - 1].reset();
  return VYBDQ_OK;
}

extern "C" int64_t vybdq_st_info(int64_t h, int what) {
  ST_GET(h, g);
  switch (what) {
    case 0: return static_cast<int64_t>(g->tensors.size());
    case 1: return static_cast<int64_t>(g->meta.size());
    case 2: return static_cast<int64_t>(g->header_len);
    case 3: return static_cast<int64_t>(g->data_base);
    case 4: return static_cast<int64_t>(g->file_size);
    default: return set_error(VYBDQ_ERR_ARG, "safetensors: unknown info field");
  }
}

extern "C" int64_t vybdq_st_find(int64_t h, const char *name) {
  ST_GET(h, g);
  VYBDQ_REQUIRE(name, VYBDQ_ERR_ARG, "null name");
  auto it = g->by_name.find(name);
  return it == g->by_name.end() ? -1 : it->second;
}

extern "C" int64_t vybdq_st_tensor_name(int64_t h, int64_t i, char *buf, int64_t cap) {
  ST_GET(h, g);
  ST_TENSOR(g, i);
  return st_copy_str(g->tensors[i].name, buf, cap);
}

extern "C" int64_t vybdq_st_tensor_dtype(int64_t h, int64_t i, char *buf, int64_t cap) {
  ST_GET(h, g);
  ST_TENSOR(g, i);
  return st_copy_str(g->tensors[i].dtype, buf, cap);
}

extern "C" int64_t vybdq_st_tensor_field(int64_t h, int64_t i, int what) {
  ST_GET(h, g);
  ST_TENSOR(g, i);
  const StTensor &t = g->tensors[i];
  if (what == 0) return st_dtype_size(t.dtype);
  if (what == 1) return static_cast<int64_t>(t.shape.size());
  if (what >= 2 && what - 2 < static_cast<int>(t.shape.size())) return t.shape[what - 2];
  if (what == -1) return static_cast<int64_t>(g->data_base + t.begin);
  if (what == -2) return static_cast<int64_t>(t.end - t.begin);
  return set_error(VYBDQ_ERR_ARG, "safetensors: unknown tensor field");
}

extern "C" int64_t vybdq_st_meta(int64_t h, const char *key, char *buf, int64_t cap) {
  ST_GET(h, g);
  VYBDQ_REQUIRE(key, VYBDQ_ERR_ARG, "null key");
  for (auto &m : g->meta)
    if (m.first == key) return st_copy_str(m.second, buf, cap);
  return -1;
}

extern "C" int64_t vybdq_st_meta_key(int64_t h, int64_t i, char *buf, int64_t cap) {
  ST_GET(h, g);
  VYBDQ_REQUIRE(i >= 0 && i < static_cast<int64_t>(g->meta.size()), VYBDQ_ERR_ARG, "metadata index out of range");
  return st_copy_str(g->meta[i].first, buf, cap);
}

extern "C" int64_t vybdq_st_read(int64_t h, int64_t i, void *dst, int64_t cap) {
  ST_GET(h, g);
  ST_TENSOR(g, i);
  const StTensor &t = g->tensors[i];
  const int64_t n = static_cast<int64_t>(t.end - t.begin);
  VYBDQ_REQUIRE(dst && cap >= n, VYBDQ_ERR_ARG, "destination missing or too small");
  FILE *f = fopen(g->path.c_str(), "rb");
  if (!f) return set_error(VYBDQ_ERR_ARG, "safetensors: cannot reopen " + g->path);
  std::unique_ptr<FILE, int (*)(FILE *)> guard(f, fclose);
  if (fseeko(f, static_cast<off_t>(g->data_base + t.begin), SEEK_SET) != 0 ||
      (n && fread(dst, 1, n, f) != static_cast<size_t>(n)))
    return set_error(VYBDQ_ERR_ARG, "safetensors: read failed");
  return n;
}

// Copies tensor i's bytes to device memory dev (dev_bytes >= its size) on stream, through a host
// buffer in 64 MB pieces; returns the byte count once the last copy has finished.
extern "C" int64_t vybdq_st_upload(int64_t h, int64_t i, uint64_t dev, int64_t dev_bytes, uint64_t stream) {
  ST_GET(h, g);
  ST_TENSOR(g, i);
  const StTensor &t = g->tensors[i];
  const int64_t n = static_cast<int64_t>(t.end - t.begin);
  VYBDQ_REQUIRE(dev || n == 0, VYBDQ_ERR_ARG, "null device buffer");
  VYBDQ_REQUIRE(dev_bytes >= n, VYBDQ_ERR_WORKSPACE, "device buffer smaller than the tensor");
  FILE *f = fopen(g->path.c_str(), "rb");
  if (!f) return set_error(VYBDQ_ERR_ARG, "safetensors: cannot reopen " + g->path);
  std::unique_ptr<FILE, int (*)(FILE *)> guard(f, fclose);
  if (fseeko(f, static_cast<off_t>(g->data_base + t.begin), SEEK_SET) != 0)
    return set_error(VYBDQ_ERR_ARG, "safetensors: seek failed");
  constexpr int64_t kChunk = 64 << 20;
  std::vector<char> buf;
  hipStream_t s = as_stream(stream);
  for (int64_t done = 0; done < n;) {
    const int64_t m = n - done < kChunk ? n - done : kChunk;
    buf.resize(static_cast<size_t>(m));
    if (fread(buf.data(), 1, m, f) != static_cast<size_t>(m)) return set_error(VYBDQ_ERR_ARG, "safetensors: read failed");
    hipError_t e = hipMemcpyAsync(reinterpret_cast<char *>(dev) + done, buf.data(), m, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);  // the host buffer is reused
    if (e != hipSuccess) return set_error(VYBDQ_ERR_HIP, std::string("safetensors: copy to the device: ") + hipGetErrorString(e));
    done += m;
  }
  return n;
}

extern "C" int64_t vybdq_st_index_open(const char *path) {
  VYBDQ_REQUIRE(path, VYBDQ_ERR_ARG, "null path");
  std::unique_ptr<StIndex> x(new StIndex);
  const int rc = parse_index(path, *x);
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(st_mu);
  st_indexes.push_back(std::move(x));
  return static_cast<int64_t>(st_indexes.size());
}

extern "C" int vybdq_st_index_close(int64_t h) {
  std::lock_guard<std::mutex> lk(st_mu);
  if (h < 1 || h > static_cast<int64_t>(st_indexes.size()) || !st_indexes[h - 1])
    return set_error(VYBDQ_ERR_ARG, "safetensors index: unknown handle");
  st_indexes[h - 1].reset();
  return VYBDQ_OK;
}

extern "C" int64_t vybdq_st_index_count(int64_t h) {
  StIndex *x = idx_lookup(h);
  if (!x) return set_error(VYBDQ_ERR_ARG, "safetensors index: unknown handle");
  return static_cast<int64_t>(x->map.size());
}

extern "C" int64_t vybdq_st_index_entry(int64_t h, int64_t i, char *name, int64_t name_cap, char *shard, int64_t shard_cap) {
  StIndex *x = idx_lookup(h);
  if (!x) return set_error(VYBDQ_ERR_ARG, "safetensors index: unknown handle");
  VYBDQ_REQUIRE(i >= 0 && i < static_cast<int64_t>(x->map.size()), VYBDQ_ERR_ARG, "index entry out of range");
  st_copy_str(x->map[i].second, shard, shard_cap);
  return st_copy_str(x->map[i].first, name, name_cap);
}

extern "C" int64_t vybdq_st_index_shard(int64_t h, const char *name, char *buf, int64_t cap) {
  StIndex *x = idx_lookup(h);
  if (!x) return set_error(VYBDQ_ERR_ARG, "safetensors index: unknown handle");
  VYBDQ_REQUIRE(name, VYBDQ_ERR_ARG, "null name");
  auto it = x->by_name.find(name);
  if (it == x->by_name.end()) return -1;
  return st_copy_str(x->map[it->second].second, buf, cap);
}
