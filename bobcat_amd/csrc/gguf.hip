// GGUF model files: the parser of crates/bobcat-gguf/src/lib.rs (every read
// checked against the end of the file, every size computation against
// overflow, the same error kinds), and the model loaders of lfm2.rs:186-232,
// 737-1004 and qwen35.rs:186-230, 630-745 that fill the driver's model
// structs with pointers into the file.  Host code only.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "runtime.h"

namespace {

constexpr uint32_t kMagic = 0x46554747u;
constexpr uint64_t kDefaultAlignment = 32;
constexpr uint32_t kMaxDims = 4;
constexpr uint64_t kMinKvBytes = 8 + 4 + 1;             // empty key, type, one-byte value
constexpr uint64_t kMinTensorBytes = 8 + 4 + 8 + 4 + 8;  // empty name, one dim, type, offset

enum ValueType : uint32_t { U8 = 0, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 };

int fixed_size(uint32_t t) {
  switch (t) {
    case U8: case I8: case BOOL: return 1;
    case U16: case I16: return 2;
    case U32: case I32: case F32: return 4;
    case U64: case I64: case F64: return 8;
    default: return 0;
  }
}

// (elements per block, bytes per block) of a tensor type bobcat reads, or (0, 0).
std::pair<uint64_t, uint64_t> block_of(uint32_t id) {
  switch (id) {
    case 0: return {1, 4};
    case 1: case 30: return {1, 2};
    case 2: return {32, 18};
    case 8: return {32, 34};
    case 12: return {256, 144};
    case 13: return {256, 176};
    case 14: return {256, 210};
    default: return {0, 0};
  }
}

struct Value {
  uint32_t type = 0;
  uint64_t bits = 0;              // fixed-size value, little-endian, zero-extended
  uint64_t start = 0, end = 0;    // string bytes, or array data
  uint32_t element = 0;           // array element type
  uint64_t count = 0;             // array element count
};

struct Reader {
  const uint8_t *p;
  uint64_t size, pos = 0;
  uint64_t remaining() const { return size > pos ? size - pos : 0; }
  bool take(uint64_t n, const uint8_t **out) {
    if (n > remaining()) return false;
    *out = p + pos;
    pos += n;
    return true;
  }
  bool u32(uint32_t *v) {
    const uint8_t *b;
    if (!take(4, &b)) return false;
    memcpy(v, b, 4);
    return true;
  }
  bool u64(uint64_t *v) {
    const uint8_t *b;
    if (!take(8, &b)) return false;
    memcpy(v, b, 8);
    return true;
  }
  bool string(uint64_t *start, uint64_t *end) {
    uint64_t len;
    const uint8_t *b;
    if (!u64(&len)) return false;
    *start = pos;
    if (!take(len, &b)) return false;
    *end = pos;
    return true;
  }
};

// UTF-8 as Rust's String::from_utf8 accepts it: no overlong forms, no
// surrogates, nothing above U+10FFFF.
bool valid_utf8(const uint8_t *s, uint64_t n) {
  uint64_t i = 0;
  while (i < n) {
    const uint8_t c = s[i];
    uint64_t k;
    if (c < 0x80)
      k = 0;
    else if (c >= 0xC2 && c <= 0xDF)
      k = 1;
    else if ((c & 0xF0) == 0xE0)
      k = 2;
    else if (c >= 0xF0 && c <= 0xF4)
      k = 3;
    else
      return false;
    if (k > n - i - 1) return false;
    for (uint64_t j = 1; j <= k; j++)
      if ((s[i + j] & 0xC0) != 0x80) return false;
    if (c == 0xE0 && s[i + 1] < 0xA0) return false;  // overlong
    if (c == 0xED && s[i + 1] >= 0xA0) return false;  // surrogate
    if (c == 0xF0 && s[i + 1] < 0x90) return false;  // overlong
    if (c == 0xF4 && s[i + 1] >= 0x90) return false;  // above U+10FFFF
    i += k + 1;
  }
  return true;
}

bool read_value(Reader &r, uint32_t type, Value *v) {
  v->type = type;
  const int fs = fixed_size(type);
  if (fs) {
    const uint8_t *b;
    if (!r.take((uint64_t)fs, &b)) return false;
    v->bits = 0;
    memcpy(&v->bits, b, fs);
    return true;
  }
  if (type == STRING) return r.string(&v->start, &v->end);
  if (type != ARRAY) return false;
  uint32_t element;
  uint64_t count;
  if (!r.u32(&element) || !r.u64(&count)) return false;
  v->element = element;
  v->count = count;
  v->start = r.pos;
  if (element == STRING) {
    // Each string needs at least its 8-byte length.
    if (count > r.remaining() / 8) return false;
    for (uint64_t i = 0; i < count; i++) {
      uint64_t s, e;
      if (!r.string(&s, &e)) return false;
    }
  } else {
    const int es = fixed_size(element);
    if (!es) return false;  // unknown element types and nested arrays
    if (count > r.remaining() / (uint64_t)es) return false;
    const uint8_t *b;
    if (!r.take(count * (uint64_t)es, &b)) return false;
  }
  v->end = r.pos;
  return true;
}

// A value as u32 when it is an integer that fits (lib.rs Value::as_u32).
bool as_u32(const Value &v, uint32_t *out) {
  uint64_t u = v.bits;
  switch (v.type) {
    case U8: case U16: case U32: case U64: break;
    case I8: if ((int8_t)u < 0) return false; u = (uint64_t)(int8_t)u; break;
    case I16: if ((int16_t)u < 0) return false; u = (uint64_t)(int16_t)u; break;
    case I32: if ((int32_t)u < 0) return false; u = (uint64_t)(int32_t)u; break;
    case I64: if ((int64_t)u < 0) return false; break;
    default: return false;
  }
  if (u > 0xffffffffull) return false;
  *out = (uint32_t)u;
  return true;
}

}  // namespace

struct bch_gguf {
  const uint8_t *data = nullptr;
  uint64_t size = 0;
  void *map = nullptr;  // the file's mapping, when opened by path
  std::unordered_map<std::string, Value> meta;
  struct Tensor {
    std::string name;
    uint32_t n_dims = 0;
    uint64_t ne[kMaxDims] = {1, 1, 1, 1};
    uint32_t type = 0;
    uint64_t start = 0, end = 0;
  };
  std::vector<Tensor> tensors;
  std::unordered_map<std::string, size_t> by_name;

  ~bch_gguf() {
    if (map) munmap(map, size);
  }

  const Value *get(const char *key) const {
    auto it = meta.find(key);
    return it == meta.end() ? nullptr : &it->second;
  }
  const Tensor *tensor(const std::string &name) const {
    auto it = by_name.find(name);
    return it == by_name.end() ? nullptr : &tensors[it->second];
  }
};

namespace {

// Gguf::parse (lib.rs:310-345) with parse_metadata, parse_tensors and
// locate_tensor (lib.rs:576-740).
int parse(bch_gguf *g) {
  Reader r{g->data, g->size};
  uint32_t magic, version;
  uint64_t n_tensors, n_kv;
  if (!r.u32(&magic) || magic != kMagic) return bch::fail(BCH_ERR_GGUF, "not a GGUF file");
  if (!r.u32(&version) || !r.u64(&n_tensors) || !r.u64(&n_kv)) return bch::fail(BCH_ERR_GGUF, "truncated GGUF header");
  if (version != 2 && version != 3) return bch::fail(BCH_ERR_GGUF, "unsupported GGUF version %u", version);
  if (n_kv > r.remaining() / kMinKvBytes)
    return bch::fail(BCH_ERR_GGUF, "metadata count %llu exceeds the file size", (unsigned long long)n_kv);
  for (uint64_t i = 0; i < n_kv; i++) {
    uint64_t ks, ke;
    uint32_t type;
    Value v;
    if (!r.string(&ks, &ke) || !valid_utf8(g->data + ks, ke - ks) || !r.u32(&type) || !read_value(r, type, &v))
      return bch::fail(BCH_ERR_GGUF, "metadata entry %llu is malformed", (unsigned long long)i);
    std::string key(reinterpret_cast<const char *>(g->data + ks), ke - ks);
    if (!g->meta.emplace(key, v).second)
      return bch::fail(BCH_ERR_GGUF, "metadata key %s appears twice", key.c_str());
  }
  uint64_t alignment = kDefaultAlignment;
  if (const Value *a = g->get("general.alignment")) {
    const uint32_t v = (uint32_t)a->bits;
    if (a->type != U32 || v == 0 || (v & (v - 1))) return bch::fail(BCH_ERR_GGUF, "general.alignment must be a power of two");
    alignment = v;
  }
  if (n_tensors > r.remaining() / kMinTensorBytes)
    return bch::fail(BCH_ERR_GGUF, "tensor count %llu exceeds the file size", (unsigned long long)n_tensors);
  struct Header {
    std::string name;
    uint32_t n_dims;
    uint64_t ne[kMaxDims];
    uint32_t type;
    uint64_t offset;
  };
  std::vector<Header> headers;
  headers.reserve(n_tensors);
  for (uint64_t i = 0; i < n_tensors; i++) {
    Header h{};
    uint64_t ns, ne_;
    for (auto &d : h.ne) d = 1;
    bool ok = r.string(&ns, &ne_) && valid_utf8(g->data + ns, ne_ - ns) && r.u32(&h.n_dims);
    if (ok) {
      h.name.assign(reinterpret_cast<const char *>(g->data + ns), ne_ - ns);
      if (h.n_dims >= 1 && h.n_dims <= kMaxDims)
        for (uint32_t d = 0; d < h.n_dims && ok; d++) ok = r.u64(&h.ne[d]);
      ok = ok && r.u32(&h.type) && r.u64(&h.offset);
    }
    if (!ok) return bch::fail(BCH_ERR_GGUF, "tensor %llu is malformed", (unsigned long long)i);
    if (h.n_dims < 1 || h.n_dims > kMaxDims)
      return bch::fail(BCH_ERR_GGUF, "tensor %s has %u dimensions", h.name.c_str(), h.n_dims);
    headers.push_back(std::move(h));
  }
  // The data section starts at the next multiple of the alignment.
  const uint64_t header_end = r.pos;
  if (header_end > UINT64_MAX - (alignment - 1)) return bch::fail(BCH_ERR_GGUF, "data section lies outside the file");
  const uint64_t data_start = (header_end + alignment - 1) / alignment * alignment;
  for (auto &h : headers) {
    uint64_t n = 1;
    for (uint32_t d = 0; d < kMaxDims; d++) {
      if (h.ne[d] == 0 || n > UINT64_MAX / h.ne[d]) return bch::fail(BCH_ERR_GGUF, "tensor %s has an invalid shape", h.name.c_str());
      n *= h.ne[d];
    }
    const auto [block, bytes] = block_of(h.type);
    if (!block) return bch::fail(BCH_ERR_GGUF, "tensor %s has unsupported type %u", h.name.c_str(), h.type);
    if (h.ne[0] % block)
      return bch::fail(BCH_ERR_GGUF, "tensor %s has rows of %llu elements, which blocks of %llu cannot divide",
                       h.name.c_str(), (unsigned long long)h.ne[0], (unsigned long long)block);
    if (n % block || n / block > UINT64_MAX / bytes) return bch::fail(BCH_ERR_GGUF, "tensor %s is too large", h.name.c_str());
    const uint64_t n_bytes = n / block * bytes;
    if (h.offset > UINT64_MAX - data_start || data_start + h.offset > UINT64_MAX - n_bytes || h.offset % alignment ||
        data_start + h.offset + n_bytes > g->size)
      return bch::fail(BCH_ERR_GGUF, "tensor %s lies outside the file", h.name.c_str());
    bch_gguf::Tensor t;
    t.name = h.name;
    t.n_dims = h.n_dims;
    for (uint32_t d = 0; d < kMaxDims; d++) t.ne[d] = h.ne[d];
    t.type = h.type;
    t.start = data_start + h.offset;
    t.end = t.start + n_bytes;
    if (!g->by_name.emplace(t.name, g->tensors.size()).second)
      return bch::fail(BCH_ERR_GGUF, "tensor %s appears twice", t.name.c_str());
    g->tensors.push_back(std::move(t));
  }
  return BCH_OK;
}

// --- model loading ------------------------------------------------------

int model_fail(const char *fmt, const char *what) { return bch::fail(BCH_ERR_MODEL, fmt, what); }

bool meta_u32(const bch_gguf *g, const std::string &key, uint32_t *out) {
  const Value *v = g->get(key.c_str());
  return v && as_u32(*v, out);
}

bool meta_f32(const bch_gguf *g, const std::string &key, float *out) {
  const Value *v = g->get(key.c_str());
  if (!v) return false;
  if (v->type == F32) {
    memcpy(out, &v->bits, 4);
    return true;
  }
  if (v->type == F64) {
    double d;
    memcpy(&d, &v->bits, 8);
    *out = (float)d;
    return true;
  }
  return false;
}

int require_u32(const bch_gguf *g, const std::string &key, uint32_t *out) {
  return meta_u32(g, key, out) ? BCH_OK : model_fail("missing or malformed metadata %s", key.c_str());
}

int require_f32(const bch_gguf *g, const std::string &key, float *out) {
  return meta_f32(g, key, out) ? BCH_OK : model_fail("missing or malformed metadata %s", key.c_str());
}

// require_tensor (lfm2.rs:850-866): the tensor with exactly the shape `want`.
int require_tensor(const bch_gguf *g, const std::string &name, std::initializer_list<uint64_t> want,
                   const bch_gguf::Tensor **out) {
  const bch_gguf::Tensor *t = g->tensor(name);
  if (!t) return model_fail("missing tensor %s", name.c_str());
  bool same = t->n_dims == want.size();
  uint32_t d = 0;
  for (uint64_t w : want) same = same && t->ne[d++] == w;
  if (!same) return model_fail("tensor %s has the wrong shape", name.c_str());
  *out = t;
  return BCH_OK;
}

int require_matrix(const bch_gguf *g, const std::string &name, uint64_t n_cols, uint64_t n_rows, bch_matrix *m) {
  const bch_gguf::Tensor *t;
  BCH_TRY(require_tensor(g, name, {n_cols, n_rows}, &t));
  if (n_rows > 0xffffffffull || n_cols > 0xffffffffull) return model_fail("tensor %s is too large", name.c_str());
  *m = bch_matrix{t->type, (uint32_t)n_rows, (uint32_t)n_cols, g->data + t->start};
  return BCH_OK;
}

int require_experts(const bch_gguf *g, const std::string &name, uint64_t n_cols, uint64_t n_rows, uint64_t n_exp,
                    bch_matrix *m) {
  const bch_gguf::Tensor *t;
  BCH_TRY(require_tensor(g, name, {n_cols, n_rows, n_exp}, &t));
  if (n_rows * n_exp > 0xffffffffull || n_cols > 0xffffffffull) return model_fail("tensor %s is too large", name.c_str());
  *m = bch_matrix{t->type, (uint32_t)(n_rows * n_exp), (uint32_t)n_cols, g->data + t->start};
  return BCH_OK;
}

int require_vector(const bch_gguf *g, const std::string &name, std::initializer_list<uint64_t> want, const float **v) {
  const bch_gguf::Tensor *t;
  BCH_TRY(require_tensor(g, name, want, &t));
  if (t->type != 0) return model_fail("tensor %s is not F32", name.c_str());
  *v = reinterpret_cast<const float *>(g->data + t->start);
  return BCH_OK;
}

std::string blk(uint32_t il, const char *suffix) { return "blk." + std::to_string(il) + "." + suffix; }

}  // namespace

extern "C" {

int bch_gguf_parse(const void *bytes, uint64_t size, bch_gguf **out) {
  if (!out) return bch::fail(BCH_ERR_ARGUMENT, "gguf_parse: no output");
  *out = nullptr;
  if (!bytes && size) return bch::fail(BCH_ERR_ARGUMENT, "gguf_parse: no bytes");
  auto *g = new bch_gguf();
  g->data = static_cast<const uint8_t *>(bytes);
  g->size = size;
  if (int rc = parse(g)) {
    delete g;
    return rc;
  }
  *out = g;
  return BCH_OK;
}

int bch_gguf_open(const char *path, bch_gguf **out) {
  if (!out || !path) return bch::fail(BCH_ERR_ARGUMENT, "gguf_open: no path");
  *out = nullptr;
  const int fd = open(path, O_RDONLY);
  if (fd < 0) return bch::fail(BCH_ERR_ARGUMENT, "cannot open %s", path);
  struct stat st;
  if (fstat(fd, &st) != 0) {
    close(fd);
    return bch::fail(BCH_ERR_ARGUMENT, "cannot stat %s", path);
  }
  void *map = nullptr;
  if (st.st_size > 0) {
    map = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (map == MAP_FAILED) {
      close(fd);
      return bch::fail(BCH_ERR_ARGUMENT, "cannot map %s", path);
    }
  }
  close(fd);
  auto *g = new bch_gguf();
  g->data = static_cast<const uint8_t *>(map);
  g->size = (uint64_t)st.st_size;
  g->map = map;
  if (int rc = parse(g)) {
    delete g;
    return rc;
  }
  *out = g;
  return BCH_OK;
}

void bch_gguf_free(bch_gguf *g) { delete g; }

const void *bch_gguf_bytes(const bch_gguf *g, uint64_t *size) {
  if (size) *size = g ? g->size : 0;
  return g ? g->data : nullptr;
}

int bch_gguf_u32(const bch_gguf *g, const char *key, uint32_t *out) {
  const Value *v = g->get(key);
  return v && as_u32(*v, out) ? BCH_OK : bch::fail(BCH_ERR_ARGUMENT, "no integer metadata %s", key);
}

int bch_gguf_f32(const bch_gguf *g, const char *key, float *out) {
  return meta_f32(g, key, out) ? BCH_OK : bch::fail(BCH_ERR_ARGUMENT, "no float metadata %s", key);
}

int bch_gguf_bool(const bch_gguf *g, const char *key, int *out) {
  const Value *v = g->get(key);
  if (!v || v->type != BOOL) return bch::fail(BCH_ERR_ARGUMENT, "no boolean metadata %s", key);
  *out = (v->bits & 0xff) != 0;
  return BCH_OK;
}

int bch_gguf_string(const bch_gguf *g, const char *key, const char **ptr, uint64_t *len) {
  const Value *v = g->get(key);
  if (!v || v->type != STRING) return bch::fail(BCH_ERR_ARGUMENT, "no string metadata %s", key);
  *ptr = reinterpret_cast<const char *>(g->data + v->start);
  *len = v->end - v->start;
  return BCH_OK;
}

int bch_gguf_array_len(const bch_gguf *g, const char *key, uint64_t *count) {
  const Value *v = g->get(key);
  if (!v || v->type != ARRAY) return bch::fail(BCH_ERR_ARGUMENT, "no array metadata %s", key);
  *count = v->count;
  return BCH_OK;
}

int bch_gguf_array_u32(const bch_gguf *g, const char *key, uint64_t index, uint32_t *out) {
  const Value *v = g->get(key);
  if (!v || v->type != ARRAY || index >= v->count || !fixed_size(v->element))
    return bch::fail(BCH_ERR_ARGUMENT, "no integer element %llu of %s", (unsigned long long)index, key);
  Value e;
  e.type = v->element;
  memcpy(&e.bits, g->data + v->start + index * (uint64_t)fixed_size(v->element), fixed_size(v->element));
  return as_u32(e, out) ? BCH_OK : bch::fail(BCH_ERR_ARGUMENT, "element %llu of %s is no u32", (unsigned long long)index, key);
}

int bch_gguf_array_string(const bch_gguf *g, const char *key, uint64_t index, const char **ptr, uint64_t *len) {
  const Value *v = g->get(key);
  if (!v || v->type != ARRAY || v->element != STRING || index >= v->count)
    return bch::fail(BCH_ERR_ARGUMENT, "no string element %llu of %s", (unsigned long long)index, key);
  // The parser checked that every string lies inside the array's data.
  Reader r{g->data, v->end, v->start};
  uint64_t s = 0, e = 0;
  for (uint64_t i = 0; i <= index; i++) r.string(&s, &e);
  *ptr = reinterpret_cast<const char *>(g->data + s);
  *len = e - s;
  return BCH_OK;
}

uint64_t bch_gguf_n_tensors(const bch_gguf *g) { return g ? g->tensors.size() : 0; }

static void fill_info(const bch_gguf *g, const bch_gguf::Tensor &t, bch_gguf_tensor_info *out) {
  out->name = t.name.c_str();
  out->n_dims = t.n_dims;
  for (uint32_t d = 0; d < kMaxDims; d++) out->ne[d] = t.ne[d];
  out->type = t.type;
  out->data = g->data + t.start;
  out->offset = t.start;
  out->bytes = t.end - t.start;
}

int bch_gguf_tensor(const bch_gguf *g, const char *name, bch_gguf_tensor_info *out) {
  const bch_gguf::Tensor *t = g->tensor(name);
  if (!t) return bch::fail(BCH_ERR_ARGUMENT, "no tensor %s", name);
  fill_info(g, *t, out);
  return BCH_OK;
}

int bch_gguf_tensor_at(const bch_gguf *g, uint64_t index, bch_gguf_tensor_info *out) {
  if (index >= g->tensors.size()) return bch::fail(BCH_ERR_ARGUMENT, "no tensor %llu", (unsigned long long)index);
  fill_info(g, g->tensors[index], out);
  return BCH_OK;
}

// lfm2::Model::load (lfm2.rs:186-232) with load_hyperparameters and
// load_layer (:737-1004).
int bch_lfm2_model_from_gguf(const bch_gguf *g, bch_lfm2_model *model, bch_lfm2_layer *layers, uint32_t max_layers) {
  if (!g || !model) return bch::fail(BCH_ERR_ARGUMENT, "lfm2_model_from_gguf: no file or model");
  const Value *arch = g->get("general.architecture");
  if (!arch || arch->type != STRING) return model_fail("missing or malformed metadata %s", "general.architecture");
  const std::string a(reinterpret_cast<const char *>(g->data + arch->start), arch->end - arch->start);
  if (a != "lfm2" && a != "lfm2moe") return model_fail("unsupported architecture %s", a.c_str());
  const bool moe = a == "lfm2moe";
  auto key = [&](const char *s) { return a + "." + s; };
  bch_lfm2_model m{};
  BCH_TRY(require_u32(g, key("block_count"), &m.n_layers));
  BCH_TRY(require_u32(g, key("embedding_length"), &m.n_embd));
  BCH_TRY(require_u32(g, key("feed_forward_length"), &m.n_ff));
  BCH_TRY(require_u32(g, key("attention.head_count"), &m.n_heads));
  BCH_TRY(require_u32(g, key("shortconv.l_cache"), &m.conv_kernel));
  BCH_TRY(require_f32(g, key("rope.freq_base"), &m.rope_theta));
  BCH_TRY(require_f32(g, key("attention.layer_norm_rms_epsilon"), &m.norm_eps));
  uint32_t n_dense = m.n_layers;
  if (moe) {
    uint32_t gating;
    BCH_TRY(require_u32(g, key("expert_gating_func"), &gating));
    if (gating != 2) return model_fail("missing or malformed metadata %s", key("expert_gating_func").c_str());
    BCH_TRY(require_u32(g, key("expert_count"), &m.n_experts));
    BCH_TRY(require_u32(g, key("expert_used_count"), &m.n_experts_used));
    BCH_TRY(require_u32(g, key("expert_feed_forward_length"), &m.n_ff_expert));
    if (!meta_u32(g, key("leading_dense_block_count"), &n_dense)) n_dense = 0;
  }
  if (m.n_layers == 0 || m.n_embd == 0 || m.n_ff == 0 || m.n_heads == 0 || m.n_embd % m.n_heads || m.conv_kernel < 2 ||
      (moe && (m.n_experts_used == 0 || m.n_experts_used > m.n_experts || m.n_ff_expert == 0)))
    return model_fail("invalid hyperparameters%s", "");
  m.head_dim = m.n_embd / m.n_heads;
  if (m.head_dim % 2) return model_fail("odd head dimension%s", "");
  if (!layers || max_layers < m.n_layers) return bch::fail(BCH_ERR_ARGUMENT, "lfm2_model_from_gguf: room for %u layers needed", m.n_layers);
  const uint64_t n = m.n_embd;
  const std::string kv_key = key("attention.head_count_kv");
  for (uint32_t il = 0; il < m.n_layers; il++) {
    bch_lfm2_layer L{};
    // One KV-head count per layer (zero for a convolution layer), or one for all.
    uint32_t n_kv = 0;
    const Value *kv = g->get(kv_key.c_str());
    if (kv && kv->type == ARRAY && kv->count == m.n_layers) {
      BCH_TRY(bch_gguf_array_u32(g, kv_key.c_str(), il, &n_kv));
    } else if (!meta_u32(g, kv_key, &n_kv)) {
      return model_fail("missing or malformed metadata %s", kv_key.c_str());
    }
    BCH_TRY(require_vector(g, blk(il, "attn_norm.weight"), {n}, &L.attn_norm));
    BCH_TRY(require_vector(g, blk(il, "ffn_norm.weight"), {n}, &L.ffn_norm));
    if (il < n_dense) {
      BCH_TRY(require_matrix(g, blk(il, "ffn_gate.weight"), n, m.n_ff, &L.gate));
      BCH_TRY(require_matrix(g, blk(il, "ffn_up.weight"), n, m.n_ff, &L.up));
      BCH_TRY(require_matrix(g, blk(il, "ffn_down.weight"), m.n_ff, n, &L.down));
    } else {
      L.is_moe = 1;
      BCH_TRY(require_matrix(g, blk(il, "ffn_gate_inp.weight"), n, m.n_experts, &L.router));
      BCH_TRY(require_vector(g, blk(il, "exp_probs_b.bias"), {m.n_experts}, &L.expert_bias));
      BCH_TRY(require_experts(g, blk(il, "ffn_gate_exps.weight"), n, m.n_ff_expert, m.n_experts, &L.gate_exps));
      BCH_TRY(require_experts(g, blk(il, "ffn_up_exps.weight"), n, m.n_ff_expert, m.n_experts, &L.up_exps));
      BCH_TRY(require_experts(g, blk(il, "ffn_down_exps.weight"), m.n_ff_expert, n, m.n_experts, &L.down_exps));
    }
    if (n_kv == 0) {
      BCH_TRY(require_vector(g, blk(il, "shortconv.conv.weight"), {m.conv_kernel, n}, &L.conv_taps));
      BCH_TRY(require_matrix(g, blk(il, "shortconv.in_proj.weight"), n, 3 * n, &L.in_proj));
      BCH_TRY(require_matrix(g, blk(il, "shortconv.out_proj.weight"), n, n, &L.out_proj));
    } else {
      if (m.n_kv_heads == 0) m.n_kv_heads = n_kv;
      if (n_kv != m.n_kv_heads || m.n_heads % n_kv)
        return bch::fail(BCH_ERR_MODEL, "layer %u has %u KV heads", il, n_kv);
      L.is_attention = 1;
      const uint64_t q = (uint64_t)m.n_heads * m.head_dim, kvd = (uint64_t)n_kv * m.head_dim;
      BCH_TRY(require_matrix(g, blk(il, "attn_q.weight"), n, q, &L.wq));
      BCH_TRY(require_matrix(g, blk(il, "attn_k.weight"), n, kvd, &L.wk));
      BCH_TRY(require_matrix(g, blk(il, "attn_v.weight"), n, kvd, &L.wv));
      BCH_TRY(require_matrix(g, blk(il, "attn_output.weight"), q, n, &L.wo));
      BCH_TRY(require_vector(g, blk(il, "attn_q_norm.weight"), {m.head_dim}, &L.q_norm));
      BCH_TRY(require_vector(g, blk(il, "attn_k_norm.weight"), {m.head_dim}, &L.k_norm));
    }
    layers[il] = L;
  }
  const bch_gguf::Tensor *e = g->tensor("token_embd.weight");
  if (!e || e->n_dims != 2) return model_fail("missing tensor %s", "token_embd.weight");
  if (e->ne[1] > 0xffffffffull) return model_fail("invalid hyperparameters%s", "");
  m.n_vocab = (uint32_t)e->ne[1];
  BCH_TRY(require_matrix(g, "token_embd.weight", n, m.n_vocab, &m.token_embd));
  BCH_TRY(require_vector(g, "token_embd_norm.weight", {n}, &m.output_norm));
  // LFM2 ties the output matrix to the embeddings unless the file has its own.
  if (g->tensor("output.weight"))
    BCH_TRY(require_matrix(g, "output.weight", n, m.n_vocab, &m.output));
  else
    m.output = m.token_embd;
  m.layers = layers;
  *model = m;
  return BCH_OK;
}

// qwen35::Model::load (qwen35.rs:186-230) with its hyperparameters and
// layers (:630-745).
int bch_qwen35_model_from_gguf(const bch_gguf *g, bch_qwen35_model *model, bch_qwen35_layer *layers,
                               uint32_t max_layers) {
  if (!g || !model) return bch::fail(BCH_ERR_ARGUMENT, "qwen35_model_from_gguf: no file or model");
  const Value *arch = g->get("general.architecture");
  if (!arch || arch->type != STRING) return model_fail("missing or malformed metadata %s", "general.architecture");
  const std::string a(reinterpret_cast<const char *>(g->data + arch->start), arch->end - arch->start);
  if (a != "qwen35") return model_fail("unsupported architecture %s", a.c_str());
  auto key = [&](const char *s) { return std::string("qwen35.") + s; };
  bch_qwen35_model m{};
  uint32_t block_count, n_nextn = 0, inner, value_length;
  BCH_TRY(require_u32(g, key("block_count"), &block_count));
  if (!meta_u32(g, key("nextn_predict_layers"), &n_nextn)) n_nextn = 0;
  if (n_nextn > block_count) return model_fail("invalid hyperparameters%s", "");
  m.n_layers = block_count - n_nextn;
  BCH_TRY(require_u32(g, key("attention.key_length"), &m.head_dim));
  BCH_TRY(require_u32(g, key("ssm.time_step_rank"), &m.n_v_heads));
  BCH_TRY(require_u32(g, key("ssm.inner_size"), &inner));
  BCH_TRY(require_u32(g, key("embedding_length"), &m.n_embd));
  BCH_TRY(require_u32(g, key("feed_forward_length"), &m.n_ff));
  BCH_TRY(require_u32(g, key("attention.head_count"), &m.n_heads));
  BCH_TRY(require_u32(g, key("attention.head_count_kv"), &m.n_kv_heads));
  BCH_TRY(require_u32(g, key("rope.dimension_count"), &m.n_rot));
  BCH_TRY(require_f32(g, key("rope.freq_base"), &m.rope_theta));
  BCH_TRY(require_f32(g, key("attention.layer_norm_rms_epsilon"), &m.norm_eps));
  BCH_TRY(require_u32(g, key("ssm.conv_kernel"), &m.conv_kernel));
  BCH_TRY(require_u32(g, key("ssm.group_count"), &m.n_k_heads));
  BCH_TRY(require_u32(g, key("ssm.state_size"), &m.k_head_dim));
  BCH_TRY(require_u32(g, key("attention.value_length"), &value_length));
  m.v_head_dim = m.n_v_heads ? inner / m.n_v_heads : 0;
  if (m.n_layers == 0 || m.n_embd == 0 || m.n_heads == 0 || m.n_kv_heads == 0 || m.n_heads % m.n_kv_heads ||
      m.head_dim == 0 || value_length != m.head_dim || m.n_rot == 0 || m.n_rot % 2 || m.n_rot > m.head_dim ||
      m.conv_kernel < 2 || m.n_k_heads == 0 || m.n_v_heads == 0 || m.n_v_heads % m.n_k_heads || m.k_head_dim == 0 ||
      m.v_head_dim == 0 || (uint64_t)m.n_v_heads * m.v_head_dim != inner ||
      (uint64_t)m.n_k_heads * m.k_head_dim * 2 + inner > 0xffffffffull ||
      (uint64_t)m.k_head_dim * m.v_head_dim > 0xffffffffull)
    return model_fail("invalid hyperparameters%s", "");
  if (!layers || max_layers < m.n_layers)
    return bch::fail(BCH_ERR_ARGUMENT, "qwen35_model_from_gguf: room for %u layers needed", m.n_layers);
  const uint64_t n = m.n_embd, value_dim = inner, conv_dim = 2ull * m.n_k_heads * m.k_head_dim + inner;
  for (uint32_t il = 0; il < m.n_layers; il++) {
    bch_qwen35_layer L{};
    if (g->tensor(blk(il, "ssm_a"))) {
      BCH_TRY(require_matrix(g, blk(il, "attn_qkv.weight"), n, conv_dim, &L.qkv));
      BCH_TRY(require_matrix(g, blk(il, "attn_gate.weight"), n, value_dim, &L.z));
      BCH_TRY(require_matrix(g, blk(il, "ssm_beta.weight"), n, m.n_v_heads, &L.beta));
      BCH_TRY(require_matrix(g, blk(il, "ssm_alpha.weight"), n, m.n_v_heads, &L.alpha));
      BCH_TRY(require_vector(g, blk(il, "ssm_conv1d.weight"), {m.conv_kernel, conv_dim}, &L.conv_taps));
      BCH_TRY(require_vector(g, blk(il, "ssm_dt.bias"), {m.n_v_heads}, &L.dt_bias));
      BCH_TRY(require_vector(g, blk(il, "ssm_a"), {m.n_v_heads}, &L.a));
      BCH_TRY(require_vector(g, blk(il, "ssm_norm.weight"), {m.v_head_dim}, &L.ssm_norm));
      BCH_TRY(require_matrix(g, blk(il, "ssm_out.weight"), value_dim, n, &L.out));
    } else {
      L.is_attention = 1;
      const uint64_t q = (uint64_t)m.n_heads * m.head_dim, kvd = (uint64_t)m.n_kv_heads * m.head_dim;
      BCH_TRY(require_matrix(g, blk(il, "attn_q.weight"), n, 2 * q, &L.wq));
      BCH_TRY(require_matrix(g, blk(il, "attn_k.weight"), n, kvd, &L.wk));
      BCH_TRY(require_matrix(g, blk(il, "attn_v.weight"), n, kvd, &L.wv));
      BCH_TRY(require_matrix(g, blk(il, "attn_output.weight"), q, n, &L.wo));
      BCH_TRY(require_vector(g, blk(il, "attn_q_norm.weight"), {m.head_dim}, &L.q_norm));
      BCH_TRY(require_vector(g, blk(il, "attn_k_norm.weight"), {m.head_dim}, &L.k_norm));
    }
    BCH_TRY(require_vector(g, blk(il, "attn_norm.weight"), {n}, &L.attn_norm));
    BCH_TRY(require_vector(g, blk(il, "post_attention_norm.weight"), {n}, &L.ffn_norm));
    BCH_TRY(require_matrix(g, blk(il, "ffn_gate.weight"), n, m.n_ff, &L.gate));
    BCH_TRY(require_matrix(g, blk(il, "ffn_up.weight"), n, m.n_ff, &L.up));
    BCH_TRY(require_matrix(g, blk(il, "ffn_down.weight"), m.n_ff, n, &L.down));
    layers[il] = L;
  }
  const bch_gguf::Tensor *e = g->tensor("token_embd.weight");
  if (!e || e->n_dims != 2) return model_fail("missing tensor %s", "token_embd.weight");
  if (e->ne[1] > 0xffffffffull) return model_fail("invalid hyperparameters%s", "");
  m.n_vocab = (uint32_t)e->ne[1];
  BCH_TRY(require_matrix(g, "token_embd.weight", n, m.n_vocab, &m.token_embd));
  BCH_TRY(require_vector(g, "output_norm.weight", {n}, &m.output_norm));
  if (g->tensor("output.weight"))
    BCH_TRY(require_matrix(g, "output.weight", n, m.n_vocab, &m.output));
  else
    m.output = m.token_embd;
  m.layers = layers;
  *model = m;
  return BCH_OK;
}

}  // extern "C"
