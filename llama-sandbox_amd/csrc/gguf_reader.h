// GGUF reader for the expert tensors of one MoE layer (host code).
//
// A GGUF file (versions 2 and 3) is: "GGUF", u32 version, u64 tensor count,
// u64 key/value count, the key/value pairs (u64-length strings, u32 value
// type, value), the tensor infos (name, u32 n_dims, u64 ne[n_dims], u32 ggml
// type, u64 offset from the data section), padding to general.alignment
// (default 32), then the data.  A model split over several files names them
// <stem>-00001-of-000NN.gguf ...; the metadata is read from the first, the
// tensors from whichever file holds them (moe-serv/make_stub.py:150-219
// reads the same layout).
//
// The files are mapped read-only and every read is bounds-checked: the
// file is input, not trusted.  Only the pieces the MoE layer needs are
// interpreted: the `<arch>.*` keys of the expert block and the tensors
// blk.N.ffn_{gate,up,down}_exps.weight / _shexp.weight, which
// nano-glm/lib/models/deepseek4/model.h:366-372 and glm_dsa/model.h:251-257
// bind by the same names.
#pragma once

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

namespace gguf {

enum : uint32_t { T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 };
constexpr uint32_t GGML_TYPE_F32 = 0, GGML_TYPE_F16 = 1, GGML_TYPE_BF16 = 30;
constexpr uint32_t GGML_TYPE_MXFP4 = 39;  // 32 weights in 17 bytes
constexpr int MAX_DIMS = 4;

struct kv {
  std::string key;
  uint32_t type = 0;
  uint64_t at = 0;        // file offset of the value (of the first element for arrays)
  uint32_t arr_type = 0;  // element type (arrays)
  uint64_t arr_n = 0;     // element count (arrays)
};

struct tensor {
  std::string name;
  uint32_t n_dims = 0;
  uint64_t ne[MAX_DIMS] = {1, 1, 1, 1};
  uint32_t type = 0;
  uint64_t rel = 0;  // offset inside the data section
  int shard = 0;
};

struct mapped {
  int fd = -1;
  const uint8_t *p = nullptr;
  size_t n = 0;
  uint64_t data = 0;  // file offset of the data section
  ~mapped() {
    if (p) munmap(const_cast<uint8_t *>(p), n);
    if (fd >= 0) close(fd);
  }
};

inline size_t scalar_size(uint32_t t) {
  switch (t) {
    case T_U8: case T_I8: case T_BOOL: return 1;
    case T_U16: case T_I16: return 2;
    case T_U32: case T_I32: case T_F32: return 4;
    case T_U64: case T_I64: case T_F64: return 8;
    default: return 0;
  }
}

class reader {
 public:
  reader(const uint8_t *p, size_t n) : p_(p), n_(n) {}
  bool ok() const { return ok_; }
  uint64_t pos() const { return pos_; }
  bool need(uint64_t k) {
    if (!ok_ || k > n_ - pos_) ok_ = false;
    return ok_;
  }
  uint32_t u32() {
    uint32_t v = 0;
    if (need(4)) memcpy(&v, p_ + pos_, 4), pos_ += 4;
    return v;
  }
  uint64_t u64() {
    uint64_t v = 0;
    if (need(8)) memcpy(&v, p_ + pos_, 8), pos_ += 8;
    return v;
  }
  void skip(uint64_t k) {
    if (need(k)) pos_ += k;
  }
  std::string str(uint64_t max_len) {
    const uint64_t len = u64();
    if (!ok_ || len > max_len || !need(len)) {
      ok_ = false;
      return {};
    }
    std::string s(reinterpret_cast<const char *>(p_ + pos_), len);
    pos_ += len;
    return s;
  }

 private:
  const uint8_t *p_;
  size_t n_;
  uint64_t pos_ = 0;
  bool ok_ = true;
};

// One model: its first file's metadata and the tensor infos of all files.
struct model {
  std::vector<std::unique_ptr<mapped>> files;
  std::vector<kv> kvs;
  std::vector<tensor> tensors;
  std::string err;

  bool fail(const std::string &m) {
    if (err.empty()) err = m;
    return false;
  }

  const kv *find(const std::string &key) const {
    for (const kv &k : kvs)
      if (k.key == key) return &k;
    return nullptr;
  }
  const tensor *find_tensor(const std::string &name) const {
    for (const tensor &t : tensors)
      if (t.name == name) return &t;
    return nullptr;
  }

  // Integer key of any integer type (or bool) into *v; false if absent or not an integer.
  bool get_int(const std::string &key, int64_t *v) const {
    const kv *k = find(key);
    if (!k) return false;
    const uint8_t *a = files[0]->p + k->at;
    switch (k->type) {
      case T_U8: *v = a[0]; return true;
      case T_I8: *v = (int8_t)a[0]; return true;
      case T_BOOL: *v = a[0] != 0; return true;
      case T_U16: { uint16_t x; memcpy(&x, a, 2); *v = x; return true; }
      case T_I16: { int16_t x; memcpy(&x, a, 2); *v = x; return true; }
      case T_U32: { uint32_t x; memcpy(&x, a, 4); *v = x; return true; }
      case T_I32: { int32_t x; memcpy(&x, a, 4); *v = x; return true; }
      case T_U64: { uint64_t x; memcpy(&x, a, 8); *v = x > (uint64_t)INT64_MAX ? INT64_MAX : (int64_t)x; return true; }
      case T_I64: { int64_t x; memcpy(&x, a, 8); *v = x; return true; }
      default: return false;
    }
  }
  bool get_f32(const std::string &key, float *v) const {
    const kv *k = find(key);
    if (!k) return false;
    if (k->type == T_F32) return memcpy(v, files[0]->p + k->at, 4), true;
    if (k->type == T_F64) {
      double d;
      memcpy(&d, files[0]->p + k->at, 8);
      *v = (float)d;
      return true;
    }
    return false;
  }
  bool get_str(const std::string &key, std::string *v) const {
    const kv *k = find(key);
    if (!k || k->type != T_STR) return false;
    uint64_t len;
    memcpy(&len, files[0]->p + k->at, 8);
    v->assign(reinterpret_cast<const char *>(files[0]->p + k->at + 8), len);
    return true;
  }
  // Element i of an f32 array key; false if absent, not f32 or too short.
  bool get_f32_at(const std::string &key, uint64_t i, float *v) const {
    const kv *k = find(key);
    if (!k || k->type != T_ARR || k->arr_type != T_F32 || i >= k->arr_n) return false;
    memcpy(v, files[0]->p + k->at + 4 * i, 4);
    return true;
  }

  // Bytes of a tensor of this type, or 0 when the type is not one this
  // reader sizes (MXFP4 experts; f32 / f16 / bf16 router weights and bias).
  static uint64_t bytes_of(const tensor &t) {
    uint64_t n;
    if (t.type == GGML_TYPE_MXFP4) {
      if (t.ne[0] % 32) return 0;
      n = t.ne[0] / 32 * 17;
    } else if (t.type == GGML_TYPE_F32) {
      if (t.ne[0] > UINT64_MAX / 4) return 0;
      n = t.ne[0] * 4;
    } else if (t.type == GGML_TYPE_F16 || t.type == GGML_TYPE_BF16) {
      if (t.ne[0] > UINT64_MAX / 2) return 0;
      n = t.ne[0] * 2;
    } else {
      return 0;
    }
    for (int d = 1; d < MAX_DIMS; d++) {
      if (t.ne[d] && n > UINT64_MAX / t.ne[d]) return 0;
      n *= t.ne[d];
    }
    return n;
  }

  // Pointer to a tensor's bytes after checking that they lie inside its file.
  const uint8_t *data_of(const tensor &t) {
    const mapped &f = *files[t.shard];
    const uint64_t n = bytes_of(t);
    if (n == 0) return fail("tensor " + t.name + " has a type or shape this reader does not size"), nullptr;
    if (t.rel > f.n || f.data > f.n - t.rel || n > f.n - f.data - t.rel)
      return fail("tensor " + t.name + " runs past the end of its file"), nullptr;
    return f.p + f.data + t.rel;
  }

  // An f32 / f16 / bf16 tensor of `count` elements as f32 into out.
  bool read_f32(const tensor &t, uint64_t count, std::vector<float> &out) {
    uint64_t ne = 1;
    for (int d = 0; d < MAX_DIMS && ne <= count; d++) ne = t.ne[d] <= count ? ne * t.ne[d] : count + 1;
    if (ne != count) return fail("tensor " + t.name + " does not hold " + std::to_string(count) + " elements");
    if (t.type != GGML_TYPE_F32 && t.type != GGML_TYPE_F16 && t.type != GGML_TYPE_BF16)
      return fail("tensor " + t.name + " is not f32, f16 or bf16 (type " + std::to_string(t.type) + ")");
    const uint8_t *p = data_of(t);
    if (!p) return false;
    out.resize(count);
    for (uint64_t i = 0; i < count; i++) {
      if (t.type == GGML_TYPE_F32) {
        memcpy(&out[i], p + 4 * i, 4);
      } else {
        uint16_t h;
        memcpy(&h, p + 2 * i, 2);
        out[i] = t.type == GGML_TYPE_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
      }
    }
    return true;
  }

  static float bf16_to_f32(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
  }
  // IEEE binary16 -> binary32, exact (subnormals, inf and NaN included).
  static float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31, ex = (h >> 10) & 31, man = h & 1023;
    uint32_t u;
    if (ex == 31) {
      u = sign | 0x7f800000u | (man << 13);
    } else if (ex) {
      u = sign | ((ex + 112) << 23) | (man << 13);
    } else {
      float f = (float)man * 0x1p-24f;  // subnormal or zero: exact in f32
      memcpy(&u, &f, 4);
      u |= sign;
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
  }

  bool open_one(const std::string &path, bool first) {
    auto m = std::make_unique<mapped>();
    m->fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (m->fd < 0) return fail("cannot open " + path);
    struct stat st;
    if (fstat(m->fd, &st) != 0 || st.st_size < 24) return fail(path + ": not a GGUF file (too short)");
    m->n = (size_t)st.st_size;
    void *p = mmap(nullptr, m->n, PROT_READ, MAP_SHARED, m->fd, 0);
    if (p == MAP_FAILED) return fail("cannot map " + path);
    m->p = static_cast<const uint8_t *>(p);
    reader r(m->p, m->n);
    if (memcmp(m->p, "GGUF", 4) != 0) return fail(path + ": not a GGUF file (magic)");
    r.skip(4);
    const uint32_t version = r.u32();
    if (version != 2 && version != 3) return fail(path + ": GGUF version " + std::to_string(version) + " (2 or 3)");
    const uint64_t n_tensors = r.u64(), n_kv = r.u64();
    uint64_t align = 32;
    for (uint64_t i = 0; i < n_kv && r.ok(); i++) {
      kv k;
      k.key = r.str(1 << 16);
      k.type = r.u32();
      if (!r.ok()) break;
      k.at = r.pos();
      if (k.type == T_STR) {
        r.str(UINT64_MAX >> 1);
      } else if (k.type == T_ARR) {
        k.arr_type = r.u32();
        k.arr_n = r.u64();
        k.at = r.pos();
        if (k.arr_type == T_STR) {
          for (uint64_t j = 0; j < k.arr_n && r.ok(); j++) r.str(UINT64_MAX >> 1);
        } else {
          const size_t es = scalar_size(k.arr_type);
          if (es == 0) return fail(path + ": key " + k.key + " is an array of type " + std::to_string(k.arr_type));
          if (k.arr_n > (UINT64_MAX >> 4)) return fail(path + ": key " + k.key + " has a bad length");
          r.skip(k.arr_n * es);
        }
      } else {
        const size_t s = scalar_size(k.type);
        if (s == 0) return fail(path + ": key " + k.key + " has value type " + std::to_string(k.type));
        r.skip(s);
      }
      if (!r.ok()) break;
      if (k.key == "general.alignment") {
        if (k.type != T_U32) return fail(path + ": general.alignment is not a u32");
        uint32_t a;
        memcpy(&a, m->p + k.at, 4);
        if (a == 0 || (a & (a - 1))) return fail(path + ": general.alignment is not a power of two");
        align = a;
      }
      if (first) kvs.push_back(std::move(k));
    }
    if (!r.ok()) return fail(path + ": truncated key/value section");
    const int shard = (int)files.size();
    for (uint64_t i = 0; i < n_tensors && r.ok(); i++) {
      tensor t;
      t.name = r.str(1 << 12);
      t.n_dims = r.u32();
      if (!r.ok()) break;
      if (t.n_dims < 1 || t.n_dims > MAX_DIMS) return fail(path + ": tensor " + t.name + " has " +
                                                           std::to_string(t.n_dims) + " dims");
      for (uint32_t d = 0; d < t.n_dims; d++) t.ne[d] = r.u64();
      t.type = r.u32();
      t.rel = r.u64();
      t.shard = shard;
      if (r.ok() && t.rel % align) return fail(path + ": tensor " + t.name + " is not aligned");
      tensors.push_back(std::move(t));
    }
    if (!r.ok()) return fail(path + ": truncated tensor infos");
    m->data = (r.pos() + align - 1) / align * align;
    if (m->data > m->n) return fail(path + ": no data section");
    files.push_back(std::move(m));
    return true;
  }

  // Open a model: one file, or every file of a split whose first is `path`.
  bool open(const std::string &path) {
    if (!open_one(path, true)) return false;
    const std::string tag = "-00001-of-";
    const size_t at = path.rfind(tag);
    if (at == std::string::npos) return true;
    const size_t dot = path.find(".gguf", at);
    if (dot == std::string::npos) return true;
    const std::string count = path.substr(at + tag.size(), dot - at - tag.size());
    if (count.empty() || count.size() > 5 || count.find_first_not_of("0123456789") != std::string::npos)
      return true;
    const int total = std::stoi(count);
    for (int i = 2; i <= total; i++) {
      char part[16];
      snprintf(part, sizeof(part), "-%05d-of-", i);
      if (!open_one(path.substr(0, at) + part + path.substr(at + tag.size()), false)) return false;
    }
    return true;
  }
};

}  // namespace gguf
