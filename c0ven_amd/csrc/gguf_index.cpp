// The GGUF index (gguf_index.h) and the C calls of include/c0ven_gguf.h.
//
// File format (GGUF version 3, little-endian), as the format defines it:
//   "GGUF" | u32 version | u64 tensor count | u64 key count
//   key count x  { string key | u32 value tag | value }
//   tensor count x { string name | u32 dims | u64 x dims | u32 ggml type | u64 offset in the data section }
//   padding to general.alignment (32 when the key is absent) | data section
// where a string is a u64 byte count and the bytes, and an array value is a u32 element tag, a u64 count and the
// elements. Scalar tags 0..12 are u8 i8 u16 i16 u32 i32 f32 bool string array u64 i64 f64.
#include "gguf_index.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdio>
#include <cstring>
#include <numeric>

namespace c0ven {
namespace {

constexpr uint32_t kTagString = 8, kTagArray = 9, kTagBool = 7;
constexpr uint32_t kScalarBytes[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
constexpr int kMaxArrayDepth = 4;

bool is_int_tag(uint32_t t) { return t <= 5 || t == kTagBool || t == 10 || t == 11; }

// The unread bytes of the header, consumed front to back. Every read checks what is left first.
struct Cursor {
  const uint8_t *p;
  uint64_t left;
  bool skip(uint64_t n) {
    if (n > left) return false;
    p += n, left -= n;
    return true;
  }
  template <typename T>
  bool get(T &v) {
    if (sizeof(T) > left) return false;
    std::memcpy(&v, p, sizeof(T));
    return skip(sizeof(T));
  }
  bool name(std::string &s) {
    uint64_t n;
    if (!get(n) || n > left) return false;
    s.assign((const char *)p, (size_t)n);
    return skip(n);
  }
};

// Bytes a value of tag occupies at c (the tag already read); false when it is malformed or runs past the header.
bool measure(Cursor c, uint32_t tag, uint64_t &len, int depth = 0) {
  const uint64_t before = c.left;
  if (tag < 13 && kScalarBytes[tag]) {
    if (!c.skip(kScalarBytes[tag])) return false;
  } else if (tag == kTagString) {
    uint64_t n;
    if (!c.get(n) || !c.skip(n)) return false;
  } else if (tag == kTagArray && depth < kMaxArrayDepth) {
    uint32_t et;
    uint64_t n;
    if (!c.get(et) || !c.get(n)) return false;
    if (et < 13 && kScalarBytes[et]) {
      if (n > c.left / kScalarBytes[et] || !c.skip(n * kScalarBytes[et])) return false;
    } else {
      for (uint64_t i = 0; i < n; i++) {
        uint64_t el;
        if (!measure(c, et, el, depth + 1) || !c.skip(el)) return false;
      }
    }
  } else {
    return false;
  }
  len = before - c.left;
  return true;
}

int64_t scalar_int(uint32_t tag, const uint8_t *p) {
  switch (tag) {
    case 0: return *p;
    case 1: return (int8_t)*p;
    case 2: { uint16_t v; std::memcpy(&v, p, 2); return v; }
    case 3: { int16_t v; std::memcpy(&v, p, 2); return v; }
    case 4: { uint32_t v; std::memcpy(&v, p, 4); return v; }
    case 5: { int32_t v; std::memcpy(&v, p, 4); return v; }
    case kTagBool: return *p != 0;
    case 10: { uint64_t v; std::memcpy(&v, p, 8); return (int64_t)v; }
    default: { int64_t v; std::memcpy(&v, p, 8); return v; }
  }
}

struct Mapping {
  int fd = -1;
  uint8_t *base = nullptr;
  uint64_t size = 0;
};

bool map_file(const std::string &path, Mapping &m, std::string &err) {
  m.fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (m.fd < 0) {
    err = "cannot open " + path + ": " + std::strerror(errno);
    return false;
  }
  struct stat st;
  if (fstat(m.fd, &st) != 0 || st.st_size < 24) {
    err = path + " is not a GGUF file (shorter than its fixed header)";
    return false;
  }
  m.size = (uint64_t)st.st_size;
  void *p = mmap(nullptr, m.size, PROT_READ, MAP_PRIVATE, m.fd, 0);
  if (p == MAP_FAILED) {
    err = "mmap of " + path + " failed: " + std::strerror(errno);
    return false;
  }
  m.base = (uint8_t *)p;
  return true;
}

void unmap(Mapping &m) {
  if (m.base) munmap(m.base, m.size);
  if (m.fd >= 0) ::close(m.fd);
  m = Mapping{};
}

// The fixed header; leaves c at the first key.
bool fixed_header(const Mapping &m, const std::string &path, Cursor &c, uint64_t &ntensor, uint64_t &nkv,
                  std::string &err) {
  c = Cursor{m.base, m.size};
  uint32_t version = 0;
  if (std::memcmp(m.base, "GGUF", 4) != 0) {
    err = path + ": bad magic (not a GGUF file)";
    return false;
  }
  c.skip(4);
  if (!c.get(version) || !c.get(ntensor) || !c.get(nkv)) return false;
  if (version != 3) {
    err = path + ": GGUF version " + std::to_string(version) + " (this reader takes version 3)";
    return false;
  }
  return true;
}

// Walks the key/value section, handing each pair to f; false on a malformed pair.
template <typename F>
bool walk_kv(Cursor &c, uint64_t nkv, const std::string &path, std::string &err, F &&f) {
  for (uint64_t i = 0; i < nkv; i++) {
    std::string key;
    uint32_t tag;
    uint64_t len;
    if (!c.name(key) || !c.get(tag) || !measure(c, tag, len)) {
      err = path + ": key/value pair " + std::to_string(i) + " is malformed or cut short";
      return false;
    }
    f(std::move(key), tag, c.p, len);
    c.skip(len);
  }
  return true;
}

// "<stem>-NNNNN-of-MMMMM.gguf": the stem and the file count, or count 0 for a single file.
uint32_t split_set(const std::string &path, std::string &stem) {
  const size_t n = path.size();
  static const size_t kSuffix = sizeof("-00001-of-00002.gguf") - 1;
  if (n < kSuffix) return 0;
  unsigned idx = 0, cnt = 0;
  char tail[8] = {0};
  if (std::sscanf(path.c_str() + n - kSuffix, "-%5u-of-%5u%7s", &idx, &cnt, tail) != 3 || std::strcmp(tail, ".gguf"))
    return 0;
  if (idx < 1 || cnt < 1 || idx > cnt) return 0;
  stem = path.substr(0, n - kSuffix);
  return cnt;
}

}  // namespace

GgufIndex::~GgufIndex() {
  for (Mapped &f : files) {
    Mapping m{f.fd, f.base, f.size};
    unmap(m);
  }
}

bool GgufIndex::open(const std::string &path) {
  std::string stem;
  const uint32_t nsplit = split_set(path, stem);
  std::vector<std::string> paths;
  if (nsplit == 0) {
    paths.push_back(path);
  } else {
    for (uint32_t i = 1; i <= nsplit; i++) {
      char tail[32];
      std::snprintf(tail, sizeof tail, "-%05u-of-%05u.gguf", i, nsplit);
      paths.push_back(stem + tail);
    }
  }
  struct Pending {
    std::string name;
    gguf_tensor_info info;
  };
  std::vector<Pending> pend;
  for (uint32_t fi = 0; fi < paths.size(); fi++) {
    Mapping m;
    files.push_back(Mapped{paths[fi]});
    if (!map_file(paths[fi], m, err)) {
      if (m.fd >= 0) ::close(m.fd);
      return false;
    }
    Mapped &f = files.back();
    f.fd = m.fd, f.base = m.base, f.size = m.size;
    Cursor c{nullptr, 0};
    uint64_t ntensor = 0, nkv = 0;
    const std::string cut = paths[fi] + ": the header is cut short";
    if (!fixed_header(m, paths[fi], c, ntensor, nkv, err)) {
      if (err.empty()) err = cut;
      return false;
    }
    int64_t align = 32;
    const bool ok = walk_kv(c, nkv, paths[fi], err, [&](std::string key, uint32_t tag, const uint8_t *val,
                                                        uint64_t len) {
      if (key == "general.alignment" && is_int_tag(tag)) align = scalar_int(tag, val);
      // Later files of a set repeat the split.* bookkeeping with their own numbers: the first file's stands.
      if (fi > 0 && key.compare(0, 6, "split.") == 0) return;
      kv.push_back(KvView{std::move(key), tag, val, len, fi});
    });
    if (!ok) return false;
    if (align <= 0 || (align & (align - 1)) || align > (1 << 20)) {
      err = paths[fi] + ": general.alignment " + std::to_string(align) + " is not a power of two";
      return false;
    }
    f.align = (uint32_t)align;
    const size_t first = pend.size();
    for (uint64_t t = 0; t < ntensor; t++) {
      Pending p{};
      uint32_t nd = 0;
      if (!c.name(p.name) || !c.get(nd) || nd < 1 || nd > 4) {
        err = paths[fi] + ": tensor record " + std::to_string(t) + " is malformed or cut short";
        return false;
      }
      gguf_tensor_info &ti = p.info;
      ti.n_dims = nd;
      for (int d = 0; d < 4; d++) ti.shape[d] = 1;
      for (uint32_t d = 0; d < nd; d++)
        if (!c.get(ti.shape[d])) {
          err = cut;
          return false;
        }
      if (!c.get(ti.type) || !c.get(ti.offset)) {
        err = cut;
        return false;
      }
      ti.shard = fi;
      pend.push_back(std::move(p));
    }
    const uint64_t header_end = m.size - c.left;
    f.data_at = (header_end + f.align - 1) / f.align * f.align;
    for (size_t i = first; i < pend.size(); i++) {
      gguf_tensor_info &ti = pend[i].info;
      uint64_t elements = 1;
      for (int d = 0; d < 4; d++)
        if (__builtin_mul_overflow(elements, ti.shape[d], &elements)) {
          err = paths[fi] + ": tensor " + pend[i].name + " has more elements than 64 bits count";
          return false;
        }
      ti.bytes = gguf_type_bytes(ti.type, elements);
      if (ti.bytes == 0 && elements != 0) {
        err = paths[fi] + ": tensor " + pend[i].name + " has type " + std::to_string(ti.type) +
              ", unknown here, or a length that is not whole blocks";
        return false;
      }
      uint64_t at;
      if (ti.offset % f.align || __builtin_add_overflow(f.data_at, ti.offset, &at) || at > m.size ||
          ti.bytes > m.size - at) {
        err = paths[fi] + ": tensor " + pend[i].name + " lies outside the file or off the alignment";
        return false;
      }
      ti.offset = at;  // from here on: the byte offset in its file
      ti.data = m.base + at;
    }
  }
  // Keys: sorted, the first file's value of a repeated key kept (stable sort keeps file order among equals).
  std::stable_sort(kv.begin(), kv.end(), [](const KvView &a, const KvView &b) { return a.key < b.key; });
  kv.erase(std::unique(kv.begin(), kv.end(), [](const KvView &a, const KvView &b) { return a.key == b.key; }),
           kv.end());
  std::vector<size_t> order(pend.size());
  std::iota(order.begin(), order.end(), 0);
  std::sort(order.begin(), order.end(), [&](size_t a, size_t b) { return pend[a].name < pend[b].name; });
  for (size_t i = 1; i < order.size(); i++)
    if (pend[order[i]].name == pend[order[i - 1]].name) {
      err = "tensor name " + pend[order[i]].name + " is defined more than once";
      return false;
    }
  names.reserve(order.size());
  tensors.reserve(order.size());
  for (size_t i : order) {
    names.push_back(std::move(pend[i].name));
    tensors.push_back(pend[i].info);
  }
  for (size_t i = 0; i < tensors.size(); i++) tensors[i].name = names[i].c_str();
  return true;
}

const KvView *GgufIndex::key(const char *k) const {
  auto it = std::lower_bound(kv.begin(), kv.end(), k, [](const KvView &a, const char *b) { return a.key < b; });
  return it != kv.end() && it->key == k ? &*it : nullptr;
}

const gguf_tensor_info *GgufIndex::tensor(const char *name) const {
  auto it = std::lower_bound(tensors.begin(), tensors.end(), name,
                             [](const gguf_tensor_info &a, const char *b) { return std::strcmp(a.name, b) < 0; });
  return it != tensors.end() && std::strcmp(it->name, name) == 0 ? &*it : nullptr;
}

// The whole pages inside the range go back to the kernel; the private read-only mapping refaults them from the file.
bool GgufIndex::drop_pages(const gguf_tensor_info &t, uint64_t off, uint64_t bytes) const {
  const uint64_t page = (uint64_t)sysconf(_SC_PAGESIZE);
  const uintptr_t lo = (uintptr_t)t.data + off, hi = lo + bytes;
  const uintptr_t a = (lo + page - 1) / page * page, b = hi / page * page;
  if (b <= a) return true;
  if (madvise((void *)a, b - a, MADV_DONTNEED) != 0) {
    err = std::string("madvise failed: ") + std::strerror(errno);
    return false;
  }
  return true;
}

bool gguf_read_architecture(const std::string &path, std::string &arch, std::string &err) {
  Mapping m;
  if (!map_file(path, m, err)) {
    unmap(m);
    return false;
  }
  Cursor c{nullptr, 0};
  uint64_t nt = 0, nkv = 0;
  bool found = false;
  bool ok = fixed_header(m, path, c, nt, nkv, err) && walk_kv(c, nkv, path, err, [&](std::string key, uint32_t tag,
                                                                                      const uint8_t *val, uint64_t) {
              if (!found && tag == kTagString && key == "general.architecture") {
                KvView v{key, tag, val, 0, 0};
                found = kv_text(v, arch);
              }
            });
  unmap(m);
  if (ok && !found) err = path + " names no general.architecture";
  if (!ok && err.empty()) err = path + ": the header is cut short";
  return ok && found;
}

bool kv_int(const KvView &v, int64_t &out) {
  if (!is_int_tag(v.tag)) return false;
  out = scalar_int(v.tag, v.val);
  return true;
}

bool kv_real(const KvView &v, double &out) {
  if (v.tag == 6) {
    float f;
    std::memcpy(&f, v.val, 4);
    out = f;
  } else if (v.tag == 12) {
    std::memcpy(&out, v.val, 8);
  } else {
    int64_t i;
    if (!kv_int(v, i)) return false;
    out = (double)i;
  }
  return true;
}

bool kv_text(const KvView &v, std::string &out) {
  if (v.tag != kTagString) return false;
  uint64_t n;
  std::memcpy(&n, v.val, 8);
  out.assign((const char *)v.val + 8, (size_t)n);
  return true;
}

bool kv_int_array(const KvView &v, std::vector<int64_t> &out) {
  if (v.tag != kTagArray) return false;
  uint32_t et;
  uint64_t n;
  std::memcpy(&et, v.val, 4);
  std::memcpy(&n, v.val + 4, 8);
  if (!is_int_tag(et)) return false;
  out.resize(n);
  for (uint64_t i = 0; i < n; i++) out[i] = scalar_int(et, v.val + 12 + i * kScalarBytes[et]);
  return true;
}

}  // namespace c0ven

using c0ven::KvView;

namespace {

thread_local std::string t_open_msg;

moe_status fail(const c0ven_gguf *g, moe_status st, std::string m) {
  (g ? g->msg : t_open_msg) = std::move(m);
  return st;
}

moe_status done(const c0ven_gguf *g) {
  (g ? g->msg : t_open_msg).clear();
  return MOE_OK;
}

const KvView *lookup(const c0ven_gguf *g, const char *key) {
  if (!key) {
    g->msg = "null key";
    return nullptr;
  }
  const KvView *v = g->ix.key(key);
  if (!v) g->msg = std::string("the file has no key ") + key;
  return v;
}

}  // namespace

extern "C" {

MOE_API moe_status gguf_open(const char *path, c0ven_gguf **out) {
  if (!path || !out) return fail(nullptr, MOE_BAD_ARGUMENT, "null path or out");
  *out = nullptr;
  c0ven_gguf *g = new (std::nothrow) c0ven_gguf;
  if (!g) return fail(nullptr, MOE_ERROR, "out of host memory");
  bool ok;
  try {
    ok = g->ix.open(path);
  } catch (const std::exception &e) {  // allocation failures of the index's containers
    g->ix.err = e.what();
    ok = false;
  }
  if (!ok) {
    const std::string m = g->ix.err;
    delete g;  // unmaps whatever was mapped
    return fail(nullptr, MOE_BAD_ARGUMENT, m);
  }
  *out = g;
  return done(nullptr);
}

MOE_API void gguf_close(c0ven_gguf *g) { delete g; }

MOE_API const char *gguf_last_error(const c0ven_gguf *g) { return g ? g->msg.c_str() : t_open_msg.c_str(); }

MOE_API uint32_t gguf_n_files(const c0ven_gguf *g) { return g ? (uint32_t)g->ix.files.size() : 0; }
MOE_API uint64_t gguf_n_tensors(const c0ven_gguf *g) { return g ? g->ix.tensors.size() : 0; }

MOE_API moe_status gguf_tensor_at(const c0ven_gguf *g, uint64_t i, gguf_tensor_info *out) {
  if (!g || !out) return MOE_BAD_ARGUMENT;
  if (i >= g->ix.tensors.size()) return fail(g, MOE_BAD_ARGUMENT, "tensor index past the table");
  *out = g->ix.tensors[i];
  return done(g);
}

MOE_API moe_status gguf_find_tensor(const c0ven_gguf *g, const char *name, gguf_tensor_info *out) {
  if (!g || !out || !name) return MOE_BAD_ARGUMENT;
  const gguf_tensor_info *t = g->ix.tensor(name);
  if (!t) return fail(g, MOE_BAD_ARGUMENT, std::string("no tensor named ") + name);
  *out = *t;
  return done(g);
}

MOE_API int gguf_has_key(const c0ven_gguf *g, const char *key) { return g && key && g->ix.key(key) ? 1 : 0; }

MOE_API moe_status gguf_get_int(const c0ven_gguf *g, const char *key, int64_t *out) {
  if (!g || !out) return MOE_BAD_ARGUMENT;
  const KvView *v = lookup(g, key);
  if (!v) return MOE_BAD_ARGUMENT;
  if (!c0ven::kv_int(*v, *out)) return fail(g, MOE_BAD_ARGUMENT, std::string(key) + " holds no integer");
  return done(g);
}

MOE_API moe_status gguf_get_float(const c0ven_gguf *g, const char *key, double *out) {
  if (!g || !out) return MOE_BAD_ARGUMENT;
  const KvView *v = lookup(g, key);
  if (!v) return MOE_BAD_ARGUMENT;
  if (!c0ven::kv_real(*v, *out)) return fail(g, MOE_BAD_ARGUMENT, std::string(key) + " holds no number");
  return done(g);
}

MOE_API moe_status gguf_get_string(const c0ven_gguf *g, const char *key, char *buf, uint64_t cap, uint64_t *len) {
  if (!g) return MOE_BAD_ARGUMENT;
  const KvView *v = lookup(g, key);
  if (!v) return MOE_BAD_ARGUMENT;
  std::string s;
  if (!c0ven::kv_text(*v, s)) return fail(g, MOE_BAD_ARGUMENT, std::string(key) + " holds no string");
  if (len) *len = s.size();
  if (buf) {
    if (cap <= s.size()) return fail(g, MOE_BAD_ARGUMENT, std::string("the string of ") + key + " needs a larger buffer");
    std::memcpy(buf, s.c_str(), s.size() + 1);
  }
  return done(g);
}

MOE_API moe_status gguf_get_ints(const c0ven_gguf *g, const char *key, int64_t *out, uint64_t cap, uint64_t *n) {
  if (!g) return MOE_BAD_ARGUMENT;
  const KvView *v = lookup(g, key);
  if (!v) return MOE_BAD_ARGUMENT;
  std::vector<int64_t> a;
  if (!c0ven::kv_int_array(*v, a)) return fail(g, MOE_BAD_ARGUMENT, std::string(key) + " holds no integer array");
  if (n) *n = a.size();
  if (out && cap) std::memcpy(out, a.data(), sizeof(int64_t) * std::min<uint64_t>(cap, a.size()));
  return done(g);
}

MOE_API moe_status gguf_architecture(const char *path, char *buf, uint64_t cap) {
  if (!path || !buf) return fail(nullptr, MOE_BAD_ARGUMENT, "null path or buffer");
  std::string arch, err;
  if (!c0ven::gguf_read_architecture(path, arch, err)) return fail(nullptr, MOE_BAD_ARGUMENT, err);
  if (cap <= arch.size()) return fail(nullptr, MOE_BAD_ARGUMENT, "the architecture name needs a larger buffer");
  std::memcpy(buf, arch.c_str(), arch.size() + 1);
  return done(nullptr);
}

MOE_API moe_status gguf_release(const c0ven_gguf *g, const char *name, uint64_t off, uint64_t bytes) {
  if (!g || !name) return MOE_BAD_ARGUMENT;
  const gguf_tensor_info *t = g->ix.tensor(name);
  if (!t) return fail(g, MOE_BAD_ARGUMENT, std::string("no tensor named ") + name);
  if (off > t->bytes || bytes > t->bytes - off) return fail(g, MOE_BAD_ARGUMENT, "range reaches past the tensor");
  if (!g->ix.drop_pages(*t, off, bytes)) return fail(g, MOE_ERROR, g->ix.err);
  return done(g);
}

MOE_API uint64_t gguf_type_bytes(uint32_t type, uint64_t elements) {
  // Unquantised element types first; block types take their sizes from c0ven_quant.h.
  const uint32_t per = type == QT_F32 || type == QT_F16 || type == QT_BF16 ? 1 : quant_block_values(type);
  const uint32_t bytes = type == QT_F32 ? 4 : type == QT_F16 || type == QT_BF16 ? 2 : quant_block_bytes(type);
  if (!bytes || !per || elements % per) return 0;
  uint64_t out;
  return __builtin_mul_overflow(elements / per, (uint64_t)bytes, &out) ? 0 : out;
}

}  // extern "C"
