// GGUF v3 reader (include/c0ven_gguf.h). The layout read here is ggml's file format: "GGUF", version, tensor count,
// key count (u64 each after the two u32); keys as (u64 length, bytes), a u32 value type and the value; tensor infos as
// (name, u32 dims, u64 dims..., u32 ggml type, u64 offset into the data section); the data section starts at the
// next multiple of general.alignment (32 when absent) after the infos.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdio>
#include <cstring>

#include "gguf_reader.h"

namespace c0ven {
namespace {

enum : uint32_t { kU8, kI8, kU16, kI16, kU32, kI32, kF32, kBoolT, kStringT, kArrayT, kU64, kI64, kF64 };

struct Fail : std::runtime_error {
  moe_status st;
  Fail(moe_status s, const std::string &m) : std::runtime_error(m), st(s) {}
};

// A bounds-checked walk over the mapped header.
struct Reader {
  const uint8_t *at, *end;
  const std::string &path;
  void need(uint64_t n) const {
    if ((uint64_t)(end - at) < n) throw Fail(MOE_ERROR, path + ": the GGUF header runs past the end of the file");
  }
  template <typename T>
  T take() {
    need(sizeof(T));
    T v;
    std::memcpy(&v, at, sizeof(T));
    at += sizeof(T);
    return v;
  }
  std::string text() {
    const uint64_t n = take<uint64_t>();
    need(n);
    std::string s((const char *)at, (size_t)n);
    at += n;
    return s;
  }
  int64_t integer(uint32_t t) {
    switch (t) {
      case kU8: return take<uint8_t>();
      case kI8: return take<int8_t>();
      case kU16: return take<uint16_t>();
      case kI16: return take<int16_t>();
      case kU32: return take<uint32_t>();
      case kI32: return take<int32_t>();
      case kU64: return (int64_t)take<uint64_t>();
      case kI64: return take<int64_t>();
      case kBoolT: return take<uint8_t>();
      default: throw Fail(MOE_ERROR, path + ": GGUF value type " + std::to_string(t) + " is not an integer");
    }
  }
  double number(uint32_t t) { return t == kF32 ? (double)take<float>() : take<double>(); }
  GgufMeta value(uint32_t t) {
    GgufMeta m;
    if (t == kStringT) {
      m.kind = GgufMeta::kString, m.s = text();
    } else if (t == kBoolT) {
      m.kind = GgufMeta::kBool, m.i = take<uint8_t>() != 0;
    } else if (t == kF32 || t == kF64) {
      m.kind = GgufMeta::kFloat, m.f = number(t);
    } else if (t == kArrayT) {
      const uint32_t et = take<uint32_t>();
      const uint64_t n = take<uint64_t>();
      if (et == kStringT) {
        m.kind = GgufMeta::kStrings;
        for (uint64_t i = 0; i < n; i++) m.strings.push_back(text());
      } else if (et == kF32 || et == kF64) {
        m.kind = GgufMeta::kFloats;
        need(n * (et == kF32 ? 4 : 8));
        m.floats.resize(n);
        for (auto &x : m.floats) x = number(et);
      } else if (et == kArrayT) {
        throw Fail(MOE_ERROR, path + ": nested GGUF arrays are not read");
      } else {
        m.kind = GgufMeta::kInts;
        m.ints.resize(n);
        for (auto &x : m.ints) x = integer(et);
      }
    } else {
      m.kind = GgufMeta::kInt, m.i = integer(t);
    }
    return m;
  }
};

void map_readonly(const std::string &path, int &fd, const uint8_t *&base, uint64_t &size) {
  fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) throw Fail(MOE_BAD_ARGUMENT, path + ": cannot open: " + std::strerror(errno));
  struct stat st;
  if (fstat(fd, &st) != 0) throw Fail(MOE_ERROR, path + ": cannot stat");
  size = (uint64_t)st.st_size;
  void *p = size ? mmap(nullptr, size, PROT_READ, MAP_SHARED, fd, 0) : MAP_FAILED;
  if (p == MAP_FAILED) throw Fail(MOE_ERROR, path + ": cannot map");
  base = (const uint8_t *)p;
}

Reader header(const std::string &path, const uint8_t *base, uint64_t size, uint64_t &ntensors, uint64_t &nkeys) {
  Reader r{base, base + size, path};
  if (r.take<uint32_t>() != 0x46554747u) throw Fail(MOE_BAD_ARGUMENT, path + ": not a GGUF file");
  const uint32_t version = r.take<uint32_t>();
  if (version != 3) throw Fail(MOE_BAD_ARGUMENT, path + ": GGUF version " + std::to_string(version) + ", not 3");
  ntensors = r.take<uint64_t>();
  nkeys = r.take<uint64_t>();
  return r;
}

// "<stem>-0000i-of-0000N.gguf": every shard's name; any other name is one file.
std::vector<std::string> shard_paths(const std::string &path) {
  const std::string tail = ".gguf";
  const size_t n = path.size();
  // -XXXXX-of-YYYYY.gguf is 20 characters.
  if (n > 20 && path.compare(n - tail.size(), tail.size(), tail) == 0 && path.compare(n - 14, 4, "-of-") == 0 &&
      path[n - 20] == '-') {
    const std::string a = path.substr(n - 19, 5), b = path.substr(n - 10, 5);
    if (std::all_of(a.begin(), a.end(), ::isdigit) && std::all_of(b.begin(), b.end(), ::isdigit)) {
      const int count = std::stoi(b);
      std::vector<std::string> out;
      for (int i = 1; i <= count; i++) {
        char buf[32];
        std::snprintf(buf, sizeof buf, "-%05d-of-%05d.gguf", i, count);
        out.push_back(path.substr(0, n - 20) + buf);
      }
      if (!out.empty()) return out;
    }
  }
  return {path};
}

}  // namespace

GgufFile::GgufFile(const std::string &path) {
  paths_ = shard_paths(path);
  try {
    for (uint32_t i = 0; i < paths_.size(); i++) open_one(paths_[i], i);
  } catch (...) {
    for (auto &m : maps_) {
      if (m.base) munmap((void *)m.base, m.size);
      if (m.fd >= 0) ::close(m.fd);
    }
    throw;
  }
  std::sort(tensors_.begin(), tensors_.end(), [](const GgufEntry &a, const GgufEntry &b) { return a.name < b.name; });
  for (size_t i = 0; i < tensors_.size(); i++) {
    tensors_[i].info.name = tensors_[i].name.c_str();
    if (!index_.emplace(tensors_[i].name, i).second)
      throw Fail(MOE_ERROR, "tensor " + tensors_[i].name + " appears twice");
  }
}

GgufFile::~GgufFile() {
  for (auto &m : maps_) {
    if (m.base) munmap((void *)m.base, m.size);
    if (m.fd >= 0) ::close(m.fd);
  }
}

void GgufFile::open_one(const std::string &path, uint32_t shard) {
  Mapping &m = maps_.emplace_back();
  map_readonly(path, m.fd, m.base, m.size);
  uint64_t ntensors, nkeys;
  Reader r = header(path, m.base, m.size, ntensors, nkeys);
  for (uint64_t i = 0; i < nkeys; i++) {
    std::string key = r.text();
    GgufMeta v = r.value(r.take<uint32_t>());
    if (shard == 0 || key.rfind("split.", 0) != 0) meta_.emplace(std::move(key), std::move(v));
  }
  const size_t first = tensors_.size();
  for (uint64_t i = 0; i < ntensors; i++) {
    GgufEntry e;
    e.name = r.text();
    const uint32_t nd = r.take<uint32_t>();
    if (nd < 1 || nd > 4) throw Fail(MOE_ERROR, path + ": tensor " + e.name + " has " + std::to_string(nd) + " dims");
    e.info.n_dims = nd;
    for (uint32_t d = 0; d < 4; d++) e.info.shape[d] = d < nd ? r.take<uint64_t>() : 1;
    e.info.type = r.take<uint32_t>();
    e.info.offset = r.take<uint64_t>();
    e.info.shard = shard;
    tensors_.push_back(std::move(e));
  }
  uint64_t align = 32;
  if (auto it = meta_.find("general.alignment"); it != meta_.end() && it->second.kind == GgufMeta::kInt)
    align = (uint64_t)it->second.i;
  if (align == 0) throw Fail(MOE_ERROR, path + ": general.alignment is 0");
  const uint64_t data = ((uint64_t)(r.at - m.base) + align - 1) / align * align;
  for (size_t i = first; i < tensors_.size(); i++) {
    gguf_tensor_info &t = tensors_[i].info;
    const uint64_t el = t.shape[0] * t.shape[1] * t.shape[2] * t.shape[3];
    t.offset += data;
    t.bytes = gguf_type_bytes(t.type, el);
    if (t.bytes == 0)
      throw Fail(MOE_ERROR, path + ": tensor " + tensors_[i].name + " has type " + std::to_string(t.type) +
                                " (no block size here) or a partial block");
    if (t.offset + t.bytes > m.size) throw Fail(MOE_ERROR, path + ": tensor " + tensors_[i].name + " runs past the end");
    t.data = m.base + t.offset;
  }
}

const GgufEntry *GgufFile::find(const std::string &name) const {
  auto it = index_.find(name);
  return it == index_.end() ? nullptr : &tensors_[it->second];
}

void GgufFile::release(const GgufEntry &t, uint64_t off, uint64_t bytes) const {
  const Mapping &m = maps_.at(t.info.shard);
  const uint64_t page = (uint64_t)sysconf(_SC_PAGESIZE), at = t.info.offset + off;
  const uint64_t a = (at + page - 1) / page * page, b = (at + bytes) / page * page;
  if (b > a) madvise((void *)(m.base + a), b - a, MADV_DONTNEED);
  posix_fadvise(m.fd, (off_t)at, (off_t)bytes, POSIX_FADV_DONTNEED);
}

std::string GgufFile::architecture(const std::string &path) {
  int fd = -1;
  const uint8_t *base = nullptr;
  uint64_t size = 0;
  struct Close {
    int &fd;
    const uint8_t *&base;
    uint64_t &size;
    ~Close() {
      if (base) munmap((void *)base, size);
      if (fd >= 0) ::close(fd);
    }
  } closer{fd, base, size};
  map_readonly(path, fd, base, size);
  uint64_t ntensors, nkeys;
  Reader r = header(path, base, size, ntensors, nkeys);
  for (uint64_t i = 0; i < nkeys; i++) {
    const std::string key = r.text();
    const uint32_t t = r.take<uint32_t>();
    if (key == "general.architecture" && t == kStringT) return r.text();
    (void)r.value(t);
  }
  throw Fail(MOE_BAD_ARGUMENT, path + ": no general.architecture");
}

}  // namespace c0ven

using namespace c0ven;

namespace {

std::string g_open_err;

template <typename F>
moe_status guard(const c0ven_gguf *g, F f) {
  std::string &err = g ? g->err : g_open_err;
  try {
    f();
    err.clear();
    return MOE_OK;
  } catch (const Fail &e) {
    err = e.what();
    return e.st;
  } catch (const std::exception &e) {
    err = e.what();
    return MOE_ERROR;
  }
}

const GgufMeta &key_of(const c0ven_gguf *g, const char *key) {
  if (!key) throw Fail(MOE_BAD_ARGUMENT, "null key");
  auto it = g->file->meta().find(key);
  if (it == g->file->meta().end()) throw Fail(MOE_BAD_ARGUMENT, std::string("GGUF key missing: ") + key);
  return it->second;
}

}  // namespace

extern "C" {

MOE_API moe_status gguf_open(const char *path, c0ven_gguf **out) {
  if (!path || !out) return MOE_BAD_ARGUMENT;
  *out = nullptr;
  return guard(nullptr, [&] {
    auto *g = new c0ven_gguf;
    try {
      g->file = new GgufFile(path);
    } catch (...) {
      delete g;
      throw;
    }
    *out = g;
  });
}

MOE_API void gguf_close(c0ven_gguf *g) {
  if (!g) return;
  delete g->file;
  delete g;
}

MOE_API const char *gguf_last_error(const c0ven_gguf *g) { return g ? g->err.c_str() : g_open_err.c_str(); }

MOE_API uint32_t gguf_n_files(const c0ven_gguf *g) { return g ? (uint32_t)g->file->paths().size() : 0; }
MOE_API uint64_t gguf_n_tensors(const c0ven_gguf *g) { return g ? g->file->tensors().size() : 0; }

MOE_API moe_status gguf_tensor_at(const c0ven_gguf *g, uint64_t i, gguf_tensor_info *out) {
  if (!g || !out) return MOE_BAD_ARGUMENT;
  return guard(g, [&] {
    if (i >= g->file->tensors().size()) throw Fail(MOE_BAD_ARGUMENT, "tensor index out of range");
    *out = g->file->tensors()[i].info;
  });
}

MOE_API moe_status gguf_find_tensor(const c0ven_gguf *g, const char *name, gguf_tensor_info *out) {
  if (!g || !out || !name) return MOE_BAD_ARGUMENT;
  return guard(g, [&] {
    const GgufEntry *e = g->file->find(name);
    if (!e) throw Fail(MOE_BAD_ARGUMENT, std::string("tensor missing from the file: ") + name);
    *out = e->info;
  });
}

MOE_API int gguf_has_key(const c0ven_gguf *g, const char *key) {
  return g && key && g->file->meta().count(key) ? 1 : 0;
}

MOE_API moe_status gguf_get_int(const c0ven_gguf *g, const char *key, int64_t *out) {
  if (!g || !out) return MOE_BAD_ARGUMENT;
  return guard(g, [&] {
    const GgufMeta &m = key_of(g, key);
    if (m.kind != GgufMeta::kInt && m.kind != GgufMeta::kBool)
      throw Fail(MOE_BAD_ARGUMENT, std::string("GGUF key is not an integer: ") + key);
    *out = m.i;
  });
}

MOE_API moe_status gguf_get_float(const c0ven_gguf *g, const char *key, double *out) {
  if (!g || !out) return MOE_BAD_ARGUMENT;
  return guard(g, [&] {
    const GgufMeta &m = key_of(g, key);
    if (m.kind == GgufMeta::kFloat)
      *out = m.f;
    else if (m.kind == GgufMeta::kInt)
      *out = (double)m.i;
    else
      throw Fail(MOE_BAD_ARGUMENT, std::string("GGUF key is not a number: ") + key);
  });
}

MOE_API moe_status gguf_get_string(const c0ven_gguf *g, const char *key, char *buf, uint64_t cap, uint64_t *len) {
  if (!g) return MOE_BAD_ARGUMENT;
  return guard(g, [&] {
    const GgufMeta &m = key_of(g, key);
    if (m.kind != GgufMeta::kString) throw Fail(MOE_BAD_ARGUMENT, std::string("GGUF key is not a string: ") + key);
    if (len) *len = m.s.size();
    if (buf) {
      if (cap < m.s.size() + 1) throw Fail(MOE_BAD_ARGUMENT, "buffer too small for the string");
      std::memcpy(buf, m.s.c_str(), m.s.size() + 1);
    }
  });
}

MOE_API moe_status gguf_get_ints(const c0ven_gguf *g, const char *key, int64_t *out, uint64_t cap, uint64_t *n) {
  if (!g) return MOE_BAD_ARGUMENT;
  return guard(g, [&] {
    const GgufMeta &m = key_of(g, key);
    if (m.kind != GgufMeta::kInts) throw Fail(MOE_BAD_ARGUMENT, std::string("GGUF key is not an integer array: ") + key);
    if (n) *n = m.ints.size();
    if (out) std::memcpy(out, m.ints.data(), sizeof(int64_t) * std::min<uint64_t>(cap, m.ints.size()));
  });
}

MOE_API moe_status gguf_architecture(const char *path, char *buf, uint64_t cap) {
  if (!path || !buf) return MOE_BAD_ARGUMENT;
  return guard(nullptr, [&] {
    const std::string a = GgufFile::architecture(path);
    if (cap < a.size() + 1) throw Fail(MOE_BAD_ARGUMENT, "buffer too small for the architecture");
    std::memcpy(buf, a.c_str(), a.size() + 1);
  });
}

MOE_API moe_status gguf_release(const c0ven_gguf *g, const char *name, uint64_t off, uint64_t bytes) {
  if (!g || !name) return MOE_BAD_ARGUMENT;
  return guard(g, [&] {
    const GgufEntry *e = g->file->find(name);
    if (!e) throw Fail(MOE_BAD_ARGUMENT, std::string("tensor missing from the file: ") + name);
    if (off > e->info.bytes || bytes > e->info.bytes - off) throw Fail(MOE_BAD_ARGUMENT, "range past the tensor");
    g->file->release(*e, off, bytes);
  });
}

MOE_API uint64_t gguf_type_bytes(uint32_t type, uint64_t elements) {
  uint32_t bv, bb;
  switch (type) {  // the unquantised types ggml files hold, then the block types c0ven_quant.h sizes
    case QT_F32: bv = 1, bb = 4; break;
    case QT_F16: case QT_BF16: bv = 1, bb = 2; break;
    default: bv = quant_block_values(type), bb = quant_block_bytes(type);
  }
  if (bb == 0 || bv == 0 || elements % bv) return 0;
  return elements / bv * bb;
}

}  // extern "C"
