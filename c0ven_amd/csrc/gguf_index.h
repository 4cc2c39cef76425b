// The GGUF index behind include/c0ven_gguf.h (host code).
//
// One validating pass per file builds a flat index: every key/value pair is kept as a view of its encoded bytes in
// the read-only mapping (decoded only when a getter asks for it), every tensor as a gguf_tensor_info whose data
// pointer is already resolved into its file's mapping. The reader throws nothing: each step returns false and leaves
// a message in the index, which the C calls turn into a moe_status.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "../../include/c0ven_gguf.h"

namespace c0ven {

// A metadata value as it sits in the file: its type tag and the bytes that follow the tag (for an array: the
// element type and count, then the elements).
struct KvView {
  std::string key;
  uint32_t tag = 0;
  const uint8_t *val = nullptr;
  uint64_t len = 0;  // bytes of the encoded value
  uint32_t file = 0;
};

struct GgufIndex {
  struct Mapped {
    std::string path;
    int fd = -1;
    uint8_t *base = nullptr;
    uint64_t size = 0;
    uint64_t data_at = 0;  // start of this file's data section
    uint32_t align = 32;
  };
  std::vector<Mapped> files;
  std::vector<KvView> kv;                 // sorted by key, first file's value of a key kept
  std::vector<gguf_tensor_info> tensors;  // sorted by name
  std::vector<std::string> names;         // owns the names tensors[].name points at
  mutable std::string err;

  ~GgufIndex();
  // Maps path and, when its name ends in -NNNNN-of-MMMMM.gguf, every file of the set; false with err set on failure.
  bool open(const std::string &path);
  const KvView *key(const char *k) const;
  const gguf_tensor_info *tensor(const char *name) const;
  bool drop_pages(const gguf_tensor_info &t, uint64_t off, uint64_t bytes) const;
};

// general.architecture of one file, from its key/value section only.
bool gguf_read_architecture(const std::string &path, std::string &arch, std::string &err);

// Integers (and bools) of a value, widened to int64; false when the value is of another kind.
bool kv_int(const KvView &v, int64_t &out);
bool kv_real(const KvView &v, double &out);
bool kv_text(const KvView &v, std::string &out);
bool kv_int_array(const KvView &v, std::vector<int64_t> &out);

}  // namespace c0ven

struct c0ven_gguf {
  c0ven::GgufIndex ix;
  mutable std::string msg;
};
