// The GGUF v3 reader behind include/c0ven_gguf.h (host code): the files mapped read-only, metadata decoded into
// tagged values, tensor infos resolved to mapped addresses.
#pragma once

#include <cstdint>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/c0ven_gguf.h"

namespace c0ven {

struct GgufMeta {
  enum Kind { kInt, kFloat, kBool, kString, kInts, kFloats, kStrings } kind = kInt;
  int64_t i = 0;
  double f = 0.0;
  std::string s;
  std::vector<int64_t> ints;
  std::vector<double> floats;
  std::vector<std::string> strings;
};

struct GgufEntry {
  std::string name;
  gguf_tensor_info info{};
};

class GgufFile {
 public:
  explicit GgufFile(const std::string &path);
  ~GgufFile();
  GgufFile(const GgufFile &) = delete;
  GgufFile &operator=(const GgufFile &) = delete;

  const std::vector<std::string> &paths() const { return paths_; }
  const std::map<std::string, GgufMeta> &meta() const { return meta_; }
  const std::vector<GgufEntry> &tensors() const { return tensors_; }  // in name order
  const GgufEntry *find(const std::string &name) const;
  void release(const GgufEntry &t, uint64_t off, uint64_t bytes) const;

  // general.architecture from the header of one file, without the tensor table.
  static std::string architecture(const std::string &path);

 private:
  struct Mapping {
    int fd = -1;
    const uint8_t *base = nullptr;
    uint64_t size = 0;
  };
  void open_one(const std::string &path, uint32_t shard);
  std::vector<std::string> paths_;
  std::vector<Mapping> maps_;
  std::map<std::string, GgufMeta> meta_;
  std::vector<GgufEntry> tensors_;
  std::map<std::string, size_t> index_;
};

}  // namespace c0ven

struct c0ven_gguf {
  c0ven::GgufFile *file = nullptr;
  mutable std::string err;
};
