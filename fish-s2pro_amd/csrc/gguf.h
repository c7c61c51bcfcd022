// gguf.h -- GGUF v3 reader (memory mapped) for the s2hip weight loader.
//
// Format as read by the reference (crates/fish_s2_core/src/gguf.rs:35-120,
// 326-453): magic "GGUF", u32 version, u64 tensor count, u64 metadata count,
// typed metadata values, tensor infos {name, u32 n_dims, u64 dims (ne0 first),
// u32 type, u64 offset}, tensor data starting at the next 32-byte boundary.
#pragma once

#include <stdint.h>

#include <map>
#include <string>
#include <vector>

namespace s2 {

struct GgufTensor {
  std::string name;
  std::vector<uint64_t> dims;
  uint32_t type = 0;
  uint64_t offset = 0;  // absolute file offset
  uint64_t bytes = 0;
  const uint8_t* data = nullptr;
  uint64_t elements() const;
};

struct GgufValue {
  uint32_t type = 0;
  uint64_t u = 0;
  int64_t i = 0;
  double f = 0.0;
  bool b = false;
  std::string s;
};

class GgufFile {
 public:
  GgufFile() = default;
  GgufFile(const GgufFile&) = delete;
  GgufFile& operator=(const GgufFile&) = delete;
  ~GgufFile();

  void open(const std::string& path);  // throws std::runtime_error
  const GgufTensor* find(const std::string& name) const;
  const GgufTensor& tensor(const std::string& name) const;
  const GgufValue& value(const std::string& key) const;
  uint32_t u32(const std::string& key) const;
  float f32(const std::string& key) const;
  bool flag(const std::string& key) const;
  std::string str(const std::string& key) const;
  const std::vector<GgufTensor>& tensors() const { return tensors_; }

 private:
  int fd_ = -1;
  uint8_t* map_ = nullptr;
  uint64_t size_ = 0;
  std::string path_;
  std::map<std::string, GgufValue> meta_;
  std::vector<GgufTensor> tensors_;
  std::map<std::string, size_t> index_;
};

uint64_t ggml_row_bytes(uint32_t type, uint64_t n);  // throws for unsupported types

}  // namespace s2
