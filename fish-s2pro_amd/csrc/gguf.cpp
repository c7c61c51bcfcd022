// gguf.cpp -- GGUF v3 reader for the s2hip weight loader.
#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdint>
#include <cstring>
#include <stdexcept>

namespace s2 {
namespace {

[[noreturn]] void bad(const std::string& m) { throw std::runtime_error(m); }

struct Cursor {
  const uint8_t* p;
  const uint8_t* end;
  void need(uint64_t n) const {
    if (uint64_t(end - p) < n) bad("truncated GGUF header");
  }
  template <class T>
  T get() {
    need(sizeof(T));
    T v;
    memcpy(&v, p, sizeof(T));
    p += sizeof(T);
    return v;
  }
  std::string str() {
    const uint64_t n = get<uint64_t>();
    need(n);
    std::string s(reinterpret_cast<const char*>(p), size_t(n));
    p += n;
    return s;
  }
  void skip(uint32_t type) {
    switch (type) {
      case 0: case 1: case 7: need(1); p += 1; break;
      case 2: case 3: need(2); p += 2; break;
      case 4: case 5: case 6: need(4); p += 4; break;
      case 10: case 11: case 12: need(8); p += 8; break;
      case 8: (void)str(); break;
      case 9: {
        const uint32_t et = get<uint32_t>();
        const uint64_t n = get<uint64_t>();
        for (uint64_t k = 0; k < n; ++k) skip(et);
        break;
      }
      default: bad("unknown GGUF value type " + std::to_string(type));
    }
  }
};

// GgmlType::byte_len (crates/fish_s2_core/src/gguf.rs:233-258)
uint64_t type_bytes(uint32_t type, uint64_t n) {
  if (n > UINT64_MAX / 8) bad("tensor byte length overflows");
  switch (type) {
    case 0: case 18: return n * 4;
    case 1: case 17: case 30: return n * 2;
    case 16: return n;
    case 19: case 20: return n * 8;
    case 2: return (n + 31) / 32 * 18;
    case 3: return (n + 31) / 32 * 20;
    case 6: return (n + 31) / 32 * 22;
    case 7: return (n + 31) / 32 * 24;
    case 8: return (n + 31) / 32 * 34;
    case 9: return (n + 31) / 32 * 40;
    default: bad("unsupported GGML tensor type " + std::to_string(type));
  }
}

}  // namespace

// Element counts and byte ranges are checked for overflow, as the reference
// does with checked_mul / checked_add (crates/fish_s2_core/src/gguf.rs:161,
// 254, 351): a malformed header fails with the tensor's name instead of
// wrapping into an in-range offset.
uint64_t GgufTensor::elements() const {
  uint64_t n = 1;
  for (uint64_t d : dims)
    if (__builtin_mul_overflow(n, d, &n)) bad("tensor " + name + ": element count overflows");
  return n;
}

uint64_t ggml_row_bytes(uint32_t type, uint64_t n) {
  if ((type == 2 || type == 8) && n % 32) bad("quantised row length must be a multiple of 32");
  return type_bytes(type, n);
}

GgufFile::~GgufFile() {
  if (map_) munmap(map_, size_);
  if (fd_ >= 0) close(fd_);
}

void GgufFile::open(const std::string& path) {
  path_ = path;
  fd_ = ::open(path.c_str(), O_RDONLY);
  if (fd_ < 0) bad("cannot open " + path);
  struct stat st;
  if (fstat(fd_, &st) != 0) bad("cannot stat " + path);
  size_ = uint64_t(st.st_size);
  if (size_ < 24) bad("not a GGUF file: " + path);
  void* m = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0);
  if (m == MAP_FAILED) bad("mmap failed: " + path);
  map_ = static_cast<uint8_t*>(m);
  Cursor c{map_, map_ + size_};
  if (memcmp(c.p, "GGUF", 4) != 0) bad("not a GGUF file: " + path);
  c.p += 4;
  const uint32_t version = c.get<uint32_t>();
  if (version < 2 || version > 3) bad("unsupported GGUF version " + std::to_string(version));
  const uint64_t n_tensors = c.get<uint64_t>();
  const uint64_t n_meta = c.get<uint64_t>();
  for (uint64_t i = 0; i < n_meta; ++i) {
    const std::string key = c.str();
    GgufValue v;
    v.type = c.get<uint32_t>();
    switch (v.type) {
      case 0: v.u = c.get<uint8_t>(); break;
      case 1: v.i = c.get<int8_t>(); break;
      case 2: v.u = c.get<uint16_t>(); break;
      case 3: v.i = c.get<int16_t>(); break;
      case 4: v.u = c.get<uint32_t>(); break;
      case 5: v.i = c.get<int32_t>(); break;
      case 6: v.f = c.get<float>(); break;
      case 7: v.b = c.get<uint8_t>() != 0; break;
      case 8: v.s = c.str(); break;
      case 10: v.u = c.get<uint64_t>(); break;
      case 11: v.i = c.get<int64_t>(); break;
      case 12: v.f = c.get<double>(); break;
      case 9: {
        const uint32_t et = c.get<uint32_t>();
        const uint64_t n = c.get<uint64_t>();
        for (uint64_t k = 0; k < n; ++k) c.skip(et);
        break;
      }
      default: bad("unknown GGUF value type " + std::to_string(v.type));
    }
    meta_[key] = v;
  }
  for (uint64_t i = 0; i < n_tensors; ++i) {
    GgufTensor t;
    t.name = c.str();
    const uint32_t nd = c.get<uint32_t>();
    if (nd > 4) bad("tensor " + t.name + " has too many dimensions");
    for (uint32_t d = 0; d < nd; ++d) t.dims.push_back(c.get<uint64_t>());
    t.type = c.get<uint32_t>();
    t.offset = c.get<uint64_t>();
    index_[t.name] = tensors_.size();
    tensors_.push_back(t);
  }
  const uint64_t data_start = (uint64_t(c.p - map_) + 31) / 32 * 32;
  for (GgufTensor& t : tensors_) {
    t.bytes = type_bytes(t.type, t.elements());
    if (__builtin_add_overflow(t.offset, data_start, &t.offset) || t.offset > size_ || t.bytes > size_ - t.offset)
      bad("tensor " + t.name + " extends past file end");
    t.data = map_ + t.offset;
  }
}

const GgufTensor* GgufFile::find(const std::string& name) const {
  auto it = index_.find(name);
  return it == index_.end() ? nullptr : &tensors_[it->second];
}

const GgufTensor& GgufFile::tensor(const std::string& name) const {
  const GgufTensor* t = find(name);
  if (!t) bad("tensor not found: " + name);
  return *t;
}

const GgufValue& GgufFile::value(const std::string& key) const {
  auto it = meta_.find(key);
  if (it == meta_.end()) bad("missing " + key);
  return it->second;
}

uint32_t GgufFile::u32(const std::string& key) const {
  const GgufValue& v = value(key);
  switch (v.type) {
    case 0: case 2: case 4: case 10: return uint32_t(v.u);
    case 1: case 3: case 5: case 11: return uint32_t(v.i);
    default: bad("invalid u32 metadata " + key);
  }
}

float GgufFile::f32(const std::string& key) const {
  const GgufValue& v = value(key);
  if (v.type == 6 || v.type == 12) return float(v.f);
  bad("invalid f32 metadata " + key);
}

bool GgufFile::flag(const std::string& key) const {
  const GgufValue& v = value(key);
  if (v.type == 7) return v.b;
  bad("invalid bool metadata " + key);
}

std::string GgufFile::str(const std::string& key) const {
  const GgufValue& v = value(key);
  if (v.type == 8) return v.s;
  bad("invalid string metadata " + key);
}

}  // namespace s2
