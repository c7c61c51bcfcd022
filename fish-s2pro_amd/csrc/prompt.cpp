// prompt.cpp -- host-side prompt preparation behind the C ABI.
//
// transpose_to_time_major (crates/fish_s2_infer/src/prompt.rs:79-103): the
// reference's prompt tensor is codebook-major (rows x cols: row 0 the
// vocabulary ids, rows 1..num_codebooks the codes, 0 at text positions);
// the token loop takes it time-major, flat[t * rows + r] = data[r * cols + t].
// Same checks and messages: rows must be non-zero, rows * cols must not
// overflow and must equal the data length, every value must fit i32.
#include <cstdint>
#include <cstdio>
#include <cstring>

#include "s2hip.h"

namespace {
void put_err(char* err, size_t cap, const char* msg) {
  if (err && cap) snprintf(err, cap, "%s", msg);
}
}  // namespace

extern "C" int32_t s2hip_transpose_to_time_major(const uint32_t* data, size_t data_len, uint32_t rows, size_t cols,
                                                 int32_t* flat_out, char* err, size_t err_cap) {
  if (rows == 0) {
    put_err(err, err_cap, "prompt rows must be non-zero");
    return 0;
  }
  size_t expected = 0;
  if (__builtin_mul_overflow(size_t(rows), cols, &expected)) {
    put_err(err, err_cap, "prompt data length overflow");
    return 0;
  }
  if (data_len != expected) {
    char msg[128];
    snprintf(msg, sizeof(msg), "prompt data length mismatch: expected %zu, got %zu", expected, data_len);
    put_err(err, err_cap, msg);
    return 0;
  }
  if (expected && (!data || !flat_out)) {
    put_err(err, err_cap, "NULL argument");
    return 0;
  }
  for (size_t i = 0; i < expected; ++i)
    if (data[i] > uint32_t(INT32_MAX)) {
      put_err(err, err_cap, "prompt token id does not fit i32");
      return 0;
    }
  for (size_t t = 0; t < cols; ++t)
    for (size_t r = 0; r < rows; ++r) flat_out[t * rows + r] = int32_t(data[r * cols + t]);
  return 1;
}
