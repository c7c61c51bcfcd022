// s2_oracle.cpp -- CPU restatement of the reference's Slow-AR + Fast-AR loop.
//
// TEST INFRASTRUCTURE ONLY: the parity checker for the HIP path and the timed
// CPU baseline.  Only tests/, __graft_entry__.smoke() and bench.py's
// cpu_baseline leg load it.  Build with -ffp-contract=off and without
// -ffast-math: every sum below is a sequential left-to-right f32 sum, exactly
// as Rust's Iterator::sum / fold compute it, and Rust never fuses a*b+c.
//
// Paths cited as crates/<crate>/src/<file>:<line> are in stevenke1981/fish-s2pro.

#include "s2_oracle.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <condition_variable>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

namespace {

struct OracleError : std::runtime_error {
  explicit OracleError(const std::string& m) : std::runtime_error(m) {}
};

[[noreturn]] void fail(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  throw OracleError(buf);
}

void copy_err(const std::exception& e, char* err, size_t cap) {
  if (err && cap) {
    snprintf(err, cap, "%s", e.what());
  }
}

// ---------------------------------------------------------------------------
// f16 <-> f32 (crates/fish_s2_infer/src/tensor.rs:266-325)
// ---------------------------------------------------------------------------
float f16_to_f32(uint16_t bits) {
  uint32_t sign = uint32_t(bits & 0x8000u) << 16;
  uint32_t exponent = (bits >> 10) & 0x1fu;
  uint32_t fraction = bits & 0x03ffu;
  uint32_t out;
  if (exponent == 0 && fraction == 0) {
    out = sign;
  } else if (exponent == 0) {
    // subnormal: fraction * 2^-24, exact in f32 (tensor.rs:272-279)
    float v = float(fraction) * 5.9604644775390625e-08f;
    return sign ? -v : v;
  } else if (exponent == 0x1f && fraction == 0) {
    out = sign | 0x7f800000u;
  } else if (exponent == 0x1f) {
    out = sign | 0x7f800000u | (fraction << 13);
  } else {
    out = sign | ((exponent + 112u) << 23) | (fraction << 13);
  }
  float f;
  memcpy(&f, &out, 4);
  return f;
}

uint16_t f32_to_f16(float value) {
  uint32_t bits;
  memcpy(&bits, &value, 4);
  uint16_t sign = uint16_t((bits >> 16) & 0x8000u);
  int32_t exponent = int32_t((bits >> 23) & 0xffu);
  uint32_t mantissa = bits & 0x007fffffu;
  if (exponent == 0xff) {
    return mantissa == 0 ? uint16_t(sign | 0x7c00u) : uint16_t(sign | 0x7e00u);
  }
  int32_t half_exp = exponent - 127 + 15;
  if (half_exp >= 0x1f) return uint16_t(sign | 0x7c00u);
  if (half_exp <= 0) {
    if (half_exp < -10) return sign;
    uint32_t m = mantissa | 0x00800000u;
    uint32_t shift = uint32_t(14 - half_exp);
    uint32_t rounded = m + ((1u << (shift - 1)) - 1) + ((m >> shift) & 1u);
    return uint16_t(sign | uint16_t(rounded >> shift));
  }
  uint32_t rounded = mantissa + 0x00000fffu + ((mantissa >> 13) & 1u);
  if (rounded & 0x00800000u) {
    int32_t next_exp = half_exp + 1;
    if (next_exp >= 0x1f) return uint16_t(sign | 0x7c00u);
    return uint16_t(sign | uint16_t(next_exp << 10));
  }
  return uint16_t(sign | uint16_t(half_exp << 10) | uint16_t(rounded >> 13));
}

// ---------------------------------------------------------------------------
// GGML block formats.  The reference only knows their byte sizes
// (crates/fish_s2_core/src/gguf.rs:233-258): Q8_0 = 34 B / 32 elements
// {f16 d; i8 q[32]}, Q4_0 = 18 B / 32 elements {f16 d; u8 qs[16]} with
// element j in the low nibble of qs[j] and element 16+j in the high nibble.
// Dequantisation x = f32(d) * q is exact in f32.
// ---------------------------------------------------------------------------
enum : uint32_t { T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q8_0 = 8 };

size_t row_bytes(uint32_t type, size_t n) {
  switch (type) {
    case T_F32: return n * 4;
    case T_F16: return n * 2;
    case T_Q8_0: return (n / 32) * 34;
    case T_Q4_0: return (n / 32) * 18;
    default: fail("unsupported ggml type %u", type);
  }
}

void dequant_row(const uint8_t* src, uint32_t type, size_t n, float* out) {
  switch (type) {
    case T_F32:
      memcpy(out, src, n * 4);
      return;
    case T_F16:
      for (size_t i = 0; i < n; ++i) {
        uint16_t b;
        memcpy(&b, src + 2 * i, 2);
        out[i] = f16_to_f32(b);
      }
      return;
    case T_Q8_0: {
      if (n % 32) fail("Q8_0 row length %zu not a multiple of 32", n);
      for (size_t blk = 0; blk < n / 32; ++blk) {
        const uint8_t* b = src + blk * 34;
        uint16_t dbits;
        memcpy(&dbits, b, 2);
        float d = f16_to_f32(dbits);
        for (int j = 0; j < 32; ++j) out[blk * 32 + j] = float(int8_t(b[2 + j])) * d;
      }
      return;
    }
    case T_Q4_0: {
      if (n % 32) fail("Q4_0 row length %zu not a multiple of 32", n);
      for (size_t blk = 0; blk < n / 32; ++blk) {
        const uint8_t* b = src + blk * 18;
        uint16_t dbits;
        memcpy(&dbits, b, 2);
        float d = f16_to_f32(dbits);
        for (int j = 0; j < 16; ++j) {
          int lo = int(b[2 + j] & 0x0f) - 8;
          int hi = int(b[2 + j] >> 4) - 8;
          out[blk * 32 + j] = float(lo) * d;
          out[blk * 32 + 16 + j] = float(hi) * d;
        }
      }
      return;
    }
    default:
      fail("unsupported ggml type %u", type);
  }
}

// ---------------------------------------------------------------------------
// Thread pool: row-parallel work like Rayon's par_iter_mut over output rows
// (crates/fish_s2_infer/src/backend.rs:64-71).  Scheduling never changes the
// per-element arithmetic order.
// ---------------------------------------------------------------------------
class Pool {
 public:
  explicit Pool(unsigned n) : n_(n ? n : 1) {
    for (unsigned i = 1; i < n_; ++i) workers_.emplace_back([this] { loop(); });
  }
  ~Pool() {
    {
      std::lock_guard<std::mutex> g(mu_);
      stop_ = true;
      ++gen_;
    }
    cv_.notify_all();
    for (auto& t : workers_) t.join();
  }
  unsigned size() const { return n_; }
  // fn(begin, end) over [0, n) in chunks of `grain`
  void run(size_t n, size_t grain, const std::function<void(size_t, size_t)>& fn) {
    if (n == 0) return;
    if (n_ == 1 || n <= grain) {
      fn(0, n);
      return;
    }
    {
      std::lock_guard<std::mutex> g(mu_);
      fn_ = &fn;
      total_ = n;
      grain_ = grain;
      next_.store(0);
      pending_ = n_ - 1;
      ++gen_;
    }
    cv_.notify_all();
    work();
    std::unique_lock<std::mutex> lk(mu_);
    done_cv_.wait(lk, [this] { return pending_ == 0; });
    fn_ = nullptr;
  }

 private:
  void work() {
    for (;;) {
      size_t b = next_.fetch_add(grain_);
      if (b >= total_) break;
      (*fn_)(b, std::min(total_, b + grain_));
    }
  }
  void loop() {
    uint64_t seen = 0;
    for (;;) {
      {
        std::unique_lock<std::mutex> lk(mu_);
        cv_.wait(lk, [&] { return gen_ != seen; });
        seen = gen_;
        if (stop_) return;
      }
      work();
      {
        std::lock_guard<std::mutex> g(mu_);
        if (--pending_ == 0) done_cv_.notify_all();
      }
    }
  }
  unsigned n_;
  std::vector<std::thread> workers_;
  std::mutex mu_;
  std::condition_variable cv_, done_cv_;
  const std::function<void(size_t, size_t)>* fn_ = nullptr;
  size_t total_ = 0, grain_ = 1;
  std::atomic<size_t> next_{0};
  unsigned pending_ = 0;
  uint64_t gen_ = 0;
  bool stop_ = false;
};

// ---------------------------------------------------------------------------
// Ops
// ---------------------------------------------------------------------------

// rms_norm_f32 (crates/fish_s2_infer/src/backend.rs:84-102):
// ms = (sum x^2) / n; scale = 1 / sqrt(ms + eps); y = (x * scale) * w.
void rms_norm(const float* x, const float* w, size_t n, float eps, float* out) {
  if (n == 0) fail("rms_norm input is empty");
  float sum = 0.0f;
  for (size_t i = 0; i < n; ++i) sum += x[i] * x[i];
  float ms = sum / float(n);
  float scale = 1.0f / std::sqrt(ms + eps);
  for (size_t i = 0; i < n; ++i) out[i] = x[i] * scale * w[i];
}

// rms_norm_heads_f32 (backend.rs:104-121)
void rms_norm_heads(const float* x, const float* w, size_t n, size_t hd, float eps, float* out) {
  if (hd == 0 || n % hd) fail("head RMSNorm input length %zu is not a multiple of head_dim %zu", n, hd);
  for (size_t h = 0; h < n / hd; ++h) rms_norm(x + h * hd, w, hd, eps, out + h * hd);
}

// apply_rope_normal (crates/fish_s2_infer/src/attention.rs:172-206): adjacent
// pairs, theta = pos / base^(pair/hd) with libm powf, sin/cos via libm.
void rope_normal(float* v, size_t len, size_t hd, size_t pos, float base) {
  if (hd == 0 || hd % 2) fail("RoPE head_dim must be non-zero and even, got %zu", hd);
  if (len % hd) fail("RoPE values length %zu is not a multiple of head_dim %zu", len, hd);
  if (!(base > 0.0f)) fail("RoPE base must be positive");
  for (size_t h = 0; h < len / hd; ++h) {
    float* head = v + h * hd;
    for (size_t pair = 0; pair < hd; pair += 2) {
      float theta = float(pos) / powf(base, float(pair) / float(hd));
      float s = sinf(theta), c = cosf(theta);
      float x0 = head[pair], x1 = head[pair + 1];
      head[pair] = x0 * c - x1 * s;
      head[pair + 1] = x0 * s + x1 * c;
    }
  }
}

float dot(const float* a, const float* b, size_t n) {
  float s = 0.0f;
  for (size_t i = 0; i < n; ++i) s += a[i] * b[i];
  return s;
}

// gqa_decode_attention + softmax_in_place (attention.rs:208-247, 296-309).
// keys/values: [token][kv_head][head_dim].
void gqa_attention(const float* q, const float* k, const float* v, size_t H, size_t Hkv, size_t hd,
                   size_t T, float scale, float* out) {
  if (Hkv == 0 || H % Hkv) fail("invalid GQA split: heads=%zu, kv_heads=%zu", H, Hkv);
  if (hd == 0 || T == 0) fail("invalid attention dims: head_dim=%zu, token_count=%zu", hd, T);
  size_t rep = H / Hkv;
  std::vector<float> scores(T);
  for (size_t i = 0; i < H * hd; ++i) out[i] = 0.0f;
  for (size_t h = 0; h < H; ++h) {
    size_t kvh = h / rep;
    const float* qh = q + h * hd;
    for (size_t t = 0; t < T; ++t) scores[t] = dot(qh, k + (t * Hkv + kvh) * hd, hd) * scale;
    float mx = -INFINITY;
    for (size_t t = 0; t < T; ++t) mx = std::fmax(mx, scores[t]);  // f32::max ignores NaN
    float sum = 0.0f;
    for (size_t t = 0; t < T; ++t) {
      scores[t] = expf(scores[t] - mx);
      sum += scores[t];
    }
    for (size_t t = 0; t < T; ++t) scores[t] /= sum;
    float* o = out + h * hd;
    for (size_t t = 0; t < T; ++t) {
      const float* vt = v + (t * Hkv + kvh) * hd;
      for (size_t d = 0; d < hd; ++d) o[d] += scores[t] * vt[d];
    }
  }
}

// swiglu_split, Slow (crates/fish_s2_infer/src/slow_ar.rs:1215-1232): g * sigmoid(g) * u
void swiglu_slow(const float* g, const float* u, size_t n, float* out) {
  for (size_t i = 0; i < n; ++i) {
    float sig = 1.0f / (1.0f + expf(-g[i]));
    out[i] = g[i] * sig * u[i];
  }
}

// swiglu_split, Fast (crates/fish_s2_infer/src/fast_ar.rs:472-485): g / (1 + e^-g) * u
void swiglu_fast(const float* g, const float* u, size_t n, float* out) {
  for (size_t i = 0; i < n; ++i) out[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
}

// SeededRng (crates/fish_s2_infer/src/sampling.rs:34-52)
double rng_next_unit(uint64_t* state) {
  *state = *state * 6364136223846793005ull + 1ull;
  uint64_t mantissa = (*state >> 11) & ((1ull << 53) - 1);
  return double(mantissa) / double(1ull << 53);
}

// apply_softmax (sampling.rs:202-225)
void apply_softmax(std::vector<float>& p, float temperature) {
  if (p.empty()) return;
  float mx = -INFINITY;
  for (float v : p) mx = std::fmax(mx, v);
  float sum = 0.0f;
  for (float& v : p) {
    if (temperature > 0.0f) {
      v = expf((v - mx) / temperature);
    } else {
      v = std::fabs(v - mx) < 1e-6f ? 1.0f : 0.0f;
    }
    sum += v;
  }
  if (sum > 0.0f) {
    for (float& v : p) v /= sum;
  }
}

// How far one draw of sample_token lies from the nearest point where a
// perturbation of the logits could change its result (all in the sampler's
// own f32 values; a diagnostic for parity checks, not part of the reference):
//   draw: distance of the draw target from the cumulative-sum boundaries
//         around the chosen item (sample_discrete, sampling.rs:227-241);
//   cut:  distance of the top-p cumulative sums from top_p around the cut
//         (sampling.rs:172-181), +inf when top_p never cuts;
//   tie:  logit gap between the chosen item and its neighbours in the stable
//         descending order (sampling.rs:132-160), +inf without neighbours.
struct SampleMargins {
  float draw = INFINITY, cut = INFINITY, tie = INFINITY;
};

// sample_token (sampling.rs:120-200) + sample_discrete (sampling.rs:227-241)
uint32_t sample_token(const float* logits, size_t n, float temperature, float top_p, int32_t top_k,
                      int64_t always_include, uint64_t* rng, SampleMargins* mg = nullptr) {
  if (n == 0) return 0;
  struct Item {
    float v;
    uint32_t id;
  };
  std::vector<Item> items(n);
  for (size_t i = 0; i < n; ++i) items[i] = {logits[i], uint32_t(i)};
  auto desc = [](const Item& a, const Item& b) { return a.v > b.v; };  // stable, descending
  std::stable_sort(items.begin(), items.end(), desc);
  std::vector<Item> all;
  if (mg) all = items;
  size_t k = top_k > 0 ? std::min(size_t(top_k), n) : n;
  items.resize(k);
  if (always_include >= 0 && size_t(always_include) < n) {
    float fl = logits[always_include];
    bool present = false;
    for (const Item& it : items) present |= (it.id == uint32_t(always_include));
    if (fl > -1e30f && !present) items.push_back({fl, uint32_t(always_include)});
  }
  std::stable_sort(items.begin(), items.end(), desc);
  size_t m = items.size();
  if (m == 0) return 0;
  std::vector<float> probs(m);
  for (size_t i = 0; i < m; ++i) probs[i] = items[i].v;
  apply_softmax(probs, temperature);
  long always_pos = -1;
  if (always_include >= 0) {
    for (size_t i = 0; i < m; ++i)
      if (items[i].id == uint32_t(always_include)) {
        always_pos = long(i);
        break;
      }
  }
  size_t p_idx = 0;
  float cumsum = 0.0f, prev = 0.0f;
  bool cut = false;
  while (p_idx < m) {
    prev = cumsum;
    cumsum += probs[p_idx];
    p_idx += 1;
    if (cumsum >= top_p) {
      cut = true;
      break;
    }
  }
  if (mg) {
    if (cut)
      mg->cut = std::min(cumsum - top_p, p_idx > 1 ? top_p - prev : INFINITY);
    else if (m > 0)
      mg->cut = top_p - cumsum;
  }
  if (p_idx == 0) p_idx = 1;
  if (always_pos >= 0 && size_t(always_pos) >= p_idx) p_idx = size_t(always_pos) + 1;
  items.resize(p_idx);
  probs.resize(p_idx);
  float sum_p = 0.0f;
  for (float v : probs) sum_p += v;
  if (sum_p > 0.0f) {
    for (float& v : probs) v /= sum_p;
  }
  double draw = rng_next_unit(rng);
  float target = std::min(std::max(float(draw), 0.0f), 1.0f - 1e-7f);
  float cs = 0.0f;
  size_t chosen = probs.size() - 1;
  float lo = 0.0f, hi = 0.0f;
  bool hit = false;
  for (size_t i = 0; i < probs.size(); ++i) {
    lo = cs;
    cs += probs[i];
    if (target < cs) {
      chosen = i;
      hi = cs;
      hit = true;
      break;
    }
  }
  if (mg) {
    mg->draw = hit ? std::min(target - lo, hi - target) : target - cs;
    const uint32_t id = items[chosen].id;
    for (size_t j = 0; j < all.size(); ++j) {
      if (all[j].id != id) continue;
      if (j > 0) mg->tie = std::min(mg->tie, std::fabs(all[j - 1].v - all[j].v));
      if (j + 1 < all.size()) mg->tie = std::min(mg->tie, std::fabs(all[j + 1].v - all[j].v));
      break;
    }
  }
  return items[chosen].id;
}

// Linear over n_tok inputs: y[t][o] = sum_i x[t][i] * W[o][i] with W stored as
// GGML rows (backend.rs:55-82, tensor.rs:220-264).  Each dot product is a
// sequential f32 sum in i; tokens are independent chains, so interleaving
// them (the inner loop over t is vectorised by the compiler) keeps the order.
void linear_multi(Pool& pool, const float* x, size_t n_tok, const uint8_t* w, uint32_t type,
                  size_t in, size_t out, float* y) {
  const size_t rb = row_bytes(type, in);
  constexpr size_t TB = 8;
  // x transposed per block of 8 tokens: xt[blk][i][8]
  size_t nblk = (n_tok + TB - 1) / TB;
  std::vector<float> xt;
  if (n_tok > 1) {
    xt.assign(nblk * in * TB, 0.0f);
    for (size_t t = 0; t < n_tok; ++t)
      for (size_t i = 0; i < in; ++i) xt[((t / TB) * in + i) * TB + (t % TB)] = x[t * in + i];
  }
  pool.run(out, n_tok > 1 ? 4 : 16, [&](size_t r0, size_t r1) {
    std::vector<float> wrow(in * 4);
    size_t r = r0;
    if (n_tok == 1) {
      for (; r + 4 <= r1; r += 4) {
        for (int k = 0; k < 4; ++k) dequant_row(w + (r + k) * rb, type, in, wrow.data() + k * in);
        const float *w0 = wrow.data(), *w1 = w0 + in, *w2 = w1 + in, *w3 = w2 + in;
        float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
        for (size_t i = 0; i < in; ++i) {
          s0 += x[i] * w0[i];
          s1 += x[i] * w1[i];
          s2 += x[i] * w2[i];
          s3 += x[i] * w3[i];
        }
        y[r] = s0;
        y[r + 1] = s1;
        y[r + 2] = s2;
        y[r + 3] = s3;
      }
      for (; r < r1; ++r) {
        dequant_row(w + r * rb, type, in, wrow.data());
        y[r] = dot(x, wrow.data(), in);
      }
      return;
    }
    for (; r < r1; ++r) {
      dequant_row(w + r * rb, type, in, wrow.data());
      const float* wr = wrow.data();
      for (size_t b = 0; b < nblk; ++b) {
        float acc[TB] = {0, 0, 0, 0, 0, 0, 0, 0};
        const float* xb = xt.data() + b * in * TB;
        for (size_t i = 0; i < in; ++i) {
          const float wi = wr[i];
          for (size_t t = 0; t < TB; ++t) acc[t] += xb[i * TB + t] * wi;
        }
        for (size_t t = 0; t < TB && b * TB + t < n_tok; ++t) y[(b * TB + t) * out + r] = acc[t];
      }
    }
  });
}

// ---------------------------------------------------------------------------
// GGUF v3 reader (crates/fish_s2_core/src/gguf.rs:35-120, 326-453)
// ---------------------------------------------------------------------------
struct TensorInfo {
  std::string name;
  std::vector<uint64_t> dims;
  uint32_t type = 0;
  uint64_t rel_offset = 0;
  uint64_t abs_offset = 0;
  size_t bytes = 0;
  const uint8_t* data = nullptr;
  uint64_t elements() const {
    uint64_t n = 1;
    for (uint64_t d : dims) n *= d;
    return n;
  }
};

struct MetaValue {
  uint32_t type = 0;
  uint64_t u = 0;
  int64_t i = 0;
  double f = 0;
  bool b = false;
  std::string s;
};

size_t type_byte_len(uint32_t type, uint64_t n) {
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
    default: fail("unsupported GGML tensor type: %u", type);
  }
}

struct Gguf {
  int fd = -1;
  uint8_t* map = nullptr;
  size_t size = 0;
  std::string path;
  uint32_t version = 0;
  std::map<std::string, MetaValue> meta;
  std::vector<TensorInfo> tensors;
  std::map<std::string, size_t> by_name;
  uint64_t data_start = 0;

  ~Gguf() {
    if (map) munmap(map, size);
    if (fd >= 0) close(fd);
  }

  struct Cur {
    const uint8_t* p;
    const uint8_t* end;
    void need(size_t n) {
      if (size_t(end - p) < n) fail("unexpected end of GGUF header");
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
      uint64_t n = get<uint64_t>();
      need(n);
      std::string s(reinterpret_cast<const char*>(p), n);
      p += n;
      return s;
    }
  };

  static void skip_value(Cur& c, uint32_t t) {
    switch (t) {
      case 0: case 1: case 7: c.need(1); c.p += 1; break;
      case 2: case 3: c.need(2); c.p += 2; break;
      case 4: case 5: case 6: c.need(4); c.p += 4; break;
      case 10: case 11: case 12: c.need(8); c.p += 8; break;
      case 8: c.str(); break;
      case 9: {
        uint32_t et = c.get<uint32_t>();
        uint64_t n = c.get<uint64_t>();
        for (uint64_t i = 0; i < n; ++i) skip_value(c, et);
        break;
      }
      default: fail("unknown GGUF value type: %u", t);
    }
  }

  void open_file(const char* p) {
    path = p;
    fd = ::open(p, O_RDONLY);
    if (fd < 0) fail("cannot open %s", p);
    struct stat st;
    if (fstat(fd, &st) != 0) fail("cannot stat %s", p);
    size = size_t(st.st_size);
    if (size < 24) fail("not a GGUF file: %s", p);
    map = static_cast<uint8_t*>(mmap(nullptr, size, PROT_READ, MAP_SHARED, fd, 0));
    if (map == MAP_FAILED) {
      map = nullptr;
      fail("mmap failed for %s", p);
    }
    Cur c{map, map + size};
    if (memcmp(c.p, "GGUF", 4) != 0) fail("not a GGUF file: %s", p);
    c.p += 4;
    version = c.get<uint32_t>();
    uint64_t n_tensors = c.get<uint64_t>();
    uint64_t n_kv = c.get<uint64_t>();
    for (uint64_t i = 0; i < n_kv; ++i) {
      std::string key = c.str();
      MetaValue v;
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
          uint32_t et = c.get<uint32_t>();
          uint64_t n = c.get<uint64_t>();
          for (uint64_t k = 0; k < n; ++k) skip_value(c, et);
          break;
        }
        default: fail("unknown GGUF value type: %u", v.type);
      }
      meta[key] = v;
    }
    for (uint64_t i = 0; i < n_tensors; ++i) {
      TensorInfo t;
      t.name = c.str();
      uint32_t nd = c.get<uint32_t>();
      for (uint32_t d = 0; d < nd; ++d) t.dims.push_back(c.get<uint64_t>());
      t.type = c.get<uint32_t>();
      t.rel_offset = c.get<uint64_t>();
      by_name[t.name] = tensors.size();
      tensors.push_back(t);
    }
    uint64_t pos = uint64_t(c.p - map);
    data_start = (pos + 31) / 32 * 32;
    for (TensorInfo& t : tensors) {
      t.bytes = type_byte_len(t.type, t.elements());
      t.abs_offset = data_start + t.rel_offset;
      if (t.abs_offset + t.bytes > size)
        fail("tensor %s extends past file end: %llu > %zu", t.name.c_str(),
             (unsigned long long)(t.abs_offset + t.bytes), size);
      t.data = map + t.abs_offset;
    }
  }

  const TensorInfo& tensor(const std::string& n) const {
    auto it = by_name.find(n);
    if (it == by_name.end()) fail("tensor not found: %s", n.c_str());
    return tensors[it->second];
  }
  bool has(const std::string& n) const { return by_name.count(n) != 0; }
  const MetaValue& m(const std::string& k) const {
    auto it = meta.find(k);
    if (it == meta.end()) fail("missing %s", k.c_str());
    return it->second;
  }
  uint32_t mu32(const std::string& k) const {
    const MetaValue& v = m(k);
    if (v.type == 4 || v.type == 0 || v.type == 2 || v.type == 10) return uint32_t(v.u);
    if (v.type == 5 || v.type == 1 || v.type == 3 || v.type == 11) return uint32_t(v.i);
    fail("invalid u32 metadata %s", k.c_str());
  }
  float mf32(const std::string& k) const {
    const MetaValue& v = m(k);
    if (v.type == 6 || v.type == 12) return float(v.f);
    fail("invalid f32 metadata %s", k.c_str());
  }
  bool mbool(const std::string& k) const {
    const MetaValue& v = m(k);
    if (v.type == 7) return v.b;
    fail("invalid bool metadata %s", k.c_str());
  }
};

// ---------------------------------------------------------------------------
// Model
// ---------------------------------------------------------------------------
struct Lin {
  const TensorInfo* t = nullptr;
  size_t in = 0, out = 0;
};

struct SlowLayer {
  std::vector<float> attn_norm, q_norm, k_norm, ffn_norm;
  Lin wqkv, wo, w1, w2, w3;
};

struct FastLayer {
  std::vector<float> attn_norm, ffn_norm;
  Lin wqkv, wo, w1, w2, w3;
  // faithful mode: f32 expansion at load time (fast_ar.rs:202-213)
  std::vector<float> wqkv32, wo32, w132, w232, w332;
};

std::vector<float> load_vec(const Gguf& g, const std::string& name, size_t n) {
  const TensorInfo& t = g.tensor(name);
  if (t.elements() != n) fail("%s: expected %zu elements, got %llu", name.c_str(), n,
                              (unsigned long long)t.elements());
  std::vector<float> v(n);
  dequant_row(t.data, t.type, n, v.data());
  return v;
}

Lin load_lin(const Gguf& g, const std::string& name, size_t in, size_t out) {
  const TensorInfo& t = g.tensor(name);
  if (t.dims.size() != 2 || t.dims[0] != in || t.dims[1] != out)
    fail("%s dimensions mismatch: expected [%zu, %zu]", name.c_str(), in, out);
  if (t.type != T_F16 && t.type != T_Q8_0 && t.type != T_Q4_0 && t.type != T_F32)
    fail("%s: unsupported linear type %u", name.c_str(), t.type);
  Lin l;
  l.t = &t;
  l.in = in;
  l.out = out;
  return l;
}

}  // namespace

struct orc_model {
  Gguf g;
  orc_spec spec{};
  uint32_t im_end = 0;
  uint32_t flags = 0;
  std::unique_ptr<Pool> pool;
  std::vector<SlowLayer> slow;
  std::vector<FastLayer> fast;
  const TensorInfo* emb = nullptr;     // [vocab][dim] f16
  const TensorInfo* cb_emb = nullptr;  // [cb_rows][dim] f16
  const TensorInfo* fast_emb = nullptr;
  std::vector<float> norm, fast_norm;
  Lin fast_out;
  uint32_t max_seq = 0, n_past = 0;
  std::vector<float> kc, vc;  // [layer][tok][kvh][hd] (attention.rs:151-169)
  // incremental Fast-AR state
  std::vector<float> fk, fv;  // [layer][pos][kvh][hd]
  uint32_t fast_pos = 0;
};

namespace {

std::string lname(const char* pre, uint32_t l, const char* suf) {
  return std::string(pre) + "." + std::to_string(l) + "." + suf;
}

// DualArGraphSpec::from_gguf (crates/fish_s2_infer/src/registry.rs:45-214),
// shape-generic: slow head_dim comes from the q_norm length when QK-norm is on.
void build_model(orc_model* m) {
  Gguf& g = m->g;
  if (g.m("general.architecture").s != "fish-speech")
    fail("expected fish-speech transformer GGUF, got %s", g.m("general.architecture").s.c_str());
  orc_spec& s = m->spec;
  s.slow_layers = g.mu32("fish-speech.block_count");
  s.dim = g.mu32("fish-speech.embedding_length");
  s.ffn = g.mu32("fish-speech.feed_forward_length");
  s.heads = g.mu32("fish-speech.attention.head_count");
  s.kv_heads = g.mu32("fish-speech.attention.head_count_kv");
  s.rope_base = g.mf32("fish-speech.rope.freq_base");
  s.eps = g.mf32("fish-speech.attention.layer_norm_rms_epsilon");
  s.slow_qk_norm = g.mbool("fish_speech.attention_qk_norm");
  if (s.slow_qk_norm)
    s.head_dim = uint32_t(g.tensor("layers.0.attention.q_norm.weight").elements());
  else
    s.head_dim = s.dim / s.heads;
  s.fast_layers = g.mu32("fish_speech.fast_block_count");
  s.fast_dim = g.mu32("fish_speech.fast_embedding_length");
  s.fast_ffn = g.mu32("fish_speech.fast_feed_forward_length");
  s.fast_heads = g.mu32("fish_speech.fast_head_count");
  s.fast_kv_heads = g.mu32("fish_speech.fast_head_count_kv");
  s.fast_head_dim = g.mu32("fish_speech.fast_head_dim");
  s.fast_rope_base = g.mf32("fish_speech.fast_rope_freq_base");
  s.fast_eps = g.mf32("fish_speech.fast_layer_norm_rms_eps");
  s.codebook_size = g.mu32("fish_speech.codebook_size");
  s.num_codebooks = g.mu32("fish_speech.num_codebooks");
  s.semantic_begin = g.mu32("fish_speech.semantic_begin_id");
  s.semantic_end = g.mu32("fish_speech.semantic_end_id");
  s.scale_codebook_embeddings = g.mbool("fish_speech.scale_codebook_embeddings");
  if (g.mbool("fish_speech.fast_project_in"))
    fail("fast_project_in is not implemented");  // fast_ar.rs:366-370
  if (s.fast_dim != s.dim) fail("fast embedding_length must equal slow embedding_length");
  if (s.kv_heads == 0 || s.heads % s.kv_heads) fail("invalid GQA head split");
  if (s.fast_kv_heads == 0 || s.fast_heads % s.fast_kv_heads) fail("invalid fast GQA head split");
  if (s.head_dim == 0 || s.head_dim % 2 || s.fast_head_dim == 0 || s.fast_head_dim % 2)
    fail("head_dim must be non-zero and even");

  m->emb = &g.tensor("embeddings.weight");
  if (m->emb->dims.size() != 2 || m->emb->dims[0] != s.dim || m->emb->type != T_F16)
    fail("embeddings.weight shape/type mismatch");
  s.vocab = uint32_t(m->emb->dims[1]);
  m->cb_emb = &g.tensor("codebook_embeddings.weight");
  if (m->cb_emb->dims.size() != 2 || m->cb_emb->dims[0] != s.dim || m->cb_emb->type != T_F16 ||
      m->cb_emb->dims[1] < uint64_t(s.num_codebooks) * s.codebook_size)
    fail("codebook_embeddings.weight shape/type mismatch");
  m->fast_emb = &g.tensor("fast_embeddings.weight");
  if (m->fast_emb->dims.size() != 2 || m->fast_emb->dims[0] != s.dim || m->fast_emb->type != T_F16 ||
      m->fast_emb->dims[1] < s.codebook_size)
    fail("fast_embeddings.weight shape/type mismatch");
  m->norm = load_vec(g, "norm.weight", s.dim);
  m->fast_norm = load_vec(g, "fast_norm.weight", s.dim);
  m->fast_out = load_lin(g, "fast_output.weight", s.dim, s.codebook_size);

  const size_t q = size_t(s.heads) * s.head_dim, kv = size_t(s.kv_heads) * s.head_dim;
  m->slow.resize(s.slow_layers);
  for (uint32_t l = 0; l < s.slow_layers; ++l) {
    SlowLayer& L = m->slow[l];
    L.attn_norm = load_vec(g, lname("layers", l, "attention_norm.weight"), s.dim);
    L.ffn_norm = load_vec(g, lname("layers", l, "ffn_norm.weight"), s.dim);
    if (s.slow_qk_norm) {
      L.q_norm = load_vec(g, lname("layers", l, "attention.q_norm.weight"), s.head_dim);
      L.k_norm = load_vec(g, lname("layers", l, "attention.k_norm.weight"), s.head_dim);
    }
    L.wqkv = load_lin(g, lname("layers", l, "attention.wqkv.weight"), s.dim, q + 2 * kv);
    L.wo = load_lin(g, lname("layers", l, "attention.wo.weight"), q, s.dim);
    L.w1 = load_lin(g, lname("layers", l, "feed_forward.w1.weight"), s.dim, s.ffn);
    L.w2 = load_lin(g, lname("layers", l, "feed_forward.w2.weight"), s.ffn, s.dim);
    L.w3 = load_lin(g, lname("layers", l, "feed_forward.w3.weight"), s.dim, s.ffn);
  }
  s.linear_type = s.slow_layers ? m->slow[0].wqkv.t->type : uint32_t(T_F16);
  const size_t fq = size_t(s.fast_heads) * s.fast_head_dim,
               fkv = size_t(s.fast_kv_heads) * s.fast_head_dim;
  m->fast.resize(s.fast_layers);
  for (uint32_t l = 0; l < s.fast_layers; ++l) {
    FastLayer& L = m->fast[l];
    L.attn_norm = load_vec(g, lname("fast_layers", l, "attention_norm.weight"), s.dim);
    L.ffn_norm = load_vec(g, lname("fast_layers", l, "ffn_norm.weight"), s.dim);
    L.wqkv = load_lin(g, lname("fast_layers", l, "attention.wqkv.weight"), s.dim, fq + 2 * fkv);
    L.wo = load_lin(g, lname("fast_layers", l, "attention.wo.weight"), fq, s.dim);
    L.w1 = load_lin(g, lname("fast_layers", l, "feed_forward.w1.weight"), s.dim, s.fast_ffn);
    L.w2 = load_lin(g, lname("fast_layers", l, "feed_forward.w2.weight"), s.fast_ffn, s.dim);
    L.w3 = load_lin(g, lname("fast_layers", l, "feed_forward.w3.weight"), s.dim, s.fast_ffn);
  }
}

std::vector<float> expand(const Lin& l) {
  std::vector<float> v(l.in * l.out);
  const size_t rb = row_bytes(l.t->type, l.in);
  for (size_t r = 0; r < l.out; ++r) dequant_row(l.t->data + r * rb, l.t->type, l.in, v.data() + r * l.in);
  return v;
}

// F16TensorView::from_gguf per call (tensor.rs:22-45 via gguf.rs:111-120):
// open + seek + read the tensor bytes, then expand to f32.  Used by the
// faithful Slow-AR mode, which repeats it for every layer of every eval
// (slow_ar.rs:1029, 1189).
std::vector<float> reload_expand(const orc_model* m, const Lin& l) {
  std::vector<uint8_t> bytes(l.t->bytes);
  int fd = ::open(m->g.path.c_str(), O_RDONLY);
  if (fd < 0) fail("cannot reopen %s", m->g.path.c_str());
  size_t done = 0;
  while (done < bytes.size()) {
    ssize_t r = pread(fd, bytes.data() + done, bytes.size() - done, off_t(l.t->abs_offset + done));
    if (r <= 0) {
      ::close(fd);
      fail("short read of %s", l.t->name.c_str());
    }
    done += size_t(r);
  }
  ::close(fd);
  std::vector<float> v(l.in * l.out);
  const size_t rb = row_bytes(l.t->type, l.in);
  for (size_t r = 0; r < l.out; ++r) dequant_row(bytes.data() + r * rb, l.t->type, l.in, v.data() + r * l.in);
  return v;
}

void run_lin(orc_model* m, const Lin& l, const float* w32, const float* x, size_t n_tok, float* y) {
  if (w32)
    linear_multi(*m->pool, x, n_tok, reinterpret_cast<const uint8_t*>(w32), T_F32, l.in, l.out, y);
  else
    linear_multi(*m->pool, x, n_tok, l.t->data, l.t->type, l.in, l.out, y);
}

void emb_row(const TensorInfo* t, size_t dim, size_t row, float* out) {
  if (row >= t->dims[1]) fail("embedding index %zu out of range for vocab_dim %llu", row,
                              (unsigned long long)t->dims[1]);
  dequant_row(t->data + row * dim * 2, T_F16, dim, out);
}

// embed_slow_ar_time_major (crates/fish_s2_infer/src/slow_ar.rs:1041-1133)
void embed(orc_model* m, const int32_t* flat, size_t n_tok, float* out) {
  const orc_spec& s = m->spec;
  const size_t cdim = s.num_codebooks + 1;
  const float sem_scale = s.scale_codebook_embeddings ? 1.0f / std::sqrt(float(cdim)) : 1.0f;
  std::vector<float> cbsum(s.dim), row(s.dim);
  for (size_t t = 0; t < n_tok; ++t) {
    const int32_t* tok = flat + t * cdim;
    if (tok[0] < 0) fail("semantic token id must be non-negative, got %d", tok[0]);
    uint32_t id = uint32_t(tok[0]);
    bool is_sem = id >= s.semantic_begin && id <= s.semantic_end;
    float* h = out + t * s.dim;
    emb_row(m->emb, s.dim, id, h);
    if (is_sem) {
      std::fill(cbsum.begin(), cbsum.end(), 0.0f);
      for (uint32_t cb = 0; cb < s.num_codebooks; ++cb) {
        int32_t raw = tok[1 + cb];
        if (raw < 0) fail("codebook token must be non-negative, got %d", raw);
        emb_row(m->cb_emb, s.dim, size_t(raw) + size_t(cb) * s.codebook_size, row.data());
        for (size_t i = 0; i < s.dim; ++i) cbsum[i] += row[i];
      }
      for (size_t i = 0; i < s.dim; ++i) h[i] += cbsum[i];
    }
    if (s.scale_codebook_embeddings) {
      float sc = is_sem ? sem_scale : 1.0f;
      for (size_t i = 0; i < s.dim; ++i) h[i] *= sc;
    }
  }
}

// Slow-AR layer over a token chunk: forward_block_prefill_sequence /
// forward_decode_token_with_backend (slow_ar.rs:558-617, 637-854).
void slow_layer(orc_model* m, uint32_t layer, float* hid, size_t n_tok, uint32_t start) {
  const orc_spec& s = m->spec;
  SlowLayer& L = m->slow[layer];
  const size_t d = s.dim, hd = s.head_dim, H = s.heads, Hkv = s.kv_heads;
  const size_t q = H * hd, kv = Hkv * hd, qkv_n = q + 2 * kv;
  std::vector<float> w_qkv, w_o, w_1, w_2, w_3;
  if (m->flags & ORC_FAITHFUL_SLOW_RELOAD) {
    w_qkv = reload_expand(m, L.wqkv);
    w_o = reload_expand(m, L.wo);
    w_1 = reload_expand(m, L.w1);
    w_2 = reload_expand(m, L.w2);
    w_3 = reload_expand(m, L.w3);
  }
  auto wp = [](std::vector<float>& v) -> const float* { return v.empty() ? nullptr : v.data(); };
  std::vector<float> normed(n_tok * d), qkv(n_tok * qkv_n), qh(n_tok * q), att(n_tok * q),
      proj(n_tok * d);
  for (size_t t = 0; t < n_tok; ++t) rms_norm(hid + t * d, L.attn_norm.data(), d, s.eps, normed.data() + t * d);
  run_lin(m, L.wqkv, wp(w_qkv), normed.data(), n_tok, qkv.data());
  std::vector<float> kh(kv);
  const float scale = 1.0f / std::sqrt(float(hd));  // slow_ar.rs:59-61
  for (size_t t = 0; t < n_tok; ++t) {
    const float* row = qkv.data() + t * qkv_n;
    float* qt = qh.data() + t * q;
    const size_t pos = start + t;
    if (s.slow_qk_norm) {
      rms_norm_heads(row, L.q_norm.data(), q, hd, s.eps, qt);
      rms_norm_heads(row + q, L.k_norm.data(), kv, hd, s.eps, kh.data());
    } else {
      memcpy(qt, row, q * 4);
      memcpy(kh.data(), row + q, kv * 4);
    }
    rope_normal(qt, q, hd, pos, s.rope_base);
    rope_normal(kh.data(), kv, hd, pos, s.rope_base);
    // SlowArKvCache::write_token (attention.rs:56-76); with ORC_KV_F16 the
    // stored values are the f16 roundings of K and V
    size_t off = (size_t(layer) * m->max_seq + pos) * kv;
    memcpy(m->kc.data() + off, kh.data(), kv * 4);
    memcpy(m->vc.data() + off, row + q + kv, kv * 4);
    if (m->flags & ORC_KV_F16) {
      for (size_t i = 0; i < kv; ++i) {
        m->kc[off + i] = f16_to_f32(f32_to_f16(m->kc[off + i]));
        m->vc[off + i] = f16_to_f32(f32_to_f16(m->vc[off + i]));
      }
    }
  }
  for (size_t t = 0; t < n_tok; ++t) {
    size_t visible = start + t + 1;
    const float* kbase = m->kc.data() + size_t(layer) * m->max_seq * kv;
    const float* vbase = m->vc.data() + size_t(layer) * m->max_seq * kv;
    gqa_attention(qh.data() + t * q, kbase, vbase, H, Hkv, hd, visible, scale, att.data() + t * q);
  }
  run_lin(m, L.wo, wp(w_o), att.data(), n_tok, proj.data());
  for (size_t i = 0; i < n_tok * d; ++i) hid[i] = hid[i] + proj[i];
  // forward_feed_forward_with_backend (slow_ar.rs:659-710)
  const size_t f = s.ffn;
  std::vector<float> gate(n_tok * f), up(n_tok * f), act(n_tok * f);
  for (size_t t = 0; t < n_tok; ++t) rms_norm(hid + t * d, L.ffn_norm.data(), d, s.eps, normed.data() + t * d);
  run_lin(m, L.w1, wp(w_1), normed.data(), n_tok, gate.data());
  run_lin(m, L.w3, wp(w_3), normed.data(), n_tok, up.data());
  swiglu_slow(gate.data(), up.data(), n_tok * f, act.data());
  run_lin(m, L.w2, wp(w_2), act.data(), n_tok, proj.data());
  for (size_t i = 0; i < n_tok * d; ++i) hid[i] = hid[i] + proj[i];
}

// SlowArState::eval (slow_ar.rs:456-527)
void slow_eval(orc_model* m, const int32_t* flat, size_t n_tok, float* hidden_out, float* logits_out) {
  const orc_spec& s = m->spec;
  if (n_tok == 0) fail("expected at least one token");
  if (size_t(m->n_past) + n_tok > m->max_seq)
    fail("KV cache overflow: n_past=%u n_tokens=%zu max_seq_len=%u", m->n_past, n_tok, m->max_seq);
  std::vector<float> hid(n_tok * s.dim);
  embed(m, flat, n_tok, hid.data());
  for (uint32_t l = 0; l < s.slow_layers; ++l) slow_layer(m, l, hid.data(), n_tok, m->n_past);
  // output head on the last token (slow_ar.rs:510-521, 943-955)
  const float* last = hid.data() + (n_tok - 1) * s.dim;
  rms_norm(last, m->norm.data(), s.dim, s.eps, hidden_out);
  if (logits_out)
    linear_multi(*m->pool, hidden_out, 1, m->emb->data, T_F16, s.dim, s.vocab, logits_out);
  m->n_past += uint32_t(n_tok);
}

// FastArLayerSkeleton::forward_prefill (fast_ar.rs:245-292) for one layer over
// a whole sequence -- the reference's recompute path.
void fast_layer_prefill(orc_model* m, uint32_t layer, std::vector<float>& seq, size_t n) {
  const orc_spec& s = m->spec;
  FastLayer& L = m->fast[layer];
  const size_t d = s.dim, hd = s.fast_head_dim, H = s.fast_heads, Hkv = s.fast_kv_heads;
  const size_t q = H * hd, kv = Hkv * hd, qkv_n = q + 2 * kv, f = s.fast_ffn;
  const bool faithful = (m->flags & ORC_FAITHFUL_FAST_RECOMPUTE) != 0;
  auto w = [&](const std::vector<float>& v) -> const float* { return faithful ? v.data() : nullptr; };
  std::vector<float> normed(n * d), qkv(n * qkv_n), qs(n * q), ks(n * kv), vs(n * kv), att(q), proj(d),
      out_h(d), gate(f), up(f), act(f), y(n * d);
  for (size_t t = 0; t < n; ++t) rms_norm(seq.data() + t * d, L.attn_norm.data(), d, s.fast_eps, normed.data() + t * d);
  run_lin(m, L.wqkv, w(L.wqkv32), normed.data(), n, qkv.data());
  for (size_t t = 0; t < n; ++t) {
    memcpy(qs.data() + t * q, qkv.data() + t * qkv_n, q * 4);
    memcpy(ks.data() + t * kv, qkv.data() + t * qkv_n + q, kv * 4);
    memcpy(vs.data() + t * kv, qkv.data() + t * qkv_n + q + kv, kv * 4);
    rope_normal(qs.data() + t * q, q, hd, t, s.fast_rope_base);
    rope_normal(ks.data() + t * kv, kv, hd, t, s.fast_rope_base);
  }
  const float scale = 1.0f / std::sqrt(float(hd));
  for (size_t t = 0; t < n; ++t) {
    gqa_attention(qs.data() + t * q, ks.data(), vs.data(), H, Hkv, hd, t + 1, scale, att.data());
    run_lin(m, L.wo, w(L.wo32), att.data(), 1, proj.data());
    const float* hin = seq.data() + t * d;
    for (size_t i = 0; i < d; ++i) out_h[i] = hin[i] + proj[i];
    std::vector<float> nf(d);
    rms_norm(out_h.data(), L.ffn_norm.data(), d, s.fast_eps, nf.data());
    run_lin(m, L.w1, w(L.w132), nf.data(), 1, gate.data());
    run_lin(m, L.w3, w(L.w332), nf.data(), 1, up.data());
    swiglu_fast(gate.data(), up.data(), f, act.data());
    run_lin(m, L.w2, w(L.w232), act.data(), 1, proj.data());
    for (size_t i = 0; i < d; ++i) y[t * d + i] = out_h[i] + proj[i];
  }
  seq.swap(y);
}

// Incremental equivalent: appends position `pos` through every Fast layer
// using cached K/V of earlier positions.  Causality makes each position's
// arithmetic identical to the recompute above.
void fast_append(orc_model* m, const float* x, uint32_t pos, float* out_hidden) {
  const orc_spec& s = m->spec;
  const size_t d = s.dim, hd = s.fast_head_dim, H = s.fast_heads, Hkv = s.fast_kv_heads;
  const size_t q = H * hd, kv = Hkv * hd, qkv_n = q + 2 * kv, f = s.fast_ffn;
  const size_t ctx = s.num_codebooks + 1;
  std::vector<float> h(x, x + d), normed(d), qkv(qkv_n), att(q), proj(d), gate(f), up(f), act(f);
  const float scale = 1.0f / std::sqrt(float(hd));
  for (uint32_t l = 0; l < s.fast_layers; ++l) {
    FastLayer& L = m->fast[l];
    rms_norm(h.data(), L.attn_norm.data(), d, s.fast_eps, normed.data());
    run_lin(m, L.wqkv, nullptr, normed.data(), 1, qkv.data());
    rope_normal(qkv.data(), q, hd, pos, s.fast_rope_base);
    rope_normal(qkv.data() + q, kv, hd, pos, s.fast_rope_base);
    float* kb = m->fk.data() + size_t(l) * ctx * kv;
    float* vb = m->fv.data() + size_t(l) * ctx * kv;
    memcpy(kb + size_t(pos) * kv, qkv.data() + q, kv * 4);
    memcpy(vb + size_t(pos) * kv, qkv.data() + q + kv, kv * 4);
    gqa_attention(qkv.data(), kb, vb, H, Hkv, hd, pos + 1, scale, att.data());
    run_lin(m, L.wo, nullptr, att.data(), 1, proj.data());
    for (size_t i = 0; i < d; ++i) h[i] = h[i] + proj[i];
    rms_norm(h.data(), L.ffn_norm.data(), d, s.fast_eps, normed.data());
    run_lin(m, L.w1, nullptr, normed.data(), 1, gate.data());
    run_lin(m, L.w3, nullptr, normed.data(), 1, up.data());
    swiglu_fast(gate.data(), up.data(), f, act.data());
    run_lin(m, L.w2, nullptr, act.data(), 1, proj.data());
    for (size_t i = 0; i < d; ++i) h[i] = h[i] + proj[i];
  }
  memcpy(out_hidden, h.data(), d * 4);
}

void fast_head(orc_model* m, const float* last, float* logits) {
  const orc_spec& s = m->spec;
  std::vector<float> normed(s.dim);
  rms_norm(last, m->fast_norm.data(), s.dim, s.fast_eps, normed.data());
  run_lin(m, m->fast_out, nullptr, normed.data(), 1, logits);
}

// forward_codebook_prefix (fast_ar.rs:360-437), recompute form.
void fast_logits_recompute(orc_model* m, const float* hidden, const uint32_t* prefix, size_t plen,
                           float* logits) {
  const orc_spec& s = m->spec;
  if (plen >= s.num_codebooks) fail("fast prefix too long: %zu codes", plen);
  size_t n = 1 + plen;
  std::vector<float> seq(n * s.dim);
  memcpy(seq.data(), hidden, s.dim * 4);
  for (size_t i = 0; i < plen; ++i) emb_row(m->fast_emb, s.dim, prefix[i], seq.data() + (1 + i) * s.dim);
  for (uint32_t l = 0; l < s.fast_layers; ++l) fast_layer_prefill(m, l, seq, n);
  fast_head(m, seq.data() + (n - 1) * s.dim, logits);
}

// forward_codebook_prefix by the incremental form that fast_codebooks uses:
// position 0 (the Slow hidden) and the prefix codes' fast_emb rows appended
// one at a time over the cached K/V, then the head on the last position.
void fast_logits_incremental(orc_model* m, const float* hidden, const uint32_t* prefix, size_t plen,
                             float* logits) {
  const orc_spec& s = m->spec;
  if (plen >= s.num_codebooks) fail("fast prefix too long: %zu codes", plen);
  std::vector<float> h(s.dim), row(s.dim);
  fast_append(m, hidden, 0, h.data());
  for (size_t i = 0; i < plen; ++i) {
    emb_row(m->fast_emb, s.dim, prefix[i], row.data());
    fast_append(m, row.data(), uint32_t(i + 1), h.data());
  }
  fast_head(m, h.data(), logits);
}

// generate_codebooks_for_semantic (fast_ar.rs:440-470)
void fast_codebooks(orc_model* m, const float* hidden, uint32_t sem, float T, float top_p, int32_t top_k,
                    uint64_t* rng, uint32_t* codes) {
  const orc_spec& s = m->spec;
  if (sem >= s.codebook_size) fail("semantic_code %u >= codebook_size %u", sem, s.codebook_size);
  std::vector<uint32_t> prefix{sem};
  std::vector<float> logits(s.codebook_size), h(s.dim), row(s.dim);
  codes[0] = sem;
  const bool recompute = (m->flags & ORC_FAITHFUL_FAST_RECOMPUTE) != 0;
  if (!recompute) {
    fast_append(m, hidden, 0, h.data());
    emb_row(m->fast_emb, s.dim, sem, row.data());
    fast_append(m, row.data(), 1, h.data());
  }
  for (uint32_t cb = 1; cb < s.num_codebooks; ++cb) {
    if (recompute) {
      fast_logits_recompute(m, hidden, prefix.data(), prefix.size(), logits.data());
    } else {
      fast_head(m, h.data(), logits.data());
    }
    uint32_t tok = sample_token(logits.data(), s.codebook_size, T, top_p, top_k, -1, rng);
    if (tok >= s.codebook_size) fail("sampled codebook token %u >= codebook_size", tok);
    prefix.push_back(tok);
    codes[cb] = tok;
    if (!recompute && cb + 1 < s.num_codebooks) {
      emb_row(m->fast_emb, s.dim, tok, row.data());
      fast_append(m, row.data(), cb + 1, h.data());
    }
  }
}

// build_semantic_bias + apply_semantic_bias (sampling.rs:54-100): bias 0 on
// [sem_begin, sem_end] and on im_end, -inf elsewhere, added to the logits;
// im_end then forced to -inf when blocked.  im_end < 0 means None.
void semantic_bias(float* l, size_t n, uint32_t sem_begin, uint32_t sem_end, int64_t im_end, bool block) {
  for (size_t i = 0; i < n; ++i) {
    bool allowed = (i >= sem_begin && i <= sem_end) || (im_end >= 0 && i == size_t(im_end));
    l[i] += allowed ? 0.0f : -INFINITY;
  }
  if (block && im_end >= 0 && size_t(im_end) < n) l[im_end] = -INFINITY;
}

// sample_semantic_token (generate.rs:284-298) with build_semantic_bias /
// apply_semantic_bias (sampling.rs:54-100).
uint32_t sample_semantic(orc_model* m, const float* logits_full, size_t generated_after_prefill,
                         uint32_t min_before_end, float T, float top_p, int32_t top_k, uint64_t* rng) {
  const orc_spec& s = m->spec;
  std::vector<float> l(logits_full, logits_full + s.vocab);
  bool block = uint32_t(generated_after_prefill) < min_before_end;
  semantic_bias(l.data(), s.vocab, s.semantic_begin, s.semantic_end, int64_t(m->im_end), block);
  return sample_token(l.data(), s.vocab, T, top_p, top_k, block ? -1 : int64_t(m->im_end), rng);
}

// semantic_to_codebook_id (generate.rs:273-282)
uint32_t sem_to_code(const orc_spec& s, uint32_t tok) {
  if (tok < s.semantic_begin || tok > s.semantic_end) return 0;
  uint32_t c = tok - s.semantic_begin;
  return c >= s.codebook_size ? s.codebook_size - 1 : c;
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" {

uint16_t orc_f32_to_f16(float v) { return f32_to_f16(v); }
float orc_f16_to_f32(uint16_t b) { return f16_to_f32(b); }

int32_t orc_dequant_row(const uint8_t* src, uint32_t type, size_t n, float* out) {
  try {
    dequant_row(src, type, n, out);
    return 1;
  } catch (const std::exception&) {
    return 0;
  }
}

int32_t orc_rms_norm(const float* x, const float* w, size_t n, float eps, float* out) {
  try {
    rms_norm(x, w, n, eps, out);
    return 1;
  } catch (const std::exception&) {
    return 0;
  }
}

int32_t orc_rms_norm_heads(const float* x, const float* w, size_t n, size_t hd, float eps, float* out) {
  try {
    rms_norm_heads(x, w, n, hd, eps, out);
    return 1;
  } catch (const std::exception&) {
    return 0;
  }
}

int32_t orc_linear(const float* x, const uint8_t* w, uint32_t type, size_t in, size_t out, float* y) {
  try {
    Pool p(1);
    linear_multi(p, x, 1, w, type, in, out, y);
    return 1;
  } catch (const std::exception&) {
    return 0;
  }
}

int32_t orc_rope_normal(float* v, size_t len, size_t hd, size_t pos, float base) {
  try {
    rope_normal(v, len, hd, pos, base);
    return 1;
  } catch (const std::exception&) {
    return 0;
  }
}

int32_t orc_gqa_attention(const float* q, const float* k, const float* v, size_t H, size_t Hkv, size_t hd,
                          size_t T, float scale, float* out) {
  try {
    gqa_attention(q, k, v, H, Hkv, hd, T, scale, out);
    return 1;
  } catch (const std::exception&) {
    return 0;
  }
}

void orc_swiglu_slow(const float* g, const float* u, size_t n, float* out) { swiglu_slow(g, u, n, out); }
void orc_swiglu_fast(const float* g, const float* u, size_t n, float* out) { swiglu_fast(g, u, n, out); }
double orc_rng_next_unit(uint64_t* s) { return rng_next_unit(s); }

int32_t orc_sample_token(const float* logits, size_t n, float T, float top_p, int32_t top_k,
                         int64_t always_include, uint64_t* rng, uint32_t* out) {
  *out = sample_token(logits, n, T, top_p, top_k, always_include, rng);
  return 1;
}

int32_t orc_sample_token_margins(const float* logits, size_t n, float T, float top_p, int32_t top_k,
                                 int64_t always_include, uint64_t* rng, uint32_t* out, float* margins) {
  SampleMargins mg;
  *out = sample_token(logits, n, T, top_p, top_k, always_include, rng, &mg);
  margins[0] = mg.draw;
  margins[1] = mg.cut;
  margins[2] = mg.tie;
  return 1;
}

void orc_semantic_bias(float* logits, size_t n, uint32_t sem_begin, uint32_t sem_end, int64_t im_end,
                       int32_t block_im_end) {
  semantic_bias(logits, n, sem_begin, sem_end, im_end, block_im_end != 0);
}

// f32::exp of the reference: the C library's expf
void orc_expf(const float* x, size_t n, float* y) {
  for (size_t i = 0; i < n; ++i) y[i] = expf(x[i]);
}

int32_t orc_transpose_to_time_major(const uint32_t* data, uint32_t rows, size_t cols, int32_t* flat) {
  if (rows == 0) return 0;
  for (size_t t = 0; t < cols; ++t)
    for (size_t r = 0; r < rows; ++r) flat[t * rows + r] = int32_t(data[r * cols + t]);
  return 1;
}

// compact_codes (generate.rs:346-390)
size_t orc_compact_codes(int32_t* codes, uint32_t ncb, uint32_t max_new, uint32_t n_frames) {
  if (n_frames >= max_new) return size_t(ncb) * n_frames;
  std::vector<int32_t> out(size_t(ncb) * n_frames);
  for (size_t cb = 0; cb < ncb; ++cb)
    for (size_t t = 0; t < n_frames; ++t) out[cb * n_frames + t] = codes[cb * max_new + t];
  memcpy(codes, out.data(), out.size() * 4);
  return out.size();
}

orc_model* orc_open(const char* path, uint32_t max_seq, uint32_t im_end, uint32_t flags, uint32_t threads,
                    char* err, size_t cap) {
  std::unique_ptr<orc_model> m(new orc_model());
  try {
    if (max_seq == 0) fail("max_seq_len must be non-zero");
    m->g.open_file(path);
    m->im_end = im_end;
    m->flags = flags;
    unsigned nt = threads ? threads : std::max(1u, std::thread::hardware_concurrency());
    m->pool.reset(new Pool(nt));
    build_model(m.get());
    m->max_seq = max_seq;
    const orc_spec& s = m->spec;
    size_t kv = size_t(s.kv_heads) * s.head_dim;
    m->kc.assign(size_t(s.slow_layers) * max_seq * kv, 0.0f);
    m->vc.assign(size_t(s.slow_layers) * max_seq * kv, 0.0f);
    size_t fkv = size_t(s.fast_kv_heads) * s.fast_head_dim;
    m->fk.assign(size_t(s.fast_layers) * (s.num_codebooks + 1) * fkv, 0.0f);
    m->fv.assign(m->fk.size(), 0.0f);
    if (flags & ORC_FAITHFUL_FAST_RECOMPUTE) {
      for (FastLayer& L : m->fast) {
        L.wqkv32 = expand(L.wqkv);
        L.wo32 = expand(L.wo);
        L.w132 = expand(L.w1);
        L.w232 = expand(L.w2);
        L.w332 = expand(L.w3);
      }
    }
    return m.release();
  } catch (const std::exception& e) {
    copy_err(e, err, cap);
    return nullptr;
  }
}

void orc_close(orc_model* m) { delete m; }

int32_t orc_get_spec(const orc_model* m, orc_spec* out) {
  *out = m->spec;
  return 1;
}

// SlowArState::reset (slow_ar.rs:434-438): n_past = 0, fresh zeroed cache
void orc_reset(orc_model* m) {
  m->n_past = 0;
  std::fill(m->kc.begin(), m->kc.end(), 0.0f);
  std::fill(m->vc.begin(), m->vc.end(), 0.0f);
}

uint32_t orc_n_past(const orc_model* m) { return m->n_past; }

int32_t orc_eval(orc_model* m, const int32_t* flat, size_t n_tok, float* hidden, float* logits, char* err,
                 size_t cap) {
  try {
    slow_eval(m, flat, n_tok, hidden, logits);
    return 1;
  } catch (const std::exception& e) {
    copy_err(e, err, cap);
    return 0;
  }
}

// embed_slow_ar_time_major (slow_ar.rs:1041-1133) on its own: out [n_tok][dim]
int32_t orc_embed(orc_model* m, const int32_t* flat, size_t n_tok, float* out, char* err, size_t cap) {
  try {
    if (n_tok == 0) return 1;
    for (size_t t = 0; t < n_tok; ++t) {
      const int32_t* tok = flat + t * (m->spec.num_codebooks + 1);
      if (tok[0] >= 0 && uint32_t(tok[0]) >= m->spec.vocab)
        fail("embedding index %d out of range for vocab_dim %u", tok[0], m->spec.vocab);
    }
    embed(m, flat, n_tok, out);
    return 1;
  } catch (const std::exception& e) {
    copy_err(e, err, cap);
    return 0;
  }
}

int32_t orc_fast_logits(orc_model* m, const float* hidden, const uint32_t* prefix, size_t plen, float* logits,
                        char* err, size_t cap) {
  try {
    if (m->flags & ORC_FAITHFUL_FAST_RECOMPUTE)
      fast_logits_recompute(m, hidden, prefix, plen, logits);
    else
      fast_logits_incremental(m, hidden, prefix, plen, logits);
    return 1;
  } catch (const std::exception& e) {
    copy_err(e, err, cap);
    return 0;
  }
}

int32_t orc_fast_codebooks(orc_model* m, const float* hidden, uint32_t sem, float T, float top_p, int32_t top_k,
                           uint64_t* rng, uint32_t* codes, char* err, size_t cap) {
  try {
    fast_codebooks(m, hidden, sem, T, top_p, top_k, rng, codes);
    return 1;
  } catch (const std::exception& e) {
    copy_err(e, err, cap);
    return 0;
  }
}

// generate_codes (crates/fish_s2_infer/src/generate.rs:117-221)
int32_t orc_generate_codes(orc_model* m, const int32_t* prompt, size_t cols, uint32_t max_new, float T,
                           float top_p, int32_t top_k, uint32_t min_before_end, uint64_t* rng, int32_t* codes,
                           uint32_t* n_frames_out, double* prefill_s, double* decode_s, char* err, size_t cap) {
  try {
    const orc_spec& s = m->spec;
    const size_t cdim = s.num_codebooks + 1;
    auto t0 = std::chrono::steady_clock::now();
    orc_reset(m);
    std::vector<float> hidden(s.dim), logits(s.vocab);
    slow_eval(m, prompt, cols, hidden.data(), logits.data());
    auto t1 = std::chrono::steady_clock::now();
    const uint32_t ncb = std::max(1u, s.num_codebooks);
    std::fill(codes, codes + size_t(ncb) * max_new, 0);
    uint32_t main = sample_semantic(m, logits.data(), 0, min_before_end, T, top_p, top_k, rng);
    uint32_t step = 0;
    std::vector<uint32_t> cbs(s.num_codebooks);
    std::vector<int32_t> in(cdim);
    while (main != m->im_end && step < max_new) {
      uint32_t sem = sem_to_code(s, main);
      fast_codebooks(m, hidden.data(), sem, T, top_p, top_k, rng, cbs.data());
      for (uint32_t cb = 0; cb < ncb && cb < s.num_codebooks; ++cb) codes[size_t(cb) * max_new + step] = int32_t(cbs[cb]);
      // build_step_input (generate.rs:300-344)
      std::fill(in.begin(), in.end(), 0);
      in[0] = int32_t(main);
      if (main >= s.semantic_begin && main <= s.semantic_end)
        for (uint32_t cb = 0; cb < s.num_codebooks; ++cb) in[1 + cb] = int32_t(cbs[cb]);
      slow_eval(m, in.data(), 1, hidden.data(), logits.data());
      step += 1;
      size_t gen = size_t(m->n_past >= cols ? m->n_past - cols : 0) + step;
      main = sample_semantic(m, logits.data(), gen, min_before_end, T, top_p, top_k, rng);
    }
    auto t2 = std::chrono::steady_clock::now();
    orc_compact_codes(codes, ncb, max_new, step);
    *n_frames_out = step;
    if (prefill_s) *prefill_s = std::chrono::duration<double>(t1 - t0).count();
    if (decode_s) *decode_s = std::chrono::duration<double>(t2 - t1).count();
    return 1;
  } catch (const std::exception& e) {
    copy_err(e, err, cap);
    return 0;
  }
}

}  // extern "C"

// ===========================================================================
// RVQ codec decode (crates/fish_s2_infer/src/codec.rs): decode_waveform
// (:1690-1714) = rvq_lookup_codes (:2536-2596) -> forward_codec_post_module
// (:986-1018) -> forward_codec_upsample (:2302-2325) -> forward_codec_decoder
// (:1941-2001).  Every F16 tensor is read as f32 values (F16TensorView,
// tensor.rs:8-60).  Each output element is summed in the reference's order;
// loops run several independent outputs side by side (vectorised across
// output channels) and threads split output frames, which changes no sum.
// ===========================================================================
namespace {

constexpr size_t CX_HIDDEN = 1024, CX_PROJ = 8, CX_SEM_CB = 4096, CX_RES_CB = 1024, CX_RES_Q = 9;
constexpr size_t CX_LAYERS = 8, CX_QKV = 3072, CX_FFN = 3072, CX_HEADS = 16, CX_HD = 64, CX_WINDOW = 128;
constexpr size_t CX_EXPANDED = 4096, CX_DW_K = 7, CX_ENTRY = 1536;
constexpr float CX_RMS_EPS = 1e-5f, CX_LN_EPS = 1e-6f, CX_ROPE_BASE = 10000.0f;
constexpr size_t CX_RATES[4] = {8, 8, 4, 2};
constexpr size_t CX_CH[5] = {1536, 768, 384, 192, 96};

float round_to_f16(float v) { return f16_to_f32(f32_to_f16(v)); }

// snake_activation_frame_major (codec.rs:2162-2186)
void cx_snake(const float* in, size_t frames, size_t ch, const float* alpha, float* out) {
  for (size_t f = 0; f < frames; ++f) {
    for (size_t c = 0; c < ch; ++c) {
      const float a = std::fabs(alpha[c]) < 1e-8f ? 1e-8f : alpha[c];
      const float x = in[f * ch + c];
      const float s = sinf(a * x);
      out[f * ch + c] = x + (s * s) / a;
    }
  }
}

// causal_conv_1d_frame_major with stride 1 (codec.rs:2212-2293): the input is
// rounded to f16, left-padded by (k - 1) * dilation zero frames (the extra
// right padding of extra_padding_for_conv1d, :2188-2201, is 0 at stride 1),
// and out[t][o] = bias[o] + sum over tap, then input channel, of
// x16[t + tap*d - (k-1)*d][i] * W[o][i][tap] (ggml index tap + k*i + k*in*o).
// Padding frames contribute +-0 products, which leave a non-zero sum unchanged.
void cx_conv1d(Pool& pool, const float* in, size_t frames, size_t in_ch, size_t out_ch, size_t dilation,
               const float* w, size_t w_len, const float* bias, float* out) {
  if (in_ch == 0 || out_ch == 0) fail("causal conv channel count is zero");
  const size_t k = w_len / (in_ch * out_ch);
  if (k == 0 || k * in_ch * out_ch != w_len)
    fail("causal conv weight length mismatch: expected %zu, got %zu", k * in_ch * out_ch, w_len);
  std::vector<float> x16(frames * in_ch);
  for (size_t i = 0; i < x16.size(); ++i) x16[i] = round_to_f16(in[i]);
  std::vector<float> wt(k * in_ch * out_ch);  // [tap][i][o]
  for (size_t o = 0; o < out_ch; ++o)
    for (size_t i = 0; i < in_ch; ++i)
      for (size_t t = 0; t < k; ++t) wt[(t * in_ch + i) * out_ch + o] = w[t + k * i + k * in_ch * o];
  const size_t span = (k - 1) * dilation;
  pool.run(frames, 16, [&](size_t f0, size_t f1) {
    std::vector<float> acc(out_ch);
    for (size_t f = f0; f < f1; ++f) {
      for (size_t o = 0; o < out_ch; ++o) acc[o] = bias[o];
      for (size_t t = 0; t < k; ++t) {
        const size_t p = f + t * dilation;  // padded frame
        if (p < span) continue;
        const float* xr = x16.data() + (p - span) * in_ch;
        const float* wr = wt.data() + t * in_ch * out_ch;
        for (size_t i = 0; i < in_ch; ++i) {
          const float xv = xr[i];
          const float* wi = wr + i * out_ch;
          for (size_t o = 0; o < out_ch; ++o) acc[o] += xv * wi[o];
        }
      }
      std::copy(acc.begin(), acc.end(), out + f * out_ch);
    }
  });
}

// causal_conv_transpose_1d with crop_right 0 (codec.rs:3505-3574): output
// frames = frames * stride; out[r][o] accumulates, from 0, over input frames f
// in ascending order with tap kk = r - f*stride in [0, k), then input channel,
// x[f][i] * W[i][o][kk] (ggml index kk + k*o + k*out*i); bias is added last.
// Taps that land past the last output frame are dropped.  No f16 rounding.
void cx_conv_transpose(Pool& pool, const float* in, size_t frames, size_t in_ch, size_t out_ch, size_t stride,
                       const float* w, size_t w_len, const float* bias, float* out) {
  if (in_ch == 0 || out_ch == 0 || stride == 0) fail("conv_transpose dims are zero");
  const size_t k = w_len / (in_ch * out_ch);
  if (k == 0 || k * in_ch * out_ch != w_len)
    fail("conv_transpose weight length mismatch: expected %zu, got %zu", k * in_ch * out_ch, w_len);
  std::vector<float> wt(k * in_ch * out_ch);  // [tap][i][o]
  for (size_t i = 0; i < in_ch; ++i)
    for (size_t o = 0; o < out_ch; ++o)
      for (size_t t = 0; t < k; ++t) wt[(t * in_ch + i) * out_ch + o] = w[t + k * o + k * out_ch * i];
  const size_t out_frames = frames * stride;
  pool.run(out_frames, 16, [&](size_t r0, size_t r1) {
    std::vector<float> acc(out_ch);
    for (size_t r = r0; r < r1; ++r) {
      std::fill(acc.begin(), acc.end(), 0.0f);
      const size_t f_lo = r + 1 > k ? (r + 1 - k + stride - 1) / stride : 0;
      for (size_t f = f_lo; f * stride <= r && f < frames; ++f) {
        const size_t kk = r - f * stride;
        const float* xr = in + f * in_ch;
        const float* wr = wt.data() + kk * in_ch * out_ch;
        for (size_t i = 0; i < in_ch; ++i) {
          const float xv = xr[i];
          const float* wi = wr + i * out_ch;
          for (size_t o = 0; o < out_ch; ++o) acc[o] += xv * wi[o];
        }
      }
      for (size_t o = 0; o < out_ch; ++o) out[r * out_ch + o] = acc[o] + bias[o];
    }
  });
}

// depthwise_causal_conv1d (codec.rs:3576-3619): left padding k - 1,
// out[t][c] = bias[c] + sum_kk x[t + kk - (k-1)][c] * W[c][kk] (index kk + k*c).
void cx_depthwise(const float* in, size_t frames, size_t ch, size_t k, const float* w, const float* bias,
                  float* out) {
  for (size_t f = 0; f < frames; ++f) {
    for (size_t c = 0; c < ch; ++c) {
      float sum = bias[c];
      for (size_t kk = 0; kk < k; ++kk) {
        if (f + kk < k - 1) continue;
        const size_t src = f + kk - (k - 1);
        if (src < frames) sum += in[src * ch + c] * w[kk + k * c];
      }
      out[f * ch + c] = sum;
    }
  }
}

// layer_norm_affine_frame_major (codec.rs:3621-3654)
void cx_layer_norm(float* x, size_t frames, size_t ch, const float* w, const float* b, float eps) {
  for (size_t f = 0; f < frames; ++f) {
    float* row = x + f * ch;
    float s = 0.0f;
    for (size_t c = 0; c < ch; ++c) s += row[c];
    const float mean = s / float(ch);
    float v = 0.0f;
    for (size_t c = 0; c < ch; ++c) {
      const float d = row[c] - mean;
      v += d * d;
    }
    const float var = v / float(ch);
    const float scale = 1.0f / std::sqrt(var + eps);
    for (size_t c = 0; c < ch; ++c) row[c] = (row[c] - mean) * scale * w[c] + b[c];
  }
}

// erf_approx (codec.rs:3890-3899): Abramowitz-Stegun 7.1.26 with f32 constants.
float cx_erf(float value) {
  const float sign = value < 0.0f ? -1.0f : 1.0f;
  const float x = std::fabs(value);
  const float t = 1.0f / (1.0f + 0.3275911f * x);
  const float poly = (((((1.0614054f * t - 1.4531521f) * t) + 1.4214138f) * t - 0.28449672f) * t + 0.2548296f) * t;
  return sign * (1.0f - poly * expf(-x * x));
}

// gelu_erf (codec.rs:3886-3888)
float cx_gelu(float v) { return 0.5f * v * (1.0f + cx_erf(v * 0.70710677f)); }

// silu (codec.rs:3882-3884)
float cx_silu(float v) { return v / (1.0f + expf(-v)); }

struct CxLayer {
  std::vector<float> attn_norm, ffn_norm, als, fls;
  const uint8_t *wqkv, *wo, *w1, *w2, *w3;  // raw F16 rows [out][in]
};
struct CxStage {
  std::vector<float> ct_w, ct_b, gamma, dw_w, dw_b, ln_w, ln_b, pw1_b, pw2_b;
  const uint8_t *pw1, *pw2;
};
struct CxRes {
  std::vector<float> a0, w0, b0, a1, w1, b1;
};
struct CxBlock {
  std::vector<float> alpha, ct_w, ct_b;
  CxRes res[3];
};

}  // namespace

struct orc_codec {
  Gguf g;
  Pool pool;
  std::vector<float> cb[10], proj_w[10], proj_b[10];
  CxLayer layers[CX_LAYERS];
  std::vector<float> post_norm;
  CxStage stages[2];
  std::vector<float> entry_w, entry_b, tail_alpha, out_w, out_b;
  CxBlock blocks[4];
  explicit orc_codec(unsigned threads) : pool(threads) {}
};

namespace {

// F16TensorView::from_gguf (tensor.rs:21-45) plus validate_f16_dims (codec.rs:3751-3759)
std::vector<float> cx_tensor(const Gguf& g, const std::string& name, std::vector<uint64_t> dims) {
  const TensorInfo& t = g.tensor(name);
  if (t.type != T_F16) fail("expected F16 tensor %s, got type %u", name.c_str(), t.type);
  if (t.dims != dims) fail("codec tensor %s has unexpected dimensions", name.c_str());
  std::vector<float> v(t.elements());
  const uint16_t* p = reinterpret_cast<const uint16_t*>(t.data);
  for (size_t i = 0; i < v.size(); ++i) v[i] = f16_to_f32(p[i]);
  return v;
}
const uint8_t* cx_raw(const Gguf& g, const std::string& name, std::vector<uint64_t> dims) {
  const TensorInfo& t = g.tensor(name);
  if (t.type != T_F16) fail("expected F16 tensor %s, got type %u", name.c_str(), t.type);
  if (t.dims != dims) fail("codec tensor %s has unexpected dimensions", name.c_str());
  return t.data;
}

void cx_load(orc_codec* c) {
  const Gguf& g = c->g;
  auto it = g.meta.find("general.architecture");
  if (it == g.meta.end()) fail("missing general.architecture");
  if (it->second.s != "fish-speech-codec") fail("expected fish-speech-codec codec GGUF, got %s", it->second.s.c_str());
  for (size_t q = 0; q < 10; ++q) {
    const std::string p = q == 0 ? "quantizer.semantic_quantizer.quantizers.0"
                                 : "quantizer.quantizer.quantizers." + std::to_string(q - 1);
    c->cb[q] = cx_tensor(g, p + ".codebook.weight", {CX_PROJ, q == 0 ? CX_SEM_CB : CX_RES_CB});
    c->proj_w[q] = cx_tensor(g, p + ".out_proj.weight", {CX_PROJ, CX_HIDDEN});
    c->proj_b[q] = cx_tensor(g, p + ".out_proj.bias", {CX_HIDDEN});
  }
  for (size_t l = 0; l < CX_LAYERS; ++l) {
    const std::string p = "quantizer.post_module.layers." + std::to_string(l);
    CxLayer& L = c->layers[l];
    L.attn_norm = cx_tensor(g, p + ".attention_norm.weight", {CX_HIDDEN});
    L.ffn_norm = cx_tensor(g, p + ".ffn_norm.weight", {CX_HIDDEN});
    L.als = cx_tensor(g, p + ".attention_layer_scale.gamma", {CX_HIDDEN});
    L.fls = cx_tensor(g, p + ".ffn_layer_scale.gamma", {CX_HIDDEN});
    L.wqkv = cx_raw(g, p + ".attention.wqkv.weight", {CX_HIDDEN, CX_QKV});
    L.wo = cx_raw(g, p + ".attention.wo.weight", {CX_HIDDEN, CX_HIDDEN});
    L.w1 = cx_raw(g, p + ".feed_forward.w1.weight", {CX_HIDDEN, CX_FFN});
    L.w2 = cx_raw(g, p + ".feed_forward.w2.weight", {CX_FFN, CX_HIDDEN});
    L.w3 = cx_raw(g, p + ".feed_forward.w3.weight", {CX_HIDDEN, CX_FFN});
  }
  c->post_norm = cx_tensor(g, "quantizer.post_module.norm.weight", {CX_HIDDEN});
  for (size_t s = 0; s < 2; ++s) {
    const std::string p = "quantizer.upsample." + std::to_string(s);
    CxStage& S = c->stages[s];
    S.ct_w = cx_tensor(g, p + ".0.conv.weight", {2, CX_HIDDEN, CX_HIDDEN});
    S.ct_b = cx_tensor(g, p + ".0.conv.bias", {CX_HIDDEN});
    S.gamma = cx_tensor(g, p + ".1.gamma", {CX_HIDDEN});
    S.dw_w = cx_tensor(g, p + ".1.dwconv.conv.weight", {CX_DW_K, 1, CX_HIDDEN});
    S.dw_b = cx_tensor(g, p + ".1.dwconv.conv.bias", {CX_HIDDEN});
    S.ln_w = cx_tensor(g, p + ".1.norm.weight", {CX_HIDDEN});
    S.ln_b = cx_tensor(g, p + ".1.norm.bias", {CX_HIDDEN});
    S.pw1 = cx_raw(g, p + ".1.pwconv1.weight", {CX_HIDDEN, CX_EXPANDED});
    S.pw1_b = cx_tensor(g, p + ".1.pwconv1.bias", {CX_EXPANDED});
    S.pw2 = cx_raw(g, p + ".1.pwconv2.weight", {CX_EXPANDED, CX_HIDDEN});
    S.pw2_b = cx_tensor(g, p + ".1.pwconv2.bias", {CX_HIDDEN});
  }
  c->entry_w = cx_tensor(g, "decoder.model.0.conv.weight", {7, CX_HIDDEN, CX_ENTRY});
  c->entry_b = cx_tensor(g, "decoder.model.0.conv.bias", {CX_ENTRY});
  for (size_t b = 0; b < 4; ++b) {
    const std::string p = "decoder.model." + std::to_string(b + 1) + ".block";
    const uint64_t ci = CX_CH[b], co = CX_CH[b + 1];
    CxBlock& B = c->blocks[b];
    B.alpha = cx_tensor(g, p + ".0.alpha", {1, ci, 1});
    B.ct_w = cx_tensor(g, p + ".1.conv.weight", {2 * CX_RATES[b], co, ci});
    B.ct_b = cx_tensor(g, p + ".1.conv.bias", {co});
    for (size_t r = 0; r < 3; ++r) {
      const std::string q = p + "." + std::to_string(r + 2) + ".block";
      CxRes& R = B.res[r];
      R.a0 = cx_tensor(g, q + ".0.alpha", {1, co, 1});
      R.w0 = cx_tensor(g, q + ".1.conv.weight", {7, co, co});
      R.b0 = cx_tensor(g, q + ".1.conv.bias", {co});
      R.a1 = cx_tensor(g, q + ".2.alpha", {1, co, 1});
      R.w1 = cx_tensor(g, q + ".3.conv.weight", {1, co, co});
      R.b1 = cx_tensor(g, q + ".3.conv.bias", {co});
    }
  }
  c->tail_alpha = cx_tensor(g, "decoder.model.5.alpha", {1, 96, 1});
  c->out_w = cx_tensor(g, "decoder.model.6.conv.weight", {7, 96, 1});
  c->out_b = cx_tensor(g, "decoder.model.6.conv.bias", {1});
}

// rvq_lookup_codes (codec.rs:2536-2596) with project_code (:2428-2445) and
// embedding_lookup_rows (tensor.rs:160-193): latents start at 0 and add each
// codebook's projection (codebook row . out_proj row + bias) in codebook order.
void cx_rvq_lookup(orc_codec* c, const int32_t* codes, uint32_t ncb, uint32_t n_frames, float* latents) {
  if (ncb != 10) fail("codec codebook count mismatch: expected 10, got %u", ncb);
  const size_t F = n_frames;
  std::fill(latents, latents + F * CX_HIDDEN, 0.0f);
  std::vector<float> proj(CX_HIDDEN);
  for (size_t f = 0; f < F; ++f) {
    for (size_t q = 0; q < ncb; ++q) {
      const int32_t code = codes[q * F + f];
      if (code < 0) fail("codec code must be non-negative, got %d", code);
      const size_t size = q == 0 ? CX_SEM_CB : CX_RES_CB;
      if (size_t(code) >= size) fail("embedding index %d out of range for vocab_dim %zu", code, size);
      const float* z = c->cb[q].data() + size_t(code) * CX_PROJ;
      for (size_t o = 0; o < CX_HIDDEN; ++o)
        proj[o] = dot(z, c->proj_w[q].data() + o * CX_PROJ, CX_PROJ) + c->proj_b[q][o];
      float* row = latents + f * CX_HIDDEN;
      for (size_t o = 0; o < CX_HIDDEN; ++o) row[o] += proj[o];
    }
  }
}

// forward_codec_post_module (codec.rs:986-1018) over
// forward_codec_transformer_layer_with_window (:3229-3336): window 128,
// 16 heads of 64 (no GQA sharing), RoPE base 1e4 at the frame position,
// attention scale 1/sqrt(64), layer scales on both residual branches.
void cx_post_module(orc_codec* c, const float* latents, uint32_t n_frames, float* hidden) {
  if (n_frames == 0) fail("codec transformer requires at least one frame");
  const size_t T = n_frames, D = CX_HIDDEN;
  std::vector<float> x(latents, latents + T * D), nrm(T * D), qkv(T * CX_QKV), att(T * D), proj(T * D);
  std::vector<float> g(T * CX_FFN), u(T * CX_FFN), act(T * CX_FFN);
  std::vector<float> keys, vals;
  for (size_t l = 0; l < CX_LAYERS; ++l) {
    const CxLayer& L = c->layers[l];
    for (size_t t = 0; t < T; ++t) rms_norm(&x[t * D], L.attn_norm.data(), D, CX_RMS_EPS, &nrm[t * D]);
    linear_multi(c->pool, nrm.data(), T, L.wqkv, T_F16, D, CX_QKV, qkv.data());
    for (size_t t = 0; t < T; ++t) {
      rope_normal(&qkv[t * CX_QKV], D, CX_HD, t, CX_ROPE_BASE);
      rope_normal(&qkv[t * CX_QKV + D], D, CX_HD, t, CX_ROPE_BASE);
    }
    c->pool.run(T, 4, [&](size_t t0, size_t t1) {
      std::vector<float> k, v;
      for (size_t t = t0; t < t1; ++t) {
        const size_t start = t + 1 > CX_WINDOW ? t + 1 - CX_WINDOW : 0, n = t + 1 - start;
        k.resize(n * D);
        v.resize(n * D);
        for (size_t j = 0; j < n; ++j) {
          std::copy_n(&qkv[(start + j) * CX_QKV + D], D, &k[j * D]);
          std::copy_n(&qkv[(start + j) * CX_QKV + 2 * D], D, &v[j * D]);
        }
        gqa_attention(&qkv[t * CX_QKV], k.data(), v.data(), CX_HEADS, CX_HEADS, CX_HD, n, 1.0f / std::sqrt(64.0f),
                      &att[t * D]);
      }
    });
    linear_multi(c->pool, att.data(), T, L.wo, T_F16, D, D, proj.data());
    for (size_t t = 0; t < T; ++t)
      for (size_t i = 0; i < D; ++i) x[t * D + i] = x[t * D + i] + proj[t * D + i] * L.als[i];
    for (size_t t = 0; t < T; ++t) rms_norm(&x[t * D], L.ffn_norm.data(), D, CX_RMS_EPS, &nrm[t * D]);
    linear_multi(c->pool, nrm.data(), T, L.w1, T_F16, D, CX_FFN, g.data());
    linear_multi(c->pool, nrm.data(), T, L.w3, T_F16, D, CX_FFN, u.data());
    for (size_t i = 0; i < T * CX_FFN; ++i) act[i] = cx_silu(g[i]) * u[i];
    linear_multi(c->pool, act.data(), T, L.w2, T_F16, CX_FFN, D, proj.data());
    for (size_t t = 0; t < T; ++t)
      for (size_t i = 0; i < D; ++i) x[t * D + i] = x[t * D + i] + proj[t * D + i] * L.fls[i];
  }
  for (size_t t = 0; t < T; ++t) rms_norm(&x[t * D], c->post_norm.data(), D, CX_RMS_EPS, hidden + t * D);
}

// forward_codec_upsample (codec.rs:2302-2325): two stages of
// forward_codec_upsample_stage (:3338-3358) = conv_transpose (stride 2,
// kernel 2) then forward_codec_convnext_block (:3438-3483).
void cx_upsample(orc_codec* c, const float* hidden, uint32_t n_frames, float* out) {
  size_t F = n_frames;
  const size_t D = CX_HIDDEN;
  std::vector<float> cur(hidden, hidden + F * D);
  for (size_t s = 0; s < 2; ++s) {
    const CxStage& S = c->stages[s];
    std::vector<float> conv(2 * F * D);
    cx_conv_transpose(c->pool, cur.data(), F, D, D, 2, S.ct_w.data(), S.ct_w.size(), S.ct_b.data(), conv.data());
    F *= 2;
    std::vector<float> x(F * D), h(F * CX_EXPANDED), y(F * D);
    cx_depthwise(conv.data(), F, D, CX_DW_K, S.dw_w.data(), S.dw_b.data(), x.data());
    cx_layer_norm(x.data(), F, D, S.ln_w.data(), S.ln_b.data(), CX_LN_EPS);
    // linear_bias_frame_major (:3656-3679): linear, then + bias
    linear_multi(c->pool, x.data(), F, S.pw1, T_F16, D, CX_EXPANDED, h.data());
    for (size_t f = 0; f < F; ++f)
      for (size_t i = 0; i < CX_EXPANDED; ++i) h[f * CX_EXPANDED + i] = cx_gelu(h[f * CX_EXPANDED + i] + S.pw1_b[i]);
    linear_multi(c->pool, h.data(), F, S.pw2, T_F16, CX_EXPANDED, D, y.data());
    cur.resize(F * D);
    for (size_t f = 0; f < F; ++f)
      for (size_t i = 0; i < D; ++i) {
        const float v = (y[f * D + i] + S.pw2_b[i]) * S.gamma[i];
        cur[f * D + i] = conv[f * D + i] + v;
      }
  }
  std::copy(cur.begin(), cur.end(), out);
}

// forward_codec_decoder (codec.rs:1941-2001) with forward_codec_decoder_block
// (:2015-2044) and forward_codec_residual_unit_impl (:2085-2160).
// stop_block <= 4 returns the residual stream after that many blocks
// (frames * prod(rates[0..stop_block]) x channels), a stage checkpoint;
// 5 and above run the whole decoder.
void cx_decoder(orc_codec* c, const float* hidden, uint32_t n_frames, uint32_t hidden_dim, float* out,
                uint32_t stop_block = 5) {
  if (hidden_dim != CX_HIDDEN) fail("decoder expects latent dim %zu, got %u", CX_HIDDEN, hidden_dim);
  size_t F = n_frames;
  std::vector<float> x(F * CX_ENTRY);
  cx_conv1d(c->pool, hidden, F, CX_HIDDEN, CX_ENTRY, 1, c->entry_w.data(), c->entry_w.size(), c->entry_b.data(),
            x.data());
  size_t ch = CX_ENTRY;
  for (size_t b = 0; b < 4 && b < stop_block; ++b) {
    const CxBlock& B = c->blocks[b];
    const size_t co = CX_CH[b + 1], s = CX_RATES[b];
    std::vector<float> sn(F * ch);
    cx_snake(x.data(), F, ch, B.alpha.data(), sn.data());
    std::vector<float> y(F * s * co);
    cx_conv_transpose(c->pool, sn.data(), F, ch, co, s, B.ct_w.data(), B.ct_w.size(), B.ct_b.data(), y.data());
    F *= s;
    ch = co;
    x.swap(y);
    std::vector<float> br(F * ch), br2(F * ch);
    const size_t dil[3] = {1, 3, 9};
    for (size_t r = 0; r < 3; ++r) {
      const CxRes& R = B.res[r];
      cx_snake(x.data(), F, ch, R.a0.data(), br.data());
      cx_conv1d(c->pool, br.data(), F, ch, ch, dil[r], R.w0.data(), R.w0.size(), R.b0.data(), br2.data());
      cx_snake(br2.data(), F, ch, R.a1.data(), br.data());
      cx_conv1d(c->pool, br.data(), F, ch, ch, 1, R.w1.data(), R.w1.size(), R.b1.data(), br2.data());
      for (size_t i = 0; i < F * ch; ++i) x[i] = x[i] + br2[i];
    }
  }
  if (stop_block <= 4) {
    std::copy(x.begin(), x.end(), out);
    return;
  }
  std::vector<float> sn(F * ch);
  cx_snake(x.data(), F, ch, c->tail_alpha.data(), sn.data());
  cx_conv1d(c->pool, sn.data(), F, ch, 1, 1, c->out_w.data(), c->out_w.size(), c->out_b.data(), out);
  for (size_t i = 0; i < F; ++i) out[i] = tanhf(out[i]);
}

}  // namespace

extern "C" {

orc_codec* orc_codec_open(const char* path, uint32_t threads, char* err, size_t cap) {
  try {
    std::unique_ptr<orc_codec> c(new orc_codec(threads ? threads : std::max(1u, std::thread::hardware_concurrency())));
    c->g.open_file(path);
    cx_load(c.get());
    return c.release();
  } catch (const std::exception& e) {
    copy_err(e, err, cap);
    return nullptr;
  }
}

void orc_codec_close(orc_codec* c) { delete c; }

int32_t orc_codec_rvq_lookup(orc_codec* c, const int32_t* codes, uint32_t ncb, uint32_t n_frames, float* latents,
                             char* err, size_t cap) {
  try {
    cx_rvq_lookup(c, codes, ncb, n_frames, latents);
    return 1;
  } catch (const std::exception& e) {
    copy_err(e, err, cap);
    return 0;
  }
}

int32_t orc_codec_post_module(orc_codec* c, const float* latents, uint32_t n_frames, float* hidden, char* err,
                              size_t cap) {
  try {
    cx_post_module(c, latents, n_frames, hidden);
    return 1;
  } catch (const std::exception& e) {
    copy_err(e, err, cap);
    return 0;
  }
}

int32_t orc_codec_upsample(orc_codec* c, const float* hidden, uint32_t n_frames, float* out, char* err, size_t cap) {
  try {
    cx_upsample(c, hidden, n_frames, out);
    return 1;
  } catch (const std::exception& e) {
    copy_err(e, err, cap);
    return 0;
  }
}

int32_t orc_codec_decoder(orc_codec* c, const float* hidden, uint32_t n_frames, uint32_t hidden_dim,
                          uint32_t stop_block, float* out, char* err, size_t cap) {
  try {
    cx_decoder(c, hidden, n_frames, hidden_dim, out, stop_block);
    return 1;
  } catch (const std::exception& e) {
    copy_err(e, err, cap);
    return 0;
  }
}

int32_t orc_codec_decode_waveform(orc_codec* c, const int32_t* codes, uint32_t ncb, uint32_t n_frames,
                                  float* samples, char* err, size_t cap) {
  try {
    std::vector<float> lat(size_t(n_frames) * CX_HIDDEN), post(size_t(n_frames) * CX_HIDDEN);
    std::vector<float> up(size_t(n_frames) * 4 * CX_HIDDEN);
    cx_rvq_lookup(c, codes, ncb, n_frames, lat.data());
    cx_post_module(c, lat.data(), n_frames, post.data());
    cx_upsample(c, post.data(), n_frames, up.data());
    cx_decoder(c, up.data(), n_frames * 4, CX_HIDDEN, samples);
    return 1;
  } catch (const std::exception& e) {
    copy_err(e, err, cap);
    return 0;
  }
}

void orc_codec_snake(const float* x, size_t frames, size_t ch, const float* alpha, float* out) {
  cx_snake(x, frames, ch, alpha, out);
}

int32_t orc_codec_conv1d(const float* x, size_t frames, size_t in_ch, size_t out_ch, size_t dilation,
                         const float* w, size_t w_len, const float* bias, float* out, char* err, size_t cap) {
  try {
    Pool pool(1);
    cx_conv1d(pool, x, frames, in_ch, out_ch, dilation, w, w_len, bias, out);
    return 1;
  } catch (const std::exception& e) {
    copy_err(e, err, cap);
    return 0;
  }
}

int32_t orc_codec_conv_transpose(const float* x, size_t frames, size_t in_ch, size_t out_ch, size_t stride,
                                 const float* w, size_t w_len, const float* bias, float* out, char* err, size_t cap) {
  try {
    Pool pool(1);
    cx_conv_transpose(pool, x, frames, in_ch, out_ch, stride, w, w_len, bias, out);
    return 1;
  } catch (const std::exception& e) {
    copy_err(e, err, cap);
    return 0;
  }
}

void orc_codec_depthwise(const float* x, size_t frames, size_t ch, size_t k, const float* w, const float* bias,
                         float* out) {
  cx_depthwise(x, frames, ch, k, w, bias, out);
}

void orc_codec_layer_norm(float* x, size_t frames, size_t ch, const float* w, const float* b, float eps) {
  cx_layer_norm(x, frames, ch, w, b, eps);
}

float orc_codec_erf(float v) { return cx_erf(v); }
float orc_codec_gelu(float v) { return cx_gelu(v); }

}  // extern "C"
