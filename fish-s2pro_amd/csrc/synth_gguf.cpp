// synth_gguf.cpp -- seeded synthetic dual-AR GGUF writer (host only).
//
// Writes a GGUF v3 file with the tensor names, shapes and metadata keys the
// reference's registry reads (crates/fish_s2_infer/src/registry.rs:45-99,
// 360-496, 625-650), filled with random-init weights: N(0, std) rounded to
// f16 (round-to-nearest-even), RMSNorm gains = 1.  Linear weights can be
// written as GGML Q8_0 or Q4_0 blocks quantised from those f16 values.
//
// The generator is counter based (SplitMix64 + Box-Muller in double), so a
// tensor's values depend only on (seed, tensor index, element index) and not
// on thread scheduling.

#include "synth_gguf.h"

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

namespace {

struct SynthError : std::runtime_error {
  explicit SynthError(const std::string& m) : std::runtime_error(m) {}
};

[[noreturn]] void fail(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  throw SynthError(buf);
}

uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

// IEEE binary32 -> binary16, round to nearest even (overflow -> inf).
uint16_t to_half(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t absx = x & 0x7fffffffu;
  if (absx >= 0x7f800000u) return uint16_t(sign | 0x7c00u | (absx > 0x7f800000u ? 0x200u : 0u));
  if (absx >= 0x477ff000u) return uint16_t(sign | 0x7c00u);  // rounds to >= 65520
  if (absx < 0x38800000u) {                                  // below the smallest normal half
    if (absx < 0x33000000u) return uint16_t(sign);           // < 2^-25 rounds to 0
    const uint32_t e = absx >> 23;
    const uint32_t mant = (absx & 0x7fffffu) | 0x800000u;
    const uint32_t shift = 126u - e;  // value = mant * 2^(e-150); half ulp 2^-24
    uint32_t q = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t halfway = 1u << (shift - 1u);
    if (rem > halfway || (rem == halfway && (q & 1u))) ++q;
    return uint16_t(sign | q);
  }
  uint32_t h = ((absx >> 13) - (112u << 10));
  const uint32_t rem = absx & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
  return uint16_t(sign | h);
}

float from_half(uint16_t h) {
  const uint32_t sign = uint32_t(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0) {
    float v = std::ldexp(float(m), -24);
    return sign ? -v : v;
  }
  uint32_t bits = e == 0x1f ? (sign | 0x7f800000u | (m << 13)) : (sign | ((e + 112u) << 23) | (m << 13));
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

struct Tensor {
  std::string name;
  std::vector<uint64_t> dims;  // ne0 (contiguous) first
  uint32_t type;               // 1 F16, 2 Q4_0, 8 Q8_0
  uint16_t fill;               // RMSNorm gain: every element this f16 value (0: random weights)
  double stdv = -1.0;          // random weights: N(mean, stdv); negative: the file's default std
  double mean = 0.0;
  bool zero_first = false;     // element 0 written as +0 (a zero snake alpha, for instance)
  uint64_t offset = 0;
  uint64_t bytes = 0;
  uint64_t elements() const {
    uint64_t n = 1;
    for (uint64_t d : dims) n *= d;
    return n;
  }
};

uint64_t tensor_bytes(const Tensor& t) {
  const uint64_t n = t.elements();
  if (t.type == 1) return n * 2;
  if (t.type == 8) return n / 32 * 34;
  if (t.type == 2) return n / 32 * 18;
  fail("unsupported tensor type %u", t.type);
}

class Writer {
 public:
  explicit Writer(const char* path) : f_(fopen(path, "wb")) {
    if (!f_) fail("cannot create %s", path);
  }
  ~Writer() {
    if (f_) fclose(f_);
  }
  void bytes(const void* p, size_t n) {
    if (n && fwrite(p, 1, n, f_) != n) fail("write failed");
    pos_ += n;
  }
  template <class T>
  void put(T v) { bytes(&v, sizeof v); }
  void str(const std::string& s) {
    put<uint64_t>(s.size());
    bytes(s.data(), s.size());
  }
  void pad(uint64_t align) {
    static const uint8_t zeros[64] = {0};
    while (pos_ % align) bytes(zeros, size_t(std::min<uint64_t>(align - pos_ % align, 64)));
  }
  void close() {
    if (fclose(f_) != 0) fail("close failed");
    f_ = nullptr;
  }
  uint64_t pos() const { return pos_; }

 private:
  FILE* f_;
  uint64_t pos_ = 0;
};

struct Meta {
  std::string key;
  uint32_t type;  // 4 u32, 6 f32, 7 bool, 8 string
  uint32_t u = 0;
  float f = 0;
  std::string s;
};

// One f16 weight value: N(mean, std) from (seed, tensor, element).
inline uint16_t weight_half(uint64_t tkey, uint64_t e, double stdv, double mean = 0.0) {
  const uint64_t p = e >> 1;
  const uint64_t h1 = splitmix64(tkey + 2 * p), h2 = splitmix64(tkey + 2 * p + 1);
  const double u1 = double((h1 >> 11) + 1) * 0x1.0p-53;  // (0, 1]
  const double u2 = double(h2 >> 11) * 0x1.0p-53;        // [0, 1)
  const double r = std::sqrt(-2.0 * std::log(u1));
  const double a = 6.283185307179586 * u2;
  const double z = (e & 1) ? r * std::sin(a) : r * std::cos(a);
  return to_half(float(mean + stdv * z));
}

// GGML Q8_0: d = max|x| / 127, q = round(x / d) (round half away from zero).
void quant_q8_0(const float* x, uint8_t* out) {
  float amax = 0.0f;
  for (int j = 0; j < 32; ++j) amax = std::fmax(amax, std::fabs(x[j]));
  const float d = amax / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  const uint16_t dh = to_half(d);
  memcpy(out, &dh, 2);
  for (int j = 0; j < 32; ++j) out[2 + j] = uint8_t(int8_t(std::lround(x[j] * id)));
}

// GGML Q4_0: d = (signed value of largest magnitude) / -8,
// q = min(15, trunc(x / d + 8.5)); element j -> low nibble of qs[j],
// element 16+j -> high nibble.
void quant_q4_0(const float* x, uint8_t* out) {
  float amax = 0.0f, maxv = 0.0f;
  for (int j = 0; j < 32; ++j) {
    if (std::fabs(x[j]) > amax) {
      amax = std::fabs(x[j]);
      maxv = x[j];
    }
  }
  const float d = maxv / -8.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  const uint16_t dh = to_half(d);
  memcpy(out, &dh, 2);
  for (int j = 0; j < 16; ++j) {
    int lo = int(int8_t(x[j] * id + 8.5f));
    int hi = int(int8_t(x[16 + j] * id + 8.5f));
    lo = lo > 15 ? 15 : lo;
    hi = hi > 15 ? 15 : hi;
    out[2 + j] = uint8_t(lo | (hi << 4));
  }
}

void fill_rows(const Tensor& t, uint64_t tkey, double stdv, uint64_t r0, uint64_t r1, uint8_t* dst) {
  const uint64_t in = t.dims[0];
  if (t.stdv >= 0.0) stdv = t.stdv;
  std::vector<float> row(in);
  const uint64_t rb = t.type == 1 ? in * 2 : (t.type == 8 ? in / 32 * 34 : in / 32 * 18);
  for (uint64_t r = r0; r < r1; ++r) {
    uint8_t* out = dst + (r - r0) * rb;
    if (t.type == 1) {
      uint16_t* o = reinterpret_cast<uint16_t*>(out);
      for (uint64_t i = 0; i < in; ++i) o[i] = t.fill ? t.fill : weight_half(tkey, r * in + i, stdv, t.mean);
      if (t.zero_first && r == 0) o[0] = 0;
      continue;
    }
    for (uint64_t i = 0; i < in; ++i) row[i] = from_half(weight_half(tkey, r * in + i, stdv));
    for (uint64_t b = 0; b < in / 32; ++b) {
      if (t.type == 8)
        quant_q8_0(row.data() + b * 32, out + b * 34);
      else
        quant_q4_0(row.data() + b * 32, out + b * 18);
    }
  }
}

// Writes the GGUF v3 header (metadata, tensor table) and every tensor's
// seeded values.  Tensor values depend on (seed, table position, element).
void emit_gguf(const char* path, const std::vector<Meta>& meta, std::vector<Tensor>& ts, uint64_t seed,
               double stdv, unsigned threads) {
  uint64_t off = 0;
  for (Tensor& t : ts) {
    t.offset = off;
    t.bytes = tensor_bytes(t);
    off = (off + t.bytes + 31) / 32 * 32;
  }
  Writer w(path);
  w.bytes("GGUF", 4);
  w.put<uint32_t>(3);
  w.put<uint64_t>(ts.size());
  w.put<uint64_t>(meta.size());
  for (const Meta& m : meta) {
    w.str(m.key);
    w.put<uint32_t>(m.type);
    if (m.type == 4) w.put<uint32_t>(m.u);
    if (m.type == 6) w.put<float>(m.f);
    if (m.type == 7) w.put<uint8_t>(uint8_t(m.u));
    if (m.type == 8) w.str(m.s);
  }
  for (const Tensor& t : ts) {
    w.str(t.name);
    w.put<uint32_t>(uint32_t(t.dims.size()));
    for (uint64_t dd : t.dims) w.put<uint64_t>(dd);
    w.put<uint32_t>(t.type);
    w.put<uint64_t>(t.offset);
  }
  w.pad(32);
  const uint64_t data_start = w.pos();
  const unsigned nt = threads ? threads : std::max(1u, std::thread::hardware_concurrency());
  std::vector<uint8_t> buf;
  const bool progress = getenv("S2SYNTH_PROGRESS") != nullptr;
  uint64_t reported = 0;
  for (size_t ti = 0; ti < ts.size(); ++ti) {
    const Tensor& t = ts[ti];
    const uint64_t tkey = splitmix64(seed ^ splitmix64(0x5EED0000ull + ti));
    const uint64_t rows = t.dims.empty() ? 1 : t.elements() / t.dims[0];
    const uint64_t rb = t.bytes / rows;
    buf.resize(t.bytes);
    std::vector<std::thread> pool;
    const uint64_t per = (rows + nt - 1) / nt;
    for (unsigned k = 0; k < nt; ++k) {
      const uint64_t r0 = k * per, r1 = std::min(rows, r0 + per);
      if (r0 >= r1) break;
      pool.emplace_back([&, r0, r1] { fill_rows(t, tkey, stdv, r0, r1, buf.data() + r0 * rb); });
    }
    for (auto& th : pool) th.join();
    if (w.pos() != data_start + t.offset) fail("internal offset mismatch for %s", t.name.c_str());
    w.bytes(buf.data(), buf.size());
    w.pad(32);
    if (progress && (w.pos() >> 30) != reported) {
      reported = w.pos() >> 30;
      fprintf(stderr, "[s2synth] %s: %.2f GB written\n", path, double(w.pos()) / 1e9);
    }
  }
  w.close();
}

void write_gguf(const char* path, const s2synth_config& c, unsigned threads) {
  if (c.linear_type != 1 && c.linear_type != 8 && c.linear_type != 2) fail("linear_type must be 1, 2 or 8");
  if (c.heads % c.kv_heads || c.fast_heads % c.fast_kv_heads) fail("invalid GQA split");
  if (c.semantic_end < c.semantic_begin || c.semantic_end >= c.vocab) fail("invalid semantic range");
  if (c.linear_type != 1) {
    if (c.dim % 32 || c.ffn % 32 || (c.heads * c.head_dim) % 32 || c.fast_ffn % 32 ||
        (c.fast_heads * c.fast_head_dim) % 32)
      fail("quantised linears need every input dimension to be a multiple of 32");
  }
  const uint64_t d = c.dim;
  const uint64_t q = uint64_t(c.heads) * c.head_dim, kv = uint64_t(c.kv_heads) * c.head_dim;
  const uint64_t fq = uint64_t(c.fast_heads) * c.fast_head_dim, fkv = uint64_t(c.fast_kv_heads) * c.fast_head_dim;
  std::vector<Tensor> ts;
  // gains: 0 = random weights, 1 = unit gain (QK-norm), 2 = the residual-stream gain
  const uint16_t gain_bits = to_half(c.norm_gain != 0.0f ? c.norm_gain : 1.0f);
  auto add = [&](const std::string& n, std::vector<uint64_t> dims, uint32_t type, int gain) {
    ts.push_back(Tensor{n, dims, type, uint16_t(gain == 0 ? 0u : gain == 1 ? 0x3c00u : gain_bits)});
  };
  const uint32_t lt = c.linear_type;
  add("embeddings.weight", {d, c.vocab}, 1, 0);
  add("codebook_embeddings.weight", {d, uint64_t(c.codebook_size) * c.num_codebooks}, 1, 0);
  add("norm.weight", {d}, 1, 2);
  add("fast_embeddings.weight", {d, c.codebook_size}, 1, 0);
  add("fast_norm.weight", {d}, 1, 2);
  add("fast_output.weight", {d, c.codebook_size}, lt, 0);
  for (uint32_t l = 0; l < c.slow_layers; ++l) {
    const std::string p = "layers." + std::to_string(l) + ".";
    add(p + "attention_norm.weight", {d}, 1, 2);
    add(p + "attention.q_norm.weight", {c.head_dim}, 1, 1);
    add(p + "attention.k_norm.weight", {c.head_dim}, 1, 1);
    add(p + "attention.wqkv.weight", {d, q + 2 * kv}, lt, 0);
    add(p + "attention.wo.weight", {q, d}, lt, 0);
    add(p + "ffn_norm.weight", {d}, 1, 2);
    add(p + "feed_forward.w1.weight", {d, c.ffn}, lt, 0);
    add(p + "feed_forward.w2.weight", {c.ffn, d}, lt, 0);
    add(p + "feed_forward.w3.weight", {d, c.ffn}, lt, 0);
  }
  for (uint32_t l = 0; l < c.fast_layers; ++l) {
    const std::string p = "fast_layers." + std::to_string(l) + ".";
    add(p + "attention_norm.weight", {d}, 1, 2);
    add(p + "attention.wqkv.weight", {d, fq + 2 * fkv}, lt, 0);
    add(p + "attention.wo.weight", {fq, d}, lt, 0);
    add(p + "ffn_norm.weight", {d}, 1, 2);
    add(p + "feed_forward.w1.weight", {d, c.fast_ffn}, lt, 0);
    add(p + "feed_forward.w2.weight", {c.fast_ffn, d}, lt, 0);
    add(p + "feed_forward.w3.weight", {d, c.fast_ffn}, lt, 0);
  }
  std::vector<Meta> meta;
  auto mu = [&](const char* k, uint32_t v) { meta.push_back(Meta{k, 4, v, 0, ""}); };
  auto mf = [&](const char* k, float v) { meta.push_back(Meta{k, 6, 0, v, ""}); };
  auto mb = [&](const char* k, bool v) { meta.push_back(Meta{k, 7, v ? 1u : 0u, 0, ""}); };
  meta.push_back(Meta{"general.architecture", 8, 0, 0, "fish-speech"});
  meta.push_back(Meta{"general.name", 8, 0, 0, "s2hip-synthetic"});
  mu("fish-speech.context_length", c.context_length);
  mu("fish-speech.embedding_length", c.dim);
  mu("fish-speech.feed_forward_length", c.ffn);
  mu("fish-speech.block_count", c.slow_layers);
  mu("fish-speech.attention.head_count", c.heads);
  mu("fish-speech.attention.head_count_kv", c.kv_heads);
  mf("fish-speech.rope.freq_base", c.rope_base);
  mf("fish-speech.attention.layer_norm_rms_epsilon", c.eps);
  mb("fish_speech.attention_qk_norm", true);
  mu("fish_speech.fast_context_length", c.num_codebooks + 1);
  mu("fish_speech.fast_embedding_length", c.dim);
  mu("fish_speech.fast_feed_forward_length", c.fast_ffn);
  mu("fish_speech.fast_block_count", c.fast_layers);
  mu("fish_speech.fast_head_count", c.fast_heads);
  mu("fish_speech.fast_head_count_kv", c.fast_kv_heads);
  mu("fish_speech.fast_head_dim", c.fast_head_dim);
  mf("fish_speech.fast_rope_freq_base", c.fast_rope_base);
  mf("fish_speech.fast_layer_norm_rms_eps", c.fast_eps);
  mb("fish_speech.fast_attention_qk_norm", false);
  mu("fish_speech.codebook_size", c.codebook_size);
  mu("fish_speech.num_codebooks", c.num_codebooks);
  mu("fish_speech.semantic_begin_id", c.semantic_begin);
  mu("fish_speech.semantic_end_id", c.semantic_end);
  mb("fish_speech.scale_codebook_embeddings", true);
  mb("fish_speech.tie_word_embeddings", true);
  mb("fish_speech.fast_project_in", false);
  emit_gguf(path, meta, ts, c.seed, c.init_std, threads);
}



// Decode side of the codec GGUF (tensor names and ggml dims as the
// reference's codec registry reads them, crates/fish_s2_infer/src/codec.rs:
// quantizers :277-296, post_module layers :316-331 and norm :515, upsample
// stages :431-444, decoder :1299-1317, 1393-1420 and the dims checked at
// :1643-1681; decoder block conv_transpose kernels are 2 x stride, residual
// units k7 then k1).  Weights are N(0, 1/sqrt(fan_in)) so activations stay
// O(1) through the decoder; norms, layer scales and snake alphas are drawn
// around their working values, and element 0 of every snake alpha is 0 so the
// reference's near-zero alpha guard is exercised.
void write_codec_gguf(const char* path, uint64_t seed, unsigned threads) {
  std::vector<Tensor> ts;
  auto add = [&](const std::string& n, std::vector<uint64_t> dims, double stdv, double mean = 0.0,
                 bool zero_first = false) {
    Tensor t{n, dims, 1, 0};
    t.stdv = stdv;
    t.mean = mean;
    t.zero_first = zero_first;
    ts.push_back(t);
  };
  const uint64_t H = 1024, P = 8;
  auto quantizer = [&](const std::string& p, uint64_t size) {
    add(p + ".in_proj.weight", {H, P}, 1.0 / 32.0);
    add(p + ".in_proj.bias", {P}, 0.02);
    add(p + ".out_proj.weight", {P, H}, 1.0 / std::sqrt(8.0));
    add(p + ".out_proj.bias", {H}, 0.02);
    add(p + ".codebook.weight", {P, size}, 1.0);
  };
  quantizer("quantizer.semantic_quantizer.quantizers.0", 4096);
  for (int i = 0; i < 9; ++i) quantizer("quantizer.quantizer.quantizers." + std::to_string(i), 1024);
  for (int l = 0; l < 8; ++l) {
    const std::string p = "quantizer.post_module.layers." + std::to_string(l);
    add(p + ".attention.wqkv.weight", {H, 3072}, 1.0 / 32.0);
    add(p + ".attention.wo.weight", {H, H}, 1.0 / 32.0);
    add(p + ".attention_norm.weight", {H}, 0.1, 1.0);
    add(p + ".ffn_norm.weight", {H}, 0.1, 1.0);
    add(p + ".feed_forward.w1.weight", {H, 3072}, 1.0 / 32.0);
    add(p + ".feed_forward.w2.weight", {3072, H}, 1.0 / std::sqrt(3072.0));
    add(p + ".feed_forward.w3.weight", {H, 3072}, 1.0 / 32.0);
    add(p + ".attention_layer_scale.gamma", {H}, 0.05, 0.3);
    add(p + ".ffn_layer_scale.gamma", {H}, 0.05, 0.3);
  }
  add("quantizer.post_module.norm.weight", {H}, 0.1, 1.0);
  for (int st = 0; st < 2; ++st) {
    const std::string p = "quantizer.upsample." + std::to_string(st);
    add(p + ".0.conv.weight", {2, H, H}, 1.0 / 32.0);
    add(p + ".0.conv.bias", {H}, 0.02);
    add(p + ".1.gamma", {H}, 0.05, 0.3);
    add(p + ".1.dwconv.conv.weight", {7, 1, H}, 1.0 / std::sqrt(7.0));
    add(p + ".1.dwconv.conv.bias", {H}, 0.02);
    add(p + ".1.norm.weight", {H}, 0.1, 1.0);
    add(p + ".1.norm.bias", {H}, 0.1);
    add(p + ".1.pwconv1.weight", {H, 4096}, 1.0 / 32.0);
    add(p + ".1.pwconv1.bias", {4096}, 0.02);
    add(p + ".1.pwconv2.weight", {4096, H}, 1.0 / 64.0);
    add(p + ".1.pwconv2.bias", {H}, 0.02);
  }
  add("decoder.model.0.conv.weight", {7, H, 1536}, 1.0 / std::sqrt(7.0 * 1024.0));
  add("decoder.model.0.conv.bias", {1536}, 0.02);
  const uint64_t ch[5] = {1536, 768, 384, 192, 96};
  const uint64_t rate[4] = {8, 8, 4, 2};
  for (int b = 0; b < 4; ++b) {
    const std::string p = "decoder.model." + std::to_string(b + 1) + ".block";
    const uint64_t ci = ch[b], co = ch[b + 1];
    add(p + ".0.alpha", {1, ci, 1}, 0.2, 1.0, true);
    add(p + ".1.conv.weight", {2 * rate[b], co, ci}, 1.0 / std::sqrt(2.0 * double(ci)));
    add(p + ".1.conv.bias", {co}, 0.02);
    for (int r = 0; r < 3; ++r) {
      const std::string q = p + "." + std::to_string(r + 2) + ".block";
      add(q + ".0.alpha", {1, co, 1}, 0.2, 1.0, true);
      add(q + ".1.conv.weight", {7, co, co}, 1.0 / std::sqrt(7.0 * double(co)));
      add(q + ".1.conv.bias", {co}, 0.02);
      add(q + ".2.alpha", {1, co, 1}, 0.2, 1.0, true);
      add(q + ".3.conv.weight", {1, co, co}, 0.5 / std::sqrt(double(co)));
      add(q + ".3.conv.bias", {co}, 0.02);
    }
  }
  add("decoder.model.5.alpha", {1, 96, 1}, 0.2, 1.0, true);
  add("decoder.model.6.conv.weight", {7, 96, 1}, 0.08 / std::sqrt(7.0 * 96.0));
  add("decoder.model.6.conv.bias", {1}, 0.02);
  std::vector<Meta> meta;
  meta.push_back(Meta{"general.architecture", 8, 0, 0, "fish-speech-codec"});
  meta.push_back(Meta{"general.name", 8, 0, 0, "s2hip-synthetic-codec"});
  emit_gguf(path, meta, ts, seed, 0.02, threads);
}

}  // namespace

extern "C" {

int32_t s2synth_write_gguf(const char* path, const s2synth_config* cfg, uint32_t threads, char* err,
                           size_t err_cap) {
  try {
    write_gguf(path, *cfg, threads);
    return 1;
  } catch (const std::exception& e) {
    if (err && err_cap) snprintf(err, err_cap, "%s", e.what());
    return 0;
  }
}

int32_t s2synth_write_codec_gguf(const char* path, uint64_t seed, uint32_t threads, char* err, size_t err_cap) {
  try {
    write_codec_gguf(path, seed, threads);
    return 1;
  } catch (const std::exception& e) {
    if (err && err_cap) snprintf(err, err_cap, "%s", e.what());
    return 0;
  }
}

uint16_t s2synth_f32_to_f16(float v) { return to_half(v); }

int32_t s2synth_quantize_block(uint32_t type, const float* x, uint8_t* out) {
  if (type == 8) {
    quant_q8_0(x, out);
    return 1;
  }
  if (type == 2) {
    quant_q4_0(x, out);
    return 1;
  }
  return 0;
}

}  // extern "C"
