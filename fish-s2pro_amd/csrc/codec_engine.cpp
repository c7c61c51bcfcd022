// codec_engine.cpp -- RVQ codec decode on the GPU behind the C ABI
// (include/s2hip.h, s2hip_codec_*): decode_waveform
// (crates/fish_s2_infer/src/codec.rs:1690-1714) and its stages.
//
// Weights come from the codec GGUF (decode-side tensors, names and dims as
// the reference's registry reads them) and stay resident in HBM: small
// vectors as f32, transformer linears as their F16 rows (the MFMA prefill
// GEMM's layout), convolution weights packed for conv_gemm_kernel.  Buffers
// are sized once for max_frames code frames.

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "codec.h"
#include "gguf.h"
#include "sin_cw.h"
#include "kernels.h"
#include "s2hip.h"

namespace s2 {
namespace {

struct CodecFailure : std::runtime_error {
  explicit CodecFailure(const std::string& m) : std::runtime_error(m) {}
};
void hipc(hipError_t e, const char* what) {
  if (e != hipSuccess) throw CodecFailure(std::string(what) + ": " + hipGetErrorString(e));
}
#define CHK(expr) hipc((expr), #expr)
[[noreturn]] void cfail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void cfail(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  throw CodecFailure(buf);
}

constexpr uint32_t H = 1024, NCB = 10, LAYERS = 8, QKV = 3072, FFN = 3072, EXP = 4096, ENTRY = 1536;
constexpr uint32_t RATES[4] = {8, 8, 4, 2};
constexpr uint32_t CHS[5] = {1536, 768, 384, 192, 96};
constexpr uint32_t SAMPLES_PER_FRAME = 2048;  // 4 latent frames x 8 x 8 x 4 x 2

float half_to_float(uint16_t h) {
  const uint32_t sign = uint32_t(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0) {
    const float v = std::ldexp(float(m), -24);
    return sign ? -v : v;
  }
  const uint32_t bits = e == 0x1f ? (sign | 0x7f800000u | (m << 13)) : (sign | ((e + 112u) << 23) | (m << 13));
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

struct ConvW {
  _Float16* w = nullptr;
  float* bias = nullptr;
  ConvTile tile{4, 32};
  uint32_t G = 1, M = 0, C = 0, phases = 1;
};

class CodecEngine {
 public:
  CodecEngine(const char* path, uint32_t max_frames, int32_t device) : max_frames_(max_frames), device_(device) {
    if (max_frames == 0) cfail("codec max_frames must be positive");
    if (max_frames > 4096) cfail("codec max_frames %u exceeds 4096", max_frames);
    select();
    CHK(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
    g_.open(path);
    if (g_.str("general.architecture") != "fish-speech-codec")
      cfail("expected fish-speech-codec codec GGUF, got %s", g_.str("general.architecture").c_str());
    load_weights();
    alloc_buffers();
  }
  ~CodecEngine() {
    select();
    if (stream_) (void)hipStreamSynchronize(stream_);
    for (void* p : allocs_) (void)hipFree(p);
    if (stream_) (void)hipStreamDestroy(stream_);
  }

  void select() { CHK(hipSetDevice(device_)); }
  hipStream_t stream() const { return stream_; }
  uint32_t max_frames() const { return max_frames_; }

  // ---- host entry points (host buffers in and out) ----
  void rvq_lookup_host(const int32_t* codes, uint32_t ncb, uint32_t n, float* latents) {
    validate_codes(codes, ncb, n);
    if (n == 0) return;
    CHK(hipMemcpyAsync(codes_, codes, size_t(NCB) * n * 4, hipMemcpyHostToDevice, stream_));
    rvq(n, nullptr);
    download(latents, lat_, size_t(n) * H);
  }
  void post_module_host(const float* latents, uint32_t n, float* hidden) {
    check_frames(n);
    if (n == 0) cfail("codec transformer requires at least one frame");
    upload(lat_, latents, size_t(n) * H);
    post_module(n);
    download(hidden, hid_, size_t(n) * H);
  }
  void upsample_host(const float* hidden, uint32_t n, float* out) {
    check_frames(n);
    if (n == 0) return;
    upload(hid_, hidden, size_t(n) * H);
    const float* r = upsample(n, false);
    download(out, r, size_t(4) * n * H);
  }
  void decode_latents_host(const float* latents, uint32_t n, float* out) {
    check_frames(n);
    if (n == 0) cfail("codec transformer requires at least one frame");
    upload(lat_, latents, size_t(n) * H);
    post_module(n);
    const float* r = upsample(n, false);
    download(out, r, size_t(4) * n * H);
  }
  // forward_codec_decoder over `frames` latent frames; stop_block <= 4: the
  // residual stream after that many blocks
  size_t decoder_host(const float* hidden, uint32_t frames, uint32_t hidden_dim, uint32_t stop_block, float* out,
                      size_t out_cap) {
    if (hidden_dim != H) cfail("decoder expects latent dim %u, got %u", H, hidden_dim);
    if (frames > 4 * max_frames_) cfail("decoder frames %u exceed the configured capacity %u", frames, 4 * max_frames_);
    const size_t need = decoder_out_elems(frames, stop_block);
    if (out_cap < need) cfail("decoder output buffer holds %zu floats, %zu needed", out_cap, need);
    if (frames == 0) return 0;
    upload(up32_, hidden, size_t(frames) * H);
    to_f16(up32_, a16_, size_t(frames) * H);
    const void* r = decoder(frames, stop_block);
    download(out, static_cast<const float*>(r), need);
    return need;
  }
  size_t decode_waveform_host(const int32_t* codes, uint32_t ncb, uint32_t n, float* samples, size_t cap) {
    validate_codes(codes, ncb, n);
    if (n == 0) cfail("codec transformer requires at least one frame");
    check_frames(n);
    const size_t ns = size_t(n) * SAMPLES_PER_FRAME;
    if (cap < ns) cfail("samples buffer holds %zu floats, %zu needed", cap, ns);
    CHK(hipMemcpyAsync(codes_, codes, size_t(NCB) * n * 4, hipMemcpyHostToDevice, stream_));
    waveform(n, nullptr, samples_);
    download(samples, samples_, ns);
    return ns;
  }
  // device-resident codes [10][n] and samples [n * 2048]; codes are checked
  // on the device (the first failing code is not identified)
  void decode_waveform_device(const int32_t* codes_dev, uint32_t ncb, uint32_t n, float* samples_dev) {
    if (ncb != NCB) cfail("codec codebook count mismatch: expected %u, got %u", NCB, ncb);
    if (n == 0) cfail("codec transformer requires at least one frame");
    check_frames(n);
    CHK(hipMemsetAsync(err_, 0, 4, stream_));
    CHK(launch_codec_check_codes(codes_dev, n, err_, stream_));
    waveform(n, codes_dev, samples_dev);
    uint32_t e = 0;
    CHK(hipMemcpyAsync(&e, err_, 4, hipMemcpyDeviceToHost, stream_));
    CHK(hipStreamSynchronize(stream_));
    if (e) cfail("codec code out of range for its codebook (device-side check)");
  }

  // Average device time of `what` with HIP events on the codec stream, over
  // reps launches after one untimed decode of n frames of fixed codes:
  // "decode" (the whole decode_waveform, device-resident codes and samples)
  // or one convolution of that decode by name (entry, b1_convT,
  // b4_r2_conv0, up1_pw1, ...), relaunched with the same arguments.
  // flops: 2 x multiply-adds of one launch (of the convolutions, for decode).
  void time(const std::string& what, uint32_t n, uint32_t reps, double* avg_us, double* flops) {
    if (n == 0 || reps == 0) cfail("timing needs frames and reps");
    check_frames(n);
    std::vector<int32_t> codes(size_t(NCB) * n);
    for (uint32_t q = 0; q < NCB; ++q)
      for (uint32_t f = 0; f < n; ++f)
        codes[size_t(q) * n + f] = int32_t((uint64_t(f) * 7919u + uint64_t(q) * 104729u + 17u) % cb_size_[q]);
    CHK(hipMemcpyAsync(codes_, codes.data(), codes.size() * 4, hipMemcpyHostToDevice, stream_));
    rec_.clear();
    recording_ = true;
    waveform(n, nullptr, samples_);
    recording_ = false;
    CHK(hipStreamSynchronize(stream_));
    double total_flops = 0.0;
    for (const Rec& r : rec_) total_flops += r.flops;
    const Rec* one = nullptr;
    for (const Rec& r : rec_)
      if (r.name == what) one = &r;
    if (what != "decode" && !one) cfail("unknown codec timing target %s", what.c_str());
    hipEvent_t e0, e1;
    CHK(hipEventCreate(&e0));
    CHK(hipEventCreate(&e1));
    auto launch = [&] {
      if (one && one->phases == 0)
        CHK(launch_residual_unit(one->a, one->tile, stream_));
      else if (one)
        CHK(launch_conv_gemm(one->a, one->phases, one->tile, stream_));
      else
        waveform(n, nullptr, samples_);
    };
    launch();
    CHK(hipEventRecord(e0, stream_));
    for (uint32_t i = 0; i < reps; ++i) launch();
    CHK(hipEventRecord(e1, stream_));
    CHK(hipEventSynchronize(e1));
    float ms = 0.0f;
    CHK(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    *avg_us = 1e3 * double(ms) / reps;
    *flops = one ? one->flops : total_flops;
  }

 private:
  template <class T>
  T* dalloc(size_t n) {
    void* p = nullptr;
    CHK(hipMalloc(&p, std::max<size_t>(n, 1) * sizeof(T)));
    allocs_.push_back(p);
    return static_cast<T*>(p);
  }
  template <class T>
  T* upload_vec(const std::vector<T>& v) {
    T* d = dalloc<T>(v.size());
    CHK(hipMemcpy(d, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice));
    return d;
  }
  const GgufTensor& tensor(const std::string& name, std::vector<uint64_t> dims) {
    const GgufTensor& t = g_.tensor(name);
    if (t.type != 1) cfail("expected F16 tensor %s, got type %u", name.c_str(), t.type);
    if (t.dims != dims) cfail("codec tensor %s has unexpected dimensions", name.c_str());
    return t;
  }
  const uint16_t* bits(const std::string& name, std::vector<uint64_t> dims) {
    return reinterpret_cast<const uint16_t*>(tensor(name, dims).data);
  }
  float* vec(const std::string& name, std::vector<uint64_t> dims) {
    const GgufTensor& t = tensor(name, dims);
    std::vector<float> v(t.elements());
    const uint16_t* p = reinterpret_cast<const uint16_t*>(t.data);
    for (size_t i = 0; i < v.size(); ++i) v[i] = half_to_float(p[i]);
    return upload_vec(v);
  }
  uint8_t* rows(const std::string& name, std::vector<uint64_t> dims) {
    const GgufTensor& t = tensor(name, dims);
    uint8_t* d = dalloc<uint8_t>(t.bytes + 256);
    CHK(hipMemcpy(d, t.data, t.bytes, hipMemcpyHostToDevice));
    CHK(hipMemset(d + t.bytes, 0, 256));
    return d;
  }
  template <class Src>
  ConvW packed(uint32_t phases, uint32_t M, uint32_t G, uint32_t C, bool split, Src src) {
    ConvW c;
    c.tile = conv_tile(M, G, split);
    c.G = G;
    c.M = M;
    c.C = C;
    c.phases = phases;
    std::vector<uint16_t> h(conv_packed_halfs(phases, M, G, C, c.tile));
    pack_conv_weights(h.data(), phases, M, G, C, c.tile, src);
    c.w = reinterpret_cast<_Float16*>(upload_vec(h));
    return c;
  }
  // causal_conv_1d weight, ggml [k][in][out] (index tap + k*in_i + k*in*o)
  ConvW conv1d(const std::string& p, uint32_t k, uint32_t cin, uint32_t cout) {
    const uint16_t* w = bits(p + ".conv.weight", {k, cin, cout});
    ConvW c = packed(1, cout, k, cin, false, [&](uint32_t, uint32_t m, uint32_t g, uint32_t ch) {
      return w[g + size_t(k) * ch + size_t(k) * cin * m];
    });
    c.bias = vec(p + ".conv.bias", {cout});
    return c;
  }
  // causal_conv_transpose_1d weight, ggml [k][out][in] (index kk + k*o + k*out*in_i);
  // phase r, tap j uses kk = r + j*stride on input frame f - j
  ConvW conv_t(const std::string& p, uint32_t stride, uint32_t k, uint32_t cin, uint32_t cout) {
    const uint16_t* w = bits(p + ".conv.weight", {k, cout, cin});
    if (k % stride) cfail("%s: kernel %u is not a multiple of stride %u", p.c_str(), k, stride);
    ConvW c = packed(stride, cout, k / stride, cin, true, [&](uint32_t r, uint32_t m, uint32_t j, uint32_t ch) {
      return w[(r + j * stride) + size_t(k) * m + size_t(k) * cout * ch];
    });
    c.bias = vec(p + ".conv.bias", {cout});
    return c;
  }
  // linear [out][in] rows
  ConvW linear(const std::string& p, uint32_t in, uint32_t out) {
    const uint16_t* w = bits(p + ".weight", {in, out});
    ConvW c = packed(1, out, 1, in, true, [&](uint32_t, uint32_t m, uint32_t, uint32_t ch) {
      return w[size_t(m) * in + ch];
    });
    c.bias = vec(p + ".bias", {out});
    return c;
  }

  struct Layer {
    uint8_t *wqkv, *wo, *w1, *w2, *w3;
    float *attn_norm, *ffn_norm, *als, *fls;
  };
  struct Stage {
    ConvW ct, pw1, pw2;
    float *gamma, *dw_w, *dw_b, *ln_w, *ln_b;
  };
  struct Res {
    float *a0, *a1;
    ConvW c0, c1;
  };
  struct Block {
    float* alpha;
    ConvW ct;
    Res res[3];
  };

  void load_weights() {
    for (uint32_t q = 0; q < NCB; ++q) {
      const std::string p = q == 0 ? "quantizer.semantic_quantizer.quantizers.0"
                                   : "quantizer.quantizer.quantizers." + std::to_string(q - 1);
      cb_size_[q] = q == 0 ? 4096u : 1024u;
      cb_[q] = vec(p + ".codebook.weight", {8, cb_size_[q]});
      pw_[q] = vec(p + ".out_proj.weight", {8, H});
      pb_[q] = vec(p + ".out_proj.bias", {H});
    }
    for (uint32_t l = 0; l < LAYERS; ++l) {
      const std::string p = "quantizer.post_module.layers." + std::to_string(l);
      Layer& L = layers_[l];
      L.attn_norm = vec(p + ".attention_norm.weight", {H});
      L.ffn_norm = vec(p + ".ffn_norm.weight", {H});
      L.als = vec(p + ".attention_layer_scale.gamma", {H});
      L.fls = vec(p + ".ffn_layer_scale.gamma", {H});
      L.wqkv = rows(p + ".attention.wqkv.weight", {H, QKV});
      L.wo = rows(p + ".attention.wo.weight", {H, H});
      L.w1 = rows(p + ".feed_forward.w1.weight", {H, FFN});
      L.w2 = rows(p + ".feed_forward.w2.weight", {FFN, H});
      L.w3 = rows(p + ".feed_forward.w3.weight", {H, FFN});
    }
    post_norm_ = vec("quantizer.post_module.norm.weight", {H});
    for (uint32_t s = 0; s < 2; ++s) {
      const std::string p = "quantizer.upsample." + std::to_string(s);
      Stage& S = stages_[s];
      S.ct = conv_t(p + ".0", 2, 2, H, H);
      S.gamma = vec(p + ".1.gamma", {H});
      {
        // depthwise weight ggml [7][1][1024] (index kk + 7 c): [c][kk]
        S.dw_w = vec(p + ".1.dwconv.conv.weight", {7, 1, H});
      }
      S.dw_b = vec(p + ".1.dwconv.conv.bias", {H});
      S.ln_w = vec(p + ".1.norm.weight", {H});
      S.ln_b = vec(p + ".1.norm.bias", {H});
      S.pw1 = linear(p + ".1.pwconv1", H, EXP);
      S.pw2 = linear(p + ".1.pwconv2", EXP, H);
    }
    entry_ = conv1d("decoder.model.0", 7, H, ENTRY);
    for (uint32_t b = 0; b < 4; ++b) {
      const std::string p = "decoder.model." + std::to_string(b + 1) + ".block";
      const uint32_t ci = CHS[b], co = CHS[b + 1];
      Block& B = blocks_[b];
      B.alpha = vec(p + ".0.alpha", {1, ci, 1});
      B.ct = conv_t(p + ".1", RATES[b], 2 * RATES[b], ci, co);
      for (uint32_t r = 0; r < 3; ++r) {
        const std::string q = p + "." + std::to_string(r + 2) + ".block";
        B.res[r].a0 = vec(q + ".0.alpha", {1, co, 1});
        B.res[r].c0 = conv1d(q + ".1", 7, co, co);
        B.res[r].a1 = vec(q + ".2.alpha", {1, co, 1});
        B.res[r].c1 = conv1d(q + ".3", 1, co, co);
      }
    }
    for (uint32_t b = 0; b < 4; ++b) {
      const std::string p = "b" + std::to_string(b + 1);
      names_[b][0] = p + "_convT";
      for (uint32_t r = 0; r < 3; ++r) {
        names_[b][1 + 2 * r] = p + "_r" + std::to_string(r + 1) + "_conv0";
        names_[b][2 + 2 * r] = p + "_r" + std::to_string(r + 1) + "_conv1";
      }
    }
    tail_alpha_ = vec("decoder.model.5.alpha", {1, 96, 1});
    out_w_ = vec("decoder.model.6.conv.weight", {7, 96, 1});  // index tap + 7 c
    out_b_ = half_to_float(bits("decoder.model.6.conv.bias", {1})[0]);
    // RoPE (cos, sin) per position and pair, as apply_rope_normal computes
    // them (attention.rs:172-206): theta = pos / powf(1e4, pair / 64)
    std::vector<float2> tab(size_t(max_frames_) * 32);
    for (uint32_t t = 0; t < max_frames_; ++t)
      for (uint32_t i = 0; i < 32; ++i) {
        const float theta = float(t) / powf(10000.0f, float(2 * i) / 64.0f);
        tab[size_t(t) * 32 + i] = make_float2(cosf(theta), sinf(theta));
      }
    rope_ = upload_vec(tab);
  }

  void alloc_buffers() {
    const size_t F = max_frames_;
    npad_ = gemm_rows_pad(uint32_t(F));
    codes_ = dalloc<int32_t>(NCB * F);
    err_ = dalloc<uint32_t>(1);
    lat_ = dalloc<float>(F * H);
    hid_ = dalloc<float>(F * H);
    qkv_ = dalloc<float>(F * QKV);
    att_ = dalloc<float>(F * H);
    act_ = dalloc<float>(F * FFN);
    proj_ = dalloc<float>(F * H);
    pxh_ = dalloc<_Float16>(npad_ * FFN);
    pxl_ = dalloc<_Float16>(npad_ * FFN);
    prs_ = dalloc<float>(npad_);
    part_cap_ = gemm_part_floats(uint32_t(npad_), QKV);
    part_ = dalloc<float>(part_cap_);
    up32_ = dalloc<float>(4 * F * H);
    upx_ = dalloc<float>(4 * F * H);
    qh_ = dalloc<_Float16>(4 * F * H);
    ql_ = dalloc<_Float16>(4 * F * H);
    ph_ = dalloc<_Float16>(4 * F * EXP);
    pl_ = dalloc<_Float16>(4 * F * EXP);
    const size_t big = F * 196608;  // largest decoder activation: frames x channels
    x32_ = dalloc<float>(big);
    a16_ = dalloc<_Float16>(big);
    b16_ = dalloc<_Float16>(big);
    dh_ = dalloc<_Float16>(big);
    dl_ = dalloc<_Float16>(big);
    samples_ = dalloc<float>(F * SAMPLES_PER_FRAME);
    cpart_cap_ = F * 32768;  // K-split partial sums of the short-grid products
    cpart_ = dalloc<float>(cpart_cap_);
  }

  void check_frames(uint32_t n) {
    if (n > max_frames_) cfail("codec n_frames %u exceeds the configured max_frames %u", n, max_frames_);
  }
  // rvq_lookup_codes checks (codec.rs:2542-2575), in its order
  void validate_codes(const int32_t* codes, uint32_t ncb, uint32_t n) {
    if (ncb != NCB) cfail("codec codebook count mismatch: expected %u, got %u", NCB, ncb);
    check_frames(n);
    for (uint32_t f = 0; f < n; ++f)
      for (uint32_t q = 0; q < NCB; ++q) {
        const int32_t c = codes[size_t(q) * n + f];
        if (c < 0) cfail("codec code must be non-negative, got %d", c);
        if (uint32_t(c) >= cb_size_[q]) cfail("embedding index %d out of range for vocab_dim %u", c, cb_size_[q]);
      }
  }
  void upload(float* d, const float* h, size_t n) {
    CHK(hipMemcpyAsync(d, h, n * 4, hipMemcpyHostToDevice, stream_));
  }
  void download(float* h, const float* d, size_t n) {
    CHK(hipMemcpyAsync(h, d, n * 4, hipMemcpyDeviceToHost, stream_));
    CHK(hipStreamSynchronize(stream_));
  }
  void to_f16(const float* x, _Float16* h, size_t n) {
    // f16 plane only: split16 with the lo plane written to the b16 buffer
    CHK(launch_codec_split16(x, h, b16_, n, stream_));
  }

  void rvq(uint32_t n, const int32_t* codes_dev) {
    RvqArgs a{};
    a.codes = codes_dev ? codes_dev : codes_;
    a.F = n;
    for (uint32_t q = 0; q < NCB; ++q) {
      a.cb[q] = cb_[q];
      a.pw[q] = pw_[q];
      a.pb[q] = pb_[q];
      a.cb_size[q] = cb_size_[q];
    }
    a.err = codes_dev ? err_ : nullptr;
    a.out = lat_;
    CHK(launch_codec_rvq(a, stream_));
  }

  void gemm(const uint8_t* w, const uint8_t* w3, uint32_t in, uint32_t out, int epi, uint32_t n, float* y,
            uint32_t ldy) {
    GemmArgs g{};
    g.w = w;
    g.w3 = w3;
    g.row_bytes = size_t(in) * 2;
    g.M = out;
    g.K = in;
    g.xh = pxh_;
    g.xl = pxl_;
    g.rs = prs_;
    g.N = n;
    g.y = y;
    g.ldy = ldy;
    g.part = part_;
    g.part_cap = part_cap_;
    CHK(launch_gemm_mfma(W_F16, epi, g, stream_));
  }
  void split(const float* x, uint32_t ld, const float* norm, uint32_t n, uint32_t k) {
    CHK(launch_split_rows(x, ld, norm, 1e-5f, n, gemm_rows_pad(n), k, pxh_, pxl_, prs_, nullptr, stream_));
  }

  // forward_codec_post_module (codec.rs:986-1018): lat_ -> hid_
  void post_module(uint32_t n) {
    for (uint32_t l = 0; l < LAYERS; ++l) {
      const Layer& L = layers_[l];
      split(lat_, H, L.attn_norm, n, H);
      gemm(L.wqkv, nullptr, H, QKV, EPI_STORE, n, qkv_, QKV);
      CHK(launch_codec_rope(qkv_, n, rope_, stream_));
      CHK(launch_codec_attention(qkv_, n, att_, stream_));
      split(att_, H, nullptr, n, H);
      gemm(L.wo, nullptr, H, H, EPI_STORE, n, proj_, H);
      CHK(launch_codec_scaled_residual(lat_, proj_, L.als, n, H, stream_));
      split(lat_, H, L.ffn_norm, n, H);
      gemm(L.w1, L.w3, H, FFN, EPI_SWIGLU_FAST, n, act_, FFN);
      split(act_, FFN, nullptr, n, FFN);
      gemm(L.w2, nullptr, FFN, H, EPI_STORE, n, proj_, H);
      CHK(launch_codec_scaled_residual(lat_, proj_, L.fls, n, H, stream_));
    }
    CHK(launch_rms_norm(lat_, post_norm_, hid_, H, n, 1e-5f, nullptr, stream_));
  }

  ConvGemmArgs cargs(const ConvW& w, const _Float16* xh, const _Float16* xl, uint32_t frames) {
    ConvGemmArgs a{};
    a.xh = xh;
    a.xl = xl;
    a.ldx = w.C;
    a.C = w.C;
    a.F = frames;
    a.G = w.G;
    a.w = w.w;
    a.M = w.M;
    a.ostride = w.phases;
    a.bias = w.bias;
    a.part = cpart_;
    a.part_cap = cpart_cap_;
    return a;
  }
  void run(const ConvGemmArgs& a, const ConvW& w, const char* name) {
    CHK(launch_conv_gemm(a, w.phases, w.tile, stream_));
    if (recording_) {
      const double flops = 2.0 * double(a.F) * w.phases * w.M * w.G * w.C;
      rec_.push_back(Rec{name, a, w.phases, w.tile, flops});
    }
  }
  struct Rec {
    std::string name;
    ConvGemmArgs a;
    uint32_t phases;
    ConvTile tile;
    double flops;  // 2 x multiply-adds of the convolution (the reference's arithmetic)
    // phases 0: a fused residual unit (launch_residual_unit)
  };
  bool recording_ = false;
  std::vector<Rec> rec_;

  // forward_codec_upsample (codec.rs:2302-2325) on hid_ (n frames); returns the
  // f32 result [4n][1024]; with to_decoder the f16 copy goes to a16_ too
  const float* upsample(uint32_t n, bool to_decoder) {
    const float* in = hid_;
    uint32_t F = n;
    for (uint32_t s = 0; s < 2; ++s) {
      const Stage& S = stages_[s];
      CHK(launch_codec_split16(in, qh_, ql_, size_t(F) * H, stream_));
      ConvGemmArgs c = cargs(S.ct, qh_, ql_, F);  // conv_transpose, stride 2, kernel 2: one tap per phase
      c.off0 = 0;
      c.ostep = -1;
      c.y32 = up32_;
      c.ldy = H;
      run(c, S.ct, s ? "up2_convT" : "up1_convT");
      F *= 2;
      CHK(launch_codec_dwconv_ln(up32_, F, S.dw_w, S.dw_b, S.ln_w, S.ln_b, 1e-6f, qh_, ql_, stream_));
      ConvGemmArgs p1 = cargs(S.pw1, qh_, ql_, F);
      p1.off0 = 0;
      p1.ostep = 1;
      p1.gelu = 1;
      p1.yh = ph_;
      p1.yl = pl_;
      p1.ldh = EXP;
      run(p1, S.pw1, s ? "up2_pw1" : "up1_pw1");
      ConvGemmArgs p2 = cargs(S.pw2, ph_, pl_, F);
      p2.off0 = 0;
      p2.ostep = 1;
      p2.gamma = S.gamma;
      p2.res = up32_;
      p2.ldres = H;
      p2.y32 = upx_;
      p2.ldy = H;
      if (s == 1 && to_decoder) {
        p2.yh = a16_;
        p2.ldh = H;
      }
      run(p2, S.pw2, s ? "up2_pw2" : "up1_pw2");
      in = upx_;
    }
    return upx_;
  }

  // outputs of a residual unit's k1 conv: the updated residual stream (kept
  // when another unit of the block or a checkpoint reads it) and the snake of
  // whatever comes next, as f16 or hi / lo planes
  void set_unit_outputs(ConvGemmArgs& c, const Block& B, uint32_t b, uint32_t r, uint32_t co, bool stop_here) {
    if (r < 2 || stop_here) {
      c.y32 = x32_;
      c.ldy = co;
    }
    c.ldh = co;
    if (r < 2) {  // the next residual unit's conv0 input
      c.alpha = B.res[r + 1].a0;
      c.yh = a16_;
    } else if (!stop_here) {
      if (b < 3) {  // the next block's conv_transpose input
        c.alpha = blocks_[b + 1].alpha;
        c.yh = dh_;
        c.yl = dl_;
      } else {  // the output conv's input
        c.alpha = tail_alpha_;
        c.yh = a16_;
      }
    }
  }

  static size_t decoder_out_elems(uint32_t frames, uint32_t stop_block) {
    if (stop_block >= 5) return size_t(frames) * 512;
    size_t f = frames;
    for (uint32_t b = 0; b < stop_block; ++b) f *= RATES[b];
    return f * CHS[stop_block];
  }

  // forward_codec_decoder (codec.rs:1941-2001) from a16_ (f16 latents,
  // `frames` x 1024); returns samples_ or, for stop_block <= 4, x32_
  const void* decoder(uint32_t frames, uint32_t stop_block, float* samples_out = nullptr) {
    ConvGemmArgs e = cargs(entry_, a16_, nullptr, frames);
    e.off0 = -6;
    e.ostep = 1;
    e.alpha = blocks_[0].alpha;
    e.yh = dh_;
    e.yl = dl_;
    e.ldh = ENTRY;
    if (stop_block == 0) {
      e.y32 = x32_;
      e.ldy = ENTRY;
    }
    run(e, entry_, "entry");
    if (stop_block == 0) return x32_;
    uint32_t F = frames;
    const _Float16* out_in = a16_;  // the output conv's input (snake of the last residual stream)
    for (uint32_t b = 0; b < 4; ++b) {
      const Block& B = blocks_[b];
      const uint32_t co = CHS[b + 1];
      ConvGemmArgs t = cargs(B.ct, dh_, dl_, F);
      t.off0 = 0;
      t.ostep = -1;
      t.y32 = x32_;
      t.ldy = co;
      t.alpha = B.res[0].a0;
      t.yh = a16_;
      t.ldh = co;
      run(t, B.ct, names_[b][0].c_str());
      F *= RATES[b];
      const uint32_t dil[3] = {1, 3, 9};
      const bool stop_here = stop_block == b + 1;
      for (uint32_t r = 0; r < 3; ++r) {
        const Res& R = B.res[r];
        const bool fused = co % 32u == 0 && co <= 32u * R.c0.tile.mc && R.c1.tile.mc == R.c0.tile.mc && R.c0.tile.mc <= 4;
        if (fused) {  // k7 conv + snake + k1 conv in one launch (the block holds every channel)
          // the k7 conv reads other tiles' rows (its halo), so the unit's f16
          // output goes to the other buffer: units read a16, b16, a16 and
          // write b16, a16, b16
          _Float16* uin = (r & 1u) ? b16_ : a16_;
          _Float16* uout = (r & 1u) ? a16_ : b16_;
          ConvGemmArgs u = cargs(R.c0, uin, nullptr, F);
          u.off0 = -6 * int32_t(dil[r]);
          u.ostep = int32_t(dil[r]);
          u.part = nullptr;
          u.w1 = R.c1.w;
          u.bias_mid = R.c0.bias;
          u.alpha_mid = R.a1;
          u.bias = R.c1.bias;
          u.res = x32_;
          u.ldres = co;
          set_unit_outputs(u, B, b, r, co, stop_here);
          if (u.yh == a16_) u.yh = uout;  // dh_ / dl_ outputs are separate buffers already
          if (r == 2 && b == 3) out_in = uout;
          CHK(launch_residual_unit(u, R.c0.tile, stream_));
          if (recording_)
            rec_.push_back(Rec{names_[b][1 + 2 * r].substr(0, 5) + "_unit", u, 0, R.c0.tile,
                               2.0 * double(F) * co * (7.0 * co + co)});
          continue;
        }
        ConvGemmArgs c0 = cargs(R.c0, a16_, nullptr, F);
        c0.off0 = -6 * int32_t(dil[r]);
        c0.ostep = int32_t(dil[r]);
        c0.alpha = R.a1;
        c0.yh = b16_;
        c0.ldh = co;
        run(c0, R.c0, names_[b][1 + 2 * r].c_str());
        ConvGemmArgs c1 = cargs(R.c1, b16_, nullptr, F);
        c1.off0 = 0;
        c1.ostep = 1;
        c1.res = x32_;
        c1.ldres = co;
        set_unit_outputs(c1, B, b, r, co, stop_here);
        run(c1, R.c1, names_[b][2 + 2 * r].c_str());
      }
      if (stop_here) return x32_;
    }
    float* out = samples_out ? samples_out : samples_;
    CHK(launch_codec_out_conv(out_in, F, out_w_, out_b_, out, stream_));
    return out;
  }

  void waveform(uint32_t n, const int32_t* codes_dev, float* out) {
    rvq(n, codes_dev);
    post_module(n);
    upsample(n, true);
    decoder(4 * n, 5, out);
  }

  GgufFile g_;
  uint32_t max_frames_;
  int32_t device_;
  hipStream_t stream_ = nullptr;
  std::vector<void*> allocs_;
  // weights
  float* cb_[NCB];
  float* pw_[NCB];
  float* pb_[NCB];
  uint32_t cb_size_[NCB];
  Layer layers_[LAYERS];
  float* post_norm_ = nullptr;
  float2* rope_ = nullptr;
  Stage stages_[2];
  ConvW entry_;
  Block blocks_[4];
  std::string names_[4][7];
  float* tail_alpha_ = nullptr;
  float* out_w_ = nullptr;
  float out_b_ = 0.0f;
  // buffers
  size_t npad_ = 0, part_cap_ = 0;
  int32_t* codes_ = nullptr;
  uint32_t* err_ = nullptr;
  float *lat_ = nullptr, *hid_ = nullptr, *qkv_ = nullptr, *att_ = nullptr, *act_ = nullptr, *proj_ = nullptr;
  _Float16 *pxh_ = nullptr, *pxl_ = nullptr;
  float *prs_ = nullptr, *part_ = nullptr;
  float *up32_ = nullptr, *upx_ = nullptr;
  _Float16 *qh_ = nullptr, *ql_ = nullptr, *ph_ = nullptr, *pl_ = nullptr;
  float* x32_ = nullptr;
  _Float16 *a16_ = nullptr, *b16_ = nullptr, *dh_ = nullptr, *dl_ = nullptr;
  float* samples_ = nullptr;
  float* cpart_ = nullptr;
  size_t cpart_cap_ = 0;
};

void copy_err(const std::exception& e, char* err, size_t cap) {
  if (err && cap) snprintf(err, cap, "%s", e.what());
}

}  // namespace
}  // namespace s2

struct s2hip_codec {
  std::unique_ptr<s2::CodecEngine> eng;
};

using s2::copy_err;

extern "C" {

s2hip_codec* s2hip_codec_open(const char* codec_gguf_path, uint32_t max_frames, int32_t device, char* err,
                              size_t err_cap) {
  try {
    if (!codec_gguf_path) throw std::runtime_error("codec_gguf_path is null");
    std::unique_ptr<s2hip_codec> c(new s2hip_codec);
    c->eng.reset(new s2::CodecEngine(codec_gguf_path, max_frames, device));
    return c.release();
  } catch (const std::exception& e) {
    copy_err(e, err, err_cap);
    return nullptr;
  }
}

void s2hip_codec_close(s2hip_codec* codec) { delete codec; }

#define CODEC_CALL(body)                                   \
  try {                                                    \
    if (!codec) throw std::runtime_error("codec is null"); \
    codec->eng->select();                                  \
    body;                                                  \
    return 1;                                              \
  } catch (const std::exception& e) {                      \
    copy_err(e, err, err_cap);                             \
    return 0;                                              \
  }

int32_t s2hip_codec_rvq_lookup(s2hip_codec* codec, const int32_t* codes, uint32_t num_codebooks, uint32_t n_frames,
                               float* latents, char* err, size_t err_cap) {
  CODEC_CALL(codec->eng->rvq_lookup_host(codes, num_codebooks, n_frames, latents))
}

int32_t s2hip_codec_post_module(s2hip_codec* codec, const float* latents, uint32_t n_frames, float* hidden, char* err,
                                size_t err_cap) {
  CODEC_CALL(codec->eng->post_module_host(latents, n_frames, hidden))
}

int32_t s2hip_codec_upsample(s2hip_codec* codec, const float* hidden, uint32_t n_frames, float* out, char* err,
                             size_t err_cap) {
  CODEC_CALL(codec->eng->upsample_host(hidden, n_frames, out))
}

int32_t s2hip_codec_decode_latents(s2hip_codec* codec, const float* latents, uint32_t n_frames, float* out,
                                   char* err, size_t err_cap) {
  CODEC_CALL(codec->eng->decode_latents_host(latents, n_frames, out))
}

int32_t s2hip_codec_decoder(s2hip_codec* codec, const float* hidden, uint32_t n_frames, uint32_t hidden_dim,
                            uint32_t stop_block, float* out, size_t out_cap, size_t* out_len, char* err,
                            size_t err_cap) {
  CODEC_CALL({
    const size_t n = codec->eng->decoder_host(hidden, n_frames, hidden_dim, stop_block, out, out_cap);
    if (out_len) *out_len = n;
  })
}

int32_t s2hip_codec_decode_waveform(s2hip_codec* codec, const int32_t* codes, uint32_t num_codebooks,
                                    uint32_t n_frames, float* samples, size_t samples_cap, s2hip_waveform_info* info,
                                    char* err, size_t err_cap) {
  CODEC_CALL({
    const size_t n = codec->eng->decode_waveform_host(codes, num_codebooks, n_frames, samples, samples_cap);
    if (info) {
      info->sample_rate = 44100;
      info->input_frames = n_frames;
      info->latent_frames = 4 * n_frames;
      info->num_samples = n;
    }
  })
}

int32_t s2hip_codec_decode_waveform_device(s2hip_codec* codec, const int32_t* codes_dev, uint32_t num_codebooks,
                                           uint32_t n_frames, float* samples_dev, char* err, size_t err_cap) {
  CODEC_CALL(codec->eng->decode_waveform_device(codes_dev, num_codebooks, n_frames, samples_dev))
}

void s2hip_codec_snake_host(const float* x, size_t n, const float* alpha, float* y) {
  for (size_t i = 0; i < n; ++i) y[i] = s2::snake_cw(x[i], alpha[i]);
}

int32_t s2hip_codec_time(s2hip_codec* codec, const char* what, uint32_t n_frames, uint32_t reps, double* avg_us,
                         double* flops, char* err, size_t err_cap) {
  CODEC_CALL({
    if (!what || !avg_us || !flops) throw std::runtime_error("null argument");
    codec->eng->time(what, n_frames, reps, avg_us, flops);
  })
}

}  // extern "C"
