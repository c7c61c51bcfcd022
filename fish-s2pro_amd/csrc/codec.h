// codec.h -- HIP kernels of the RVQ codec decode (decode_waveform,
// crates/fish_s2_infer/src/codec.rs:1690-1714).  Activations are frame-major
// ([frame][channel]) throughout, as in the reference.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

namespace s2 {

// Implicit-GEMM convolution on MFMA (v_mfma_f32_32x32x16_f16):
//   y[f * ostride + phase][m] = epilogue( sum_g sum_c A[f + off0 + g * ostep][c] * W[phase][m][g][c] )
// for frames f < F and output channels m < M.  A rows outside [0, F) are
// zero (causal left padding).  A is one f16 plane (conv inputs, which the
// reference rounds to f16) or two planes hi + lo with hi = f16(x),
// lo = f16(x - hi), whose products sum to the f32 input's product within
// ~2^-22 relative (transposed-conv and pointwise inputs, f32 in the
// reference).  W is packed by pack_conv_weights.
// Epilogue, in this order: v = acc + bias[m]; gelu; v *= gamma[m];
// v = res[row][m] + v; y32[row][m] = v; v = snake(v, alpha[m]);
// yh[row][m] = f16(v) (and yl = f16(v - yh) when yl is given).
struct ConvGemmArgs {
  const _Float16* xh;
  const _Float16* xl;  // null: one plane
  uint32_t ldx;        // elements per input row
  uint32_t C;          // input channels (a multiple of the stage width, 16 or 32)
  uint32_t F;          // frames per phase (input frames)
  uint32_t G;          // taps
  int32_t off0, ostep; // tap g reads input frame f + off0 + g * ostep
  const _Float16* w;   // packed weights
  uint32_t M;          // output channels
  uint32_t ostride;    // output row = f * ostride + phase
  const float* bias;
  uint32_t gelu;
  const float* gamma;
  const float* res;
  uint32_t ldres;
  float* y32;
  uint32_t ldy;
  const float* alpha;
  _Float16* yh;
  _Float16* yl;
  uint32_t ldh;
  // K split (nullable): when a launch would leave CUs idle, splits of the
  // input-channel stages write partial sums to part ([split][row][M] f32,
  // part_cap floats) and a reduce kernel adds them in split order and
  // applies the epilogue
  float* part;
  size_t part_cap;
  // Fused residual unit (M <= 128, one m tile): the product above is the unit's
  // k7 conv; Y = f16(snake(acc + bias_mid, alpha_mid)) goes to LDS and acc =
  // Y . W1 (the unit's k1 conv, w1 packed like any k1 conv of M channels)
  // before the epilogue, which then uses bias (the k1 conv's) onwards.
  const _Float16* w1;
  const float* bias_mid;
  const float* alpha_mid;
};

// Tile geometry of a packed weight: TM = 32 * mc output channels per tile,
// kc input channels per stage.
struct ConvTile {
  uint32_t mc, kc;
};
ConvTile conv_tile(uint32_t M, uint32_t G, bool split);
// Packs W(phase, m, g, c) = src(phase, m, g, c) into the layout the kernel
// streams: [phase][m_tile][c / kc][g][TM][kc], zero rows for m >= M.
// Host side; returns halfs written (phases * m_tiles * TM * G * C).
size_t conv_packed_halfs(uint32_t phases, uint32_t M, uint32_t G, uint32_t C, ConvTile t);
template <class Src>
void pack_conv_weights(uint16_t* dst, uint32_t phases, uint32_t M, uint32_t G, uint32_t C, ConvTile t, Src src) {
  const uint32_t TM = 32 * t.mc, mt = (M + TM - 1) / TM, nch = C / t.kc;
  size_t o = 0;
  for (uint32_t p = 0; p < phases; ++p)
    for (uint32_t ti = 0; ti < mt; ++ti)
      for (uint32_t ch = 0; ch < nch; ++ch)
        for (uint32_t g = 0; g < G; ++g)
          for (uint32_t r = 0; r < TM; ++r)
            for (uint32_t k = 0; k < t.kc; ++k) {
              const uint32_t m = ti * TM + r;
              dst[o++] = m < M ? src(p, m, g, ch * t.kc + k) : uint16_t(0);
            }
}
hipError_t launch_conv_gemm(const ConvGemmArgs& a, uint32_t phases, ConvTile t, hipStream_t s);
// The residual unit's k7 conv + snake + k1 conv in one launch (a.w1 set; M a
// multiple of 32, at most 128; tile t of the k7 conv).
hipError_t launch_residual_unit(const ConvGemmArgs& a, ConvTile t, hipStream_t s);

// rvq_lookup_codes: latents[f][o] = sum over codebooks q (in order) of
// (codebook_q[code] . proj_w_q[o] + proj_b_q[o]); codes codebook-major
// [10][F], already validated.  tables: per quantizer {codebook [size][8],
// proj_w [1024][8], proj_b [1024]} f32.
struct RvqArgs {
  const int32_t* codes;
  uint32_t F;
  const float* cb[10];
  const float* pw[10];
  const float* pb[10];
  uint32_t cb_size[10];
  uint32_t* err;  // set to 1 when a code is out of range (device-side codes)
  float* out;
};
hipError_t launch_codec_rvq(const RvqArgs& a, hipStream_t s);

// RoPE on the q and k parts of qkv rows [T][3072] (16 heads of 64, adjacent
// pairs) from a (cos, sin) table [position][32].
hipError_t launch_codec_rope(float* qkv, uint32_t T, const float2* table, hipStream_t s);

// Causal attention over a 128-frame window: 16 heads of 64, scale 1/8.
hipError_t launch_codec_attention(const float* qkv, uint32_t T, float* out, hipStream_t s);

// x[t][i] = x[t][i] + p[t][i] * scale[i]
hipError_t launch_codec_scaled_residual(float* x, const float* p, const float* scale, uint32_t T, uint32_t D,
                                        hipStream_t s);

// hi = f16(x), lo = f16(x - hi) over n elements
hipError_t launch_codec_split16(const float* x, _Float16* hi, _Float16* lo, size_t n, hipStream_t s);

// ConvNeXt front: depthwise causal conv (k 7) + LayerNorm (eps) per frame of
// 1024 channels, output as hi / lo planes.  w: [1024][7] f32.
hipError_t launch_codec_dwconv_ln(const float* x, uint32_t F, const float* w, const float* b, const float* ln_w,
                                  const float* ln_b, float eps, _Float16* hi, _Float16* lo, hipStream_t s);

// Output conv (96 -> 1, k 7, causal) over f16 inputs, then tanh.  w: [96][7] f32.
hipError_t launch_codec_out_conv(const _Float16* x, uint32_t T, const float* w, float b, float* out, hipStream_t s);

// Sets *err = 1 when a code in codes[10][F] is out of range for its codebook.
hipError_t launch_codec_check_codes(const int32_t* codes, uint32_t F, uint32_t* err, hipStream_t s);

}  // namespace s2
