/*
 * s2_oracle.h -- CPU restatement of the reference's dual-AR token loop.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * path and the timed CPU baseline.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it; the product library (libs2hip)
 * never links or calls it.
 *
 * Every function restates a function of stevenke1981/fish-s2pro's rust-pure
 * path (crates/fish_s2_infer/src/...) with the same f32 operation order:
 * sequential left-to-right sums, no FMA contraction, glibc expf/powf/sinf/cosf,
 * correctly rounded sqrt and division.  Citations are next to each definition
 * in s2_oracle.cpp.  Generalisations over the reference (it hard-codes the
 * full S2-Pro shapes and F16): shapes come from GGUF metadata and tensor
 * dimensions, Q8_0/Q4_0 linear weights are dequantised exactly, and the
 * Fast-AR can run incrementally (bit-identical to the reference's prefix
 * recompute, which the "faithful" mode keeps).
 */
#ifndef S2_ORACLE_H
#define S2_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar / vector primitives -------------------------------------- */
uint16_t orc_f32_to_f16(float value);
float orc_f16_to_f32(uint16_t bits);
/* GGML type ids: 0 F32, 1 F16, 2 Q4_0, 8 Q8_0 */
int32_t orc_dequant_row(const uint8_t* src, uint32_t ggml_type, size_t n, float* out);
int32_t orc_rms_norm(const float* x, const float* w, size_t n, float eps, float* out);
int32_t orc_rms_norm_heads(const float* x, const float* w, size_t n, size_t head_dim, float eps,
                           float* out);
/* y[o] = sum_i x[i] * W[o][i]; W given as raw GGML rows of `in_dim` elements */
int32_t orc_linear(const float* x, const uint8_t* w, uint32_t ggml_type, size_t in_dim,
                   size_t out_dim, float* y);
int32_t orc_rope_normal(float* values, size_t len, size_t head_dim, size_t position,
                        float rope_base);
int32_t orc_gqa_attention(const float* q, const float* keys, const float* values,
                          size_t head_count, size_t head_count_kv, size_t head_dim,
                          size_t token_count, float attn_scale, float* out);
void orc_swiglu_slow(const float* gate, const float* up, size_t n, float* out);
void orc_swiglu_fast(const float* gate, const float* up, size_t n, float* out);
double orc_rng_next_unit(uint64_t* state);
/* always_include < 0 means None. Returns 1 on success. */
int32_t orc_sample_token(const float* logits, size_t n, float temperature, float top_p,
                         int32_t top_k, int64_t always_include, uint64_t* rng_state,
                         uint32_t* token_out);
/* sample_token plus margins[3] = {draw, cut, tie}: how far the draw target
 * lies from the cumulative-sum boundaries around the chosen item, how far the
 * top-p cumulative sums lie from top_p around the cut (+inf: no cut), and the
 * logit gap between the chosen item and its neighbours in the sort order. */
int32_t orc_sample_token_margins(const float* logits, size_t n, float temperature, float top_p,
                                 int32_t top_k, int64_t always_include, uint64_t* rng_state,
                                 uint32_t* token_out, float* margins);
/* build_semantic_bias + apply_semantic_bias in place; im_end < 0 means None */
void orc_semantic_bias(float* logits, size_t n, uint32_t sem_begin, uint32_t sem_end, int64_t im_end,
                       int32_t block_im_end);
/* the C library's expf, which Rust's f32::exp calls */
void orc_expf(const float* x, size_t n, float* y);
int32_t orc_transpose_to_time_major(const uint32_t* data, uint32_t rows, size_t cols,
                                    int32_t* flat_out);
/* codes is resized in place: returns the number of kept entries */
size_t orc_compact_codes(int32_t* codes, uint32_t num_codebooks, uint32_t max_new,
                         uint32_t n_frames);

/* ---- model ----------------------------------------------------------- */
typedef struct orc_model orc_model;

typedef struct {
  uint32_t slow_layers, fast_layers;
  uint32_t dim, ffn, heads, kv_heads, head_dim;
  uint32_t fast_dim, fast_ffn, fast_heads, fast_kv_heads, fast_head_dim;
  uint32_t vocab, codebook_size, num_codebooks;
  uint32_t semantic_begin, semantic_end;
  uint32_t slow_qk_norm, scale_codebook_embeddings;
  uint32_t linear_type; /* GGML type of layers.0.attention.wqkv.weight */
  float rope_base, fast_rope_base, eps, fast_eps;
} orc_spec;

enum {
  ORC_FAITHFUL_SLOW_RELOAD = 1, /* re-read + expand each Slow layer from the file per call */
  ORC_FAITHFUL_FAST_RECOMPUTE = 2, /* Fast-AR prefix recompute (no KV) */
  ORC_KV_F16 = 4 /* Slow-AR K/V rounded to f16 (RNE) when written to the cache, as an f16 KV store holds
                    them (KvCacheSpec's f16 layout, registry.rs:83,292-302); off: f32 as SlowArKvCache */
};

orc_model* orc_open(const char* gguf_path, uint32_t max_seq_len, uint32_t im_end_id,
                    uint32_t flags, uint32_t threads, char* err, size_t err_cap);
void orc_close(orc_model* m);
int32_t orc_get_spec(const orc_model* m, orc_spec* out);
void orc_reset(orc_model* m);
uint32_t orc_n_past(const orc_model* m);
/* hidden_out: post-final-norm hidden [dim]; logits_out: full vocab (nullable) */
int32_t orc_eval(orc_model* m, const int32_t* flat_tokens, size_t n_tokens, float* hidden_out,
                 float* logits_out, char* err, size_t err_cap);
/* embed_slow_ar_time_major alone: out [n_tokens][dim] */
int32_t orc_embed(orc_model* m, const int32_t* flat_tokens, size_t n_tokens, float* out, char* err,
                  size_t err_cap);
/* logits of the Fast-AR's last position after [slow_hidden, fast_emb[prefix]...]:
 * the recompute form with ORC_FAITHFUL_FAST_RECOMPUTE, else the incremental one */
int32_t orc_fast_logits(orc_model* m, const float* slow_hidden, const uint32_t* prefix,
                        size_t prefix_len, float* logits_out, char* err, size_t err_cap);
int32_t orc_fast_codebooks(orc_model* m, const float* slow_hidden, uint32_t semantic_code,
                           float temperature, float top_p, int32_t top_k, uint64_t* rng_state,
                           uint32_t* codes_out, char* err, size_t err_cap);
/* codes_out holds num_codebooks * max_new entries; compacted codebook-major on return */
int32_t orc_generate_codes(orc_model* m, const int32_t* prompt_flat, size_t prompt_cols,
                           uint32_t max_new_tokens, float temperature, float top_p,
                           int32_t top_k, uint32_t min_tokens_before_end, uint64_t* rng_state,
                           int32_t* codes_out, uint32_t* n_frames_out, double* prefill_seconds,
                           double* decode_seconds, char* err, size_t err_cap);


/* RVQ codec decode (crates/fish_s2_infer/src/codec.rs:1690-1714) on the CPU.
   Buffers are frame-major f32: latents/hidden [frames][1024]; the upsample
   output [4 frames][1024]; decoder samples [frames * 512]; with stop_block
   <= 4 the decoder writes the residual stream after that many blocks, with 5
   and above the samples. */
typedef struct orc_codec orc_codec;
orc_codec* orc_codec_open(const char* path, uint32_t threads, char* err, size_t cap);
void orc_codec_close(orc_codec* c);
int32_t orc_codec_rvq_lookup(orc_codec* c, const int32_t* codes, uint32_t ncb, uint32_t n_frames, float* latents,
                             char* err, size_t cap);
int32_t orc_codec_post_module(orc_codec* c, const float* latents, uint32_t n_frames, float* hidden, char* err,
                              size_t cap);
int32_t orc_codec_upsample(orc_codec* c, const float* hidden, uint32_t n_frames, float* out, char* err, size_t cap);
int32_t orc_codec_decoder(orc_codec* c, const float* hidden, uint32_t n_frames, uint32_t hidden_dim,
                          uint32_t stop_block, float* out, char* err, size_t cap);
int32_t orc_codec_decode_waveform(orc_codec* c, const int32_t* codes, uint32_t ncb, uint32_t n_frames,
                                  float* samples, char* err, size_t cap);
void orc_codec_snake(const float* x, size_t frames, size_t ch, const float* alpha, float* out);
int32_t orc_codec_conv1d(const float* x, size_t frames, size_t in_ch, size_t out_ch, size_t dilation,
                         const float* w, size_t w_len, const float* bias, float* out, char* err, size_t cap);
int32_t orc_codec_conv_transpose(const float* x, size_t frames, size_t in_ch, size_t out_ch, size_t stride,
                                 const float* w, size_t w_len, const float* bias, float* out, char* err, size_t cap);
void orc_codec_depthwise(const float* x, size_t frames, size_t ch, size_t k, const float* w, const float* bias,
                         float* out);
void orc_codec_layer_norm(float* x, size_t frames, size_t ch, const float* w, const float* b, float eps);
float orc_codec_erf(float v);
float orc_codec_gelu(float v);

#ifdef __cplusplus
}
#endif
#endif
