/*
 * s2hip.h -- C ABI of the MI355X (gfx950) dual-AR token loop.
 *
 * Drop-in for the Slow-AR / Fast-AR code generation of stevenke1981/fish-s2pro's
 * rust-pure backend (crates/fish_s2_infer).  The ABI follows the reference's
 * own native-engine convention (crates/fish_s2_infer/ffi/s2_engine_ffi.h:10-37):
 * an opaque handle from *_create (NULL on failure), int32_t returns with
 * 1 = success / 0 = failure, and the failure text copied (truncated,
 * NUL-terminated) into a caller-provided err buffer of err_cap bytes.
 * No HIP, torch or device types cross this boundary: inputs are caller-owned
 * host pointers and outputs go to caller-provided host buffers.
 *
 * Threading: a handle is not thread-safe; the caller serialises calls on one
 * handle, as the reference serialises InferenceEngine behind a Mutex
 * (crates/fish_s2_infer/src/server.rs:57, engine.rs:159).  Each handle owns
 * one HIP stream on its device.
 */
#ifndef S2HIP_H
#define S2HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define S2HIP_ABI_VERSION 1

/* GGML tensor type ids (crates/fish_s2_core/src/gguf.rs:178-200). */
#define S2HIP_GGML_F32 0u
#define S2HIP_GGML_F16 1u
#define S2HIP_GGML_Q4_0 2u
#define S2HIP_GGML_Q8_0 8u

/* s2hip_config.flags */
#define S2HIP_FLAG_NO_GRAPH 1u /* launch every frame kernel directly instead of replaying a HIP graph */
/* Store the Slow-AR KV cache as f16 (K and V rounded to nearest even when
 * written): half the KV bytes of the f32 SlowArKvCache (attention.rs:42-43),
 * in the layout KvCacheSpec describes (registry.rs:83,292-302).  Results then
 * follow an f32 cache only to about 1e-3; the Fast-AR cache stays f32. */
#define S2HIP_FLAG_KV_F16 2u
/* Collect the SlowArDecodeProfile counterpart (s2hip_last_slow_profile):
 * frames are then launched directly, one at a time, with HIP events between
 * the Slow-AR kernel groups (slower; for profiling). */
#define S2HIP_FLAG_PROFILE 4u

typedef struct s2hip_engine s2hip_engine;

typedef struct {
  const char* gguf_path;  /* transformer GGUF: F16, Q8_0 or Q4_0 linear weights */
  uint32_t max_seq_len;   /* Slow-AR KV capacity (positions), 1..32768 (SLOW_CONTEXT_LENGTH, registry.rs:10) */
  uint32_t im_end_id;     /* tokenizer <|im_end|> id (tokenizer.rs:36-62) */
  int32_t device;         /* HIP device ordinal */
  uint32_t flags;         /* S2HIP_FLAG_* */
} s2hip_config;

/* Model shape read from GGUF metadata (registry.rs:45-214), shape-generic. */
typedef struct {
  uint32_t slow_layers, fast_layers;
  uint32_t dim, ffn, heads, kv_heads, head_dim;
  uint32_t fast_ffn, fast_heads, fast_kv_heads, fast_head_dim;
  uint32_t vocab, codebook_size, num_codebooks;
  uint32_t semantic_begin, semantic_end;
  uint32_t slow_qk_norm, scale_codebook_embeddings;
  uint32_t linear_type; /* GGML type of the linear weights */
  uint32_t max_seq_len;
  float rope_base, fast_rope_base, eps, fast_eps;
  uint64_t weight_bytes; /* bytes resident in HBM for all tensors */
} s2hip_spec;

/* SamplerParams (crates/fish_s2_infer/src/sampling.rs:12-27). */
typedef struct {
  float temperature;
  float top_p;
  int32_t top_k;
} s2hip_sampler;

/* GenerateParams (crates/fish_s2_infer/src/generate.rs:13-32). */
typedef struct {
  uint32_t max_new_tokens;
  float temperature;
  float top_p;
  int32_t top_k;
  uint32_t min_tokens_before_end;
} s2hip_gen_params;

/* Timing of one s2hip_generate_codes call (HIP events on the engine stream). */
typedef struct {
  double prefill_ms; /* prompt prefill + first semantic sample */
  double decode_ms;  /* all frames: Fast-AR codebooks + Slow-AR step + sampling */
  uint32_t n_frames;
  uint32_t graph_used;
  /* 1 when an activation beyond the range of the batched product (one more
   * than 2^15 times the largest of the first 256 in its wave's share of the
   * row) made the call run again from its inputs with every multi-column
   * linear on the per-column paths, whose split scale covers the whole row */
  uint32_t per_column_rerun;
  /* 1: a one-request greedy call met a tie at the max of a Fast-AR sample
   * folded into the next sub-step's first linear, and ran again from its
   * inputs with the sampler kernel, which resolves ties as the reference */
  uint32_t greedy_rerun;
} s2hip_gen_stats;

/* SlowArDecodeProfile (crates/fish_s2_infer/src/slow_ar.rs:248-319, filled by
 * generate_codes at generate.rs:129,195 and shown by the GUI at app.rs:664-669):
 * device time of the Slow-AR decode steps of the last generate call, by
 * operation, in milliseconds.  The kernels fuse the reference's operations,
 * so each kernel's time goes to one field: linear = wqkv (with the attention
 * RMSNorm), wo (+ residual), w1/w3 (with the FFN RMSNorm and SwiGLU) and w2
 * (+ residual); gqa_attention = QK-norm, RoPE, KV write, attention and the
 * cross-chunk merge; output_head = final RMSNorm + head rows.  rms_norm,
 * rope, kv_write and swiglu are 0: they run inside those kernels. */
typedef struct {
  double rms_norm_ms, linear_ms, gqa_attention_ms, rope_ms, kv_write_ms, swiglu_ms, output_head_ms;
  uint32_t steps; /* Slow-AR decode steps (frames x requests) covered */
} s2hip_slow_profile;

const char* s2hip_version(void);

/* SlowArState::open (crates/fish_s2_infer/src/slow_ar.rs:387-412) +
 * FastArWeights::from_gguf (fast_ar.rs:202-224): parse the GGUF once and
 * upload every tensor to HBM in its native block layout; allocate the
 * device KV cache for max_seq_len positions. */
s2hip_engine* s2hip_create(const s2hip_config* cfg, char* err, size_t err_cap);
void s2hip_destroy(s2hip_engine* engine);
int32_t s2hip_get_spec(const s2hip_engine* engine, s2hip_spec* out);

/* SlowArState::reset (slow_ar.rs:434-438). */
int32_t s2hip_reset(s2hip_engine* engine, char* err, size_t err_cap);
/* SlowArState::n_past (slow_ar.rs:418-420). */
uint32_t s2hip_n_past(const s2hip_engine* engine);

/* The same on KV slot `slot` (0..15).  The engine holds up to 16 independent
 * sequence states: slot 0 is the one s2hip_reset / s2hip_eval / s2hip_n_past
 * act on, and request b of s2hip_generate_codes_batch leaves its state in
 * slot b.  The reference's SlowArState holds one sequence
 * (slow_ar.rs:372-438); a caller keeping several sequences open (a server
 * with concurrent requests) uses one slot per sequence. */
int32_t s2hip_reset_slot(s2hip_engine* engine, uint32_t slot, char* err, size_t err_cap);
uint32_t s2hip_n_past_slot(const s2hip_engine* engine, uint32_t slot);
int32_t s2hip_eval_slot(s2hip_engine* engine, uint32_t slot, const int32_t* flat_tokens, size_t n_tokens,
                        float* hidden_out, float* logits_out, char* err, size_t err_cap);

/* transpose_to_time_major (crates/fish_s2_infer/src/prompt.rs:79-103):
 * data holds the codebook-major prompt tensor of build_prompt, rows x cols
 * (row 0 vocabulary ids, rows 1.. codes); flat_out[t * rows + r] =
 * data[r * cols + t], the layout the entry points below take.  Fails (0) with
 * the reference's messages when rows == 0, rows * cols overflows or differs
 * from data_len, or a value does not fit i32.  Host only: no engine, no
 * device. */
int32_t s2hip_transpose_to_time_major(const uint32_t* data, size_t data_len, uint32_t rows, size_t cols,
                                      int32_t* flat_out, char* err, size_t err_cap);

/* SlowArState::prefill / step / eval (slow_ar.rs:440-527): flat_tokens is
 * time-major [n_tokens][num_codebooks + 1].  hidden_out receives the
 * post-final-norm hidden of the last token [dim]; logits_out (nullable)
 * receives the full-vocabulary logits [vocab]. */
int32_t s2hip_eval(s2hip_engine* engine, const int32_t* flat_tokens, size_t n_tokens, float* hidden_out,
                   float* logits_out, char* err, size_t err_cap);

/* forward_codebook_prefix (crates/fish_s2_infer/src/fast_ar.rs:360-437):
 * logits_out [codebook_size]. */
int32_t s2hip_fast_logits(s2hip_engine* engine, const float* slow_hidden, const uint32_t* prefix_codes,
                          size_t prefix_len, float* logits_out, char* err, size_t err_cap);

/* generate_codebooks_for_semantic (fast_ar.rs:440-470): codes_out
 * [num_codebooks]; rng_state is the SeededRng state (sampling.rs:34-52),
 * updated in place. */
int32_t s2hip_fast_codebooks(s2hip_engine* engine, const float* slow_hidden, uint32_t semantic_code,
                             const s2hip_sampler* sampler, uint64_t* rng_state, uint32_t* codes_out, char* err,
                             size_t err_cap);

/* generate_codes (crates/fish_s2_infer/src/generate.rs:117-221): prompt_flat is
 * time-major [prompt_cols][num_codebooks + 1] (prompt.rs:77-103).  codes_out
 * holds num_codebooks * max_new_tokens entries and receives the compacted
 * codebook-major codes [num_codebooks][n_frames] (generate.rs:346-390).
 * stats is nullable. */
int32_t s2hip_generate_codes(s2hip_engine* engine, const int32_t* prompt_flat, size_t prompt_cols,
                             const s2hip_gen_params* params, uint64_t* rng_state, int32_t* codes_out,
                             uint32_t* n_frames_out, s2hip_gen_stats* stats, char* err, size_t err_cap);

/* The profile of the last s2hip_generate_codes / _batch call on an engine
 * created with S2HIP_FLAG_PROFILE (all zero otherwise); engine.rs:221
 * (last_slow_ar_profile). */
int32_t s2hip_last_slow_profile(const s2hip_engine* engine, s2hip_slow_profile* out);

/* Batched generate_codes: n_requests (1..16) independent requests decoded
 * together, each in its own KV slot, so every frame reads each weight matrix
 * once for the whole batch.  Request b is prompts[b] ([prompt_cols[b]]
 * [num_codebooks + 1], time-major), its SeededRng state rng_states[b]
 * (updated in place), and its output codes[b] / n_frames_out[b] exactly as
 * for s2hip_generate_codes; params are shared.  A finished request stops
 * contributing codes while the others continue.  The reference serves one
 * request at a time (single SlowArState, slow_ar.rs:387-438); this entry
 * point has no counterpart there and is for callers serving concurrent
 * requests, which the reference's server runs one at a time behind a Mutex
 * (server.rs:57).  stats->n_frames is
 * the total over requests.  Slot KV memory (max_seq_len positions per
 * request) is allocated on the first call with a larger batch; afterwards the
 * engine's sequence state (s2hip_n_past, s2hip_eval) is request 0's. */
int32_t s2hip_generate_codes_batch(s2hip_engine* engine, uint32_t n_requests, const int32_t* const* prompts,
                                   const size_t* prompt_cols, const s2hip_gen_params* params,
                                   uint64_t* rng_states, int32_t* const* codes_out, uint32_t* n_frames_out,
                                   s2hip_gen_stats* stats, char* err, size_t err_cap);

/* ---- op level: the MatmulBackend seam (crates/fish_s2_infer/src/backend.rs:5-39)
 * and the other per-op functions, run on the engine's device with host
 * inputs/outputs.  Used by parity dumps and tests. */

/* MatmulBackend::linear (backend.rs:8-14) generalised to GGML row types:
 * y[c][o] = sum_i x[c][i] * W[o][i] for n_cols input columns.  weight holds
 * out_dim GGML rows of in_dim elements (F16 / Q8_0 / Q4_0). */
int32_t s2hip_op_linear(s2hip_engine* engine, const void* weight, uint32_t ggml_type, size_t in_dim,
                        size_t out_dim, const float* x, size_t n_cols, float* y, char* err, size_t err_cap);
/* MatmulBackend::rms_norm (backend.rs:16-18) over n_cols vectors. */
int32_t s2hip_op_rms_norm(s2hip_engine* engine, const float* x, const float* weight, size_t n, size_t n_cols,
                          float eps, float* y, char* err, size_t err_cap);
/* Q-block / f16 dequantisation of `rows` GGML rows to f32 (bit-exact). */
int32_t s2hip_op_dequant_rows(s2hip_engine* engine, const void* weight, uint32_t ggml_type, size_t in_dim,
                              size_t rows, float* out, char* err, size_t err_cap);
/* Slow-AR prepare step: QK-norm (if q_norm/k_norm non-NULL) + apply_rope_normal
 * (attention.rs:172-206) at `position`, on one token's qkv row
 * [(heads + 2 kv_heads) head_dim]; outputs q [heads*hd], k and v [kv_heads*hd]. */
int32_t s2hip_op_qk_rope(s2hip_engine* engine, const float* qkv, uint32_t heads, uint32_t kv_heads,
                         uint32_t head_dim, uint32_t position, float rope_base, const float* q_norm,
                         const float* k_norm, float eps, float* q_out, float* k_out, float* v_out, char* err,
                         size_t err_cap);
/* MatmulBackend::gqa_decode_attention (backend.rs:30-38): keys/values
 * [token_count][kv_heads][head_dim]. */
int32_t s2hip_op_attention(s2hip_engine* engine, const float* q, const float* keys, const float* values,
                           uint32_t heads, uint32_t kv_heads, uint32_t head_dim, uint32_t token_count,
                           float attn_scale, float* out, char* err, size_t err_cap);
/* swiglu_split: Slow (slow_ar.rs:1215-1232) when fast == 0, Fast (fast_ar.rs:472-485) otherwise. */
int32_t s2hip_op_swiglu(s2hip_engine* engine, const float* gate, const float* up, size_t n, int32_t fast,
                        float* out, char* err, size_t err_cap);
/* sample_token (sampling.rs:120-241); always_include < 0 means None. */
int32_t s2hip_op_sample(s2hip_engine* engine, const float* logits, size_t n, const s2hip_sampler* sampler,
                        int64_t always_include, uint64_t* rng_state, uint32_t* token_out, char* err,
                        size_t err_cap);

/* s2hip_op_sample without any device allocation: no hipMalloc / hipFree, the
 * logits and the RNG / token / error words are staged in a file-scope device
 * array of 32 KiB + 256 B per GPU (held until the process ends), so n is at
 * most 8191 (larger n fails with an error naming the limit).  Same results
 * as s2hip_op_sample.  No counterpart in the reference: for callers that
 * cannot allocate device memory (tight serving loops, code that forbids
 * hipMalloc).  Calls that overlap on one GPU race on the shared array. */
int32_t s2hip_op_sample_noalloc(s2hip_engine* engine, const float* logits, size_t n, const s2hip_sampler* sampler,
                                int64_t always_include, uint64_t* rng_state, uint32_t* token_out, char* err,
                                size_t err_cap);

/* Test hook, no counterpart in the reference: the number of device
 * allocations (hipMalloc) the dual-AR engines of this process have made so
 * far, so that a test can check that an entry point allocates nothing. */
void s2hip_device_allocations(uint64_t* count_out);

/* The samplers' sequential f32 running sums (softmax normaliser, top-p
 * cumulative sum and draw of sample_token, sampling.rs:202-241, whose Rust
 * loops add term by term in index order): prefix_out[i] = fl(prefix_out[i-1]
 * + terms[i]) for n <= 8192 terms, total_out = the last one (0 for n = 0).
 * A test hook for the device summation routine. */
int32_t s2hip_op_running_sums(s2hip_engine* engine, const float* terms, size_t n, float* prefix_out,
                              float* total_out, char* err, size_t err_cap);

/* The samplers' cut search (sampling.rs:202-241: the top-p loop stops at the
 * first item whose running sum reaches top_p; the draw takes the first item
 * whose running sum exceeds the target): over n <= 8192 non-negative terms,
 * cut_out = the first i with prefix(i) >= threshold (n if none; a NaN
 * threshold never matches), sum_out = prefix(cut) (the total if none),
 * at_sum_out = prefix(at) when at < n.  absorb != 0 lets the device stop once
 * the terms no longer change the sum; it requires non-increasing terms.
 * Results equal those of the full sequential loop.  A test hook. */
int32_t s2hip_op_running_cut(s2hip_engine* engine, const float* terms, size_t n, float threshold, int32_t absorb,
                             size_t at, size_t* cut_out, float* sum_out, float* at_sum_out, char* err,
                             size_t err_cap);

/* embed_slow_ar_time_major (crates/fish_s2_infer/src/slow_ar.rs:1041-1133):
 * out[t][dim] = emb[id] (+ the sum of the token's codebook rows, then the
 * 1/sqrt(num_codebooks + 1) scale, for semantic ids) for flat_tokens
 * time-major [n_tokens][num_codebooks + 1]; the token checks of eval. */
int32_t s2hip_op_embed(s2hip_engine* engine, const int32_t* flat_tokens, size_t n_tokens, float* out, char* err,
                       size_t err_cap);

/* The device exp of the samplers' softmax (sampling.rs:202-225) and the
 * SwiGLU sigmoids (slow_ar.rs:1215-1232, fast_ar.rs:472-485), whose Rust code
 * calls f32::exp, i.e. the C library's expf: y[i] = exp(x[i]) with the
 * results of glibc's expf, computed on the device.  A test hook. */
int32_t s2hip_op_expf(s2hip_engine* engine, const float* x, size_t n, float* y, char* err, size_t err_cap);
/* The same routine compiled for the host (no device needed): the CPU test of
 * its bits against the C library's expf.  A test hook. */
void s2hip_expf_host(const float* x, size_t n, float* y);

/* Measurement: average device time of one launch of a named decode kernel,
 * timed with HIP events on the engine stream over `reps` passes across every
 * layer (so no pass re-reads weights from cache).  kernel: "slow_w13",
 * "slow_wqkv", "slow_wo", "slow_w2", "slow_head", "slow_attn", "fast_attn",
 * "fast_head", "sample_fast", "sample_slow" (greedy; with suffix "_topp":
 * T 0.7, top-p 0.9; "_default": T 0.7, top-p 0.7, top-k 30), "fast_frame", "empty" (one
 * one-wave launch), "hbm_copy" (a 256 MiB device copy, the calibration kernel
 * for HBM byte counters).  bytes_per_launch receives the algorithmic HBM
 * bytes of one launch (weights + input + output) where defined, else 0.
 * No counterpart in the reference (a measurement hook). */
int32_t s2hip_time_kernel(s2hip_engine* engine, const char* kernel, uint32_t reps, double* avg_us,
                          double* bytes_per_launch, char* err, size_t err_cap);

/* ---------------------------------------------------------------------------
 * RVQ codec decode on the GPU: decode_waveform (crates/fish_s2_infer/src/codec.rs:1690-1714)
 * = rvq_lookup_codes (:2536-2596) -> forward_codec_post_module (:986-1018) ->
 * forward_codec_upsample (:2302-2325) -> forward_codec_decoder (:1941-2001),
 * the pipeline's stage after generate_codes (pipeline.rs:166-199).  Weights come
 * from the codec GGUF (architecture "fish-speech-codec"; the decode-side
 * tensors the reference's registry names, codec.rs:58-265, all F16) and stay
 * in HBM.  Buffers are frame-major f32 on the host: codes codebook-major
 * [num_codebooks][n_frames]; latents / hidden [n_frames][1024]; the
 * upsample output [4 n_frames][1024]; samples [n_frames * 2048] (44.1 kHz).
 * Errors follow the reference's texts (codebook count, negative code,
 * "embedding index N out of range for vocab_dim V", "codec transformer
 * requires at least one frame", "decoder expects latent dim 1024, got N").
 * Unlike the reference, a handle decodes at most max_frames code frames per
 * call (buffers are sized once at open).
 * ------------------------------------------------------------------------- */
typedef struct s2hip_codec s2hip_codec;

/* CodecWaveformResult (codec.rs:1681-1688) without the samples themselves. */
typedef struct {
  uint32_t sample_rate; /* 44100 */
  uint32_t input_frames;
  uint32_t latent_frames;
  size_t num_samples;
} s2hip_waveform_info;

/* CodecF16Weights / CodecPostModuleF16Weights / CodecUpsampleF16Weights /
 * CodecDecoderF16Weights ::from_gguf (codec.rs:2334-2360, 502-520, 1614-1640);
 * max_frames: 1..4096 code frames per call. */
s2hip_codec* s2hip_codec_open(const char* codec_gguf_path, uint32_t max_frames, int32_t device, char* err,
                              size_t err_cap);
void s2hip_codec_close(s2hip_codec* codec);
/* rvq_lookup_codes (codec.rs:2536-2596): latents [n_frames][1024]. */
int32_t s2hip_codec_rvq_lookup(s2hip_codec* codec, const int32_t* codes, uint32_t num_codebooks, uint32_t n_frames,
                               float* latents, char* err, size_t err_cap);
/* forward_codec_post_module (codec.rs:986-1018). */
int32_t s2hip_codec_post_module(s2hip_codec* codec, const float* latents, uint32_t n_frames, float* hidden,
                                char* err, size_t err_cap);
/* forward_codec_upsample (codec.rs:2302-2325): out [4 n_frames][1024]. */
int32_t s2hip_codec_upsample(s2hip_codec* codec, const float* hidden, uint32_t n_frames, float* out, char* err,
                             size_t err_cap);
/* rvq_decode_latents (codec.rs:1282-1297): post-module then upsample. */
int32_t s2hip_codec_decode_latents(s2hip_codec* codec, const float* latents, uint32_t n_frames, float* out,
                                   char* err, size_t err_cap);
/* forward_codec_decoder (codec.rs:1941-2001) over n_frames latent frames:
 * stop_block >= 5 writes the samples [n_frames * 512]; 0..4 writes the
 * residual stream after that many decoder blocks (a stage checkpoint,
 * [n_frames * prod(rates[:stop_block])][channels], rates 8, 8, 4, 2, channels
 * 1536, 768, 384, 192, 96).  out_len receives the floats written. */
int32_t s2hip_codec_decoder(s2hip_codec* codec, const float* hidden, uint32_t n_frames, uint32_t hidden_dim,
                            uint32_t stop_block, float* out, size_t out_cap, size_t* out_len, char* err,
                            size_t err_cap);
/* decode_waveform (codec.rs:1690-1714): samples [n_frames * 2048] in [-1, 1]. */
int32_t s2hip_codec_decode_waveform(s2hip_codec* codec, const int32_t* codes, uint32_t num_codebooks,
                                    uint32_t n_frames, float* samples, size_t samples_cap, s2hip_waveform_info* info,
                                    char* err, size_t err_cap);
/* decode_waveform with codes and samples in device memory of the codec's
 * device (the pipeline keeps generate_codes' output on the GPU); codes are
 * range-checked on the device.  No counterpart in the reference. */
int32_t s2hip_codec_decode_waveform_device(s2hip_codec* codec, const int32_t* codes_dev, uint32_t num_codebooks,
                                           uint32_t n_frames, float* samples_dev, char* err, size_t err_cap);
/* The snake activation of the codec's device kernels, x + sin(a x)^2 / a with
 * the reference's guard (snake_activation_frame_major, codec.rs:2162-2186),
 * evaluated on the host by the same routine: y[i] = snake(x[i], alpha[i]).
 * A test hook (its sin is not the C library's sinf). */
void s2hip_codec_snake_host(const float* x, size_t n, const float* alpha, float* y);
/* Measurement: average device time (HIP events on the codec stream) of
 * `what` over `reps` launches, after one untimed decode of n_frames frames of
 * fixed codes: "decode" (the whole decode_waveform on device buffers) or one
 * convolution of that decode by name ("entry", "b1_convT" .. "b4_convT",
 * "b<1-4>_r<1-3>_conv0" / "_conv1", "up1_convT", "up1_pw1", "up1_pw2",
 * "up2_..."), relaunched with the same arguments.  flops receives 2 x the
 * multiply-adds of one launch (for "decode": of all its convolutions).
 * No counterpart in the reference (a measurement hook). */
int32_t s2hip_codec_time(s2hip_codec* codec, const char* what, uint32_t n_frames, uint32_t reps, double* avg_us,
                         double* flops, char* err, size_t err_cap);

#ifdef __cplusplus
}
#endif
#endif
