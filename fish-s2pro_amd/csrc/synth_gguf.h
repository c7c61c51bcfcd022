/* synth_gguf.h -- seeded synthetic dual-AR and codec GGUF writers (host-only helper). */
#ifndef S2SYNTH_GGUF_H
#define S2SYNTH_GGUF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
  uint32_t slow_layers, dim, ffn, heads, kv_heads, head_dim;
  uint32_t fast_layers, fast_ffn, fast_heads, fast_kv_heads, fast_head_dim;
  uint32_t vocab, codebook_size, num_codebooks, semantic_begin, semantic_end;
  uint32_t context_length;
  uint32_t linear_type; /* GGML type of every linear weight: 1 F16, 8 Q8_0, 2 Q4_0 */
  float rope_base, fast_rope_base, eps, fast_eps;
  float init_std;
  float norm_gain; /* value of every residual-stream RMSNorm gain (attention/ffn/final norms); 0 means 1 */
  uint64_t seed;
} s2synth_config;

/* Returns 1 on success, 0 on failure with a message in err. */
int32_t s2synth_write_gguf(const char* path, const s2synth_config* cfg, uint32_t threads, char* err,
                           size_t err_cap);
/* Decode-side tensors of a synthetic RVQ codec GGUF (quantizers, post_module,
   upsample, decoder), seeded; every tensor F16. */
int32_t s2synth_write_codec_gguf(const char* path, uint64_t seed, uint32_t threads, char* err, size_t err_cap);
uint16_t s2synth_f32_to_f16(float v);
/* Quantise one 32-element block into Q8_0 (34 B) or Q4_0 (18 B). */
int32_t s2synth_quantize_block(uint32_t type, const float* x, uint8_t* out);

#ifdef __cplusplus
}
#endif
#endif
