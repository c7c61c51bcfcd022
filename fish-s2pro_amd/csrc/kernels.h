// kernels.h -- launch interface of the s2hip device kernels (gfx950, wave64).
//
// All activations are f32.  Weights stay in their GGUF block layout:
// row-major [out][in] with `in` contiguous; F16 rows, or GGML Q8_0 / Q4_0
// blocks of 32 elements along `in`.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace s2 {

enum WeightType : uint32_t { W_F16 = 1, W_Q4_0 = 2, W_Q8_0 = 8 };

enum Epilogue : int {
  EPI_STORE = 0,        // y[c][o] = acc
  EPI_RESID = 1,        // y[c][o] = y[c][o] + acc (residual add in place)
  EPI_SWIGLU_SLOW = 2,  // y[c][o] = g * (1 / (1 + e^-g)) * u
  EPI_SWIGLU_FAST = 3,  // y[c][o] = g / (1 + e^-g) * u
};

// Per-sequence device state read by graph-replayed kernels.
struct DevState {
  uint32_t n_past;      // Slow-AR positions already in the KV cache
  uint32_t step_index;  // frames generated
  uint32_t done;        // set once im_end is sampled or max_new frames exist
  uint32_t main_token;  // last sampled Slow-AR token
  uint32_t err;         // error bits (ERR_*)
  uint32_t prompt_cols;
  uint32_t max_new;
  uint32_t min_tokens_before_end;
  uint64_t rng;         // SeededRng state
  uint32_t codes_frame[16];  // codebook ids of the frame being built
};

enum : uint32_t {
  ERR_TOKEN_RANGE = 1u,
  ERR_KV_OVERFLOW = 2u,
  ERR_SAMPLER = 4u,
  ERR_F16_RANGE = 8u,
  ERR_NONFINITE = 16u,
  ERR_GREEDY_TIE = 32u,  // a folded greedy sample met a tie (the call re-runs with the sampler kernel)
};
constexpr uint32_t NO_ROW = 0xffffffffu;

// Weight rows of the GEMV launched next, read into L2 by extra blocks of a
// latency-bound kernel (decode attention) while HBM would otherwise idle.
// GEMV block cb covers bytes [cb span, cb span + span) from base (and from
// base3) and runs on XCD cb % 8: workgroups go to the 8 XCDs round-robin by
// linear index, each XCD with its own L2.  The warming block at linear index
// L reads only consumer blocks with cb % 8 == L % 8, so each row lands in the
// L2 that reads it next.  Reads only: a different mapping costs bandwidth,
// never results.
struct L2Warm {
  const uint8_t* base;   // nullptr: no warming blocks
  const uint8_t* base3;  // nullable: second matrix, same layout (w3 of SwiGLU)
  uint32_t span;         // bytes per consumer block, multiple of 16
  uint32_t cb_begin;     // consumer blocks [cb_begin, cb_end) are warmed;
  uint32_t cb_end;       //   cb_begin is a multiple of 8
  uint32_t blocks;       // warming blocks, multiple of 8
  uint32_t depth;        // 16-byte loads per thread in flight: 4, 8 or 16
};
// The Fast-AR greedy sample folded into the next sub-step's first linear
// (one column, RMSNorm): every block reduces the codebook logits to their
// argmax and reads x = emb[argmax] (f16 rows of `in` elements) instead of x;
// block 0 also writes x to x_out, the code to st->codes_frame[cb_index] and
// steps st->rng once, as the sampler kernel would.  A maximum that is not
// unique within 1e-6 (or not finite) sets ERR_GREEDY_TIE.
struct GreedyFold {
  const float* logits;   // nullptr: no fold
  uint32_t n;            // codebook size (a multiple of 4)
  const uint16_t* emb;   // [n][in] f16
  DevState* st;
  uint32_t cb_index;
  float* x_out;          // [dim]
  uint32_t dim;          // row length of emb / x_out (the linear's input length)
};

struct GemvArgs {
  const uint8_t* w;      // weight rows
  const uint8_t* w3;     // second matrix for SwiGLU epilogues (same shape)
  size_t row_bytes;
  // logical row r < out maps to weight row row_base + r, except that when
  // extra_row != NO_ROW the last logical row (out - 1) maps to extra_row
  uint32_t row_base;
  uint32_t extra_row;
  uint32_t in, out;      // `out` logical rows
  const float* x;        // [ncol][ldx]
  uint32_t ldx;
  const float* norm;     // optional RMSNorm gain [in] applied to x first
  float eps;
  float* y;              // [ncol][ldy]
  uint32_t ldy;
  const uint32_t* done;  // optional early-exit flag
  // Q8_0 / Q4_0 only, nullable: the rows repacked by launch_repack_q (quant
  // plane, f16 scale plane); with them, one column runs gemv_q_kernel
  const uint8_t* qp;
  const uint8_t* qp3;
  const uint16_t* qs;
  const uint16_t* qs3;
  GreedyFold fold;       // fold.logits != nullptr: x comes from the greedy sample
  // nullable, with norm: block 0 also writes the normalised x (x * scale *
  // gain, [ncol][ldx]) there (the RMSNorm GEMV form serves such launches)
  float* xn_out;
};

// Q8_0 / Q4_0 rows repacked for the decode GEMV: block b of row r (32
// elements) -> quant plane at (r * in / 32 + b) * QB bytes (QB = 32 for Q8_0:
// the int8 values; 16 for Q4_0: the 16 nibble bytes, GGML order) and its f16
// scale at scale plane index r * in / 32 + b.
uint32_t repack_quant_bytes(uint32_t wtype);  // QB, 0 for other types
hipError_t launch_repack_q(const uint8_t* rows, size_t row_bytes, uint32_t wtype, uint32_t in, uint32_t nrows,
                           uint8_t* qplane, uint16_t* splane, hipStream_t s);

struct SamplerCfg {
  float temperature;
  float top_p;
  int32_t top_k;
};

// GEMV over `ncol` input columns (1, 2, 4 or 8).
hipError_t launch_gemv(uint32_t wtype, int epi, int ncol, const GemvArgs& a, hipStream_t s);

// Per-column RMSNorm: y[c] = (x[c] * scale_c) * w.
hipError_t launch_rms_norm(const float* x, const float* w, float* y, uint32_t n, uint32_t ncol, float eps,
                           const uint32_t* done, hipStream_t s);

// QK-norm (optional) + NORMAL RoPE + KV append for `ncol` consecutive positions
// starting at *pos_ptr + pos_offset.  qkv: [ncol][(H + 2 Hkv) hd].
struct QkvPostArgs {
  const float* qkv;
  float* q_out;            // [ncol][H hd]
  float* k_cache;          // [Hkv][max_seq][hd] for this layer
  float* v_cache;
  const float* q_norm;     // nullable
  const float* k_norm;     // nullable
  const float2* rope;      // [max_pos][hd/2] (cos, sin)
  const uint32_t* pos_ptr; // nullable: base position = *pos_ptr + pos_offset
  uint32_t pos_offset;
  uint32_t H, Hkv, hd, max_seq, ncol;
  float eps;
  const uint32_t* done;
  uint32_t* err;
  uint32_t kv_f16;         // 1: the caches hold f16 (K and V rounded to nearest even when written)
};
hipError_t launch_qkv_post(const QkvPostArgs& a, hipStream_t s);

// Warming planes a kernel of `plane` blocks per plane appends for w (0 when
// w.base is null); hipErrorInvalidValue in *err for a malformed descriptor.
uint32_t l2_warm_planes(const L2Warm& w, uint32_t plane, hipError_t* err);
// Rows per block of the decode GEMV launch_gemv picks for 1-2 columns, this
// weight type and row length (norm: RMS-normalised input; dual: SwiGLU
// pair), or 0 when another kernel serves the shape.
uint32_t gemv_rows_per_block(uint32_t wtype, uint32_t in, uint32_t out, bool norm, bool dual, uint32_t ncol);

// Fused decode attention for ncol / cols_per_seq sequences, each with
// cols_per_seq consecutive query positions starting at its *pos_ptr +
// pos_offset: QK-norm (optional) + RoPE of q and of the new k, KV append at
// the position, split-T GQA attention over positions [0, pos] and the
// cross-chunk combine.  qkv: [ncol][(H + 2 Hkv) hd] raw wqkv output,
// sequence-major.  hd must be 64 or 128, H / Hkv <= 4, cols_per_seq <= 4.
struct AttnArgs {
  const float* qkv;
  const float* q_norm;     // nullable
  const float* k_norm;     // nullable
  float eps;
  const float2* rope;      // [max_pos][hd/2] (cos, sin)
  float* k_cache;          // [Hkv][max_seq][hd] for this layer, sequence 0
  float* v_cache;
  float* part;             // [ncol][Hkv][max_chunks][rep][hd + 2]
  uint32_t* counters;      // [ncol][Hkv], zero between launches
  float* out;              // [ncol][H hd]
  const uint32_t* pos_ptr; // nullable (positions from pos_offset alone)
  uint32_t pos_offset;
  uint32_t H, Hkv, hd, max_seq, ncol;
  uint32_t max_chunks;     // attention_chunks(max_seq, mode)
  uint32_t mode;           // ATTN_SPLIT: partial + merge kernels; ATTN_FUSED: one kernel, last block merges
  float scale;
  const uint32_t* done;    // nullable
  uint32_t* err;
  // sequences: 0 = one sequence of ncol columns.  Sequence b uses the caches
  // at + b * seq_stride_kv floats and the pos / done / err words at
  // + b * seq_stride_words.
  uint32_t cols_per_seq;
  uint32_t seq_stride_words;
  size_t seq_stride_kv;
  L2Warm warm;             // rows of the next GEMV (wo) warmed by extra blocks of the partial kernel
  uint32_t kv_f16;         // 1: k_cache / v_cache hold f16 (seq_stride_kv and offsets in elements)
  // nonzero: chunks >= check_from read their sequence's position before
  // their K/V tile and end without loading it when they lie past the
  // sequence; chunks below it load the tile first (set it to a lower bound of
  // every sequence's chunk count, so that only chunks that may be dead wait)
  uint32_t check_from;
  // one column: q / k / v from row `code` of qkv_rows ([fold.n][(H + 2 Hkv)
  // hd]) instead of qkv, code = *code_ptr or, with fold.logits, the greedy
  // sample of the logits (then block 0 also has the sampler's side effects,
  // as GemvArgs::fold).  nullptr: qkv.
  const float* qkv_rows;
  const uint32_t* code_ptr;
  GreedyFold fold;
};
enum : uint32_t { ATTN_SPLIT = 0u, ATTN_FUSED = 1u };
constexpr uint32_t ATTN_CHUNK = 32;         // cache positions per decode attention block
constexpr uint32_t ATTN_MAX_CHUNKS = 1024;  // max_seq <= 32768
uint32_t attention_chunks(uint32_t max_seq, uint32_t mode);
hipError_t launch_attention(const AttnArgs& a, hipStream_t s);

// Slow-AR token embedding (time-major flat ids [n][cdim]).
struct EmbedArgs {
  const int32_t* tokens;       // nullable: use the device step input built from state
  const DevState* state;       // used when tokens == nullptr: row t from state[t]
  const uint16_t* emb;         // [vocab][dim] f16
  const uint16_t* cb_emb;      // [cb_rows][dim] f16
  float* h;                    // [n][dim]
  uint32_t n, dim, vocab, cb_rows, num_codebooks, codebook_size, sem_begin, sem_end;
  float sem_scale;             // 1/sqrt(num_codebooks+1) or 1
  uint32_t scale_enabled;
  const uint32_t* done;
  uint32_t* err;
  L2Warm warm;                 // rows of the next GEMV (layer 0 wqkv), warmed by extra blocks
};
hipError_t launch_embed(const EmbedArgs& a, hipStream_t s);

// Fast-AR frame start of n_seq sequences: st[b].codes_frame[0] = semantic code
// of st[b].main_token, fh[b][0] = slow_hidden[b], fh[b][1] = fast_emb[code0].
hipError_t launch_fast_begin(DevState* st, const float* slow_hidden, const uint16_t* fast_emb, float* fh,
                             uint32_t dim, uint32_t codebook_size, uint32_t sem_begin, uint32_t sem_end,
                             uint32_t n_seq, hipStream_t s);

// Batch completion word set when every sequence of a batch is done.
struct BatchState {
  uint32_t done_all;
  uint32_t done_count;
  uint32_t n_seq;
};

// Sampling.  Slow mode: logits over candidate rows `ids` (ascending vocab ids),
// full vocab `vocab`; applies the semantic mask / im_end rule and updates the
// frame state.  Fast mode: logits over codebook ids, writes codes_frame[cb] and
// the next Fast-AR input row.
struct SampleArgs {
  const float* logits;
  const uint32_t* ids;       // nullable: id = index
  uint32_t n;                // candidates
  uint32_t vocab;            // full vocabulary size
  SamplerCfg cfg;
  DevState* st;
  // slow mode
  uint32_t im_end;
  uint32_t after_step;       // 1: a Slow step just ran (advance frame counters)
  uint32_t advance;          // added to n_past of each unfinished sequence first (the step's position)
  int32_t* codes_out;        // [num_codebooks][max_new] codebook-major (nullable)
  uint32_t num_codebooks;
  // fast mode
  uint32_t cb_index;         // codebook being sampled (1..num_codebooks-1)
  const uint16_t* fast_emb;  // next-input gather (nullable)
  float* next_input;
  uint32_t dim;
  uint32_t* token_out;       // optional copy of the sampled id
  // n_seq sequences (0 means 1): sequence b reads logits + b * n and uses
  // st[b], codes_out + b * codes_stride, next_input + b * dim, token_out[b]
  uint32_t n_seq;
  size_t codes_stride;
  BatchState* batch;         // nullable: counts finished sequences
  L2Warm warm;               // rows of the next GEMV, warmed by extra blocks
};
hipError_t launch_sample_slow(const SampleArgs& a, hipStream_t s);
hipError_t launch_sample_fast(const SampleArgs& a, hipStream_t s);
// Plain sample_token over `n` logits (ids = index) with optional always-include id.
hipError_t launch_sample_plain(const float* logits, uint32_t n, SamplerCfg cfg, int64_t always_include,
                               uint64_t* rng, uint32_t* token_out, uint32_t* err, hipStream_t s);

// Expand GGML rows to f32 (bit-exact dequantisation).
hipError_t launch_dequant_rows(uint32_t wtype, const uint8_t* w, size_t row_bytes, uint32_t rows, uint32_t in,
                               float* out, hipStream_t s);

hipError_t launch_swiglu(const float* g, const float* u, float* out, uint32_t n, int fast, hipStream_t s);
// y[i] = expf_glibc(x[i]) (the device exp of the samplers and SwiGLU epilogues).
hipError_t launch_expf(const float* x, float* y, size_t n, hipStream_t s);
// Sequential f32 running sums of n <= 8192 terms (the samplers' summation routine).
hipError_t launch_running_sum(const float* terms, uint32_t n, float* prefix, float* total, hipStream_t s);
// The samplers' cut search over n <= 8192 terms: cut[0] = first index whose
// running sum reaches thr (n if none; a NaN thr never does), sums[0] = the
// running sum there (the total if none), sums[1] = the running sum at `at`
// (at < n).  Terms non-negative; absorb: also non-increasing.
hipError_t launch_running_cut(const float* terms, uint32_t n, float thr, uint32_t absorb, uint32_t at, uint32_t* cut,
                              float* sums, hipStream_t s);
// n_past += n for each of the n_seq sequences not done
hipError_t launch_add_position(DevState* st, uint32_t n, uint32_t n_seq, hipStream_t s);
// Plain device copy (bytes and both pointers 16-byte aligned).
hipError_t launch_copy(const void* src, void* dst, size_t bytes, hipStream_t s);

// ---- prompt prefill (prefill.hip) ----
// Activation rows -> f16 hi / lo planes [Npad][K] and a power-of-two row
// scale rs[Npad] (optionally RMSNorm first); rows N..Npad-1 are zero.
// Npad >= N, a multiple of 16 (gemm_rows_pad(N) for launch_gemm_mfma, 16 for
// launch_skinny_mfma); K must be a multiple of 32.
uint32_t gemm_rows_pad(uint32_t n);
// err (nullable): ERR_NONFINITE is or-ed in when a row holds a non-finite value.
hipError_t launch_split_rows(const float* x, uint32_t ldx, const float* norm, float eps, uint32_t N, uint32_t Npad,
                             uint32_t K, _Float16* xh, _Float16* xl, float* rs, uint32_t* err, hipStream_t s);

// MFMA product y[n][m] (op)= rs[n] * sum_k W[m][k] * x[n][k] for n < N, m < M,
// x given as the split planes; epilogues as for launch_gemv (SwiGLU uses w3).
// part (nullable): workspace of part_cap floats for K-split partial sums
// (gemm_part_floats(Npad, M) floats lets every short-M product split).
struct GemmArgs {
  const uint8_t* w;
  const uint8_t* w3;
  size_t row_bytes;
  uint32_t M, K;
  const _Float16* xh;
  const _Float16* xl;
  const float* rs;
  uint32_t N;
  float* y;
  uint32_t ldy;
  float* part;
  size_t part_cap;
};
size_t gemm_part_floats(uint32_t n_pad, uint32_t m);
hipError_t launch_gemm_mfma(uint32_t wtype, int epi, const GemmArgs& a, hipStream_t s);

// Skinny MFMA product for 1..16 columns (batched decode): x as split planes
// with 16 rows ([16][K], rows N..15 zero); K a multiple of 256.
struct SkinnyArgs {
  const uint8_t* w;
  const uint8_t* w3;
  size_t row_bytes;
  uint32_t row_base, extra_row;  // logical row -> weight row, as in GemvArgs
  uint32_t M, K;
  const _Float16* xh;
  const _Float16* xl;
  const float* rs;
  uint32_t N;
  float* y;
  uint32_t ldy;
  const uint32_t* done;
};
hipError_t launch_skinny_mfma(uint32_t wtype, int epi, const SkinnyArgs& a, hipStream_t s);

// ---- batched decode products (batched.hip) ----
// Weights in MFMA fragment order: tile (tm, tk) of 16 rows x 32 k is 512
// contiguous halfs, lane l's 8 at l * 8 = W[16 tm + l % 16][32 tk + 8 (l / 16)
// + e]; rows padded to bmm_rows_pad(M) with zeros.  launch_tile_f16 builds it
// from F16 rows [*][K] (logical row r -> row_base + r, the last logical row
// -> extra_row unless NO_ROW).
uint32_t bmm_rows_pad(uint32_t m);
hipError_t launch_tile_f16(const uint16_t* src, uint32_t K, uint32_t M, uint32_t row_base, uint32_t extra_row,
                           uint16_t* dst, hipStream_t s);
// y[n][m] (op)= sum_k W[m][k] xn[n][k] for n < N <= 16, m < M; xn = x, or
// RMSNorm(x) with gain `norm`; epilogues as for launch_gemv.  K % 256 == 0.
// Each wave scales each column by a power of two from its first activations
// (any magnitude keeps ~2^-22 relative accuracy); a non-finite activation,
// or one 2^15 times larger than those, sets ERR_F16_RANGE in *err.
struct BmmArgs {
  const _Float16* wt;
  const _Float16* wt3;   // second matrix for SwiGLU epilogues
  uint32_t M, K;
  const float* x;        // [N][ldx]
  uint32_t ldx, N;
  const float* norm;     // nullable
  float eps;
  float* y;              // [N][ldy]
  uint32_t ldy;
  const uint32_t* done;  // nullable: skip the stores once set
  uint32_t* err;         // nullable
  uint32_t waves;        // 0: bmm_waves(M, K); else 1, 2 or 4
};
uint32_t bmm_waves(uint32_t M, uint32_t K);
hipError_t launch_bmm(int epi, const BmmArgs& a, hipStream_t s);

// Causal GQA attention of N prompt queries at positions *pos_ptr + pos_offset
// + c over the KV cache (their own K/V already appended).
struct PrefillAttnArgs {
  const float* q;          // [N][H hd], QK-normed and rotated
  const float* k_cache;    // [Hkv][max_seq][hd] for this layer
  const float* v_cache;
  float* out;              // [N][H hd]
  const uint32_t* pos_ptr;
  uint32_t pos_offset;
  uint32_t N, H, Hkv, hd, max_seq;
  float scale;
  uint32_t kv_f16;         // 1: the caches hold f16
  uint32_t* err;           // ERR_F16_RANGE when a q, k or v is beyond the f16 range (nullable)
  float* part;             // key-split workspace of part_cap floats (nullable: no split)
  size_t part_cap;
};
hipError_t launch_attention_prefill(const PrefillAttnArgs& a, hipStream_t s);
size_t attn_prefill_part_floats(uint32_t n, uint32_t heads, uint32_t hd);

}  // namespace s2
