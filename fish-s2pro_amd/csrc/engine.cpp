// engine.cpp -- s2hip engine: HBM-resident dual-AR state behind the C ABI.
//
// One engine = one loaded transformer GGUF on one device:
//   * every tensor uploaded once in its GGUF layout (F16 / Q8_0 / Q4_0 rows),
//     RMSNorm gains expanded to f32;
//   * Slow-AR KV cache f32 [slot][layer][kv_head][max_seq][head_dim];
//   * Fast-AR KV cache f32 [slot][layer][kv_head][num_codebooks + 1][head_dim],
//     filled incrementally (9 weight passes per frame instead of the
//     reference's prefix recompute, crates/fish_s2_infer/src/fast_ar.rs:417-424);
//   * a DevState block per slot (positions, frame counter, RNG state, frame
//     codes) so one captured HIP graph replays every frame with no host round
//     trip.  A batch of requests decodes together, one slot each: every frame
//     kernel reads a weight matrix once for all of the batch's columns.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "expf_glibc.h"
#include "gguf.h"
#include "kernels.h"
#include "s2hip.h"

namespace s2 {
namespace {

struct HipFailure : std::runtime_error {
  explicit HipFailure(const std::string& m) : std::runtime_error(m) {}
};

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw HipFailure(std::string(what) + ": " + hipGetErrorString(e));
}
#define HIPC(expr) hip_check((expr), #expr)

// device allocations the dual-AR engines of this process have made
// (s2hip_device_allocations)
std::atomic<uint64_t> g_device_allocs{0};
void count_device_alloc() { g_device_allocs.fetch_add(1, std::memory_order_relaxed); }

[[noreturn]] void fail(const std::string& m) { throw std::runtime_error(m); }

constexpr uint32_t PREFILL_COLS = 4;     // decode-path columns per pass of the GEMV prefill
constexpr uint32_t MAX_SEQS = 16;        // requests per batched generate call
constexpr uint32_t BMM_MAX_K = 10240;    // input width limit of the batched product
constexpr uint32_t ACT_COLS = 2 * MAX_SEQS;  // activation columns (Fast-AR pass 0 has two per request)
constexpr uint32_t PREFILL_CHUNK = 512;  // prompt tokens per MFMA prefill pass
constexpr uint32_t FRAME_BATCH = 4;
constexpr uint32_t ATTN_CHECK_MIN_SEQS = 2;  // batched requests: tail attention chunks check first
constexpr size_t WEIGHT_PAD = 256;  // trailing bytes so block loads never leave a buffer

// Device scratch of the allocation-free sampler entry point
// (s2hip_op_sample_noalloc): the staged logits, then the RNG state, token and
// error words.  One copy per GPU, for the process lifetime; host code uses the
// address hipGetSymbolAddress returns for the current device (the array's name
// is only a host-side stand-in).  Calls that overlap on one GPU race on it.
constexpr size_t NOALLOC_MAX_LOGITS = 8191;  // the device sampler's limit
constexpr size_t NOALLOC_STATE_OFF = 32768;  // after the logits (8191 * 4 B, padded)
constexpr size_t NOALLOC_SCRATCH_BYTES = NOALLOC_STATE_OFF + 256;
static_assert(NOALLOC_MAX_LOGITS * 4 <= NOALLOC_STATE_OFF, "logits overlap the state words");
struct NoallocState {
  uint64_t rng;
  uint32_t token;
  uint32_t err;
};
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

float f16_to_f32(uint16_t h) {
  const uint32_t sign = uint32_t(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  uint32_t bits;
  if (e == 0) {
    const float v = std::ldexp(float(m), -24);
    return sign ? -v : v;
  }
  bits = e == 0x1f ? (sign | 0x7f800000u | (m << 13)) : (sign | ((e + 112u) << 23) | (m << 13));
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

struct DevLin {
  uint8_t* w = nullptr;
  uint32_t type = 0;
  uint32_t in = 0, out = 0;
  size_t row_bytes = 0;
  uint64_t bytes = 0;
  // F16 weights in MFMA fragment order for the batched product (built on
  // first use); its rows are the logical rows (any row mapping baked in)
  _Float16* wt = nullptr;
  // Q8_0 / Q4_0 rows repacked for the one-column decode GEMV (built on
  // first use): 16-byte-aligned block values and an f16 scale plane
  uint8_t* qp = nullptr;
  uint16_t* qs = nullptr;
};

struct SlowLayer {
  float *attn_norm = nullptr, *ffn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
  DevLin wqkv, wo, w1, w2, w3;
};

struct FastLayer {
  float *attn_norm = nullptr, *ffn_norm = nullptr;
  DevLin wqkv, wo, w1, w2, w3;
};

std::string lname(const char* pre, uint32_t l, const char* suf) {
  return std::string(pre) + "." + std::to_string(l) + "." + suf;
}

}  // namespace

class Engine {
 public:
  explicit Engine(const s2hip_config& cfg);
  ~Engine();

  s2hip_spec spec{};
  int device = 0;

  void select() { HIPC(hipSetDevice(device)); }
  void reset(uint32_t slot = 0);
  void eval(const int32_t* flat, size_t n_tok, float* hidden_out, float* logits_out, uint32_t slot = 0);
  void fast_logits(const float* hidden, const uint32_t* prefix, size_t plen, float* logits);
  void fast_codebooks(const float* hidden, uint32_t sem, const s2hip_sampler& smp, uint64_t* rng, uint32_t* codes);
  void generate(uint32_t nseq, const int32_t* const* prompts, const size_t* cols, const s2hip_gen_params& p,
                uint64_t* rngs, int32_t* const* codes, uint32_t* n_frames, s2hip_gen_stats* stats);
  uint32_t n_past_host[16] = {};  // per KV slot (MAX_SEQS)
  s2hip_slow_profile slow_prof{};  // last generate call (S2HIP_FLAG_PROFILE)

  // op level
  void op_linear(const void* w, uint32_t type, size_t in, size_t out, const float* x, size_t ncol, float* y);
  void op_rms_norm(const float* x, const float* w, size_t n, size_t ncol, float eps, float* y);
  void op_dequant(const void* w, uint32_t type, size_t in, size_t rows, float* out);
  void op_qk_rope(const float* qkv, uint32_t H, uint32_t Hkv, uint32_t hd, uint32_t pos, float base,
                  const float* qn, const float* kn, float eps, float* q, float* k, float* v);
  void op_attention(const float* q, const float* k, const float* v, uint32_t H, uint32_t Hkv, uint32_t hd,
                    uint32_t T, float scale, float* out);
  void op_swiglu(const float* g, const float* u, size_t n, int fast, float* out);
  void op_running_sums(const float* terms, size_t n, float* prefix, float* total);
  void op_running_cut(const float* terms, size_t n, float thr, bool absorb, size_t at, size_t* cut, float* sum,
                      float* at_sum);
  void op_expf(const float* x, size_t n, float* y);
  void op_embed(const int32_t* flat, size_t n_tok, float* out);
  void op_sample(const float* logits, size_t n, const s2hip_sampler& smp, int64_t always, uint64_t* rng,
                 uint32_t* tok);
  void op_sample_noalloc(const float* logits, size_t n, const s2hip_sampler& smp, int64_t always, uint64_t* rng,
                         uint32_t* tok);
  void time_kernel(const std::string& name, uint32_t reps, double* avg_us, double* bytes);

 private:
  template <class T>
  T* dalloc(size_t count, size_t pad = 0) {
    void* p = nullptr;
    HIPC(hipMalloc(&p, count * sizeof(T) + pad));
    count_device_alloc();
    allocs_.push_back(p);
    return static_cast<T*>(p);
  }
  void upload(void* dst, const void* src, size_t bytes);
  DevLin load_lin(const GgufFile& g, const std::string& name, uint64_t in, uint64_t out);
  float* load_norm(const GgufFile& g, const std::string& name, uint64_t n);
  uint16_t* load_f16_table(const GgufFile& g, const std::string& name, uint64_t dim, uint64_t min_rows,
                           uint64_t* rows_out);
  void build_rope(float2* dst, uint32_t positions, uint32_t hd, float base);

  void gemv(const DevLin& L, const DevLin* L3, int epi, uint32_t ncol, const float* x, uint32_t ldx,
            const float* norm, float eps, float* y, uint32_t ldy, uint32_t row_base, uint32_t extra_row, uint32_t out_rows,
            const uint32_t* done, const GreedyFold* fold = nullptr);
  // linear over ncol columns: GEMV kernels for 1-2, skinny MFMA for more
  // (bmm_waves: waves per tile when the batched product serves it, 0 = its default)
  void lin(const DevLin& L, const DevLin* L3, int epi, uint32_t ncol, const float* x, uint32_t ldx,
           const float* norm, float eps, float* y, uint32_t ldy, uint32_t row_base, uint32_t extra_row,
           uint32_t out_rows, const uint32_t* done, uint32_t bmm_waves = 0, const GreedyFold* fold = nullptr);
  // ncol = nseq * cps columns of slots seq0 .. seq0 + nseq - 1 in h_
  // advance: add cps to each unfinished slot's n_past afterwards (the frame
  // loop leaves it to its sampler instead)
  void enqueue_slow_layers(uint32_t nseq, uint32_t cps, uint32_t seq0, const uint32_t* done, bool advance = true);
  void enqueue_head(uint32_t ncol, float* hn, float* logits, bool full, const uint32_t* done);
  // fold (nullable): the first linear takes its input from the greedy sample
  // code (nullable): the single column is the embedding of *code (the first
  // linear's output comes from fast_table_)
  void enqueue_fast_layers(uint32_t nseq, uint32_t cps, uint32_t p0, const uint32_t* done,
                           const GreedyFold* fold = nullptr, const uint32_t* code = nullptr);
  void enqueue_fast_frame(const SamplerCfg& cfg, uint32_t nseq, const uint32_t* done);
  bool fold_greedy(const SamplerCfg& cfg, uint32_t nseq) const;
  void enqueue_frame(const SamplerCfg& cfg, uint32_t nseq, size_t codes_stride);
  void enqueue_prefill(const int32_t* prompt_dev, size_t n_tok, uint32_t seq);
  void enqueue_prefill_gemv(const int32_t* prompt_dev, size_t n_tok, uint32_t seq);
  void ensure_slots(uint32_t n);
  void ensure_tiled();
  void repack(DevLin& L);
  void tile(DevLin& L, uint32_t rows, uint32_t row_base, uint32_t extra_row);
  void bmm(const DevLin& L, const DevLin* L3, int epi, uint32_t ncol, const float* x, uint32_t ldx, const float* norm,
           float eps, float* y, uint32_t ldy, const uint32_t* done, uint32_t* err, uint32_t waves = 0);
  void validate_prompt(const int32_t* prompt, size_t cols);
  void validate_tokens(const int32_t* flat, size_t n_tok);
  void mm(const DevLin& L, const DevLin* L3, int epi, const float* x, uint32_t ldx, const float* norm, float eps,
          uint32_t n, uint32_t npad, float* y, uint32_t ldy);
  // batched columns (3..16): split planes + skinny MFMA product
  void mm_skinny(const DevLin& L, const DevLin* L3, int epi, const float* x, uint32_t ldx, const float* norm,
                 float eps, uint32_t n, float* y, uint32_t ldy, uint32_t row_base, uint32_t extra_row,
                 uint32_t out_rows, const uint32_t* done);
  bool uses_bmm(const DevLin& L, const DevLin* L3, uint32_t ncol) const;
  L2Warm warm_for(const DevLin& L, const DevLin* L3, uint32_t ncol, bool norm, uint32_t pct_begin,
                  uint32_t pct_end) const;
  void ensure_prompt(size_t n_int);
  void ensure_codes(size_t n_int);
  void check_state_err(uint32_t nseq = 1);

  hipStream_t stream_ = nullptr;
  std::vector<void*> allocs_;
  uint8_t* scratch_dev_ = nullptr;  // this device's `scratch` (hipGetSymbolAddress at set-up)
  // S2HIP_FLAG_PROFILE: events between the Slow-AR kernel groups of one frame
  // (booked after each frame into slow_prof)
  bool profiling_ = false;
  std::vector<hipEvent_t> prof_ev_;
  std::vector<int> prof_kind_;  // field the interval that ends at event i goes to (-1: none)
  void prof_mark(int kind);
  void prof_book(uint32_t nseq);
  uint8_t* staging_[2] = {nullptr, nullptr};
  hipEvent_t staging_ev_[2] = {nullptr, nullptr};
  static constexpr size_t STAGING = 64u << 20;
  uint32_t im_end_ = 0;
  uint32_t flags_ = 0;
  uint32_t kv_f16_ = 0;   // Slow-AR KV cache stored as f16 (S2HIP_FLAG_KV_F16)
  // element `elems` of a Slow-AR cache buffer (f32 or f16 elements)
  float* kvp(float* base, size_t elems) const {
    return reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(base) + elems * (kv_f16_ ? 2 : 4));
  }

  // weights
  uint16_t *emb_ = nullptr, *cb_emb_ = nullptr, *fast_emb_ = nullptr;
  uint64_t cb_rows_ = 0;
  float *norm_ = nullptr, *fast_norm_ = nullptr;
  DevLin head_full_, fast_out_;
  DevLin head_cand_;  // the candidate rows of the head (tiled copy only)
  bool tiled_ = false;
  uint32_t bmm_min_cols_ = 2;  // columns from which F16 linears use the batched product
  // Set while a call is re-run after ERR_F16_RANGE: every multi-column linear
  // then takes the per-column paths (two-column GEMV, or the skinny product
  // over rows split with a whole-row scale), which have no per-wave range.
  bool bmm_off_ = false;
  bool any_f16_range(uint32_t nseq) const { return any_err(nseq, ERR_F16_RANGE); }
  bool any_err(uint32_t nseq, uint32_t bits) const {
    for (uint32_t b = 0; b < nseq; ++b)
      if (st_host_[b].err & bits) return true;
    return false;
  }
  // the Fast-AR greedy samples run as sampler kernels (after a tie at a
  // folded sample's max)
  bool fold_off_ = false;
  bool fold_env_off_ = false;  // S2HIP_NO_GREEDY_FOLD: always the sampler kernel
  // The Fast-AR's first wqkv for every code: row c = wqkv(RMSNorm(fast_emb[c]))
  // as the one-column GEMV computes it.  A sub-step whose input is one code's
  // embedding (one request, after the first) then reads its q / k / v from
  // the table instead of running the linear.  S2HIP_NO_FAST_TABLE: off.
  float* fast_table_ = nullptr;
  bool fast_table_off_ = false;
  void ensure_fast_table();
  // L2 warming of the output projection by decode attention
  uint32_t warm_blocks_ = 256;            // warming blocks per kernel (0: off)
  float* gemv_xn_ = nullptr;              // normalised-x output of the next gemv() launch (consumed there)
  uint32_t warm_depth_ = 4;               // 16-byte loads per thread in flight
  // % of the Slow-AR wo rows warmed by the attention partials: none by default
  // (default decode 309.0-309.4 frames/s against 307.4-307.9 with all of them
  // and 305.6-306.1 with 30-60 %; the Fast-AR warming pays, 1 % on the line)
  uint32_t warm_slow_ = 0;
  uint32_t warm_fast_ = 100;              // % of the Fast-AR rows warmed (one attention kernel)
  uint32_t warm_step_ = 0;                // % of the first linear's rows warmed by embedding / sampler (no measured gain: off)
  size_t warm_bytes_ = size_t(24) << 20;  // at most this many weight bytes warmed (8 L2s of 4 MiB)
  std::vector<SlowLayer> slow_;
  std::vector<FastLayer> fast_;
  uint32_t* head_rows_ = nullptr;  // vocabulary id of each candidate logit
  uint32_t head_extra_ = NO_ROW;
  uint32_t n_cand_ = 0;

  // activations
  float *h_ = nullptr, *qkv_ = nullptr, *q_ = nullptr, *att_ = nullptr, *part_ = nullptr, *act_ = nullptr;
  float *hn_ = nullptr, *logits_c_ = nullptr, *logits_full_ = nullptr;
  float *kc_ = nullptr, *vc_ = nullptr;
  size_t slot_kv_ = 0, fslot_kv_ = 0;  // floats per slot in the slow / fast caches
  uint32_t kv_slots_ = 0;
  uint64_t kv_gen_ = 0;  // bumped whenever the caches are reallocated
  float2 *rope_slow_ = nullptr, *rope_fast_ = nullptr;
  uint32_t attn_chunks_ = 1;
  uint32_t attn_mode_ = ATTN_SPLIT;
  bool prefill_gemv_ = false;
  uint32_t* counters_ = nullptr;
  // prompt prefill (MFMA path): chunk activations and the split planes
  float *ph_ = nullptr, *pqkv_ = nullptr, *pq_ = nullptr, *patt_ = nullptr, *pact_ = nullptr, *prs_ = nullptr;
  _Float16 *pxh_ = nullptr, *pxl_ = nullptr;
  float* ppart_ = nullptr;  // K-split partial sums of the prefill products
  size_t ppart_cap_ = 0;
  float *fh_ = nullptr, *fqkv_ = nullptr, *fq_ = nullptr, *fatt_ = nullptr, *fpart_ = nullptr, *fact_ = nullptr;
  float *flogits_ = nullptr, *fkc_ = nullptr, *fvc_ = nullptr;
  uint32_t fctx_ = 11;

  DevState* st_ = nullptr;        // [MAX_SEQS]
  DevState* st_host_ = nullptr;   // pinned [MAX_SEQS]
  BatchState* batch_ = nullptr;
  uint32_t* done_host_ = nullptr;  // pinned [2]
  int32_t* codes_dev_ = nullptr;
  size_t codes_cap_ = 0;
  int32_t* prompt_dev_ = nullptr;
  size_t prompt_cap_ = 0;

  hipGraphExec_t graph_exec_ = nullptr;
  hipGraph_t graph_ = nullptr;
  // what the captured frame depends on
  SamplerCfg graph_cfg_{};
  int32_t* graph_codes_ = nullptr;
  size_t graph_codes_stride_ = 0;
  uint32_t graph_nseq_ = 0;
  uint64_t graph_kv_gen_ = 0;
  bool graph_bmm_off_ = false;
  bool graph_fold_off_ = false;
  uint32_t graph_check_from_ = 0;
  // Slow-AR decode attention of batched requests: chunks from here on check
  // the position before their K/V tile (0: every chunk loads it first).  Set
  // by each generate call from its prompts; it decides only which blocks wait
  // for the position, never a result.
  uint32_t attn_check_from_ = 0;
};

Engine::Engine(const s2hip_config& cfg) {
  if (!cfg.gguf_path) fail("gguf_path is NULL");
  if (cfg.max_seq_len == 0) fail("max_seq_len must be non-zero");
  if (cfg.max_seq_len > 32u * ATTN_MAX_CHUNKS)
    fail("max_seq_len above " + std::to_string(32u * ATTN_MAX_CHUNKS) + " is not supported");
  device = cfg.device;
  flags_ = cfg.flags;
  kv_f16_ = (cfg.flags & S2HIP_FLAG_KV_F16) ? 1u : 0u;
  im_end_ = cfg.im_end_id;
  // the file is parsed and validated (host only) before any device resource is taken
  GgufFile g;
  g.open(cfg.gguf_path);
  int ndev = 0;
  HIPC(hipGetDeviceCount(&ndev));
  if (device < 0 || device >= ndev) fail("HIP device " + std::to_string(device) + " not present");
  select();
  HIPC(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
  // this device's copy of the allocation-free entry point's scratch
  HIPC(hipGetSymbolAddress(reinterpret_cast<void**>(&scratch_dev_), HIP_SYMBOL(scratch)));
  for (int i = 0; i < 2; ++i) {
    HIPC(hipHostMalloc(reinterpret_cast<void**>(&staging_[i]), STAGING, hipHostMallocDefault));
    HIPC(hipEventCreateWithFlags(&staging_ev_[i], hipEventDisableTiming));
  }

  // DualArGraphSpec::from_gguf (crates/fish_s2_infer/src/registry.rs:45-214), shape-generic.
  if (g.str("general.architecture") != "fish-speech")
    fail("expected fish-speech transformer GGUF, got " + g.str("general.architecture"));
  s2hip_spec& s = spec;
  s.slow_layers = g.u32("fish-speech.block_count");
  s.dim = g.u32("fish-speech.embedding_length");
  s.ffn = g.u32("fish-speech.feed_forward_length");
  s.heads = g.u32("fish-speech.attention.head_count");
  s.kv_heads = g.u32("fish-speech.attention.head_count_kv");
  s.rope_base = g.f32("fish-speech.rope.freq_base");
  s.eps = g.f32("fish-speech.attention.layer_norm_rms_epsilon");
  s.slow_qk_norm = g.flag("fish_speech.attention_qk_norm") ? 1u : 0u;
  s.head_dim = s.slow_qk_norm ? uint32_t(g.tensor("layers.0.attention.q_norm.weight").elements())
                              : s.dim / std::max(1u, s.heads);
  s.fast_layers = g.u32("fish_speech.fast_block_count");
  const uint32_t fast_dim = g.u32("fish_speech.fast_embedding_length");
  s.fast_ffn = g.u32("fish_speech.fast_feed_forward_length");
  s.fast_heads = g.u32("fish_speech.fast_head_count");
  s.fast_kv_heads = g.u32("fish_speech.fast_head_count_kv");
  s.fast_head_dim = g.u32("fish_speech.fast_head_dim");
  s.fast_rope_base = g.f32("fish_speech.fast_rope_freq_base");
  s.fast_eps = g.f32("fish_speech.fast_layer_norm_rms_eps");
  s.codebook_size = g.u32("fish_speech.codebook_size");
  s.num_codebooks = g.u32("fish_speech.num_codebooks");
  s.semantic_begin = g.u32("fish_speech.semantic_begin_id");
  s.semantic_end = g.u32("fish_speech.semantic_end_id");
  s.scale_codebook_embeddings = g.flag("fish_speech.scale_codebook_embeddings") ? 1u : 0u;
  if (g.flag("fish_speech.fast_project_in")) fail("fast_project_in is not implemented");  // fast_ar.rs:366-370
  if (fast_dim != s.dim) fail("fast embedding_length must equal the slow embedding_length");
  if (s.kv_heads == 0 || s.heads % s.kv_heads) fail("invalid GQA head split");
  if (s.fast_kv_heads == 0 || s.fast_heads % s.fast_kv_heads) fail("invalid fast GQA head split");
  if ((s.head_dim != 64 && s.head_dim != 128) || (s.fast_head_dim != 64 && s.fast_head_dim != 128))
    fail("head_dim must be 64 or 128");
  if (s.heads / s.kv_heads > 4 || s.fast_heads / s.fast_kv_heads > 4)
    fail("at most 4 query heads per kv head are supported");
  if (s.num_codebooks == 0 || s.num_codebooks > 16) fail("num_codebooks must be in 1..16");
  if (s.semantic_end < s.semantic_begin) fail("invalid semantic id range");
  if (s.dim % 8) fail("embedding_length must be a multiple of 8");
  s.max_seq_len = cfg.max_seq_len;

  uint64_t vocab_rows = 0;
  emb_ = load_f16_table(g, "embeddings.weight", s.dim, 1, &vocab_rows);
  s.vocab = uint32_t(vocab_rows);
  if (s.semantic_end >= s.vocab) fail("semantic ids exceed the vocabulary");
  cb_emb_ = load_f16_table(g, "codebook_embeddings.weight", s.dim, uint64_t(s.num_codebooks) * s.codebook_size,
                           &cb_rows_);
  uint64_t fast_rows = 0;
  fast_emb_ = load_f16_table(g, "fast_embeddings.weight", s.dim, s.codebook_size, &fast_rows);
  norm_ = load_norm(g, "norm.weight", s.dim);
  fast_norm_ = load_norm(g, "fast_norm.weight", s.dim);
  fast_out_ = load_lin(g, "fast_output.weight", s.dim, s.codebook_size);
  head_full_.w = reinterpret_cast<uint8_t*>(emb_);
  head_full_.type = W_F16;
  head_full_.in = s.dim;
  head_full_.out = s.vocab;
  head_full_.row_bytes = size_t(s.dim) * 2;
  head_full_.bytes = uint64_t(s.vocab) * s.dim * 2;

  const uint64_t q = uint64_t(s.heads) * s.head_dim, kv = uint64_t(s.kv_heads) * s.head_dim;
  slow_.resize(s.slow_layers);
  for (uint32_t l = 0; l < s.slow_layers; ++l) {
    SlowLayer& L = slow_[l];
    L.attn_norm = load_norm(g, lname("layers", l, "attention_norm.weight"), s.dim);
    L.ffn_norm = load_norm(g, lname("layers", l, "ffn_norm.weight"), s.dim);
    if (s.slow_qk_norm) {
      L.q_norm = load_norm(g, lname("layers", l, "attention.q_norm.weight"), s.head_dim);
      L.k_norm = load_norm(g, lname("layers", l, "attention.k_norm.weight"), s.head_dim);
    }
    L.wqkv = load_lin(g, lname("layers", l, "attention.wqkv.weight"), s.dim, q + 2 * kv);
    L.wo = load_lin(g, lname("layers", l, "attention.wo.weight"), q, s.dim);
    L.w1 = load_lin(g, lname("layers", l, "feed_forward.w1.weight"), s.dim, s.ffn);
    L.w2 = load_lin(g, lname("layers", l, "feed_forward.w2.weight"), s.ffn, s.dim);
    L.w3 = load_lin(g, lname("layers", l, "feed_forward.w3.weight"), s.dim, s.ffn);
  }
  s.linear_type = s.slow_layers ? slow_[0].wqkv.type : uint32_t(W_F16);
  const uint64_t fq = uint64_t(s.fast_heads) * s.fast_head_dim, fkv = uint64_t(s.fast_kv_heads) * s.fast_head_dim;
  fast_.resize(s.fast_layers);
  for (uint32_t l = 0; l < s.fast_layers; ++l) {
    FastLayer& L = fast_[l];
    L.attn_norm = load_norm(g, lname("fast_layers", l, "attention_norm.weight"), s.dim);
    L.ffn_norm = load_norm(g, lname("fast_layers", l, "ffn_norm.weight"), s.dim);
    L.wqkv = load_lin(g, lname("fast_layers", l, "attention.wqkv.weight"), s.dim, fq + 2 * fkv);
    L.wo = load_lin(g, lname("fast_layers", l, "attention.wo.weight"), fq, s.dim);
    L.w1 = load_lin(g, lname("fast_layers", l, "feed_forward.w1.weight"), s.dim, s.fast_ffn);
    L.w2 = load_lin(g, lname("fast_layers", l, "feed_forward.w2.weight"), s.fast_ffn, s.dim);
    L.w3 = load_lin(g, lname("fast_layers", l, "feed_forward.w3.weight"), s.dim, s.fast_ffn);
  }
  HIPC(hipStreamSynchronize(stream_));
  for (int i = 0; i < 2; ++i) {
    HIPC(hipHostFree(staging_[i]));
    staging_[i] = nullptr;
  }

  // candidate rows of the output head: semantic ids + im_end, ascending
  // (semantic ids, then im_end when it lies outside them: the sampler orders
  // candidates by value and id, not by position)
  std::vector<uint32_t> rows;
  for (uint32_t id = s.semantic_begin; id <= s.semantic_end; ++id) rows.push_back(id);
  if (im_end_ < s.vocab && (im_end_ < s.semantic_begin || im_end_ > s.semantic_end)) {
    rows.push_back(im_end_);
    head_extra_ = im_end_;
  }
  n_cand_ = uint32_t(rows.size());
  if (n_cand_ > 8191) fail("too many sampling candidates");
  head_cand_ = head_full_;
  head_cand_.out = n_cand_;
  head_rows_ = dalloc<uint32_t>(rows.size());
  HIPC(hipMemcpy(head_rows_, rows.data(), rows.size() * 4, hipMemcpyHostToDevice));

  // activations: Slow-AR decode columns for a batch of MAX_SEQS requests,
  // Fast-AR columns for twice that (two per request in the first pass of a
  // frame)
  static_assert(PREFILL_COLS <= MAX_SEQS, "GEMV prefill columns");
  const uint32_t NC = MAX_SEQS;
  const uint64_t qkv_w = q + 2 * kv;
  // two attention kernels per layer (partials, then merge) by default; with
  // S2HIP_ATTN_FUSED=1 one kernel whose last block per kv head merges (its
  // store-wait + counter + reload chain measures slower than the kernel
  // boundary it replaces: 18.7 vs 13.2 us at T = 384 on the S2-Pro shape)
  attn_mode_ = getenv("S2HIP_ATTN_FUSED") ? ATTN_FUSED : ATTN_SPLIT;
  fold_env_off_ = getenv("S2HIP_NO_GREEDY_FOLD") != nullptr;
  fast_table_off_ = getenv("S2HIP_NO_FAST_TABLE") != nullptr;
  prefill_gemv_ = getenv("S2HIP_PREFILL_GEMV") != nullptr;
  attn_chunks_ = attention_chunks(s.max_seq_len, attn_mode_);
  // S2HIP_BMM_MIN_COLS=n: F16 linears over >= n columns use the batched MFMA
  // product (0 disables it)
  if (const char* v = getenv("S2HIP_BMM_MIN_COLS")) bmm_min_cols_ = uint32_t(strtoul(v, nullptr, 10));
  // S2HIP_L2_WARM=blocks[,depth[,slow%[,fast%[,step%]]]]: the warming blocks
  // that decode attention, the step embedding and the Fast-AR sampler carry
  // to read the next linear's rows into L2 (blocks rounded down to a
  // multiple of 8; 0: off)
  if (const char* v = getenv("S2HIP_L2_WARM")) {
    unsigned b = 0, d = warm_depth_, sp = warm_slow_, fp = warm_fast_, ep = warm_step_;
    const int n = sscanf(v, "%u,%u,%u,%u,%u", &b, &d, &sp, &fp, &ep);
    if (n >= 1) warm_blocks_ = b & ~7u;
    if (n >= 2) warm_depth_ = d;
    if (n >= 3) warm_slow_ = std::min(sp, 100u);
    if (n >= 4) warm_fast_ = std::min(fp, 100u);
    if (n >= 5) warm_step_ = std::min(ep, 100u);
  }
  h_ = dalloc<float>(size_t(NC) * s.dim);
  qkv_ = dalloc<float>(size_t(NC) * qkv_w);
  q_ = dalloc<float>(size_t(NC) * q);
  att_ = dalloc<float>(size_t(NC) * q);
  part_ = dalloc<float>(size_t(NC) * s.heads * attn_chunks_ * (s.head_dim + 2));
  counters_ = dalloc<uint32_t>(size_t(ACT_COLS) * std::max(s.kv_heads, s.fast_kv_heads));
  HIPC(hipMemset(counters_, 0, size_t(ACT_COLS) * std::max(s.kv_heads, s.fast_kv_heads) * 4));
  act_ = dalloc<float>(size_t(NC) * s.ffn);
  {
    const size_t CH = PREFILL_CHUNK, CHP = gemm_rows_pad(PREFILL_CHUNK);
    const size_t kmax = std::max<size_t>({s.dim, q, s.ffn});
    ph_ = dalloc<float>(CH * s.dim);
    pqkv_ = dalloc<float>(CH * qkv_w);
    pq_ = dalloc<float>(CH * q);
    patt_ = dalloc<float>(CH * q);
    pact_ = dalloc<float>(CH * s.ffn);
    prs_ = dalloc<float>(CHP);
    pxh_ = dalloc<_Float16>(CHP * kmax);
    pxl_ = dalloc<_Float16>(CHP * kmax);
    ppart_cap_ = std::max(gemm_part_floats(uint32_t(CHP), std::max<uint32_t>(qkv_w, s.dim)),
                          attn_prefill_part_floats(uint32_t(CH), s.heads, s.head_dim));
    ppart_ = dalloc<float>(ppart_cap_);
    if (s.dim % 32 || q % 32 || s.ffn % 32) fail("prefill needs embedding, attention and FFN widths divisible by 32");
  }
  hn_ = dalloc<float>(size_t(MAX_SEQS) * s.dim);
  logits_c_ = dalloc<float>(size_t(MAX_SEQS) * n_cand_);
  logits_full_ = dalloc<float>(s.vocab);
  fctx_ = s.num_codebooks + 1;
  slot_kv_ = size_t(s.slow_layers) * kv * s.max_seq_len;
  fslot_kv_ = size_t(s.fast_layers) * fkv * fctx_;
  rope_slow_ = dalloc<float2>(size_t(s.max_seq_len) * (s.head_dim / 2));
  rope_fast_ = dalloc<float2>(size_t(fctx_) * (s.fast_head_dim / 2));
  build_rope(rope_slow_, s.max_seq_len, s.head_dim, s.rope_base);
  build_rope(rope_fast_, fctx_, s.fast_head_dim, s.fast_rope_base);
  const uint32_t FC = ACT_COLS;
  fh_ = dalloc<float>(size_t(FC) * s.dim);
  fqkv_ = dalloc<float>(size_t(FC) * (fq + 2 * fkv));
  fq_ = dalloc<float>(size_t(FC) * fq);
  fatt_ = dalloc<float>(size_t(FC) * fq);
  fpart_ = dalloc<float>(size_t(FC) * s.fast_heads * attention_chunks(fctx_, attn_mode_) * (s.fast_head_dim + 2));
  fact_ = dalloc<float>(size_t(FC) * s.fast_ffn);
  flogits_ = dalloc<float>(size_t(MAX_SEQS) * s.codebook_size);
  ensure_slots(1);
  static_assert(sizeof(DevState) % 4 == 0, "DevState words");
  st_ = dalloc<DevState>(MAX_SEQS);
  HIPC(hipMemset(st_, 0, MAX_SEQS * sizeof(DevState)));
  batch_ = dalloc<BatchState>(1);
  HIPC(hipMemset(batch_, 0, sizeof(BatchState)));
  HIPC(hipHostMalloc(reinterpret_cast<void**>(&st_host_), MAX_SEQS * sizeof(DevState), hipHostMallocDefault));
  HIPC(hipHostMalloc(reinterpret_cast<void**>(&done_host_), 2 * sizeof(uint32_t), hipHostMallocDefault));
  s.weight_bytes = 0;
  for (auto& L : slow_) s.weight_bytes += L.wqkv.bytes + L.wo.bytes + L.w1.bytes + L.w2.bytes + L.w3.bytes;
  for (auto& L : fast_) s.weight_bytes += L.wqkv.bytes + L.wo.bytes + L.w1.bytes + L.w2.bytes + L.w3.bytes;
  s.weight_bytes += head_full_.bytes + cb_rows_ * s.dim * 2 + fast_rows * s.dim * 2 + fast_out_.bytes;
  HIPC(hipDeviceSynchronize());
}

Engine::~Engine() {
  if (device >= 0) (void)hipSetDevice(device);
  if (stream_) (void)hipStreamSynchronize(stream_);
  for (hipEvent_t e : prof_ev_) (void)hipEventDestroy(e);
  if (graph_exec_) (void)hipGraphExecDestroy(graph_exec_);
  if (graph_) (void)hipGraphDestroy(graph_);
  for (void* p : allocs_) (void)hipFree(p);
  for (int i = 0; i < 2; ++i) {
    if (staging_[i]) (void)hipHostFree(staging_[i]);
    if (staging_ev_[i]) (void)hipEventDestroy(staging_ev_[i]);
  }
  if (st_host_) (void)hipHostFree(st_host_);
  if (done_host_) (void)hipHostFree(done_host_);
  if (stream_) (void)hipStreamDestroy(stream_);
}

// Chunked pinned double-buffered upload from the mapped file.
void Engine::upload(void* dst, const void* src, size_t bytes) {
  static int slot = 0;
  const uint8_t* s8 = static_cast<const uint8_t*>(src);
  uint8_t* d8 = static_cast<uint8_t*>(dst);
  for (size_t off = 0; off < bytes; off += STAGING) {
    const size_t n = std::min(STAGING, bytes - off);
    HIPC(hipEventSynchronize(staging_ev_[slot]));
    memcpy(staging_[slot], s8 + off, n);
    HIPC(hipMemcpyAsync(d8 + off, staging_[slot], n, hipMemcpyHostToDevice, stream_));
    HIPC(hipEventRecord(staging_ev_[slot], stream_));
    slot ^= 1;
  }
}

DevLin Engine::load_lin(const GgufFile& g, const std::string& name, uint64_t in, uint64_t out) {
  const GgufTensor& t = g.tensor(name);
  if (t.dims.size() != 2 || t.dims[0] != in || t.dims[1] != out)
    fail(name + " dimensions mismatch: expected [" + std::to_string(in) + ", " + std::to_string(out) + "]");
  if (t.type != W_F16 && t.type != W_Q8_0 && t.type != W_Q4_0)
    fail(name + ": unsupported linear weight type " + std::to_string(t.type));
  DevLin L;
  L.type = t.type;
  L.in = uint32_t(in);
  L.out = uint32_t(out);
  L.row_bytes = size_t(ggml_row_bytes(t.type, in));
  L.bytes = t.bytes;
  L.w = dalloc<uint8_t>(t.bytes, WEIGHT_PAD);
  HIPC(hipMemsetAsync(L.w + t.bytes, 0, WEIGHT_PAD, stream_));
  upload(L.w, t.data, t.bytes);
  return L;
}

float* Engine::load_norm(const GgufFile& g, const std::string& name, uint64_t n) {
  const GgufTensor& t = g.tensor(name);
  if (t.elements() != n) fail(name + ": expected " + std::to_string(n) + " elements");
  std::vector<float> v(n);
  if (t.type == 1) {
    for (uint64_t i = 0; i < n; ++i) {
      uint16_t b;
      memcpy(&b, t.data + 2 * i, 2);
      v[i] = f16_to_f32(b);
    }
  } else if (t.type == 0) {
    memcpy(v.data(), t.data, n * 4);
  } else {
    fail(name + ": norm weights must be F16 or F32");
  }
  float* d = dalloc<float>(n);
  HIPC(hipMemcpy(d, v.data(), n * 4, hipMemcpyHostToDevice));
  return d;
}

uint16_t* Engine::load_f16_table(const GgufFile& g, const std::string& name, uint64_t dim, uint64_t min_rows,
                                 uint64_t* rows_out) {
  const GgufTensor& t = g.tensor(name);
  if (t.dims.size() != 2 || t.dims[0] != dim || t.type != 1 || t.dims[1] < min_rows)
    fail(name + ": expected an F16 [" + std::to_string(dim) + ", >=" + std::to_string(min_rows) + "] table");
  *rows_out = t.dims[1];
  uint16_t* d = dalloc<uint16_t>(t.bytes / 2, WEIGHT_PAD);
  upload(d, t.data, t.bytes);
  return d;
}

// apply_rope_normal's angles (crates/fish_s2_infer/src/attention.rs:195-203),
// evaluated once on the host with the same libm calls in f32.
void Engine::build_rope(float2* dst, uint32_t positions, uint32_t hd, float base) {
  std::vector<float2> t(size_t(positions) * (hd / 2));
  for (uint32_t pos = 0; pos < positions; ++pos) {
    for (uint32_t pair = 0; pair < hd; pair += 2) {
      const float theta = float(pos) / powf(base, float(pair) / float(hd));
      t[size_t(pos) * (hd / 2) + pair / 2] = make_float2(cosf(theta), sinf(theta));
    }
  }
  HIPC(hipMemcpy(dst, t.data(), t.size() * sizeof(float2), hipMemcpyHostToDevice));
}

void Engine::gemv(const DevLin& L, const DevLin* L3, int epi, uint32_t ncol, const float* x, uint32_t ldx,
                  const float* norm, float eps, float* y, uint32_t ldy, uint32_t row_base, uint32_t extra_row, uint32_t out_rows,
                  const uint32_t* done, const GreedyFold* fold) {
  if (fold && ncol != 1) fail("the greedy fold feeds one column");
  uint32_t c = 0;
  while (c < ncol) {
    uint32_t w = 8;
    while (w > 1 && (w > ncol - c || size_t(w) * L.in * 4 > 150 * 1024)) w >>= 1;
    GemvArgs a{};
    a.w = L.w;
    a.w3 = L3 ? L3->w : nullptr;
    a.row_bytes = L.row_bytes;
    a.row_base = row_base;
    a.extra_row = extra_row;
    a.in = L.in;
    a.out = out_rows;
    a.x = x + size_t(c) * ldx;
    a.ldx = ldx;
    a.norm = norm;
    a.eps = eps;
    a.y = y + size_t(c) * ldy;
    a.ldy = ldy;
    a.done = done;
    a.qp = L.qp;
    a.qs = L.qs;
    a.qp3 = L3 ? L3->qp : nullptr;
    a.qs3 = L3 ? L3->qs : nullptr;
    if (fold) a.fold = *fold;
    if (gemv_xn_) a.xn_out = gemv_xn_ + size_t(c) * ldx;
    HIPC(launch_gemv(L.type, epi, int(w), a, stream_));
    c += w;
  }
}

void Engine::bmm(const DevLin& L, const DevLin* L3, int epi, uint32_t ncol, const float* x, uint32_t ldx,
                 const float* norm, float eps, float* y, uint32_t ldy, const uint32_t* done, uint32_t* err,
                 uint32_t waves) {
  for (uint32_t c = 0; c < ncol; c += 16) {
    BmmArgs b{};
    b.wt = L.wt;
    b.wt3 = L3 ? L3->wt : nullptr;
    b.M = L.out;
    b.K = L.in;
    b.x = x + size_t(c) * ldx;
    b.ldx = ldx;
    b.N = std::min(16u, ncol - c);
    b.norm = norm;
    b.eps = eps;
    b.y = y + size_t(c) * ldy;
    b.ldy = ldy;
    b.done = done;
    b.err = err;
    b.waves = waves;
    HIPC(launch_bmm(epi, b, stream_));
  }
}

// Whether lin() runs L over ncol columns on the batched MFMA product.  At
// two columns every S2-Pro linear is faster on the two-column GEMV (wqkv 8.3
// vs 12.6 us, wo 7.6 vs 8.5, w1/w3 18.5 vs 23.4, w2 12.3 vs 16.6; the first
// Fast-AR sub-step of a frame runs two columns: default decode 308.5-308.7
// frames/s against 304.1-304.3 with w1/w3 and w2 on the product).
bool Engine::uses_bmm(const DevLin& L, const DevLin* L3, uint32_t ncol) const {
  if (bmm_off_ || !L.wt || !bmm_min_cols_ || ncol < bmm_min_cols_ || (L3 && !L3->wt)) return false;
  return !(ncol == 2 && gemv_rows_per_block(L.type, L.in, L.out, false, L3 != nullptr, ncol) != 0);
}

void Engine::lin(const DevLin& L, const DevLin* L3, int epi, uint32_t ncol, const float* x, uint32_t ldx,
                 const float* norm, float eps, float* y, uint32_t ldy, uint32_t row_base, uint32_t extra_row,
                 uint32_t out_rows, const uint32_t* done, uint32_t bmm_waves, const GreedyFold* fold) {
  if (fold) {  // one column (checked by gemv), never on the batched product
    gemv(L, L3, epi, ncol, x, ldx, norm, eps, y, ldy, row_base, extra_row, out_rows, done, fold);
    return;
  }
  if (uses_bmm(L, L3, ncol)) {
    bmm(L, L3, epi, ncol, x, ldx, norm, eps, y, ldy, done, &st_->err, bmm_waves);
    return;
  }
  if (ncol <= 2 || L.in % 256) {
    gemv(L, L3, epi, ncol, x, ldx, norm, eps, y, ldy, row_base, extra_row, out_rows, done);
    return;
  }
  for (uint32_t c = 0; c < ncol; c += 16) {
    const uint32_t n = std::min(16u, ncol - c);
    mm_skinny(L, L3, epi, x + size_t(c) * ldx, ldx, norm, eps, n, y + size_t(c) * ldy, ldy, row_base, extra_row,
              out_rows, done);
  }
}

// The rows lin() reads next for L over ncol columns, as the warming blocks of
// a kernel before it should read them: only when lin() takes the decode GEMV
// (1-2 columns, no batched product), whose block shape fixes the span.  The
// consumer blocks from pct_begin % to pct_end % of the warmed range (at most
// warm_bytes_) are covered.
L2Warm Engine::warm_for(const DevLin& L, const DevLin* L3, uint32_t ncol, bool norm, uint32_t pct_begin,
                        uint32_t pct_end) const {
  L2Warm w{};
  if (!warm_blocks_ || ncol > 2 || !L.w || pct_end <= pct_begin || uses_bmm(L, L3, ncol)) return w;
  // Q8_0 / Q4_0 GEMVs read the repacked planes, except one matrix with
  // 2560-wide rows and an RMSNorm (wqkv, the heads): that stays on the GGUF rows
  if (L.qp && ncol <= 2 && !(norm && !L3 && L.in == 2560)) return w;
  const uint32_t rpb = gemv_rows_per_block(L.type, L.in, L.out, norm, L3 != nullptr, ncol);
  const size_t span = size_t(rpb) * L.row_bytes;
  if (!rpb || span % 16 || span > UINT32_MAX || reinterpret_cast<uintptr_t>(L.w) % 16 ||
      (L3 && reinterpret_cast<uintptr_t>(L3->w) % 16))
    return w;
  const size_t nb = std::min<size_t>(L.out / rpb, warm_bytes_ / (span * (L3 ? 2 : 1)));  // whole blocks only
  const uint32_t b0 = uint32_t(nb * pct_begin / 100) & ~7u, b1 = uint32_t(nb * pct_end / 100);
  if (b1 <= b0) return w;
  w.base = L.w;
  w.base3 = L3 ? L3->w : nullptr;
  w.span = uint32_t(span);
  w.cb_begin = b0;
  w.cb_end = b1;
  w.blocks = warm_blocks_;
  w.depth = warm_depth_;
  return w;
}

enum { PROF_NONE = -1, PROF_LINEAR = 0, PROF_ATTN = 1, PROF_HEAD = 2 };

// Marks the end of the interval since the previous mark; `kind` names what
// ran in it (PROF_NONE for the first mark of a group).
void Engine::prof_mark(int kind) {
  if (!profiling_) return;
  const size_t i = prof_kind_.size();
  if (i == prof_ev_.size()) {
    hipEvent_t e;
    HIPC(hipEventCreate(&e));
    prof_ev_.push_back(e);
  }
  HIPC(hipEventRecord(prof_ev_[i], stream_));
  prof_kind_.push_back(kind);
}

void Engine::prof_book(uint32_t nseq) {
  if (!profiling_ || prof_kind_.empty()) return;
  HIPC(hipEventSynchronize(prof_ev_[prof_kind_.size() - 1]));
  for (size_t i = 1; i < prof_kind_.size(); ++i) {
    if (prof_kind_[i] == PROF_NONE) continue;
    float ms = 0.0f;
    HIPC(hipEventElapsedTime(&ms, prof_ev_[i - 1], prof_ev_[i]));
    double* f = prof_kind_[i] == PROF_LINEAR ? &slow_prof.linear_ms
              : prof_kind_[i] == PROF_ATTN   ? &slow_prof.gqa_attention_ms
                                             : &slow_prof.output_head_ms;
    *f += ms;
  }
  slow_prof.steps += nseq;
  prof_kind_.clear();
}

// Slow-AR layers (forward_decode_sequence, slow_ar.rs:539-556) over nseq
// slots from seq0 with cps consecutive positions each, then n_past += cps per
// slot.  done (nullable) stops the linears; attention and the position
// update skip each finished slot by its own done word.
void Engine::enqueue_slow_layers(uint32_t nseq, uint32_t cps, uint32_t seq0, const uint32_t* done, bool advance) {
  const s2hip_spec& s = spec;
  const uint32_t q = s.heads * s.head_dim, kv = s.kv_heads * s.head_dim, qkv_w = q + 2 * kv;
  const uint32_t ncol = nseq * cps;
  DevState* st = st_ + seq0;
  for (uint32_t l = 0; l < s.slow_layers; ++l) {
    const SlowLayer& L = slow_[l];
    prof_mark(PROF_NONE);
    lin(L.wqkv, nullptr, EPI_STORE, ncol, h_, s.dim, L.attn_norm, s.eps, qkv_, qkv_w, 0, NO_ROW, L.wqkv.out, done);
    prof_mark(PROF_LINEAR);
    AttnArgs aa{};
    aa.qkv = qkv_;
    aa.q_norm = L.q_norm;
    aa.k_norm = L.k_norm;
    aa.eps = s.eps;
    aa.rope = rope_slow_;
    aa.k_cache = kvp(kc_, size_t(seq0) * slot_kv_ + size_t(l) * kv * s.max_seq_len);
    aa.v_cache = kvp(vc_, size_t(seq0) * slot_kv_ + size_t(l) * kv * s.max_seq_len);
    aa.kv_f16 = kv_f16_;
    aa.part = part_;
    aa.counters = counters_;
    aa.out = att_;
    aa.pos_ptr = &st->n_past;
    aa.pos_offset = 0;
    aa.H = s.heads;
    aa.Hkv = s.kv_heads;
    aa.hd = s.head_dim;
    aa.max_seq = s.max_seq_len;
    aa.ncol = ncol;
    aa.max_chunks = attn_chunks_;
    aa.mode = attn_mode_;
    aa.scale = 1.0f / std::sqrt(float(s.head_dim));  // slow_ar.rs:59-61
    aa.done = done ? &st->done : nullptr;
    aa.err = &st->err;
    aa.cols_per_seq = cps;
    aa.seq_stride_words = sizeof(DevState) / 4;
    aa.seq_stride_kv = slot_kv_;
    // (the merge kernel carries no warming: its 128-thread blocks warm too
    // slowly, and it waits for them -- 292.3-292.7 against 307.4-308.1
    // frames/s with half the rows given to it)
    aa.check_from = nseq >= ATTN_CHECK_MIN_SEQS ? attn_check_from_ : 0u;
    aa.warm = warm_for(L.wo, nullptr, ncol, false, 0, warm_slow_);
    HIPC(launch_attention(aa, stream_));
    prof_mark(PROF_ATTN);
    lin(L.wo, nullptr, EPI_RESID, ncol, att_, q, nullptr, 0.0f, h_, s.dim, 0, NO_ROW, L.wo.out, done);
    lin(L.w1, &L.w3, EPI_SWIGLU_SLOW, ncol, h_, s.dim, L.ffn_norm, s.eps, act_, s.ffn, 0, NO_ROW, L.w1.out, done);
    lin(L.w2, nullptr, EPI_RESID, ncol, act_, s.ffn, nullptr, 0.0f, h_, s.dim, 0, NO_ROW, L.w2.out, done);
    prof_mark(PROF_LINEAR);
  }
  if (advance) HIPC(launch_add_position(st, cps, nseq, stream_));
}

// SlowArOutputHeadF16Weights::forward_logits (slow_ar.rs:943-955): post-norm
// hidden of the first ncol columns of h_ -> tied embedding rows.  Generation
// only needs the candidate rows (semantic ids + im_end); every other id is
// masked to -inf before sampling.  hn [ncol][dim], logits [ncol][n_cand].
void Engine::enqueue_head(uint32_t ncol, float* hn, float* logits, bool full, const uint32_t* done) {
  const s2hip_spec& s = spec;
  if (ncol == 1 && (s.dim == 512 || s.dim == 1536 || s.dim == 2560)) {
    // one column: the RMSNorm is the head GEMV's own (its block 0 writes the
    // normalised row to hn, which the Fast-AR and the full head read)
    gemv_xn_ = hn;
    lin(head_cand_, nullptr, EPI_STORE, 1, h_, s.dim, norm_, s.eps, logits, n_cand_, s.semantic_begin, head_extra_,
        n_cand_, done);
    gemv_xn_ = nullptr;
  } else {
    HIPC(launch_rms_norm(h_, norm_, hn, s.dim, ncol, s.eps, done, stream_));
    lin(head_cand_, nullptr, EPI_STORE, ncol, hn, s.dim, nullptr, 0.0f, logits, n_cand_, s.semantic_begin,
        head_extra_, n_cand_, done);
  }
  if (full)
    gemv(head_full_, nullptr, EPI_STORE, 1, hn, s.dim, nullptr, 0.0f, logits_full_, s.vocab, 0, NO_ROW, s.vocab, done);
}

// Fast-AR layers (forward_prefill, fast_ar.rs:245-358) over nseq slots with cps consecutive
// positions each from p0 (every slot is at the same Fast-AR position).
void Engine::enqueue_fast_layers(uint32_t nseq, uint32_t cps, uint32_t p0, const uint32_t* done,
                                 const GreedyFold* fold, const uint32_t* code) {
  const s2hip_spec& s = spec;
  const uint32_t fq = s.fast_heads * s.fast_head_dim, fkv = s.fast_kv_heads * s.fast_head_dim;
  const uint32_t w = fq + 2 * fkv;
  const uint32_t ncol = nseq * cps;
  for (uint32_t l = 0; l < s.fast_layers; ++l) {
    const FastLayer& L = fast_[l];
    // layer 0 of a table sub-step: q / k / v from the table (the attention
    // takes the code, sampling it itself under a fold)
    const bool table = l == 0 && fast_table_ && ncol == 1 && (code || fold);
    if (!table)
      lin(L.wqkv, nullptr, EPI_STORE, ncol, fh_, s.dim, L.attn_norm, s.fast_eps, fqkv_, w, 0, NO_ROW, L.wqkv.out,
          done, 0, l == 0 ? fold : nullptr);
    AttnArgs aa{};
    aa.qkv = fqkv_;
    if (table) {
      aa.qkv_rows = fast_table_;
      if (fold) aa.fold = *fold;
      else aa.code_ptr = code;
      aa.fold.n = s.codebook_size;
    }
    aa.q_norm = nullptr;  // the Fast-AR applies no QK-norm (fast_ar.rs:310-334)
    aa.k_norm = nullptr;
    aa.eps = s.fast_eps;
    aa.rope = rope_fast_;
    aa.k_cache = fkc_ + size_t(l) * fkv * fctx_;
    aa.v_cache = fvc_ + size_t(l) * fkv * fctx_;
    aa.part = fpart_;
    aa.counters = counters_;
    aa.out = fatt_;
    aa.pos_ptr = nullptr;
    aa.pos_offset = p0;
    aa.H = s.fast_heads;
    aa.Hkv = s.fast_kv_heads;
    aa.hd = s.fast_head_dim;
    aa.max_seq = fctx_;
    aa.ncol = ncol;
    aa.max_chunks = attention_chunks(fctx_, attn_mode_);
    aa.mode = table ? ATTN_SPLIT : attn_mode_;  // (a table sub-step: the partial kernel's table form)
    aa.scale = 1.0f / std::sqrt(float(s.fast_head_dim));  // fast_ar.rs:60-62
    aa.done = done ? &st_->done : nullptr;
    aa.err = &st_->err;
    aa.cols_per_seq = cps;
    aa.seq_stride_words = sizeof(DevState) / 4;
    aa.seq_stride_kv = fslot_kv_;
    // The last layer's outputs feed only the head, which reads each slot's
    // last position: with several positions per slot (the first pass), wo,
    // w1/w3 and w2 run on those columns alone (strided views of fatt_ and
    // fh_; the earlier positions' rows are rewritten before the next pass
    // reads fh_, and their K/V were appended by the attention above).
    const bool last_only = l + 1 == s.fast_layers && cps > 1;
    const uint32_t fcols = last_only ? nseq : ncol;
    const float* att_in = fatt_ + (last_only ? size_t(cps - 1) * fq : 0);
    const uint32_t att_ld = last_only ? cps * fq : fq;
    float* res = fh_ + (last_only ? size_t(cps - 1) * s.dim : 0);
    const uint32_t res_ld = last_only ? cps * s.dim : s.dim;
    aa.warm = warm_for(L.wo, nullptr, fcols, false, 0, warm_fast_);
    HIPC(launch_attention(aa, stream_));
    lin(L.wo, nullptr, EPI_RESID, fcols, att_in, att_ld, nullptr, 0.0f, res, res_ld, 0, NO_ROW, L.wo.out, done);
    // one wave per tile from 8 columns: the Fast-AR weights are re-read every
    // sub-step and this product runs warm (batch 8: 22.3 us against 24.2 us
    // with the two waves that suit the Slow-AR layers; 3-7 columns keep two
    // waves; 2 columns take the GEMV)
    lin(L.w1, &L.w3, EPI_SWIGLU_FAST, fcols, res, res_ld, L.ffn_norm, s.fast_eps, fact_, s.fast_ffn, 0, NO_ROW,
        L.w1.out, done, fcols >= 8 && (L.w1.out + 15) / 16 >= 512 ? 1u : 0u);
    lin(L.w2, nullptr, EPI_RESID, fcols, fact_, s.fast_ffn, nullptr, 0.0f, res, res_ld, 0, NO_ROW, L.w2.out, done);
  }
}

// generate_codebooks_for_semantic (fast_ar.rs:440-470), incremental, for the
// slots 0 .. nseq - 1: sub-step 1 runs positions 0 (slow hidden) and 1
// (fast_emb[code0]) together, each later sub-step appends one position.  The
// sampler writes each slot's next input row.  A greedy sample of one slot
// before a further sub-step is folded into that sub-step's first linear
// (GreedyFold): one kernel less per codebook; a tie at the max sets
// ERR_GREEDY_TIE and the caller runs again with the sampler kernel.
bool Engine::fold_greedy(const SamplerCfg& cfg, uint32_t nseq) const {
  const s2hip_spec& s = spec;
  const DevLin& L = fast_[0].wqkv;
  if (fold_off_ || fold_env_off_ || nseq != 1 || cfg.temperature > 0.0f || s.codebook_size % 4 || s.fast_layers == 0) return false;
  // the one-column wqkv kernel (the GGUF-row kernel for every weight type)
  if (L.type == W_F16) return s.dim == 512 || s.dim == 1536 || s.dim == 2560;
  return (L.type == W_Q8_0 || L.type == W_Q4_0) && s.dim == 2560;
}

void Engine::enqueue_fast_frame(const SamplerCfg& cfg, uint32_t nseq, const uint32_t* done) {
  const s2hip_spec& s = spec;
  HIPC(launch_fast_begin(st_, hn_, fast_emb_, fh_, s.dim, s.codebook_size, s.semantic_begin, s.semantic_end, nseq,
                         stream_));
  const bool fold = fold_greedy(cfg, nseq);
  const bool table = fast_table_ && nseq == 1;
  GreedyFold gf{};
  const uint32_t* code = nullptr;  // the code whose embedding the next sub-step takes (table sub-steps)
  uint32_t cps = 2, p0 = 0;
  for (uint32_t cb = 1; cb < s.num_codebooks; ++cb) {
    enqueue_fast_layers(nseq, cps, p0, done, gf.logits ? &gf : nullptr, code);
    // the last position of each slot: rows cps - 1, 2 cps - 1, ...
    lin(fast_out_, nullptr, EPI_STORE, nseq, fh_ + size_t(cps - 1) * s.dim, cps * s.dim, fast_norm_, s.fast_eps,
        flogits_, s.codebook_size, 0, NO_ROW, s.codebook_size, done);
    p0 += cps;
    cps = 1;
    if (fold && cb + 1 < s.num_codebooks) {
      gf.logits = flogits_;
      gf.n = s.codebook_size;
      gf.emb = fast_emb_;
      gf.st = st_;
      gf.cb_index = cb;
      gf.x_out = fh_;
      gf.dim = s.dim;
      continue;
    }
    gf = GreedyFold{};
    code = (table && cb + 1 < s.num_codebooks) ? &st_->codes_frame[cb] : nullptr;
    SampleArgs sa{};
    sa.logits = flogits_;
    sa.n = s.codebook_size;
    sa.vocab = s.codebook_size;
    sa.cfg = cfg;
    sa.st = st_;
    sa.cb_index = cb;
    sa.fast_emb = fast_emb_;
    sa.next_input = (cb + 1 < s.num_codebooks) ? fh_ : nullptr;
    sa.dim = s.dim;
    sa.n_seq = nseq;
    // the next sub-step's first linear (one column per slot); the general
    // path (tens of microseconds on one CU, HBM idle) reads all of its rows
    if (sa.next_input && !table)
      sa.warm = warm_for(fast_[0].wqkv, nullptr, nseq, true, 0, cfg.temperature > 0.0f ? 100u : warm_step_);
    HIPC(launch_sample_fast(sa, stream_));
  }
}

// One generate_codes loop iteration (generate.rs:165-211) for the slots
// 0 .. nseq - 1: Fast-AR codebooks for each current main token, one Slow-AR
// step on each [main, codes...], the next samples.  Every kernel stops once
// the whole batch is done; finished slots are skipped by their own state.
void Engine::enqueue_frame(const SamplerCfg& cfg, uint32_t nseq, size_t codes_stride) {
  const s2hip_spec& s = spec;
  const uint32_t* done = &batch_->done_all;
  enqueue_fast_frame(cfg, nseq, done);
  EmbedArgs ea{};
  ea.tokens = nullptr;
  ea.state = st_;
  ea.emb = emb_;
  ea.cb_emb = cb_emb_;
  ea.h = h_;
  ea.n = nseq;
  ea.dim = s.dim;
  ea.vocab = s.vocab;
  ea.cb_rows = uint32_t(cb_rows_);
  ea.num_codebooks = s.num_codebooks;
  ea.codebook_size = s.codebook_size;
  ea.sem_begin = s.semantic_begin;
  ea.sem_end = s.semantic_end;
  ea.sem_scale = 1.0f / std::sqrt(float(s.num_codebooks + 1));
  ea.scale_enabled = s.scale_codebook_embeddings;
  ea.done = done;
  ea.err = &st_->err;
  ea.warm = warm_for(slow_[0].wqkv, nullptr, nseq, true, 0, warm_step_);
  HIPC(launch_embed(ea, stream_));
  enqueue_slow_layers(nseq, 1, 0, done, false);  // the sampler advances n_past
  prof_mark(PROF_NONE);
  enqueue_head(nseq, hn_, logits_c_, false, done);
  prof_mark(PROF_HEAD);
  SampleArgs sa{};
  sa.logits = logits_c_;
  sa.ids = head_rows_;
  sa.n = n_cand_;
  sa.vocab = s.vocab;
  sa.cfg = cfg;
  sa.st = st_;
  sa.im_end = im_end_;
  sa.after_step = 1;
  sa.advance = 1;
  sa.codes_out = codes_dev_;
  sa.num_codebooks = s.num_codebooks;
  sa.n_seq = nseq;
  sa.codes_stride = codes_stride;
  sa.batch = batch_;
  HIPC(launch_sample_slow(sa, stream_));
}

// Prompt prefill (forward_slow_ar_block_prefill_layers_cached, slow_ar.rs:1002-1039):
// chunks of up to PREFILL_CHUNK tokens go through each layer together: every
// linear is one MFMA product over the chunk (weights read once per chunk),
// QK-norm + RoPE + KV append for all of the chunk's positions, then causal
// attention of each token over the cache.  One slot (`seq`) at a time;
// leaves the last token's residual row in decode column 0 for the output head.
void Engine::mm(const DevLin& L, const DevLin* L3, int epi, const float* x, uint32_t ldx, const float* norm, float eps,
                uint32_t n, uint32_t npad, float* y, uint32_t ldy) {
  HIPC(launch_split_rows(x, ldx, norm, eps, n, npad, L.in, pxh_, pxl_, prs_, nullptr, stream_));
  GemmArgs g{};
  g.w = L.w;
  g.w3 = L3 ? L3->w : nullptr;
  g.row_bytes = L.row_bytes;
  g.M = L.out;
  g.K = L.in;
  g.xh = pxh_;
  g.xl = pxl_;
  g.rs = prs_;
  g.N = n;
  g.y = y;
  g.ldy = ldy;
  g.part = ppart_;
  g.part_cap = ppart_cap_;
  HIPC(launch_gemm_mfma(L.type, epi, g, stream_));
}

// The decode kernels over 4 columns at a time (weights re-read every 4
// tokens); S2HIP_PREFILL_GEMV=1 selects it, for comparisons.
void Engine::mm_skinny(const DevLin& L, const DevLin* L3, int epi, const float* x, uint32_t ldx, const float* norm,
                       float eps, uint32_t n, float* y, uint32_t ldy, uint32_t row_base, uint32_t extra_row,
                       uint32_t out_rows, const uint32_t* done) {
  HIPC(launch_split_rows(x, ldx, norm, eps, n, 16, L.in, pxh_, pxl_, prs_, &st_->err, stream_));
  SkinnyArgs g{};
  g.w = L.w;
  g.w3 = L3 ? L3->w : nullptr;
  g.row_bytes = L.row_bytes;
  g.row_base = row_base;
  g.extra_row = extra_row;
  g.M = out_rows;
  g.K = L.in;
  g.xh = pxh_;
  g.xl = pxl_;
  g.rs = prs_;
  g.N = n;
  g.y = y;
  g.ldy = ldy;
  g.done = done;
  HIPC(launch_skinny_mfma(L.type, epi, g, stream_));
}

void Engine::enqueue_prefill_gemv(const int32_t* prompt_dev, size_t n_tok, uint32_t seq) {
  const s2hip_spec& s = spec;
  const uint32_t cdim = s.num_codebooks + 1;
  size_t t = 0;
  uint32_t nc = 0;
  while (t < n_tok) {
    nc = uint32_t(std::min<size_t>(PREFILL_COLS, n_tok - t));
    EmbedArgs ea{};
    ea.tokens = prompt_dev + t * cdim;
    ea.emb = emb_;
    ea.cb_emb = cb_emb_;
    ea.h = h_;
    ea.n = nc;
    ea.dim = s.dim;
    ea.vocab = s.vocab;
    ea.cb_rows = uint32_t(cb_rows_);
    ea.num_codebooks = s.num_codebooks;
    ea.codebook_size = s.codebook_size;
    ea.sem_begin = s.semantic_begin;
    ea.sem_end = s.semantic_end;
    ea.sem_scale = 1.0f / std::sqrt(float(cdim));
    ea.scale_enabled = s.scale_codebook_embeddings;
    ea.err = &st_[seq].err;
    HIPC(launch_embed(ea, stream_));
    enqueue_slow_layers(1, nc, seq, nullptr);
    t += nc;
  }
  if (nc > 1) HIPC(hipMemcpyAsync(h_, h_ + size_t(nc - 1) * s.dim, size_t(s.dim) * 4, hipMemcpyDeviceToDevice, stream_));
}

void Engine::enqueue_prefill(const int32_t* prompt_dev, size_t n_tok, uint32_t seq) {
  if (prefill_gemv_) {
    enqueue_prefill_gemv(prompt_dev, n_tok, seq);
    return;
  }
  const s2hip_spec& s = spec;
  const uint32_t cdim = s.num_codebooks + 1;
  const uint32_t q = s.heads * s.head_dim, kv = s.kv_heads * s.head_dim, qkv_w = q + 2 * kv;
  DevState* st = st_ + seq;
  size_t t = 0;
  uint32_t nc = 0;
  while (t < n_tok) {
    nc = uint32_t(std::min<size_t>(PREFILL_CHUNK, n_tok - t));
    const uint32_t npad = gemm_rows_pad(nc);
    EmbedArgs ea{};
    ea.tokens = prompt_dev + t * cdim;
    ea.emb = emb_;
    ea.cb_emb = cb_emb_;
    ea.h = ph_;
    ea.n = nc;
    ea.dim = s.dim;
    ea.vocab = s.vocab;
    ea.cb_rows = uint32_t(cb_rows_);
    ea.num_codebooks = s.num_codebooks;
    ea.codebook_size = s.codebook_size;
    ea.sem_begin = s.semantic_begin;
    ea.sem_end = s.semantic_end;
    ea.sem_scale = 1.0f / std::sqrt(float(cdim));
    ea.scale_enabled = s.scale_codebook_embeddings;
    ea.err = &st->err;
    HIPC(launch_embed(ea, stream_));
    for (uint32_t l = 0; l < s.slow_layers; ++l) {
      const SlowLayer& L = slow_[l];
      float* kcl = kvp(kc_, size_t(seq) * slot_kv_ + size_t(l) * kv * s.max_seq_len);
      float* vcl = kvp(vc_, size_t(seq) * slot_kv_ + size_t(l) * kv * s.max_seq_len);
      mm(L.wqkv, nullptr, EPI_STORE, ph_, s.dim, L.attn_norm, s.eps, nc, npad, pqkv_, qkv_w);
      QkvPostArgs qa{};
      qa.qkv = pqkv_;
      qa.q_out = pq_;
      qa.k_cache = kcl;
      qa.v_cache = vcl;
      qa.q_norm = L.q_norm;
      qa.k_norm = L.k_norm;
      qa.rope = rope_slow_;
      qa.pos_ptr = &st->n_past;
      qa.pos_offset = 0;
      qa.H = s.heads;
      qa.Hkv = s.kv_heads;
      qa.hd = s.head_dim;
      qa.max_seq = s.max_seq_len;
      qa.ncol = nc;
      qa.eps = s.eps;
      qa.err = &st->err;
      qa.kv_f16 = kv_f16_;
      HIPC(launch_qkv_post(qa, stream_));
      PrefillAttnArgs pa{};
      pa.q = pq_;
      pa.k_cache = kcl;
      pa.v_cache = vcl;
      pa.out = patt_;
      pa.pos_ptr = &st->n_past;
      pa.pos_offset = 0;
      pa.N = nc;
      pa.H = s.heads;
      pa.Hkv = s.kv_heads;
      pa.hd = s.head_dim;
      pa.max_seq = s.max_seq_len;
      pa.scale = 1.0f / std::sqrt(float(s.head_dim));  // slow_ar.rs:59-61
      pa.kv_f16 = kv_f16_;
      pa.err = &st->err;
      pa.part = ppart_;
      pa.part_cap = ppart_cap_;
      HIPC(launch_attention_prefill(pa, stream_));
      mm(L.wo, nullptr, EPI_RESID, patt_, q, nullptr, 0.0f, nc, npad, ph_, s.dim);
      mm(L.w1, &L.w3, EPI_SWIGLU_SLOW, ph_, s.dim, L.ffn_norm, s.eps, nc, npad, pact_, s.ffn);
      mm(L.w2, nullptr, EPI_RESID, pact_, s.ffn, nullptr, 0.0f, nc, npad, ph_, s.dim);
    }
    HIPC(launch_add_position(st, nc, 1, stream_));
    t += nc;
  }
  if (nc) HIPC(hipMemcpyAsync(h_, ph_ + size_t(nc - 1) * s.dim, size_t(s.dim) * 4, hipMemcpyDeviceToDevice, stream_));
}

void Engine::ensure_prompt(size_t n_int) {
  if (n_int <= prompt_cap_) return;
  if (prompt_dev_) {
    HIPC(hipStreamSynchronize(stream_));
    HIPC(hipFree(prompt_dev_));
    allocs_.erase(std::find(allocs_.begin(), allocs_.end(), static_cast<void*>(prompt_dev_)));
  }
  prompt_cap_ = std::max<size_t>(n_int, 4096);
  prompt_dev_ = dalloc<int32_t>(prompt_cap_);
}

void Engine::ensure_codes(size_t n_int) {
  if (n_int <= codes_cap_ && codes_dev_) return;
  if (codes_dev_) {
    HIPC(hipStreamSynchronize(stream_));
    HIPC(hipFree(codes_dev_));
    allocs_.erase(std::find(allocs_.begin(), allocs_.end(), static_cast<void*>(codes_dev_)));
  }
  codes_cap_ = std::max<size_t>(n_int, 16 * 1024);
  codes_dev_ = dalloc<int32_t>(codes_cap_);
}

void Engine::ensure_slots(uint32_t n) {
  if (n <= kv_slots_) return;
  HIPC(hipStreamSynchronize(stream_));
  // the Slow-AR caches grow with the existing slots' contents kept (slot-major
  // layout: the old buffer is a prefix of the new one); the Fast-AR caches are
  // per-frame scratch
  const size_t eb = kv_f16_ ? 2 : 4;
  const size_t old_bytes = size_t(kv_slots_) * slot_kv_ * eb, kv_bytes = size_t(n) * slot_kv_ * eb;
  for (float** p : {&kc_, &vc_}) {
    float* nb = dalloc<float>((kv_bytes + 3) / 4);
    HIPC(hipMemset(nb, 0, kv_bytes));
    if (*p) {
      HIPC(hipMemcpy(nb, *p, old_bytes, hipMemcpyDeviceToDevice));
      HIPC(hipFree(*p));
      allocs_.erase(std::find(allocs_.begin(), allocs_.end(), static_cast<void*>(*p)));
    }
    *p = nb;
  }
  for (float** p : {&fkc_, &fvc_}) {
    if (*p) {
      HIPC(hipFree(*p));
      allocs_.erase(std::find(allocs_.begin(), allocs_.end(), static_cast<void*>(*p)));
    }
    *p = dalloc<float>(size_t(n) * fslot_kv_);
    HIPC(hipMemset(*p, 0, size_t(n) * fslot_kv_ * 4));
  }
  kv_slots_ = n;
  ++kv_gen_;
}

void Engine::repack(DevLin& L) {
  const uint32_t qb = repack_quant_bytes(L.type);
  if (!qb || L.in % 32 || L.qp) return;
  const size_t nblk = size_t(L.in / 32) * L.out;
  L.qp = dalloc<uint8_t>(nblk * qb);
  L.qs = dalloc<uint16_t>(nblk);
  HIPC(launch_repack_q(L.w, L.row_bytes, L.type, L.in, L.out, L.qp, L.qs, stream_));
}

void Engine::tile(DevLin& L, uint32_t rows, uint32_t row_base, uint32_t extra_row) {
  if (L.type != W_F16 || L.in % 256 || L.in > BMM_MAX_K || L.wt) return;
  L.wt = dalloc<_Float16>(size_t(bmm_rows_pad(rows)) * L.in);
  HIPC(launch_tile_f16(reinterpret_cast<const uint16_t*>(L.w), L.in, rows, row_base, extra_row,
                       reinterpret_cast<uint16_t*>(L.wt), stream_));
}

// The batched product's copies of the F16 linears and the repacked Q8_0 /
// Q4_0 linears of the one-column GEMV (one more HBM copy of the weights),
// built once, the first time a decode needs them.
void Engine::ensure_tiled() {
  if (tiled_) return;
  for (auto& L : slow_)
    for (DevLin* d : {&L.wqkv, &L.wo, &L.w1, &L.w2, &L.w3}) repack(*d);
  for (auto& L : fast_)
    for (DevLin* d : {&L.wqkv, &L.wo, &L.w1, &L.w2, &L.w3}) repack(*d);
  repack(fast_out_);
  if (!bmm_min_cols_) {
    HIPC(hipStreamSynchronize(stream_));
    tiled_ = true;
    return;
  }
  for (auto& L : slow_)
    for (DevLin* d : {&L.wqkv, &L.wo, &L.w1, &L.w2, &L.w3}) tile(*d, d->out, 0, NO_ROW);
  for (auto& L : fast_)
    for (DevLin* d : {&L.wqkv, &L.wo, &L.w1, &L.w2, &L.w3}) tile(*d, d->out, 0, NO_ROW);
  tile(fast_out_, fast_out_.out, 0, NO_ROW);
  tile(head_cand_, n_cand_, spec.semantic_begin, head_extra_);
  HIPC(hipStreamSynchronize(stream_));
  tiled_ = true;
}

void Engine::check_state_err(uint32_t nseq) {
  for (uint32_t b = 0; b < nseq; ++b) {
    const std::string who = nseq > 1 ? " (request " + std::to_string(b) + ")" : std::string();
    if (st_host_[b].err & ERR_TOKEN_RANGE) fail("token id out of range" + who);
    if (st_host_[b].err & ERR_KV_OVERFLOW) fail("KV cache overflow" + who);
    if (st_host_[b].err & ERR_SAMPLER) fail("sampler failure" + who);
    if (st_host_[b].err & ERR_F16_RANGE) fail("activation not finite or beyond the range of the batched product");
    if (st_host_[b].err & ERR_NONFINITE) fail("activation not finite");
    if (st_host_[b].err & ERR_GREEDY_TIE) fail("tie at a folded greedy sample" + who);
  }
}

void Engine::reset(uint32_t slot) {
  select();
  if (slot >= MAX_SEQS) fail("slot " + std::to_string(slot) + " out of range (0.." + std::to_string(MAX_SEQS - 1) + ")");
  HIPC(hipStreamSynchronize(stream_));
  HIPC(hipMemsetAsync(st_ + slot, 0, sizeof(DevState), stream_));
  HIPC(hipStreamSynchronize(stream_));
  n_past_host[slot] = 0;
}

// Token ids of a time-major [n_tok][num_codebooks + 1] block, checked as
// embed_slow_ar_time_major does (slow_ar.rs:1041-1133).
void Engine::validate_tokens(const int32_t* flat, size_t n_tok) {
  const s2hip_spec& s = spec;
  const uint32_t cdim = s.num_codebooks + 1;
  for (size_t t = 0; t < n_tok; ++t) {
    const int32_t id = flat[t * cdim];
    if (id < 0) fail("semantic token id must be non-negative, got " + std::to_string(id));
    if (uint32_t(id) >= s.vocab) fail("embedding index " + std::to_string(id) + " out of range");
    if (uint32_t(id) >= s.semantic_begin && uint32_t(id) <= s.semantic_end)
      for (uint32_t cb = 0; cb < s.num_codebooks; ++cb)
        if (flat[t * cdim + 1 + cb] < 0 ||
            uint64_t(flat[t * cdim + 1 + cb]) + uint64_t(cb) * s.codebook_size >= cb_rows_)
          fail("codebook token out of range");
  }
}

void Engine::eval(const int32_t* flat, size_t n_tok, float* hidden_out, float* logits_out, uint32_t slot) {
  select();
  const s2hip_spec& s = spec;
  const uint32_t cdim = s.num_codebooks + 1;
  if (slot >= MAX_SEQS) fail("slot " + std::to_string(slot) + " out of range (0.." + std::to_string(MAX_SEQS - 1) + ")");
  if (n_tok == 0) fail("expected at least one token");
  if (n_past_host[slot] + n_tok > s.max_seq_len)
    fail("KV cache overflow: n_past=" + std::to_string(n_past_host[slot]) + " n_tokens=" + std::to_string(n_tok) +
         " max_seq_len=" + std::to_string(s.max_seq_len));
  validate_tokens(flat, n_tok);
  ensure_slots(slot + 1);
  ensure_prompt(n_tok * cdim);
  HIPC(hipMemcpyAsync(prompt_dev_, flat, n_tok * cdim * 4, hipMemcpyHostToDevice, stream_));
  // done = 0, err = 0 (eval never runs under a finished frame loop)
  HIPC(hipMemsetAsync(&st_[slot].done, 0, sizeof(uint32_t), stream_));
  HIPC(hipMemsetAsync(&st_[slot].err, 0, sizeof(uint32_t), stream_));
  enqueue_prefill(prompt_dev_, n_tok, slot);
  enqueue_head(1, hn_, logits_c_, logits_out != nullptr, nullptr);
  HIPC(hipMemcpyAsync(hidden_out, hn_, s.dim * 4, hipMemcpyDeviceToHost, stream_));
  if (logits_out) HIPC(hipMemcpyAsync(logits_out, logits_full_, size_t(s.vocab) * 4, hipMemcpyDeviceToHost, stream_));
  HIPC(hipMemcpyAsync(st_host_ + slot, st_ + slot, sizeof(DevState), hipMemcpyDeviceToHost, stream_));
  HIPC(hipStreamSynchronize(stream_));
  const uint32_t e = st_host_[slot].err;
  if (e & ERR_TOKEN_RANGE) fail("token id out of range");
  if (e & ERR_KV_OVERFLOW) fail("KV cache overflow");
  if (e & ERR_F16_RANGE) fail("activation not finite or beyond the range of the batched product");
  if (e & ERR_NONFINITE) fail("activation not finite");
  n_past_host[slot] += uint32_t(n_tok);
}

void Engine::fast_logits(const float* hidden, const uint32_t* prefix, size_t plen, float* logits) {
  select();
  const s2hip_spec& s = spec;
  if (plen >= s.num_codebooks) fail("fast prefix too long: " + std::to_string(plen) + " codes");
  std::vector<uint16_t> row(s.dim);
  std::vector<float> rowf(s.dim);
  HIPC(hipMemcpyAsync(fh_, hidden, s.dim * 4, hipMemcpyHostToDevice, stream_));
  enqueue_fast_layers(1, 1, 0, nullptr);
  for (size_t j = 0; j < plen; ++j) {
    if (prefix[j] >= s.codebook_size) fail("fast prefix code out of range");
    HIPC(hipMemcpyAsync(row.data(), fast_emb_ + size_t(prefix[j]) * s.dim, s.dim * 2, hipMemcpyDeviceToHost,
                        stream_));
    HIPC(hipStreamSynchronize(stream_));
    for (uint32_t i = 0; i < s.dim; ++i) rowf[i] = f16_to_f32(row[i]);
    HIPC(hipMemcpyAsync(fh_, rowf.data(), s.dim * 4, hipMemcpyHostToDevice, stream_));
    enqueue_fast_layers(1, 1, uint32_t(j + 1), nullptr);
  }
  gemv(fast_out_, nullptr, EPI_STORE, 1, fh_, s.dim, fast_norm_, s.fast_eps, flogits_, s.codebook_size, 0, NO_ROW,
       s.codebook_size, nullptr);
  HIPC(hipMemcpyAsync(logits, flogits_, s.codebook_size * 4, hipMemcpyDeviceToHost, stream_));
  HIPC(hipStreamSynchronize(stream_));
}

void Engine::fast_codebooks(const float* hidden, uint32_t sem, const s2hip_sampler& smp, uint64_t* rng,
                            uint32_t* codes) {
  select();
  const s2hip_spec& s = spec;
  if (sem >= s.codebook_size) fail("semantic_code " + std::to_string(sem) + " >= codebook_size");
  DevState init{};
  init.main_token = s.semantic_begin + sem;
  init.rng = *rng;
  HIPC(hipMemcpyAsync(st_host_, st_, sizeof(DevState), hipMemcpyDeviceToHost, stream_));
  HIPC(hipStreamSynchronize(stream_));
  init.n_past = st_host_->n_past;  // keep the Slow-AR position
  *st_host_ = init;
  HIPC(hipMemcpyAsync(st_, st_host_, sizeof(DevState), hipMemcpyHostToDevice, stream_));
  HIPC(hipMemcpyAsync(hn_, hidden, s.dim * 4, hipMemcpyHostToDevice, stream_));
  ensure_fast_table();
  enqueue_fast_frame(SamplerCfg{smp.temperature, smp.top_p, smp.top_k}, 1, nullptr);
  HIPC(hipMemcpyAsync(st_host_, st_, sizeof(DevState), hipMemcpyDeviceToHost, stream_));
  HIPC(hipStreamSynchronize(stream_));
  const bool range = !bmm_off_ && any_f16_range(1), tie = !fold_off_ && any_err(1, ERR_GREEDY_TIE);
  if (range || tie) {  // again on the per-column paths / with the sampler kernels (as in generate)
    const bool bmm0 = bmm_off_, fold0 = fold_off_;
    bmm_off_ = bmm_off_ || range;
    fold_off_ = fold_off_ || tie;
    try {
      fast_codebooks(hidden, sem, smp, rng, codes);
    } catch (...) {
      bmm_off_ = bmm0;
      fold_off_ = fold0;
      throw;
    }
    bmm_off_ = bmm0;
    fold_off_ = fold0;
    return;
  }
  check_state_err();
  for (uint32_t cb = 0; cb < s.num_codebooks; ++cb) codes[cb] = st_host_->codes_frame[cb];
  *rng = st_host_->rng;
}

void Engine::validate_prompt(const int32_t* prompt, size_t cols) {
  const s2hip_spec& s = spec;
  const uint32_t cdim = s.num_codebooks + 1;
  if (cols == 0) fail("expected at least one token");
  if (cols > s.max_seq_len)
    fail("KV cache overflow: n_past=0 n_tokens=" + std::to_string(cols) + " max_seq_len=" + std::to_string(s.max_seq_len));
  for (size_t t = 0; t < cols; ++t) {
    const int32_t id = prompt[t * cdim];
    if (id < 0 || uint32_t(id) >= s.vocab) fail("prompt token id out of range: " + std::to_string(id));
    if (uint32_t(id) >= s.semantic_begin && uint32_t(id) <= s.semantic_end)
      for (uint32_t cb = 0; cb < s.num_codebooks; ++cb)
        if (prompt[t * cdim + 1 + cb] < 0 ||
            uint64_t(prompt[t * cdim + 1 + cb]) + uint64_t(cb) * s.codebook_size >= cb_rows_)
          fail("prompt codebook token out of range");
  }
}

// generate_codes (crates/fish_s2_infer/src/generate.rs:117-221) for nseq
// independent requests, one slot each, decoded together.  Every request's
// codes are those of its own generate_codes call; one request is the nseq = 1
// case of the same kernels.
void Engine::generate(uint32_t nseq, const int32_t* const* prompts, const size_t* cols, const s2hip_gen_params& p,
                      uint64_t* rngs, int32_t* const* codes, uint32_t* n_frames, s2hip_gen_stats* stats) {
  select();
  const s2hip_spec& s = spec;
  const uint32_t cdim = s.num_codebooks + 1;
  if (nseq == 0 || nseq > MAX_SEQS) fail("batch of " + std::to_string(nseq) + " requests (1.." +
                                         std::to_string(MAX_SEQS) + " supported)");
  size_t total_cols = 0;
  for (uint32_t b = 0; b < nseq; ++b) {
    validate_prompt(prompts[b], cols[b]);
    total_cols += cols[b];
  }
  const SamplerCfg cfg{p.temperature, p.top_p, p.top_k};
  const size_t ncodes = size_t(s.num_codebooks) * p.max_new_tokens;
  ensure_slots(nseq);
  ensure_tiled();
  ensure_fast_table();
  ensure_codes(ncodes * nseq);
  ensure_prompt(total_cols * cdim);
  HIPC(hipStreamSynchronize(stream_));
  // SlowArState::reset + sampler state, per slot
  for (uint32_t b = 0; b < nseq; ++b) {
    DevState init{};
    init.rng = rngs[b];
    init.prompt_cols = uint32_t(cols[b]);
    init.max_new = p.max_new_tokens;
    init.min_tokens_before_end = p.min_tokens_before_end;
    st_host_[b] = init;
  }
  HIPC(hipMemcpyAsync(st_, st_host_, nseq * sizeof(DevState), hipMemcpyHostToDevice, stream_));
  const BatchState bs{0u, 0u, nseq};
  HIPC(hipMemcpyAsync(batch_, &bs, sizeof(bs), hipMemcpyHostToDevice, stream_));
  if (ncodes) HIPC(hipMemsetAsync(codes_dev_, 0, ncodes * nseq * 4, stream_));
  {
    size_t off = 0;
    for (uint32_t b = 0; b < nseq; ++b) {
      HIPC(hipMemcpyAsync(prompt_dev_ + off, prompts[b], cols[b] * cdim * 4, hipMemcpyHostToDevice, stream_));
      off += cols[b] * cdim;
    }
  }
  hipEvent_t ev[3];
  for (auto& e : ev) HIPC(hipEventCreate(&e));
  HIPC(hipEventRecord(ev[0], stream_));
  // prompt prefill and the first semantic sample, request by request
  {
    size_t off = 0;
    for (uint32_t b = 0; b < nseq; ++b) {
      enqueue_prefill(prompt_dev_ + off, cols[b], b);
      off += cols[b] * cdim;
      enqueue_head(1, hn_ + size_t(b) * s.dim, logits_c_ + size_t(b) * n_cand_, false, nullptr);
      SampleArgs sa{};
      sa.logits = logits_c_ + size_t(b) * n_cand_;
      sa.ids = head_rows_;
      sa.n = n_cand_;
      sa.vocab = s.vocab;
      sa.cfg = cfg;
      sa.st = st_ + b;
      sa.im_end = im_end_;
      sa.after_step = 0;
      sa.num_codebooks = s.num_codebooks;
      sa.n_seq = 1;
      sa.batch = batch_;
      HIPC(launch_sample_slow(sa, stream_));
    }
  }
  HIPC(hipEventRecord(ev[1], stream_));

  // No cap at the KV capacity: a frame that would write past max_seq_len sets
  // ERR_KV_OVERFLOW on the device and the call fails, as SlowArState::eval does
  // (slow_ar.rs:469-474).
  const uint32_t max_frames = p.max_new_tokens;
  // Batched requests: the Slow-AR attention grid spans max_seq_len, and the
  // chunks past every request's prompt read the position before their K/V
  // tile, so chunks past a request's end read nothing (one request keeps
  // every tile load ahead of the position: its attention is bound by
  // latency, not by bytes)
  {
    size_t min_cols = cols[0];
    for (uint32_t b = 1; b < nseq; ++b) min_cols = std::min(min_cols, cols[b]);
    attn_check_from_ = nseq >= ATTN_CHECK_MIN_SEQS ? uint32_t(min_cols / ATTN_CHUNK + 1) : 0u;
  }
  const bool profile = (flags_ & S2HIP_FLAG_PROFILE) != 0;
  bool use_graph = !(flags_ & S2HIP_FLAG_NO_GRAPH) && !profile;
  slow_prof = s2hip_slow_profile{};
  profiling_ = profile;
  prof_kind_.clear();
  uint32_t launched = 0;
  if (max_frames > 0) {
    enqueue_frame(cfg, nseq, ncodes);  // frame 0 eagerly (also configures every kernel)
    prof_book(nseq);
    launched = 1;
  }
  if (use_graph && launched < max_frames) {
    const bool stale = !graph_exec_ || graph_codes_ != codes_dev_ || graph_codes_stride_ != ncodes ||
                       graph_nseq_ != nseq || graph_kv_gen_ != kv_gen_ || graph_bmm_off_ != bmm_off_ ||
                       graph_fold_off_ != fold_off_ || graph_check_from_ != attn_check_from_ ||
                       graph_cfg_.temperature != cfg.temperature ||
                       graph_cfg_.top_p != cfg.top_p || graph_cfg_.top_k != cfg.top_k;
    if (stale) {
      if (graph_exec_) {
        HIPC(hipGraphExecDestroy(graph_exec_));
        graph_exec_ = nullptr;
      }
      if (graph_) {
        HIPC(hipGraphDestroy(graph_));
        graph_ = nullptr;
      }
      HIPC(hipStreamBeginCapture(stream_, hipStreamCaptureModeRelaxed));
      try {
        enqueue_frame(cfg, nseq, ncodes);
      } catch (...) {
        hipGraph_t g = nullptr;
        (void)hipStreamEndCapture(stream_, &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
      }
      HIPC(hipStreamEndCapture(stream_, &graph_));
      HIPC(hipGraphInstantiate(&graph_exec_, graph_, nullptr, nullptr, 0));
      graph_cfg_ = cfg;
      graph_codes_ = codes_dev_;
      graph_codes_stride_ = ncodes;
      graph_nseq_ = nseq;
      graph_kv_gen_ = kv_gen_;
      graph_bmm_off_ = bmm_off_;
      graph_fold_off_ = fold_off_;
      graph_check_from_ = attn_check_from_;
    }
  }
  // Frames in batches; the done flag of batch i is read while batch i+1 runs.
  int pending = -1;
  hipEvent_t flag_ev[2];
  for (auto& e : flag_ev) HIPC(hipEventCreateWithFlags(&e, hipEventDisableTiming));
  int slot = 0;
  bool finished = false;
  while (launched < max_frames && !finished) {
    const uint32_t n = std::min(profile ? 1u : FRAME_BATCH, max_frames - launched);
    for (uint32_t i = 0; i < n; ++i) {
      if (use_graph) {
        HIPC(hipGraphLaunch(graph_exec_, stream_));
      } else {
        enqueue_frame(cfg, nseq, ncodes);
        prof_book(nseq);
      }
    }
    launched += n;
    HIPC(hipMemcpyAsync(&done_host_[slot], &batch_->done_all, 4, hipMemcpyDeviceToHost, stream_));
    HIPC(hipEventRecord(flag_ev[slot], stream_));
    if (pending >= 0) {
      HIPC(hipEventSynchronize(flag_ev[pending]));
      if (done_host_[pending]) finished = true;
    }
    pending = slot;
    slot ^= 1;
  }
  HIPC(hipEventRecord(ev[2], stream_));
  profiling_ = false;
  HIPC(hipMemcpyAsync(st_host_, st_, nseq * sizeof(DevState), hipMemcpyDeviceToHost, stream_));
  HIPC(hipStreamSynchronize(stream_));
  for (auto& e : flag_ev) (void)hipEventDestroy(e);
  float ms_prefill = 0.0f, ms_decode = 0.0f;
  HIPC(hipEventElapsedTime(&ms_prefill, ev[0], ev[1]));
  HIPC(hipEventElapsedTime(&ms_decode, ev[1], ev[2]));
  for (auto& e : ev) (void)hipEventDestroy(e);
  const bool range = !bmm_off_ && any_f16_range(nseq), tie = !fold_off_ && any_err(nseq, ERR_GREEDY_TIE);
  if (range || tie) {
    // An activation beyond the batched product's per-wave range (one more
    // than 2^15 times the largest of the first 256 of its wave's k range),
    // or a tie at the max of a folded greedy sample: the whole call runs
    // again from its inputs (rngs and codes are only written below) with
    // the per-column paths / the sampler kernels.
    const bool bmm0 = bmm_off_, fold0 = fold_off_;
    bmm_off_ = bmm_off_ || range;
    fold_off_ = fold_off_ || tie;
    try {
      generate(nseq, prompts, cols, p, rngs, codes, n_frames, stats);
    } catch (...) {
      bmm_off_ = bmm0;
      fold_off_ = fold0;
      throw;
    }
    bmm_off_ = bmm0;
    fold_off_ = fold0;
    if (stats) {
      stats->per_column_rerun = stats->per_column_rerun || range;
      stats->greedy_rerun = stats->greedy_rerun || tie;
    }
    return;
  }
  check_state_err(nseq);
  std::vector<int32_t> full(ncodes * nseq);
  if (ncodes) HIPC(hipMemcpy(full.data(), codes_dev_, ncodes * nseq * 4, hipMemcpyDeviceToHost));
  uint32_t total = 0;
  for (uint32_t b = 0; b < nseq; ++b) {
    const uint32_t nf = st_host_[b].step_index;
    const int32_t* src = full.data() + size_t(b) * ncodes;
    // compact_codes (generate.rs:346-390): codebook-major [num_codebooks][n_frames]
    for (uint32_t cb = 0; cb < s.num_codebooks; ++cb)
      for (uint32_t t = 0; t < nf; ++t) codes[b][size_t(cb) * nf + t] = src[size_t(cb) * p.max_new_tokens + t];
    n_frames[b] = nf;
    rngs[b] = st_host_[b].rng;
    total += nf;
  }
  for (uint32_t b = 0; b < nseq; ++b) n_past_host[b] = st_host_[b].n_past;  // request b's state is slot b's
  if (stats) {
    stats->prefill_ms = ms_prefill;
    stats->decode_ms = ms_decode;
    stats->n_frames = total;
    stats->graph_used = use_graph ? 1u : 0u;
    stats->per_column_rerun = 0;
    stats->greedy_rerun = 0;
  }
}

// ---------------------------------------------------------------------------
// op level
// ---------------------------------------------------------------------------
namespace {
struct TmpBuf {
  void* p = nullptr;
  TmpBuf(size_t bytes) {
    hip_check(hipMalloc(&p, bytes + WEIGHT_PAD), "hipMalloc");
    count_device_alloc();
  }
  ~TmpBuf() { (void)hipFree(p); }
  template <class T>
  T* as() { return static_cast<T*>(p); }
};
}  // namespace

void Engine::ensure_fast_table() {
  const s2hip_spec& s = spec;
  if (fast_table_ || fast_table_off_ || s.fast_layers == 0) return;
  ensure_tiled();  // the repacked rows decide which one-column kernel the linear takes
  const DevLin& L = fast_[0].wqkv;
  const uint32_t w = (s.fast_heads + 2 * s.fast_kv_heads) * s.fast_head_dim;
  float* tab = dalloc<float>(size_t(s.codebook_size) * w);
  TmpBuf x(size_t(s.codebook_size) * s.dim * 4);
  HIPC(launch_dequant_rows(W_F16, reinterpret_cast<const uint8_t*>(fast_emb_), size_t(s.dim) * 2, s.codebook_size,
                           s.dim, x.as<float>(), stream_));
  // the same one-column call a sub-step makes (enqueue_fast_layers, layer 0)
  for (uint32_t c = 0; c < s.codebook_size; ++c)
    lin(L, nullptr, EPI_STORE, 1, x.as<float>() + size_t(c) * s.dim, s.dim, fast_[0].attn_norm, s.fast_eps,
        tab + size_t(c) * w, w, 0, NO_ROW, L.out, nullptr);
  HIPC(hipStreamSynchronize(stream_));
  fast_table_ = tab;
}

void Engine::op_linear(const void* w, uint32_t type, size_t in, size_t out, const float* x, size_t ncol, float* y) {
  select();
  if (type != W_F16 && type != W_Q8_0 && type != W_Q4_0) fail("unsupported weight type");
  if (in == 0 || out == 0 || ncol == 0) fail("empty linear");
  const size_t rb = size_t(ggml_row_bytes(type, in));
  TmpBuf dw(rb * out), dx(in * ncol * 4), dy(out * ncol * 4);
  HIPC(hipMemsetAsync(dw.as<uint8_t>() + rb * out, 0, WEIGHT_PAD, stream_));
  HIPC(hipMemcpyAsync(dw.p, w, rb * out, hipMemcpyHostToDevice, stream_));
  HIPC(hipMemcpyAsync(dx.p, x, in * ncol * 4, hipMemcpyHostToDevice, stream_));
  DevLin L;
  L.w = dw.as<uint8_t>();
  L.type = type;
  L.in = uint32_t(in);
  L.out = uint32_t(out);
  L.row_bytes = rb;
  const bool batched = bmm_min_cols_ && ncol >= bmm_min_cols_ && in % 256 == 0 && in <= BMM_MAX_K;
  if (batched && type == W_F16) {  // batched-decode product on a tiled copy
    TmpBuf dt(size_t(bmm_rows_pad(uint32_t(out))) * in * 2), derr(4);
    L.wt = dt.as<_Float16>();
    HIPC(launch_tile_f16(reinterpret_cast<const uint16_t*>(L.w), uint32_t(in), uint32_t(out), 0, NO_ROW,
                         reinterpret_cast<uint16_t*>(L.wt), stream_));
    HIPC(hipMemsetAsync(derr.p, 0, 4, stream_));
    bmm(L, nullptr, EPI_STORE, uint32_t(ncol), dx.as<float>(), uint32_t(in), nullptr, 0.0f, dy.as<float>(),
        uint32_t(out), nullptr, derr.as<uint32_t>());
    uint32_t herr = 0;
    HIPC(hipMemcpyAsync(y, dy.p, out * ncol * 4, hipMemcpyDeviceToHost, stream_));
    HIPC(hipMemcpyAsync(&herr, derr.p, 4, hipMemcpyDeviceToHost, stream_));
    HIPC(hipStreamSynchronize(stream_));
    if (!(herr & ERR_F16_RANGE)) return;
    for (size_t i = 0; i < in * ncol; ++i)
      if (!std::isfinite(x[i])) fail("activation not finite or beyond the range of the batched product");
    // finite but beyond the per-wave range: the per-column paths below
    // (whole-row scale) give the product
  }
  // quantized rows: the repacked planes that one-column decode GEMVs read
  std::unique_ptr<TmpBuf> dq, dsc;
  if (const uint32_t qb = repack_quant_bytes(type); qb && in % 32 == 0) {
    const size_t nblk = in / 32 * out;
    dq = std::make_unique<TmpBuf>(nblk * qb);
    dsc = std::make_unique<TmpBuf>(nblk * 2);
    L.qp = dq->as<uint8_t>();
    L.qs = dsc->as<uint16_t>();
    HIPC(launch_repack_q(L.w, rb, type, uint32_t(in), uint32_t(out), L.qp, L.qs, stream_));
  }
  if (ncol >= 3 && ncol <= 16 && in % 256 == 0)  // batched-decode product (quantized rows)
    mm_skinny(L, nullptr, EPI_STORE, dx.as<float>(), uint32_t(in), nullptr, 0.0f, uint32_t(ncol), dy.as<float>(),
              uint32_t(out), 0, NO_ROW, uint32_t(out), nullptr);
  else
    gemv(L, nullptr, EPI_STORE, uint32_t(ncol), dx.as<float>(), uint32_t(in), nullptr, 0.0f, dy.as<float>(),
         uint32_t(out), 0, NO_ROW, uint32_t(out), nullptr);
  HIPC(hipMemcpyAsync(y, dy.p, out * ncol * 4, hipMemcpyDeviceToHost, stream_));
  HIPC(hipStreamSynchronize(stream_));
}

void Engine::op_rms_norm(const float* x, const float* w, size_t n, size_t ncol, float eps, float* y) {
  select();
  if (n == 0) fail("rms_norm input is empty");
  TmpBuf dx(n * ncol * 4), dw(n * 4), dy(n * ncol * 4);
  HIPC(hipMemcpyAsync(dx.p, x, n * ncol * 4, hipMemcpyHostToDevice, stream_));
  HIPC(hipMemcpyAsync(dw.p, w, n * 4, hipMemcpyHostToDevice, stream_));
  HIPC(launch_rms_norm(dx.as<float>(), dw.as<float>(), dy.as<float>(), uint32_t(n), uint32_t(ncol), eps, nullptr,
                       stream_));
  HIPC(hipMemcpyAsync(y, dy.p, n * ncol * 4, hipMemcpyDeviceToHost, stream_));
  HIPC(hipStreamSynchronize(stream_));
}

void Engine::op_dequant(const void* w, uint32_t type, size_t in, size_t rows, float* out) {
  select();
  if (type != W_F16 && type != W_Q8_0 && type != W_Q4_0) fail("unsupported weight type");
  const size_t rb = size_t(ggml_row_bytes(type, in));
  TmpBuf dw(rb * rows), dy(in * rows * 4);
  HIPC(hipMemsetAsync(dw.as<uint8_t>() + rb * rows, 0, WEIGHT_PAD, stream_));
  HIPC(hipMemcpyAsync(dw.p, w, rb * rows, hipMemcpyHostToDevice, stream_));
  HIPC(launch_dequant_rows(type, dw.as<uint8_t>(), rb, uint32_t(rows), uint32_t(in), dy.as<float>(), stream_));
  HIPC(hipMemcpyAsync(out, dy.p, in * rows * 4, hipMemcpyDeviceToHost, stream_));
  HIPC(hipStreamSynchronize(stream_));
}

void Engine::op_qk_rope(const float* qkv, uint32_t H, uint32_t Hkv, uint32_t hd, uint32_t pos, float base,
                        const float* qn, const float* kn, float eps, float* q, float* k, float* v) {
  select();
  if (Hkv == 0 || H % Hkv || hd == 0 || hd % 2 || hd > 256) fail("invalid attention shape");
  const size_t width = size_t(H + 2 * Hkv) * hd;
  TmpBuf dqkv(width * 4), dq(size_t(H) * hd * 4), dk(size_t(Hkv) * hd * 4), dv(size_t(Hkv) * hd * 4),
      dqn(hd * 4), dkn(hd * 4), drope(size_t(pos + 1) * (hd / 2) * sizeof(float2));
  HIPC(hipMemcpyAsync(dqkv.p, qkv, width * 4, hipMemcpyHostToDevice, stream_));
  if (qn) HIPC(hipMemcpyAsync(dqn.p, qn, hd * 4, hipMemcpyHostToDevice, stream_));
  if (kn) HIPC(hipMemcpyAsync(dkn.p, kn, hd * 4, hipMemcpyHostToDevice, stream_));
  HIPC(hipStreamSynchronize(stream_));
  build_rope(drope.as<float2>(), pos + 1, hd, base);
  QkvPostArgs pa{};
  pa.qkv = dqkv.as<float>();
  pa.q_out = dq.as<float>();
  pa.k_cache = dk.as<float>();  // max_seq = 1: the cache row is the output
  pa.v_cache = dv.as<float>();
  pa.q_norm = qn ? dqn.as<float>() : nullptr;
  pa.k_norm = kn ? dkn.as<float>() : nullptr;
  pa.rope = drope.as<float2>() + size_t(pos) * (hd / 2);
  pa.pos_ptr = nullptr;
  pa.pos_offset = 0;
  pa.H = H;
  pa.Hkv = Hkv;
  pa.hd = hd;
  pa.max_seq = 1;
  pa.ncol = 1;
  pa.eps = eps;
  HIPC(launch_qkv_post(pa, stream_));
  HIPC(hipMemcpyAsync(q, dq.p, size_t(H) * hd * 4, hipMemcpyDeviceToHost, stream_));
  HIPC(hipMemcpyAsync(k, dk.p, size_t(Hkv) * hd * 4, hipMemcpyDeviceToHost, stream_));
  HIPC(hipMemcpyAsync(v, dv.p, size_t(Hkv) * hd * 4, hipMemcpyDeviceToHost, stream_));
  HIPC(hipStreamSynchronize(stream_));
}

// gqa_decode_attention through the fused decode kernel: the last token's
// k/v and the query travel in a qkv row (no QK-norm, identity rotation),
// earlier tokens come from the cache.
void Engine::op_attention(const float* q, const float* k, const float* v, uint32_t H, uint32_t Hkv, uint32_t hd,
                          uint32_t T, float scale, float* out) {
  select();
  if (Hkv == 0 || H % Hkv) fail("invalid GQA split");
  if (T == 0) fail("invalid attention dims");
  if ((hd != 64 && hd != 128) || H / Hkv > 4) fail("attention shape not supported on the device");
  // reference layout [token][kv_head][hd] -> cache layout [kv_head][token][hd]
  std::vector<float> kc(size_t(Hkv) * T * hd), vc(kc.size());
  for (uint32_t t = 0; t < T; ++t)
    for (uint32_t g = 0; g < Hkv; ++g)
      for (uint32_t d = 0; d < hd; ++d) {
        kc[(size_t(g) * T + t) * hd + d] = k[(size_t(t) * Hkv + g) * hd + d];
        vc[(size_t(g) * T + t) * hd + d] = v[(size_t(t) * Hkv + g) * hd + d];
      }
  const size_t width = size_t(H + 2 * Hkv) * hd;
  std::vector<float> row(width);
  memcpy(row.data(), q, size_t(H) * hd * 4);
  memcpy(row.data() + size_t(H) * hd, k + size_t(T - 1) * Hkv * hd, size_t(Hkv) * hd * 4);
  memcpy(row.data() + size_t(H + Hkv) * hd, v + size_t(T - 1) * Hkv * hd, size_t(Hkv) * hd * 4);
  std::vector<float2> rope(size_t(T) * (hd / 2), make_float2(1.0f, 0.0f));
  const uint32_t nch = attention_chunks(T, attn_mode_);
  TmpBuf drow(width * 4), dk(kc.size() * 4), dv(vc.size() * 4), dpart(size_t(Hkv) * nch * (H / Hkv) * (hd + 2) * 4),
      dout(size_t(H) * hd * 4), drope(rope.size() * sizeof(float2)), dctr(size_t(Hkv) * 4);
  HIPC(hipMemcpyAsync(drow.p, row.data(), width * 4, hipMemcpyHostToDevice, stream_));
  HIPC(hipMemcpyAsync(dk.p, kc.data(), kc.size() * 4, hipMemcpyHostToDevice, stream_));
  HIPC(hipMemcpyAsync(dv.p, vc.data(), vc.size() * 4, hipMemcpyHostToDevice, stream_));
  HIPC(hipMemcpyAsync(drope.p, rope.data(), rope.size() * sizeof(float2), hipMemcpyHostToDevice, stream_));
  HIPC(hipMemsetAsync(dctr.p, 0, size_t(Hkv) * 4, stream_));
  AttnArgs aa{};
  aa.qkv = drow.as<float>();
  aa.eps = 0.0f;
  aa.rope = drope.as<float2>();
  aa.k_cache = dk.as<float>();
  aa.v_cache = dv.as<float>();
  aa.part = dpart.as<float>();
  aa.counters = dctr.as<uint32_t>();
  aa.out = dout.as<float>();
  aa.pos_ptr = nullptr;
  aa.pos_offset = T - 1;
  aa.H = H;
  aa.Hkv = Hkv;
  aa.hd = hd;
  aa.max_seq = T;
  aa.ncol = 1;
  aa.max_chunks = nch;
  aa.mode = attn_mode_;
  aa.scale = scale;
  HIPC(launch_attention(aa, stream_));
  HIPC(hipMemcpyAsync(out, dout.p, size_t(H) * hd * 4, hipMemcpyDeviceToHost, stream_));
  HIPC(hipStreamSynchronize(stream_));
}

void Engine::op_swiglu(const float* g, const float* u, size_t n, int fast, float* out) {
  select();
  if (n == 0) return;
  TmpBuf dg(n * 4), du(n * 4), dy(n * 4);
  HIPC(hipMemcpyAsync(dg.p, g, n * 4, hipMemcpyHostToDevice, stream_));
  HIPC(hipMemcpyAsync(du.p, u, n * 4, hipMemcpyHostToDevice, stream_));
  HIPC(launch_swiglu(dg.as<float>(), du.as<float>(), dy.as<float>(), uint32_t(n), fast, stream_));
  HIPC(hipMemcpyAsync(out, dy.p, n * 4, hipMemcpyDeviceToHost, stream_));
  HIPC(hipStreamSynchronize(stream_));
}

void Engine::op_running_sums(const float* terms, size_t n, float* prefix, float* total) {
  select();
  if (n == 0) {
    *total = 0.0f;
    return;
  }
  if (n > 8192) fail("running sums support at most 8192 terms on the device");
  TmpBuf dt(n * 4), dp(n * 4), ds(4);
  HIPC(hipMemcpyAsync(dt.p, terms, n * 4, hipMemcpyHostToDevice, stream_));
  HIPC(launch_running_sum(dt.as<float>(), uint32_t(n), dp.as<float>(), ds.as<float>(), stream_));
  HIPC(hipMemcpyAsync(prefix, dp.p, n * 4, hipMemcpyDeviceToHost, stream_));
  HIPC(hipMemcpyAsync(total, ds.p, 4, hipMemcpyDeviceToHost, stream_));
  HIPC(hipStreamSynchronize(stream_));
}

void Engine::op_running_cut(const float* terms, size_t n, float thr, bool absorb, size_t at, size_t* cut, float* sum,
                            float* at_sum) {
  select();
  if (n > 8192) fail("running sums support at most 8192 terms on the device");
  for (size_t i = 0; i < n; ++i)
    if (!(terms[i] >= 0.0f)) fail("the cut search needs non-negative terms");
  if (absorb)
    for (size_t i = 1; i < n; ++i)
      if (terms[i] > terms[i - 1]) fail("absorb needs non-increasing terms");
  TmpBuf dt(n ? n * 4 : 4), dc(4), ds(8);
  if (n) HIPC(hipMemcpyAsync(dt.p, terms, n * 4, hipMemcpyHostToDevice, stream_));
  const uint32_t at32 = at < n ? uint32_t(at) : 0xffffffffu;
  HIPC(launch_running_cut(dt.as<float>(), uint32_t(n), thr, absorb ? 1u : 0u, at32, dc.as<uint32_t>(), ds.as<float>(),
                          stream_));
  uint32_t c = 0;
  float sums[2] = {0.0f, 0.0f};
  HIPC(hipMemcpyAsync(&c, dc.p, 4, hipMemcpyDeviceToHost, stream_));
  HIPC(hipMemcpyAsync(sums, ds.p, 8, hipMemcpyDeviceToHost, stream_));
  HIPC(hipStreamSynchronize(stream_));
  *cut = c;
  *sum = sums[0];
  *at_sum = at < n ? sums[1] : 0.0f;
}

void Engine::op_embed(const int32_t* flat, size_t n_tok, float* out) {
  select();
  const s2hip_spec& s = spec;
  const uint32_t cdim = s.num_codebooks + 1;
  if (n_tok == 0) return;
  if (n_tok > 65535) fail("embed supports at most 65535 tokens per call");
  validate_tokens(flat, n_tok);
  TmpBuf dt(n_tok * cdim * 4), dh(n_tok * s.dim * 4), de(4);
  HIPC(hipMemcpyAsync(dt.p, flat, n_tok * cdim * 4, hipMemcpyHostToDevice, stream_));
  HIPC(hipMemsetAsync(de.p, 0, 4, stream_));
  EmbedArgs ea{};
  ea.tokens = dt.as<int32_t>();
  ea.emb = emb_;
  ea.cb_emb = cb_emb_;
  ea.h = dh.as<float>();
  ea.n = uint32_t(n_tok);
  ea.dim = s.dim;
  ea.vocab = s.vocab;
  ea.cb_rows = uint32_t(cb_rows_);
  ea.num_codebooks = s.num_codebooks;
  ea.codebook_size = s.codebook_size;
  ea.sem_begin = s.semantic_begin;
  ea.sem_end = s.semantic_end;
  ea.sem_scale = 1.0f / std::sqrt(float(s.num_codebooks + 1));  // scale_codebook_embeddings (registry.rs:94-97)
  ea.scale_enabled = s.scale_codebook_embeddings;
  ea.err = de.as<uint32_t>();
  HIPC(launch_embed(ea, stream_));
  uint32_t e = 0;
  HIPC(hipMemcpyAsync(out, dh.p, n_tok * s.dim * 4, hipMemcpyDeviceToHost, stream_));
  HIPC(hipMemcpyAsync(&e, de.p, 4, hipMemcpyDeviceToHost, stream_));
  HIPC(hipStreamSynchronize(stream_));
  if (e) fail("token id out of range");
}

void Engine::op_expf(const float* x, size_t n, float* y) {
  select();
  if (n == 0) return;
  TmpBuf dx(n * 4), dy(n * 4);
  HIPC(hipMemcpyAsync(dx.p, x, n * 4, hipMemcpyHostToDevice, stream_));
  HIPC(launch_expf(dx.as<float>(), dy.as<float>(), n, stream_));
  HIPC(hipMemcpyAsync(y, dy.p, n * 4, hipMemcpyDeviceToHost, stream_));
  HIPC(hipStreamSynchronize(stream_));
}

void Engine::op_sample(const float* logits, size_t n, const s2hip_sampler& smp, int64_t always, uint64_t* rng,
                       uint32_t* tok) {
  select();
  if (n == 0) {
    *tok = 0;
    return;
  }
  if (n > 8191) fail("sample_token supports at most 8191 logits on the device");
  TmpBuf dl(n * 4), dr(8), dt(4), de(4);
  HIPC(hipMemcpyAsync(dl.p, logits, n * 4, hipMemcpyHostToDevice, stream_));
  HIPC(hipMemcpyAsync(dr.p, rng, 8, hipMemcpyHostToDevice, stream_));
  HIPC(hipMemsetAsync(de.p, 0, 4, stream_));
  HIPC(launch_sample_plain(dl.as<float>(), uint32_t(n), SamplerCfg{smp.temperature, smp.top_p, smp.top_k}, always,
                           dr.as<uint64_t>(), dt.as<uint32_t>(), de.as<uint32_t>(), stream_));
  uint32_t e = 0;
  HIPC(hipMemcpyAsync(rng, dr.p, 8, hipMemcpyDeviceToHost, stream_));
  HIPC(hipMemcpyAsync(tok, dt.p, 4, hipMemcpyDeviceToHost, stream_));
  HIPC(hipMemcpyAsync(&e, de.p, 4, hipMemcpyDeviceToHost, stream_));
  HIPC(hipStreamSynchronize(stream_));
  if (e) fail("sampler failure");
}

// op_sample with no device allocation: the logits and the state words are
// staged in this device's `scratch` (the state words copied in whole, so the
// token and error words start at zero without a memset).
void Engine::op_sample_noalloc(const float* logits, size_t n, const s2hip_sampler& smp, int64_t always,
                               uint64_t* rng, uint32_t* tok) {
  select();
  if (n == 0) {
    *tok = 0;
    return;
  }
  if (n > NOALLOC_MAX_LOGITS)
    fail("sample_token without allocation supports at most " + std::to_string(NOALLOC_MAX_LOGITS) + " logits, got " +
         std::to_string(n));
  if (!scratch_dev_) fail("scratch buffer not set up");
  float* dl = reinterpret_cast<float*>(scratch_dev_);
  NoallocState* ds = reinterpret_cast<NoallocState*>(scratch_dev_ + NOALLOC_STATE_OFF);
  NoallocState hs{*rng, 0u, 0u};
  HIPC(hipMemcpyAsync(dl, logits, n * 4, hipMemcpyHostToDevice, stream_));
  HIPC(hipMemcpyAsync(ds, &hs, sizeof(hs), hipMemcpyHostToDevice, stream_));
  HIPC(launch_sample_plain(dl, uint32_t(n), SamplerCfg{smp.temperature, smp.top_p, smp.top_k}, always, &ds->rng,
                           &ds->token, &ds->err, stream_));
  HIPC(hipMemcpyAsync(&hs, ds, sizeof(hs), hipMemcpyDeviceToHost, stream_));
  HIPC(hipStreamSynchronize(stream_));
  if (hs.err) fail("sampler failure");
  *rng = hs.rng;
  *tok = hs.token;
}

void Engine::time_kernel(const std::string& full_name, uint32_t reps, double* avg_us, double* bytes) {
  select();
  const s2hip_spec& s = spec;
  if (reps == 0) reps = 1;
  // "<name>_b<N>": the Slow-AR linears over N columns (a decode batch of N)
  // by the engine's routing; "<name>_s<N>": the skinny MFMA product for N
  // columns whatever N is; "<name>_g<N>": the GEMV kernels for N columns;
  // "<name>_t<N>[w<W>]": the batched product (W waves per block)
  std::string name = full_name;
  uint32_t ncol = 1, waves = 0;
  char force = 'b';
  {
    const size_t at = full_name.rfind('_');
    if (full_name.rfind("slow_w", 0) == 0 && at != std::string::npos && at + 2 < full_name.size() &&
        std::string("bsgt").find(full_name[at + 1]) != std::string::npos) {
      const std::string arg = full_name.substr(at + 2);
      const size_t wpos = arg.find('w');
      const std::string cols = arg.substr(0, wpos), wv = wpos == std::string::npos ? "" : arg.substr(wpos + 1);
      const bool ok = !cols.empty() && cols.find_first_not_of("0123456789") == std::string::npos &&
                      wv.find_first_not_of("0123456789") == std::string::npos &&
                      (wpos == std::string::npos || (!wv.empty() && full_name[at + 1] == 't'));
      if (ok) {
        ncol = uint32_t(std::stoul(cols));
        waves = wv.empty() ? 0u : uint32_t(std::stoul(wv));
        force = full_name[at + 1];
        name = full_name.substr(0, at);
        if (ncol == 0 || ncol > MAX_SEQS) fail("batch columns out of range in " + full_name);
      }
    }
  }
  if (force == 't') {
    ensure_tiled();
    if (!tiled_) fail("the batched product is disabled");
  }
  auto tlin = [&](const DevLin& L, const DevLin* L3, int epi, const float* x, uint32_t ldx, const float* norm,
                  float eps, float* y, uint32_t ldy) {
    if (force == 's') {
      if (L.in % 256) fail("skinny product needs in % 256 == 0");
      mm_skinny(L, L3, epi, x, ldx, norm, eps, ncol, y, ldy, 0, NO_ROW, L.out, nullptr);
    } else if (force == 'g') {
      gemv(L, L3, epi, ncol, x, ldx, norm, eps, y, ldy, 0, NO_ROW, L.out, nullptr);
    } else if (force == 't') {
      if (!L.wt) fail("no batched-product copy of this matrix (F16 with in % 256 == 0 only)");
      bmm(L, L3, epi, ncol, x, ldx, norm, eps, y, ldy, nullptr, &st_->err, waves);
    } else {
      lin(L, L3, epi, ncol, x, ldx, norm, eps, y, ldy, 0, NO_ROW, L.out, nullptr);
    }
  };
  const uint32_t q = s.heads * s.head_dim, kv = s.kv_heads * s.head_dim;
  // activations: pseudo-random values in [-1, 1] (what the decode feeds the
  // kernels; all-zero operands would let the MFMA kernels run cooler)
  auto fill = [&](float* dst, size_t count, uint64_t seed) {
    std::vector<float> v(count);
    uint64_t z = seed * 0x9E3779B97F4A7C15ull + 1;
    for (float& f : v) {
      z = z * 6364136223846793005ull + 1442695040888963407ull;
      f = float(int64_t(z >> 40) % 2001 - 1000) * 1e-3f;
    }
    HIPC(hipMemcpyAsync(dst, v.data(), count * 4, hipMemcpyHostToDevice, stream_));
    HIPC(hipStreamSynchronize(stream_));
  };
  fill(h_, size_t(MAX_SEQS) * s.dim, 1);
  fill(att_, size_t(MAX_SEQS) * q, 2);
  fill(act_, size_t(MAX_SEQS) * s.ffn, 3);
  // hbm_copy: a 256 MiB device-to-device copy (counter calibration)
  constexpr size_t COPY_BYTES = size_t(256) << 20;
  std::unique_ptr<TmpBuf> copy_a, copy_b;
  void *copy_src = nullptr, *copy_dst = nullptr;
  if (name == "hbm_copy") {
    copy_a.reset(new TmpBuf(COPY_BYTES));
    copy_b.reset(new TmpBuf(COPY_BYTES));
    copy_src = copy_a->p;
    copy_dst = copy_b->p;
    HIPC(hipMemsetAsync(copy_src, 0, COPY_BYTES, stream_));
  }
  auto pass = [&](uint32_t l) {
    const SlowLayer& L = slow_[l];
    if (name == "slow_w13")
      tlin(L.w1, &L.w3, EPI_SWIGLU_SLOW, h_, s.dim, L.ffn_norm, s.eps, act_, s.ffn);
    else if (name == "slow_wqkv")
      tlin(L.wqkv, nullptr, EPI_STORE, h_, s.dim, L.attn_norm, s.eps, qkv_, q + 2 * kv);
    else if (name == "slow_wo")
      tlin(L.wo, nullptr, EPI_STORE, att_, q, nullptr, 0.0f, h_, s.dim);
    else if (name == "slow_w2")
      tlin(L.w2, nullptr, EPI_STORE, act_, s.ffn, nullptr, 0.0f, qkv_, s.dim);
    else if (name == "slow_attn" || name == "fast_attn") {
      const bool fast = name == "fast_attn";
      AttnArgs aa{};
      aa.qkv = fast ? fqkv_ : qkv_;
      aa.q_norm = fast ? nullptr : L.q_norm;
      aa.k_norm = fast ? nullptr : L.k_norm;
      aa.eps = s.eps;
      aa.rope = fast ? rope_fast_ : rope_slow_;
      const uint32_t kvw = fast ? s.fast_kv_heads * s.fast_head_dim : kv;
      aa.k_cache = fast ? fkc_ + size_t(l % s.fast_layers) * kvw * fctx_ : kvp(kc_, size_t(l) * kv * s.max_seq_len);
      aa.v_cache = fast ? fvc_ + size_t(l % s.fast_layers) * kvw * fctx_ : kvp(vc_, size_t(l) * kv * s.max_seq_len);
      aa.kv_f16 = fast ? 0u : kv_f16_;
      aa.part = fast ? fpart_ : part_;
      aa.counters = counters_;
      aa.out = fast ? fatt_ : att_;
      aa.pos_ptr = nullptr;
      aa.pos_offset = fast ? 5u : std::min(s.max_seq_len - 1, 383u);
      aa.H = fast ? s.fast_heads : s.heads;
      aa.Hkv = fast ? s.fast_kv_heads : s.kv_heads;
      aa.hd = fast ? s.fast_head_dim : s.head_dim;
      aa.max_seq = fast ? fctx_ : s.max_seq_len;
      aa.ncol = 1;
      aa.max_chunks = fast ? attention_chunks(fctx_, attn_mode_) : attn_chunks_;
      aa.mode = attn_mode_;
      aa.scale = 0.08838834764831845f;
      HIPC(launch_attention(aa, stream_));
    } else if (name.rfind("sample_fast", 0) == 0 || name.rfind("sample_slow", 0) == 0) {
      SampleArgs sa{};
      const bool fast = name.rfind("sample_fast", 0) == 0;
      sa.logits = fast ? flogits_ : logits_c_;
      sa.ids = fast ? nullptr : head_rows_;
      sa.n = fast ? s.codebook_size : n_cand_;
      sa.vocab = fast ? s.codebook_size : s.vocab;
      // greedy; "_topp": T 0.7, top-p 0.9; "_default": GenerateParams::default()
      // (generate.rs:22-31: T 0.7, top-p 0.7, top-k 30)
      sa.cfg = SamplerCfg{0.0f, 1.0f, 0};
      if (name.find("_topp") != std::string::npos) sa.cfg = SamplerCfg{0.7f, 0.9f, 0};
      if (name.find("_default") != std::string::npos) sa.cfg = SamplerCfg{0.7f, 0.7f, 30};
      sa.st = st_;
      sa.im_end = im_end_;
      sa.cb_index = 1;
      sa.fast_emb = fast_emb_;
      sa.next_input = fast ? fh_ : nullptr;
      sa.dim = s.dim;
      sa.num_codebooks = s.num_codebooks;
      HIPC(fast ? launch_sample_fast(sa, stream_) : launch_sample_slow(sa, stream_));
    } else if (name == "fast_head") {
      gemv(fast_out_, nullptr, EPI_STORE, 1, fh_, s.dim, fast_norm_, s.fast_eps, flogits_, s.codebook_size, 0, NO_ROW,
           s.codebook_size, nullptr);
    } else if (name == "fast_frame") {
      enqueue_fast_frame(SamplerCfg{0.0f, 1.0f, 0}, 1, nullptr);
    } else if (name == "empty") {
      HIPC(launch_add_position(st_, 0, 1, stream_));
    } else if (name == "hbm_copy") {
      HIPC(launch_copy(copy_src, copy_dst, COPY_BYTES, stream_));
    }
    else if (name == "slow_head")
      gemv(head_full_, nullptr, EPI_STORE, 1, hn_, s.dim, nullptr, 0.0f, logits_c_, n_cand_, s.semantic_begin, head_extra_,
           n_cand_,
           nullptr);
    else
      fail("unknown kernel name " + name);
  };
  double b = 0;
  const SlowLayer& L0 = slow_[0];
  if (name == "slow_w13") b = double(L0.w1.bytes + L0.w3.bytes) + 4.0 * ncol * (s.dim + s.ffn) + 4.0 * s.dim;
  else if (name == "slow_wqkv") b = double(L0.wqkv.bytes) + 4.0 * ncol * (s.dim + q + 2 * kv) + 4.0 * s.dim;
  else if (name == "slow_wo") b = double(L0.wo.bytes) + 4.0 * ncol * (q + s.dim);
  else if (name == "slow_w2") b = double(L0.w2.bytes) + 4.0 * ncol * (s.ffn + s.dim);
  else if (name == "slow_head") b = double(n_cand_) * s.dim * 2 + 4.0 * (s.dim + n_cand_);
  else if (name == "hbm_copy") b = 2.0 * double(COPY_BYTES);
  const bool per_layer = name.rfind("slow_", 0) == 0 && name != "slow_head" && name != "sample_slow";
  const uint32_t layers = per_layer || name == "fast_attn" ? s.slow_layers : 1u;
  if (name == "fast_frame" || name.rfind("sample_", 0) == 0 || name == "empty") {
    // a clean state: nothing finished, frame counters at zero
    HIPC(hipStreamSynchronize(stream_));
    DevState init{};
    init.max_new = 1u << 30;
    init.min_tokens_before_end = 1u << 30;
    *st_host_ = init;
    HIPC(hipMemcpyAsync(st_, st_host_, sizeof(DevState), hipMemcpyHostToDevice, stream_));
    HIPC(hipMemsetAsync(hn_, 0, size_t(s.dim) * 4, stream_));
    // distinct pseudo-random logits (the greedy path of a real frame)
    std::vector<float> rl(std::max<size_t>(s.codebook_size, n_cand_));
    uint64_t z = 0x9E3779B97F4A7C15ull;
    for (float& v : rl) {
      z = z * 6364136223846793005ull + 1442695040888963407ull;
      v = float(int64_t(z >> 11) % 2000003) * 1e-6f;
    }
    HIPC(hipMemcpy(flogits_, rl.data(), size_t(s.codebook_size) * 4, hipMemcpyHostToDevice));
    HIPC(hipMemcpy(logits_c_, rl.data(), size_t(n_cand_) * 4, hipMemcpyHostToDevice));
    HIPC(hipMemsetAsync(fh_, 0, 2 * size_t(s.dim) * 4, stream_));
  }
  if (name == "slow_attn" || name == "fast_attn") {
    fill(qkv_, size_t(PREFILL_COLS) * (q + 2 * kv), 4);
    fill(fqkv_, 2 * size_t(s.fast_heads + 2 * s.fast_kv_heads) * s.fast_head_dim, 5);
  }
  for (uint32_t l = 0; l < layers; ++l) pass(l);  // warm-up
  hipEvent_t e0, e1;
  HIPC(hipEventCreate(&e0));
  HIPC(hipEventCreate(&e1));
  HIPC(hipEventRecord(e0, stream_));
  for (uint32_t r = 0; r < reps; ++r)
    for (uint32_t l = 0; l < layers; ++l) pass(l);
  HIPC(hipEventRecord(e1, stream_));
  HIPC(hipEventSynchronize(e1));
  float ms = 0.0f;
  HIPC(hipEventElapsedTime(&ms, e0, e1));
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  *avg_us = double(ms) * 1000.0 / double(reps * layers);
  *bytes = b;
}

}  // namespace s2

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
struct s2hip_engine {
  std::unique_ptr<s2::Engine> e;
};

namespace {
void set_err(char* err, size_t cap, const char* msg) {
  if (err && cap) snprintf(err, cap, "%s", msg);
}

template <class F>
int32_t guarded(char* err, size_t cap, F&& f) {
  try {
    f();
    return 1;
  } catch (const std::exception& ex) {
    set_err(err, cap, ex.what());
    return 0;
  } catch (...) {
    set_err(err, cap, "unknown error");
    return 0;
  }
}
}  // namespace

extern "C" {

const char* s2hip_version(void) { return "s2hip 0.1.0 (gfx950)"; }

s2hip_engine* s2hip_create(const s2hip_config* cfg, char* err, size_t err_cap) {
  if (!cfg) {
    set_err(err, err_cap, "config is NULL");
    return nullptr;
  }
  s2hip_engine* h = nullptr;
  guarded(err, err_cap, [&] {
    std::unique_ptr<s2hip_engine> tmp(new s2hip_engine());
    tmp->e.reset(new s2::Engine(*cfg));
    h = tmp.release();
  });
  return h;
}

void s2hip_destroy(s2hip_engine* engine) { delete engine; }

int32_t s2hip_get_spec(const s2hip_engine* engine, s2hip_spec* out) {
  if (!engine || !out) return 0;
  *out = engine->e->spec;
  return 1;
}

int32_t s2hip_reset(s2hip_engine* engine, char* err, size_t err_cap) {
  if (!engine) {
    set_err(err, err_cap, "NULL argument");
    return 0;
  }
  return guarded(err, err_cap, [&] { engine->e->reset(); });
}

uint32_t s2hip_n_past(const s2hip_engine* engine) { return engine ? engine->e->n_past_host[0] : 0u; }

int32_t s2hip_last_slow_profile(const s2hip_engine* engine, s2hip_slow_profile* out) {
  if (!engine || !out) return 0;
  *out = engine->e->slow_prof;
  return 1;
}

int32_t s2hip_reset_slot(s2hip_engine* engine, uint32_t slot, char* err, size_t err_cap) {
  if (!engine) {
    set_err(err, err_cap, "NULL argument");
    return 0;
  }
  return guarded(err, err_cap, [&] { engine->e->reset(slot); });
}

uint32_t s2hip_n_past_slot(const s2hip_engine* engine, uint32_t slot) {
  return engine && slot < 16 ? engine->e->n_past_host[slot] : 0u;
}

int32_t s2hip_eval_slot(s2hip_engine* engine, uint32_t slot, const int32_t* flat, size_t n_tokens, float* hidden_out,
                        float* logits_out, char* err, size_t err_cap) {
  if (!engine || !flat || !hidden_out) {
    set_err(err, err_cap, "NULL argument");
    return 0;
  }
  return guarded(err, err_cap, [&] { engine->e->eval(flat, n_tokens, hidden_out, logits_out, slot); });
}

int32_t s2hip_op_embed(s2hip_engine* engine, const int32_t* flat, size_t n_tokens, float* out, char* err,
                       size_t err_cap) {
  if (!engine || (n_tokens && (!flat || !out))) {
    set_err(err, err_cap, "NULL argument");
    return 0;
  }
  return guarded(err, err_cap, [&] { engine->e->op_embed(flat, n_tokens, out); });
}

int32_t s2hip_eval(s2hip_engine* engine, const int32_t* flat, size_t n_tokens, float* hidden_out, float* logits_out,
                   char* err, size_t err_cap) {
  if (!engine || !flat || !hidden_out) {
    set_err(err, err_cap, "NULL argument");
    return 0;
  }
  return guarded(err, err_cap, [&] { engine->e->eval(flat, n_tokens, hidden_out, logits_out); });
}

int32_t s2hip_fast_logits(s2hip_engine* engine, const float* hidden, const uint32_t* prefix, size_t plen,
                          float* logits, char* err, size_t err_cap) {
  if (!engine || !hidden || !logits || (plen && !prefix)) {
    set_err(err, err_cap, "NULL argument");
    return 0;
  }
  return guarded(err, err_cap, [&] { engine->e->fast_logits(hidden, prefix, plen, logits); });
}

int32_t s2hip_fast_codebooks(s2hip_engine* engine, const float* hidden, uint32_t sem, const s2hip_sampler* smp,
                             uint64_t* rng, uint32_t* codes, char* err, size_t err_cap) {
  if (!engine || !hidden || !smp || !rng || !codes) {
    set_err(err, err_cap, "NULL argument");
    return 0;
  }
  return guarded(err, err_cap, [&] { engine->e->fast_codebooks(hidden, sem, *smp, rng, codes); });
}

int32_t s2hip_generate_codes(s2hip_engine* engine, const int32_t* prompt, size_t cols, const s2hip_gen_params* p,
                             uint64_t* rng, int32_t* codes, uint32_t* n_frames, s2hip_gen_stats* stats, char* err,
                             size_t err_cap) {
  if (!engine || !prompt || !p || !rng || !codes || !n_frames) {
    set_err(err, err_cap, "NULL argument");
    return 0;
  }
  return guarded(err, err_cap, [&] { engine->e->generate(1, &prompt, &cols, *p, rng, &codes, n_frames, stats); });
}

int32_t s2hip_generate_codes_batch(s2hip_engine* engine, uint32_t n_requests, const int32_t* const* prompts,
                                   const size_t* prompt_cols, const s2hip_gen_params* p, uint64_t* rng_states,
                                   int32_t* const* codes, uint32_t* n_frames, s2hip_gen_stats* stats, char* err,
                                   size_t err_cap) {
  if (!engine || !prompts || !prompt_cols || !p || !rng_states || !codes || !n_frames) {
    set_err(err, err_cap, "NULL argument");
    return 0;
  }
  for (uint32_t b = 0; b < n_requests; ++b)
    if (!prompts[b] || !codes[b]) {
      set_err(err, err_cap, "NULL argument");
      return 0;
    }
  return guarded(err, err_cap,
                 [&] { engine->e->generate(n_requests, prompts, prompt_cols, *p, rng_states, codes, n_frames, stats); });
}

int32_t s2hip_op_linear(s2hip_engine* engine, const void* w, uint32_t type, size_t in, size_t out, const float* x,
                        size_t ncol, float* y, char* err, size_t err_cap) {
  if (!engine || !w || !x || !y) {
    set_err(err, err_cap, "NULL argument");
    return 0;
  }
  return guarded(err, err_cap, [&] { engine->e->op_linear(w, type, in, out, x, ncol, y); });
}

int32_t s2hip_op_rms_norm(s2hip_engine* engine, const float* x, const float* w, size_t n, size_t ncol, float eps,
                          float* y, char* err, size_t err_cap) {
  if (!engine || !x || !w || !y) {
    set_err(err, err_cap, "NULL argument");
    return 0;
  }
  return guarded(err, err_cap, [&] { engine->e->op_rms_norm(x, w, n, ncol, eps, y); });
}

int32_t s2hip_op_dequant_rows(s2hip_engine* engine, const void* w, uint32_t type, size_t in, size_t rows, float* out,
                              char* err, size_t err_cap) {
  if (!engine || !w || !out) {
    set_err(err, err_cap, "NULL argument");
    return 0;
  }
  return guarded(err, err_cap, [&] { engine->e->op_dequant(w, type, in, rows, out); });
}

int32_t s2hip_op_qk_rope(s2hip_engine* engine, const float* qkv, uint32_t H, uint32_t Hkv, uint32_t hd,
                         uint32_t pos, float base, const float* qn, const float* kn, float eps, float* q, float* k,
                         float* v, char* err, size_t err_cap) {
  if (!engine || !qkv || !q || !k || !v) {
    set_err(err, err_cap, "NULL argument");
    return 0;
  }
  return guarded(err, err_cap, [&] { engine->e->op_qk_rope(qkv, H, Hkv, hd, pos, base, qn, kn, eps, q, k, v); });
}

int32_t s2hip_op_attention(s2hip_engine* engine, const float* q, const float* k, const float* v, uint32_t H,
                           uint32_t Hkv, uint32_t hd, uint32_t T, float scale, float* out, char* err, size_t err_cap) {
  if (!engine || !q || !k || !v || !out) {
    set_err(err, err_cap, "NULL argument");
    return 0;
  }
  return guarded(err, err_cap, [&] { engine->e->op_attention(q, k, v, H, Hkv, hd, T, scale, out); });
}

int32_t s2hip_op_swiglu(s2hip_engine* engine, const float* g, const float* u, size_t n, int32_t fast, float* out,
                        char* err, size_t err_cap) {
  if (!engine || !g || !u || !out) {
    set_err(err, err_cap, "NULL argument");
    return 0;
  }
  return guarded(err, err_cap, [&] { engine->e->op_swiglu(g, u, n, fast, out); });
}

int32_t s2hip_op_sample(s2hip_engine* engine, const float* logits, size_t n, const s2hip_sampler* smp,
                        int64_t always, uint64_t* rng, uint32_t* tok, char* err, size_t err_cap) {
  if (!engine || !logits || !smp || !rng || !tok) {
    set_err(err, err_cap, "NULL argument");
    return 0;
  }
  return guarded(err, err_cap, [&] { engine->e->op_sample(logits, n, *smp, always, rng, tok); });
}

int32_t s2hip_op_sample_noalloc(s2hip_engine* engine, const float* logits, size_t n, const s2hip_sampler* smp,
                                int64_t always, uint64_t* rng, uint32_t* tok, char* err, size_t err_cap) {
  if (!engine || (n && !logits) || !smp || !rng || !tok) {
    set_err(err, err_cap, "NULL argument");
    return 0;
  }
  return guarded(err, err_cap, [&] { engine->e->op_sample_noalloc(logits, n, *smp, always, rng, tok); });
}

void s2hip_device_allocations(uint64_t* count_out) {
  if (count_out) *count_out = s2::g_device_allocs.load(std::memory_order_relaxed);
}

int32_t s2hip_op_running_sums(s2hip_engine* engine, const float* terms, size_t n, float* prefix_out,
                              float* total_out, char* err, size_t err_cap) {
  if (!engine || (n && (!terms || !prefix_out)) || !total_out) {
    set_err(err, err_cap, "NULL argument");
    return 0;
  }
  return guarded(err, err_cap, [&] { engine->e->op_running_sums(terms, n, prefix_out, total_out); });
}

int32_t s2hip_op_running_cut(s2hip_engine* engine, const float* terms, size_t n, float threshold, int32_t absorb,
                             size_t at, size_t* cut_out, float* sum_out, float* at_sum_out, char* err,
                             size_t err_cap) {
  if (!engine || (n && !terms) || !cut_out || !sum_out || !at_sum_out) {
    set_err(err, err_cap, "NULL argument");
    return 0;
  }
  return guarded(err, err_cap, [&] {
    engine->e->op_running_cut(terms, n, threshold, absorb != 0, at, cut_out, sum_out, at_sum_out);
  });
}

int32_t s2hip_op_expf(s2hip_engine* engine, const float* x, size_t n, float* y, char* err, size_t err_cap) {
  if (!engine || (n && (!x || !y))) {
    set_err(err, err_cap, "NULL argument");
    return 0;
  }
  return guarded(err, err_cap, [&] { engine->e->op_expf(x, n, y); });
}

void s2hip_expf_host(const float* x, size_t n, float* y) {
  for (size_t i = 0; i < n; ++i) y[i] = s2::expf_glibc(x[i]);
}

int32_t s2hip_time_kernel(s2hip_engine* engine, const char* kernel, uint32_t reps, double* avg_us, double* bytes,
                          char* err, size_t err_cap) {
  if (!engine || !kernel || !avg_us || !bytes) {
    set_err(err, err_cap, "NULL argument");
    return 0;
  }
  return guarded(err, err_cap, [&] { engine->e->time_kernel(kernel, reps, avg_us, bytes); });
}

}  // extern "C"
