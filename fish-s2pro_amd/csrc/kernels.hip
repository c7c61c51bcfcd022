// kernels.hip -- s2hip device kernels for gfx950 (CDNA4, wave64).
//
// Decode is HBM bound: every kernel here streams its operand once with
// coalesced 16-byte loads per lane and keeps activations in f32.  Weights are
// read in their GGUF block layout (F16 rows, GGML Q8_0 / Q4_0 blocks) and
// dequantised in registers.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <math.h>

#include <type_traits>

#include "expf_glibc.h"
#include "kernels.h"
#include "wave.h"

namespace s2 {
namespace {

constexpr int WAVE = 64;
constexpr int GEMV_THREADS = 256;
constexpr int GEMV_WAVES = GEMV_THREADS / WAVE;
constexpr int SAMPLE_THREADS = 1024;
constexpr uint32_t SAMPLE_MAX = 8192;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float half_bits_to_float(uint16_t b) {
  return static_cast<float>(__builtin_bit_cast(_Float16, b));
}

// A zero word in device memory: optional state pointers are read through
// `opt_word`, which selects the address instead of branching, so the load
// can be issued together with a kernel's other independent loads.
__device__ const uint32_t kZeroWord = 0u;
// (The pointer is cast to the global address space: a generic pointer would
// become a flat load, whose waits also drain every vector load in flight.)
__device__ __forceinline__ uint32_t opt_word(const uint32_t* p) {
  typedef const __attribute__((address_space(1))) uint32_t gword;
  return *(gword*)(p ? p : &kZeroWord);
}

// Two optional words at p0 + off and p1 + off (null: zero), both loads
// issued before either is made wave-uniform, so one wait covers both.
__device__ __forceinline__ void opt_words2(const uint32_t* p0, const uint32_t* p1, size_t off, uint32_t& w0,
                                           uint32_t& w1) {
  typedef const __attribute__((address_space(1))) uint32_t gword;
  const uint32_t v0 = *(gword*)(p0 ? p0 + off : &kZeroWord);
  const uint32_t v1 = *(gword*)(p1 ? p1 + off : &kZeroWord);
  w0 = uint32_t(__builtin_amdgcn_readfirstlane(int(v0)));
  w1 = uint32_t(__builtin_amdgcn_readfirstlane(int(v1)));
}

// Values read through the global address space (see opt_word)
__device__ __forceinline__ float gload_f32(const float* p) {
  typedef const __attribute__((address_space(1))) float gfloat;
  return *(gfloat*)p;
}
__device__ __forceinline__ float2 gload_f2(const float2* p) {
  typedef float f2v __attribute__((ext_vector_type(2)));
  typedef const __attribute__((address_space(1))) f2v gf2v;
  const f2v v = *(gf2v*)p;
  return make_float2(v.x, v.y);
}
__device__ __forceinline__ float4 gload_f4(const float4* p) {
  typedef float f4v __attribute__((ext_vector_type(4)));
  typedef const __attribute__((address_space(1))) f4v gf4v;
  const f4v v = *(gf4v*)p;
  return make_float4(v.x, v.y, v.z, v.w);
}

// Unit gains: the stand-in for an absent QK-norm gain, so that the gain loads
// need no branch.
__device__ const float kUnitGain[256] = {
#define S2_ONE8 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f
#define S2_ONE64 S2_ONE8, S2_ONE8, S2_ONE8, S2_ONE8, S2_ONE8, S2_ONE8, S2_ONE8, S2_ONE8
    S2_ONE64, S2_ONE64, S2_ONE64, S2_ONE64
#undef S2_ONE64
#undef S2_ONE8
};

// ---------------------------------------------------------------------------
// Greedy keys: the largest value m1 with the smallest id among its copies and
// the second largest m2 (a second copy of the largest counts), so that the
// reference's greedy test -- one value within 1e-6 of the max -- holds
// exactly when m2 is not within 1e-6 of m1 (x -> |x - M| never increases for
// x <= M).  Values that are not > -inf (masked, -inf, NaN) take no part.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void greedy_add(float& m1, uint32_t& id1, float& m2, float v, uint32_t id) {
  if (v > m1) {
    m2 = m1;
    m1 = v;
    id1 = id;
  } else {
    if (v == m1) id1 = min(id1, id);
    m2 = fmaxf(m2, v);
  }
}

__device__ __forceinline__ void greedy_merge(float& a1, uint32_t& ai, float& a2, float b1, uint32_t bi, float b2) {
  const uint32_t wi = a1 > b1 ? ai : (b1 > a1 ? bi : min(ai, bi));
  a2 = fmaxf(fminf(a1, b1), fmaxf(a2, b2));
  a1 = fmaxf(a1, b1);
  ai = wi;
}

// The wave's keys in every lane: rows of 16 lanes by DPP exchanges (the
// mirrors pair already-merged quads and half-rows), then the four rows' keys
// read into scalars.  All 64 lanes active.
__device__ __forceinline__ void greedy_wave(float& m1, uint32_t& id1, float& m2) {
  greedy_merge(m1, id1, m2, dpp_f32<DPP_QUAD_XOR1>(m1), dpp_u32<DPP_QUAD_XOR1>(id1), dpp_f32<DPP_QUAD_XOR1>(m2));
  greedy_merge(m1, id1, m2, dpp_f32<DPP_QUAD_XOR2>(m1), dpp_u32<DPP_QUAD_XOR2>(id1), dpp_f32<DPP_QUAD_XOR2>(m2));
  greedy_merge(m1, id1, m2, dpp_f32<DPP_ROW_HALF_MIRROR>(m1), dpp_u32<DPP_ROW_HALF_MIRROR>(id1),
               dpp_f32<DPP_ROW_HALF_MIRROR>(m2));
  greedy_merge(m1, id1, m2, dpp_f32<DPP_ROW_MIRROR>(m1), dpp_u32<DPP_ROW_MIRROR>(id1), dpp_f32<DPP_ROW_MIRROR>(m2));
  float r1[4], r2[4];
  uint32_t ri[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    r1[r] = lane_read_f32(m1, 16 * r);
    r2[r] = lane_read_f32(m2, 16 * r);
    ri[r] = lane_read_u32(id1, 16 * r);
  }
  greedy_merge(r1[0], ri[0], r2[0], r1[1], ri[1], r2[1]);
  greedy_merge(r1[2], ri[2], r2[2], r1[3], ri[3], r2[3]);
  greedy_merge(r1[0], ri[0], r2[0], r1[2], ri[2], r2[2]);
  m1 = r1[0];
  id1 = ri[0];
  m2 = r2[0];
}

// SeededRng state step (the draw is the top 53 bits of the new state)
__device__ __forceinline__ uint64_t lcg_step(uint64_t s) { return s * 6364136223846793005ull + 1ull; }

// The greedy test on a merged key: `count` values took part.  +inf as the
// max fails it (inf - inf is NaN), as the reference counts no value then.
__device__ __forceinline__ bool greedy_unique(uint32_t count, float m1, float m2) {
  return count > 0 && fabsf(m1 - m1) < 1e-6f && !(fabsf(m2 - m1) < 1e-6f);
}

// The greedy sample of logits[0, n) (n % 4 == 0, n > 0) by a block of NW
// waves, in two parts so that a kernel can issue the loads early:
// greedy_loads issues U float4 per thread (addresses clamped into the
// logits; values past n are dropped by the second part), block_greedy_keys
// adds any remainder and reduces over the block (LDS scratch of NW entries
// each).  Every thread gets the token (id 0 when no value is finite) and
// whether the greedy test failed (a tie within 1e-6 at the max, or a
// non-finite max) while some value was finite.
template <int NW, int U>
__device__ __forceinline__ void greedy_loads(const float* logits, uint32_t n, float4 (&lg)[U]) {
  const float4* l4 = reinterpret_cast<const float4*>(logits);
  const uint32_t n4 = n / 4u;
#pragma unroll
  for (int r = 0; r < U; ++r) lg[r] = gload_f4(l4 + min(threadIdx.x + uint32_t(r) * NW * 64u, n4 - 1u));
}

template <int NW, int U>
__device__ __forceinline__ void block_greedy_keys(const float4 (&lg)[U], const float* logits, uint32_t n, float* s1,
                                                  float* s2, uint32_t* sid, uint32_t* scnt, uint32_t& tok,
                                                  uint32_t& tie) {
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t n4 = n / 4u;
  float m1 = -INFINITY, m2 = -INFINITY;
  uint32_t id1 = 0xffffffffu, cnt = 0;
  auto add4 = [&](const float4 q, uint32_t i) {
    const float v4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (v4[c] > -INFINITY) {
        ++cnt;
        greedy_add(m1, id1, m2, v4[c], 4u * i + uint32_t(c));
      }
    }
  };
#pragma unroll
  for (int r = 0; r < U; ++r) {
    const uint32_t i = tid + uint32_t(r) * NW * 64u;
    if (i < n4) add4(lg[r], i);
  }
  const float4* l4 = reinterpret_cast<const float4*>(logits);
  for (uint32_t i = tid + uint32_t(U) * NW * 64u; i < n4; i += NW * 64u) add4(gload_f4(l4 + i), i);
  greedy_wave(m1, id1, m2);
  cnt = wave_sum_u32(cnt);
  if (lane == 0) {
    s1[wave] = m1;
    s2[wave] = m2;
    sid[wave] = id1;
    scnt[wave] = cnt;
  }
  __syncthreads();
  float a1 = s1[0], a2 = s2[0];
  uint32_t ai = sid[0], c = scnt[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) {
    greedy_merge(a1, ai, a2, s1[w], sid[w], s2[w]);
    c += scnt[w];
  }
  tok = c > 0 ? min(ai, n - 1u) : 0u;
  tie = (c > 0 && !greedy_unique(c, a1, a2)) ? 1u : 0u;
}


// ---------------------------------------------------------------------------
// Raw weight payload for 8 consecutive elements, loaded first and decoded
// later so a wave can keep many independent 16-byte loads in flight.
// ---------------------------------------------------------------------------
template <uint32_t WT>
struct Raw8 {
  uint32_t d, w0, w1, w2;  // Q8_0 / Q4_0: d bits | shift << 16 | part << 20; aligned 12-byte window
};
template <>
struct Raw8<W_F16> {
  half8 v;
};

template <uint32_t WT>
__device__ __forceinline__ Raw8<WT> load_raw(const uint8_t* row, uint32_t e) {
  Raw8<WT> r;
  if constexpr (WT == W_F16) {
    // each F16 weight byte is read once per launch: a non-temporal load
    // streams it without displacing reusable lines (x, the warmed rows) from
    // L2 (w13 17.4 -> 16.5 us)
    r.v = __builtin_nontemporal_load(reinterpret_cast<const half8*>(row + size_t(e) * 2));
  } else {
    constexpr uint32_t BB = (WT == W_Q8_0) ? 34u : 18u;
    const uint32_t b = e >> 5, p = (e >> 3) & 3u;
    const uint8_t* blk = row + size_t(b) * BB;
    const uint32_t qoff = (WT == W_Q8_0) ? 2 + p * 8 : 2 + (p & 1u) * 8;
    // aligned window by pointer arithmetic (an integer round trip would lose
    // the global address space and turn these into flat loads)
    const uint8_t* q = blk + qoff;
    const uint32_t mis = uint32_t(reinterpret_cast<uintptr_t>(q) & 3u);
    const uint32_t* base = reinterpret_cast<const uint32_t*>(q - mis);
    r.d = uint32_t(*reinterpret_cast<const uint16_t*>(blk)) | (mis << 16) | (p << 20);
    // plain loads: neighbouring lanes' windows share cache lines (measured
    // 4-5 % slower as non-temporal loads)
    r.w0 = base[0];
    r.w1 = base[1];
    r.w2 = base[2];
  }
  return r;
}

template <uint32_t WT>
__device__ __forceinline__ void decode8(const Raw8<WT>& r, float w[8]) {
  if constexpr (WT == W_F16) {
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = static_cast<float>(r.v[i]);
  } else {
    const float d = half_bits_to_float(uint16_t(r.d & 0xffffu));
    const uint32_t sh = (r.d >> 16) & 3u, p = (r.d >> 20) & 3u;
    const uint32_t lo = __builtin_amdgcn_alignbyte(r.w1, r.w0, sh);
    const uint32_t hi = __builtin_amdgcn_alignbyte(r.w2, r.w1, sh);
    if constexpr (WT == W_Q8_0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        w[i] = static_cast<float>(static_cast<int8_t>((lo >> (8 * i)) & 0xffu)) * d;
        w[4 + i] = static_cast<float>(static_cast<int8_t>((hi >> (8 * i)) & 0xffu)) * d;
      }
    } else {
      const uint32_t ns = (p >= 2) ? 4u : 0u;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        w[i] = static_cast<float>(int((lo >> (8 * i + ns)) & 0xfu) - 8) * d;
        w[4 + i] = static_cast<float>(int((hi >> (8 * i + ns)) & 0xfu) - 8) * d;
      }
    }
  }
}

template <uint32_t WT>
__device__ __forceinline__ void load_w8(const uint8_t* row, uint32_t e, float w[8]) {
  decode8<WT>(load_raw<WT>(row, e), w);
}

// ---------------------------------------------------------------------------
// GEMV: y[c][o] (+)= sum_i x[c][i] * W[o][i]
//   block = 4 waves; each wave owns R consecutive output rows and each lane
//   handles 8 consecutive elements per 512-element step.  The first batch of
//   PF steps of weight loads is issued before x is staged (and optionally
//   RMS-normalised) in LDS, so the x prologue hides under HBM latency.
// ---------------------------------------------------------------------------
template <uint32_t WT, int NCOL, int R, int EPI>
__global__ __launch_bounds__(GEMV_THREADS) void gemv_kernel(GemvArgs a) {
  if (a.done && *a.done) return;
  extern __shared__ float xs[];  // [NCOL][in]
  __shared__ float red[GEMV_WAVES][NCOL];
  constexpr bool DUAL = (EPI == EPI_SWIGLU_SLOW || EPI == EPI_SWIGLU_FAST);
  constexpr int PF = 16 / (R * (DUAL ? 2 : 1) * (NCOL > 2 ? 2 : 1));
  const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid >> 6;
  const uint32_t in = a.in;
  const uint32_t kit = (in + WAVE * 8 - 1) / (WAVE * 8);

  const uint32_t row0 = (blockIdx.x * GEMV_WAVES + wave) * R;
  const uint8_t* rp[R];
  const uint8_t* rp3[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    uint32_t lr = row0 + r;
    if (lr >= a.out) lr = 0;  // clamp; result discarded
    const uint32_t wr = (a.extra_row != NO_ROW && lr == a.out - 1) ? a.extra_row : a.row_base + lr;
    rp[r] = a.w + size_t(wr) * a.row_bytes;
    rp3[r] = DUAL ? a.w3 + size_t(wr) * a.row_bytes : nullptr;
  }

  Raw8<WT> wb[R][PF];
  Raw8<WT> wb3[DUAL ? R : 1][PF];
  auto load_batch = [&](uint32_t it0) {
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const uint32_t e = (it0 + j) * (WAVE * 8) + lane * 8;
      if (it0 + j < kit && e < in) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          wb[r][j] = load_raw<WT>(rp[r], e);
          if constexpr (DUAL) wb3[r][j] = load_raw<WT>(rp3[r], e);
        }
      }
    }
  };
  load_batch(0);

  // stage x (16-byte loads), with the RMSNorm sum of squares on the way
  const bool vec = (in % 4 == 0) && (a.ldx % 4 == 0);
#pragma unroll
  for (int c = 0; c < NCOL; ++c) {
    const float* xc = a.x + size_t(c) * a.ldx;
    float ss = 0.0f;
    if (vec) {
      for (uint32_t i = tid * 4; i < in; i += GEMV_THREADS * 4) {
        const float4 v = *reinterpret_cast<const float4*>(xc + i);
        *reinterpret_cast<float4*>(&xs[c * in + i]) = v;
        ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
      }
    } else {
      for (uint32_t i = tid; i < in; i += GEMV_THREADS) {
        const float v = xc[i];
        xs[c * in + i] = v;
        ss += v * v;
      }
    }
    if (a.norm) {
      ss = wave_sum(ss);
      if (lane == 0) red[wave][c] = ss;
    }
  }
  if (a.norm) {
    __syncthreads();
#pragma unroll
    for (int c = 0; c < NCOL; ++c) {
      const float tot = (red[0][c] + red[1][c]) + (red[2][c] + red[3][c]);
      const float scale = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(tot, float(in)), a.eps)));
      for (uint32_t i = tid; i < in; i += GEMV_THREADS)
        xs[c * in + i] = __fmul_rn(__fmul_rn(xs[c * in + i], scale), a.norm[i]);
    }
  }
  __syncthreads();

  float acc[R][NCOL];
  float acc3[R][NCOL];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < NCOL; ++c) {
      acc[r][c] = 0.0f;
      acc3[r][c] = 0.0f;
    }

  for (uint32_t it0 = 0; it0 < kit; it0 += PF) {
    if (it0 > 0) load_batch(it0);
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const uint32_t e = (it0 + j) * (WAVE * 8) + lane * 8;
      if (it0 + j < kit && e < in) {
        float w[R][8];
        float w3[DUAL ? R : 1][8];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          decode8<WT>(wb[r][j], w[r]);
          if constexpr (DUAL) decode8<WT>(wb3[r][j], w3[r]);
        }
#pragma unroll
        for (int c = 0; c < NCOL; ++c) {
          const float4 xa = *reinterpret_cast<const float4*>(&xs[c * in + e]);
          const float4 xb = *reinterpret_cast<const float4*>(&xs[c * in + e + 4]);
          const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
          for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int k = 0; k < 8; ++k) acc[r][c] = fmaf(w[r][k], xv[k], acc[r][c]);
            if constexpr (DUAL) {
#pragma unroll
              for (int k = 0; k < 8; ++k) acc3[r][c] = fmaf(w3[r][k], xv[k], acc3[r][c]);
            }
          }
        }
      }
    }
  }

#pragma unroll
  for (int r = 0; r < R; ++r) {
#pragma unroll
    for (int c = 0; c < NCOL; ++c) {
      const float g = wave_sum(acc[r][c]);
      float u = 0.0f;
      if constexpr (DUAL) u = wave_sum(acc3[r][c]);
      const uint32_t lr = row0 + r;
      if (lane == 0 && lr < a.out) {
        float* dst = a.y + size_t(c) * a.ldy + lr;
        if constexpr (EPI == EPI_STORE) {
          *dst = g;
        } else if constexpr (EPI == EPI_RESID) {
          *dst = __fadd_rn(*dst, g);
        } else if constexpr (EPI == EPI_SWIGLU_SLOW) {
          const float sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf_glibc(-g)));
          *dst = __fmul_rn(__fmul_rn(g, sig), u);
        } else {
          *dst = __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, expf_glibc(-g))), u);
        }
      }
    }
  }
}

template <uint32_t WT, int NCOL, int R, int EPI>
hipError_t gemv_launch_one(const GemvArgs& a, hipStream_t s) {
  const size_t lds = size_t(NCOL) * a.in * sizeof(float);
  static bool configured = false;
  if (!configured) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(gemv_kernel<WT, NCOL, R, EPI>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024 - 1024);
    if (e != hipSuccess) return e;
    configured = true;
  }
  const uint32_t rows_per_block = GEMV_WAVES * R;
  const dim3 grid((a.out + rows_per_block - 1) / rows_per_block);
  hipLaunchKernelGGL((gemv_kernel<WT, NCOL, R, EPI>), grid, dim3(GEMV_THREADS), lds, s, a);
  return hipGetLastError();
}

template <uint32_t WT, int NCOL, int EPI>
hipError_t gemv_pick_r(const GemvArgs& a, hipStream_t s) {
  constexpr bool DUAL = (EPI == EPI_SWIGLU_SLOW || EPI == EPI_SWIGLU_FAST);
  if (NCOL == 1 && !DUAL && a.out > 4096) return gemv_launch_one<WT, NCOL, 2, EPI>(a, s);
  return gemv_launch_one<WT, NCOL, 1, EPI>(a, s);
}

template <uint32_t WT, int EPI>
hipError_t gemv_pick_ncol(int ncol, const GemvArgs& a, hipStream_t s) {
  switch (ncol) {
    case 1: return gemv_pick_r<WT, 1, EPI>(a, s);
    case 2: return gemv_pick_r<WT, 2, EPI>(a, s);
    case 4: return gemv_pick_r<WT, 4, EPI>(a, s);
    case 8: return gemv_pick_r<WT, 8, EPI>(a, s);
    default: return hipErrorInvalidValue;
  }
}

template <uint32_t WT>
hipError_t gemv_pick_epi(int epi, int ncol, const GemvArgs& a, hipStream_t s) {
  switch (epi) {
    case EPI_STORE: return gemv_pick_ncol<WT, EPI_STORE>(ncol, a, s);
    case EPI_RESID: return gemv_pick_ncol<WT, EPI_RESID>(ncol, a, s);
    case EPI_SWIGLU_SLOW: return gemv_pick_ncol<WT, EPI_SWIGLU_SLOW>(ncol, a, s);
    case EPI_SWIGLU_FAST: return gemv_pick_ncol<WT, EPI_SWIGLU_FAST>(ncol, a, s);
    default: return hipErrorInvalidValue;
  }
}

// ---------------------------------------------------------------------------
// Decode GEMV (1-2 input columns): every weight load of a wave's R rows is
// issued up front (predicated on the runtime step count, at most KMAX
// 512-element steps per row), x and the RMSNorm gain are read through the
// L1 cache, and the only block-level synchronisation is the RMSNorm scale.
// ---------------------------------------------------------------------------
template <uint32_t WT, int NCOL, int R, int EPI, int KMAX, int WPB, bool XREG>
__global__ __launch_bounds__(64 * WPB) void gemv_direct_kernel(GemvArgs a) {
  if (a.done && *a.done) return;
  constexpr bool DUAL = (EPI == EPI_SWIGLU_SLOW || EPI == EPI_SWIGLU_FAST);
  // XREG: x (and the norm gain) held in registers, loaded before the weights
  constexpr int XK = XREG ? KMAX : 1;
  __shared__ float red[WPB][NCOL];
  const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid >> 6;
  const uint32_t in = a.in;
  const uint32_t kit = in / (WAVE * 8);  // host guarantees in % 512 == 0
  const uint32_t row0 = (blockIdx.x * WPB + wave) * R;

  float4 xr[NCOL][XK][2];
  float4 gr[XK][2];
  if constexpr (XREG) {
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
      if (k < kit) {
        const uint32_t e = k * (WAVE * 8) + lane * 8;
#pragma unroll
        for (int c = 0; c < NCOL; ++c) {
          const float* xc = a.x + size_t(c) * a.ldx + e;
          xr[c][k][0] = *reinterpret_cast<const float4*>(xc);
          xr[c][k][1] = *reinterpret_cast<const float4*>(xc + 4);
        }
        if (a.norm) {
          gr[k][0] = *reinterpret_cast<const float4*>(a.norm + e);
          gr[k][1] = *reinterpret_cast<const float4*>(a.norm + e + 4);
        }
      }
    }
  }

  const uint8_t* rp[R];
  const uint8_t* rp3[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    uint32_t lr = row0 + r;
    if (lr >= a.out) lr = 0;  // clamp; result discarded
    const uint32_t wr = (a.extra_row != NO_ROW && lr == a.out - 1) ? a.extra_row : a.row_base + lr;
    rp[r] = a.w + size_t(wr) * a.row_bytes;
    rp3[r] = DUAL ? a.w3 + size_t(wr) * a.row_bytes : nullptr;
  }
  Raw8<WT> wb[R][KMAX];
  Raw8<WT> wb3[DUAL ? R : 1][KMAX];
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    if (k < kit) {
      const uint32_t e = k * (WAVE * 8) + lane * 8;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        wb[r][k] = load_raw<WT>(rp[r], e);
        if constexpr (DUAL) wb3[r][k] = load_raw<WT>(rp3[r], e);
      }
    }
  }

  float scale[NCOL];
#pragma unroll
  for (int c = 0; c < NCOL; ++c) scale[c] = 1.0f;
  if (a.norm) {
    if constexpr (XREG) {
      // every lane holds in/64 elements of each column: a wave sum covers x
#pragma unroll
      for (int c = 0; c < NCOL; ++c) {
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < KMAX; ++k) {
          if (k < kit) {
            const float4 u = xr[c][k][0], v = xr[c][k][1];
            ss += u.x * u.x + u.y * u.y + u.z * u.z + u.w * u.w;
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
          }
        }
        ss = wave_sum(ss);
        scale[c] = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, float(in)), a.eps)));
      }
    } else {
#pragma unroll
      for (int c = 0; c < NCOL; ++c) {
        const float* xc = a.x + size_t(c) * a.ldx;
        float ss = 0.0f;
        for (uint32_t i = tid * 4; i < in; i += 64 * WPB * 4) {
          const float4 v = *reinterpret_cast<const float4*>(xc + i);
          ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
        ss = wave_sum(ss);
        if (lane == 0) red[wave][c] = ss;
      }
      if constexpr (WPB > 1) __syncthreads();
#pragma unroll
      for (int c = 0; c < NCOL; ++c) {
        float tot = red[0][c];
#pragma unroll
        for (int w = 1; w < WPB; ++w) tot += red[w][c];
        scale[c] = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(tot, float(in)), a.eps)));
      }
    }
  }

  float acc[R][NCOL];
  float acc3[R][NCOL];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < NCOL; ++c) {
      acc[r][c] = 0.0f;
      acc3[r][c] = 0.0f;
    }
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    if (k < kit) {
      const uint32_t e = k * (WAVE * 8) + lane * 8;
      float w[R][8];
      float w3[DUAL ? R : 1][8];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        decode8<WT>(wb[r][k], w[r]);
        if constexpr (DUAL) decode8<WT>(wb3[r][k], w3[r]);
      }
      float4 ga, gb;
      if (a.norm) {
        if constexpr (XREG) {
          ga = gr[k][0];
          gb = gr[k][1];
        } else {
          ga = *reinterpret_cast<const float4*>(a.norm + e);
          gb = *reinterpret_cast<const float4*>(a.norm + e + 4);
        }
      }
#pragma unroll
      for (int c = 0; c < NCOL; ++c) {
        float4 xa, xb;
        if constexpr (XREG) {
          xa = xr[c][k][0];
          xb = xr[c][k][1];
        } else {
          const float* xc = a.x + size_t(c) * a.ldx + e;
          xa = *reinterpret_cast<const float4*>(xc);
          xb = *reinterpret_cast<const float4*>(xc + 4);
        }
        float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
        if (a.norm) {
          const float g[8] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w};
#pragma unroll
          for (int i = 0; i < 8; ++i) xv[i] = __fmul_rn(__fmul_rn(xv[i], scale[c]), g[i]);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[r][c] = fmaf(w[r][i], xv[i], acc[r][c]);
          if constexpr (DUAL) {
#pragma unroll
            for (int i = 0; i < 8; ++i) acc3[r][c] = fmaf(w3[r][i], xv[i], acc3[r][c]);
          }
        }
      }
    }
  }

#pragma unroll
  for (int r = 0; r < R; ++r) {
#pragma unroll
    for (int c = 0; c < NCOL; ++c) {
      const float gsum = wave_sum(acc[r][c]);
      float u = 0.0f;
      if constexpr (DUAL) u = wave_sum(acc3[r][c]);
      const uint32_t lr = row0 + r;
      if (lane == 0 && lr < a.out) {
        float* dst = a.y + size_t(c) * a.ldy + lr;
        if constexpr (EPI == EPI_STORE) {
          *dst = gsum;
        } else if constexpr (EPI == EPI_RESID) {
          *dst = __fadd_rn(*dst, gsum);
        } else if constexpr (EPI == EPI_SWIGLU_SLOW) {
          const float sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf_glibc_wave(-gsum)));
          *dst = __fmul_rn(__fmul_rn(gsum, sig), u);
        } else {
          *dst = __fmul_rn(__fdiv_rn(gsum, __fadd_rn(1.0f, expf_glibc_wave(-gsum))), u);
        }
      }
    }
  }
}

template <uint32_t WT, int NCOL, int R, int EPI, int KMAX, int WPB = 4, bool XREG = false>
hipError_t gemv_direct_launch(const GemvArgs& a, hipStream_t s) {
  const uint32_t rows_per_block = WPB * R;
  const dim3 grid((a.out + rows_per_block - 1) / rows_per_block);
  hipLaunchKernelGGL((gemv_direct_kernel<WT, NCOL, R, EPI, KMAX, WPB, XREG>), grid, dim3(64 * WPB), 0, s, a);
  return hipGetLastError();
}

template <uint32_t WT, int NCOL, int EPI>
hipError_t gemv_direct_pick(const GemvArgs& a, hipStream_t s) {
  constexpr bool DUAL = (EPI == EPI_SWIGLU_SLOW || EPI == EPI_SWIGLU_FAST);
  if (a.in <= 8 * 512) {
    if (!DUAL && NCOL == 1 && a.out > 4096) return gemv_direct_launch<WT, NCOL, 2, EPI, 8>(a, s);
    return gemv_direct_launch<WT, NCOL, 1, EPI, 8>(a, s);
  }
  return gemv_direct_launch<WT, NCOL, 1, EPI, 20>(a, s);
}

template <uint32_t WT, int EPI>
hipError_t gemv_direct_ncol(int ncol, const GemvArgs& a, hipStream_t s) {
  if (ncol == 1) return gemv_direct_pick<WT, 1, EPI>(a, s);
  return gemv_direct_pick<WT, 2, EPI>(a, s);
}

template <uint32_t WT>
hipError_t gemv_direct_epi(int epi, int ncol, const GemvArgs& a, hipStream_t s) {
  switch (epi) {
    case EPI_STORE: return gemv_direct_ncol<WT, EPI_STORE>(ncol, a, s);
    case EPI_RESID: return gemv_direct_ncol<WT, EPI_RESID>(ncol, a, s);
    case EPI_SWIGLU_SLOW: return gemv_direct_ncol<WT, EPI_SWIGLU_SLOW>(ncol, a, s);
    case EPI_SWIGLU_FAST: return gemv_direct_ncol<WT, EPI_SWIGLU_FAST>(ncol, a, s);
    default: return hipErrorInvalidValue;
  }
}

// ---------------------------------------------------------------------------
// Decode GEMV with a compile-time row length (KIT 512-element steps): no
// predication, every weight load of the wave's R rows issued at once.  The
// RMSNorm x loads go out before the weights (loads complete in order), so
// each wave has its norm scale by the time its weights land, with no block
// barrier.  The early-exit flag is read after the loads are in flight.
// ---------------------------------------------------------------------------
template <uint32_t WT, int NCOL, int R, int EPI, int KIT, int WPB, bool NORM>
__global__ __launch_bounds__(64 * WPB) void gemv_k_kernel(GemvArgs a) {
  constexpr bool DUAL = (EPI == EPI_SWIGLU_SLOW || EPI == EPI_SWIGLU_FAST);
  const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid >> 6;
  constexpr uint32_t IN = uint32_t(KIT) * WAVE * 8;
  constexpr int XK = NORM ? KIT : 1;
  const uint32_t row0 = (blockIdx.x * WPB + wave) * R;
  (void)tid;

  // 1. x loads of the normalised GEMVs (kept in registers for the FMA loop)
  float4 xr[NCOL][XK][2];
  if constexpr (NORM) {
#pragma unroll
    for (int c = 0; c < NCOL; ++c)
#pragma unroll
      for (int k = 0; k < KIT; ++k) {
        const float* xc = a.x + size_t(c) * a.ldx + k * 512 + lane * 8;
        xr[c][k][0] = *reinterpret_cast<const float4*>(xc);
        xr[c][k][1] = *reinterpret_cast<const float4*>(xc + 4);
      }
  }
  // 2. weight loads: all of the wave's rows at once
  const uint8_t* rp[R];
  const uint8_t* rp3[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    uint32_t lr = row0 + r;
    if (lr >= a.out) lr = 0;  // clamp; result discarded
    const uint32_t wr = (a.extra_row != NO_ROW && lr == a.out - 1) ? a.extra_row : a.row_base + lr;
    rp[r] = a.w + size_t(wr) * a.row_bytes;
    rp3[r] = DUAL ? a.w3 + size_t(wr) * a.row_bytes : nullptr;
  }
  Raw8<WT> wb[R][KIT];
  Raw8<WT> wb3[DUAL ? R : 1][KIT];
#pragma unroll
  for (int k = 0; k < KIT; ++k) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      wb[r][k] = load_raw<WT>(rp[r], k * 512 + lane * 8);
      if constexpr (DUAL) wb3[r][k] = load_raw<WT>(rp3[r], k * 512 + lane * 8);
    }
  }
  // read after the weight loads are issued: the scalar wait then overlaps them
  const uint32_t done = a.done ? __builtin_nontemporal_load(a.done) : 0u;
  // 3. RMSNorm scale: each lane holds in/64 elements, a wave sum covers x
  float scale[NCOL];
#pragma unroll
  for (int c = 0; c < NCOL; ++c) {
    scale[c] = 1.0f;
    if constexpr (NORM) {
      float ss = 0.0f;
#pragma unroll
      for (int k = 0; k < KIT; ++k) {
        const float4 u = xr[c][k][0], v = xr[c][k][1];
        ss += u.x * u.x + u.y * u.y + u.z * u.z + u.w * u.w;
        ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
      }
      ss = wave_sum(ss);
      scale[c] = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, float(IN)), a.eps)));
    }
  }
  if (done) return;

  float acc[R][NCOL];
  float acc3[R][NCOL];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < NCOL; ++c) {
      acc[r][c] = 0.0f;
      acc3[r][c] = 0.0f;
    }
#pragma unroll
  for (int k = 0; k < KIT; ++k) {
    const uint32_t e = k * 512 + lane * 8;
    float w[R][8];
    float w3[DUAL ? R : 1][8];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      decode8<WT>(wb[r][k], w[r]);
      if constexpr (DUAL) decode8<WT>(wb3[r][k], w3[r]);
    }
    float g[8];
    if constexpr (NORM) {
      const float4 ga = *reinterpret_cast<const float4*>(a.norm + e);
      const float4 gb = *reinterpret_cast<const float4*>(a.norm + e + 4);
      g[0] = ga.x; g[1] = ga.y; g[2] = ga.z; g[3] = ga.w;
      g[4] = gb.x; g[5] = gb.y; g[6] = gb.z; g[7] = gb.w;
    }
#pragma unroll
    for (int c = 0; c < NCOL; ++c) {
      float4 xa, xb;
      if constexpr (NORM) {
        xa = xr[c][k][0];
        xb = xr[c][k][1];
      } else {
        const float* xc = a.x + size_t(c) * a.ldx + e;
        xa = *reinterpret_cast<const float4*>(xc);
        xb = *reinterpret_cast<const float4*>(xc + 4);
      }
      float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
      if constexpr (NORM) {
#pragma unroll
        for (int i = 0; i < 8; ++i) xv[i] = __fmul_rn(__fmul_rn(xv[i], scale[c]), g[i]);
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[r][c] = fmaf(w[r][i], xv[i], acc[r][c]);
        if constexpr (DUAL) {
#pragma unroll
          for (int i = 0; i < 8; ++i) acc3[r][c] = fmaf(w3[r][i], xv[i], acc3[r][c]);
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
#pragma unroll
    for (int c = 0; c < NCOL; ++c) {
      const float gsum = wave_sum(acc[r][c]);
      float u = 0.0f;
      if constexpr (DUAL) u = wave_sum(acc3[r][c]);
      const uint32_t lr = row0 + r;
      if (lane == 0 && lr < a.out) {
        float* dst = a.y + size_t(c) * a.ldy + lr;
        if constexpr (EPI == EPI_STORE) {
          *dst = gsum;
        } else if constexpr (EPI == EPI_RESID) {
          *dst = __fadd_rn(*dst, gsum);
        } else if constexpr (EPI == EPI_SWIGLU_SLOW) {
          const float sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf_glibc_wave(-gsum)));
          *dst = __fmul_rn(__fmul_rn(gsum, sig), u);
        } else {
          *dst = __fmul_rn(__fdiv_rn(gsum, __fadd_rn(1.0f, expf_glibc_wave(-gsum))), u);
        }
      }
    }
  }
}

template <uint32_t WT, int NCOL, int R, int EPI, int KIT, int WPB>
hipError_t gemv_k_launch(const GemvArgs& a, hipStream_t s) {
  const uint32_t rows_per_block = WPB * R;
  const dim3 grid((a.out + rows_per_block - 1) / rows_per_block);
  if (a.norm)
    hipLaunchKernelGGL((gemv_k_kernel<WT, NCOL, R, EPI, KIT, WPB, true>), grid, dim3(64 * WPB), 0, s, a);
  else
    hipLaunchKernelGGL((gemv_k_kernel<WT, NCOL, R, EPI, KIT, WPB, false>), grid, dim3(64 * WPB), 0, s, a);
  return hipGetLastError();
}

// Warming block r (of w.blocks) at linear grid index L: consumer blocks
// cb = cb_begin + 8 q + (L % 8) for q = r / 8, r / 8 + blocks / 8, ...  The
// block's loads (per consumer block and matrix, `per` loads of 16 bytes per
// thread) are walked as one list, D distinct loads per thread in flight; the
// walk position is uniform over the block (scalar registers) and past the end
// of the list stays on the last load.
template <int D>
__device__ __forceinline__ void l2_warm_walk(const L2Warm& w, uint32_t L, uint32_t r, uint32_t tid, uint32_t nthr) {
  const uint32_t stride = nthr * 16u;
  const uint32_t per = (w.span + stride - 1) / stride;
  const uint32_t mats = w.base3 ? 2u : 1u;
  const uint32_t cb0 = w.cb_begin + 8u * (r >> 3) + (L & 7u);
  if (cb0 >= w.cb_end) return;
  const uint32_t total = (w.cb_end - cb0 + w.blocks - 1) / w.blocks * mats * per;
  const uint32_t off0 = tid * 16u, last = w.span - 16u;
  uint32_t i = 0, m = 0, j = 0, acc = 0;
  for (uint32_t u0 = 0; u0 < total; u0 += D) {
    uint32_t v[D];
#pragma unroll
    for (int k = 0; k < D; ++k) {
      const uint8_t* p = (m ? w.base3 : w.base) + size_t(cb0 + i * w.blocks) * w.span;
      // one word per 16 bytes: every 64-byte sector of the rows is read
      v[k] = *reinterpret_cast<const uint32_t*>(p + min(off0 + j * stride, last));
      if (u0 + k + 1 < total) {
        if (++j == per) {
          j = 0;
          if (++m == mats) {
            m = 0;
            ++i;
          }
        }
      }
    }
#pragma unroll
    for (int k = 0; k < D; ++k) acc ^= v[k];
  }
  asm volatile("" : : "v"(acc));  // the loads are kept; nothing is stored
}

__device__ __forceinline__ void l2_warm(const L2Warm& w, uint32_t L, uint32_t r, uint32_t tid, uint32_t nthr) {
  if (r >= w.blocks) return;
  if (w.depth >= 16)
    l2_warm_walk<16>(w, L, r, tid, nthr);
  else if (w.depth >= 8)
    l2_warm_walk<8>(w, L, r, tid, nthr);
  else
    l2_warm_walk<4>(w, L, r, tid, nthr);
}

// ---------------------------------------------------------------------------
// Decode GEMV with x shared through LDS (NORM: RMS-normalised input).
//   Each wave loads only the 512-element steps k = wave (mod WPB) of x and of
//   the gain, then issues all of its weight loads; the block reduces the sum of
//   squares, writes x * scale * gain (NORM) or x once to LDS, and every wave
//   reads x from there.  The x / gain loads are issued first, so the
//   waits before the two barriers cover them and not the weights (vector
//   memory counters retire in order), and the LDS staging overlaps the HBM
//   latency of the weight rows.  One row (two for SwiGLU: w1 and w3) per wave.
//
// FOLD (one column, RMSNorm, store): x is emb[argmax of fold.logits], the
//   greedy sample of the previous sub-step (GreedyFold).  The logit loads go
//   first, then the first half of the weight loads; the block reduces the
//   greedy keys while those are in flight, loads the embedding row, and only
//   then issues the rest of the weights, so the wait for the row drains only
//   the loads issued before it.
// ---------------------------------------------------------------------------
template <uint32_t WT, int NCOL, int EPI, int KIT, int WPB, bool NORM, bool FOLD = false>
__global__ __launch_bounds__(64 * WPB) void gemv_n_kernel(const uint8_t* w_rows, const uint8_t* w3_rows, const float* x_in,
                                                              const float* gain, const uint32_t* done_ptr,
                                                              uint32_t row_bytes, uint32_t out, uint32_t row_base,
                                                              uint32_t extra_row, GemvArgs a) {
  constexpr bool DUAL = (EPI == EPI_SWIGLU_SLOW || EPI == EPI_SWIGLU_FAST);
  static_assert(!FOLD || (NCOL == 1 && NORM && EPI == EPI_STORE), "the greedy fold feeds one normalised column");
  constexpr uint32_t IN = uint32_t(KIT) * WAVE * 8;
  constexpr int KW = (KIT + WPB - 1) / WPB;
  constexpr uint32_t NT = 64u * WPB;
  // FOLD: weight steps loaded before the embedding row (the rest after it)
  constexpr int KA = FOLD ? (KIT + 1) / 2 : KIT;
  __shared__ float4 xs[NCOL][IN / 4];
  __shared__ float red[NCOL][WPB];
  __shared__ float fold_m1[FOLD ? WPB : 1], fold_m2[FOLD ? WPB : 1];
  __shared__ uint32_t fold_id[FOLD ? WPB : 1], fold_cnt[FOLD ? WPB : 1];
  const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x >> 6;
  const uint32_t row = blockIdx.x * WPB + wave;

  // 1. this wave's steps of x and of the gain (steps past KIT re-read the last
  //    step; they are not used); FOLD: the logits instead of x
  float4 xv[NCOL][KW][2], gv[KW][2];
  float4 lg[2];
  uint32_t st_done = 0;
  uint64_t st_rng = 0;
  if constexpr (FOLD) {
    const float4* l4 = reinterpret_cast<const float4*>(a.fold.logits);
    const uint32_t n4 = a.fold.n / 4u;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const uint32_t i = threadIdx.x + uint32_t(r) * NT;
      lg[r] = i < n4 ? l4[i] : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
    }
    st_done = a.fold.st->done;  // uniform: scalar loads, no vector wait later
    st_rng = a.fold.st->rng;
  }
#pragma unroll
  for (int j = 0; j < KW; ++j) {
    const int k = min(wave + j * WPB, KIT - 1);
    const uint32_t e = k * 512 + lane * 8;
    if constexpr (!FOLD) {
#pragma unroll
      for (int c = 0; c < NCOL; ++c) {
        const float* xc = x_in + size_t(c) * a.ldx + e;
        xv[c][j][0] = *reinterpret_cast<const float4*>(xc);
        xv[c][j][1] = *reinterpret_cast<const float4*>(xc + 4);
      }
    }
    if constexpr (NORM) {
      gv[j][0] = *reinterpret_cast<const float4*>(gain + e);
      gv[j][1] = *reinterpret_cast<const float4*>(gain + e + 4);
    }
  }
  // (pinned: left to the scheduler, the gain loads sink below the weight
  // loads, and the staging wait for them then drains every weight load)
  __builtin_amdgcn_sched_barrier(0);
  // 2. weight loads of the wave's row
  uint32_t lr = row < out ? row : out - 1;  // clamp; result discarded
  const uint32_t wr = (extra_row != NO_ROW && lr == out - 1) ? extra_row : row_base + lr;
  const uint8_t* rp = w_rows + size_t(wr) * row_bytes;
  const uint8_t* rp3 = DUAL ? w3_rows + size_t(wr) * row_bytes : nullptr;
  Raw8<WT> wb[KIT];
  Raw8<WT> wb3[DUAL ? KIT : 1];
#pragma unroll
  for (int k = 0; k < KA; ++k) {
    wb[k] = load_raw<WT>(rp, k * 512 + lane * 8);
    if constexpr (DUAL) wb3[k] = load_raw<WT>(rp3, k * 512 + lane * 8);
  }
  uint32_t fold_tok = 0, fold_tie = 0;
  if constexpr (FOLD) {
    // greedy keys of the logits (ids 4 i .. 4 i + 3 for float4 i)
    float m1 = -INFINITY, m2 = -INFINITY;
    uint32_t id1 = 0xffffffffu, cnt = 0;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const uint32_t id0 = 4u * (threadIdx.x + uint32_t(r) * NT);
      const float v4[4] = {lg[r].x, lg[r].y, lg[r].z, lg[r].w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if (v4[c] > -INFINITY) {
          ++cnt;
          greedy_add(m1, id1, m2, v4[c], id0 + uint32_t(c));
        }
      }
    }
    const float4* l4 = reinterpret_cast<const float4*>(a.fold.logits);
    for (uint32_t i = threadIdx.x + 2u * NT; i < a.fold.n / 4u; i += NT) {
      const float4 q = l4[i];
      const float v4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if (v4[c] > -INFINITY) {
          ++cnt;
          greedy_add(m1, id1, m2, v4[c], 4u * i + uint32_t(c));
        }
      }
    }
    greedy_wave(m1, id1, m2);
    cnt = wave_sum_u32(cnt);
    if (lane == 0) {
      fold_m1[wave] = m1;
      fold_m2[wave] = m2;
      fold_id[wave] = id1;
      fold_cnt[wave] = cnt;
    }
    __syncthreads();
    float a1 = fold_m1[0], a2 = fold_m2[0];
    uint32_t ai = fold_id[0], c = fold_cnt[0];
#pragma unroll
    for (int w = 1; w < WPB; ++w) {
      greedy_merge(a1, ai, a2, fold_m1[w], fold_id[w], fold_m2[w]);
      c += fold_cnt[w];
    }
    // no finite logit: the reference returns id 0 (a draw is still taken)
    fold_tok = c > 0 ? ai : 0u;
    fold_tie = (c > 0 && !greedy_unique(c, a1, a2)) ? 1u : 0u;
    // the embedding row (f16) of the sample
    const uint16_t* er = a.fold.emb + size_t(fold_tok) * IN;
#pragma unroll
    for (int j = 0; j < KW; ++j) {
      const int k = min(wave + j * WPB, KIT - 1);
      const uint4 raw = *reinterpret_cast<const uint4*>(er + k * 512 + lane * 8);
      const uint32_t h[4] = {raw.x, raw.y, raw.z, raw.w};
      float f[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f[2 * i] = half_bits_to_float(uint16_t(h[i] & 0xffffu));
        f[2 * i + 1] = half_bits_to_float(uint16_t(h[i] >> 16));
      }
      xv[0][j][0] = make_float4(f[0], f[1], f[2], f[3]);
      xv[0][j][1] = make_float4(f[4], f[5], f[6], f[7]);
    }
#pragma unroll
    for (int k = KA; k < KIT; ++k) wb[k] = load_raw<WT>(rp, k * 512 + lane * 8);
  }
  const uint32_t done = done_ptr ? __builtin_nontemporal_load(done_ptr) : 0u;
  // the argument-block fields used later are read now, while the loads above
  // are in flight (left to the compiler, the y pointer is read at the store)
  float eps = a.eps;
  float* ybase = a.y;
  uint32_t ldy = a.ldy;
  asm volatile("" : "+s"(eps), "+s"(ybase), "+s"(ldy));
  // RESID: the residual values are loaded now, behind the weight loads, so
  // the epilogue does not add a memory round trip to the wave's tail
  // (every lane reads its wave's row: one request, no branch, and a global
  // load whose wait drains only the loads issued before it)
  float yres[NCOL];
#pragma unroll
  for (int c = 0; c < NCOL; ++c) {
    yres[c] = 0.0f;
    if constexpr (EPI == EPI_RESID) yres[c] = gload_f32(ybase + size_t(c) * ldy + (row < out ? row : out - 1));
  }
  // 3. block sum of squares -> scale
#pragma unroll
  for (int c = 0; c < NCOL && NORM; ++c) {
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < KW; ++j) {
      if (wave + j * WPB < KIT) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float4 u = xv[c][j][h];
          ss += u.x * u.x + u.y * u.y + u.z * u.z + u.w * u.w;
        }
      }
    }
    ss = wave_sum(ss);
    if (lane == 0) red[c][wave] = ss;
  }
  if constexpr (NORM) __syncthreads();
  // 4. (normalised) x into LDS (and, xn_out, from block 0 to memory)
  const bool xn0 = NORM && !FOLD && a.xn_out != nullptr && blockIdx.x == 0;
#pragma unroll
  for (int c = 0; c < NCOL; ++c) {
    float scale = 1.0f;
    if constexpr (NORM) {
      float tot = 0.0f;
#pragma unroll
      for (int i = 0; i < WPB; ++i) tot += red[c][i];
      scale = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(tot, float(IN)), eps)));
    }
#pragma unroll
    for (int j = 0; j < KW; ++j) {
      const int k = wave + j * WPB;
      if (k < KIT) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          float4 u = xv[c][j][h];
          if constexpr (NORM) {
            const float4 g = gv[j][h];
            u.x = __fmul_rn(__fmul_rn(u.x, scale), g.x);
            u.y = __fmul_rn(__fmul_rn(u.y, scale), g.y);
            u.z = __fmul_rn(__fmul_rn(u.z, scale), g.z);
            u.w = __fmul_rn(__fmul_rn(u.w, scale), g.w);
          }
          xs[c][(k * 512 + lane * 8) / 4 + h] = u;
          if constexpr (NORM && !FOLD) {
            if (xn0) *reinterpret_cast<float4*>(a.xn_out + size_t(c) * a.ldx + k * 512 + lane * 8 + 4 * h) = u;
          }
        }
      }
    }
  }
  __syncthreads();
  if constexpr (FOLD) {
    // the sampler's side effects, once: the next input row (as f32), the
    // code, one SeededRng step
    if (blockIdx.x == 0 && !st_done) {
#pragma unroll
      for (int j = 0; j < KW; ++j) {
        const int k = wave + j * WPB;
        if (k < KIT) {
          float* xo = a.fold.x_out + k * 512 + lane * 8;
          *reinterpret_cast<float4*>(xo) = xv[0][j][0];
          *reinterpret_cast<float4*>(xo + 4) = xv[0][j][1];
        }
      }
      if (threadIdx.x == 0) {
        DevState* st = a.fold.st;
        st->rng = lcg_step(st_rng);
        st->codes_frame[a.fold.cb_index] = fold_tok;
        if (fold_tie) atomicOr(&st->err, ERR_GREEDY_TIE);
      }
    }
  }
  if (done) return;
  // 5. dot products against the LDS copy
  float acc[NCOL], acc3[NCOL];
#pragma unroll
  for (int c = 0; c < NCOL; ++c) acc[c] = acc3[c] = 0.0f;
#pragma unroll
  for (int k = 0; k < KIT; ++k) {
    float w[8], w3[8];
    decode8<WT>(wb[k], w);
    if constexpr (DUAL) decode8<WT>(wb3[k], w3);
#pragma unroll
    for (int c = 0; c < NCOL; ++c) {
      const float4 xa = xs[c][(k * 512 + lane * 8) / 4];
      const float4 xb = xs[c][(k * 512 + lane * 8) / 4 + 1];
      const float xv8[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[c] = fmaf(w[i], xv8[i], acc[c]);
      if constexpr (DUAL) {
#pragma unroll
        for (int i = 0; i < 8; ++i) acc3[c] = fmaf(w3[i], xv8[i], acc3[c]);
      }
    }
  }
  // 6. epilogue
#pragma unroll
  for (int c = 0; c < NCOL; ++c) {
    const float gsum = wave_sum(acc[c]);
    float u = 0.0f;
    if constexpr (DUAL) u = wave_sum(acc3[c]);
    if (lane == 0 && row < out) {
      float* dst = ybase + size_t(c) * ldy + row;
      if constexpr (EPI == EPI_STORE) {
        *dst = gsum;
      } else if constexpr (EPI == EPI_RESID) {
        *dst = __fadd_rn(yres[c], gsum);
      } else if constexpr (EPI == EPI_SWIGLU_SLOW) {
        const float sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf_glibc_wave(-gsum)));
        *dst = __fmul_rn(__fmul_rn(gsum, sig), u);
      } else {
        *dst = __fmul_rn(__fdiv_rn(gsum, __fadd_rn(1.0f, expf_glibc_wave(-gsum))), u);
      }
    }
  }
}

template <uint32_t WT, int NCOL, int EPI, int KIT, bool NORM = true, int WPB = 8, bool FOLD = false>
hipError_t gemv_n_launch(const GemvArgs& a, hipStream_t s) {
  const dim3 grid((a.out + WPB - 1) / WPB);
  if (a.row_bytes > UINT32_MAX) return hipErrorInvalidValue;
  hipLaunchKernelGGL((gemv_n_kernel<WT, NCOL, EPI, KIT, WPB, NORM, FOLD>), grid, dim3(64 * WPB), 0, s, a.w, a.w3, a.x,
                     a.norm, a.done, uint32_t(a.row_bytes), a.out, a.row_base, a.extra_row, a);
  return hipGetLastError();
}

// The greedy fold's shapes: one column into an RMSNorm + store linear with
// 512 / 1536 / 2560-wide rows (the Fast-AR wqkv of the S2-Pro family).
template <uint32_t WT>
hipError_t gemv_fold_launch(const GemvArgs& a, hipStream_t s) {
  if (!a.norm || !a.fold.emb || !a.fold.st || !a.fold.x_out || a.fold.n == 0 || a.fold.n % 4 ||
      reinterpret_cast<uintptr_t>(a.fold.logits) % 16 || reinterpret_cast<uintptr_t>(a.fold.emb) % 16 ||
      reinterpret_cast<uintptr_t>(a.fold.x_out) % 16 || a.fold.cb_index >= 16)
    return hipErrorInvalidValue;
  switch (a.in) {
    case 512: return gemv_n_launch<WT, 1, EPI_STORE, 1, true, 8, true>(a, s);
    case 1536: return gemv_n_launch<WT, 1, EPI_STORE, 3, true, 8, true>(a, s);
    case 2560:
      if (a.out <= 4096) return gemv_n_launch<WT, 1, EPI_STORE, 5, true, 16, true>(a, s);
      return gemv_n_launch<WT, 1, EPI_STORE, 5, true, 12, true>(a, s);
    default: return hipErrorNotSupported;
  }
}

// ---------------------------------------------------------------------------
// Decode GEMV, one column, each row's steps split over the block's waves.
//   The block owns R consecutive rows; wave w takes the 512-element steps
//   k = w, w + WPB, ... (k < KIT) of all R rows: it loads only those steps of
//   x into registers and issues its weight loads (R per step) before anything
//   waits.  x never goes through LDS: each x element is read once per block,
//   by the one wave that uses it, and reused across the R rows from
//   registers.  Each row's partial sums are reduced in the wave (DPP) and
//   then over the waves in a fixed order through LDS, so the result does not
//   depend on timing.  Lane r < R of wave 0 finishes row r; its residual
//   (RESID) is loaded with the weights.  This form keeps whole blocks per CU
//   where one row per wave would not (w2: 2560 rows of 9728 -> 512 blocks).
// ---------------------------------------------------------------------------
template <uint32_t WT, int NCOL, int EPI, int KIT, int WPB, int R>
__global__ __launch_bounds__(64 * WPB) void gemv_ks_kernel(const uint8_t* w_rows, const float* x_in,
                                                               const uint32_t* done_ptr, uint32_t row_bytes,
                                                               uint32_t out, uint32_t row_base, uint32_t extra_row,
                                                               GemvArgs a) {
  static_assert(EPI == EPI_STORE || EPI == EPI_RESID, "one matrix, no activation");
  static_assert(NCOL * R <= WAVE, "one epilogue lane per (column, row)");
  constexpr int KW = (KIT + WPB - 1) / WPB;
  __shared__ float part[NCOL][R][WPB];
  const int lane = threadIdx.x & (WAVE - 1);
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const uint32_t row0 = blockIdx.x * R;
  const uint32_t ldx = a.ldx;
  // 1. this wave's steps of x (a step past KIT re-reads the last one)
  //    No branch in the load phase: a branch around loads leaves the wait
  //    counts at the join conservative, and the first use then waits for
  //    nearly every load in flight.
  float4 xv[NCOL][KW][2];
#pragma unroll
  for (int j = 0; j < KW; ++j) {
    const uint32_t e = uint32_t(min(wave + j * WPB, KIT - 1)) * 512u + lane * 8u;
#pragma unroll
    for (int c = 0; c < NCOL; ++c) {
      xv[c][j][0] = *reinterpret_cast<const float4*>(x_in + size_t(c) * ldx + e);
      xv[c][j][1] = *reinterpret_cast<const float4*>(x_in + size_t(c) * ldx + e + 4);
    }
  }
  // 2. weight loads: step-major, so the dot loop consumes them in issue order;
  //    a step past KIT reads x's first lines instead (cached, no HBM bytes;
  //    the values are not used)
  const uint8_t* rp[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint32_t lr = min(row0 + uint32_t(r), out - 1u);  // clamp; result discarded
    const uint32_t wr = (extra_row != NO_ROW && lr == out - 1u) ? extra_row : row_base + lr;
    rp[r] = w_rows + size_t(wr) * row_bytes;
  }
  Raw8<WT> wb[KW][R];
#pragma unroll
  for (int j = 0; j < KW; ++j) {
    const bool live = wave + j * WPB < KIT;
    const uint32_t e = live ? uint32_t(wave + j * WPB) * 512u + lane * 8u : lane * 8u;
#pragma unroll
    for (int r = 0; r < R; ++r) wb[j][r] = load_raw<WT>(live ? rp[r] : reinterpret_cast<const uint8_t*>(x_in), e);
  }
  const uint32_t done = done_ptr ? __builtin_nontemporal_load(done_ptr) : 0u;
  float* ybase = a.y;
  uint32_t ldy = a.ldy;
  asm volatile("" : "+s"(ybase), "+s"(ldy));
  // lane c R + r finishes (column c, row r): its residual (clamped address),
  // behind the weight loads
  const uint32_t ec = min(uint32_t(lane) / uint32_t(R), uint32_t(NCOL) - 1u), er = uint32_t(lane) % uint32_t(R);
  const uint32_t my_row = min(row0 + er, out - 1u);
  const float yres = EPI == EPI_RESID ? gload_f32(ybase + size_t(ec) * ldy + my_row) : 0.0f;
  // 3. dot products of the wave's steps
  float acc[NCOL][R];
#pragma unroll
  for (int c = 0; c < NCOL; ++c)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[c][r] = 0.0f;
#pragma unroll
  for (int j = 0; j < KW; ++j) {
    if (wave + j * WPB < KIT) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float w[8];
        decode8<WT>(wb[j][r], w);
#pragma unroll
        for (int c = 0; c < NCOL; ++c) {
          const float xv8[8] = {xv[c][j][0].x, xv[c][j][0].y, xv[c][j][0].z, xv[c][j][0].w,
                                xv[c][j][1].x, xv[c][j][1].y, xv[c][j][1].z, xv[c][j][1].w};
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[c][r] = fmaf(w[i], xv8[i], acc[c][r]);
        }
      }
    }
  }
  // 4. per-row sums: the wave's, then the waves' in order
#pragma unroll
  for (int c = 0; c < NCOL; ++c) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float g = wave_sum(acc[c][r]);
      if (lane == 0) part[c][r][wave] = g;
    }
  }
  __syncthreads();
  if (done || wave != 0 || lane >= NCOL * R) return;
  const uint32_t row = row0 + er;
  if (row >= out) return;
  float gsum = part[ec][er][0];
#pragma unroll
  for (int i = 1; i < WPB; ++i) gsum += part[ec][er][i];
  ybase[size_t(ec) * ldy + row] = EPI == EPI_RESID ? __fadd_rn(yres, gsum) : gsum;
}

template <uint32_t WT, int NCOL, int EPI, int KIT, int WPB, int R>
hipError_t gemv_ks_launch(const GemvArgs& a, hipStream_t s) {
  if (a.row_bytes > UINT32_MAX) return hipErrorInvalidValue;
  const dim3 grid((a.out + R - 1) / R);
  hipLaunchKernelGGL((gemv_ks_kernel<WT, NCOL, EPI, KIT, WPB, R>), grid, dim3(64 * WPB), 0, s, a.w, a.x, a.done,
                     uint32_t(a.row_bytes), a.out, a.row_base, a.extra_row, a);
  return hipGetLastError();
}

// Row shapes of the S2-Pro family: 512 / 1536 (tiny), 2560, 4096, 9728.
// Returns hipErrorNotSupported for other row lengths.
template <uint32_t WT, int NCOL, int EPI>
hipError_t gemv_k_pick(const GemvArgs& a, hipStream_t s) {
  constexpr bool DUAL = (EPI == EPI_SWIGLU_SLOW || EPI == EPI_SWIGLU_FAST);
  constexpr int RS = DUAL ? 1 : 2;  // rows per wave for short rows
  if (a.norm) {
    switch (a.in) {
      case 512: return gemv_n_launch<WT, NCOL, EPI, 1>(a, s);
      case 1536: return gemv_n_launch<WT, NCOL, EPI, 3>(a, s);
      case 2560:
        // one column, one matrix: whole blocks per CU on 256 CUs (wqkv, 6144
        // rows: 12 waves, 512 blocks, 7.1 -> 6.6 us; a 4096-row head: 16
        // waves, 256 blocks, 5.6 -> 5.4 us); w1/w3 keep 8 (4 and 16 waves:
        // 18.9 and 20.3 us against 16.5)
        if constexpr (NCOL == 1 && !DUAL) {
          if (a.out <= 4096) return gemv_n_launch<WT, 1, EPI, 5, true, 16>(a, s);
          return gemv_n_launch<WT, 1, EPI, 5, true, 12>(a, s);
        }
        // (two columns keep 8: wqkv 8.4 us against 9.4 / 8.7 / 10.1 with 4 /
        // 12 / 16 waves, w1/w3 19.9 against 21.4 / 26.2 / 27.1)
        return gemv_n_launch<WT, NCOL, EPI, 5>(a, s);
      default: break;
    }
  }
  switch (a.in) {
    case 512: return gemv_k_launch<WT, NCOL, RS, EPI, 1, 4>(a, s);
    case 1536: return gemv_k_launch<WT, NCOL, RS, EPI, 3, 4>(a, s);
    case 2560: return gemv_k_launch<WT, NCOL, RS, EPI, 5, 4>(a, s);
    // long rows (wo, w2): x staged once per block in LDS.  Per-wave x reads
    // from L2/L1 were 2x the weight bytes; 2 / 4 waves per block keep 1280 /
    // 640 blocks for the 256 CUs (8 left a quarter of the CUs with two
    // blocks): w2 12.1 -> 10.9 us, wo 6.3 -> 5.9 us
    // wo at one column: 10 waves, one 256-block round with x staged 256
    // times instead of 1280 (5.3 -> 5.0 us); w2 in this form kept 4 (5 and
    // 10 waves: 10.5 and 10.9 us against 10.3)
    // (wo in the split-step form -- 8/4/8 waves x 10/5/5 rows -- ran the
    // default decode at 295.2-296.2 / 286.4-286.5 / 286.6-287.2 frames/s
    // against 299.5-300.3 with this one)
    // (two columns: 10 waves as well, 5.9 us against 7.6 / 6.5 / 7.4 with 2
    // / 4 / 8)
    case 4096: return gemv_n_launch<WT, NCOL, EPI, 8, false, 10>(a, s);
    // w2 at one column (F16): the split-step form, 10 waves x 5 rows, 512
    // blocks (default decode 300.3-300.6 frames/s against 298.2-298.4)
    case 9728:
      if constexpr (NCOL <= 2 && WT == W_F16 && (EPI == EPI_STORE || EPI == EPI_RESID))
        return gemv_ks_launch<WT, NCOL, EPI, 19, 10, 5>(a, s);
      return gemv_n_launch<WT, NCOL, EPI, 19, false, 4>(a, s);
    default: return hipErrorNotSupported;
  }
}

template <uint32_t WT, int EPI>
hipError_t gemv_k_ncol(int ncol, const GemvArgs& a, hipStream_t s) {
  if (ncol == 1) return gemv_k_pick<WT, 1, EPI>(a, s);
  return gemv_k_pick<WT, 2, EPI>(a, s);
}

template <uint32_t WT>
hipError_t gemv_k_epi(int epi, int ncol, const GemvArgs& a, hipStream_t s) {
  switch (epi) {
    case EPI_STORE: return gemv_k_ncol<WT, EPI_STORE>(ncol, a, s);
    case EPI_RESID: return gemv_k_ncol<WT, EPI_RESID>(ncol, a, s);
    case EPI_SWIGLU_SLOW: return gemv_k_ncol<WT, EPI_SWIGLU_SLOW>(ncol, a, s);
    case EPI_SWIGLU_FAST: return gemv_k_ncol<WT, EPI_SWIGLU_FAST>(ncol, a, s);
    default: return hipErrorInvalidValue;
  }
}

// ---------------------------------------------------------------------------
// Decode GEMV over repacked Q8_0 / Q4_0 rows (one column).
//   Lane l of a wave takes whole 32-element blocks b = 64 s + l (s = 0, 1,
//   ...) of its row: one 16-byte load (two for Q8_0) of the block's values
//   and one 2-byte scale load, all issued up front.  The block's sum
//   sum_j q_j x_j (Q4_0: q_j - 8) is taken in f32, scaled once by d and
//   added to the lane's running sum.
//   x (RMS-normalised when NORM, as in gemv_n_kernel) is staged once per
//   block in LDS with one spare float per 32 (block b at 33 b), so the
//   lanes' reads of their blocks fall in distinct banks.  One row (two for
//   SwiGLU: w1 and w3) per wave.
// ---------------------------------------------------------------------------
// x of a Q GEMV in LDS: the 32 elements of block b as eight 16-byte chunks,
// chunk c at position c ^ qswz(b), so that the chunk reads of 8 (or 16)
// consecutive lanes -- consecutive blocks -- hit distinct banks with 32 (or
// 64) banks; block b's sum of x follows the blocks (qsum_base).
__device__ __forceinline__ uint32_t qswz(uint32_t b) { return (b ^ (b >> 3)) & 7u; }

// sum_j q'_j x[c][j] of one block for NC columns, q' the stored unsigned value
// (Q4_0: the nibble, Q8_0: the byte + 128), each byte converted to f32 in one
// instruction; the caller subtracts 8 (128) times the block's sum of x.
template <uint32_t WT, int NC>
__device__ __forceinline__ void qblock_dot(const uint4 (&q)[WT == W_Q8_0 ? 2 : 1], const float* xs, uint32_t b,
                                           uint32_t xstride, float (&accb)[NC]) {
#pragma unroll
  for (int c = 0; c < NC; ++c) accb[c] = 0.0f;
  const float* xb = xs + b * 32u;
  const uint32_t sw = qswz(b);
  auto chunk = [&](int c, uint32_t ch) -> float4 {
    return *reinterpret_cast<const float4*>(xb + c * xstride + ((ch ^ sw) << 2));
  };
  auto dot4 = [&](uint32_t w, int c, uint32_t ch) {
    const float4 x = chunk(c, ch);
    float a = accb[c];
    // (w >> 8 i) & 0xff as f32 is one v_cvt_f32_ubyte<i>
    a = fmaf(float(w & 0xffu), x.x, a);
    a = fmaf(float((w >> 8) & 0xffu), x.y, a);
    a = fmaf(float((w >> 16) & 0xffu), x.z, a);
    a = fmaf(float(w >> 24), x.w, a);
    accb[c] = a;
  };
  if constexpr (WT == W_Q8_0) {
    const uint32_t qw[8] = {q[0].x, q[0].y, q[0].z, q[0].w, q[1].x, q[1].y, q[1].z, q[1].w};
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const uint32_t u = qw[m] ^ 0x80808080u;  // int8 q -> q + 128
#pragma unroll
      for (int c = 0; c < NC; ++c) dot4(u, c, uint32_t(m));
    }
  } else {
    const uint32_t qw[4] = {q[0].x, q[0].y, q[0].z, q[0].w};
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const uint32_t lo = qw[m] & 0x0f0f0f0fu, hi = (qw[m] >> 4) & 0x0f0f0f0fu;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        dot4(lo, c, uint32_t(m));      // elements 4 m .. 4 m + 3
        dot4(hi, c, uint32_t(4 + m));  // elements 16 + 4 m ..
      }
    }
  }
}

template <uint32_t WT, int EPI, int KIT, int WPB, bool NORM, int NC = 1>
__global__ __launch_bounds__(64 * WPB) void gemv_q_kernel(const uint8_t* qp, const uint8_t* qp3, const uint16_t* qs,
                                                          const uint16_t* qs3, const float* x_in, const float* gain,
                                                          const uint32_t* done_ptr, uint32_t out, GemvArgs a) {
  constexpr bool DUAL = (EPI == EPI_SWIGLU_SLOW || EPI == EPI_SWIGLU_FAST);
  constexpr uint32_t IN = uint32_t(KIT) * WAVE * 8, NB = IN / 32;
  constexpr uint32_t QW = WT == W_Q8_0 ? 2 : 1;  // 16-byte loads per block
  constexpr int KW = (KIT + WPB - 1) / WPB;
  constexpr uint32_t XS = NB * 32 + NB;  // floats per staged column: the blocks, then their sums
  __shared__ float xs[NC * XS];
  __shared__ float red[NC][WPB];
  const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x >> 6;
  const uint32_t row = blockIdx.x * WPB + wave;

  // 1. this wave's 512-element steps of x (every column) and of the gain
  float4 xv[NC][KW][2], gv[KW][2];
#pragma unroll
  for (int j = 0; j < KW; ++j) {
    const int k = min(wave + j * WPB, KIT - 1);
    const uint32_t e = k * 512 + lane * 8;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      xv[c][j][0] = *reinterpret_cast<const float4*>(x_in + size_t(c) * a.ldx + e);
      xv[c][j][1] = *reinterpret_cast<const float4*>(x_in + size_t(c) * a.ldx + e + 4);
    }
    if constexpr (NORM) {
      gv[j][0] = *reinterpret_cast<const float4*>(gain + e);
      gv[j][1] = *reinterpret_cast<const float4*>(gain + e + 4);
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // x / gain loads before the weights (as in gemv_n_kernel)
  // 2. block values and scales of the wave's row (clamped; unused past the
  //    end).  SwiGLU rows index w1's and w3's blocks as one list of 2 NB
  //    (i < NB: w1 block i, else w3 block i - NB), which fills the lanes
  //    better than two lists of NB (80 blocks per row: 3 groups against 4)
  constexpr uint32_t NL = DUAL ? 2 * NB : NB, NG = (NL + WAVE - 1) / WAVE;
  const uint32_t lr = row < out ? row : out - 1;
  const uint4* qrow = reinterpret_cast<const uint4*>(qp + size_t(lr) * NB * QW * 16);
  const uint4* qrow3 = DUAL ? reinterpret_cast<const uint4*>(qp3 + size_t(lr) * NB * QW * 16) : qrow;
  const uint16_t* srow = qs + size_t(lr) * NB;
  const uint16_t* srow3 = DUAL ? qs3 + size_t(lr) * NB : srow;
  uint4 wq[NG][QW];
  uint16_t wd[NG];
#pragma unroll
  for (uint32_t st = 0; st < NG; ++st) {
    const uint32_t i = min(st * WAVE + lane, NL - 1);
    const bool second = DUAL && i >= NB;
    const uint32_t b = second ? i - NB : i;
    const uint4* src = second ? qrow3 : qrow;
#pragma unroll
    for (uint32_t j = 0; j < QW; ++j) wq[st][j] = src[b * QW + j];
    wd[st] = (second ? srow3 : srow)[b];
  }
  const uint32_t done = done_ptr ? __builtin_nontemporal_load(done_ptr) : 0u;
  float eps = a.eps;
  float* ybase = a.y;
  uint32_t ldy = a.ldy;
  asm volatile("" : "+s"(eps), "+s"(ybase), "+s"(ldy));
  // RESID: the residual values go out behind the weight loads (as in
  // gemv_n_kernel)
  float yres[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    yres[c] = 0.0f;
    if constexpr (EPI == EPI_RESID) yres[c] = gload_f32(ybase + size_t(c) * ldy + (row < out ? row : out - 1));
  }
  // 3. block sum of squares -> scale (per column)
  if constexpr (NORM) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      float ss = 0.0f;
#pragma unroll
      for (int j = 0; j < KW; ++j) {
        if (wave + j * WPB < KIT) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const float4 u = xv[c][j][h];
            ss += u.x * u.x + u.y * u.y + u.z * u.z + u.w * u.w;
          }
        }
      }
      ss = wave_sum(ss);
      if (lane == 0) red[c][wave] = ss;
    }
    __syncthreads();
  }
  // 4. (normalised) x into LDS in swizzled chunks (qswz), and each block's sum
  //    of x (the lane's 8 elements, then the 4 lanes of a block)
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    float scale = 1.0f;
    if constexpr (NORM) {
      float tot = 0.0f;
#pragma unroll
      for (int i = 0; i < WPB; ++i) tot += red[c][i];
      scale = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(tot, float(IN)), eps)));
    }
#pragma unroll
    for (int j = 0; j < KW; ++j) {
      const int k = wave + j * WPB;
      if (k < KIT) {
        float part = 0.0f;
        const uint32_t e0 = k * 512 + lane * 8, b = e0 >> 5;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          float4 u = xv[c][j][h];
          if constexpr (NORM) {
            const float4 g = gv[j][h];
            u.x = __fmul_rn(__fmul_rn(u.x, scale), g.x);
            u.y = __fmul_rn(__fmul_rn(u.y, scale), g.y);
            u.z = __fmul_rn(__fmul_rn(u.z, scale), g.z);
            u.w = __fmul_rn(__fmul_rn(u.w, scale), g.w);
          }
          const uint32_t ch = ((e0 & 31u) >> 2) + h;  // chunk of the block
          *reinterpret_cast<float4*>(xs + c * XS + b * 32u + ((ch ^ qswz(b)) << 2)) = u;
          part += (u.x + u.y) + (u.z + u.w);
        }
        part += dpp_f32<DPP_QUAD_XOR1>(part);
        part += dpp_f32<DPP_QUAD_XOR2>(part);
        if ((lane & 3) == 0) xs[c * XS + NB * 32u + b] = part;
      }
    }
  }
  __syncthreads();
  if (done) return;
  // 5. blocks: f32 sum of q_j x_j, scaled by d, into w1's (acc) or w3's
  //    (acc3) sum
  float acc[NC], acc3[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) acc[c] = acc3[c] = 0.0f;
#pragma unroll
  for (uint32_t st = 0; st < NG; ++st) {
    const uint32_t i = st * WAVE + lane;
    const bool live = i < NL, second = DUAL && i >= NB;
    const uint32_t b = live ? (second ? i - NB : i) : 0u;
    const float d = half_bits_to_float(wd[st]);
    float bs[NC];
    qblock_dot<WT, NC>(wq[st], xs, b, XS, bs);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const float v = d * fmaf(-(WT == W_Q8_0 ? 128.0f : 8.0f), xs[c * XS + NB * 32u + b], bs[c]);
      acc[c] = (live && !second) ? __fadd_rn(acc[c], v) : acc[c];
      if constexpr (DUAL) acc3[c] = (live && second) ? __fadd_rn(acc3[c], v) : acc3[c];
    }
  }
  // 6. epilogue (as gemv_n_kernel)
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const float gsum = wave_sum(acc[c]);
    float u = 0.0f;
    if constexpr (DUAL) u = wave_sum(acc3[c]);
    if (lane == 0 && row < out) {
      float* dst = ybase + size_t(c) * ldy + row;
      if constexpr (EPI == EPI_STORE) {
        *dst = gsum;
      } else if constexpr (EPI == EPI_RESID) {
        *dst = __fadd_rn(yres[c], gsum);
      } else if constexpr (EPI == EPI_SWIGLU_SLOW) {
        const float sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf_glibc_wave(-gsum)));
        *dst = __fmul_rn(__fmul_rn(gsum, sig), u);
      } else {
        *dst = __fmul_rn(__fdiv_rn(gsum, __fadd_rn(1.0f, expf_glibc_wave(-gsum))), u);
      }
    }
  }
}

template <uint32_t WT, int EPI, int KIT, int WPB, bool NORM, int NC = 1>
hipError_t gemv_q_launch(const GemvArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((gemv_q_kernel<WT, EPI, KIT, WPB, NORM, NC>), dim3((a.out + WPB - 1) / WPB), dim3(64 * WPB), 0,
                     s, a.qp, a.qp3, a.qs, a.qs3, a.x, a.norm, a.done, a.out, a);
  return hipGetLastError();
}

// Block shapes as the F16 GEMV (whole blocks per CU on the S2-Pro shapes);
// hipErrorNotSupported for row lengths or epilogues without an instance.
template <uint32_t WT, int EPI, int NC>
hipError_t gemv_q_pick(const GemvArgs& a, hipStream_t s) {
  constexpr bool DUAL = (EPI == EPI_SWIGLU_SLOW || EPI == EPI_SWIGLU_FAST);
  if (a.norm) {
    switch (a.in) {
      case 512: return gemv_q_launch<WT, EPI, 1, 8, true, NC>(a, s);
      case 1536: return gemv_q_launch<WT, EPI, 3, 8, true, NC>(a, s);
      case 2560:
        // 80 blocks per row leave the second lane group a quarter full; one
        // matrix (wqkv, heads) is faster on the GGUF-layout kernel (Q8_0
        // wqkv 5.9 against 6.6 us), w1 / w3 share the x reads and gain
        // (Q8_0 15.4 -> 12.6 us)
        if constexpr (DUAL) return gemv_q_launch<WT, EPI, 5, 8, true, NC>(a, s);
        return hipErrorNotSupported;
      default: return hipErrorNotSupported;
    }
  }
  if constexpr (DUAL) {
    return hipErrorNotSupported;
  } else {
    switch (a.in) {
      case 512: return gemv_q_launch<WT, EPI, 1, 4, false, NC>(a, s);
      case 1536: return gemv_q_launch<WT, EPI, 3, 4, false, NC>(a, s);
      case 4096: return gemv_q_launch<WT, EPI, 8, 10, false, NC>(a, s);
      // 4 waves as the F16 w2 (8 and 10 waves: Q4_0 8.1 and 7.5 us, Q8_0
      // 10.1 and 9.3 us, against 7.3 and 8.0).  Two columns of 9728-wide
      // rows would hold 80 x registers per lane (one wave per SIMD): the
      // GGUF-layout kernel takes them
      case 9728:
        if constexpr (NC == 1) return gemv_q_launch<WT, EPI, 19, 4, false, 1>(a, s);
        return hipErrorNotSupported;
      default: return hipErrorNotSupported;
    }
  }
}

template <uint32_t WT, int NC>
hipError_t gemv_q_epi(int epi, const GemvArgs& a, hipStream_t s) {
  switch (epi) {
    case EPI_STORE: return gemv_q_pick<WT, EPI_STORE, NC>(a, s);
    case EPI_RESID: return gemv_q_pick<WT, EPI_RESID, NC>(a, s);
    case EPI_SWIGLU_SLOW: return gemv_q_pick<WT, EPI_SWIGLU_SLOW, NC>(a, s);
    case EPI_SWIGLU_FAST: return gemv_q_pick<WT, EPI_SWIGLU_FAST, NC>(a, s);
    default: return hipErrorNotSupported;
  }
}

// One thread per (row, block): the GGUF block's values and scale into the
// two planes.
__global__ __launch_bounds__(256) void repack_q_kernel(const uint8_t* rows, size_t row_bytes, uint32_t wt,
                                                       uint32_t nb, uint32_t nrows, uint8_t* qplane,
                                                       uint16_t* splane) {
  const size_t i = size_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= size_t(nb) * nrows) return;
  const size_t r = i / nb, b = i % nb;
  const uint32_t bb = wt == W_Q8_0 ? 34u : 18u, qb = bb - 2u;
  const uint8_t* blk = rows + r * row_bytes + b * bb;
  splane[i] = uint16_t(blk[0] | (uint32_t(blk[1]) << 8));
  uint8_t* dst = qplane + i * qb;
  for (uint32_t j = 0; j < qb; ++j) dst[j] = blk[2 + j];
}

bool gemv_k_supported(uint32_t in) { return in == 512 || in == 1536 || in == 2560 || in == 4096 || in == 9728; }


// ---------------------------------------------------------------------------
// RMSNorm over `ncol` vectors (one block per column).
// ---------------------------------------------------------------------------
// One block per column.  Rows of up to 256 * RN_REG elements are held in
// registers (x and the gain loaded in one batch); longer rows loop.
constexpr int RN_REG = 16;
__global__ __launch_bounds__(256) void rms_norm_kernel(const float* x, const float* w, float* y, uint32_t n,
                                                       float eps, const uint32_t* done) {
  __shared__ float red[4];
  const uint32_t c = blockIdx.x;
  const float* xc = x + size_t(c) * n;
  float ss = 0.0f;
  if (n <= 256u * RN_REG) {
    float xv[RN_REG], gv[RN_REG];
#pragma unroll
    for (int j = 0; j < RN_REG; ++j) {
      const uint32_t i = threadIdx.x + 256u * j;
      xv[j] = i < n ? xc[i] : 0.0f;
      gv[j] = i < n ? w[i] : 0.0f;
    }
    if (done && *done) return;
#pragma unroll
    for (int j = 0; j < RN_REG; ++j) ss += xv[j] * xv[j];
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float tot = (red[0] + red[1]) + (red[2] + red[3]);
    const float scale = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(tot, float(n)), eps)));
#pragma unroll
    for (int j = 0; j < RN_REG; ++j) {
      const uint32_t i = threadIdx.x + 256u * j;
      if (i < n) y[size_t(c) * n + i] = __fmul_rn(__fmul_rn(xv[j], scale), gv[j]);
    }
    return;
  }
  if (done && *done) return;
  for (uint32_t i = threadIdx.x; i < n; i += 256) ss += xc[i] * xc[i];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float tot = (red[0] + red[1]) + (red[2] + red[3]);
  const float scale = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(tot, float(n)), eps)));
  for (uint32_t i = threadIdx.x; i < n; i += 256) y[size_t(c) * n + i] = __fmul_rn(__fmul_rn(xc[i], scale), w[i]);
}

// ---------------------------------------------------------------------------
// Per-head QK-norm (optional) + NORMAL RoPE for one wave: pairs (2p, 2p+1)
// rotated by the host-built (cos, sin) row of the position.
// ---------------------------------------------------------------------------
// f32 -> f16 bits, round to nearest even (v_cvt_f16_f32), and back
__device__ __forceinline__ uint16_t f16_bits_rn(float x) { return __half_as_ushort(__float2half_rn(x)); }
__device__ __forceinline__ float f16_round(float x) { return __half2float(__float2half_rn(x)); }

// Four f16 values (8 bytes) as a float4 (exact)
__device__ __forceinline__ float4 load_half4(const uint16_t* p) {
  const uint2 r = *reinterpret_cast<const uint2*>(p);
  return make_float4(half_bits_to_float(uint16_t(r.x & 0xffffu)), half_bits_to_float(uint16_t(r.x >> 16)),
                     half_bits_to_float(uint16_t(r.y & 0xffffu)), half_bits_to_float(uint16_t(r.y >> 16)));
}

// dst16 non-null: the result is stored as f16 bits there instead of dst
__device__ __forceinline__ void head_norm_rope(const float* src, const float* norm, float eps,
                                               const float2* rope_row, uint32_t hd, uint32_t lane, float* dst,
                                               uint16_t* dst16 = nullptr) {
  float scale = 1.0f;
  if (norm) {
    float ss = 0.0f;
    for (uint32_t i = lane; i < hd; i += 64) ss += src[i] * src[i];
    ss = wave_sum(ss);
    scale = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, float(hd)), eps)));
  }
  for (uint32_t p = lane; p < hd / 2; p += 64) {
    float x0 = src[2 * p], x1 = src[2 * p + 1];
    if (norm) {
      x0 = __fmul_rn(__fmul_rn(x0, scale), norm[2 * p]);
      x1 = __fmul_rn(__fmul_rn(x1, scale), norm[2 * p + 1]);
    }
    const float cs = rope_row[p].x, sn = rope_row[p].y;
    const float y0 = __fsub_rn(__fmul_rn(x0, cs), __fmul_rn(x1, sn));
    const float y1 = __fadd_rn(__fmul_rn(x0, sn), __fmul_rn(x1, cs));
    if (dst16) {
      dst16[2 * p] = f16_bits_rn(y0);
      dst16[2 * p + 1] = f16_bits_rn(y1);
    } else {
      dst[2 * p] = y0;
      dst[2 * p + 1] = y1;
    }
  }
}

// QK-norm + RoPE + KV append as a standalone step (one wave per head; grid
// (H + 2 Hkv, ncol)); the decode path fuses the same math into attention.
__global__ __launch_bounds__(64) void qkv_post_kernel(QkvPostArgs a) {
  if (a.done && *a.done) return;
  const uint32_t hi = blockIdx.x, col = blockIdx.y, lane = threadIdx.x;
  const uint32_t pos = (a.pos_ptr ? *a.pos_ptr : 0u) + a.pos_offset + col;
  if (pos >= a.max_seq) {
    if (lane == 0 && a.err) atomicOr(a.err, ERR_KV_OVERFLOW);
    return;
  }
  const uint32_t hd = a.hd, width = (a.H + 2 * a.Hkv) * hd;
  const float* src = a.qkv + size_t(col) * width + size_t(hi) * hd;
  const float2* rope_row = a.rope + size_t(pos) * (hd / 2);
  if (hi < a.H) {
    head_norm_rope(src, a.q_norm, a.eps, rope_row, hd, lane, a.q_out + size_t(col) * a.H * hd + size_t(hi) * hd);
  } else if (hi < a.H + a.Hkv) {
    const size_t off = (size_t(hi - a.H) * a.max_seq + pos) * hd;
    if (a.kv_f16)
      head_norm_rope(src, a.k_norm, a.eps, rope_row, hd, lane, nullptr, reinterpret_cast<uint16_t*>(a.k_cache) + off);
    else
      head_norm_rope(src, a.k_norm, a.eps, rope_row, hd, lane, a.k_cache + off);
  } else {
    const size_t off = (size_t(hi - a.H - a.Hkv) * a.max_seq + pos) * hd;
    if (a.kv_f16) {
      uint16_t* vd = reinterpret_cast<uint16_t*>(a.v_cache) + off;
      for (uint32_t i = lane; i < hd; i += 64) vd[i] = f16_bits_rn(src[i]);
    } else {
      float* vd = a.v_cache + off;
      for (uint32_t i = lane; i < hd; i += 64) vd[i] = src[i];
    }
  }
}

// ---------------------------------------------------------------------------
// Decode attention for one layer: QK-norm + RoPE of the new positions, KV
// append, split-T GQA attention over the cache, cross-chunk combine.
//   grid (max_chunks, Hkv, ncol), 256 threads; block (c, g, col) covers cache
//   positions [CH c, CH c + CH) of kv head g for query column col, and wave w
//   serves q head g * rep + w.  Every load that does not depend on the
//   position goes out first and together: the state words, the q rows and the
//   whole K/V tile (every tile position lies inside the cache, so the tile is
//   read before the position is known and positions past it are ignored).
//   Positions of this launch's own columns are recomputed from their qkv rows
//   (another block may still be appending them).  With one chunk the block
//   writes the output.  Otherwise it writes its (max, sum, o) partial and:
//     LAST = false: attn_combine_kernel merges the partials afterwards;
//     LAST = true:  the partials are written with agent-scope atomic stores
//       (coherent across the XCD L2s without a cache write-back), a counter
//       per (col, g) elects the last block of the pair, which merges them with
//       agent-scope loads and resets the counter for the next launch.
// ---------------------------------------------------------------------------
template <int HD, int CH, bool LAST, bool KH, bool GATHER = false, bool WARM = true>
__global__ __launch_bounds__(256) void attn_partial_kernel(const float* qkv, void* k_cache, void* v_cache,
                                                             const uint32_t* pos_ptr, const uint32_t* done_ptr,
                                                             uint32_t ncol_cf, uint32_t max_seq, uint32_t kv_stride,
                                                             uint32_t shape, AttnArgs a) {
  // ncol | check_from << 8: both among the preloaded arguments, so blocks
  // below check_from issue their tile loads without waiting on a scalar load
  const uint32_t ncol = ncol_cf & 0xffu, check_from = ncol_cf >> 8;
  using KT = std::conditional_t<KH, uint16_t, float>;  // cache element: f16 bits or f32
  constexpr int KS = HD + 1;
  constexpr int PER = CH * HD / 4 / 256;  // float4 per thread per tile
  static_assert(PER >= 1, "tile too small");
  __shared__ float kt[CH * KS];
  __shared__ float vt[CH * HD];
  __shared__ float qs[GEMV_WAVES][HD];
  __shared__ float ps[GEMV_WAVES][CH];
  __shared__ float knew[4][HD], vnew[4][HD];
  __shared__ uint32_t is_last;
  __shared__ float gm1[GATHER ? GEMV_WAVES : 1], gm2[GATHER ? GEMV_WAVES : 1];
  __shared__ uint32_t gid[GATHER ? GEMV_WAVES : 1], gcnt[GATHER ? GEMV_WAVES : 1];
  // warming planes after the attention blocks (laid out last); launches
  // without warming use the form compiled without this path (its keep-alive
  // asm statement makes the compiler treat memory as written, which turns
  // the state-word reads below into vector loads)
  if constexpr (WARM) {
    if (__builtin_expect(blockIdx.z >= ncol, 0)) {
      const uint32_t L = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
      l2_warm(a.warm, L, L - gridDim.x * gridDim.y * ncol, threadIdx.x, 256u);
      return;
    }
  }
  const uint32_t H = shape & 0xffu, Hkv = (shape >> 8) & 0xffu, cps_ = (shape >> 16) & 0xffu, sw = shape >> 24;
  const uint32_t chunk = blockIdx.x, g = blockIdx.y, col = blockIdx.z;
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t rep = H / Hkv;
  const uint32_t width = (H + 2 * Hkv) * HD;
  // column col = (sequence seq, its column lc); each sequence has its own
  // KV cache, position word and done word
  const uint32_t cps = cps_, seq = col / cps, lc = col % cps;
  const float* row = qkv + size_t(col) * width;
  KT* kseq = reinterpret_cast<KT*>(k_cache) + size_t(seq) * kv_stride;
  KT* vseq = reinterpret_cast<KT*>(v_cache) + size_t(seq) * kv_stride;
  const KT* kc = kseq + size_t(g) * max_seq * HD;
  const KT* vc = vseq + size_t(g) * max_seq * HD;
  const uint32_t t0 = chunk * CH;

  // 0. position-independent loads, all in flight together: the state words
  //    and the K/V tile (addresses from the preloaded arguments) first, then
  //    the new rows and the QK-norm gains (gain pointers from the argument
  //    block)
  const uint32_t done = opt_word(done_ptr ? done_ptr + size_t(seq) * sw : nullptr);
  const uint32_t pbase = opt_word(pos_ptr ? pos_ptr + size_t(seq) * sw : nullptr);
  // GATHER: what picks the table row goes out before the tile, so that the
  // wait for it leaves the tile in flight: the logits of the greedy fold (or
  // the sampled code word) and the state words of the sampler's side effects
  //   (no branch: absent inputs read stand-ins, so all of these go out
  //   together; the sampled-code form reads a unit gain row as its logits)
  float4 glg[GATHER ? 4 : 1];
  uint32_t code_word = 0, st_done = 1;
  if constexpr (GATHER) {
    const bool fl = a.fold.logits != nullptr;
    greedy_loads<GEMV_WAVES, 4>(fl ? a.fold.logits : kUnitGain, fl ? a.fold.n : 4u, glg);
    code_word = opt_word(a.code_ptr);
    st_done = opt_word(fl ? &a.fold.st->done : nullptr);
  }
  // chunks from check_from on may lie past the sequence (the bound is known
  // where the launch is recorded): they wait for the position and a dead one
  // ends here, before its tile is read
  if constexpr (!GATHER) {
    if (check_from != 0u && chunk >= check_from) {
      if (done || t0 >= pbase + a.pos_offset + lc + 1u) return;
    }
  }
  float4 kr[PER], vr[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const uint32_t idx = j * 256 + tid;
    const uint32_t t = idx / (HD / 4), d = (idx % (HD / 4)) * 4;
    const uint32_t tt = min(t0 + t, max_seq - 1);
    if constexpr (KH) {
      kr[j] = load_half4(kc + size_t(tt) * HD + d);
      vr[j] = load_half4(vc + size_t(tt) * HD + d);
    } else {
      kr[j] = *reinterpret_cast<const float4*>(kc + size_t(tt) * HD + d);
      vr[j] = *reinterpret_cast<const float4*>(vc + size_t(tt) * HD + d);
    }
  }
  // the whole tile is issued before anything that needs the position word
  // (left to itself, the scheduler moves the position arithmetic, and so the
  // wait for the state words, in between the tile loads)
  if constexpr (!GATHER) __builtin_amdgcn_sched_barrier(0);
  // rotation rows of the query position and of column `wave`'s position:
  // they need only the position word, so they go out with the loads above
  // (addresses clamped into the table, which has max_seq rows; values for
  // lanes and positions outside the ranges are dropped below)
  const uint32_t pos = pbase + a.pos_offset + lc;
  const uint32_t base = pos - lc;   // first position of this sequence's columns
  const uint32_t tk = base + wave;  // position of column `wave`
  const uint32_t hl = lane & (HD / 2 - 1);
  float2 rp_raw, rk_raw;
  auto rope_loads = [&] {
    rp_raw = gload_f2(a.rope + size_t(min(pos, max_seq - 1)) * (HD / 2) + hl);
    rk_raw = gload_f2(a.rope + size_t(min(tk, max_seq - 1)) * (HD / 2) + hl);
  };
  if constexpr (GATHER) rope_loads();
  // one column from a table row: its code (the greedy sample of the logits,
  // reduced by every block, or a sampled code), and block 0 carries the
  // sampler's side effects (input row, code, SeededRng step, tie flag)
  if constexpr (GATHER) {
    uint32_t code;
    if (a.fold.logits) {
      uint32_t tie;
      block_greedy_keys<GEMV_WAVES, 4>(glg, a.fold.logits, a.fold.n, gm1, gm2, gid, gcnt, code, tie);
      if (chunk == 0 && g == 0 && !st_done) {
        // the next input row (f16 -> f32), 8 elements per thread with every
        // load of a pass issued before its stores (fold.dim % 8 == 0)
        const uint4* er = reinterpret_cast<const uint4*>(a.fold.emb + size_t(code) * a.fold.dim);
        const uint32_t n8 = a.fold.dim / 8u;
        for (uint32_t b0 = 0; b0 < n8; b0 += 2u * 256u) {
          uint4 raw[2];
#pragma unroll
          for (int u = 0; u < 2; ++u) raw[u] = er[min(b0 + tid + uint32_t(u) * 256u, n8 - 1u)];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const uint32_t b = b0 + tid + uint32_t(u) * 256u;
            if (b < n8) {
              const uint32_t h[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
              float f[8];
#pragma unroll
              for (int k = 0; k < 4; ++k) {
                f[2 * k] = half_bits_to_float(uint16_t(h[k] & 0xffffu));
                f[2 * k + 1] = half_bits_to_float(uint16_t(h[k] >> 16));
              }
              float4* xo = reinterpret_cast<float4*>(a.fold.x_out + size_t(b) * 8u);
              xo[0] = make_float4(f[0], f[1], f[2], f[3]);
              xo[1] = make_float4(f[4], f[5], f[6], f[7]);
            }
          }
        }
        if (tid == 0) {
          DevState* st = a.fold.st;
          st->rng = lcg_step(st->rng);
          st->codes_frame[a.fold.cb_index] = code;
          if (tie) atomicOr(&st->err, ERR_GREEDY_TIE);
        }
      }
    } else {
      code = min(code_word, a.fold.n - 1u);  // table rows: fold.n
    }
    row = a.qkv_rows + size_t(code) * width;
  }
  // q row of head g * rep + wave and the k / v rows of this sequence's
  // columns (wave w <-> column w <= lc): every lane loads from a clamped,
  // valid address and lanes outside the ranges drop the value, so no branch
  // holds the loads back
  const uint32_t e2 = 2 * (lane & (HD / 2 - 1));
  const bool qlane = wave < rep && lane < HD / 2;
  const bool kwave = wave < cps && wave <= lc;
  const float2 qraw = *reinterpret_cast<const float2*>(row + size_t(g * rep + min(wave, rep - 1)) * HD + e2);
  const float* r2 = GATHER ? row : qkv + size_t(seq * cps + min(wave, lc)) * width;
  const float2 kraw = *reinterpret_cast<const float2*>(r2 + size_t(H + g) * HD + e2);
  const float2 vraw = *reinterpret_cast<const float2*>(r2 + size_t(H + Hkv + g) * HD + e2);
  // (global-space loads: a generic pointer would make flat loads, whose
  // waits drain every load in flight, the K/V tile included)
  const float2 qn = gload_f2(reinterpret_cast<const float2*>((a.q_norm ? a.q_norm : kUnitGain) + e2));
  const float2 kn = gload_f2(reinterpret_cast<const float2*>((a.k_norm ? a.k_norm : kUnitGain) + e2));
  if constexpr (!GATHER) rope_loads();
  const float2 zero2 = make_float2(0.f, 0.f);
  const float2 qv = qlane ? qraw : zero2;
  const float2 kx = (kwave && lane < HD / 2) ? kraw : zero2;
  const float2 vx = (kwave && lane < HD / 2) ? vraw : zero2;
  const uint32_t T = pos + 1;
  const uint32_t nch = (T + CH - 1) / CH;
  if (done || pos >= max_seq || chunk >= nch) {
    if (!done && pos >= max_seq && tid == 0 && chunk == 0 && a.err)
      atomicOr(a.err + size_t(seq) * sw, ERR_KV_OVERFLOW);
    // The exit path also reads the loaded values, so the compiler keeps the
    // loads ahead of this branch (where they overlap the state read) instead
    // of sinking them behind it.  The test is never true for finite data.
    float keep = qv.x + qv.y + kx.x + kx.y + vx.x + vx.y + qn.x + qn.y + kn.x + kn.y + rp_raw.x + rp_raw.y +
                 rk_raw.x + rk_raw.y;
    if constexpr (GATHER) {
#pragma unroll
      for (int r = 0; r < 4; ++r) keep += (glg[r].x + glg[r].y) + (glg[r].z + glg[r].w);
      keep += float(code_word) + float(st_done);
    }
#pragma unroll
    for (int j = 0; j < PER; ++j)
      keep += (kr[j].x + kr[j].y) + (kr[j].z + kr[j].w) + (vr[j].x + vr[j].y) + (vr[j].z + vr[j].w);
    if (keep == 3.0e38f && a.err) atomicOr(a.err, 0u);
    return;
  }
  const uint32_t t1 = min(T, t0 + CH), nt = t1 - t0;
  const uint32_t lo = max(t0, min(base, t1));  // [lo, t1): positions of this launch

  // 1. q and the new k: QK-norm (optional) + rotation
  const bool khere = kwave && tk >= t0 && tk < t1;
  const float2 rp = qlane ? rp_raw : make_float2(1.f, 0.f);
  const float2 rk = (khere && lane < HD / 2) ? rk_raw : make_float2(1.f, 0.f);
  if (khere) {
    float x0 = kx.x, x1 = kx.y;
    if (a.k_norm) {
      const float ss = wave_sum(x0 * x0 + x1 * x1);
      const float sc = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, float(HD)), a.eps)));
      x0 = __fmul_rn(__fmul_rn(x0, sc), kn.x);
      x1 = __fmul_rn(__fmul_rn(x1, sc), kn.y);
    }
    if (lane < HD / 2) {
      knew[wave][2 * lane] = __fsub_rn(__fmul_rn(x0, rk.x), __fmul_rn(x1, rk.y));
      knew[wave][2 * lane + 1] = __fadd_rn(__fmul_rn(x0, rk.y), __fmul_rn(x1, rk.x));
      vnew[wave][2 * lane] = vx.x;
      vnew[wave][2 * lane + 1] = vx.y;
    }
  }
  if (wave < rep) {
    float x0 = qv.x, x1 = qv.y;
    if (a.q_norm) {
      const float ss = wave_sum(x0 * x0 + x1 * x1);
      const float sc = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, float(HD)), a.eps)));
      x0 = __fmul_rn(__fmul_rn(x0, sc), qn.x);
      x1 = __fmul_rn(__fmul_rn(x1, sc), qn.y);
    }
    if (qlane) {
      qs[wave][2 * lane] = __fsub_rn(__fmul_rn(x0, rp.x), __fmul_rn(x1, rp.y));
      qs[wave][2 * lane + 1] = __fadd_rn(__fmul_rn(x0, rp.y), __fmul_rn(x1, rp.x));
    }
  }
  // 2. tile to LDS (positions >= lo are replaced below or unused)
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const uint32_t idx = j * 256 + tid;
    const uint32_t t = idx / (HD / 4), d = (idx % (HD / 4)) * 4;
    kt[t * KS + d] = kr[j].x;
    kt[t * KS + d + 1] = kr[j].y;
    kt[t * KS + d + 2] = kr[j].z;
    kt[t * KS + d + 3] = kr[j].w;
    *reinterpret_cast<float4*>(&vt[t * HD + d]) = vr[j];
  }
  __syncthreads();
  // 3. this launch's positions in the chunk: columns lo - base .. t1 - base - 1
  for (uint32_t c2 = lo - base; c2 < t1 - base; ++c2) {
    const uint32_t tn = base + c2 - t0;
    for (uint32_t i = tid; i < HD; i += 256) {
      // an f16 cache holds the rounded values, and this step reads them so
      const float kn = KH ? f16_round(knew[c2][i]) : knew[c2][i];
      const float vn = KH ? f16_round(vnew[c2][i]) : vnew[c2][i];
      kt[tn * KS + i] = kn;
      vt[tn * HD + i] = vn;
      if (c2 == lc) {  // SlowArKvCache::write_token for this column's position
        if constexpr (KH) {
          kseq[(size_t(g) * max_seq + pos) * HD + i] = f16_bits_rn(kn);
          vseq[(size_t(g) * max_seq + pos) * HD + i] = f16_bits_rn(vn);
        } else {
          kseq[(size_t(g) * max_seq + pos) * HD + i] = kn;
          vseq[(size_t(g) * max_seq + pos) * HD + i] = vn;
        }
      }
    }
  }
  __syncthreads();
  // 4. scores and chunk softmax: position lane % CH, the two halves of the
  //    wave take the two halves of the head dimension (two accumulators
  //    each), joined by one cross-half exchange
  float m = -INFINITY, l = 0.0f;
  static_assert(CH == 32, "two half-waves of 32 positions");
  if (wave < rep) {
    const uint32_t tp = lane & (CH - 1), hh = lane / CH;
    const float* qh = &qs[wave][hh * (HD / 2)];
    const float* kh = &kt[tp * KS + hh * (HD / 2)];
    float d0 = 0.0f, d1 = 0.0f;
#pragma unroll 16
    for (int d = 0; d < HD / 2; d += 2) {
      d0 = fmaf(qh[d], kh[d], d0);
      d1 = fmaf(qh[d + 1], kh[d + 1], d1);
    }
    float dsum = d0 + d1;
    dsum += __shfl_xor(dsum, 32);
    const bool live = hh == 0 && tp < nt;
    const float s = live ? dsum * a.scale : -INFINITY;
    m = wave_max(s);
    const float p = live ? expf(s - m) : 0.0f;
    l = wave_sum(p);
    if (lane < CH) ps[wave][lane] = p;
  }
  __syncthreads();
  // 5. PV (lane = head-dim element)
  float* pair_part = a.part + (size_t(col) * Hkv + g) * a.max_chunks * rep * (HD + 2);
  if (wave < rep) {
    const uint32_t h = g * rep + wave;
    float o[HD / 64];
#pragma unroll
    for (int j = 0; j < HD / 64; ++j) o[j] = 0.0f;
    for (uint32_t t = 0; t < nt; ++t) {
      const float pv = ps[wave][t];
#pragma unroll
      for (int j = 0; j < HD / 64; ++j) o[j] = fmaf(pv, vt[t * HD + lane + 64 * j], o[j]);
    }
    if (nch == 1) {
      float* dst = a.out + size_t(col) * H * HD + size_t(h) * HD;
      const float inv = 1.0f / l;
#pragma unroll
      for (int j = 0; j < HD / 64; ++j) dst[lane + 64 * j] = o[j] * inv;
    } else {
      float* part = pair_part + (size_t(chunk) * rep + wave) * (HD + 2);
      if constexpr (LAST) {
        if (lane == 0) {
          __hip_atomic_store(part, m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(part + 1, l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (int j = 0; j < HD / 64; ++j)
          __hip_atomic_store(part + 2 + lane + 64 * j, o[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        if (lane == 0) {
          part[0] = m;
          part[1] = l;
        }
#pragma unroll
        for (int j = 0; j < HD / 64; ++j) part[2 + lane + 64 * j] = o[j];
      }
    }
  }
  if constexpr (LAST) {
    if (nch == 1) return;
    // 6. the partial stores have completed before the block's arrival is counted
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    uint32_t* cnt = a.counters + size_t(col) * Hkv + g;
    if (tid == 0) {
      const uint32_t prev = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      is_last = prev + 1 == nch;
      if (prev + 1 == nch) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!is_last) return;
    // 7. merge: thread i -> (head w, element d) pairs
    const size_t cstride = size_t(rep) * (HD + 2);
    for (uint32_t i = tid; i < rep * HD; i += 256) {
      const uint32_t w = i / HD, d = i % HD;
      const float* pb = pair_part + size_t(w) * (HD + 2);
      float M = -INFINITY;
      for (uint32_t c = 0; c < nch; ++c)
        M = fmaxf(M, __hip_atomic_load(pb + c * cstride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
      float L = 0.0f, acc = 0.0f;
      for (uint32_t c = 0; c < nch; ++c) {
        const float* pc = pb + c * cstride;
        const float mc = __hip_atomic_load(pc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const float lc = __hip_atomic_load(pc + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const float oc = __hip_atomic_load(pc + 2 + d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const float f = expf(mc - M);
        L = fmaf(lc, f, L);
        acc = fmaf(oc, f, acc);
      }
      a.out[size_t(col) * H * HD + size_t(g * rep + w) * HD + d] = acc / L;
    }
  }
}

// Merge of the per-chunk (max, sum, o) partials: grid (H, ncol), HD threads.
// MAXC > 0: the state words and the partials of every chunk slot (up to
// MAXC >= max_chunks) are loaded together before the position is known;
// slots past this launch's chunk count hold stale data and are ignored.
// MAXC == 0: a loop over the chunks (any max_chunks).
template <int HD, int CH, int MAXC>
__global__ __launch_bounds__(HD) void attn_combine_kernel(const float* part, float* out, const uint32_t* pos_ptr,
                                                            const uint32_t* done_ptr, uint32_t ncol, uint32_t max_chunks,
                                                            uint32_t shape, uint32_t pos_offset, AttnArgs a) {
  const uint32_t H = shape & 0xffu, Hkv = (shape >> 8) & 0xffu, cps = (shape >> 16) & 0xffu, sw = shape >> 24;
  const uint32_t h = blockIdx.x, col = blockIdx.y, d = threadIdx.x;
  const uint32_t rep = H / Hkv, g = h / rep, w = h % rep;
  const float* pbase = part + ((size_t(col) * Hkv + g) * max_chunks * rep + w) * (HD + 2);
  const size_t stride = size_t(rep) * (HD + 2);
  const uint32_t seq = col / cps, lc = col % cps;
  if constexpr (MAXC > 0) {
    static_assert(MAXC <= HD, "one thread per chunk slot");
    __shared__ float2 ml[HD];  // one slot per thread: an unconditional store keeps its load up front
    // no branch before these loads: every slot is read (threads past MAXC
    // re-read the last one), the result is discarded at the store when the
    // launch has nothing to merge; the state words go out last, so the
    // wait for them (they are made wave-uniform right after their loads)
    // leaves the partials in flight no longer than they take anyway
    const float2 mlv =
        gload_f2(reinterpret_cast<const float2*>(pbase + size_t(min(min(d, uint32_t(MAXC) - 1u), max_chunks - 1)) * stride));
    float oc[MAXC];
#pragma unroll
    for (int c = 0; c < MAXC; ++c) oc[c] = gload_f32(pbase + size_t(min(uint32_t(c), max_chunks - 1)) * stride + 2 + d);
    uint32_t done, pb;
    opt_words2(done_ptr, pos_ptr, size_t(seq) * sw, done, pb);
    ml[d] = mlv;
    __syncthreads();
    const uint32_t pos = pb + pos_offset + lc;
    const bool live = !done && pos < a.max_seq;
    const uint32_t nch = live ? (pos + CH) / CH : 0u;
    float M = -INFINITY;
#pragma unroll
    for (int c = 0; c < MAXC; ++c)
      if (uint32_t(c) < nch) M = fmaxf(M, ml[c].x);
    // each chunk's weight once per block (thread c), not once per thread
    __shared__ float fw[MAXC];
    if (d < uint32_t(MAXC)) fw[d] = d < nch ? expf(ml[d].x - M) : 0.0f;
    __syncthreads();
    float L = 0.0f, acc = 0.0f;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
      if (uint32_t(c) < nch) {
        const float f = fw[c];
        L = fmaf(ml[c].y, f, L);
        acc = fmaf(oc[c], f, acc);
      }
    }
    if (nch > 1) out[size_t(col) * H * HD + size_t(h) * HD + d] = acc / L;
  } else {
    // many chunks: the chunk maxima and weights in parallel over the
    // threads, then the weighted sum of the partials with 16 loads in flight
    constexpr int NWV = HD / 64;
    __shared__ float fs[ATTN_MAX_CHUNKS];
    __shared__ float rm[NWV], rl[NWV];
    const uint32_t done = opt_word(done_ptr ? done_ptr + size_t(seq) * sw : nullptr);
    const uint32_t pb = opt_word(pos_ptr ? pos_ptr + size_t(seq) * sw : nullptr);
    const uint32_t pos = pb + pos_offset + lc;
    if (done || pos >= a.max_seq) return;
    const uint32_t nch = (pos + CH) / CH;
    if (nch <= 1) return;
    const uint32_t lane = d & 63u, wv = d >> 6;
    float mloc = -INFINITY;
    for (uint32_t c = d; c < nch; c += HD) mloc = fmaxf(mloc, pbase[c * stride]);
    mloc = wave_max(mloc);
    if (lane == 0) rm[wv] = mloc;
    __syncthreads();
    float M = rm[0];
#pragma unroll
    for (int w = 1; w < NWV; ++w) M = fmaxf(M, rm[w]);
    float lloc = 0.0f;
    for (uint32_t c = d; c < nch; c += HD) {
      const float f = expf(pbase[c * stride] - M);
      fs[c] = f;
      lloc = fmaf(pbase[c * stride + 1], f, lloc);
    }
    lloc = wave_sum(lloc);
    if (lane == 0) rl[wv] = lloc;
    __syncthreads();
    float L = rl[0];
#pragma unroll
    for (int w = 1; w < NWV; ++w) L += rl[w];
    float acc = 0.0f;
    for (uint32_t c0 = 0; c0 < nch; c0 += 16) {
      float ov[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) ov[j] = pbase[size_t(min(c0 + j, nch - 1)) * stride + 2 + d];
#pragma unroll
      for (int j = 0; j < 16; ++j) acc = fmaf(c0 + j < nch ? fs[c0 + j] : 0.0f, ov[j], acc);
    }
    out[size_t(col) * H * HD + size_t(h) * HD + d] = acc / L;
  }
}

// ---------------------------------------------------------------------------
// Slow-AR embedding (time-major ids) -- one block per token.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void embed_kernel(EmbedArgs a) {
  const uint32_t chunks = (a.dim + 255) / 256;
  if (__builtin_expect(blockIdx.y >= chunks, 0)) {  // warming rows after the embedding blocks (laid out last)
    const uint32_t L = blockIdx.x + gridDim.x * blockIdx.y;
    l2_warm(a.warm, L, L - gridDim.x * chunks, threadIdx.x, 256u);
    return;
  }
  const uint32_t t = blockIdx.x;
  const uint32_t ncb = min(a.num_codebooks, 16u);
  const uint32_t cdim = a.num_codebooks + 1;
  // 1. the done word and the token ids in one round of loads
  const uint32_t done = a.done ? *a.done : 0u;
  int32_t tok[17];
  if (a.tokens) {
    const int32_t* tr = a.tokens + size_t(t) * cdim;
#pragma unroll
    for (int k = 0; k < 17; ++k) tok[k] = tr[min(uint32_t(k), ncb)];
  } else {
    // build_step_input: [main, cb0..cb(n-1)] when main is semantic, else [main, 0..]
    const DevState* st = a.state + t;  // one sequence per token row
    tok[0] = int32_t(st->main_token);
#pragma unroll
    for (int k = 0; k < 16; ++k) tok[1 + k] = int32_t(st->codes_frame[k]);
    const uint32_t main = uint32_t(tok[0]);
    if (!(main >= a.sem_begin && main <= a.sem_end)) {
#pragma unroll
      for (int k = 0; k < 16; ++k) tok[1 + k] = 0;
    }
  }
  if (done) return;
  uint32_t id = uint32_t(tok[0]);
  if (tok[0] < 0 || id >= a.vocab) {
    if (threadIdx.x == 0 && blockIdx.y == 0 && a.err) atomicOr(a.err, ERR_TOKEN_RANGE);
    id = 0;
  }
  const bool sem = id >= a.sem_begin && id <= a.sem_end;
  // codebook rows; unused slots read row 0 (their values are not summed)
  uint32_t rows[16];
  bool bad = false;
#pragma unroll
  for (int cb = 0; cb < 16; ++cb) {
    uint32_t r = uint32_t(tok[1 + cb]) + uint32_t(cb) * a.codebook_size;
    const bool used = sem && uint32_t(cb) < ncb;
    if (used && (tok[1 + cb] < 0 || r >= a.cb_rows)) {
      bad = true;
      r = 0;
    }
    rows[cb] = used ? r : 0u;
  }
  if (bad && threadIdx.x == 0 && blockIdx.y == 0 && a.err) atomicOr(a.err, ERR_TOKEN_RANGE);
  const float sc = (a.scale_enabled && sem) ? a.sem_scale : 1.0f;
  // 2. grid (tokens, 256-element chunks): one element per thread; the
  //    element of every row is loaded in one batch (no branch around the
  //    loads), then summed in the reference's order
  const uint32_t i0 = blockIdx.y * 256 + threadIdx.x;
  const uint32_t i = min(i0, a.dim - 1);
  float v = half_bits_to_float(a.emb[size_t(id) * a.dim + i]);
  float e[16];
#pragma unroll
  for (int cb = 0; cb < 16; ++cb) e[cb] = half_bits_to_float(a.cb_emb[size_t(rows[cb]) * a.dim + i]);
  // the sum is formed on both paths, so no branch separates the loads
  float cs = 0.0f;
#pragma unroll
  for (int cb = 0; cb < 16; ++cb)
    if (uint32_t(cb) < ncb) cs = __fadd_rn(cs, e[cb]);
  if (sem) v = __fadd_rn(v, cs);
  if (a.scale_enabled) v = __fmul_rn(v, sc);
  if (i0 < a.dim) a.h[size_t(t) * a.dim + i0] = v;
}

__device__ __forceinline__ uint32_t sem_to_code(uint32_t tok, uint32_t sem_begin, uint32_t sem_end,
                                                uint32_t codebook_size) {
  if (tok < sem_begin || tok > sem_end) return 0;
  const uint32_t c = tok - sem_begin;
  return c >= codebook_size ? codebook_size - 1 : c;
}

// grid (blocks over dim, sequences): sequence b reads slow_hidden[b] and
// writes its two Fast-AR input rows fh[b][0..1].  A finished sequence keeps
// its codes but its rows are still rewritten, so the Fast-AR passes that
// run for the rest of a batch see bounded inputs.
__global__ __launch_bounds__(256) void fast_begin_kernel(DevState* st0, const float* slow_hidden,
                                                         const uint16_t* fast_emb, float* fh, uint32_t dim,
                                                         uint32_t codebook_size, uint32_t sem_begin,
                                                         uint32_t sem_end) {
  const uint32_t b = blockIdx.y;
  DevState* st = st0 + b;
  const uint32_t code = sem_to_code(st->main_token, sem_begin, sem_end, codebook_size);
  if (!st->done && blockIdx.x == 0 && threadIdx.x == 0) st->codes_frame[0] = code;
  const float* hid = slow_hidden + size_t(b) * dim;
  float* f = fh + size_t(b) * 2 * dim;
  for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < dim; i += gridDim.x * 256) {
    f[i] = hid[i];
    f[dim + i] = half_bits_to_float(fast_emb[size_t(code) * dim + i]);
  }
}

// ---------------------------------------------------------------------------
// Sampler: exact restatement of sample_token (top-k -> force-include ->
// temperature softmax -> top-p -> renormalise -> discrete draw) on one block.
// Candidates are given in ascending vocabulary-id order; every id outside
// the candidate set (or masked) has logit -inf.  Sequential f32 sums are
// done by one thread in the reference's order.
// ---------------------------------------------------------------------------
// Sort key of a finite logit: ascending key == descending value (-0 == +0).
// Non-finite / masked / padding entries use 0xffffffff, above every finite key.
__device__ __forceinline__ uint32_t value_key(float v) {
  if (v == 0.0f) v = 0.0f;
  const uint32_t bits = __float_as_uint(v);
  const uint32_t ord = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
  return ~ord;
}

__device__ __forceinline__ float key_value(uint32_t k) {
  const uint32_t ord = ~k;
  const uint32_t bits = (ord & 0x80000000u) ? (ord & 0x7fffffffu) : ~ord;
  return __uint_as_float(bits);
}

constexpr uint32_t NO_KEY = 0xffffffffu;

struct SampleShared {
  uint32_t ckey[SAMPLE_MAX];   // candidate keys in candidate (ascending id) order
  uint32_t skey[SAMPLE_MAX];   // keys in sorted order
  float probs[SAMPLE_MAX + 4]; // probs and pref double as the sort's exchange buffer
  float pref[SAMPLE_MAX + 4];  // running sums
  float redf[SAMPLE_THREADS / WAVE];
  float rede[SAMPLE_THREADS / WAVE];
  uint32_t redu[SAMPLE_THREADS / WAVE];
  uint32_t redk[SAMPLE_THREADS / WAVE];
  float bcast_f;
  uint32_t bcast_u[4];
  uint64_t rng;                // SeededRng state (read and advanced by thread 0)
};

__device__ __forceinline__ double lcg_next_unit(uint64_t* s) {
  *s = lcg_step(*s);
  const uint64_t mant = (*s >> 11) & ((1ull << 53) - 1ull);
  return double(mant) / double(1ull << 53);
}

// Block-wide sum of one uint32 per thread (result in every thread).
__device__ __forceinline__ uint32_t block_sum_u32(uint32_t v, SampleShared& sh) {
  constexpr uint32_t NW = SAMPLE_THREADS / WAVE;
  const uint32_t lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x >> 6;
  v = wave_sum_u32(v);
  __syncthreads();
  if (lane == 0) sh.redk[wave] = v;
  __syncthreads();
  uint32_t t = 0;
#pragma unroll
  for (uint32_t w = 0; w < NW; ++w) t += sh.redk[w];
  return t;
}

// Median of three unsigned words: with c = 0 the min of a and b, with
// c = ~0 the max (one VALU op for a compare-exchange half).
__device__ __forceinline__ uint32_t med3_u32(uint32_t a, uint32_t b, uint32_t c) {
  uint32_t d;
  asm("v_med3_u32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
  return d;
}

// Word of the lane `x` lanes away (lane ^ x) within a wave, for 0 < x < WAVE:
// DPP quad permutes for x < 4, bit-mask swizzles within 32 lanes below 32,
// a permute through the LDS crossbar otherwise.
template <uint32_t X>
__device__ __forceinline__ uint32_t lane_xor(uint32_t v) {
  if constexpr (X == 1) return uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0xB1, 0xF, 0xF, false));  // [1,0,3,2]
  else if constexpr (X == 2) return uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0x4E, 0xF, 0xF, false));  // [2,3,0,1]
  else if constexpr (X == 3) return uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0x1B, 0xF, 0xF, false));  // [3,2,1,0]
  else if constexpr (X < 32) return uint32_t(__builtin_amdgcn_ds_swizzle(int(v), int(0x1Fu | (X << 10))));
  else return uint32_t(__shfl_xor(int(v), int(X), WAVE));
}

// Ascending bitonic sort of P = E * SAMPLE_THREADS 32-bit keys in registers:
// element e = r * SAMPLE_THREADS + tid is register r of thread tid.  Stage K
// (merging sorted runs of K / 2) starts with the partners e ^ (K - 1) (each
// K-block folded onto itself), then e ^ J for J = K / 4 .. 1; of each pair
// the element whose bit J (K / 2 on the first step) is set keeps the max.
// With the fold no step needs a direction, so a compare-exchange half is one
// med3 against a mask.  Partners in the same thread are registers; in the
// same wave, lane permutes; otherwise they are exchanged through `xbuf`
// (2 * P words, double-buffered: one barrier per step).  K and J are template
// constants, so register indices are static.
template <int E, uint32_t K, uint32_t J, bool FOLD>
__device__ __forceinline__ void bitonic_step(uint32_t (&key)[E], uint32_t* xbuf, uint32_t& par) {
  constexpr uint32_t NT = SAMPLE_THREADS;
  constexpr uint32_t P = uint32_t(E) * NT;
  constexpr uint32_t X = FOLD ? K - 1 : J;  // partner = e ^ X
  constexpr uint32_t TX = X & (NT - 1), RX = X / NT;
  const uint32_t tid = threadIdx.x;
  // all ones where bit J of e is set (that element keeps the max)
  auto upper = [&](int r) -> uint32_t {
    if constexpr (J >= NT) return ((uint32_t(r) * NT) & J) ? ~0u : 0u;
    else return 0u - ((tid / J) & 1u);
  };
  if constexpr (TX == 0) {  // same thread (J >= NT, not a fold)
#pragma unroll
    for (int r = 0; r < E; ++r) {
      const int rp = r ^ int(RX);
      if (rp > r) {
        const uint32_t x = key[r], y = key[rp];
        key[r] = min(x, y);
        key[rp] = max(x, y);
      }
    }
  } else if constexpr (RX == 0 && TX < WAVE) {  // same wave
#pragma unroll
    for (int r = 0; r < E; ++r) key[r] = med3_u32(key[r], lane_xor<TX>(key[r]), upper(r));
  } else {
    uint32_t* buf = xbuf + par * P;
#pragma unroll
    for (int r = 0; r < E; ++r) buf[r * NT + tid] = key[r];
    __syncthreads();
#pragma unroll
    for (int r = 0; r < E; ++r) key[r] = med3_u32(key[r], buf[(uint32_t(r) ^ RX) * NT + (tid ^ TX)], upper(r));
    par ^= 1u;
  }
}

template <int E, uint32_t K, uint32_t J>
__device__ __forceinline__ void bitonic_merge(uint32_t (&key)[E], uint32_t* xbuf, uint32_t& par) {
  bitonic_step<E, K, J, false>(key, xbuf, par);
  if constexpr (J > 1) bitonic_merge<E, K, J / 2>(key, xbuf, par);
}

template <int E, uint32_t K>
__device__ __forceinline__ void bitonic_stages(uint32_t (&key)[E], uint32_t* xbuf, uint32_t& par) {
  bitonic_step<E, K, K / 2, true>(key, xbuf, par);
  if constexpr (K >= 4) bitonic_merge<E, K, K / 4>(key, xbuf, par);
  if constexpr (K < uint32_t(E) * SAMPLE_THREADS) bitonic_stages<E, 2 * K>(key, xbuf, par);
}

// upper_sorted (block-uniform): registers E/2 .. E-1 already hold ascending
// keys (one real key, then padding), as for n = E/2 * SAMPLE_THREADS + 1
// candidates: only the lower half is sorted, then the last stage merges the
// halves.  The lower half's exchanges use xbuf words [0, P), the first full
// exchange words [P, 2P), so no step writes what the previous one may still
// be reading.
template <int E>
__device__ __forceinline__ void bitonic_sort_regs(uint32_t (&key)[E], uint32_t* xbuf, bool upper_sorted = false) {
  uint32_t par = 0;
  if constexpr (E >= 2) {
    if (upper_sorted) {
      constexpr uint32_t P = uint32_t(E) * SAMPLE_THREADS;
      uint32_t (&lo)[E / 2] = *reinterpret_cast<uint32_t(*)[E / 2]>(&key[0]);
      bitonic_stages<E / 2, 2>(lo, xbuf, par);
      par = 1;
      bitonic_step<E, P, P / 2, true>(key, xbuf, par);
      bitonic_merge<E, P, P / 4>(key, xbuf, par);
      return;
    }
  }
  bitonic_stages<E, 2>(key, xbuf, par);
}

// One 32-element step of a sequential sum: add the batch into cs in order and
// leave the running sums in the batch registers.
__device__ __forceinline__ void chain_batch(float4 (&v)[8], float& cs) {
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    cs = __fadd_rn(cs, v[t].x);
    v[t].x = cs;
    cs = __fadd_rn(cs, v[t].y);
    v[t].y = cs;
    cs = __fadd_rn(cs, v[t].z);
    v[t].z = cs;
    cs = __fadd_rn(cs, v[t].w);
    v[t].w = cs;
  }
}

__device__ __forceinline__ void chain_load(float4 (&v)[8], const float* p) {
#pragma unroll
  for (int t = 0; t < 8; ++t) v[t] = *reinterpret_cast<const float4*>(p + 4 * t);
}

__device__ __forceinline__ void chain_store(const float4 (&v)[8], float* prefix) {
#pragma unroll
  for (int t = 0; t < 8; ++t) *reinterpret_cast<float4*>(prefix + 4 * t) = v[t];
}

// Running sum j of a batch (j uniform; unrolled selects, no indexed registers).
__device__ __forceinline__ float chain_pick(const float4 (&v)[8], uint32_t j) {
  float r = 0.0f;
#pragma unroll
  for (uint32_t t = 0; t < 8; ++t) {
    r = j == 4 * t + 0 ? v[t].x : r;
    r = j == 4 * t + 1 ? v[t].y : r;
    r = j == 4 * t + 2 ? v[t].z : r;
    r = j == 4 * t + 3 ? v[t].w : r;
  }
  return r;
}

// Count of running sums of a batch below thr: the offset of the first one
// >= thr, as the sums of non-negative terms never decrease.
__device__ __forceinline__ uint32_t chain_below(const float4 (&v)[8], float thr) {
  uint32_t c = 0;
#pragma unroll
  for (int t = 0; t < 8; ++t)
    c += (v[t].x < thr ? 1u : 0u) + (v[t].y < thr ? 1u : 0u) + (v[t].z < thr ? 1u : 0u) + (v[t].w < thr ? 1u : 0u);
  return c;
}

struct ChainCut {
  uint32_t cut;  // first i < n with run(i) >= thr; n if none
  float sum;     // run(cut); the total run(n - 1) (0 for n = 0) if none
  float at_sum;  // run(at) when at < n
};

// Sequential f32 running sums run(i) = fl(run(i - 1) + p[i]), run(-1) = 0,
// in index order on one lane (the reference's sampling loops add term by
// term): the first index whose running sum reaches thr (a NaN thr never
// does), the running sum there, and the running sum at one more index `at`.
// The terms must be non-negative when thr is a number (the running sums then
// never decrease and the first crossing is found from a batch's sums).
// Fast phase: groups of G batches of 32 terms read from LDS into one of two
// register sets, the next batch's reads issued before the current batch is
// added, one counter wait per batch and one test per group (waits and
// branches between the dependent adds cost more than the reads).  A group
// that reaches thr or holds `at` is added again from its start, batch by
// batch (the same adds in the same order, so the same sums), to settle the
// result; so are the last terms.  The chain stops once both results are
// settled or (absorb: terms also non-increasing) once a term that bounds
// every later one (the next term, or at a group's end the last term added)
// is below half an ulp of the running sum: no later term changes the sum.
// PREFIX: every running sum is also written to prefix (batch by batch
// throughout).
template <bool PREFIX>
__device__ __forceinline__ ChainCut seq_chain(const float* p, uint32_t n, float thr, bool absorb, uint32_t at,
                                              float* prefix) {
  constexpr uint32_t B = 32, G = 4, GT = G * B;
  ChainCut r{n, 0.0f, 0.0f};
  float cs = 0.0f;
  uint32_t i = 0;
  bool found = false, at_open = at < n;
  auto absorbs = [&](float next) -> bool {  // next < half an ulp of cs
    return absorb && cs > 0.0f && next < __uint_as_float(__float_as_uint(cs) & 0x7f800000u) * 0x1p-24f;
  };
  // the batch [i - B, i) has been added and its sums are in v: record what it
  // settles; true when the chain can stop (next: the term at i, if any)
  auto settle = [&](const float4 (&v)[8], bool has_next, float next) -> bool {
    const uint32_t base = i - B;
    if (PREFIX) chain_store(v, prefix + base);
    if (!found && cs >= thr) {
      found = true;
      const uint32_t k = chain_below(v, thr);
      r.cut = base + k;
      r.sum = chain_pick(v, k);
    }
    if (at_open && at - base < B) {
      r.at_sum = chain_pick(v, at - base);
      at_open = false;
    }
    if (found && !at_open) return true;
    return has_next && absorbs(next);
  };
  // stopped early: with no crossing the total is cs; an `at` not reached is
  // past the absorbed point, where every running sum is cs
  auto finish = [&]() -> ChainCut {
    if (!found) r.sum = cs;
    if (at_open) r.at_sum = cs;
    return r;
  };
  while (true) {
    bool event = false;
    if (!PREFIX && i + GT <= n) {
      // reads past the last full batch re-read an earlier, 16-byte aligned
      // address (never added)
      const uint32_t last = (n - B) & ~3u;
      float4 va[8], vb[8];
      chain_load(va, p + i);
      do {
        const float cs0 = cs;
        float tl = 0.0f;  // the group's last term
#pragma unroll
        for (uint32_t g = 0; g < G; g += 2) {
          chain_load(vb, p + min(i + B, last));
          __builtin_amdgcn_s_waitcnt(0xC87F);  // lgkmcnt(8): va has arrived, vb may be in flight
          __builtin_amdgcn_sched_barrier(0);
          chain_batch(va, cs);
          __builtin_amdgcn_sched_barrier(0);
          i += B;
          chain_load(va, p + min(i + B, last));
          __builtin_amdgcn_s_waitcnt(0xC87F);
          __builtin_amdgcn_sched_barrier(0);
          tl = vb[7].w;
          chain_batch(vb, cs);
          __builtin_amdgcn_sched_barrier(0);
          i += B;
        }
        if ((!found && cs >= thr) || (at_open && at < i)) {  // settle this group batch by batch
          i -= GT;
          cs = cs0;
          event = true;
          break;
        }
        // every later term is at most the group's last one (the terms never
        // increase), which is in registers: no wait for the next batch's reads
        if (absorbs(tl)) return finish();
      } while (i + GT <= n);
    }
    const uint32_t end = event ? i + GT : n;
    while (i + B <= end) {
      float4 v[8];
      chain_load(v, p + i);
      chain_batch(v, cs);
      i += B;
      if (settle(v, i < n, i < n ? p[i] : 0.0f)) return finish();
    }
    if (!event) break;
  }
  for (; i < n; ++i) {
    cs = __fadd_rn(cs, p[i]);
    if (PREFIX) prefix[i] = cs;
    if (!found && cs >= thr) {
      found = true;
      r.cut = i;
      r.sum = cs;
    }
    if (i == at) r.at_sum = cs;
  }
  if (!found) r.sum = cs;
  return r;
}

// Candidate index of the m-th (0-based, ascending index) candidate whose key
// is kc; candidates ascend in id, so this is the m-th smallest id among the
// candidates with that value.  Whole block.
__device__ __forceinline__ uint32_t block_nth_match(SampleShared& sh, uint32_t n, uint32_t kc, uint32_t m) {
  constexpr uint32_t NT = SAMPLE_THREADS, NW = SAMPLE_THREADS / WAVE;
  const uint32_t tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid >> 6;
  uint32_t base = 0;
  __syncthreads();  // earlier readers of bcast_u[2] are done
  if (tid == 0) sh.bcast_u[2] = 0xffffffffu;
  for (uint32_t r0 = 0; r0 < n; r0 += NT) {
    const uint32_t j = r0 + tid;
    const bool match = j < n && sh.ckey[j] == kc;
    const uint64_t b = __ballot(match);
    __syncthreads();
    if (lane == 0) sh.redk[wave] = uint32_t(__popcll(b));
    __syncthreads();
    uint32_t before = base, total = base;
#pragma unroll
    for (uint32_t w = 0; w < NW; ++w) {
      before += w < wave ? sh.redk[w] : 0u;
      total += sh.redk[w];
    }
    if (match && before + uint32_t(__popcll(b & ((1ull << lane) - 1ull))) == m) sh.bcast_u[2] = j;
    base = total;
    if (total > m) break;
  }
  __syncthreads();
  return sh.bcast_u[2];
}

// j-th id (ascending) of [0, vocab) that is not the id of a finite candidate
// (the masked tail of the item list).  Whole block; binary search with a
// block-wide count per step.
template <int E>
__device__ uint32_t block_masked_id(SampleShared& sh, const uint32_t* ids, uint32_t n, uint32_t j, uint32_t vocab) {
  // this thread's candidates: id and key (keys from the candidate-order copy)
  uint32_t cid[E], ckey_r[E];
#pragma unroll
  for (int r = 0; r < E; ++r) {
    const uint32_t i = uint32_t(r) * SAMPLE_THREADS + threadIdx.x;
    cid[r] = i < n ? (ids ? ids[i] : i) : 0xffffffffu;
    ckey_r[r] = sh.ckey[i];
  }
  uint32_t lo = 0, hi = vocab ? vocab - 1 : 0;
  while (lo < hi) {
    const uint32_t mid = lo + (hi - lo) / 2;
    uint32_t le = 0;
#pragma unroll
    for (int r = 0; r < E; ++r) le += (ckey_r[r] != NO_KEY && cid[r] <= mid) ? 1u : 0u;
    le = block_sum_u32(le, sh);
    const uint32_t masked_le = mid + 1 - le;
    if (masked_le >= j + 1) hi = mid; else lo = mid + 1;
  }
  return lo;
}

// General path of sample_token (sampling.rs:120-241) for n <= E * SAMPLE_THREADS.
// Candidates are sorted by value only (32-bit keys): equal values make equal
// softmax terms, so every sum is independent of the order among them, and the
// id of a chosen position is resolved afterwards as the m-th smallest id
// among the candidates with that value (the reference's stable sort order).
template <int E>
__device__ __forceinline__ uint32_t sample_general(SampleShared& sh, const float* logits, const uint32_t* ids,
                                                   uint32_t n, uint32_t vocab, SamplerCfg cfg, int64_t masked,
                                                   int64_t force, uint64_t* rng, uint32_t n_fin) {
  constexpr uint32_t NT = SAMPLE_THREADS;
  const uint32_t tid = threadIdx.x;
  // keys in candidate order stay in sh.ckey (ids are re-read where needed),
  // so no per-candidate registers live across the sums
  uint32_t key[E];
  uint32_t fi_local = 0xffffffffu;
#pragma unroll
  for (int r = 0; r < E; ++r) {
    const uint32_t i = uint32_t(r) * NT + tid;
    key[r] = NO_KEY;
    if (i < n) {
      const uint32_t id = ids ? ids[i] : i;
      const float v = (int64_t(id) == masked) ? -INFINITY : logits[i];
      if (v > -INFINITY) key[r] = value_key(v);
      if (force >= 0 && int64_t(id) == force) fi_local = i;
    }
    sh.ckey[i] = key[r];
  }
  if (tid == 0) sh.bcast_u[1] = 0xffffffffu;
  __syncthreads();
  if (fi_local != 0xffffffffu) sh.bcast_u[1] = fi_local;  // ids are unique
  bitonic_sort_regs<E>(key, reinterpret_cast<uint32_t*>(sh.probs), n <= uint32_t(E / 2) * NT + 1u);
  __syncthreads();
#pragma unroll
  for (int r = 0; r < E; ++r) sh.skey[uint32_t(r) * NT + tid] = key[r];
  __syncthreads();

  // item list: sorted finite (first min(k, n_fin)), then masked ids (if k > n_fin),
  // or the appended always-include item.
  const uint32_t k_lim = cfg.top_k > 0 ? min(uint32_t(cfg.top_k), vocab) : vocab;
  const uint32_t n_top = min(k_lim, n_fin);
  uint32_t force_pos = 0xffffffffu, appended = 0;
  const uint32_t fi = sh.bcast_u[1];
  uint32_t kf = NO_KEY;
  if (force >= 0 && uint64_t(force) < vocab && fi != 0xffffffffu && sh.ckey[fi] != NO_KEY) {
    // rank of the always-include item in the stable order
    kf = sh.ckey[fi];
    uint32_t c = 0;
#pragma unroll
    for (int r = 0; r < E; ++r) {
      const uint32_t i = uint32_t(r) * NT + tid;
      const uint32_t kr = sh.ckey[i];
      c += (kr < kf || (kr == kf && i < fi)) ? 1u : 0u;
    }
    const uint32_t rank = block_sum_u32(c, sh);
    if (rank < n_top) {
      force_pos = rank;
    } else if (key_value(kf) > -1e30f) {
      appended = 1;
      force_pos = n_top;
    }
  }
  const uint32_t n_items = appended ? n_top + 1 : k_lim;  // masked tail when k_lim > n_fin
  const uint32_t n_valued = appended ? n_top + 1 : n_top;  // items with a finite logit
  const float vmax = key_value(sh.skey[0]);
  // softmax numerators in parallel (elementwise), sums sequential
  for (uint32_t i = tid; i < n_valued; i += NT) {
    const float v = key_value((appended && i == n_top) ? kf : sh.skey[i]);
    float p;
    if (cfg.temperature > 0.0f)
      p = expf_glibc(__fdiv_rn(__fsub_rn(v, vmax), cfg.temperature));
    else
      p = fabsf(__fsub_rn(v, vmax)) < 1e-6f ? 1.0f : 0.0f;
    sh.probs[i] = p;
  }
  __syncthreads();
  // softmax denominator: sequential sum over all valued items (the appended
  // item may break the non-increasing order, so it disables the early stop)
  constexpr uint32_t NO_POS = 0xffffffffu;
  if (tid == 0) sh.bcast_f = seq_chain<false>(sh.probs, n_valued, __builtin_nanf(""), !appended, NO_POS, nullptr).sum;
  __syncthreads();
  const float sum = sh.bcast_f;
  if (sum > 0.0f)
    for (uint32_t i = tid; i < n_valued; i += NT) sh.probs[i] = __fdiv_rn(sh.probs[i], sum);
  __syncthreads();
  // top-p: the cut is the first index whose running sum of the probabilities
  // reaches top_p; kept mass: the running sum at n_pv - 1, which is the cut,
  // the always-include item's position when that extends the cut, or the
  // last valued item when nothing is cut.  Then the draw's target.
  if (tid == 0) {
    const uint32_t at = force_pos < n_valued ? force_pos : NO_POS;
    const ChainCut c = seq_chain<false>(sh.probs, n_valued, cfg.top_p, !appended, at, nullptr);
    uint32_t p_idx = c.cut < n_valued ? c.cut + 1 : n_items;  // zero-probability tail never reaches top_p either
    if (p_idx == 0) p_idx = 1;
    float sp = c.sum;
    if (force_pos != NO_POS && force_pos >= p_idx) {
      p_idx = force_pos + 1;
      sp = c.at_sum;
    }
    if (min(p_idx, n_valued) == 0) sp = 0.0f;
    sh.bcast_u[3] = p_idx;
    sh.redf[0] = sp;
    const double draw = lcg_next_unit(rng);
    sh.bcast_f = fminf(fmaxf(float(draw), 0.0f), 1.0f - 1e-7f);
  }
  __syncthreads();
  const uint32_t p_idx = sh.bcast_u[3];
  const uint32_t n_pv = min(p_idx, n_valued);
  const float sum_p = sh.redf[0];
  const float target = sh.bcast_f;
  if (sum_p > 0.0f)
    for (uint32_t i = tid; i < n_pv; i += NT) sh.probs[i] = __fdiv_rn(sh.probs[i], sum_p);
  __syncthreads();
  // draw: first index whose running sum exceeds the target (reaches the next
  // float up); items past n_valued carry probability 0 and never raise the sum
  if (tid == 0) {
    const float thr = __uint_as_float(__float_as_uint(target) + 1u);
    sh.bcast_u[3] = seq_chain<false>(sh.probs, n_pv, thr, !appended, NO_POS, nullptr).cut;
  }
  __syncthreads();
  const uint32_t hit = sh.bcast_u[3];
  const uint32_t choice = hit < n_pv ? hit : p_idx - 1;
  uint32_t tok;
  if (choice < n_top) {
    // id of sorted position `choice`: the (choice - first)-th smallest id
    // among the candidates with the same value
    const uint32_t kc = sh.skey[choice];
    uint32_t lo = 0, hi = choice;  // first sorted position holding kc
    while (lo < hi) {
      const uint32_t mid = (lo + hi) / 2;
      if (sh.skey[mid] < kc) lo = mid + 1; else hi = mid;
    }
    const uint32_t j = block_nth_match(sh, n, kc, choice - lo);
    tok = j < n ? (ids ? ids[j] : j) : 0u;  // a match always exists
  } else if (appended) {
    tok = uint32_t(force);
  } else {
    tok = block_masked_id<E>(sh, ids, n, choice - n_fin, vocab);
  }
  return tok;
}

__device__ __forceinline__ uint32_t sample_core(SampleShared& sh, const float* logits, const uint32_t* ids, uint32_t n,
                                uint32_t vocab, SamplerCfg cfg, int64_t masked, int64_t force, uint64_t* rng,
                                uint32_t* err) {
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr uint32_t NW = SAMPLE_THREADS / WAVE;
  // One pass: the finite count and the greedy keys (greedy_add)
  float m1 = -INFINITY, m2 = -INFINITY;
  uint32_t id1 = 0xffffffffu, nfin = 0;
  for (uint32_t i = tid; i < n; i += SAMPLE_THREADS) {
    const uint32_t id = ids ? ids[i] : i;
    const float v = (int64_t(id) == masked) ? -INFINITY : logits[i];
    if (v > -INFINITY) {
      ++nfin;
      greedy_add(m1, id1, m2, v, id);
    }
  }
  greedy_wave(m1, id1, m2);
  const float nf = wave_sum(float(nfin));
  if (lane == 0) {
    sh.redf[wave] = m1;
    sh.redk[wave] = id1;
    sh.rede[wave] = m2;
    sh.redu[wave] = uint32_t(nf);
  }
  __syncthreads();
  if (tid == 0) {
    float a1 = sh.redf[0], a2 = sh.rede[0];
    uint32_t ai = sh.redk[0], c = sh.redu[0];
    for (uint32_t w = 1; w < NW; ++w) {
      greedy_merge(a1, ai, a2, sh.redf[w], sh.redk[w], sh.rede[w]);
      c += sh.redu[w];
    }
    sh.bcast_f = a1;
    sh.bcast_u[0] = c;
    sh.bcast_u[1] = (!(cfg.temperature > 0.0f) && greedy_unique(c, a1, a2)) ? 1u : 0u;
    sh.bcast_u[2] = ai;
  }
  __syncthreads();
  const uint32_t n_fin = sh.bcast_u[0], greedy = sh.bcast_u[1], arg = sh.bcast_u[2];
  __syncthreads();  // every thread has read the broadcast words before they are reused

  if (n_fin == 0) {  // every candidate masked: the reference returns the first id of a -inf list
    uint32_t tok = 0;
    if (tid == 0) {
      (void)lcg_next_unit(rng);
      tok = 0;
    }
    return tok;
  }

  // greedy fast path: T <= 0 and a unique value within 1e-6 of the max
  if (greedy) {
    if (tid == 0) (void)lcg_next_unit(rng);
    __syncthreads();
    return arg;
  }

  // general path: sort finite candidates by (value desc, id asc)
  if (n > SAMPLE_MAX) {
    if (tid == 0 && err) atomicOr(err, ERR_SAMPLER);
    return 0;
  }
  if (n <= SAMPLE_THREADS) return sample_general<1>(sh, logits, ids, n, vocab, cfg, masked, force, rng, n_fin);
  if (n <= 2 * SAMPLE_THREADS) return sample_general<2>(sh, logits, ids, n, vocab, cfg, masked, force, rng, n_fin);
  if (n <= 4 * SAMPLE_THREADS) return sample_general<4>(sh, logits, ids, n, vocab, cfg, masked, force, rng, n_fin);
  return sample_general<8>(sh, logits, ids, n, vocab, cfg, masked, force, rng, n_fin);
}

// Block b samples sequence b (its logits row, state and code output).
__global__ __launch_bounds__(SAMPLE_THREADS) void sample_slow_kernel(SampleArgs a) {
  extern __shared__ uint8_t smem_raw[];
  SampleShared& sh = *reinterpret_cast<SampleShared*>(smem_raw);
  const uint32_t b = blockIdx.x;
  DevState* st = a.st + b;
  a.logits += size_t(b) * a.n;
  if (a.codes_out) a.codes_out += size_t(b) * a.codes_stride;
  if (a.token_out) a.token_out += b;
  if (st->done) return;
  __shared__ uint32_t gen;
  if (threadIdx.x == 0) {
    st->n_past += a.advance;  // the Slow step's position (an unfinished sequence only)
    if (a.after_step) {
      if (a.codes_out) {
        for (uint32_t cb = 0; cb < a.num_codebooks; ++cb)
          a.codes_out[size_t(cb) * st->max_new + st->step_index] = int32_t(st->codes_frame[cb]);
      }
      st->step_index += 1;
      const uint32_t past = st->n_past >= st->prompt_cols ? st->n_past - st->prompt_cols : 0u;
      gen = past + st->step_index;
    } else {
      gen = 0;
    }
  }
  __syncthreads();
  const bool block = gen < st->min_tokens_before_end;
  const int64_t masked = block ? int64_t(a.im_end) : -1;
  const int64_t force = block ? -1 : int64_t(a.im_end);
  if (threadIdx.x == 0) sh.rng = st->rng;
  const uint32_t tok = sample_core(sh, a.logits, a.ids, a.n, a.vocab, a.cfg, masked, force, &sh.rng, &st->err);
  if (threadIdx.x == 0) {
    st->rng = sh.rng;
    st->main_token = tok;
    if (a.token_out) *a.token_out = tok;
    if (tok == a.im_end || st->step_index >= st->max_new) {
      st->done = 1;
      // the batch is done once every sequence is
      if (a.batch && atomicAdd(&a.batch->done_count, 1u) + 1 == a.batch->n_seq) a.batch->done_all = 1;
    }
  }
}

__global__ __launch_bounds__(SAMPLE_THREADS) void sample_fast_kernel(SampleArgs a) {
  extern __shared__ uint8_t smem_raw[];
  SampleShared& sh = *reinterpret_cast<SampleShared*>(smem_raw);
  const uint32_t nseq = a.n_seq ? a.n_seq : 1u;
  if (__builtin_expect(blockIdx.x >= nseq, 0)) {  // warming blocks after the sampling blocks (laid out last)
    l2_warm(a.warm, blockIdx.x, blockIdx.x - nseq, threadIdx.x, SAMPLE_THREADS);
    return;
  }
  const uint32_t b = blockIdx.x;
  DevState* st = a.st + b;
  a.logits += size_t(b) * a.n;
  if (a.next_input) a.next_input += size_t(b) * a.dim;
  if (a.token_out) a.token_out += b;
  if (st->done) return;
  if (threadIdx.x == 0) sh.rng = st->rng;
  const uint32_t tok = sample_core(sh, a.logits, nullptr, a.n, a.vocab, a.cfg, -1, -1, &sh.rng, &st->err);
  __shared__ uint32_t tok_s;
  if (threadIdx.x == 0) {
    st->rng = sh.rng;
    uint32_t t = tok;
    if (t >= a.n) {
      atomicOr(&st->err, ERR_SAMPLER);
      t = 0;
    }
    st->codes_frame[a.cb_index] = t;
    if (a.token_out) *a.token_out = t;
    tok_s = t;
  }
  __syncthreads();
  if (a.next_input) {
    const uint32_t t = tok_s;
    for (uint32_t i = threadIdx.x; i < a.dim; i += SAMPLE_THREADS)
      a.next_input[i] = half_bits_to_float(a.fast_emb[size_t(t) * a.dim + i]);
  }
}

__global__ __launch_bounds__(SAMPLE_THREADS) void sample_plain_kernel(const float* logits, uint32_t n, SamplerCfg cfg,
                                                                      int64_t always_include, uint64_t* rng,
                                                                      uint32_t* token_out, uint32_t* err) {
  extern __shared__ uint8_t smem_raw[];
  SampleShared& sh = *reinterpret_cast<SampleShared*>(smem_raw);
  if (threadIdx.x == 0) sh.rng = *rng;
  const uint32_t tok = sample_core(sh, logits, nullptr, n, n, cfg, -1, always_include, &sh.rng, err);
  if (threadIdx.x == 0) {
    *rng = sh.rng;
    *token_out = tok;
  }
}

// Running sums of n <= SAMPLE_MAX terms through seq_chain (the samplers'
// sequential sums), for the parity test of that routine: terms and sums
// staged in LDS, one lane adding as the samplers do.
__global__ __launch_bounds__(WAVE) void running_sum_kernel(const float* terms, uint32_t n, float* prefix,
                                                              float* total) {
  __shared__ __align__(16) float t[SAMPLE_MAX];
  __shared__ __align__(16) float ps[SAMPLE_MAX];
  for (uint32_t i = threadIdx.x; i < n; i += WAVE) t[i] = terms[i];
  __syncthreads();
  if (threadIdx.x == 0) *total = seq_chain<true>(t, n, __builtin_nanf(""), false, 0xffffffffu, ps).sum;
  __syncthreads();
  for (uint32_t i = threadIdx.x; i < n; i += WAVE) prefix[i] = ps[i];
}

// The samplers' cut search through seq_chain for n <= SAMPLE_MAX terms: the
// first index whose running sum reaches thr (n if none), the running sum
// there (the total if none) and the running sum at index `at` (when at < n).
__global__ __launch_bounds__(WAVE) void running_cut_kernel(const float* terms, uint32_t n, float thr, uint32_t absorb,
                                                            uint32_t at, uint32_t* cut, float* sums) {
  __shared__ __align__(16) float t[SAMPLE_MAX];
  for (uint32_t i = threadIdx.x; i < n; i += WAVE) t[i] = terms[i];
  __syncthreads();
  if (threadIdx.x == 0) {
    const ChainCut c = seq_chain<false>(t, n, thr, absorb != 0, at, nullptr);
    *cut = c.cut;
    sums[0] = c.sum;
    sums[1] = c.at_sum;
  }
}

// expf_glibc over n inputs: the test hook of the device exp used by the
// samplers' softmax and the SwiGLU sigmoids.
__global__ __launch_bounds__(256) void expf_kernel(const float* x, float* y, size_t n) {
  for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += size_t(gridDim.x) * 256) y[i] = expf_glibc(x[i]);
}

template <uint32_t WT>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* w, size_t row_bytes, uint32_t in, float* out) {
  const uint32_t r = blockIdx.x;
  const uint8_t* row = w + size_t(r) * row_bytes;
  for (uint32_t e = threadIdx.x * 8; e < in; e += 256 * 8) {
    float v[8];
    load_w8<WT>(row, e, v);
    for (int i = 0; i < 8; ++i) out[size_t(r) * in + e + i] = v[i];
  }
}

__global__ void swiglu_kernel(const float* g, const float* u, float* out, uint32_t n, int fast) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float gv = g[i];
  if (fast)
    out[i] = __fmul_rn(__fdiv_rn(gv, __fadd_rn(1.0f, expf_glibc(-gv))), u[i]);
  else
    out[i] = __fmul_rn(__fmul_rn(gv, __fdiv_rn(1.0f, __fadd_rn(1.0f, expf_glibc(-gv)))), u[i]);
}

__global__ void add_position_kernel(DevState* st, uint32_t n, uint32_t n_seq) {
  for (uint32_t b = threadIdx.x; b < n_seq; b += blockDim.x)
    if (!st[b].done) st[b].n_past += n;
}

// Streaming copy of n4 16-byte words: the reference kernel against which HBM
// byte counters are calibrated (it reads and writes exactly 16 * n4 bytes).
__global__ __launch_bounds__(256) void copy_kernel(const float4* __restrict__ src, float4* __restrict__ dst,
                                                   size_t n4) {
  const size_t stride = size_t(gridDim.x) * 256;
  for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < n4; i += stride) dst[i] = src[i];
}

template <class K>
hipError_t set_max_lds(K kernel) {
  return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                             int(sizeof(SampleShared)));
}

}  // namespace

uint32_t l2_warm_planes(const L2Warm& w, uint32_t plane, hipError_t* err) {
  if (!w.base) return 0;
  if (w.blocks == 0 || w.blocks % 8 || w.cb_begin % 8 || w.cb_end <= w.cb_begin || w.span < 16 || w.span % 16 ||
      reinterpret_cast<uintptr_t>(w.base) % 16 || reinterpret_cast<uintptr_t>(w.base3) % 16 || plane == 0) {
    *err = hipErrorInvalidValue;
    return 0;
  }
  return (w.blocks + plane - 1) / plane;
}

// The block shapes gemv_k_pick launches (rows per wave x waves per block).
uint32_t gemv_rows_per_block(uint32_t wtype, uint32_t in, uint32_t out, bool norm, bool dual, uint32_t ncol) {
  const uint32_t rs = dual ? 1u : 2u;
  switch (in) {
    case 512:
    case 1536: return norm ? 8u : rs * 4u;
    case 2560:
      if (!norm) return rs * 4u;
      return (ncol == 1 && !dual) ? (out <= 4096 ? 16u : 12u) : 8u;
    case 4096: return norm ? 8u : 10u;
    case 9728: return norm ? 8u : (ncol == 1 && !dual && wtype == W_F16 ? 5u : 4u);  // (split-step w2: 5)
    default: return 0u;
  }
}

hipError_t launch_gemv(uint32_t wtype, int epi, int ncol, const GemvArgs& a, hipStream_t s) {
  if (wtype != W_F16 && wtype != W_Q8_0 && wtype != W_Q4_0) return hipErrorInvalidValue;
  if (a.in % (wtype == W_F16 ? 8 : 32)) return hipErrorInvalidValue;
  if (a.fold.logits) {
    if (ncol != 1 || epi != EPI_STORE) return hipErrorInvalidValue;
    switch (wtype) {
      case W_F16: return gemv_fold_launch<W_F16>(a, s);
      case W_Q8_0: return gemv_fold_launch<W_Q8_0>(a, s);
      default: return gemv_fold_launch<W_Q4_0>(a, s);
    }
  }
  // the normalised-x output: only the RMSNorm GEMV form (gemv_n_kernel) over
  // 1-2 columns of the rows it serves writes it
  if (a.xn_out && (!a.norm || a.w3 || ncol > 2 || a.fold.logits || a.ldx % 4 ||
                   (a.in != 512 && a.in != 1536 && a.in != 2560) ||
                   reinterpret_cast<uintptr_t>(a.xn_out) % 16))
    return hipErrorInvalidValue;
  if (wtype != W_F16 && !a.xn_out && (ncol == 1 || ncol == 2) && a.qp && a.qs && a.row_base == 0 && a.extra_row == NO_ROW &&
      a.ldx % 4 == 0 && !((epi == EPI_SWIGLU_SLOW || epi == EPI_SWIGLU_FAST) && (!a.qp3 || !a.qs3))) {
    const hipError_t e = ncol == 1
        ? (wtype == W_Q8_0 ? gemv_q_epi<W_Q8_0, 1>(epi, a, s) : gemv_q_epi<W_Q4_0, 1>(epi, a, s))
        : (wtype == W_Q8_0 ? gemv_q_epi<W_Q8_0, 2>(epi, a, s) : gemv_q_epi<W_Q4_0, 2>(epi, a, s));
    if (e != hipErrorNotSupported) return e;  // else the GGUF-layout kernels below
  }
  if (ncol <= 2 && a.ldx % 4 == 0 && gemv_k_supported(a.in)) {
    switch (wtype) {
      case W_F16: return gemv_k_epi<W_F16>(epi, ncol, a, s);
      case W_Q8_0: return gemv_k_epi<W_Q8_0>(epi, ncol, a, s);
      default: return gemv_k_epi<W_Q4_0>(epi, ncol, a, s);
    }
  }
  const bool direct = ncol <= 2 && a.in % 512 == 0 && a.in <= 20 * 512 && a.ldx % 4 == 0;
  if (direct) {
    switch (wtype) {
      case W_F16: return gemv_direct_epi<W_F16>(epi, ncol, a, s);
      case W_Q8_0: return gemv_direct_epi<W_Q8_0>(epi, ncol, a, s);
      default: return gemv_direct_epi<W_Q4_0>(epi, ncol, a, s);
    }
  }
  if (size_t(ncol) * a.in * sizeof(float) > 150 * 1024) return hipErrorInvalidValue;
  switch (wtype) {
    case W_F16: return gemv_pick_epi<W_F16>(epi, ncol, a, s);
    case W_Q8_0: return gemv_pick_epi<W_Q8_0>(epi, ncol, a, s);
    default: return gemv_pick_epi<W_Q4_0>(epi, ncol, a, s);
  }
}

hipError_t launch_rms_norm(const float* x, const float* w, float* y, uint32_t n, uint32_t ncol, float eps,
                           const uint32_t* done, hipStream_t s) {
  hipLaunchKernelGGL(rms_norm_kernel, dim3(ncol), dim3(256), 0, s, x, w, y, n, eps, done);
  return hipGetLastError();
}

hipError_t launch_qkv_post(const QkvPostArgs& a, hipStream_t s) {
  if (a.hd % 2 || a.hd > 256) return hipErrorInvalidValue;
  hipLaunchKernelGGL(qkv_post_kernel, dim3(a.H + 2 * a.Hkv, a.ncol), dim3(64), 0, s, a);
  return hipGetLastError();
}

uint32_t attention_chunks(uint32_t max_seq, uint32_t mode) {
  (void)mode;
  return (max_seq + ATTN_CHUNK - 1u) / ATTN_CHUNK;
}

// H | Hkv << 8 | cols_per_seq << 16 | seq_stride_words << 24: the shape word
// the attention kernels take among their preloaded arguments
uint32_t attn_shape_word(const AttnArgs& a) {
  return a.H | a.Hkv << 8 | a.cols_per_seq << 16 | a.seq_stride_words << 24;
}

template <int HD>
void launch_combine(const AttnArgs& a, dim3 grid, hipStream_t s) {
  const uint32_t sh = attn_shape_word(a);
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, dim3(HD), 0, s, a.part, a.out, a.pos_ptr, a.done, a.ncol, a.max_chunks, sh,
                       a.pos_offset, a);
  };
  if (a.max_chunks <= 8)
    go(attn_combine_kernel<HD, 32, 8>);
  else if (a.max_chunks <= 16)
    go(attn_combine_kernel<HD, 32, 16>);
  else if (a.max_chunks <= 32)
    go(attn_combine_kernel<HD, 32, 32>);
  else if (a.max_chunks <= 64)
    go(attn_combine_kernel<HD, 32, 64>);
  else
    go(attn_combine_kernel<HD, 32, 0>);
}

template <int HD, bool LAST>
void launch_partial(const AttnArgs& a, dim3 grid, hipStream_t s) {
  if (!LAST && a.qkv_rows) {  // q / k / v from a table row (f32 cache: the Fast-AR's)
    if (a.kv_f16) return;     // rejected by launch_attention
    hipLaunchKernelGGL((attn_partial_kernel<HD, 32, false, false, true>), grid, dim3(256), 0, s, a.qkv,
                       static_cast<void*>(a.k_cache), static_cast<void*>(a.v_cache), a.pos_ptr, a.done,
                       a.ncol | a.check_from << 8, a.max_seq, uint32_t(a.seq_stride_kv), attn_shape_word(a), a);
    return;
  }
  const bool warm = a.warm.base != nullptr;
  hipLaunchKernelGGL((a.kv_f16 ? (warm ? attn_partial_kernel<HD, 32, LAST, true> : attn_partial_kernel<HD, 32, LAST, true, false, false>)
                               : (warm ? attn_partial_kernel<HD, 32, LAST, false>
                                       : attn_partial_kernel<HD, 32, LAST, false, false, false>)),
                     grid, dim3(256), 0, s, a.qkv, static_cast<void*>(a.k_cache), static_cast<void*>(a.v_cache),
                     a.pos_ptr, a.done, a.ncol | a.check_from << 8, a.max_seq, uint32_t(a.seq_stride_kv),
                     attn_shape_word(a), a);
}

hipError_t launch_attention(const AttnArgs& args, hipStream_t s) {
  AttnArgs a = args;
  if (a.max_chunks > ATTN_MAX_CHUNKS) return hipErrorInvalidValue;
  if (a.cols_per_seq == 0) a.cols_per_seq = a.ncol;  // one sequence
  if (a.ncol == 0 || a.ncol % a.cols_per_seq || a.cols_per_seq > 4 || a.ncol > 64) return hipErrorInvalidValue;
  if (a.ncol > a.cols_per_seq && a.seq_stride_words == 0 && (a.pos_ptr || a.done)) return hipErrorInvalidValue;
  if (a.H % a.Hkv || a.H / a.Hkv > 4 || a.H > 255 || a.seq_stride_words > 255 || a.seq_stride_kv > UINT32_MAX)
    return hipErrorInvalidValue;
  if (a.max_chunks != attention_chunks(a.max_seq, a.mode) || a.check_from > a.max_chunks) return hipErrorInvalidValue;
  if (a.qkv_rows) {
    const GreedyFold& f = a.fold;
    if (a.ncol != 1 || a.cols_per_seq != 1 || a.mode != ATTN_SPLIT || a.kv_f16) return hipErrorInvalidValue;
    if (f.n == 0 || (f.logits ? (!f.emb || !f.st || !f.x_out || f.n % 4 || f.dim == 0 || f.dim % 8 ||
                                 f.cb_index >= 16 || reinterpret_cast<uintptr_t>(f.logits) % 16 ||
                                 reinterpret_cast<uintptr_t>(f.emb) % 16 || reinterpret_cast<uintptr_t>(f.x_out) % 16)
                              : !a.code_ptr))
      return hipErrorInvalidValue;
  }
  hipError_t werr = hipSuccess;
  const uint32_t planes = l2_warm_planes(a.warm, a.max_chunks * a.Hkv, &werr);  // z-planes of warming blocks
  if (werr != hipSuccess) return werr;
  const dim3 grid(a.max_chunks, a.Hkv, a.ncol + planes);
  if (a.hd != 64 && a.hd != 128) return hipErrorInvalidValue;
  if (a.mode == ATTN_FUSED) {
    if (!a.counters) return hipErrorInvalidValue;
    if (a.hd == 64)
      launch_partial<64, true>(a, grid, s);
    else
      launch_partial<128, true>(a, grid, s);
    return hipGetLastError();
  }
  if (a.hd == 64)
    launch_partial<64, false>(a, grid, s);
  else
    launch_partial<128, false>(a, grid, s);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.max_chunks == 1) return e;
  const dim3 cgrid(a.H, a.ncol);
  if (a.hd == 64)
    launch_combine<64>(a, cgrid, s);
  else
    launch_combine<128>(a, cgrid, s);
  return hipGetLastError();
}

hipError_t launch_embed(const EmbedArgs& a, hipStream_t s) {
  if (a.num_codebooks > 16 || a.n == 0 || a.dim == 0) return hipErrorInvalidValue;
  hipError_t werr = hipSuccess;
  const uint32_t planes = l2_warm_planes(a.warm, a.n, &werr);
  if (werr != hipSuccess) return werr;
  hipLaunchKernelGGL(embed_kernel, dim3(a.n, (a.dim + 255) / 256 + planes), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_fast_begin(DevState* st, const float* slow_hidden, const uint16_t* fast_emb, float* fh,
                             uint32_t dim, uint32_t codebook_size, uint32_t sem_begin, uint32_t sem_end,
                             uint32_t n_seq, hipStream_t s) {
  hipLaunchKernelGGL(fast_begin_kernel, dim3((dim + 255) / 256, n_seq), dim3(256), 0, s, st, slow_hidden, fast_emb,
                     fh, dim, codebook_size, sem_begin, sem_end);
  return hipGetLastError();
}

hipError_t launch_sample_slow(const SampleArgs& a, hipStream_t s) {
  static bool configured = false;
  if (!configured) {
    hipError_t e = set_max_lds(sample_slow_kernel);
    if (e != hipSuccess) return e;
    configured = true;
  }
  if (a.n > SAMPLE_MAX - 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(sample_slow_kernel, dim3(a.n_seq ? a.n_seq : 1), dim3(SAMPLE_THREADS), sizeof(SampleShared), s, a);
  return hipGetLastError();
}

hipError_t launch_sample_fast(const SampleArgs& a, hipStream_t s) {
  static bool configured = false;
  if (!configured) {
    hipError_t e = set_max_lds(sample_fast_kernel);
    if (e != hipSuccess) return e;
    configured = true;
  }
  if (a.n > SAMPLE_MAX - 1) return hipErrorInvalidValue;
  hipError_t werr = hipSuccess;
  const uint32_t wblocks = l2_warm_planes(a.warm, 1u, &werr);  // planes of one block
  if (werr != hipSuccess) return werr;
  hipLaunchKernelGGL(sample_fast_kernel, dim3((a.n_seq ? a.n_seq : 1) + wblocks), dim3(SAMPLE_THREADS),
                     sizeof(SampleShared), s, a);
  return hipGetLastError();
}

hipError_t launch_sample_plain(const float* logits, uint32_t n, SamplerCfg cfg, int64_t always_include,
                               uint64_t* rng, uint32_t* token_out, uint32_t* err, hipStream_t s) {
  static bool configured = false;
  if (!configured) {
    hipError_t e = set_max_lds(sample_plain_kernel);
    if (e != hipSuccess) return e;
    configured = true;
  }
  if (n > SAMPLE_MAX - 1 || n == 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(sample_plain_kernel, dim3(1), dim3(SAMPLE_THREADS), sizeof(SampleShared), s, logits, n, cfg,
                     always_include, rng, token_out, err);
  return hipGetLastError();
}

hipError_t launch_dequant_rows(uint32_t wtype, const uint8_t* w, size_t row_bytes, uint32_t rows, uint32_t in,
                               float* out, hipStream_t s) {
  switch (wtype) {
    case W_F16:
      if (in % 8) return hipErrorInvalidValue;
      hipLaunchKernelGGL(dequant_kernel<W_F16>, dim3(rows), dim3(256), 0, s, w, row_bytes, in, out);
      break;
    case W_Q8_0:
      if (in % 32) return hipErrorInvalidValue;
      hipLaunchKernelGGL(dequant_kernel<W_Q8_0>, dim3(rows), dim3(256), 0, s, w, row_bytes, in, out);
      break;
    case W_Q4_0:
      if (in % 32) return hipErrorInvalidValue;
      hipLaunchKernelGGL(dequant_kernel<W_Q4_0>, dim3(rows), dim3(256), 0, s, w, row_bytes, in, out);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

uint32_t repack_quant_bytes(uint32_t wtype) { return wtype == W_Q8_0 ? 32u : wtype == W_Q4_0 ? 16u : 0u; }

hipError_t launch_repack_q(const uint8_t* rows, size_t row_bytes, uint32_t wtype, uint32_t in, uint32_t nrows,
                           uint8_t* qplane, uint16_t* splane, hipStream_t s) {
  if ((wtype != W_Q8_0 && wtype != W_Q4_0) || in % 32 || nrows == 0) return hipErrorInvalidValue;
  const size_t n = size_t(in / 32) * nrows;
  hipLaunchKernelGGL(repack_q_kernel, dim3(uint32_t((n + 255) / 256)), dim3(256), 0, s, rows, row_bytes, wtype,
                     in / 32, nrows, qplane, splane);
  return hipGetLastError();
}

hipError_t launch_running_sum(const float* terms, uint32_t n, float* prefix, float* total, hipStream_t s) {
  if (n == 0 || n > SAMPLE_MAX) return hipErrorInvalidValue;
  hipLaunchKernelGGL(running_sum_kernel, dim3(1), dim3(WAVE), 0, s, terms, n, prefix, total);
  return hipGetLastError();
}

hipError_t launch_running_cut(const float* terms, uint32_t n, float thr, uint32_t absorb, uint32_t at, uint32_t* cut,
                              float* sums, hipStream_t s) {
  if (n > SAMPLE_MAX) return hipErrorInvalidValue;
  hipLaunchKernelGGL(running_cut_kernel, dim3(1), dim3(WAVE), 0, s, terms, n, thr, absorb, at, cut, sums);
  return hipGetLastError();
}

hipError_t launch_expf(const float* x, float* y, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  const size_t blocks = std::min<size_t>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(expf_kernel, dim3(uint32_t(blocks)), dim3(256), 0, s, x, y, n);
  return hipGetLastError();
}

hipError_t launch_swiglu(const float* g, const float* u, float* out, uint32_t n, int fast, hipStream_t s) {
  hipLaunchKernelGGL(swiglu_kernel, dim3((n + 255) / 256), dim3(256), 0, s, g, u, out, n, fast);
  return hipGetLastError();
}

hipError_t launch_add_position(DevState* st, uint32_t n, uint32_t n_seq, hipStream_t s) {
  hipLaunchKernelGGL(add_position_kernel, dim3(1), dim3(64), 0, s, st, n, n_seq);
  return hipGetLastError();
}

hipError_t launch_copy(const void* src, void* dst, size_t bytes, hipStream_t s) {
  if (bytes % 16 || (reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) % 16)
    return hipErrorInvalidValue;
  const size_t n4 = bytes / 16;
  const size_t blocks = std::min<size_t>(4096, (n4 + 255) / 256);
  if (blocks == 0) return hipSuccess;
  hipLaunchKernelGGL(copy_kernel, dim3(uint32_t(blocks)), dim3(256), 0, s, static_cast<const float4*>(src),
                     static_cast<float4*>(dst), n4);
  return hipGetLastError();
}

}  // namespace s2
