// prefill.hip -- prompt prefill kernels for gfx950 (CDNA4, wave64).
//
// A prompt chunk of N tokens goes through each layer as matrix products
// Y[N][M] = X[N][K] . W[M][K]^T on the MFMA units (v_mfma_f32_32x32x16_f16),
// so every weight row is read once per chunk instead of once per token.
//
// Precision: the reference computes these products in f32.  Activations are
// therefore split into two f16 planes, x = hi + lo (|x - hi - lo| <= 2^-22 |x|),
// and each product is W.hi + W.lo with f32 accumulation; the f16 weight
// values are exact in f16.  Q8_0 / Q4_0 weights (d * q, up to 19 significant
// bits) are dequantised exactly in f32 and split the same way, the low part
// scaled by 2^11 so it stays a normal f16 (W.x = Whi.xhi + Whi.xlo +
// 2^-11 (Wlo'.xhi)).  Each token row is scaled by a power of two before the
// split so that no value overflows f16; the epilogue undoes the scale.
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
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float wave_sum_f(float v) { return wave_sum(v); }
__device__ __forceinline__ float half_bits_to_float_p(uint16_t b) {
  return static_cast<float>(__builtin_bit_cast(_Float16, b));
}
__device__ __forceinline__ float wave_max_f(float v) { return wave_max(v); }

// ---------------------------------------------------------------------------
// Activation split: one block per row n < Npad.
//   xn = x[n] (or (x[n] * rms_scale) * g, the RMSNorm of the reference),
//   rs[n] = power of two with max|xn| / rs[n] in [2^13, 2^14),
//   xh[n] = f16(xn / rs), xl[n] = f16(xn / rs - xh);  rows N..Npad-1 are zero.
// ---------------------------------------------------------------------------
// The row is read once: thread t holds elements 4 (t + 256 i) .. + 3 (float4
// loads, all issued together) for rows of up to 4 * 256 * SR_REG elements;
// longer rows take the looped form below.
constexpr int SR_REG = 10;  // float4 per thread: rows up to 10240 elements

__device__ __forceinline__ float block_reduce_sum4(float v, float* red) {
  v = wave_sum_f(v);
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  const float t = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return t;
}
__device__ __forceinline__ float block_reduce_max4(float v, float* red) {
  v = wave_max_f(v);
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  const float t = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  return t;
}

// power-of-two row scale: exact to apply and to undo; max|x| / r in [2^13, 2^14)
__device__ __forceinline__ float split_scale(float mx) {
  float r = 1.0f;
  if (mx > 0.0f && mx < 3.0e38f) {
    int e;
    (void)frexpf(mx, &e);  // mx in [2^(e-1), 2^e)
    r = ldexpf(1.0f, e - 14);
  }
  return r;
}

__global__ __launch_bounds__(256) void split_rows_kernel(const float* x, uint32_t ldx, const float* norm, float eps,
                                                         uint32_t N, uint32_t K, _Float16* xh, _Float16* xl,
                                                         float* rs, uint32_t* err) {
  __shared__ float red[4];
  const uint32_t n = blockIdx.x, tid = threadIdx.x;
  _Float16* hr = xh + size_t(n) * K;
  _Float16* lr = xl + size_t(n) * K;
  if (n >= N) {
    for (uint32_t i = tid; i < K; i += 256) {
      hr[i] = _Float16(0.0f);
      lr[i] = _Float16(0.0f);
    }
    if (tid == 0) rs[n] = 1.0f;
    return;
  }
  const float* xr = x + size_t(n) * ldx;
  const uint32_t K4 = K / 4;  // K is a multiple of 32
  if (K4 <= 256u * SR_REG) {
    float4 v[SR_REG], g[SR_REG];
#pragma unroll
    for (int i = 0; i < SR_REG; ++i) {
      const uint32_t j = tid + 256u * i;
      v[i] = j < K4 ? *reinterpret_cast<const float4*>(xr + 4 * j) : make_float4(0.f, 0.f, 0.f, 0.f);
      g[i] = (norm && j < K4) ? *reinterpret_cast<const float4*>(norm + 4 * j) : make_float4(1.f, 1.f, 1.f, 1.f);
    }
    float scale = 1.0f;
    if (norm) {
      float ss = 0.0f;
#pragma unroll
      for (int i = 0; i < SR_REG; ++i) ss += v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w;
      const float tot = block_reduce_sum4(ss, red);
      scale = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(tot, float(K)), eps)));
    }
    float mx = 0.0f;
    bool nf = false;
#pragma unroll
    for (int i = 0; i < SR_REG; ++i) {
      if (norm) {
        v[i].x = __fmul_rn(__fmul_rn(v[i].x, scale), g[i].x);
        v[i].y = __fmul_rn(__fmul_rn(v[i].y, scale), g[i].y);
        v[i].z = __fmul_rn(__fmul_rn(v[i].z, scale), g[i].z);
        v[i].w = __fmul_rn(__fmul_rn(v[i].w, scale), g[i].w);
      }
      mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
      // fmaxf drops NaN: non-finite values are flagged on their own
      nf = nf || !(fabsf(v[i].x) <= 3.4028235e38f) || !(fabsf(v[i].y) <= 3.4028235e38f) ||
           !(fabsf(v[i].z) <= 3.4028235e38f) || !(fabsf(v[i].w) <= 3.4028235e38f);
    }
    if (__any(nf) && (tid & 63u) == 0 && err) atomicOr(err, ERR_NONFINITE);
    const float r = split_scale(block_reduce_max4(mx, red));
    const float inv = 1.0f / r;
#pragma unroll
    for (int i = 0; i < SR_REG; ++i) {
      const uint32_t j = tid + 256u * i;
      if (j >= K4) continue;
      const float e[4] = {v[i].x * inv, v[i].y * inv, v[i].z * inv, v[i].w * inv};
      _Float16 h[4], l[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        h[c] = _Float16(e[c]);
        l[c] = _Float16(e[c] - float(h[c]));
      }
      *reinterpret_cast<uint2*>(hr + 4 * j) = *reinterpret_cast<const uint2*>(h);
      *reinterpret_cast<uint2*>(lr + 4 * j) = *reinterpret_cast<const uint2*>(l);
    }
    if (tid == 0) rs[n] = r;
    return;
  }
  float scale = 1.0f;
  if (norm) {
    float ss = 0.0f;
    for (uint32_t i = tid; i < K; i += 256) ss += xr[i] * xr[i];
    const float tot = block_reduce_sum4(ss, red);
    scale = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(tot, float(K)), eps)));
  }
  float mx = 0.0f;
  bool nf = false;
  for (uint32_t i = tid; i < K; i += 256) {
    float v = xr[i];
    if (norm) v = __fmul_rn(__fmul_rn(v, scale), norm[i]);
    mx = fmaxf(mx, fabsf(v));
    nf = nf || !(fabsf(v) <= 3.4028235e38f);
  }
  if (__any(nf) && (tid & 63u) == 0 && err) atomicOr(err, ERR_NONFINITE);
  const float r = split_scale(block_reduce_max4(mx, red));
  const float inv = 1.0f / r;
  for (uint32_t i = tid; i < K; i += 256) {
    float v = xr[i];
    if (norm) v = __fmul_rn(__fmul_rn(v, scale), norm[i]);
    v *= inv;
    const _Float16 h = _Float16(v);
    hr[i] = h;
    lr[i] = _Float16(v - float(h));
  }
  if (tid == 0) rs[n] = r;
}

// ---------------------------------------------------------------------------
// Weight fragment: 8 consecutive elements of one row as f16 (exact for F16
// rows; Q8_0 / Q4_0 blocks dequantised to f32 and split, low part * 2^11).
// ---------------------------------------------------------------------------
template <uint32_t WT>
__device__ __forceinline__ void weight8(const uint8_t* row, uint32_t e, half8& hi, half8& lo) {
  if constexpr (WT == W_F16) {
    hi = *reinterpret_cast<const half8*>(row + size_t(e) * 2);
  } else {
    constexpr uint32_t BB = (WT == W_Q8_0) ? 34u : 18u;
    const uint32_t b = e >> 5, p = (e >> 3) & 3u;
    const uint8_t* blk = row + size_t(b) * BB;
    const float d = float(*reinterpret_cast<const _Float16*>(blk));
    float w[8];
    if constexpr (WT == W_Q8_0) {
      const int8_t* q = reinterpret_cast<const int8_t*>(blk + 2 + p * 8);
#pragma unroll
      for (int i = 0; i < 8; ++i) w[i] = float(q[i]) * d;
    } else {
      const uint8_t* q = blk + 2 + (p & 1u) * 8;
      const uint32_t sh = (p >= 2) ? 4u : 0u;
#pragma unroll
      for (int i = 0; i < 8; ++i) w[i] = float(int((q[i] >> sh) & 0xfu) - 8) * d;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const _Float16 h = _Float16(w[i]);
      hi[i] = h;
      lo[i] = _Float16((w[i] - float(h)) * 2048.0f);
    }
  }
}

// ---------------------------------------------------------------------------
// MFMA GEMM  Y[n][m] (op)= rs[n] * sum_k W[m][k] * X[n][k]
//   Block tile: 128 weight rows x 128 tokens, 4 waves in 2 x 2, each wave
//   64 rows x 64 tokens = 2 x 2 tiles of v_mfma_f32_32x32x16_f16 with the
//   token fragment as A and the weight fragment as B, so a lane's results
//   are 16 tokens x one weight row and the 32 lanes of a row group store 32
//   consecutive outputs.  Per 16-wide k step a wave reads 2 weight and 4
//   token fragments (hi and lo planes) from LDS for 8 MFMAs (F16).  K goes in
//   stages of 32 through a double buffer in LDS (swizzled rows, see tile_off);
//   the loads of the stage after next are in flight while a stage computes.
//   SwiGLU (w1 and w3): the 128 row slots hold 64 outputs as [w1 32 | w3 32 |
//   w1 32 | w3 32], so each wave holds w1 and w3 of the same outputs.
//   Tile order: blocks L and L + 8 run on the same XCD, so the n tiles (and
//   K splits) of one m tile are consecutive there and its weight rows are
//   fetched into that XCD's L2 once.
//   K split (short-M matrices): block (m, n, split) writes its unscaled sums
//   to part[split][n][m]; gemm_split_reduce_kernel adds the splits in order
//   and applies rs and the epilogue.
// ---------------------------------------------------------------------------
constexpr int TM = 128, TN = 128, KS = 32;

// LDS tile rows are KS halfs (four 16-byte chunks) with no padding; chunk j of
// row r sits at chunk position j ^ swz(r).  Both access patterns then hit
// distinct banks with 32 or 64 banks of 4 bytes: the staging stores (4 lanes
// per row, consecutive rows) and the fragment reads (one row per lane, 32
// consecutive rows, one chunk).
__device__ __forceinline__ uint32_t swz(uint32_t r) { return ((r >> 1) ^ (r >> 3)) & 3u; }
__device__ __forceinline__ uint32_t tile_off(uint32_t r, uint32_t k) {  // k: a multiple of 8
  return r * KS + (((k >> 3) ^ swz(r)) << 3);
}
constexpr uint32_t GEMM_MAX_SPLITS = 4;

// Epilogue of the MFMA GEMM: acc[tn][tm][v] = D[token 8 (v/4) + 4 (lane/32) +
// v%4][weight slot lane%32] of the wave's 2 x 2 tiles.
template <uint32_t WT, int EPI>
__device__ __forceinline__ void gemm_epilogue(const GemmArgs& a, const floatx16 (&acc)[2][2],
                                              const floatx16 (&accl)[WT != W_F16 ? 2 : 1][WT != W_F16 ? 2 : 1],
                                              uint32_t mt, uint32_t n_base, uint32_t sp, uint32_t splits,
                                              uint32_t wm, uint32_t wn, uint32_t lane) {
  constexpr bool DUAL = (EPI == EPI_SWIGLU_SLOW || EPI == EPI_SWIGLU_FAST);
  constexpr bool WSPLIT = WT != W_F16;
  const uint32_t fr = lane & 31u;
#pragma unroll
  for (int tn = 0; tn < 2; ++tn) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const uint32_t n = n_base + 64 * wn + 32 * tn + 8 * (v / 4) + 4 * (lane >> 5) + (v % 4);
      float g[2];
#pragma unroll
      for (int tm = 0; tm < 2; ++tm) {
        g[tm] = acc[tn][tm][v];
        if constexpr (WSPLIT) g[tm] = g[tm] + accl[tn][tm][v] * (1.0f / 2048.0f);
      }
      if constexpr (DUAL) {
        const uint32_t m = mt * 64u + 32u * wm + fr;
        if (n >= a.N || m >= a.M) continue;
        const float r = a.rs[n];
        const float gg = g[0] * r, u = g[1] * r;
        float* dst = a.y + size_t(n) * a.ldy + m;
        if constexpr (EPI == EPI_SWIGLU_SLOW) {
          const float sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf_glibc(-gg)));
          *dst = __fmul_rn(__fmul_rn(gg, sig), u);
        } else {
          *dst = __fmul_rn(__fdiv_rn(gg, __fadd_rn(1.0f, expf_glibc(-gg))), u);
        }
      } else {
#pragma unroll
        for (int tm = 0; tm < 2; ++tm) {
          const uint32_t m = mt * TM + 64u * wm + 32u * tm + fr;
          if (n >= a.N || m >= a.M) continue;
          if (splits > 1) {
            a.part[(size_t(sp) * a.N + n) * a.M + m] = g[tm];
          } else {
            const float gg = g[tm] * a.rs[n];
            float* dst = a.y + size_t(n) * a.ldy + m;
            if constexpr (EPI == EPI_STORE) *dst = gg;
            else *dst = __fadd_rn(*dst, gg);
          }
        }
      }
    }
  }
}

template <uint32_t WT, int EPI, int D>
__global__ __launch_bounds__(256, 3) void gemm_mfma_kernel(GemmArgs a, uint32_t m_tiles, uint32_t n_tiles,
                                                           uint32_t splits) {
  constexpr bool DUAL = (EPI == EPI_SWIGLU_SLOW || EPI == EPI_SWIGLU_FAST);
  constexpr bool WSPLIT = WT != W_F16;
  constexpr int WP = WSPLIT ? 2 : 1;  // weight planes in LDS (hi, lo * 2^11)
  __shared__ _Float16 xs[2][2][TN * KS];
  __shared__ _Float16 ws[2][WP][TM * KS];
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t wm = wave & 1u, wn = wave >> 1;
  const uint32_t L = blockIdx.x, inner = n_tiles * splits;
  const uint32_t sidx = L >> 3, mt = (sidx / inner) * 8u + (L & 7u);
  if (mt >= m_tiles) return;
  const uint32_t rr = sidx % inner, nt = rr % n_tiles, sp = rr / n_tiles;
  const uint32_t n_base = nt * TN;
  const uint32_t nst = a.K / KS, st0 = sp * nst / splits, st1 = (sp + 1) * nst / splits;

  // staging: weight chunks c = tid + 256 j (j < 2): slot c / 4, 8 elements at
  // (c % 4) * 8; token chunks c = tid + 256 j (j < 4): plane c / 512, row
  // (c / 4) % 128, 8 elements at (c % 4) * 8
  const uint8_t* wrow[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const uint32_t slot = (tid + 256u * j) >> 2;
    uint32_t row;
    const uint8_t* base = a.w;
    if constexpr (DUAL) {
      const uint32_t grp = slot >> 5;
      row = mt * 64u + (grp >> 1) * 32u + (slot & 31u);
      base = (grp & 1u) ? a.w3 : a.w;
    } else {
      row = mt * TM + slot;
    }
    wrow[j] = base + size_t(min(row, a.M - 1)) * a.row_bytes;
  }
  const uint32_t part8 = (tid & 3u) * 8u;
  const _Float16* xrow[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t c = tid + 256u * j;
    xrow[j] = ((c >> 9) ? a.xl : a.xh) + size_t(n_base + ((c >> 2) & 127u)) * a.K + part8;
  }

  // a ring of D register sets: the loads of stage st + D go out while stage
  // st computes, so D stages of global latency are hidden
  half8 rw[D][2][WP], rx[D][4];
  auto load_stage = [&](int r, uint32_t st) {
    const uint32_t k0 = min(st, st1 - 1u) * KS;  // past the range: a valid, unused stage
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      half8 lo;
      weight8<WT>(wrow[j], k0 + part8, rw[r][j][0], lo);
      if constexpr (WSPLIT) rw[r][j][WP - 1] = lo;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) rx[r][j] = *reinterpret_cast<const half8*>(xrow[j] + k0);
  };
  auto store_stage = [&](int r, uint32_t buf) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t slot = (tid + 256u * j) >> 2;
#pragma unroll
      for (int p = 0; p < WP; ++p) *reinterpret_cast<half8*>(&ws[buf][p][tile_off(slot, part8)]) = rw[r][j][p];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t c = tid + 256u * j;
      *reinterpret_cast<half8*>(&xs[buf][c >> 9][tile_off((c >> 2) & 127u, part8)]) = rx[r][j];
    }
  };

  floatx16 acc[2][2], accl[WSPLIT ? 2 : 1][WSPLIT ? 2 : 1];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = floatx16{};
  if constexpr (WSPLIT) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) accl[i][j] = floatx16{};
  }
  const uint32_t fr = lane & 31u, fk = 8u * (lane >> 5);  // fragment row / k offset
  auto compute = [&](uint32_t buf) {
#pragma unroll
    for (uint32_t kk = 0; kk < KS; kk += 16) {
      half8 xa[2][2], wb[2][WP];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int p = 0; p < 2; ++p)
          xa[t][p] = *reinterpret_cast<const half8*>(&xs[buf][p][tile_off(64 * wn + 32 * t + fr, kk + fk)]);
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int p = 0; p < WP; ++p)
          wb[t][p] = *reinterpret_cast<const half8*>(&ws[buf][p][tile_off(64 * wm + 32 * t + fr, kk + fk)]);
#pragma unroll
      for (int tn = 0; tn < 2; ++tn)
#pragma unroll
        for (int tm = 0; tm < 2; ++tm) {
          acc[tn][tm] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xa[tn][0], wb[tm][0], acc[tn][tm], 0, 0, 0);
          acc[tn][tm] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xa[tn][1], wb[tm][0], acc[tn][tm], 0, 0, 0);
          if constexpr (WSPLIT)
            accl[tn][tm] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xa[tn][0], wb[tm][WP - 1], accl[tn][tm], 0, 0, 0);
        }
    }
  };
  // prologue: stages st0 .. st0 + D - 1 in flight, the first one in LDS
#pragma unroll
  for (int r = 0; r < D; ++r) load_stage(r, st0 + r);
  store_stage(0, 0);
  __syncthreads();
  // stage st sits in LDS buffer (st - st0) & 1 and came from ring slot
  // (st - st0) % D, which is reloaded with stage st + D once stored
  for (uint32_t s0 = st0; s0 < st1; s0 += D) {
#pragma unroll
    for (int r = 0; r < D; ++r) {
      const uint32_t st = s0 + r;
      if (st < st1) {
        load_stage(r, st + D);  // ring slot r is free: stage st went to LDS
        compute((st - st0) & 1u);
        if (st + 1 < st1) {
          store_stage((r + 1) % D, (st + 1 - st0) & 1u);
          __syncthreads();
        }
      }
    }
  }

  gemm_epilogue<WT, EPI>(a, acc, accl, mt, n_base, sp, splits, wm, wn, lane);
}

// F16 weights: the same tiles, staged by LDS-DMA loads (global_load_lds_dwordx4:
// a wave's 64 lanes fill 1 KiB of LDS, lane i at byte 16 i of the wave's
// destination), so staging takes no registers and no LDS store instructions.
// A wave's 1 KiB is 16 consecutive tile rows of 64 bytes; lane i takes row
// i / 4 and physical chunk i % 4 and loads the logical chunk (i % 4) ^ swz(row),
// which puts the tile in the swizzled layout of tile_off.  Three LDS stages
// rotate: while stage st computes, stage st + 1 is in flight and stage st + 2
// is issued into the buffer that stage st - 1 has left.
constexpr uint32_t GEMM_DMA_PER_STAGE = 6;  // 16-byte loads per thread per stage (4 token + 2 weight)

constexpr bool DUAL_EPI(int epi) { return epi == EPI_SWIGLU_SLOW || epi == EPI_SWIGLU_FAST; }

// One LDS-DMA load: 16 bytes per lane from `src` into the wave's 1 KiB at
// `lds` (lane i at byte 16 i).  Written as inline assembly so that the
// compiler does not treat every later LDS read as dependent on it (it would
// wait for all loads in flight first); the kernel waits for these loads
// itself (vmcnt) before the barrier that publishes a stage.
__device__ __forceinline__ void dma16(const void* src, const _Float16* lds) {
  const uint32_t m0 = uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(reinterpret_cast<uintptr_t>(lds)))));
  asm volatile("s_nop 1\n\ts_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" : : "s"(m0), "v"(src)
               : "memory", "m0");
}

typedef __attribute__((address_space(3))) void lds_void_t;
typedef const __attribute__((address_space(1))) void glob_void_t;

template <int B>
struct StageTag {
  static constexpr int value = B;
};

template <int EPI>
__global__ __launch_bounds__(256, 2) void gemm_f16_dma_kernel(GemmArgs a, uint32_t m_tiles, uint32_t n_tiles,
                                                              uint32_t splits) {
  // one LDS object per stage buffer, always addressed with a compile-time
  // stage index: the compiler then knows which buffer a DMA writes and a
  // fragment read reads, and waits only where they meet
  __shared__ _Float16 xs0[2 * TN * KS], xs1[2 * TN * KS], xs2[2 * TN * KS];
  __shared__ _Float16 ws0[TM * KS], ws1[TM * KS], ws2[TM * KS];
  auto xbuf = [&](auto tag) -> _Float16* {
    if constexpr (decltype(tag)::value == 0) return xs0;
    else if constexpr (decltype(tag)::value == 1) return xs1;
    else return xs2;
  };
  auto wbuf = [&](auto tag) -> _Float16* {
    if constexpr (decltype(tag)::value == 0) return ws0;
    else if constexpr (decltype(tag)::value == 1) return ws1;
    else return ws2;
  };
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t wm = wave & 1u, wn = wave >> 1;
  const uint32_t L = blockIdx.x, inner = n_tiles * splits;
  const uint32_t sidx = L >> 3, mt = (sidx / inner) * 8u + (L & 7u);
  if (mt >= m_tiles) return;
  const uint32_t rr = sidx % inner, nt = rr % n_tiles, sp = rr / n_tiles;
  const uint32_t n_base = nt * TN;
  const uint32_t nst = a.K / KS, st0 = sp * nst / splits, st1 = (sp + 1) * nst / splits;

  // this lane's rows and logical chunks: token chunk c = tid + 256 j (j < 4):
  // plane c / 512, row (c / 4) % 128; weight chunk c = tid + 256 j (j < 2):
  // slot c / 4.  The LDS destination of the wave's load j is the 1 KiB at the
  // tile row of its lane 0.
  // Source addresses are a wave-uniform base (scalar registers, advanced by
  // the stage's k offset) plus a loop-invariant 32-bit lane offset, so the
  // loads take the scalar-base form and no address register is rebuilt.
  const uint32_t pc = lane & 3u;  // physical chunk
  const uint8_t* xbase[4];
  uint32_t xoff[4], xdst[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t c = tid + 256u * j, plane = c >> 9, row = (c >> 2) & 127u;
    xbase[j] = reinterpret_cast<const uint8_t*>((plane ? a.xl : a.xh) + size_t(n_base) * a.K);
    xoff[j] = (row * a.K + ((pc ^ swz(row)) << 3)) * 2u;
    xdst[j] = plane * (TN * KS) + (((c & ~63u) >> 2) & 127u) * KS;  // halfs, wave-uniform
  }
  const uint8_t* wbase[2];
  uint32_t woff[2], wdst[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const uint32_t c = tid + 256u * j, slot = c >> 2;
    uint32_t row;
    const uint8_t* base = a.w;
    if constexpr (DUAL_EPI(EPI)) {
      const uint32_t grp = slot >> 5;  // w1 / w3 alternate every 32 slots: uniform over a wave
      row = mt * 64u + (grp >> 1) * 32u + (slot & 31u);
      base = (grp & 1u) ? a.w3 : a.w;
      const uint64_t bu = reinterpret_cast<uint64_t>(base);
      base = reinterpret_cast<const uint8_t*>(
          uint64_t(uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(bu))))) |
          (uint64_t(uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(bu >> 32))))) << 32));
    } else {
      row = mt * TM + slot;
    }
    wbase[j] = base;
    woff[j] = uint32_t(min(row, a.M - 1) * a.row_bytes) + ((pc ^ swz(slot)) << 4);
    wdst[j] = ((c & ~63u) >> 2) * KS;
  }
  // The address registers of a stage's loads are kept live until the end of
  // the step that issued them (`hold`): were they reused for a fragment
  // read's result, the compiler would first wait for every load in flight.
  const uint8_t* src[6];
  auto issue = [&](uint32_t st, auto tag) {
    const uint32_t kb = min(st, st1 - 1u) * (KS * 2u);  // bytes; past the range: a valid, unused stage
    _Float16* xb = xbuf(tag);
    _Float16* wb = wbuf(tag);
#pragma unroll
    for (int j = 0; j < 4; ++j) src[j] = xbase[j] + kb + xoff[j];
#pragma unroll
    for (int j = 0; j < 2; ++j) src[4 + j] = wbase[j] + kb + woff[j];
#pragma unroll
    for (int j = 0; j < 4; ++j) dma16(src[j], xb + xdst[j]);
#pragma unroll
    for (int j = 0; j < 2; ++j) dma16(src[4 + j], wb + wdst[j]);
  };
  auto hold = [&]() {
    asm volatile("" : : "v"(src[0]), "v"(src[1]), "v"(src[2]), "v"(src[3]), "v"(src[4]), "v"(src[5]));
  };

  floatx16 acc[2][2], accl[1][1];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = floatx16{};
  const uint32_t fr = lane & 31u, fk = 8u * (lane >> 5);
  // stage st in buffer B: wait until it has landed in every thread (only the
  // next stage's loads may still be in flight), then the buffer of stage st - 1
  // is free for stage st + 2
  auto step = [&](uint32_t st, auto tag) {
    constexpr int B = decltype(tag)::value;
    __builtin_amdgcn_s_waitcnt(0x0F70 | GEMM_DMA_PER_STAGE);  // vmcnt(6); lgkmcnt / expcnt unconstrained
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    // every fragment of the stage is read before the next loads are issued
    // (an LDS read behind an LDS-DMA load makes the compiler wait for it)
    const _Float16* xb = xbuf(tag);
    const _Float16* wb = wbuf(tag);
    half8 xa[2][2][2], wf[2][2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint32_t kk = 16u * q;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int p = 0; p < 2; ++p)
          xa[q][t][p] = *reinterpret_cast<const half8*>(xb + p * (TN * KS) + tile_off(64 * wn + 32 * t + fr, kk + fk));
#pragma unroll
      for (int t = 0; t < 2; ++t)
        wf[q][t] = *reinterpret_cast<const half8*>(wb + tile_off(64 * wm + 32 * t + fr, kk + fk));
    }
    issue(st + 2, StageTag<(B + 2) % 3>{});
#pragma unroll
    for (int q = 0; q < 2; ++q)
      // the four accumulators' hi products first, then their lo products
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int tn = 0; tn < 2; ++tn)
#pragma unroll
          for (int tm = 0; tm < 2; ++tm)
            acc[tn][tm] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xa[q][tn][p], wf[q][tm], acc[tn][tm], 0, 0, 0);
    hold();
  };
  issue(st0, StageTag<0>{});
  issue(st0 + 1, StageTag<1>{});
  for (uint32_t st = st0; st < st1; st += 3) {
    step(st, StageTag<0>{});
    if (st + 1 < st1) step(st + 1, StageTag<1>{});
    if (st + 2 < st1) step(st + 2, StageTag<2>{});
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // the unused tail loads have landed before the block ends
  gemm_epilogue<W_F16, EPI>(a, acc, accl, mt, n_base, sp, splits, wm, wn, lane);
}

// y[n][m] (op)= rs[n] * (part[0][n][m] + part[1][n][m] + ...), splits added in
// order; one thread per 4 consecutive outputs (M % 4 == 0).
template <int EPI>
__global__ __launch_bounds__(256) void gemm_split_reduce_kernel(GemmArgs a, uint32_t splits) {
  const uint32_t m4 = a.M / 4u;
  const size_t i = size_t(blockIdx.x) * 256u + threadIdx.x;
  if (i >= size_t(a.N) * m4) return;
  const uint32_t n = uint32_t(i / m4), m = uint32_t(i % m4) * 4u;
  const size_t plane = size_t(a.N) * a.M;
  const float* p = a.part + size_t(n) * a.M + m;
  float4 s = *reinterpret_cast<const float4*>(p);
  for (uint32_t k = 1; k < splits; ++k) {
    const float4 t = *reinterpret_cast<const float4*>(p + k * plane);
    s.x += t.x;
    s.y += t.y;
    s.z += t.z;
    s.w += t.w;
  }
  const float r = a.rs[n];
  float* dst = a.y + size_t(n) * a.ldy + m;
  const float v[4] = {s.x * r, s.y * r, s.z * r, s.w * r};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if constexpr (EPI == EPI_STORE) dst[e] = v[e];
    else dst[e] = __fadd_rn(dst[e], v[e]);
  }
}

// ---------------------------------------------------------------------------
// Skinny MFMA product for 1..16 columns (batched decode):
//   y[c][m] (op)= rs[c] * sum_k W[m][k] * x[c][k],  x as split planes [16][K].
// Block = 16 weight rows x 8 waves; wave w covers K range [w K/8, (w+1) K/8)
// in steps of 32 (one v_mfma_f32_16x16x32_f16 per plane and weight part),
// with two 4-step register batches in flight (loads of the next batch issue
// before the current batch's MFMAs); the 8 partial 16x16 tiles are summed in
// LDS and wave 0 applies the epilogue.  Row mapping as in the decode GEMV
// (row_base / extra_row).
// ---------------------------------------------------------------------------
typedef float floatx4 __attribute__((ext_vector_type(4)));
constexpr int SK_WAVES = 8, SK_D = 4;

template <uint32_t WT, int EPI>
__global__ __launch_bounds__(SK_WAVES * 64) void skinny_mfma_kernel(SkinnyArgs a) {
  constexpr bool DUAL = (EPI == EPI_SWIGLU_SLOW || EPI == EPI_SWIGLU_FAST);
  constexpr bool WSPLIT = WT != W_F16;
  constexpr int NW = DUAL ? 2 : 1;
  __shared__ floatx4 red[SK_WAVES][2 * NW][64];
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t m0 = blockIdx.x * 16;
  uint32_t lr = min(m0 + (lane & 15u), a.M - 1);
  const uint32_t wr = (a.extra_row != NO_ROW && lr == a.M - 1) ? a.extra_row : a.row_base + lr;
  const uint8_t* wp[NW];
  wp[0] = a.w + size_t(wr) * a.row_bytes;
  if constexpr (DUAL) wp[NW - 1] = a.w3 + size_t(wr) * a.row_bytes;
  const uint32_t koff = 8u * (lane >> 4);
  const uint32_t tok = lane & 15u;
  const _Float16* xhp = a.xh + size_t(tok) * a.K + koff;
  const _Float16* xlp = a.xl + size_t(tok) * a.K + koff;
  const uint32_t kq = a.K / SK_WAVES, kbeg = wave * kq, steps = kq / 32;
  const uint32_t done = a.done ? *a.done : 0u;

  struct Step {
    half8 wh[NW], wl[NW], bh, bl;
  };
  auto load = [&](Step& st, uint32_t s) {
    const uint32_t k = kbeg + 32u * min(s, steps - 1);  // clamped: past-the-end steps reload the last one
#pragma unroll
    for (int m = 0; m < NW; ++m) weight8<WT>(wp[m], k + koff, st.wh[m], st.wl[m]);
    st.bh = *reinterpret_cast<const half8*>(xhp + k);
    st.bl = *reinterpret_cast<const half8*>(xlp + k);
  };
  floatx4 acc[NW], accl[NW];
#pragma unroll
  for (int m = 0; m < NW; ++m) {
    acc[m] = floatx4{};
    accl[m] = floatx4{};
  }
  auto compute = [&](const Step& st) {
#pragma unroll
    for (int m = 0; m < NW; ++m) {
      acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(st.wh[m], st.bh, acc[m], 0, 0, 0);
      acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(st.wh[m], st.bl, acc[m], 0, 0, 0);
      if constexpr (WSPLIT) accl[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(st.wl[m], st.bh, accl[m], 0, 0, 0);
    }
  };
  Step x0[SK_D], x1[SK_D];
#pragma unroll
  for (int i = 0; i < SK_D; ++i) load(x0[i], i);
  for (uint32_t s = 0; s < steps; s += 2 * SK_D) {
#pragma unroll
    for (int i = 0; i < SK_D; ++i) load(x1[i], s + SK_D + i);
#pragma unroll
    for (int i = 0; i < SK_D; ++i)
      if (s + i < steps) compute(x0[i]);
#pragma unroll
    for (int i = 0; i < SK_D; ++i) load(x0[i], s + 2 * SK_D + i);
#pragma unroll
    for (int i = 0; i < SK_D; ++i)
      if (s + SK_D + i < steps) compute(x1[i]);
  }
#pragma unroll
  for (int m = 0; m < NW; ++m) {
    red[wave][2 * m][lane] = acc[m];
    red[wave][2 * m + 1][lane] = accl[m];
  }
  __syncthreads();
  if (wave != 0 || done) return;
#pragma unroll
  for (int m = 0; m < NW; ++m) {
    floatx4 t = red[0][2 * m][lane], tl = red[0][2 * m + 1][lane];
#pragma unroll
    for (int w = 1; w < SK_WAVES; ++w) {
      t += red[w][2 * m][lane];
      tl += red[w][2 * m + 1][lane];
    }
    acc[m] = t;
    accl[m] = tl;
  }
  // lane holds D[4 (lane / 16) + v][lane % 16]: rows 4 (lane/16) + v, column lane % 16
  const uint32_t c = lane & 15u;
  if (c >= a.N) return;
  const float r = a.rs[c];
  float* yrow = a.y + size_t(c) * a.ldy;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const uint32_t m = m0 + 4 * (lane >> 4) + v;
    if (m >= a.M) continue;
    float g = acc[0][v];
    if constexpr (WSPLIT) g = g + accl[0][v] * (1.0f / 2048.0f);
    g *= r;
    if constexpr (EPI == EPI_STORE) {
      yrow[m] = g;
    } else if constexpr (EPI == EPI_RESID) {
      yrow[m] = __fadd_rn(yrow[m], g);
    } else {
      float u = acc[NW - 1][v];
      if constexpr (WSPLIT) u = u + accl[NW - 1][v] * (1.0f / 2048.0f);
      u *= r;
      if constexpr (EPI == EPI_SWIGLU_SLOW) {
        const float sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf_glibc(-g)));
        yrow[m] = __fmul_rn(__fmul_rn(g, sig), u);
      } else {
        yrow[m] = __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, expf_glibc(-g))), u);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Causal GQA attention for a prompt chunk on the MFMA units: query c
// (0 <= c < N) sits at position base + c and attends cache positions
// 0 .. base + c (its own K/V already appended).
//   Block (32 queries, kv head g, key split sp), wave w = q head g * rep + w;
//   the waves share each 32-key K/V tile in LDS.  Per tile a wave computes
//   the scores transposed, S^T = K Q^T (v_mfma_f32_32x32x16_f16, K as A from
//   LDS, the wave's Q as B in registers), so a lane owns one query and 16 of
//   the tile's keys: the online softmax (running max and sum per query, f32)
//   is in-lane plus one exchange with the lane 32 away.  Then O^T += V^T P^T
//   with P^T straight from the score registers as the B operand and V^T from
//   LDS, stored transposed with bits 2 and 3 of the key index swapped (the
//   key order of the score registers), so O^T also has a query per lane and
//   the softmax rescale stays in-lane.
//   Precision (the reference computes in f32): q, k, v and p are split into
//   f16 x = hi + lo (lo = f16(x - hi)), and each product is accumulated as
//   hi.hi + hi.lo + lo.hi in one f32 accumulator (~2^-22 relative per term
//   for |x| >= 2^-3; below that lo is subnormal, absolute 2^-25).  A q, k or
//   v beyond the f16 range sets ERR_F16_RANGE.
//   Key split (splits > 1): the causal key range of the block's last query
//   is cut into `splits` runs of whole tiles, one per block; each writes its
//   running (max, sum) and unnormalised O to the workspace and
//   attn_prefill_merge_kernel combines them in split order.
//   The next tile's K/V loads are in flight while the current one computes.
// ---------------------------------------------------------------------------
constexpr int AQ = 32, AT = 32;  // queries per block, keys per tile
constexpr uint32_t ATTN_MAX_SPLITS = 4;

__device__ __forceinline__ void split_h(float x, _Float16& h, _Float16& l) {
  h = _Float16(x);
  l = _Float16(x - float(h));
}

// position of key j (0..31) of a tile in the transposed V layout: bits 2 and 3 swapped
__device__ __forceinline__ uint32_t vt_pos(uint32_t j) { return (j & ~12u) | ((j & 4u) << 1) | ((j & 8u) >> 1); }

template <int HD, bool KH>
__global__ __launch_bounds__(256, 2) void attn_prefill_kernel(PrefillAttnArgs a, uint32_t splits) {
  using KT = std::conditional_t<KH, uint16_t, float>;  // cache element: f16 bits or f32
  constexpr int DS = HD / 16;          // 16-wide k steps of the scores
  constexpr int DT = HD / 32;          // 32-wide output tiles
  constexpr int KP = HD + 8;           // padded K row (halfs)
  constexpr int VP = AT + 8;           // padded V^T row (halfs)
  constexpr int KF4 = AT * HD / 4 / 256;   // K float4 per thread per tile
  constexpr int VG = HD * (AT / 4) / 256;  // V (dim, 4-key group) pairs per thread per tile
  __shared__ _Float16 ks[2][AT][KP];   // hi, lo planes
  __shared__ _Float16 vts[2][HD][VP];
  __shared__ uint32_t bad;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t q0 = blockIdx.x * AQ, g = blockIdx.y, sp = blockIdx.z;
  const uint32_t rep = a.H / a.Hkv;
  const bool active = wave < rep;
  const uint32_t h = g * rep + (active ? wave : 0u);
  const uint32_t base = *a.pos_ptr + a.pos_offset;
  const uint32_t nq = min(uint32_t(AQ), a.N - q0);
  const uint32_t t_end = base + q0 + nq;  // keys needed by the last query
  // this block's run of whole tiles
  const uint32_t n_tiles = (t_end + AT - 1) / AT, per = (n_tiles + splits - 1) / splits;
  const uint32_t tile_lo = min(sp * per, n_tiles), tile_hi = min(tile_lo + per, n_tiles);
  const uint32_t fr = lane & 31u, fk = 8u * (lane >> 5);
  if (tid == 0) bad = 0;
  uint32_t my_bad = 0;

  // the wave's queries as the B operand of S^T: query q0 + fr, dims 16 ds + fk .. + 7
  half8 qh[DS], ql[DS];
  {
    const uint32_t qi = q0 + min(fr, nq - 1u);
    const float* qrow = a.q + size_t(qi) * a.H * HD + size_t(h) * HD + fk;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      const float4 u = *reinterpret_cast<const float4*>(qrow + 16 * ds);
      const float4 w = *reinterpret_cast<const float4*>(qrow + 16 * ds + 4);
      const float x[8] = {u.x, u.y, u.z, u.w, w.x, w.y, w.z, w.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        _Float16 hh, ll;
        split_h(x[e], hh, ll);
        qh[ds][e] = hh;
        ql[ds][e] = ll;
        my_bad |= !(fabsf(x[e]) < 65504.0f);
      }
    }
  }

  const KT* kc = reinterpret_cast<const KT*>(a.k_cache) + size_t(g) * a.max_seq * HD;
  const KT* vc = reinterpret_cast<const KT*>(a.v_cache) + size_t(g) * a.max_seq * HD;
  // tile loads: K float4 f = tid + 256 j -> key f / (HD / 4), dims (f % (HD / 4)) * 4;
  // V pair p = tid + 256 j -> dim p % HD, keys 4 (p / HD) .. + 3
  float4 kr[KF4];
  float vr[VG][4];
  auto load_tile = [&](uint32_t t0) {
#pragma unroll
    for (int j = 0; j < KF4; ++j) {
      const uint32_t f = tid + 256u * j, key = f / (HD / 4), d = (f % (HD / 4)) * 4u;
      const uint32_t t = min(t0 + key, a.max_seq - 1u);
      if constexpr (KH) {
        const uint2 r = *reinterpret_cast<const uint2*>(kc + size_t(t) * HD + d);
        const __half2 lo = *reinterpret_cast<const __half2*>(&r.x), hi = *reinterpret_cast<const __half2*>(&r.y);
        const float2 x0 = __half22float2(lo), x1 = __half22float2(hi);
        kr[j] = make_float4(x0.x, x0.y, x1.x, x1.y);
      } else {
        kr[j] = *reinterpret_cast<const float4*>(kc + size_t(t) * HD + d);
      }
      // keys past the last query: zero, so that whatever an earlier call left
      // in the cache there (masked anyway) cannot flag a range error
      if (t0 + key >= t_end) kr[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int j = 0; j < VG; ++j) {
      const uint32_t p = tid + 256u * j, d = p % HD, k0 = 4u * (p / HD);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t t = t0 + k0 + i;
        float v;
        if constexpr (KH) v = half_bits_to_float_p(vc[size_t(min(t, a.max_seq - 1u)) * HD + d]);
        else v = vc[size_t(min(t, a.max_seq - 1u)) * HD + d];
        vr[j][i] = t < t_end ? v : 0.0f;  // keys past the last query: zero (p is 0 there)
      }
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int j = 0; j < KF4; ++j) {
      const uint32_t f = tid + 256u * j, key = f / (HD / 4), d = (f % (HD / 4)) * 4u;
      const float x[4] = {kr[j].x, kr[j].y, kr[j].z, kr[j].w};
      _Float16 hh[4], ll[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        split_h(x[i], hh[i], ll[i]);
        my_bad |= !(fabsf(x[i]) < 65504.0f);
      }
      *reinterpret_cast<uint2*>(&ks[0][key][d]) = *reinterpret_cast<const uint2*>(hh);
      *reinterpret_cast<uint2*>(&ks[1][key][d]) = *reinterpret_cast<const uint2*>(ll);
    }
#pragma unroll
    for (int j = 0; j < VG; ++j) {
      const uint32_t p = tid + 256u * j, d = p % HD, k0 = 4u * (p / HD);
      _Float16 hh[4], ll[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        split_h(vr[j][i], hh[i], ll[i]);
        my_bad |= !(fabsf(vr[j][i]) < 65504.0f);
      }
      // keys k0 .. k0 + 3 (k0 % 4 == 0) stay consecutive under vt_pos
      *reinterpret_cast<uint2*>(&vts[0][d][vt_pos(k0)]) = *reinterpret_cast<const uint2*>(hh);
      *reinterpret_cast<uint2*>(&vts[1][d][vt_pos(k0)]) = *reinterpret_cast<const uint2*>(ll);
    }
  };

  floatx16 o[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) o[i] = floatx16{};
  float m = -INFINITY, lsum = 0.0f;
  const uint32_t qpos = base + q0 + fr;  // this lane's query position
  const bool qvalid = fr < nq;
  if (tile_lo < tile_hi) load_tile(tile_lo * AT);
  for (uint32_t tile = tile_lo; tile < tile_hi; ++tile) {
    const uint32_t t0 = tile * AT;
    __syncthreads();  // the previous tile is consumed
    store_tile();
    __syncthreads();
    if (tile + 1 < tile_hi) load_tile(t0 + AT);  // in flight during this tile
    if (!active) continue;
    // S^T[key][query]: lane holds query fr, keys 8 (v / 4) + 4 (lane / 32) + v % 4
    floatx16 sacc = floatx16{};
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      const half8 kh = *reinterpret_cast<const half8*>(&ks[0][fr][16 * ds + fk]);
      const half8 kl = *reinterpret_cast<const half8*>(&ks[1][fr][16 * ds + fk]);
      sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kh, qh[ds], sacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kh, ql[ds], sacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kl, qh[ds], sacc, 0, 0, 0);
    }
    float s[16];
    float mt = -INFINITY;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const uint32_t key = t0 + 8u * (v / 4) + 4u * (lane >> 5) + (v % 4);
      const bool vis = qvalid && key <= qpos;
      s[v] = vis ? sacc[v] * a.scale : -INFINITY;
      mt = fmaxf(mt, s[v]);
    }
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float mn = fmaxf(m, mt);
    const float corr = (m == -INFINITY) ? 0.0f : expf(m - mn);
    float ps = 0.0f;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      s[v] = (s[v] == -INFINITY) ? 0.0f : expf(s[v] - mn);
      ps += s[v];
    }
    ps += __shfl_xor(ps, 32, 64);
    lsum = lsum * corr + ps;
    m = mn;
    // a factor of exactly 1 (no query's max moved) changes nothing
    if (__any(corr != 1.0f)) {
#pragma unroll
      for (int i = 0; i < DT; ++i) o[i] = o[i] * corr;
    }
    // P^T as the B operand: 16-key step st takes score registers 8 st .. 8 st + 7
    half8 ph[2], pl[2];
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        _Float16 hh, ll;
        split_h(s[8 * st + e], hh, ll);
        ph[st][e] = hh;
        pl[st][e] = ll;
      }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const half8 vh = *reinterpret_cast<const half8*>(&vts[0][32 * dt + fr][16 * st + fk]);
        const half8 vl = *reinterpret_cast<const half8*>(&vts[1][32 * dt + fr][16 * st + fk]);
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vh, ph[st], o[dt], 0, 0, 0);
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vh, pl[st], o[dt], 0, 0, 0);
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vl, ph[st], o[dt], 0, 0, 0);
      }
  }
  if (my_bad) bad = 1;  // any writer sets it
  __syncthreads();
  if (tid == 0 && bad && a.err) atomicOr(a.err, ERR_F16_RANGE);
  if (!active || !qvalid) return;
  // O^T[dim][query]: lane holds query fr, dims 32 dt + 8 (v / 4) + 4 (lane / 32) + v % 4
  if (splits == 1) {
    float* dst = a.out + size_t(q0 + fr) * a.H * HD + size_t(h) * HD;
    const float inv = 1.0f / lsum;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float4 v4 = make_float4(o[dt][4 * r] * inv, o[dt][4 * r + 1] * inv, o[dt][4 * r + 2] * inv,
                                      o[dt][4 * r + 3] * inv);
        *reinterpret_cast<float4*>(dst + 32 * dt + 8 * r + 4 * (lane >> 5)) = v4;
      }
  } else {
    // partial: [split][query][head][HD + 4]: unnormalised O, then (max, sum) (rows 16-byte aligned)
    float* dst = a.part + ((size_t(sp) * a.N + q0 + fr) * a.H + h) * (HD + 4);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) dst[32 * dt + 8 * r + 4 * (lane >> 5) + c] = o[dt][4 * r + c];
    if (lane < 32) {
      dst[HD] = m;
      dst[HD + 1] = lsum;
    }
  }
}

// Merges the key splits of attn_prefill_kernel: 32 threads per (query, head)
// pair, 4 dims each; every split's partial is loaded in one batch, then
// combined in split order (a split that saw no key has max -inf and adds 0).
template <int HD>
__global__ __launch_bounds__(256) void attn_prefill_merge_kernel(PrefillAttnArgs a, uint32_t splits) {
  constexpr uint32_t TPP = HD / 4;  // threads per pair
  const uint32_t pair = blockIdx.x * (256 / TPP) + threadIdx.x / TPP, d = (threadIdx.x % TPP) * 4;
  if (pair >= a.N * a.H) return;
  const uint32_t q = pair / a.H, h = pair % a.H;
  const size_t stride = size_t(a.N) * a.H * (HD + 4);
  const float* p = a.part + (size_t(q) * a.H + h) * (HD + 4);
  float ms[ATTN_MAX_SPLITS], ls[ATTN_MAX_SPLITS];
  float4 os[ATTN_MAX_SPLITS];
#pragma unroll
  for (uint32_t s = 0; s < ATTN_MAX_SPLITS; ++s) {
    const float* ps = p + min(s, splits - 1u) * stride;
    ms[s] = ps[HD];
    ls[s] = ps[HD + 1];
    os[s] = *reinterpret_cast<const float4*>(ps + d);
  }
  float M = -INFINITY;
#pragma unroll
  for (uint32_t s = 0; s < ATTN_MAX_SPLITS; ++s)
    if (s < splits) M = fmaxf(M, ms[s]);
  float L = 0.0f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (uint32_t s = 0; s < ATTN_MAX_SPLITS; ++s) {
    if (s >= splits || ms[s] == -INFINITY) continue;
    const float f = expf(ms[s] - M);
    L = fmaf(ls[s], f, L);
    acc.x = fmaf(os[s].x, f, acc.x);
    acc.y = fmaf(os[s].y, f, acc.y);
    acc.z = fmaf(os[s].z, f, acc.z);
    acc.w = fmaf(os[s].w, f, acc.w);
  }
  const float inv = 1.0f / L;
  *reinterpret_cast<float4*>(a.out + size_t(q) * a.H * HD + size_t(h) * HD + d) =
      make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
}

}  // namespace

hipError_t launch_split_rows(const float* x, uint32_t ldx, const float* norm, float eps, uint32_t N, uint32_t Npad,
                             uint32_t K, _Float16* xh, _Float16* xl, float* rs, uint32_t* err, hipStream_t s) {
  if (Npad < N || Npad % 16 || K % KS) return hipErrorInvalidValue;
  hipLaunchKernelGGL(split_rows_kernel, dim3(Npad), dim3(256), 0, s, x, ldx, norm, eps, N, K, xh, xl, rs, err);
  return hipGetLastError();
}

// Two register sets in flight (stage st + 2 loads while st computes): 3 and
// 4 sets measured the same for 1536-token prefill (92.3 / 94.3 / 93.1 ms).
constexpr int GEMM_DEPTH = 2;

static hipError_t gemm_f16(int epi, const GemmArgs& a, uint32_t m_tiles, uint32_t n_tiles, uint32_t splits,
                           hipStream_t s) {
  const dim3 grid((m_tiles + 7u) / 8u * 8u * n_tiles * splits), block(256);
  switch (epi) {
    case EPI_STORE:
      hipLaunchKernelGGL((gemm_f16_dma_kernel<EPI_STORE>), grid, block, 0, s, a, m_tiles, n_tiles, splits);
      break;
    case EPI_RESID:
      hipLaunchKernelGGL((gemm_f16_dma_kernel<EPI_RESID>), grid, block, 0, s, a, m_tiles, n_tiles, splits);
      break;
    case EPI_SWIGLU_SLOW:
      hipLaunchKernelGGL((gemm_f16_dma_kernel<EPI_SWIGLU_SLOW>), grid, block, 0, s, a, m_tiles, n_tiles, splits);
      break;
    case EPI_SWIGLU_FAST:
      hipLaunchKernelGGL((gemm_f16_dma_kernel<EPI_SWIGLU_FAST>), grid, block, 0, s, a, m_tiles, n_tiles, splits);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <uint32_t WT>
static hipError_t gemm_epi(int epi, const GemmArgs& a, uint32_t m_tiles, uint32_t n_tiles, uint32_t splits,
                           hipStream_t s) {
  const dim3 grid((m_tiles + 7u) / 8u * 8u * n_tiles * splits), block(256);
  if (WT == W_F16) {
    const hipError_t e = gemm_f16(epi, a, m_tiles, n_tiles, splits, s);
    if (e != hipSuccess) return e;
  } else {
  switch (epi) {
    case EPI_STORE:
      hipLaunchKernelGGL((gemm_mfma_kernel<WT, EPI_STORE, GEMM_DEPTH>), grid, block, 0, s, a, m_tiles, n_tiles,
                         splits);
      break;
    case EPI_RESID:
      hipLaunchKernelGGL((gemm_mfma_kernel<WT, EPI_RESID, GEMM_DEPTH>), grid, block, 0, s, a, m_tiles, n_tiles,
                         splits);
      break;
    case EPI_SWIGLU_SLOW:
      hipLaunchKernelGGL((gemm_mfma_kernel<WT, EPI_SWIGLU_SLOW, GEMM_DEPTH>), grid, block, 0, s, a, m_tiles, n_tiles,
                         splits);
      break;
    case EPI_SWIGLU_FAST:
      hipLaunchKernelGGL((gemm_mfma_kernel<WT, EPI_SWIGLU_FAST, GEMM_DEPTH>), grid, block, 0, s, a, m_tiles, n_tiles,
                         splits);
      break;
    default: return hipErrorInvalidValue;
  }
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || splits == 1) return e;
  const dim3 rgrid(uint32_t((size_t(a.N) * (a.M / 4u) + 255u) / 256u));
  if (epi == EPI_STORE)
    hipLaunchKernelGGL((gemm_split_reduce_kernel<EPI_STORE>), rgrid, block, 0, s, a, splits);
  else
    hipLaunchKernelGGL((gemm_split_reduce_kernel<EPI_RESID>), rgrid, block, 0, s, a, splits);
  return hipGetLastError();
}

uint32_t gemm_rows_pad(uint32_t n) { return (n + TN - 1) / TN * TN; }

size_t gemm_part_floats(uint32_t n_pad, uint32_t m) { return size_t(GEMM_MAX_SPLITS) * n_pad * m; }

hipError_t launch_gemm_mfma(uint32_t wtype, int epi, const GemmArgs& a, hipStream_t s) {
  if (a.K % KS || a.M == 0 || a.N == 0) return hipErrorInvalidValue;
  const bool dual = epi == EPI_SWIGLU_SLOW || epi == EPI_SWIGLU_FAST;
  if (dual && !a.w3) return hipErrorInvalidValue;
  const uint32_t m_tiles = dual ? (a.M + 63u) / 64u : (a.M + TM - 1u) / TM;
  const uint32_t n_tiles = gemm_rows_pad(a.N) / TN;
  // short-M products: split K so that the grid covers the 256 CUs (each split
  // keeps at least 8 stages of K)
  uint32_t splits = 1;
  if (!dual && a.part && a.M % 4u == 0) {
    const uint32_t tiles = m_tiles * n_tiles;
    while (splits < GEMM_MAX_SPLITS && tiles * splits < 256u && a.K / KS >= 8u * (splits + 1u) &&
           size_t(splits + 1u) * a.N * a.M <= a.part_cap)
      ++splits;
  }
  switch (wtype) {
    case W_F16: return gemm_epi<W_F16>(epi, a, m_tiles, n_tiles, splits, s);
    case W_Q8_0: return gemm_epi<W_Q8_0>(epi, a, m_tiles, n_tiles, splits, s);
    case W_Q4_0: return gemm_epi<W_Q4_0>(epi, a, m_tiles, n_tiles, splits, s);
    default: return hipErrorInvalidValue;
  }
}

template <uint32_t WT>
static hipError_t skinny_epi(int epi, const SkinnyArgs& a, dim3 grid, hipStream_t s) {
  const dim3 block(SK_WAVES * 64);
  switch (epi) {
    case EPI_STORE: hipLaunchKernelGGL((skinny_mfma_kernel<WT, EPI_STORE>), grid, block, 0, s, a); break;
    case EPI_RESID: hipLaunchKernelGGL((skinny_mfma_kernel<WT, EPI_RESID>), grid, block, 0, s, a); break;
    case EPI_SWIGLU_SLOW: hipLaunchKernelGGL((skinny_mfma_kernel<WT, EPI_SWIGLU_SLOW>), grid, block, 0, s, a); break;
    case EPI_SWIGLU_FAST: hipLaunchKernelGGL((skinny_mfma_kernel<WT, EPI_SWIGLU_FAST>), grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_skinny_mfma(uint32_t wtype, int epi, const SkinnyArgs& a, hipStream_t s) {
  if (a.N == 0 || a.N > 16 || a.M == 0 || a.K % (SK_WAVES * 32)) return hipErrorInvalidValue;
  const bool dual = epi == EPI_SWIGLU_SLOW || epi == EPI_SWIGLU_FAST;
  if (dual && !a.w3) return hipErrorInvalidValue;
  const dim3 grid((a.M + 15) / 16);
  switch (wtype) {
    case W_F16: return skinny_epi<W_F16>(epi, a, grid, s);
    case W_Q8_0: return skinny_epi<W_Q8_0>(epi, a, grid, s);
    case W_Q4_0: return skinny_epi<W_Q4_0>(epi, a, grid, s);
    default: return hipErrorInvalidValue;
  }
}

size_t attn_prefill_part_floats(uint32_t n, uint32_t heads, uint32_t hd) {
  return size_t(ATTN_MAX_SPLITS) * n * heads * (hd + 4);
}

template <int HD>
static void attn_prefill_launch(const PrefillAttnArgs& a, uint32_t splits, hipStream_t s) {
  const dim3 grid((a.N + AQ - 1) / AQ, a.Hkv, splits);
  hipLaunchKernelGGL((a.kv_f16 ? attn_prefill_kernel<HD, true> : attn_prefill_kernel<HD, false>), grid, dim3(256), 0,
                     s, a, splits);
  if (splits > 1)
    hipLaunchKernelGGL((attn_prefill_merge_kernel<HD>), dim3((a.N * a.H * (HD / 4) + 255) / 256), dim3(256), 0, s, a,
                       splits);
}

hipError_t launch_attention_prefill(const PrefillAttnArgs& a, hipStream_t s) {
  if (!a.pos_ptr || a.H % a.Hkv || a.H / a.Hkv > 4 || a.N == 0) return hipErrorInvalidValue;
  // key splits so that the grid covers the CUs twice over (two blocks fit a CU)
  const uint32_t blocks = (a.N + AQ - 1) / AQ * a.Hkv;
  uint32_t splits = 1;
  while (splits < ATTN_MAX_SPLITS && blocks * splits < 512u &&
         size_t(splits + 1) * a.N * a.H * (a.hd + 4) <= a.part_cap && a.part)
    ++splits;
  switch (a.hd) {
    case 64: attn_prefill_launch<64>(a, splits, s); break;
    case 128: attn_prefill_launch<128>(a, splits, s); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace s2
