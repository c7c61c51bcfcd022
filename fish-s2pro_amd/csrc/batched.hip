// batched.hip -- decode products for a batch of columns (gfx950, wave64).
//
// Y[n][m] (op)= sum_k W[m][k] x[n][k] for N <= 16 columns on the MFMA units
// (v_mfma_f32_16x16x32_f16).  A batch of decode columns reads every weight
// once, so the product is bound by HBM like the one-column GEMV; what
// decides its speed is the access pattern.  Weights are therefore kept a
// second time in MFMA fragment order: tile (tm, tk) of 16 rows x 32 k is one
// contiguous KiB whose 16 bytes at lane l are W[16 tm + l % 16][32 tk +
// 8 (l / 16) + e], e < 8 -- every wave load is one contiguous KiB and a wave
// walking k streams consecutive KiB.
//
// Activations stay f32 rows [N][ldx].  Each wave stages its k range of
// them through a private LDS double buffer with coalesced loads (512
// contiguous bytes per row and chunk of 4 steps, issued one chunk ahead), so
// the activation loads neither scatter over rows (the MFMA fragment puts the
// column in the fastest lane bits) nor hold up the weight loads' wait
// counter.  Each wave scales each column by a power of two that brings the
// largest |x| of its first two staged chunks (256 elements of its k range)
// to [1, 2).  Each scaled value is split into f16 hi = f16(x) and lo =
// f16((x - hi) 2^11) (x = hi + 2^-11 lo to ~2^-22 |x| for |x| >= 2^-14 of
// that maximum, absolute ~2^-35 of it below); hi and lo go through the MFMA
// with the same weight fragment, and each wave's sums are scaled back
// exactly before the waves' sums are added.  9-16 columns (bmm_kernel): the
// MFMA lanes split 8 values per step and run hi and lo through two MFMAs.
// Up to 8 columns (bmm_pk_kernel): the staging lanes split each value once
// and hi / lo share one MFMA's 16 columns.  So columns of any magnitude keep the same relative accuracy (1e-6
// or a raw pre-norm residual of 1e7 times its gain), and an element may be
// up to 2^15 times the maximum of the first chunks.  RMSNorm inputs: the sum
// of squares of each column is accumulated from the same values and the RMS
// scale is applied to the result (W.((x s) g) = s W.(x g)).  A non-finite
// activation (or one beyond that headroom) makes its column's sums
// non-finite; the epilogue reports that as ERR_F16_RANGE instead of
// returning a wrong product.
#include <hip/hip_runtime.h>
#include <math.h>

#include <algorithm>
#include <type_traits>

#include "expf_glibc.h"
#include "kernels.h"
#include "wave.h"

namespace s2 {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Tiling: destination chunk q (16 bytes) = tile q / 64, lane q % 64.  Logical
// row r < M maps to source row row_base + r, except the last one (r = M - 1)
// which maps to extra_row when extra_row != NO_ROW; rows M..Mpad-1 are zero.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void tile_f16_kernel(const uint16_t* src, uint32_t K, uint32_t M, uint32_t Mpad,
                                                       uint32_t row_base, uint32_t extra_row, uint16_t* dst) {
  const uint32_t kt = K / 32;
  const size_t chunks = size_t(Mpad / 16) * kt * 64;
  for (size_t q = size_t(blockIdx.x) * 256 + threadIdx.x; q < chunks; q += size_t(gridDim.x) * 256) {
    const size_t tile = q / 64;
    const uint32_t lane = uint32_t(q % 64);
    const uint32_t tm = uint32_t(tile / kt), tk = uint32_t(tile % kt);
    const uint32_t r = 16 * tm + lane % 16, k0 = 32 * tk + 8 * (lane / 16);
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (r < M) {
      const uint32_t sr = (extra_row != NO_ROW && r == M - 1) ? extra_row : row_base + r;
      v = *reinterpret_cast<const uint4*>(src + size_t(sr) * K + k0);
    }
    *reinterpret_cast<uint4*>(dst + q * 8) = v;
  }
}

// ---------------------------------------------------------------------------
// Batched product.  Block = WAVES waves on one 16-row tile; wave w takes the
// k steps [w KS, (w + 1) KS) (KS = K / 32 / WAVES), WIN weight steps and XW
// activation steps in flight (the schedule is pinned so the loads stay
// ahead of their MFMAs).  Lane l: column n = l % 16, k group l / 16.
// ---------------------------------------------------------------------------
constexpr int WIN = 8;        // weight steps in flight (two chunks)
constexpr int XC = 4;         // steps per staged activation chunk
constexpr int RS = 36;        // LDS floats per staged row and step (32 + 4: conflict-free fragment reads)

__device__ __forceinline__ void split8(const floatx4& a, const floatx4& b, half8& hi, half8& lo) {
  const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const _Float16 h = _Float16(v[e]);
    hi[e] = h;
    lo[e] = _Float16((v[e] - float(h)) * 2048.0f);
  }
}

// ---------------------------------------------------------------------------
// Product.  Block = WAVES waves on one 16-row tile; wave w takes the k steps
// [w KS, (w + 1) KS) (KS = K / 32 / WAVES).  The loop body has no branches
// (a branch around a load makes the compiler wait for every outstanding
// load at the join): steps run in pairs of chunks (WIN steps), loads past
// the end re-read in-bounds data, and a step past the end, or a column >= N,
// gets a zero activation by a select.  Lane l: column n = l % 16, k group
// l / 16.  NB = activation rows staged: 16 (this kernel serves 9-16
// columns; up to 8 take bmm_pk_kernel below).
// ---------------------------------------------------------------------------
// Weight fragments are read once per launch: non-temporal loads stream them
// past L2 without evicting the staged activations (8 columns: w13 24.4 ->
// 23.2 us).
__device__ __forceinline__ half8 bmm_wload(const half8* p) { return __builtin_nontemporal_load(p); }

template <int EPI, bool NORM, int WAVES, int NB>
__global__ __launch_bounds__(WAVES * 64) void bmm_kernel(BmmArgs a) {
  constexpr bool DUAL = (EPI == EPI_SWIGLU_SLOW || EPI == EPI_SWIGLU_FAST);
  constexpr int NW = DUAL ? 2 : 1;
  constexpr int CHF = XC * NB * RS;  // floats per chunk buffer
  constexpr int LDX = NB / 2;        // staging loads per chunk (2 rows x 512 B each)
  // each wave's staging buffers take its partial sums after its loop (2 NW x
  // 64 floatx4 = at most 4 KiB, inside the 2 CHF floats of the wave)
  static_assert(2 * NW * 64 * 4 <= 2 * CHF, "partials must fit the staging buffers");
  __shared__ __align__(16) float xs[WAVES][2][CHF];
  __shared__ float gs[WAVES][2][NORM ? XC * 32 : 1];
  __shared__ float ssq[WAVES][64];
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t tm = blockIdx.x, m0 = tm * 16;
  const uint32_t kt = a.K / 32, KS = kt / WAVES;
  const uint32_t n = lane & 15u, grp = lane >> 4;
  const size_t tile0 = (size_t(tm) * kt + size_t(wave) * KS) * 512 + size_t(lane) * 8;
  const _Float16* wp0 = a.wt + tile0;
  const _Float16* wp1 = DUAL ? a.wt3 + tile0 : wp0;
  const uint32_t last = KS - 1;
  const uint32_t nsc = (KS + WIN - 1) / WIN;  // pairs of chunks
  const uint32_t kbase = wave * KS * 32;
  // staging: load j of a chunk covers rows 2 j + lane / 32, 4-float group lane % 32
  const uint32_t srow = lane >> 5, sq = lane & 31u;
  float* xsw = &xs[wave][0][0];
  float* gsw = &gs[wave][0][0];

  auto stage_load = [&](floatx4 (&r)[LDX], floatx4& gr, uint32_t chunk) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < LDX; ++j) {
      const uint32_t row = 2 * j + srow;
      const uint32_t rr = row < a.N ? row : 0u;
      const uint32_t k = min(kbase + chunk * (XC * 32) + 4 * sq, a.K - 4);
      r[j] = *reinterpret_cast<const floatx4*>(a.x + size_t(rr) * a.ldx + k);
    }
    if constexpr (NORM) {
      const uint32_t k = min(kbase + chunk * (XC * 32) + 4 * (sq & 31u), a.K - 4);
      gr = *reinterpret_cast<const floatx4*>(a.norm + k);
    }
  };
  auto stage_store = [&](const floatx4 (&r)[LDX], const floatx4& gr, int buf) __attribute__((always_inline)) {
    // element (row, k = 4 sq + e) of the chunk -> step k / 32, offset k % 32
    const uint32_t st = sq / 8, off = 4 * (sq % 8);
#pragma unroll
    for (int j = 0; j < LDX; ++j) {
      const uint32_t row = 2 * j + srow;
      *reinterpret_cast<floatx4*>(xsw + buf * CHF + (st * NB + row) * RS + off) = r[j];
    }
    // both lane halves hold the same gain values: no branch around the store
    if constexpr (NORM) *reinterpret_cast<floatx4*>(gsw + buf * (XC * 32) + 4 * sq) = gr;
  };

  half8 wb[WIN][NW];
  floatx4 sxa[LDX], sxb[LDX], sga, sgb;  // staged chunks in flight (even, odd)
  // chunk 0 and 1 activations, then the first WIN weight steps
  stage_load(sxa, sga, 0);
  stage_load(sxb, sgb, 1);
#pragma unroll
  for (int i = 0; i < WIN; ++i) {
    const uint32_t t = min(uint32_t(i), last);
    wb[i][0] = bmm_wload(reinterpret_cast<const half8*>(wp0 + 512 * t));
    if constexpr (DUAL) wb[i][1] = bmm_wload(reinterpret_cast<const half8*>(wp1 + 512 * t));
  }
  stage_store(sxa, sga, 0);
  // Per-(wave, column) power-of-two scale: the largest |x g| of the first two
  // chunks of this wave's range (already in registers) is brought to [1, 2),
  // leaving 2^15 of headroom in the f16 hi part for the rest of the range.
  float rm[LDX];
#pragma unroll
  for (int j = 0; j < LDX; ++j) {
    floatx4 va = sxa[j], vb = sxb[j];
    if constexpr (NORM) {
      va = va * sga;
      vb = vb * sgb;
    }
    float m = fmaxf(fmaxf(fabsf(va.x), fabsf(va.y)), fmaxf(fabsf(va.z), fabsf(va.w)));
    m = fmaxf(m, fmaxf(fmaxf(fabsf(vb.x), fabsf(vb.y)), fmaxf(fabsf(vb.z), fabsf(vb.w))));
    rm[j] = row_reduce(m, [](float a, float b) { return fmaxf(a, b); });
  }
  // staged row 2 j is lanes 0-31, row 2 j + 1 lanes 32-63: the max of each
  // half from its two 16-lane rows, read into scalars
  float cmax = 0.0f;
#pragma unroll
  for (int j = 0; j < LDX; ++j) {
    const float lo = fmaxf(lane_read_f32(rm[j], 0), lane_read_f32(rm[j], 16));
    const float hi = fmaxf(lane_read_f32(rm[j], 32), lane_read_f32(rm[j], 48));
    cmax = (uint32_t(j) == (n >> 1)) ? ((n & 1u) ? hi : lo) : cmax;
  }
  // cmax in [2^e, 2^(e+1)): scale by 2^-e (e clamped to +-100; 0 for zero,
  // subnormal or non-finite maxima -- a non-finite value still ends as a
  // non-finite sum)
  int cexp = int((__float_as_uint(cmax) >> 23) & 0xffu) - 127;
  cexp = (cmax >= 1.0e-30f && cmax <= 1.0e30f) ? cexp : 0;
  const float cinv = __uint_as_float(uint32_t(127 - cexp) << 23);
  const float cscale = __uint_as_float(uint32_t(127 + cexp) << 23);
  __builtin_amdgcn_sched_barrier(0);

  floatx4 acc[NW], accl[NW];
#pragma unroll
  for (int m = 0; m < NW; ++m) {
    acc[m] = floatx4{};
    accl[m] = floatx4{};
  }
  float ss = 0.0f;
  const floatx4 z4 = floatx4{};
  const uint32_t rrow = n < NB ? n : n - NB;  // a valid staged row for every lane
  // the steps of chunk c from LDS buffer h (weight slots h XC .. h XC + 3)
  // the steps of chunk c from LDS buffer h (weight slots h XC .. h XC + 3);
  // each step's fragments are read from LDS one step ahead of their use
  auto chunk_steps = [&](uint32_t c, auto hc) __attribute__((always_inline)) {
    constexpr int h = decltype(hc)::value;
    const float* xb = xsw + h * CHF + rrow * RS + 8 * grp;
    const float* gb = gsw + h * (XC * 32) + 8 * grp;
    floatx4 cx0 = *reinterpret_cast<const floatx4*>(xb), cx1 = *reinterpret_cast<const floatx4*>(xb + 4);
    floatx4 cg0 = z4, cg1 = z4;
    if constexpr (NORM) {
      cg0 = *reinterpret_cast<const floatx4*>(gb);
      cg1 = *reinterpret_cast<const floatx4*>(gb + 4);
    }
#pragma unroll
    for (int i = 0; i < XC; ++i) {
      const uint32_t s = c * XC + i;
      const int wi = h * XC + i;
      floatx4 nx0 = z4, nx1 = z4, ng0 = z4, ng1 = z4;
      if (i + 1 < XC) {
        nx0 = *reinterpret_cast<const floatx4*>(xb + (i + 1) * NB * RS);
        nx1 = *reinterpret_cast<const floatx4*>(xb + (i + 1) * NB * RS + 4);
        if constexpr (NORM) {
          ng0 = *reinterpret_cast<const floatx4*>(gb + (i + 1) * 32);
          ng1 = *reinterpret_cast<const floatx4*>(gb + (i + 1) * 32 + 4);
        }
      }
      const bool live = n < a.N && s < KS;
      floatx4 x0 = live ? cx0 : z4, x1 = live ? cx1 : z4;
      if constexpr (NORM) {
        ss += (x0.x * x0.x + x0.y * x0.y) + (x0.z * x0.z + x0.w * x0.w);
        ss += (x1.x * x1.x + x1.y * x1.y) + (x1.z * x1.z + x1.w * x1.w);
        x0 = x0 * cg0;
        x1 = x1 * cg1;
      }
      x0 = x0 * cinv;
      x1 = x1 * cinv;
      half8 bh, bl;
      split8(x0, x1, bh, bl);
#pragma unroll
      for (int m = 0; m < NW; ++m) {
        acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wb[wi][m], bh, acc[m], 0, 0, 0);
        accl[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wb[wi][m], bl, accl[m], 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      const uint32_t tw = min(s + WIN, last);
      wb[wi][0] = bmm_wload(reinterpret_cast<const half8*>(wp0 + 512 * tw));
      if constexpr (DUAL) wb[wi][1] = bmm_wload(reinterpret_cast<const half8*>(wp1 + 512 * tw));
      __builtin_amdgcn_sched_barrier(0);
      cx0 = nx0;
      cx1 = nx1;
      cg0 = ng0;
      cg1 = ng1;
    }
  };
  for (uint32_t sc = 0; sc < nsc; ++sc) {
    // chunk 2 sc from buffer 0: first the odd chunk (loaded one chunk ago)
    // into buffer 1, then the loads of chunk 2 sc + 2
    stage_store(sxb, sgb, 1);
    stage_load(sxa, sga, 2 * sc + 2);
    __builtin_amdgcn_sched_barrier(0);
    chunk_steps(2 * sc, std::integral_constant<int, 0>{});
    // chunk 2 sc + 1 from buffer 1
    stage_store(sxa, sga, 0);
    stage_load(sxb, sgb, 2 * sc + 3);
    __builtin_amdgcn_sched_barrier(0);
    chunk_steps(2 * sc + 1, std::integral_constant<int, 1>{});
  }
  // partials of wave w: slot (2 m + part) lane of its own staging region
  auto red = [&](uint32_t w, int slot) __attribute__((always_inline)) -> floatx4* {
    return reinterpret_cast<floatx4*>(&xs[w][0][0]) + slot * 64 + lane;
  };
#pragma unroll
  for (int m = 0; m < NW; ++m) {
    *red(wave, 2 * m) = acc[m] * cscale;
    *red(wave, 2 * m + 1) = accl[m] * cscale;
  }
  if constexpr (NORM) ssq[wave][lane] = ss;
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int m = 0; m < NW; ++m) {
    floatx4 t = *red(0, 2 * m), tl = *red(0, 2 * m + 1);
#pragma unroll
    for (int w = 1; w < WAVES; ++w) {
      t += *red(w, 2 * m);
      tl += *red(w, 2 * m + 1);
    }
    acc[m] = t + tl * (1.0f / 2048.0f);
  }
  float r = 1.0f;
  if constexpr (NORM) {
    float t = ssq[0][lane];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) t += ssq[w][lane];
    // the four k groups of column n: lanes n, n + 16, n + 32, n + 48
    t = t + __shfl_xor(t, 16, 64);
    t = t + __shfl_xor(t, 32, 64);
    r = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(t, float(a.K)), a.eps)));
  }
  // a non-finite activation (or one beyond the split's range) leaves
  // non-finite sums
  bool bad = false;
#pragma unroll
  for (int m = 0; m < NW; ++m)
#pragma unroll
    for (int v = 0; v < 4; ++v) bad = bad || !(fabsf(acc[m][v]) <= 3.0e38f);
  bad = bad && n < a.N;
  if (__any(bad) && lane == 0 && a.err) atomicOr(a.err, ERR_F16_RANGE);
  const uint32_t done = a.done ? *a.done : 0u;
  if (done || n >= a.N) return;
  float* yrow = a.y + size_t(n) * a.ldy;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const uint32_t m = m0 + 4 * grp + v;
    if (m >= a.M) continue;
    const float g = acc[0][v] * r;
    if constexpr (EPI == EPI_STORE) {
      yrow[m] = g;
    } else if constexpr (EPI == EPI_RESID) {
      yrow[m] = __fadd_rn(yrow[m], g);
    } else {
      const float u = acc[NW - 1][v] * r;
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
// Product for up to 8 columns: hi and lo parts share one MFMA.  The B
// operand's 16 columns carry the hi parts of the 8 activation columns (0-7)
// and their lo parts (8-15), so one MFMA per weight step and matrix does the
// work of two, and no MFMA column is idle.  Each activation is split once,
// by the lane that stages it: the staging lanes scale and split their 16
// values of a chunk and write the f16 hi / lo fragments (plus, for RMSNorm
// inputs, each 4-value sum of squares) into the wave's LDS buffer; the MFMA
// lanes then read one 16-byte fragment per step and do no conversions.  The
// values, the scale, the MFMA columns' sums and every later addition are
// those of bmm_kernel, in the same order, so both give the same bits.
//   LDS per wave and buffer: XC steps x [16 fragment rows of PK_ROW halfs]
//   (row n < 8: hi of column n, row n + 8: its lo), and per step the sums of
//   squares [column][k group][half].
// ---------------------------------------------------------------------------
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
constexpr int PK_ROW = 40;                 // halfs per fragment row: 32 + 8 (conflict-free 16-byte reads)
constexpr int PK_STEP = 16 * PK_ROW + 32;  // halfs per step: +64 B puts the 4 steps' staging writes on other banks
constexpr int PK_QSTEP = 72;               // sum-of-squares floats per step: 8 columns x 4 groups x 2, +8

template <int EPI, bool NORM, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void bmm_pk_kernel(BmmArgs a) {
  constexpr bool DUAL = (EPI == EPI_SWIGLU_SLOW || EPI == EPI_SWIGLU_FAST);
  constexpr int NW = DUAL ? 2 : 1;
  constexpr int CHH = XC * PK_STEP;             // halfs per chunk buffer
  constexpr int CHQ = NORM ? XC * PK_QSTEP : 1;  // floats per chunk buffer
  constexpr int LDX = 4;                        // staging loads per chunk (8 rows, 2 per load)
  // each wave's partial sums go to its own staging buffers after its loop
  static_assert(NW * 64 * 16 <= 2 * CHH * 2, "partials must fit the staging buffers");
  __shared__ __align__(16) _Float16 fs[WAVES][2][CHH];
  __shared__ __align__(16) float qs[WAVES][2][CHQ];
  __shared__ float ssq[WAVES][64];
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t tm = blockIdx.x, m0 = tm * 16;
  const uint32_t kt = a.K / 32, KS = kt / WAVES;
  const uint32_t n = lane & 15u, grp = lane >> 4, col = n & 7u;
  const size_t tile0 = (size_t(tm) * kt + size_t(wave) * KS) * 512 + size_t(lane) * 8;
  const _Float16* wp0 = a.wt + tile0;
  const _Float16* wp1 = DUAL ? a.wt3 + tile0 : wp0;
  const uint32_t last = KS - 1;
  const uint32_t nsc = (KS + WIN - 1) / WIN;  // pairs of chunks
  const uint32_t kbase = wave * KS * 32;
  // staging: load j of a chunk covers rows 2 j + lane / 32, 4-float group lane % 32
  const uint32_t srow = lane >> 5, sq = lane & 31u;
  _Float16* fsw = &fs[wave][0][0];
  float* qsw = &qs[wave][0][0];

  auto stage_load = [&](floatx4 (&r)[LDX], floatx4& gr, uint32_t chunk) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < LDX; ++j) {
      const uint32_t row = 2 * j + srow;
      const uint32_t rr = row < a.N ? row : 0u;
      const uint32_t k = min(kbase + chunk * (XC * 32) + 4 * sq, a.K - 4);
      r[j] = *reinterpret_cast<const floatx4*>(a.x + size_t(rr) * a.ldx + k);
    }
    if constexpr (NORM) {
      const uint32_t k = min(kbase + chunk * (XC * 32) + 4 * sq, a.K - 4);
      gr = *reinterpret_cast<const floatx4*>(a.norm + k);
    }
  };

  half8 wb[WIN][NW];
  floatx4 sxa[LDX], sxb[LDX], sga, sgb;  // staged chunks in flight (even, odd)
  stage_load(sxa, sga, 0);
  stage_load(sxb, sgb, 1);
#pragma unroll
  for (int i = 0; i < WIN; ++i) {
    const uint32_t t = min(uint32_t(i), last);
    wb[i][0] = bmm_wload(reinterpret_cast<const half8*>(wp0 + 512 * t));
    if constexpr (DUAL) wb[i][1] = bmm_wload(reinterpret_cast<const half8*>(wp1 + 512 * t));
  }
  // Per-(wave, column) power-of-two scale from the largest |x g| of the first
  // two chunks of this wave's range, as in bmm_kernel.  Staging lanes need it
  // for their rows 2 j + lane / 32, MFMA lanes for column n % 8.
  float cinv_s[LDX];
  float cmax_c = 0.0f;
  auto pow2_exp = [](float cm) __attribute__((always_inline)) {
    const int e = int((__float_as_uint(cm) >> 23) & 0xffu) - 127;
    return (cm >= 1.0e-30f && cm <= 1.0e30f) ? e : 0;
  };
#pragma unroll
  for (int j = 0; j < LDX; ++j) {
    floatx4 va = sxa[j], vb = sxb[j];
    if constexpr (NORM) {
      va = va * sga;
      vb = vb * sgb;
    }
    float m = fmaxf(fmaxf(fabsf(va.x), fabsf(va.y)), fmaxf(fabsf(va.z), fabsf(va.w)));
    m = fmaxf(m, fmaxf(fmaxf(fabsf(vb.x), fabsf(vb.y)), fmaxf(fabsf(vb.z), fabsf(vb.w))));
    const float rm = row_reduce(m, [](float a, float b) { return fmaxf(a, b); });
    const float lo = fmaxf(lane_read_f32(rm, 0), lane_read_f32(rm, 16));
    const float hi = fmaxf(lane_read_f32(rm, 32), lane_read_f32(rm, 48));
    cmax_c = (uint32_t(j) == (col >> 1)) ? ((col & 1u) ? hi : lo) : cmax_c;
    cinv_s[j] = __uint_as_float(uint32_t(127 - pow2_exp(srow ? hi : lo)) << 23);
  }
  const float cscale = __uint_as_float(uint32_t(127 + pow2_exp(cmax_c)) << 23);

  // split chunk `chunk` (registers r, gains gr) into LDS buffer buf: hi of
  // row j at fragment row j, lo at row j + 8; values of steps past this
  // wave's range are zero (their weight fragments re-read in-bounds data)
  auto stage_split = [&](const floatx4 (&r)[LDX], const floatx4& gr, uint32_t chunk, int buf)
                         __attribute__((always_inline)) {
    const uint32_t st = sq >> 3, off = 4 * (sq & 7u);
    const bool live = chunk * XC + st < KS;
    _Float16* dst = fsw + buf * CHH + st * PK_STEP + off;
    const floatx4 z4 = floatx4{};
#pragma unroll
    for (int j = 0; j < LDX; ++j) {
      const uint32_t row = 2 * j + srow;
      floatx4 v = live ? r[j] : z4;
      if constexpr (NORM) {
        qsw[buf * CHQ + st * PK_QSTEP + row * 8 + (sq & 7u)] = (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
        v = v * gr;
      }
      v = v * cinv_s[j];
      half4 h, l;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        h[e] = _Float16(v[e]);
        l[e] = _Float16((v[e] - float(h[e])) * 2048.0f);
      }
      *reinterpret_cast<half4*>(dst + row * PK_ROW) = h;
      *reinterpret_cast<half4*>(dst + (row + 8) * PK_ROW) = l;
    }
  };
  stage_split(sxa, sga, 0, 0);
  __builtin_amdgcn_sched_barrier(0);

  floatx4 acc[NW];
#pragma unroll
  for (int m = 0; m < NW; ++m) acc[m] = floatx4{};
  float ss = 0.0f;
  // the steps of chunk c from LDS buffer h (weight slots h XC .. h XC + 3);
  // each step's fragment is read one step ahead of its use
  auto chunk_steps = [&](uint32_t c, auto hc) __attribute__((always_inline)) {
    constexpr int h = decltype(hc)::value;
    const _Float16* fb = fsw + h * CHH + n * PK_ROW + 8 * grp;
    const float* qb = qsw + h * CHQ + col * 8 + 2 * grp;
    half8 cf = *reinterpret_cast<const half8*>(fb);
    float2 cq = make_float2(0.f, 0.f);
    if constexpr (NORM) cq = *reinterpret_cast<const float2*>(qb);
#pragma unroll
    for (int i = 0; i < XC; ++i) {
      const uint32_t s = c * XC + i;
      const int wi = h * XC + i;
      half8 nf = cf;
      float2 nq = cq;
      if (i + 1 < XC) {
        nf = *reinterpret_cast<const half8*>(fb + (i + 1) * PK_STEP);
        if constexpr (NORM) nq = *reinterpret_cast<const float2*>(qb + (i + 1) * PK_QSTEP);
      }
      if constexpr (NORM) {
        ss += cq.x;
        ss += cq.y;
      }
#pragma unroll
      for (int m = 0; m < NW; ++m) acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wb[wi][m], cf, acc[m], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      const uint32_t tw = min(s + WIN, last);
      wb[wi][0] = bmm_wload(reinterpret_cast<const half8*>(wp0 + 512 * tw));
      if constexpr (DUAL) wb[wi][1] = bmm_wload(reinterpret_cast<const half8*>(wp1 + 512 * tw));
      __builtin_amdgcn_sched_barrier(0);
      cf = nf;
      cq = nq;
    }
  };
  for (uint32_t sc = 0; sc < nsc; ++sc) {
    // chunk 2 sc from buffer 0: first the odd chunk (loaded one chunk ago)
    // into buffer 1, then the loads of chunk 2 sc + 2
    stage_split(sxb, sgb, 2 * sc + 1, 1);
    stage_load(sxa, sga, 2 * sc + 2);
    __builtin_amdgcn_sched_barrier(0);
    chunk_steps(2 * sc, std::integral_constant<int, 0>{});
    // chunk 2 sc + 1 from buffer 1
    stage_split(sxa, sga, 2 * sc + 2, 0);
    stage_load(sxb, sgb, 2 * sc + 3);
    __builtin_amdgcn_sched_barrier(0);
    chunk_steps(2 * sc + 1, std::integral_constant<int, 1>{});
  }
  // partials of wave w: slot m, lane l of its own staging region (lanes
  // n < 8: hi sums of column n, lanes n >= 8: lo sums of column n - 8)
  auto red = [&](uint32_t w, int slot) __attribute__((always_inline)) -> floatx4* {
    return reinterpret_cast<floatx4*>(&fs[w][0][0]) + slot * 64 + lane;
  };
#pragma unroll
  for (int m = 0; m < NW; ++m) *red(wave, m) = acc[m] * cscale;
  if constexpr (NORM) ssq[wave][lane] = ss;
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int m = 0; m < NW; ++m) {
    floatx4 t = *red(0, m);
#pragma unroll
    for (int w = 1; w < WAVES; ++w) t += *red(w, m);
    floatx4 tl;
#pragma unroll
    for (int v = 0; v < 4; ++v) tl[v] = __shfl_xor(t[v], 8, 64);
    acc[m] = t + tl * (1.0f / 2048.0f);
  }
  float r = 1.0f;
  if constexpr (NORM) {
    float t = ssq[0][lane];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) t += ssq[w][lane];
    // the four k groups of column n: lanes n, n + 16, n + 32, n + 48
    t = t + __shfl_xor(t, 16, 64);
    t = t + __shfl_xor(t, 32, 64);
    r = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(t, float(a.K)), a.eps)));
  }
  // a non-finite activation (or one beyond the split's range) leaves
  // non-finite sums
  bool bad = false;
#pragma unroll
  for (int m = 0; m < NW; ++m)
#pragma unroll
    for (int v = 0; v < 4; ++v) bad = bad || !(fabsf(acc[m][v]) <= 3.0e38f);
  bad = bad && n < a.N;
  if (__any(bad) && lane == 0 && a.err) atomicOr(a.err, ERR_F16_RANGE);
  const uint32_t done = a.done ? *a.done : 0u;
  if (done || n >= a.N) return;
  float* yrow = a.y + size_t(n) * a.ldy;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const uint32_t m = m0 + 4 * grp + v;
    if (m >= a.M) continue;
    const float g = acc[0][v] * r;
    if constexpr (EPI == EPI_STORE) {
      yrow[m] = g;
    } else if constexpr (EPI == EPI_RESID) {
      yrow[m] = __fadd_rn(yrow[m], g);
    } else {
      const float u = acc[NW - 1][v] * r;
      if constexpr (EPI == EPI_SWIGLU_SLOW) {
        const float sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf_glibc(-g)));
        yrow[m] = __fmul_rn(__fmul_rn(g, sig), u);
      } else {
        yrow[m] = __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, expf_glibc(-g))), u);
      }
    }
  }
}

template <int EPI, bool NORM>
hipError_t launch_bmm_pk(const BmmArgs& a, uint32_t waves, hipStream_t s) {
  const dim3 grid((a.M + 15) / 16);
  switch (waves) {
    case 1: hipLaunchKernelGGL((bmm_pk_kernel<EPI, NORM, 1>), grid, dim3(64), 0, s, a); break;
    case 2: hipLaunchKernelGGL((bmm_pk_kernel<EPI, NORM, 2>), grid, dim3(128), 0, s, a); break;
    case 4: hipLaunchKernelGGL((bmm_pk_kernel<EPI, NORM, 4>), grid, dim3(256), 0, s, a); break;
    case 8: hipLaunchKernelGGL((bmm_pk_kernel<EPI, NORM, 8>), grid, dim3(512), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int EPI, bool NORM, int NB>
hipError_t launch_bmm_waves(const BmmArgs& a, uint32_t waves, hipStream_t s) {
  const dim3 grid((a.M + 15) / 16);
  switch (waves) {
    case 1: hipLaunchKernelGGL((bmm_kernel<EPI, NORM, 1, NB>), grid, dim3(64), 0, s, a); break;
    case 2: hipLaunchKernelGGL((bmm_kernel<EPI, NORM, 2, NB>), grid, dim3(128), 0, s, a); break;
    case 4: hipLaunchKernelGGL((bmm_kernel<EPI, NORM, 4, NB>), grid, dim3(256), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int EPI>
hipError_t launch_bmm_epi(const BmmArgs& a, uint32_t waves, hipStream_t s) {
  const bool norm = a.norm != nullptr;
  if (a.N <= 8) return norm ? launch_bmm_pk<EPI, true>(a, waves, s) : launch_bmm_pk<EPI, false>(a, waves, s);
  return norm ? launch_bmm_waves<EPI, true, 16>(a, waves, s) : launch_bmm_waves<EPI, false, 16>(a, waves, s);
}

}  // namespace

uint32_t bmm_rows_pad(uint32_t m) { return (m + 15u) / 16u * 16u; }

hipError_t launch_tile_f16(const uint16_t* src, uint32_t K, uint32_t M, uint32_t row_base, uint32_t extra_row,
                           uint16_t* dst, hipStream_t s) {
  if (K % 32 || M == 0) return hipErrorInvalidValue;
  const uint32_t Mpad = bmm_rows_pad(M);
  const size_t chunks = size_t(Mpad / 16) * (K / 32) * 64;
  const uint32_t blocks = uint32_t(std::min<size_t>((chunks + 255) / 256, 8192));
  hipLaunchKernelGGL(tile_f16_kernel, dim3(blocks), dim3(256), 0, s, src, K, M, Mpad, row_base, extra_row, dst);
  return hipGetLastError();
}

uint32_t bmm_waves(uint32_t M, uint32_t K) {
  // the k range of each 16-row tile split over waves (summed in LDS): two
  // for tall matrices, four when there are few tiles.  One wave per tile is
  // fastest back to back (w13 at 8 columns: 24.5 vs 26.2 us), but right
  // after a heavy streaming kernel it measured 33.1 us against 27.4 us with
  // two, and inside the decode step two waves win (batch 8: +2.5 % frames/s)
  const uint32_t tiles = (M + 15) / 16, steps = K / 32;
  uint32_t w = tiles >= 512 ? 2u : 4u;
  while (steps % w) w /= 2;
  return w;
}

hipError_t launch_bmm(int epi, const BmmArgs& a, hipStream_t s) {
  if (a.N == 0 || a.N > 16 || a.M == 0 || a.K % 256 || !a.wt || !a.x) return hipErrorInvalidValue;
  const bool dual = epi == EPI_SWIGLU_SLOW || epi == EPI_SWIGLU_FAST;
  if (dual && !a.wt3) return hipErrorInvalidValue;
  const uint32_t waves = a.waves ? a.waves : bmm_waves(a.M, a.K);
  if ((a.K / 32) % waves) return hipErrorInvalidValue;
  switch (epi) {
    case EPI_STORE: return launch_bmm_epi<EPI_STORE>(a, waves, s);
    case EPI_RESID: return launch_bmm_epi<EPI_RESID>(a, waves, s);
    case EPI_SWIGLU_SLOW: return launch_bmm_epi<EPI_SWIGLU_SLOW>(a, waves, s);
    case EPI_SWIGLU_FAST: return launch_bmm_epi<EPI_SWIGLU_FAST>(a, waves, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace s2
