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
// Activations stay f32 rows; each lane splits its own 8 elements per step
// into f16 hi = f16(x) and lo = f16((x - hi) 2^11), kept normal down to
// |x| ~ 2^-14 by the 2^11 (x = hi + 2^-11 lo to ~2^-22 |x|, absolute ~2^-35
// below); hi and lo go through the MFMA with the same weight fragment into
// two accumulators, combined as acc_hi + 2^-11 acc_lo.  A value outside the f16 range turns its column's results
// non-finite; the epilogue then sets ERR_F16_RANGE, so the call fails
// instead of returning a wrong product.  RMSNorm inputs: the sum of squares of
// each column is accumulated from the same loaded values and the RMS scale
// is applied to the result (W.((x s) g) = s W.(x g)).
#include <hip/hip_runtime.h>
#include <math.h>

#include <algorithm>

#include "kernels.h"

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
constexpr int WIN = 8, XW = 4;

__device__ __forceinline__ void split8(const float4& a, const float4& b, half8& hi, half8& lo) {
  const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const _Float16 h = _Float16(v[e]);
    hi[e] = h;
    lo[e] = _Float16((v[e] - float(h)) * 2048.0f);
  }
}

template <int EPI, bool NORM, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void bmm_kernel(BmmArgs a) {
  constexpr bool DUAL = (EPI == EPI_SWIGLU_SLOW || EPI == EPI_SWIGLU_FAST);
  constexpr int NW = DUAL ? 2 : 1;
  __shared__ floatx4 red[WAVES][2 * NW][64];
  __shared__ float ssq[WAVES][64];
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t tm = blockIdx.x, m0 = tm * 16;
  const uint32_t kt = a.K / 32, KS = kt / WAVES;
  const uint32_t n = lane & 15u, grp = lane >> 4;
  const size_t tile0 = (size_t(tm) * kt + size_t(wave) * KS) * 512 + size_t(lane) * 8;
  const _Float16* wp0 = a.wt + tile0;
  const _Float16* wp1 = DUAL ? a.wt3 + tile0 : wp0;
  const bool xon = n < a.N;
  const uint32_t kbeg = wave * KS * 32 + 8 * grp;
  const float* xp = a.x + size_t(xon ? n : 0u) * a.ldx + kbeg;
  const float* gp = NORM ? a.norm + kbeg : nullptr;
  // The loop body has no branches (a branch around a load makes the compiler
  // wait for every outstanding load at the join): steps run to a multiple of
  // WIN, loads past the last step re-read it (in bounds), and the activation
  // of a step past the end, or of a column >= N, is zeroed by a select.
  const uint32_t last = KS - 1;
  const uint32_t KSR = (KS + WIN - 1) / WIN * WIN;

  // loads complete in issue order for the wait counter: activations (short
  // L2 latency) go out before the weights of the same step, so waiting for
  // a step's activations does not wait for the deeper weight prefetch
  half8 wb[WIN][NW];
  float4 xv[XW][2], gv[XW][2];
#pragma unroll
  for (int i = 0; i < XW; ++i) {
    const uint32_t t = min(uint32_t(i), last);
    xv[i][0] = *reinterpret_cast<const float4*>(xp + 32 * t);
    xv[i][1] = *reinterpret_cast<const float4*>(xp + 32 * t + 4);
    if constexpr (NORM) {
      gv[i][0] = *reinterpret_cast<const float4*>(gp + 32 * t);
      gv[i][1] = *reinterpret_cast<const float4*>(gp + 32 * t + 4);
    }
  }
#pragma unroll
  for (int i = 0; i < WIN; ++i) {
    const uint32_t t = min(uint32_t(i), last);
    wb[i][0] = *reinterpret_cast<const half8*>(wp0 + 512 * t);
    if constexpr (DUAL) wb[i][1] = *reinterpret_cast<const half8*>(wp1 + 512 * t);
  }
  __builtin_amdgcn_sched_barrier(0);
  floatx4 acc[NW], accl[NW];
#pragma unroll
  for (int m = 0; m < NW; ++m) {
    acc[m] = floatx4{};
    accl[m] = floatx4{};
  }
  float ss = 0.0f;
  const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
  for (uint32_t base = 0; base < KSR; base += WIN) {
#pragma unroll
    for (int i = 0; i < WIN; ++i) {
      const uint32_t s = base + i;
      const int xi = i % XW;  // base is a multiple of WIN, WIN of XW
      const bool live = xon && s < KS;
      float4 x0 = live ? xv[xi][0] : z4, x1 = live ? xv[xi][1] : z4;
      if constexpr (NORM) {
        ss += (x0.x * x0.x + x0.y * x0.y) + (x0.z * x0.z + x0.w * x0.w);
        ss += (x1.x * x1.x + x1.y * x1.y) + (x1.z * x1.z + x1.w * x1.w);
        const float4 g0 = gv[xi][0], g1 = gv[xi][1];
        x0 = make_float4(x0.x * g0.x, x0.y * g0.y, x0.z * g0.z, x0.w * g0.w);
        x1 = make_float4(x1.x * g1.x, x1.y * g1.y, x1.z * g1.z, x1.w * g1.w);
      }
      half8 bh, bl;
      split8(x0, x1, bh, bl);
#pragma unroll
      for (int m = 0; m < NW; ++m) {
        acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wb[i][m], bh, acc[m], 0, 0, 0);
        accl[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wb[i][m], bl, accl[m], 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      const uint32_t tw = min(s + WIN, last), tx = min(s + XW, last);
      xv[xi][0] = *reinterpret_cast<const float4*>(xp + 32 * tx);
      xv[xi][1] = *reinterpret_cast<const float4*>(xp + 32 * tx + 4);
      if constexpr (NORM) {
        gv[xi][0] = *reinterpret_cast<const float4*>(gp + 32 * tx);
        gv[xi][1] = *reinterpret_cast<const float4*>(gp + 32 * tx + 4);
      }
      wb[i][0] = *reinterpret_cast<const half8*>(wp0 + 512 * tw);
      if constexpr (DUAL) wb[i][1] = *reinterpret_cast<const half8*>(wp1 + 512 * tw);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int m = 0; m < NW; ++m) {
    red[wave][2 * m][lane] = acc[m];
    red[wave][2 * m + 1][lane] = accl[m];
  }
  if constexpr (NORM) ssq[wave][lane] = ss;
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int m = 0; m < NW; ++m) {
    floatx4 t = red[0][2 * m][lane], tl = red[0][2 * m + 1][lane];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) {
      t += red[w][2 * m][lane];
      tl += red[w][2 * m + 1][lane];
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
  // an activation beyond the f16 range (or NaN) leaves non-finite sums
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
        const float sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-g)));
        yrow[m] = __fmul_rn(__fmul_rn(g, sig), u);
      } else {
        yrow[m] = __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, expf(-g))), u);
      }
    }
  }
}

template <int EPI, bool NORM>
hipError_t launch_bmm_waves(const BmmArgs& a, uint32_t waves, hipStream_t s) {
  const dim3 grid((a.M + 15) / 16);
  switch (waves) {
    case 1: hipLaunchKernelGGL((bmm_kernel<EPI, NORM, 1>), grid, dim3(64), 0, s, a); break;
    case 2: hipLaunchKernelGGL((bmm_kernel<EPI, NORM, 2>), grid, dim3(128), 0, s, a); break;
    case 4: hipLaunchKernelGGL((bmm_kernel<EPI, NORM, 4>), grid, dim3(256), 0, s, a); break;
    case 8: hipLaunchKernelGGL((bmm_kernel<EPI, NORM, 8>), grid, dim3(512), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
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
  // enough blocks x waves to cover the CUs several times over: one wave per
  // 16-row tile for tall matrices, the k range split over more waves (and
  // summed in LDS) when there are few tiles
  const uint32_t tiles = (M + 15) / 16, steps = K / 32;
  uint32_t w = 1;
  while (w < 8 && tiles * w < 2048 && steps % (2 * w) == 0 && steps / (2 * w) >= 8) w *= 2;
  return w;
}

hipError_t launch_bmm(int epi, const BmmArgs& a, hipStream_t s) {
  if (a.N == 0 || a.N > 16 || a.M == 0 || a.K % 256 || !a.wt) return hipErrorInvalidValue;
  const bool dual = epi == EPI_SWIGLU_SLOW || epi == EPI_SWIGLU_FAST;
  if (dual && !a.wt3) return hipErrorInvalidValue;
  const uint32_t waves = a.waves ? a.waves : bmm_waves(a.M, a.K);
  if ((a.K / 32) % waves) return hipErrorInvalidValue;
  const bool norm = a.norm != nullptr;
  switch (epi) {
    case EPI_STORE: return norm ? launch_bmm_waves<EPI_STORE, true>(a, waves, s)
                                : launch_bmm_waves<EPI_STORE, false>(a, waves, s);
    case EPI_RESID: return norm ? launch_bmm_waves<EPI_RESID, true>(a, waves, s)
                                : launch_bmm_waves<EPI_RESID, false>(a, waves, s);
    case EPI_SWIGLU_SLOW: return norm ? launch_bmm_waves<EPI_SWIGLU_SLOW, true>(a, waves, s)
                                      : launch_bmm_waves<EPI_SWIGLU_SLOW, false>(a, waves, s);
    case EPI_SWIGLU_FAST: return norm ? launch_bmm_waves<EPI_SWIGLU_FAST, true>(a, waves, s)
                                      : launch_bmm_waves<EPI_SWIGLU_FAST, false>(a, waves, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace s2
