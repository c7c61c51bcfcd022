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

namespace s2 {
namespace {

constexpr int WAVE = 64;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
  for (int off = WAVE / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, WAVE);
  return v;
}
__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
  for (int off = WAVE / 2; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, WAVE));
  return v;
}

// ---------------------------------------------------------------------------
// Activation split: one block per row n < Npad.
//   xn = x[n] (or (x[n] * rms_scale) * g, the RMSNorm of the reference),
//   rs[n] = power of two with max|xn| / rs[n] in [2^13, 2^14),
//   xh[n] = f16(xn / rs), xl[n] = f16(xn / rs - xh);  rows N..Npad-1 are zero.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void split_rows_kernel(const float* x, uint32_t ldx, const float* norm, float eps,
                                                         uint32_t N, uint32_t K, _Float16* xh, _Float16* xl,
                                                         float* rs) {
  __shared__ float red[8];
  const uint32_t n = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
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
  float scale = 1.0f;
  if (norm) {
    float ss = 0.0f;
    for (uint32_t i = tid; i < K; i += 256) ss += xr[i] * xr[i];
    ss = wave_sum_f(ss);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    const float tot = (red[0] + red[1]) + (red[2] + red[3]);
    scale = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(tot, float(K)), eps)));
    __syncthreads();
  }
  float mx = 0.0f;
  for (uint32_t i = tid; i < K; i += 256) {
    float v = xr[i];
    if (norm) v = __fmul_rn(__fmul_rn(v, scale), norm[i]);
    mx = fmaxf(mx, fabsf(v));
  }
  mx = wave_max_f(mx);
  if (lane == 0) red[4 + wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[4], red[5]), fmaxf(red[6], red[7]));
  // power-of-two scale: exact to apply and to undo
  float r = 1.0f;
  if (mx > 0.0f && mx < 3.0e38f) {
    int e;
    (void)frexpf(mx, &e);  // mx in [2^(e-1), 2^e)
    r = ldexpf(1.0f, e - 14);
  }
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
//   block tile 64 (m) x 64 (n), 4 waves in 2 x 2, each one 32 x 32 MFMA tile;
//   K in stages of 32 staged through LDS (rows padded to 40 halfs so the
//   16-byte fragment reads of 8 consecutive lanes hit distinct banks); the
//   next stage's global loads are in flight while the current one computes.
// ---------------------------------------------------------------------------
constexpr int GM = 64, GN = 64, GK = 32, GKP = 40;

template <uint32_t WT, int EPI>
__global__ __launch_bounds__(256) void gemm_mfma_kernel(GemmArgs a) {
  constexpr bool DUAL = (EPI == EPI_SWIGLU_SLOW || EPI == EPI_SWIGLU_FAST);
  constexpr bool WSPLIT = WT != W_F16;
  constexpr int NW = DUAL ? 2 : 1;  // weight matrices
  __shared__ _Float16 ws[2][NW][WSPLIT ? 2 : 1][GM][GKP];
  __shared__ _Float16 xs[2][2][GN][GKP];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t wm = wave & 1u, wn = wave >> 1;
  const uint32_t m_blk = blockIdx.x * GM, n_blk = blockIdx.y * GN;

  // staging assignment: thread -> (row, 8-element part) of a 64 x 32 tile
  const uint32_t srow = tid >> 2, spart = (tid & 3u) * 8u;
  const uint32_t wrow = min(m_blk + srow, a.M - 1);
  const uint8_t* wp[NW];
  wp[0] = a.w + size_t(wrow) * a.row_bytes;
  if constexpr (DUAL) wp[NW - 1] = a.w3 + size_t(wrow) * a.row_bytes;
  const _Float16* xhp = a.xh + size_t(n_blk + srow) * a.K + spart;
  const _Float16* xlp = a.xl + size_t(n_blk + srow) * a.K + spart;

  half8 rw[NW][2], rxh, rxl;
  auto load_stage = [&](uint32_t k0) {
#pragma unroll
    for (int mtx = 0; mtx < NW; ++mtx) weight8<WT>(wp[mtx], k0 + spart, rw[mtx][0], rw[mtx][1]);
    rxh = *reinterpret_cast<const half8*>(xhp + k0);
    rxl = *reinterpret_cast<const half8*>(xlp + k0);
  };
  auto store_stage = [&](uint32_t buf) {
#pragma unroll
    for (int mtx = 0; mtx < NW; ++mtx) {
      *reinterpret_cast<half8*>(&ws[buf][mtx][0][srow][spart]) = rw[mtx][0];
      if constexpr (WSPLIT) *reinterpret_cast<half8*>(&ws[buf][mtx][WSPLIT ? 1 : 0][srow][spart]) = rw[mtx][1];
    }
    *reinterpret_cast<half8*>(&xs[buf][0][srow][spart]) = rxh;
    *reinterpret_cast<half8*>(&xs[buf][1][srow][spart]) = rxl;
  };

  floatx16 acc[NW], accl[NW];
#pragma unroll
  for (int mtx = 0; mtx < NW; ++mtx) {
    acc[mtx] = floatx16{};
    accl[mtx] = floatx16{};
  }
  const uint32_t fr = lane & 31u, fk = 8u * (lane >> 5);  // fragment row / k offset
  const uint32_t nst = a.K / GK;
  load_stage(0);
  store_stage(0);
  __syncthreads();
  for (uint32_t st = 0; st < nst; ++st) {
    const uint32_t buf = st & 1u;
    if (st + 1 < nst) load_stage((st + 1) * GK);
#pragma unroll
    for (uint32_t kk = 0; kk < GK; kk += 16) {
      const half8 bh = *reinterpret_cast<const half8*>(&xs[buf][0][32 * wn + fr][kk + fk]);
      const half8 bl = *reinterpret_cast<const half8*>(&xs[buf][1][32 * wn + fr][kk + fk]);
#pragma unroll
      for (int mtx = 0; mtx < NW; ++mtx) {
        const half8 ah = *reinterpret_cast<const half8*>(&ws[buf][mtx][0][32 * wm + fr][kk + fk]);
        acc[mtx] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bh, acc[mtx], 0, 0, 0);
        acc[mtx] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bl, acc[mtx], 0, 0, 0);
        if constexpr (WSPLIT) {
          const half8 al = *reinterpret_cast<const half8*>(&ws[buf][mtx][WSPLIT ? 1 : 0][32 * wm + fr][kk + fk]);
          accl[mtx] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, bh, accl[mtx], 0, 0, 0);
        }
      }
    }
    if (st + 1 < nst) {
      store_stage(buf ^ 1u);
      __syncthreads();
    }
  }

  // epilogue: lane holds D[8 (v/4) + 4 (lane/32) + v%4][lane%32]
  const uint32_t n = n_blk + 32 * wn + (lane & 31u);
  if (n >= a.N) return;
  const float r = a.rs[n];
  float* yrow = a.y + size_t(n) * a.ldy;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const uint32_t m = m_blk + 32 * wm + 8 * (v / 4) + 4 * (lane >> 5) + (v % 4);
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
// Causal GQA attention for a prompt chunk: query c (0 <= c < N) sits at
// position base + c and attends cache positions 0 .. base + c (its own K/V
// already appended).  Block (query tile of 8, kv head g): wave w serves q
// head g * rep + w; the 4 q heads share each 64-position K/V tile in LDS.
// Online softmax per query (running max and sum), f32 throughout.
// ---------------------------------------------------------------------------
constexpr int PQ = 8, PT = 64;

// Four f16 values (8 bytes) as a float4 (exact)
__device__ __forceinline__ float4 prefill_half4(const uint16_t* p) {
  const uint2 r = *reinterpret_cast<const uint2*>(p);
  const __half2 lo = *reinterpret_cast<const __half2*>(&r.x), hi = *reinterpret_cast<const __half2*>(&r.y);
  const float2 a = __half22float2(lo), b = __half22float2(hi);
  return make_float4(a.x, a.y, b.x, b.y);
}

template <int HD, bool KH>
__global__ __launch_bounds__(256) void attn_prefill_kernel(PrefillAttnArgs a) {
  using KT = std::conditional_t<KH, uint16_t, float>;  // cache element: f16 bits or f32
  __shared__ float kt[PT][HD + 1];
  __shared__ float vt[PT][HD];
  __shared__ float qs[4][PQ][HD];
  __shared__ float ps[4][PQ][PT];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t q0 = blockIdx.x * PQ, g = blockIdx.y;
  const uint32_t rep = a.H / a.Hkv;
  const uint32_t base = *a.pos_ptr + a.pos_offset;
  const uint32_t nq = min(uint32_t(PQ), a.N - q0);
  const bool active = wave < rep;
  const uint32_t h = g * rep + (active ? wave : 0u);
  // q rows of this wave's head
  for (uint32_t i = lane; i < PQ * HD; i += 64) {
    const uint32_t c = i / HD, d = i % HD;
    qs[wave][c][d] = (active && c < nq) ? a.q[size_t(q0 + c) * a.H * HD + size_t(h) * HD + d] : 0.0f;
  }
  float m[PQ], l[PQ], o[PQ][HD / 64];
#pragma unroll
  for (int c = 0; c < PQ; ++c) {
    m[c] = -INFINITY;
    l[c] = 0.0f;
#pragma unroll
    for (int j = 0; j < HD / 64; ++j) o[c][j] = 0.0f;
  }
  const uint32_t t_end = base + q0 + nq;  // keys needed by the last query
  const KT* kc = reinterpret_cast<const KT*>(a.k_cache) + size_t(g) * a.max_seq * HD;
  const KT* vc = reinterpret_cast<const KT*>(a.v_cache) + size_t(g) * a.max_seq * HD;
  for (uint32_t t0 = 0; t0 < t_end; t0 += PT) {
    __syncthreads();  // previous tile consumed (and qs written on the first pass)
    for (uint32_t i = tid; i < PT * HD / 4; i += 256) {
      const uint32_t t = i / (HD / 4), d = (i % (HD / 4)) * 4;
      float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), vv = kv;
      if (t0 + t < t_end) {
        if constexpr (KH) {
          kv = prefill_half4(kc + size_t(t0 + t) * HD + d);
          vv = prefill_half4(vc + size_t(t0 + t) * HD + d);
        } else {
          kv = *reinterpret_cast<const float4*>(kc + size_t(t0 + t) * HD + d);
          vv = *reinterpret_cast<const float4*>(vc + size_t(t0 + t) * HD + d);
        }
      }
      kt[t][d] = kv.x;
      kt[t][d + 1] = kv.y;
      kt[t][d + 2] = kv.z;
      kt[t][d + 3] = kv.w;
      *reinterpret_cast<float4*>(&vt[t][d]) = vv;
    }
    __syncthreads();
    if (active) {
      // scores: lane = key position within the tile
      const uint32_t t = t0 + lane;
      float s[PQ];
#pragma unroll
      for (int c = 0; c < PQ; ++c) s[c] = 0.0f;
      for (int d = 0; d < HD; ++d) {
        const float kd = kt[lane][d];
#pragma unroll
        for (int c = 0; c < PQ; ++c) s[c] = fmaf(qs[wave][c][d], kd, s[c]);
      }
#pragma unroll
      for (int c = 0; c < PQ; ++c) {
        const bool vis = uint32_t(c) < nq && t <= base + q0 + c;
        const float sc = vis ? s[c] * a.scale : -INFINITY;
        const float mt = wave_max_f(sc);
        const float mn = fmaxf(m[c], mt);
        const float p = vis ? expf(sc - mn) : 0.0f;
        const float corr = (m[c] == -INFINITY) ? 0.0f : expf(m[c] - mn);
        l[c] = l[c] * corr + wave_sum_f(p);
#pragma unroll
        for (int j = 0; j < HD / 64; ++j) o[c][j] *= corr;
        m[c] = (mn == -INFINITY) ? m[c] : mn;
        ps[wave][c][lane] = p;
      }
    }
    __syncthreads();
    if (active) {
      // PV: lane = head-dim element
      for (int t = 0; t < PT; ++t) {
        float vd[HD / 64];
#pragma unroll
        for (int j = 0; j < HD / 64; ++j) vd[j] = vt[t][lane + 64 * j];
#pragma unroll
        for (int c = 0; c < PQ; ++c) {
          const float p = ps[wave][c][t];
#pragma unroll
          for (int j = 0; j < HD / 64; ++j) o[c][j] = fmaf(p, vd[j], o[c][j]);
        }
      }
    }
  }
  if (!active) return;
#pragma unroll
  for (int c = 0; c < PQ; ++c) {
    if (uint32_t(c) >= nq) continue;
    float* dst = a.out + size_t(q0 + c) * a.H * HD + size_t(h) * HD;
    const float inv = 1.0f / l[c];
#pragma unroll
    for (int j = 0; j < HD / 64; ++j) dst[lane + 64 * j] = o[c][j] * inv;
  }
}

}  // namespace

hipError_t launch_split_rows(const float* x, uint32_t ldx, const float* norm, float eps, uint32_t N, uint32_t Npad,
                             uint32_t K, _Float16* xh, _Float16* xl, float* rs, hipStream_t s) {
  if (Npad < N || Npad % 16 || K % GK) return hipErrorInvalidValue;
  hipLaunchKernelGGL(split_rows_kernel, dim3(Npad), dim3(256), 0, s, x, ldx, norm, eps, N, K, xh, xl, rs);
  return hipGetLastError();
}

template <uint32_t WT>
static hipError_t gemm_epi(int epi, const GemmArgs& a, dim3 grid, hipStream_t s) {
  switch (epi) {
    case EPI_STORE: hipLaunchKernelGGL((gemm_mfma_kernel<WT, EPI_STORE>), grid, dim3(256), 0, s, a); break;
    case EPI_RESID: hipLaunchKernelGGL((gemm_mfma_kernel<WT, EPI_RESID>), grid, dim3(256), 0, s, a); break;
    case EPI_SWIGLU_SLOW:
      hipLaunchKernelGGL((gemm_mfma_kernel<WT, EPI_SWIGLU_SLOW>), grid, dim3(256), 0, s, a);
      break;
    case EPI_SWIGLU_FAST:
      hipLaunchKernelGGL((gemm_mfma_kernel<WT, EPI_SWIGLU_FAST>), grid, dim3(256), 0, s, a);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

uint32_t gemm_rows_pad(uint32_t n) { return (n + GN - 1) / GN * GN; }

hipError_t launch_gemm_mfma(uint32_t wtype, int epi, const GemmArgs& a, hipStream_t s) {
  if (a.K % GK || a.M == 0 || a.N == 0) return hipErrorInvalidValue;
  const bool dual = epi == EPI_SWIGLU_SLOW || epi == EPI_SWIGLU_FAST;
  if (dual && !a.w3) return hipErrorInvalidValue;
  const dim3 grid((a.M + GM - 1) / GM, gemm_rows_pad(a.N) / GN);
  switch (wtype) {
    case W_F16: return gemm_epi<W_F16>(epi, a, grid, s);
    case W_Q8_0: return gemm_epi<W_Q8_0>(epi, a, grid, s);
    case W_Q4_0: return gemm_epi<W_Q4_0>(epi, a, grid, s);
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

hipError_t launch_attention_prefill(const PrefillAttnArgs& a, hipStream_t s) {
  if (!a.pos_ptr || a.H % a.Hkv || a.H / a.Hkv > 4 || a.N == 0) return hipErrorInvalidValue;
  const dim3 grid((a.N + PQ - 1) / PQ, a.Hkv);
  switch (a.hd) {
    case 64:
      hipLaunchKernelGGL((a.kv_f16 ? attn_prefill_kernel<64, true> : attn_prefill_kernel<64, false>), grid, dim3(256),
                         0, s, a);
      break;
    case 128:
      hipLaunchKernelGGL((a.kv_f16 ? attn_prefill_kernel<128, true> : attn_prefill_kernel<128, false>), grid,
                         dim3(256), 0, s, a);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace s2
