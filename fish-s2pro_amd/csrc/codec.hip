// codec.hip -- HIP kernels of the RVQ codec decode (crates/fish_s2_infer/src/codec.rs:1690-1714).
//
// The decoder's convolutions (causal conv1d, transposed conv1d, pointwise
// linears) all run on one implicit-GEMM MFMA kernel, conv_gemm_kernel:
//   * block tile: 256 frames x TM = 32 * MC output channels, 4 waves each
//     holding 64 frames x TM channels (2 x MC tiles of v_mfma_f32_32x32x16_f16,
//     frames as the A operand, weights as B, so the 32 lanes of a row group
//     store 32 consecutive channels of one frame);
//   * K runs over input-channel stages of KC (16 or 32) channels; a stage
//     holds the stage's A window -- the tile's 256 frames plus the halo the
//     taps reach back, loaded once and read by every tap at its own row
//     offset -- and the weights of all G taps for those channels;
//   * two LDS buffers: the next stage's global loads are in registers while a
//     stage computes, written to the other buffer after it, one barrier per
//     stage;
//   * tiles of one weight tile (m tile) are dealt to the same XCD, so that
//     XCD's L2 serves its weights to all of its frame tiles.
// Small per-frame kernels handle the rest: RVQ lookup, RoPE, the windowed
// attention of the post-module transformer, depthwise conv + LayerNorm, the
// output conv + tanh.

#include <algorithm>

#include "codec.h"
#include "expf_glibc.h"
#include "wave.h"
#include "sin_cw.h"

namespace s2 {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr uint32_t CG_TF = 256;    // frames per block tile
constexpr uint32_t CG_MAXLD = 10;  // 16-byte staging loads per thread per stage
constexpr size_t CG_FMAJOR_WEIGHT_BYTES = size_t(3) << 19;  // 1.5 MiB of a 4 MiB XCD L2

// LDS rows are KC halfs (CH = KC / 8 chunks of 16 bytes), chunk c of row r
// stored at c ^ swz(r).  Weight rows are read 32 at a time from a multiple
// of 32; A window rows from any offset (the tap's shift), so their swizzle
// only needs 8 consecutive rows on distinct banks.
template <uint32_t CH>
__device__ __forceinline__ uint32_t swz_a(uint32_t r) {
  return CH == 2 ? ((r >> 2) & 1u) : (((r >> 1) ^ (r >> 3)) & 3u);
}
template <uint32_t CH>
__device__ __forceinline__ uint32_t swz_w(uint32_t r) {
  return CH == 2 ? (((r >> 2) ^ (r >> 3)) & 1u) : (((r >> 1) ^ (r >> 3)) & 3u);
}

// erf_approx and gelu_erf (codec.rs:3886-3899), the reference's operation order.
__device__ __forceinline__ float erf_as(float value) {
  const float sign = value < 0.0f ? -1.0f : 1.0f;
  const float x = fabsf(value);
  const float t = __fdiv_rn(1.0f, __fadd_rn(1.0f, __fmul_rn(0.3275911f, x)));
  float p = __fsub_rn(__fmul_rn(1.0614054f, t), 1.4531521f);
  p = __fadd_rn(__fmul_rn(p, t), 1.4214138f);
  p = __fsub_rn(__fmul_rn(p, t), 0.28449672f);
  p = __fadd_rn(__fmul_rn(p, t), 0.2548296f);
  p = __fmul_rn(p, t);
  return __fmul_rn(sign, __fsub_rn(1.0f, __fmul_rn(p, expf_glibc(__fmul_rn(-x, x)))));
}
__device__ __forceinline__ float gelu_as(float v) {
  return __fmul_rn(__fmul_rn(0.5f, v), __fadd_rn(1.0f, erf_as(__fmul_rn(v, 0.70710677f))));
}
// snake_activation_frame_major (codec.rs:2162-2186), sin^2 from sin_cw.h
__device__ __forceinline__ float snake(float x, float alpha) { return snake_cw(x, alpha); }

template <int MC, int KC, int PL, bool FU = false>
__global__ __launch_bounds__(256, 2) void conv_gemm_kernel(ConvGemmArgs a, uint32_t m_tiles, uint32_t f_tiles,
                                                           uint32_t halo, int32_t wbase, int32_t toff0,
                                                           int32_t tstep, uint32_t fmajor) {
  constexpr uint32_t TM = 32 * MC, CH = KC / 8;
  extern __shared__ __align__(16) _Float16 cg_lds[];
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  // Workgroup b runs on XCD b % 8; tiles are dealt to XCDs in contiguous
  // ranges (XCD-major), in one of two orders.
  //   fmajor: over all phases, t = (ft * phases + phase) * m_tiles + mt, so
  //     the blocks that read one frame tile's input window (every phase and
  //     weight tile) run one after another on one XCD: the window comes from
  //     HBM once and from that XCD's L2 after, while the weights of every
  //     (phase, m tile), small enough, stay in each L2.
  //   otherwise: phase by phase (phase = b / (m_tiles f_tiles)), and within
  //     a phase t = mt * f_tiles + ft: an XCD works through one weight tile at
  //     a time, which its L2 serves to all of that XCD's frame tiles.
  const uint32_t nb1 = m_tiles * f_tiles;
  uint32_t b = blockIdx.x, nb = gridDim.x, phase = 0, phases = nb / nb1;
  if (!fmajor) {
    phase = b / nb1;
    b -= phase * nb1;
    nb = nb1;
  }
  const uint32_t xcd = b & 7u, slot = b >> 3, q8 = nb >> 3, r8 = nb & 7u;
  const uint32_t t = xcd < r8 ? xcd * (q8 + 1u) + slot : r8 * (q8 + 1u) + (xcd - r8) * q8 + slot;
  uint32_t mt, ft;
  if (fmajor) {
    mt = t % m_tiles;
    const uint32_t tr = t / m_tiles;
    phase = tr % phases;
    ft = tr / phases;
  } else {
    mt = t / f_tiles;
    ft = t - mt * f_tiles;
  }
  // (the divisions above are expanded on the vector unit: move the results
  // to scalar registers, where they cost no vector registers in the loop)
  mt = uint32_t(__builtin_amdgcn_readfirstlane(int(mt)));
  ft = uint32_t(__builtin_amdgcn_readfirstlane(int(ft)));
  phase = uint32_t(__builtin_amdgcn_readfirstlane(int(phase)));
  const uint32_t f0 = ft * CG_TF;
  const uint32_t AR = CG_TF + halo;
  const uint32_t a_chunks = PL * AR * CH, w_chunks = a.G * TM * CH, tot = a_chunks + w_chunks;
  const uint32_t buf_halfs = (PL * AR + a.G * TM) * KC;
  const uint32_t nst_all = a.C / KC, splits = gridDim.z, sp = blockIdx.z;
  const uint32_t st_begin = nst_all * sp / splits, nst = nst_all * (sp + 1) / splits - st_begin;
  const _Float16* wsrc = a.w + (size_t(phase) * m_tiles + mt) * (size_t(a.G) * TM * a.C);
  const int32_t row0 = int32_t(f0) + wbase;

  // Per staging slot i (chunk tid + 256 i of a stage): the element offset of
  // its 16 bytes at stage 0 and its LDS offset, with the source in bits
  // 30..31 (0: A hi plane, 1: A lo plane, 2: weights, 3: zero / no chunk).
  // Stage st adds st * KC (A) or st * G * TM * KC (weights) to the offset.
  uint32_t goff[CG_MAXLD], loff[CG_MAXLD];
#pragma unroll
  for (uint32_t i = 0; i < CG_MAXLD; ++i) {
    const uint32_t qd = tid + 256u * i;
    uint32_t kind = 3u, g = 0u, l = 0u;
    if (qd < a_chunks) {
      const uint32_t pl = PL == 2 ? qd / (AR * CH) : 0u, rem = qd - pl * (AR * CH);
      const uint32_t row = rem / CH, c = rem - row * CH;
      const int32_t src = row0 + int32_t(row);
      l = (pl * AR + row) * KC + ((c ^ swz_a<CH>(row)) << 3);
      if (src >= 0 && src < int32_t(a.F)) {
        kind = pl;
        g = uint32_t(src) * a.ldx + c * 8u;
      }
    } else if (qd < tot) {
      const uint32_t wq = qd - a_chunks, row = wq / CH, c = wq - row * CH;
      l = PL * AR * KC + row * KC + ((c ^ swz_w<CH>(row)) << 3);
      kind = 2u;
      g = wq * 8u;
    } else {
      l = 0xffffffffu >> 2;  // no chunk: nothing stored
    }
    goff[i] = g;
    loff[i] = l | (kind << 30);
  }
  const uint32_t wstage = a.G * TM * KC;

  uint4 stg[CG_MAXLD];
  auto load = [&](uint32_t st) {
#pragma unroll
    for (uint32_t i = 0; i < CG_MAXLD; ++i) {
      const uint32_t kind = loff[i] >> 30;
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      if (kind == 2u) {
        v = *reinterpret_cast<const uint4*>(wsrc + size_t(st_begin + st) * wstage + goff[i]);
      } else if (kind < 2u) {
        const _Float16* base = kind ? a.xl : a.xh;
        v = *reinterpret_cast<const uint4*>(base + size_t(goff[i]) + (st_begin + st) * KC);
      }
      stg[i] = v;
    }
  };
  auto store = [&](uint32_t bsel) {
    _Float16* B = cg_lds + bsel * buf_halfs;
#pragma unroll
    for (uint32_t i = 0; i < CG_MAXLD; ++i) {
      const uint32_t l = loff[i] & 0x3fffffffu;
      if (l != (0xffffffffu >> 2)) *reinterpret_cast<uint4*>(B + l) = stg[i];
    }
  };

  floatx16 acc[2][MC];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < MC; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  auto compute = [&](uint32_t bsel) {
    const _Float16* A = cg_lds + bsel * buf_halfs;
    const _Float16* W = A + PL * AR * KC;
    for (uint32_t g = 0; g < a.G; ++g) {
      const uint32_t toff = uint32_t(toff0 + int32_t(g) * tstep);
#pragma unroll
      for (uint32_t kk = 0; kk < uint32_t(KC / 16); ++kk) {
        const uint32_t c = kk * 2u + (lane >> 5);
        half8 bf[MC];
#pragma unroll
        for (int j = 0; j < MC; ++j) {
          const uint32_t row = g * TM + uint32_t(j) * 32u + (lane & 31u);
          bf[j] = *reinterpret_cast<const half8*>(W + row * KC + ((c ^ swz_w<CH>(row)) << 3));
        }
#pragma unroll
        for (int p = 0; p < PL; ++p) {
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            const uint32_t row = wave * 64u + uint32_t(i) * 32u + (lane & 31u) + toff;
            const half8 af =
                *reinterpret_cast<const half8*>(A + (uint32_t(p) * AR + row) * KC + ((c ^ swz_a<CH>(row)) << 3));
#pragma unroll
            for (int j = 0; j < MC; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf[j], acc[i][j], 0, 0, 0);
          }
        }
      }
    }
  };

  load(0);
  store(0);
  __syncthreads();
  if (nst > 1) load(1);
  for (uint32_t st = 0; st < nst; ++st) {
    compute(st & 1u);
    if (st + 1 < nst) store((st + 1) & 1u);
    __syncthreads();
    if (st + 2 < nst) load(st + 2);
  }

  if constexpr (FU) {
    // The residual unit's k1 conv on the tile just computed (all M channels):
    // Y = f16(snake(acc + bias_mid, alpha_mid)) in LDS ([256 frames][TM + 8]
    // halfs: 16 consecutive rows fall on distinct 16-byte bank groups), the
    // k1 weights W1 ([TM / 32 stages][TM rows][32], swizzled like W) next to
    // it; every wave left the stage buffers at the loop's last barrier.
    constexpr uint32_t YS = TM + 8;
    _Float16* Y = cg_lds;
    _Float16* W1 = cg_lds + CG_TF * YS;
    for (uint32_t q = tid; q < TM * TM / 8u; q += 256u) {
      const uint32_t st = q / (TM * 4u), rem = q - st * (TM * 4u), row = rem >> 2, c = rem & 3u;
      *reinterpret_cast<uint4*>(W1 + st * (TM * 32u) + row * 32u + ((c ^ swz_w<4>(row)) << 3)) =
          *reinterpret_cast<const uint4*>(a.w1 + size_t(q) * 8u);
    }
#pragma unroll
    for (int j = 0; j < MC; ++j) {
      const uint32_t m = uint32_t(j) * 32u + (lane & 31u);
      const float bm = m < a.M ? a.bias_mid[m] : 0.0f;
      const float am = m < a.M ? a.alpha_mid[m] : 1.0f;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const uint32_t fl = wave * 64u + uint32_t(i) * 32u + 4u * (lane >> 5);
#pragma nounroll
        for (int v = 0; v < 16; ++v) {
          const float val = snake(__fadd_rn(acc[i][j][v], bm), am);
          Y[(fl + 8u * uint32_t(v >> 2) + uint32_t(v & 3)) * YS + m] = _Float16(val);
          acc[i][j][v] = 0.0f;
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (uint32_t kk = 0; kk < TM / 16u; ++kk) {
      const uint32_t c = kk * 2u + (lane >> 5);                  // chunk of the Y row
      const uint32_t st = kk >> 1, cs = (kk & 1u) * 2u + (lane >> 5);  // W1 stage, chunk in it
      half8 bf[MC];
#pragma unroll
      for (int j = 0; j < MC; ++j) {
        const uint32_t row = uint32_t(j) * 32u + (lane & 31u);
        bf[j] = *reinterpret_cast<const half8*>(W1 + st * (TM * 32u) + row * 32u + ((cs ^ swz_w<4>(row)) << 3));
      }
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const half8 af = *reinterpret_cast<const half8*>(Y + (wave * 64u + uint32_t(i) * 32u + (lane & 31u)) * YS + c * 8u);
#pragma unroll
        for (int j = 0; j < MC; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf[j], acc[i][j], 0, 0, 0);
      }
    }
  }

  if (splits > 1) {  // partial sums; conv_split_reduce_kernel finishes
    const size_t rows = size_t(a.F) * a.ostride;
#pragma unroll
    for (int j = 0; j < MC; ++j) {
      const uint32_t m = mt * TM + uint32_t(j) * 32u + (lane & 31u);
      if (m >= a.M) continue;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const uint32_t fb = f0 + wave * 64u + uint32_t(i) * 32u + 4u * (lane >> 5);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const uint32_t f = fb + 8u * uint32_t(v >> 2) + uint32_t(v & 3);
          if (f < a.F) a.part[(size_t(sp) * rows + size_t(f) * a.ostride + phase) * a.M + m] = acc[i][j][v];
        }
      }
    }
    return;
  }
  // epilogue: acc[i][j][v] = D[frame 8 (v/4) + 4 (lane/32) + v%4][channel lane%32].
  // The residual values of a fragment are loaded together before its stores
  // (res may be the output buffer itself, so loads cannot move past stores).
#pragma unroll
  for (int j = 0; j < MC; ++j) {
    const uint32_t m = mt * TM + uint32_t(j) * 32u + (lane & 31u);
    if (m >= a.M) continue;
    const float bias = a.bias[m];
    const float gam = a.gamma ? a.gamma[m] : 1.0f;
    const float alp = a.alpha ? a.alpha[m] : 1.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t fb = f0 + wave * 64u + uint32_t(i) * 32u + 4u * (lane >> 5);
      float rv[16];
      if (a.res) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const uint32_t f = fb + 8u * uint32_t(v >> 2) + uint32_t(v & 3);
          rv[v] = f < a.F ? a.res[(size_t(f) * a.ostride + phase) * a.ldres + m] : 0.0f;
        }
      }
      // not unrolled: 2 x MC x 16 inlined snake evaluations in one block spill
#pragma nounroll
      for (int v = 0; v < 16; ++v) {
        const uint32_t f = fb + 8u * uint32_t(v >> 2) + uint32_t(v & 3);
        if (f >= a.F) continue;
        const size_t row = size_t(f) * a.ostride + phase;
        float val = __fadd_rn(acc[i][j][v], bias);
        if (a.gelu) val = gelu_as(val);
        if (a.gamma) val = __fmul_rn(val, gam);
        if (a.res) val = __fadd_rn(rv[v], val);
        if (a.y32) a.y32[row * a.ldy + m] = val;
        if (a.alpha) val = snake(val, alp);
        if (a.yh) {
          const _Float16 h = _Float16(val);
          a.yh[row * a.ldh + m] = h;
          if (a.yl) a.yl[row * a.ldh + m] = _Float16(__fsub_rn(val, float(h)));
        }
      }
    }
  }
}

// Sum of the K splits (in split order) and the conv epilogue, one thread per
// output element (row, m), rows = F * ostride.
__global__ __launch_bounds__(256) void conv_split_reduce_kernel(ConvGemmArgs a, uint32_t splits) {
  const size_t rows = size_t(a.F) * a.ostride;
  const size_t idx = size_t(blockIdx.x) * 256u + threadIdx.x;
  if (idx >= rows * a.M) return;
  const size_t row = idx / a.M;
  const uint32_t m = uint32_t(idx - row * a.M);
  float acc = a.part[idx];
  for (uint32_t z = 1; z < splits; ++z) acc = __fadd_rn(acc, a.part[size_t(z) * rows * a.M + idx]);
  float val = __fadd_rn(acc, a.bias[m]);
  if (a.gelu) val = gelu_as(val);
  if (a.gamma) val = __fmul_rn(val, a.gamma[m]);
  if (a.res) val = __fadd_rn(a.res[row * a.ldres + m], val);
  if (a.y32) a.y32[row * a.ldy + m] = val;
  if (a.alpha) val = snake(val, a.alpha[m]);
  if (a.yh) {
    const _Float16 h = _Float16(val);
    a.yh[row * a.ldh + m] = h;
    if (a.yl) a.yl[row * a.ldh + m] = _Float16(__fsub_rn(val, float(h)));
  }
}

// rvq_lookup_codes (codec.rs:2536-2596): one block per frame, 4 outputs per
// thread; every sum in the reference's order (bit-exact).
__global__ __launch_bounds__(256) void codec_rvq_kernel(RvqArgs a) {
  const uint32_t f = blockIdx.x;
#pragma unroll
  for (uint32_t k = 0; k < 4; ++k) {
    const uint32_t o = threadIdx.x + 256u * k;
    float acc = 0.0f;
    for (uint32_t q = 0; q < 10; ++q) {
      int32_t code = a.codes[size_t(q) * a.F + f];
      if (code < 0 || uint32_t(code) >= a.cb_size[q]) {
        if (a.err) *a.err = 1u;
        code = 0;
      }
      const float* z = a.cb[q] + size_t(code) * 8u;
      const float* w = a.pw[q] + size_t(o) * 8u;
      float d = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) d = __fadd_rn(d, __fmul_rn(z[j], w[j]));
      acc = __fadd_rn(acc, __fadd_rn(d, a.pb[q][o]));
    }
    a.out[size_t(f) * 1024u + o] = acc;
  }
}

__global__ __launch_bounds__(256) void codec_check_codes_kernel(const int32_t* codes, uint32_t F, uint32_t* err) {
  const size_t i = size_t(blockIdx.x) * 256u + threadIdx.x;
  if (i >= size_t(10) * F) return;
  const int32_t c = codes[i];
  const int32_t size = i < F ? 4096 : 1024;
  if (c < 0 || c >= size) *err = 1u;
}

// apply_rope_normal (attention.rs:172-206) on q and k of one frame: pairs
// (x0, x1) -> (x0 c - x1 s, x0 s + x1 c) with the table's (cos, sin).
__global__ __launch_bounds__(256) void codec_rope_kernel(float* qkv, const float2* table) {
  const uint32_t t = blockIdx.x;
  float* row = qkv + size_t(t) * 3072u;
#pragma unroll
  for (uint32_t k = 0; k < 4; ++k) {
    const uint32_t p = threadIdx.x + 256u * k;  // pair 0..1023 over q (0..511) and k (512..1023)
    const uint32_t i = p & 31u;
    float* e = row + 2u * p;
    const float2 cs = table[size_t(t) * 32u + i];
    const float x0 = e[0], x1 = e[1];
    e[0] = __fsub_rn(__fmul_rn(x0, cs.x), __fmul_rn(x1, cs.y));
    e[1] = __fadd_rn(__fmul_rn(x0, cs.y), __fmul_rn(x1, cs.x));
  }
}

// Windowed causal attention of the post-module transformer
// (forward_codec_transformer_layer_with_window, codec.rs:3278-3300, over
// gqa_decode_attention, attention.rs:208-247): block = 16 queries x one head,
// the 143 keys / values those queries see ([q0 - 127, q0 + 15]) staged in LDS
// (key rows padded to 68 floats: 16-byte aligned, and a 16-lane phase of
// float4 reads covers all 64 banks).  A wave takes 4 queries: lane j scores
// keys j and j + 64 of the query's window (four partial sums per dot
// product), softmax over the wave, the probabilities go through wave-private
// LDS, and lane d sums p_k v_k[d] (four partial sums).
constexpr uint32_t CA_Q = 16, CA_W = 128, CA_K = CA_Q + CA_W - 1, CA_KS = 68;
__global__ __launch_bounds__(256) void codec_attn_kernel(const float* qkv, uint32_t T, float* out) {
  __shared__ __align__(16) float ks[CA_K * CA_KS];
  __shared__ __align__(16) float vs[CA_K * 64];
  __shared__ __align__(16) float qs[CA_Q * 64];
  __shared__ __align__(16) float ps[4][128];
  const uint32_t q0 = blockIdx.x * CA_Q, h = blockIdx.y, tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t kstart = q0 >= CA_W - 1 ? q0 - (CA_W - 1) : 0u;
  const uint32_t kend = min(T, q0 + CA_Q);
  const uint32_t nk = kend - kstart;
  for (uint32_t e = tid; e < nk * 16u; e += 256u) {
    const uint32_t r = e >> 4, d4 = (e & 15u) * 4u;
    const float* src = qkv + size_t(kstart + r) * 3072u + h * 64u + d4;
    *reinterpret_cast<float4*>(ks + r * CA_KS + d4) = *reinterpret_cast<const float4*>(src + 1024);
    *reinterpret_cast<float4*>(vs + r * 64u + d4) = *reinterpret_cast<const float4*>(src + 2048);
  }
  {
    const uint32_t r = tid >> 4, d4 = (tid & 15u) * 4u;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (q0 + r < T) v = *reinterpret_cast<const float4*>(qkv + size_t(q0 + r) * 3072u + h * 64u + d4);
    *reinterpret_cast<float4*>(qs + r * 64u + d4) = v;
  }
  __syncthreads();
  float* pw = ps[wave];
  for (uint32_t qq = 0; qq < 4; ++qq) {
    const uint32_t ql = wave * 4u + qq, tq = q0 + ql;
    if (tq >= T) break;
    const uint32_t lo = tq >= CA_W - 1 ? tq - (CA_W - 1) : 0u, n = tq - lo + 1u;
    const float* qr = qs + ql * 64u;
    float sc[2];
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      const uint32_t j = lane + 64u * uint32_t(h2);
      sc[h2] = -INFINITY;
      if (j < n) {
        const float* kr = ks + (lo + j - kstart) * CA_KS;
        float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
        for (int i = 0; i < 64; i += 4) {
          const float4 qv = *reinterpret_cast<const float4*>(qr + i);
          const float4 kv = *reinterpret_cast<const float4*>(kr + i);
          a0 = fmaf(qv.x, kv.x, a0);
          a1 = fmaf(qv.y, kv.y, a1);
          a2 = fmaf(qv.z, kv.z, a2);
          a3 = fmaf(qv.w, kv.w, a3);
        }
        sc[h2] = ((a0 + a1) + (a2 + a3)) * 0.125f;
      }
    }
    const float mx = wave_max(fmaxf(sc[0], sc[1]));
    const float e0 = lane < n ? expf_glibc(sc[0] - mx) : 0.0f;
    const float e1 = lane + 64u < n ? expf_glibc(sc[1] - mx) : 0.0f;
    const float sum = wave_sum(e0 + e1);
    const float inv = 1.0f / sum;
    pw[lane] = e0 * inv;
    pw[lane + 64u] = e1 * inv;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const float* vb = vs + (lo - kstart) * 64u + lane;
    float o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f;
    uint32_t k = 0;
    for (; k + 4u <= n; k += 4u) {
      const float4 p4 = *reinterpret_cast<const float4*>(pw + k);
      o0 = fmaf(p4.x, vb[(k + 0u) * 64u], o0);
      o1 = fmaf(p4.y, vb[(k + 1u) * 64u], o1);
      o2 = fmaf(p4.z, vb[(k + 2u) * 64u], o2);
      o3 = fmaf(p4.w, vb[(k + 3u) * 64u], o3);
    }
    for (; k < n; ++k) o0 = fmaf(pw[k], vb[k * 64u], o0);
    out[size_t(tq) * 1024u + h * 64u + lane] = (o0 + o1) + (o2 + o3);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

__global__ __launch_bounds__(256) void codec_scaled_residual_kernel(float* x, const float* p, const float* scale,
                                                                    size_t n, uint32_t D) {
  const size_t i = size_t(blockIdx.x) * 256u + threadIdx.x;
  if (i >= n) return;
  x[i] = __fadd_rn(x[i], __fmul_rn(p[i], scale[i % D]));
}

__global__ __launch_bounds__(256) void codec_split16_kernel(const float* x, _Float16* hi, _Float16* lo, size_t n) {
  const size_t i = size_t(blockIdx.x) * 256u + threadIdx.x;
  if (i >= n) return;
  const float v = x[i];
  const _Float16 h = _Float16(v);
  hi[i] = h;
  lo[i] = _Float16(__fsub_rn(v, float(h)));
}

// forward_codec_convnext_block front (codec.rs:3444-3460): depthwise causal
// conv k7 (depthwise_causal_conv1d :3576-3619, sums in the reference order)
// then layer_norm_affine_frame_major (:3621-3654) over the frame's 1024
// channels; output as hi / lo planes for the pointwise product.
__global__ __launch_bounds__(256) void codec_dwconv_ln_kernel(const float* x, uint32_t F, const float* w,
                                                              const float* b, const float* ln_w, const float* ln_b,
                                                              float eps, _Float16* hi, _Float16* lo) {
  __shared__ float red[4];
  const uint32_t f = blockIdx.x, tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  float d[4];
  float s = 0.0f;
#pragma unroll
  for (uint32_t k = 0; k < 4; ++k) {
    const uint32_t c = tid + 256u * k;
    float acc = b[c];
#pragma unroll
    for (uint32_t kk = 0; kk < 7; ++kk) {
      if (f + kk < 6u) continue;
      const uint32_t src = f + kk - 6u;
      acc = __fadd_rn(acc, __fmul_rn(x[size_t(src) * 1024u + c], w[c * 7u + kk]));
    }
    d[k] = acc;
    s += acc;
  }
  s = wave_sum(s);
  if (lane == 0) red[wave] = s;
  __syncthreads();
  const float mean = ((red[0] + red[1]) + (red[2] + red[3])) / 1024.0f;
  __syncthreads();
  float v = 0.0f;
#pragma unroll
  for (uint32_t k = 0; k < 4; ++k) {
    const float c = d[k] - mean;
    v += c * c;
  }
  v = wave_sum(v);
  if (lane == 0) red[wave] = v;
  __syncthreads();
  const float var = ((red[0] + red[1]) + (red[2] + red[3])) / 1024.0f;
  const float scale = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(var, eps)));
#pragma unroll
  for (uint32_t k = 0; k < 4; ++k) {
    const uint32_t c = tid + 256u * k;
    const float y = __fadd_rn(__fmul_rn(__fmul_rn(__fsub_rn(d[k], mean), scale), ln_w[c]), ln_b[c]);
    const _Float16 h = _Float16(y);
    hi[size_t(f) * 1024u + c] = h;
    lo[size_t(f) * 1024u + c] = _Float16(__fsub_rn(y, float(h)));
  }
}

// Output conv of the decoder (96 -> 1, k 7, causal; causal_conv_1d_frame_major
// :2212-2293, sum = bias, then tap, then channel, in order) over the f16
// snake outputs, then tanh.  Block = 256 samples; the 262 input rows it reads
// are staged in LDS (row stride 98 halfs: 49 dwords, odd, so lanes reading
// consecutive rows hit distinct banks).
constexpr uint32_t OC_ROW = 98;
__global__ __launch_bounds__(256) void codec_out_conv_kernel(const _Float16* x, uint32_t T, const float* w, float b,
                                                             float* out) {
  __shared__ _Float16 xs[262 * OC_ROW];
  __shared__ float wsm[7][96];
  const uint32_t t0 = blockIdx.x * 256u, tid = threadIdx.x;
  for (uint32_t e = tid; e < 96u * 7u; e += 256u) wsm[e % 7u][e / 7u] = w[e];  // w[c][tap]
  for (uint32_t e = tid; e < 262u * 12u; e += 256u) {
    const uint32_t r = e / 12u, c = e - r * 12u;
    const int32_t src = int32_t(t0) + int32_t(r) - 6;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (src >= 0 && src < int32_t(T)) v = *reinterpret_cast<const uint4*>(x + size_t(src) * 96u + c * 8u);
    uint32_t* d = reinterpret_cast<uint32_t*>(xs + r * OC_ROW + c * 8u);
    d[0] = v.x;
    d[1] = v.y;
    d[2] = v.z;
    d[3] = v.w;
  }
  __syncthreads();
  const uint32_t t = t0 + tid;
  if (t >= T) return;
  float y = b;
  for (uint32_t tap = 0; tap < 7; ++tap) {
    const _Float16* row = xs + (tid + tap) * OC_ROW;
    for (uint32_t c = 0; c < 96; c += 2) {
      const uint32_t pr = *reinterpret_cast<const uint32_t*>(row + c);
      const float x0 = float(__builtin_bit_cast(_Float16, uint16_t(pr & 0xffffu)));
      const float x1 = float(__builtin_bit_cast(_Float16, uint16_t(pr >> 16)));
      y = __fadd_rn(y, __fmul_rn(x0, wsm[tap][c]));
      y = __fadd_rn(y, __fmul_rn(x1, wsm[tap][c + 1]));
    }
  }
  out[t] = tanhf(y);
}

template <int MC, int KC, int PL, bool FU = false>
hipError_t conv_gemm_launch(const ConvGemmArgs& a, uint32_t phases, hipStream_t s) {
  constexpr uint32_t TM = 32 * MC, CH = KC / 8;
  const int32_t last = a.off0 + int32_t(a.G - 1) * a.ostep;
  const int32_t wbase = a.off0 < last ? a.off0 : last;
  const uint32_t halo = uint32_t((a.off0 < last ? last : a.off0) - wbase);
  const uint32_t AR = CG_TF + halo;
  if (size_t(PL) * AR * CH + size_t(a.G) * TM * CH > 256u * CG_MAXLD) return hipErrorInvalidValue;
  size_t lds = 2u * (size_t(PL) * AR + size_t(a.G) * TM) * KC * sizeof(_Float16);
  if (FU) lds = std::max(lds, (size_t(CG_TF) * (TM + 8) + size_t(TM) * TM) * sizeof(_Float16));
  if (lds > 160u * 1024u) return hipErrorInvalidValue;
  const uint32_t m_tiles = (a.M + TM - 1) / TM, f_tiles = (a.F + CG_TF - 1) / CG_TF;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&conv_gemm_kernel<MC, KC, PL, FU>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  // K split when the grid would leave CUs idle: each split keeps >= 4 stages
  const uint32_t nst = a.C / KC, blocks = m_tiles * f_tiles * phases;
  const size_t rows = size_t(a.F) * phases;
  uint32_t splits = 1;
  if (a.part && !FU) {
    while (splits < 8 && blocks * splits < 256u && nst / (2 * splits) >= 4 &&
           size_t(2 * splits) * rows * a.M <= a.part_cap)
      splits *= 2;
  }
  // frame-tile-major block order when the weights of every (phase, m tile)
  // fit in an XCD's L2 next to the streamed input windows
  const size_t wbytes = size_t(phases) * m_tiles * a.G * TM * a.C * sizeof(_Float16);
  const uint32_t fmajor = wbytes <= CG_FMAJOR_WEIGHT_BYTES ? 1u : 0u;
  conv_gemm_kernel<MC, KC, PL, FU><<<dim3(m_tiles * f_tiles * phases, 1, splits), 256, lds, s>>>(
      a, m_tiles, f_tiles, halo, wbase, a.off0 - wbase, a.ostep, fmajor);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || splits == 1) return e;
  const size_t n = rows * a.M;
  conv_split_reduce_kernel<<<uint32_t((n + 255) / 256), 256, 0, s>>>(a, splits);
  return hipGetLastError();
}

}  // namespace

ConvTile conv_tile(uint32_t M, uint32_t G, bool split) {
  (void)split;
  ConvTile t;
  t.mc = (M % 128u != 0 && M % 96u == 0) ? 3u : 4u;
  t.kc = G > 1 ? 16u : 32u;
  return t;
}

size_t conv_packed_halfs(uint32_t phases, uint32_t M, uint32_t G, uint32_t C, ConvTile t) {
  const uint32_t TM = 32 * t.mc;
  return size_t(phases) * ((M + TM - 1) / TM) * TM * G * C;
}

hipError_t launch_conv_gemm(const ConvGemmArgs& a, uint32_t phases, ConvTile t, hipStream_t s) {
  if (a.C == 0 || a.C % t.kc || a.F == 0 || a.M == 0 || a.G == 0 || phases == 0) return hipErrorInvalidValue;
  if (a.ldx % 8u || (a.yh && a.ldh % 2u)) return hipErrorInvalidValue;
  const bool split = a.xl != nullptr;
  if (t.mc == 4 && t.kc == 16) return split ? conv_gemm_launch<4, 16, 2>(a, phases, s) : conv_gemm_launch<4, 16, 1>(a, phases, s);
  if (t.mc == 4 && t.kc == 32) return split ? conv_gemm_launch<4, 32, 2>(a, phases, s) : conv_gemm_launch<4, 32, 1>(a, phases, s);
  if (t.mc == 3 && t.kc == 16) return split ? conv_gemm_launch<3, 16, 2>(a, phases, s) : conv_gemm_launch<3, 16, 1>(a, phases, s);
  if (t.mc == 3 && t.kc == 32) return split ? conv_gemm_launch<3, 32, 2>(a, phases, s) : conv_gemm_launch<3, 32, 1>(a, phases, s);
  return hipErrorInvalidValue;
}

hipError_t launch_residual_unit(const ConvGemmArgs& a, ConvTile t, hipStream_t s) {
  if (!a.w1 || !a.bias_mid || !a.alpha_mid || a.M % 32u || a.M > 32u * t.mc || t.kc != 16 || a.xl ||
      a.C != a.M || a.ldx % 8u)
    return hipErrorInvalidValue;
  if (t.mc == 3) return conv_gemm_launch<3, 16, 1, true>(a, 1, s);
  if (t.mc == 4) return conv_gemm_launch<4, 16, 1, true>(a, 1, s);
  return hipErrorInvalidValue;
}

hipError_t launch_codec_rvq(const RvqArgs& a, hipStream_t s) {
  if (a.F == 0) return hipSuccess;
  codec_rvq_kernel<<<a.F, 256, 0, s>>>(a);
  return hipGetLastError();
}

hipError_t launch_codec_check_codes(const int32_t* codes, uint32_t F, uint32_t* err, hipStream_t s) {
  const size_t n = size_t(10) * F;
  if (n == 0) return hipSuccess;
  codec_check_codes_kernel<<<uint32_t((n + 255) / 256), 256, 0, s>>>(codes, F, err);
  return hipGetLastError();
}

hipError_t launch_codec_rope(float* qkv, uint32_t T, const float2* table, hipStream_t s) {
  if (T == 0) return hipSuccess;
  codec_rope_kernel<<<T, 256, 0, s>>>(qkv, table);
  return hipGetLastError();
}

hipError_t launch_codec_attention(const float* qkv, uint32_t T, float* out, hipStream_t s) {
  if (T == 0) return hipSuccess;
  codec_attn_kernel<<<dim3((T + CA_Q - 1) / CA_Q, 16), 256, 0, s>>>(qkv, T, out);
  return hipGetLastError();
}

hipError_t launch_codec_scaled_residual(float* x, const float* p, const float* scale, uint32_t T, uint32_t D,
                                        hipStream_t s) {
  const size_t n = size_t(T) * D;
  if (n == 0) return hipSuccess;
  codec_scaled_residual_kernel<<<uint32_t((n + 255) / 256), 256, 0, s>>>(x, p, scale, n, D);
  return hipGetLastError();
}

hipError_t launch_codec_split16(const float* x, _Float16* hi, _Float16* lo, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  codec_split16_kernel<<<uint32_t((n + 255) / 256), 256, 0, s>>>(x, hi, lo, n);
  return hipGetLastError();
}

hipError_t launch_codec_dwconv_ln(const float* x, uint32_t F, const float* w, const float* b, const float* ln_w,
                                  const float* ln_b, float eps, _Float16* hi, _Float16* lo, hipStream_t s) {
  if (F == 0) return hipSuccess;
  codec_dwconv_ln_kernel<<<F, 256, 0, s>>>(x, F, w, b, ln_w, ln_b, eps, hi, lo);
  return hipGetLastError();
}

hipError_t launch_codec_out_conv(const _Float16* x, uint32_t T, const float* w, float b, float* out, hipStream_t s) {
  if (T == 0) return hipSuccess;
  codec_out_conv_kernel<<<(T + 255) / 256, 256, 0, s>>>(x, T, w, b, out);
  return hipGetLastError();
}

}  // namespace s2
