// expf_glibc.h -- single-precision exp with the results of glibc's expf.
//
// The reference computes every f32 exp with Rust's f32::exp, which on Linux is
// a call to the C library's expf (glibc 2.35 in this image).  The sampler's
// softmax (crates/fish_s2_infer/src/sampling.rs:202-225) and the SwiGLU
// sigmoid (slow_ar.rs:1215-1232, fast_ar.rs:472-485) feed its results into
// sequential sums and draws, so a device exp that is merely accurate (or
// correctly rounded) differs from the reference in the last bit for a small
// fraction of inputs (about 6 in 10^4 in [-17, 0]).
//
// Method (published in ARM's optimized-routines, which glibc adopted for
// expf): with N = 32,
//   z = x * N / ln 2,  k = round-to-nearest-even(z),  r = z - k in [-1/2, 1/2],
//   exp(x) = 2^(k/N) * 2^(r/N) ~= s * (C0 r^3 + C1 r^2 + C2 r + 1),
// evaluated in double and rounded once to float.  s = 2^(k/N) comes from a
// 32-entry table of 2^(i/N) (each the nearest double) whose entries have
// i << 47 subtracted, so adding k << 47 to the bits also applies 2^(k div N).
// C0..C2 are the method's published minimax coefficients of 2^(r/N).  The
// rounding of k uses the 1.5 * 2^52 shift; r is formed with one fused
// multiply-add from the unrounded product, as glibc's FMA build does.
//
// Checked on the host against this image's glibc expf over all 2^32 float
// inputs: identical bits for every input (including +-inf, NaN, the overflow
// threshold 0x1.62e42ep6 and the underflow threshold -0x1.9fe368p6).
#ifndef S2HIP_EXPF_GLIBC_H
#define S2HIP_EXPF_GLIBC_H

#include <hip/hip_runtime.h>

#include <stdint.h>

namespace s2 {

// 2^(i/32) as the nearest double, minus i << 47 in the bit pattern.
static constexpr uint64_t kExp2fTab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

// `sel` maps the table index (identity, or made wave-uniform on the device).
template <class Sel>
__host__ __device__ inline float expf_glibc_impl(float x, Sel sel) {
  const uint32_t ux = __builtin_bit_cast(uint32_t, x);
  const uint32_t abstop = (ux >> 20) & 0x7ffu;
  if (abstop >= 0x42bu) {  // |x| >= 88 or NaN (0x42b = top 12 bits of 88.0f)
    if (ux == 0xff800000u) return 0.0f;  // -inf
    if (abstop >= 0x7f8u) return x + x;  // +inf, NaN
    if (x > 0x1.62e42ep6f) return __builtin_inff();  // above ln(2^128)
    if (x < -0x1.9fe368p6f) return 0.0f;  // below ln(2^-150)
  }
  const double xd = static_cast<double>(x);
  const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
  const double shift = 0x1.8p+52;
  double kd = __builtin_fma(inv_ln2_n, xd, shift);
  const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
  kd -= shift;
  const double r = __builtin_fma(inv_ln2_n, xd, -kd);
  const double s = __builtin_bit_cast(double, kExp2fTab[sel(uint32_t(ki & 31u))] + (ki << 47));
  const double c0 = 0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0);
  const double c1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32.0);
  const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
  const double z = __builtin_fma(c0, r, c1);
  double y = __builtin_fma(c2, r, 1.0);
  y = __builtin_fma(z, r * r, y);
  return static_cast<float>(y * s);
}

__host__ __device__ inline float expf_glibc(float x) {
  return expf_glibc_impl(x, [](uint32_t i) { return i; });
}

// For an x that is the same in every lane of the wave (a GEMV epilogue after
// a wave reduction): the table index is made wave-uniform, so the entry is a
// scalar-cache load instead of a vector load at the kernel's tail.
__device__ inline float expf_glibc_wave(float x) {
  return expf_glibc_impl(x, [](uint32_t i) { return uint32_t(__builtin_amdgcn_readfirstlane(int(i))); });
}

}  // namespace s2

#endif
