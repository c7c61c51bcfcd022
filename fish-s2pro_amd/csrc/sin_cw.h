// sin_cw.h -- sin^2 in single precision for the snake activation
// (snake_activation_frame_major, crates/fish_s2_infer/src/codec.rs:2162-2186,
// which evaluates sin with the C library's sinf).
//
// Method: Cody & Waite argument reduction by pi/2 with pi/2 split into three
// floats (c1 + c2 + c3, each product exact inside a fused multiply-add), then
// the minimax polynomials of the Cephes library's single-precision sin and
// cos (S. L. Moshier) on [-pi/4, pi/4]; sin^2 of the argument is the square
// of the sin polynomial for an even quadrant and of the cos polynomial for
// an odd one (the sign drops out).  Checked on the host against glibc sinf
// squared over |x| <= 1024 (tests/test_cpu_host.py).
#pragma once

#include <hip/hip_runtime.h>

namespace s2 {

__host__ __device__ inline float sin_sq_cw(float x) {
  const float k = rintf(x * 0.63661975f);  // 2 / pi
  float r = fmaf(-k, 1.57079637f, x);      // c1 = f32(pi / 2)
  r = fmaf(-k, -4.37113883e-08f, r);       // c2 = f32(pi / 2 - c1)
  r = fmaf(-k, -1.71512451e-15f, r);       // c3 = f32(pi / 2 - c1 - c2)
  const float r2 = r * r;
  const float s = fmaf(r * r2, fmaf(r2, fmaf(r2, -1.9515295891e-4f, 8.3321608736e-3f), -1.6666654611e-1f), r);
  const float c = fmaf(r2 * r2, fmaf(r2, fmaf(r2, 2.443315711809948e-5f, -1.388731625493765e-3f),
                                     4.166664568298827e-2f),
                       fmaf(-0.5f, r2, 1.0f));
  const float v = (int(k) & 1) ? c : s;
  return v * v;
}

// x + sin(a x)^2 / a with the reference's guard |a| < 1e-8 -> 1e-8
__host__ __device__ inline float snake_cw(float x, float alpha) {
  const float a = fabsf(alpha) < 1e-8f ? 1e-8f : alpha;
  return x + sin_sq_cw(a * x) / a;
}

}  // namespace s2
