// wave.h -- cross-lane reductions of a 64-lane wave (gfx950) without LDS
// round trips.
//
// Each 16-lane row is reduced with DPP operands of the VALU instruction
// itself: quad permutes pair lanes 1 and 2 apart, then the half-row mirror
// (lane i <-> 7 - i) pairs the two quads of each half-row and the row mirror
// (i <-> 15 - i) its two half-rows -- at that point the partners hold
// already-uniform quads / half-rows, so the mirrors act as exchanges 4 and 8
// lanes apart.  The four row results are then read into scalar registers
// (v_readlane) and combined, so every lane receives the wave's result as one
// uniform value.  Four dependent DPP steps and four lane reads replace six
// dependent ds_bpermute round trips through the LDS crossbar.
//
// All 64 lanes must be active (callers reduce under wave-uniform control).
#pragma once

#include <hip/hip_runtime.h>

#include <stdint.h>

namespace s2 {

enum : int {
  DPP_QUAD_XOR1 = 0xB1,        // quad_perm [1,0,3,2]
  DPP_QUAD_XOR2 = 0x4E,        // quad_perm [2,3,0,1]
  DPP_ROW_HALF_MIRROR = 0x141,  // lane i <-> 7 - i within each 8
  DPP_ROW_MIRROR = 0x140,       // lane i <-> 15 - i within each 16
};

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return uint32_t(__builtin_amdgcn_mov_dpp(int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __uint_as_float(dpp_u32<CTRL>(__float_as_uint(v)));
}
__device__ __forceinline__ uint32_t lane_read_u32(uint32_t v, int lane) {
  return uint32_t(__builtin_amdgcn_readlane(int(v), lane));
}
__device__ __forceinline__ float lane_read_f32(float v, int lane) {
  return __uint_as_float(lane_read_u32(__float_as_uint(v), lane));
}

// op over each 16-lane row: every lane of a row ends with the row's value
template <class T, class Op>
__device__ __forceinline__ T row_reduce(T v, Op op) {
  if constexpr (sizeof(T) == 4 && __is_same(T, float)) {
    v = op(v, dpp_f32<DPP_QUAD_XOR1>(v));
    v = op(v, dpp_f32<DPP_QUAD_XOR2>(v));
    v = op(v, dpp_f32<DPP_ROW_HALF_MIRROR>(v));
    v = op(v, dpp_f32<DPP_ROW_MIRROR>(v));
  } else {
    v = op(v, dpp_u32<DPP_QUAD_XOR1>(v));
    v = op(v, dpp_u32<DPP_QUAD_XOR2>(v));
    v = op(v, dpp_u32<DPP_ROW_HALF_MIRROR>(v));
    v = op(v, dpp_u32<DPP_ROW_MIRROR>(v));
  }
  return v;
}

// op over the wave, as (row0 op row1) op (row2 op row3); uniform result
template <class T, class Op>
__device__ __forceinline__ T wave_reduce(T v, Op op) {
  v = row_reduce(v, op);
  if constexpr (__is_same(T, float)) {
    return op(op(lane_read_f32(v, 0), lane_read_f32(v, 16)), op(lane_read_f32(v, 32), lane_read_f32(v, 48)));
  } else {
    return op(op(lane_read_u32(v, 0), lane_read_u32(v, 16)), op(lane_read_u32(v, 32), lane_read_u32(v, 48)));
  }
}

__device__ __forceinline__ float wave_sum(float v) {
  return wave_reduce(v, [](float a, float b) { return a + b; });
}
__device__ __forceinline__ float wave_max(float v) {
  return wave_reduce(v, [](float a, float b) { return fmaxf(a, b); });
}
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
  return wave_reduce(v, [](uint32_t a, uint32_t b) { return a + b; });
}

}  // namespace s2
