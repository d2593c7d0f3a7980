// Cross-lane sums without an LDS round trip: DPP moves for lane ^ 1 / ^ 2 and
// the 8- and 16-lane groups, v_permlane16_swap / v_permlane32_swap (gfx950)
// for lane ^ 16 / ^ 32.  Every lane of a group ends with the same value (each
// step adds a pair of values in an order-independent way).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}
// v + v of lane ^ 1, lane ^ 2 (DPP quad permutations [1,0,3,2] / [2,3,0,1])
__device__ __forceinline__ float add_xor1(float v) { return v + dpp_f32<0xB1>(v); }
__device__ __forceinline__ float add_xor2(float v) { return v + dpp_f32<0x4E>(v); }
// sum over each aligned group of 8 / 16 lanes (half-row / row mirror last)
__device__ __forceinline__ float sum8_lanes(float v) {
  v = add_xor2(add_xor1(v));
  return v + dpp_f32<0x141>(v);
}
__device__ __forceinline__ float sum16_lanes(float v) {
  v = sum8_lanes(v);
  return v + dpp_f32<0x140>(v);
}
// maximum over each aligned group of 16 lanes, in all 16
template <int CTRL>
__device__ __forceinline__ float max_dpp(float v) {
  const float u = dpp_f32<CTRL>(v);
  return u > v ? u : v;
}
__device__ __forceinline__ float max16_lanes(float v) {
  v = max_dpp<0xB1>(v);
  v = max_dpp<0x4E>(v);
  v = max_dpp<0x141>(v);
  return max_dpp<0x140>(v);
}
// v + v of lane ^ 16 / lane ^ 32 (the two rows / halves swapped whole)
__device__ __forceinline__ float add_xor16(float v) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float add_xor32(float v) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
// sum over the whole wave (64 lanes)
__device__ __forceinline__ float sum64_lanes(float v) { return add_xor32(add_xor16(sum16_lanes(v))); }

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, true);
}
__device__ __forceinline__ uint64_t umax64_pair(uint64_t a, uint32_t hi, uint32_t lo) {
  const uint64_t b = ((uint64_t)hi << 32) | lo;
  return a > b ? a : b;
}
// maximum of a 64-bit key over the whole wave, in every lane
__device__ __forceinline__ uint64_t max64_lanes(uint64_t k) {
#define MAX64_DPP(CTRL) k = umax64_pair(k, dpp_u32<CTRL>((uint32_t)(k >> 32)), dpp_u32<CTRL>((uint32_t)k))
  MAX64_DPP(0xB1);
  MAX64_DPP(0x4E);
  MAX64_DPP(0x141);
  MAX64_DPP(0x140);
#undef MAX64_DPP
  {
    const auto h = __builtin_amdgcn_permlane16_swap((uint32_t)(k >> 32), (uint32_t)(k >> 32), false, false);
    const auto l = __builtin_amdgcn_permlane16_swap((uint32_t)k, (uint32_t)k, false, false);
    k = umax64_pair(umax64_pair(0, h[0], l[0]), h[1], l[1]);
  }
  {
    const auto h = __builtin_amdgcn_permlane32_swap((uint32_t)(k >> 32), (uint32_t)(k >> 32), false, false);
    const auto l = __builtin_amdgcn_permlane32_swap((uint32_t)k, (uint32_t)k, false, false);
    k = umax64_pair(umax64_pair(0, h[0], l[0]), h[1], l[1]);
  }
  return k;
}
