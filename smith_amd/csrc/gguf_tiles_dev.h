// gguf_tiles_dev.h -- device side of the GGUF tile planes (gguf_tiles.h):
// loading one record's fields, its affine form w = s*q + c, and the
// exponent-bias f16 operand of one MFMA slice with the high bits merged.
// Included by the kernel sources after their u32x4 / half8 typedefs.
#pragma once
#include "gguf_tiles.h"

// one 32-element record as loaded
template <int F>
struct GtW {
  u32x4 q;          // nib plane: low 4 bits, element e in byte e/2
  uint32_t h0, h1;  // hb plane (Q5_0: h0; Q6_K: h0 slices 0-1, h1 slices 2-3)
  uint32_t p;       // prm plane
  uint32_t sp;      // sup plane
};

template <int F>
__device__ __forceinline__ void gt_load(GtW<F>& w, const uint8_t* __restrict__ base, const GtPlanes& P, size_t rec,
                                        size_t srec) {
  w.q = *(const u32x4*)(base + rec * 16);
  w.h0 = w.h1 = 0u;
  w.sp = 0u;
  if (F == GT_Q50) w.h0 = *(const uint32_t*)(base + P.hb + rec * 4);
  if (F == GT_Q6K) {
    const uint2 h = *(const uint2*)(base + P.hb + rec * 8);
    w.h0 = h.x;
    w.h1 = h.y;
  }
  if (F == GT_Q41) w.p = *(const uint32_t*)(base + P.prm + rec * 4);
  else w.p = *(const uint16_t*)(base + P.prm + rec * 2);
  if (F == GT_Q4K) w.sp = *(const uint32_t*)(base + P.sup + srec * 4);
  if (F == GT_Q6K) w.sp = *(const uint16_t*)(base + P.sup + srec * 2);
}

__device__ __forceinline__ float gt_h2f(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits16 & 0xFFFFu));
}

// w = s0*q + c0 for elements 0-15, s1*q + c1 for 16-31 (equal except Q6_K).
// Every product is exact in f32 (an f16 times an integer of <= 8 bits).
template <int F>
__device__ __forceinline__ void gt_affine(const GtW<F>& w, float& s0, float& c0, float& s1, float& c1) {
  if (F == GT_Q40 || F == GT_Q50) {
    s0 = gt_h2f(w.p);
    c0 = (F == GT_Q40 ? -8.0f : -16.0f) * s0;
  } else if (F == GT_Q41) {
    s0 = gt_h2f(w.p);
    c0 = gt_h2f(w.p >> 16);
  } else if (F == GT_Q4K) {
    s0 = gt_h2f(w.sp) * (float)(w.p & 63u);
    c0 = -(gt_h2f(w.sp >> 16) * (float)((w.p >> 8) & 63u));
  } else {  // Q6_K
    const float d = gt_h2f(w.sp);
    s0 = d * (float)(int8_t)(w.p & 0xFFu);
    s1 = d * (float)(int8_t)((w.p >> 8) & 0xFFu);
    c0 = -32.0f * s0;
    c1 = -32.0f * s1;
  }
  if (F != GT_Q6K) {
    s1 = s0;
    c1 = c0;
  }
}

template <int SH>
__device__ __forceinline__ uint32_t gt_shift(uint32_t v) {
  if constexpr (SH >= 0) return v >> SH;
  else return v << (-SH);
}

// (x & mask) | (base & ~mask), in plain C so the compiler's MFMA hazard
// checks see it (no inline asm next to MFMAs)
__device__ __forceinline__ uint32_t gt_bfi(uint32_t mask, uint32_t x, uint32_t base) {
  return (x & mask) | (base & ~mask);
}

// B operand of MFMA slice I (elements 8I..8I+7) in the exponent-bias form:
// slot order {0,4,1,5,2,6,3,7}; low-nibble slots hold f16 1024 + q, high-
// nibble slots 64 + q (q the full 4/5/6-bit integer)
template <int F, int I>
__device__ __forceinline__ half8 gt_to_f16(const GtW<F>& w) {
  const uint32_t x = w.q[I], y = x >> 8;
  uint32_t bx = 0x64006400u, by = 0x54005400u, bz = 0x64006400u, bw = 0x54005400u;
  if constexpr (F == GT_Q50) {
    const uint32_t W = w.h0;
    bx |= gt_shift<4 * I + 0 - 4>(W) & 0x00100010u;
    by |= gt_shift<4 * I + 1 - 8>(W) & 0x01000100u;
    bz |= gt_shift<4 * I + 2 - 4>(W) & 0x00100010u;
    bw |= gt_shift<4 * I + 3 - 8>(W) & 0x01000100u;
  } else if constexpr (F == GT_Q6K) {
    const uint32_t W = I < 2 ? w.h0 : w.h1;
    constexpr int cb = 4 * (I & 1);
    bx |= gt_shift<2 * (cb + 0) - 4>(W) & 0x00300030u;
    by |= gt_shift<2 * (cb + 1) - 8>(W) & 0x03000300u;
    bz |= gt_shift<2 * (cb + 2) - 4>(W) & 0x00300030u;
    bw |= gt_shift<2 * (cb + 3) - 8>(W) & 0x03000300u;
  }
  u32x4 u;
  u.x = gt_bfi(0x000F000Fu, x, bx);
  u.y = gt_bfi(0x00F000F0u, x, by);
  u.z = gt_bfi(0x000F000Fu, y, bz);
  u.w = gt_bfi(0x00F000F0u, y, bw);
  return __builtin_bit_cast(half8, u);
}

// the integer q of element e (0..31) of a record (prefill dequantization)
template <int F>
__device__ __forceinline__ uint32_t gt_q(const GtW<F>& w, int e) {
  const uint32_t byte = (w.q[e >> 3] >> (8 * ((e & 7) >> 1))) & 0xFFu;
  uint32_t q = (e & 1) ? (byte >> 4) : (byte & 15u);
  const int i = e >> 3, k = e & 7;
  if (F == GT_Q50) q |= ((w.h0 >> (4 * i + (k & 3) + 16 * (k >> 2))) & 1u) << 4;
  if (F == GT_Q6K) q |= (((i < 2 ? w.h0 : w.h1) >> (2 * (4 * (i & 1) + (k & 3)) + 16 * (k >> 2))) & 3u) << 4;
  return q;
}
