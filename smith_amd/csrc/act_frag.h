// act_frag.h -- prepared activation vectors ("act") for the single-row decode
// GEMV smith_agemv_q40t_*.
//
// An act buffer describes one activation vector a[0..K) (K % 32 == 0) in the
// form the MFMA GEMV consumes, so the consumer does no per-workgroup
// preparation.  It is written by the kernel that produces the vector (the
// previous projection's epilogue, the attention combine, the embedding
// lookup), 16 consecutive elements per call, with
//     a = v * gamma_out   (gamma_out null -> a = v)
// where v is the produced value; an RMSNorm in front of the consumer is then
// applied as one scalar on its output (rms is linear: W^T (x*rms*g) =
// rms * W^T (x*g)), from the sums of squares of v recorded here.
//
// Layout (bytes), G = K/32 groups, T = K/8 parts of 8 elements:
//   [0, 128*G)         f16 frag[g][u][32]: u = 0 hi = f16(a), u = 1 lo =
//                      f16((a - hi) * 2048); within each 8-element slice i
//                      (= part 4g+i) the slot order of the Q4 B-operand
//                      conversion (slot e holds element {0,4,1,5,2,6,3,7}[e])
//   [4*K, +4*T)        float c1[t] = sum over the part of a * off(slot)
//                      (hi + lo/2048), off = 1024 (low nibble slots) or 64
//                      (high nibble slots), plus 8 * sum(a) (the Q4_0 -8)
//   [.., +4*T)         float s[t]  = sum over the part of a (hi + lo/2048)
//   [.., +4*T)         float ss[t] = sum over the part of v * v
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lanes.h"

__host__ __device__ constexpr size_t act_bytes(uint32_t K) { return (size_t)K * 4 + (size_t)(K / 8) * 12; }

// All 8 lanes of an aligned 8-lane group call this together, lane L holding
// element o = o0 + (L & 7) (o0 % 8 == 0) with value v and the gamma of that
// element (1 without a norm).
__device__ __forceinline__ void act_emit8(uint8_t* __restrict__ act, uint32_t K, uint32_t o, float v, float gam) {
  const float a = v * gam;
  const _Float16 h = (_Float16)a;
  const float hf = (float)h;
  const _Float16 l = (_Float16)((a - hf) * 2048.0f);
  const float lf = (float)l;
  const uint32_t g = o >> 5, p = o & 31, i = p >> 3, s = p & 7;
  const uint32_t e = (s & 3) * 2 + (s >> 2);  // slot of element s
  _Float16* fr = (_Float16*)act;
  fr[(g * 2 + 0) * 32 + i * 8 + e] = h;
  fr[(g * 2 + 1) * 32 + i * 8 + e] = l;
  const float off = (e & 2) ? 64.0f : 1024.0f;
  float c1 = __builtin_fmaf(lf * off, 1.0f / 2048.0f, hf * off);
  float sm = __builtin_fmaf(lf, 1.0f / 2048.0f, hf);
  float ss = v * v;
  c1 = sum8_lanes(c1);
  sm = sum8_lanes(sm);
  ss = sum8_lanes(ss);
  if ((o & 7) == 0) {
    const uint32_t T = K / 8, t = o >> 3;
    float* part = (float*)(act + (size_t)K * 4);
    part[t] = __builtin_fmaf(8.0f, sm, c1);
    part[T + t] = sm;
    part[2 * T + t] = ss;
  }
}
