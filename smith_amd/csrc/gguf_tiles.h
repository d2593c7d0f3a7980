// gguf_tiles.h -- device layout of GGUF linear weights ("tile planes") for the
// decode GEMV (smith_agemv_*) and the prefill GEMM (smith_gemm_*), shared by
// the kernels and the host bridge.
//
// A weight listed [out=N, in=K] (GGUF rows of K, blocks along K) is stored as
// 32-element records (g, n), g = k / 32, in 16-column tiles:
//     rec(g, n) = ((n / 16) * G + g) * 16 + n % 16,  G = K / 32, N % 16 == 0
// so a tile is G*16 contiguous records and a wave reads a 16-column slice of
// one group with a single base address.  Planes, each indexed by rec (sup:
// by srec(s, n) = ((n / 16) * (G / 8) + s) * 16 + n % 16, s = g / 8), at
// 256-byte aligned offsets of one buffer:
//
//   nib  16 B  low 4 bits of the 32 elements, element e in byte e/2 (low
//              nibble if e even) -- the reference's order for every type
//              (src/gguf.js:187-197, :203-215, :238-259, :294-300, :318-323)
//   hb         Q5_0: 4 B, Q6_K: 8 B -- the 5th / 5th-6th bits, permuted (below)
//   prm        Q4_0 / Q5_0: f16 d (2 B); Q4_1: f16 d | f16 m << 16 (4 B);
//              Q4_K: 6-bit scale | 6-bit min << 8 of the sub-block (2 B);
//              Q6_K: int8 scale of elements 0-15 | of 16-31 << 8 (2 B)
//   sup        Q4_K: f16 d | f16 dmin << 16 (4 B); Q6_K: f16 d (2 B)
//
// Bytes per 32 weights: Q4_0 18, Q4_1 20, Q5_0 22, Q4_K 18.5, Q6_K 26.25 --
// the GGUF sizes (Q4_K / Q6_K super-block fields spread over their 8 groups).
//
// High bits are permuted for the MFMA operand conversion: element e = 8i + k
// of a record (MFMA slice i, k < 8) lands in f16 lane half (k >> 2) of dword
// (k & 3) of slice i; its bits sit at
//   Q5_0: bit  c + 16*(k >> 2)           of the hb word,  c = 4i + (k & 3)
//   Q6_K: bits 2c + 16*(k >> 2), +1      of hb word i >> 1, c = 4*(i & 1) + (k & 3)
// so every dword's pair of halves takes its bits with one shift and one mask.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define GT_Q40 3  // = FMT_Q40T of smith_kernels.hip
#define GT_Q41 4
#define GT_Q50 5
#define GT_Q4K 6
#define GT_Q6K 7

__host__ __device__ constexpr uint32_t gt_hb_bytes(int f) { return f == GT_Q50 ? 4u : (f == GT_Q6K ? 8u : 0u); }
__host__ __device__ constexpr uint32_t gt_prm_bytes(int f) { return f == GT_Q41 ? 4u : 2u; }
__host__ __device__ constexpr uint32_t gt_sup_bytes(int f) { return f == GT_Q4K ? 4u : (f == GT_Q6K ? 2u : 0u); }
__host__ __device__ constexpr bool gt_super(int f) { return f == GT_Q4K || f == GT_Q6K; }

struct GtPlanes {
  size_t hb, prm, sup, total;  // byte offsets from the start (nib at 0), total size
};

__host__ __device__ inline size_t gt_align(size_t x) { return (x + 255) & ~(size_t)255; }

__host__ __device__ inline GtPlanes gt_planes(int f, uint32_t N, uint32_t G) {
  const size_t R = (size_t)N * G;
  GtPlanes p;
  p.hb = gt_align(R * 16);
  p.prm = gt_align(p.hb + R * gt_hb_bytes(f));
  p.sup = gt_align(p.prm + R * gt_prm_bytes(f));
  p.total = gt_align(p.sup + (size_t)N * (G / 8) * gt_sup_bytes(f));
  return p;
}

// GGML type number (src/gguf.js:15-25) -> tile format, -1 if none
__host__ __device__ inline int gt_of_ggml(int type) {
  switch (type) {
    case 2: return GT_Q40;
    case 3: return GT_Q41;
    case 6: return GT_Q50;
    case 12: return GT_Q4K;
    case 14: return GT_Q6K;
    default: return -1;
  }
}
