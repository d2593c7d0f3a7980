// Floor kernels for bench.py: what any kernel reading the same bytes with
// the same grid can achieve on this GPU.  Bench-only: built into
// smith_amd/lib/smith_bench.hsaco and launched by libsmith_bench.so
// (bench_floor_host.cpp); the product library never loads them.  Every kernel takes (p, n, out) and stores
// to `out` only under a condition the data never meets, so the loads stay
// alive and nothing is written.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// An empty launch.
extern "C" __global__ void floor_empty(const uint4* p, uint64_t n, uint32_t* out) {
  if (n == 0x12345u) out[0] = (uint32_t)(size_t)p;
}

// Streaming read of n 16-byte chunks, 4 loads in flight per thread over a
// grid-stride loop.
extern "C" __global__ void floor_stream_read(const uint4* __restrict__ p, uint64_t n, uint32_t* out) {
  constexpr int U = 4;
  const uint64_t tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x, stride = (uint64_t)gridDim.x * blockDim.x;
  uint32_t acc = 0;
  for (uint64_t base = tid; base < n; base += stride * U) {
    uint4 v[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const uint64_t i = base + u * stride;
      v[u] = i < n ? p[i] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x9e3779b9u) out[0] = acc;
}

// Streaming read in per-workgroup contiguous chunks: 128 threads x 6
// 16-byte loads, all in flight (12 KB per workgroup; the fastest shape of a
// grid sweep over 64-1024 threads and 1-12 loads per thread on 12.6 MB).
extern "C" __global__ __launch_bounds__(128) void floor_block_read(const uint4* __restrict__ p, uint64_t n,
                                                                  uint32_t* out) {
  const uint64_t base = (uint64_t)blockIdx.x * 128 * 6 + threadIdx.x;
  uint4 v[6];
#pragma unroll
  for (int u = 0; u < 6; u++) {
    const uint64_t i = base + 128 * u;
    v[u] = i < n ? p[i] : make_uint4(0, 0, 0, 0);
  }
  uint32_t acc = 0;
#pragma unroll
  for (int u = 0; u < 6; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  if (acc == 0x9e3779b9u) out[0] = acc;
}

// The config-1 single-row GEMV's weight reads alone on Q4S records (n = N
// columns, K = 4096 = 128 groups): N / 16 workgroups of 8 waves; lane (c, j)
// of wave w reads the 16 + 8 bytes of record (group 16w + 4s + j, column
// 16 * block + c) for s = 0..3, as smith_qgemv1_q4s_m1_k128 does, no math.
extern "C" __global__ __launch_bounds__(512) void floor_q4s_record_read(const uint8_t* __restrict__ B, uint64_t n,
                                                                       uint32_t* out) {
  const uint32_t N = (uint32_t)n;
  const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6, c = lane & 15, j = lane >> 4;
  const uint32_t col = blockIdx.x * 16 + c;
  u32x4 q[4];
  uint2 sz[4];
#pragma unroll
  for (int s = 0; s < 4; s++) {
    const uint8_t* p = B + ((size_t)(16 * w + 4 * s + j) * N + col) * 24;
    q[s] = *(const u32x4*)p;
    sz[s] = *(const uint2*)(p + 16);
  }
  uint32_t acc = 0;
#pragma unroll
  for (int s = 0; s < 4; s++) acc ^= q[s].x ^ q[s].y ^ q[s].z ^ q[s].w ^ sz[s].x ^ sz[s].y;
  if (acc == 0x9e3779b9u) out[0] = acc;
}

// The same grid and lanes on GGUF Q4_0 tile-major planes (smith_qgemv1_q40t_m1_k128):
// B holds the nibble plane (record (g, col) at ((col / 16) * 128 + g) * 16 +
// col % 16, 16 bytes each) followed by the f16 scale plane in the same order.
extern "C" __global__ __launch_bounds__(512) void floor_q40t_record_read(const uint8_t* __restrict__ B, uint64_t n,
                                                                        uint32_t* out) {
  const uint32_t N = (uint32_t)n;
  const uint16_t* D = (const uint16_t*)(B + (size_t)N * 128 * 16);
  const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6, c = lane & 15, j = lane >> 4;
  u32x4 q[4];
  uint32_t sb[4];
#pragma unroll
  for (int s = 0; s < 4; s++) {
    const size_t rec = ((size_t)blockIdx.x * 128 + 16 * w + 4 * s + j) * 16 + c;
    q[s] = *(const u32x4*)(B + rec * 16);
    sb[s] = D[rec];
  }
  uint32_t acc = 0;
#pragma unroll
  for (int s = 0; s < 4; s++) acc ^= q[s].x ^ q[s].y ^ q[s].z ^ q[s].w ^ sb[s];
  if (acc == 0x9e3779b9u) out[0] = acc;
}

// The record loads alone of the batched and single-row GEMVs, with the
// kernel's grid and lanes: workgroup (bx, by) of GX x GY (launched as one
// dimension, b = by * GX + bx), wave wk, lane (c, j) loads the record of
// column bx * 16 CT + 16 ct + c in group by * KB + wk * 4S + 4 st + j for
// every step st < S and column tile ct < CT (clamped into range), as
// smith_qgemv1 / smith_qgemv5 do.  n packs N (bits 0-19), the group count G
// (20-39) and GX (40-59).
template <int CT, int S, int WK, bool Q40T>
__device__ __forceinline__ void rec_read(const uint8_t* __restrict__ B, uint64_t n, uint32_t* out) {
  const uint32_t N = (uint32_t)(n & 0xFFFFF), G = (uint32_t)((n >> 20) & 0xFFFFF), GX = (uint32_t)(n >> 40);
  const uint32_t bx = blockIdx.x % GX, by = blockIdx.x / GX;
  const uint32_t lane = threadIdx.x & 63, wk = threadIdx.x >> 6, c = lane & 15, j = lane >> 4;
  constexpr uint32_t KB = 4 * S * WK, BC = 16 * CT;
  const uint16_t* D = (const uint16_t*)(B + (size_t)N * G * 16);  // Q4_0 tile planes: nibbles, then scales
  u32x4 q[S][CT];
  uint32_t t[S][CT];
#pragma unroll
  for (int st = 0; st < S; st++)
#pragma unroll
    for (int ct = 0; ct < CT; ct++) {
      uint32_t g = by * KB + wk * 4 * S + 4 * st + j, col = bx * BC + ct * 16 + c;
      g = g < G ? g : G - 1;
      col = col < N ? col : N - 1;
      if (Q40T) {
        const size_t rec = ((size_t)(col / 16) * G + g) * 16 + col % 16;
        q[st][ct] = *(const u32x4*)(B + rec * 16);
        t[st][ct] = D[rec];
      } else {
        const uint8_t* p = B + ((size_t)g * N + col) * 24;
        q[st][ct] = *(const u32x4*)p;
        const uint2 sz = *(const uint2*)(p + 16);
        t[st][ct] = sz.x ^ sz.y;
      }
    }
  uint32_t acc = 0;
#pragma unroll
  for (int st = 0; st < S; st++)
#pragma unroll
    for (int ct = 0; ct < CT; ct++) acc ^= q[st][ct].x ^ q[st][ct].y ^ q[st][ct].z ^ q[st][ct].w ^ t[st][ct];
  if (acc == 0x9e3779b9u) out[0] = acc;
}

#define DEF_REC_READ(NAME, CT, S, WK)                                                                    \
  extern "C" __global__ __launch_bounds__(64 * WK) void floor_rec_q4s_##NAME(const uint8_t* __restrict__ B, \
                                                                           uint64_t n, uint32_t* out) {    \
    rec_read<CT, S, WK, false>(B, n, out);                                                               \
  }                                                                                                      \
  extern "C" __global__ __launch_bounds__(64 * WK) void floor_rec_q40t_##NAME(const uint8_t* __restrict__ B, \
                                                                            uint64_t n, uint32_t* out) {   \
    rec_read<CT, S, WK, true>(B, n, out);                                                                \
  }
// qgemv1 k128 (one / two column tiles per wave) and k448w16, qgemv5 w16 /
// k32 / k32c4 / k64c2
DEF_REC_READ(c1s4w8, 1, 4, 8)
DEF_REC_READ(c1s7w16, 1, 7, 16)
DEF_REC_READ(c2s4w8, 2, 4, 8)
DEF_REC_READ(c1s2w16, 1, 2, 16)
DEF_REC_READ(c1s1w8, 1, 1, 8)
DEF_REC_READ(c4s1w8, 4, 1, 8)
DEF_REC_READ(c2s1w16, 2, 1, 16)
