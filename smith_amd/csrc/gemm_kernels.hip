// gemm_kernels.hip -- gfx950 prefill GEMM for the quantized-weight path
// (M >= 64 rows): C[M,N] = A[M,K] . W[K,N] with W in one of the packed
// formats of smith_kernels.hip, dequantized tile by tile into LDS as f16 and
// multiplied on v_mfma_f32_16x16x32_f16 with f32 accumulation.
//
//   smith_gemm_prep_a   A (f32, optional RMSNorm with gamma) -> A16 (f16)
//   smith_gemm_<fmt>_m<BM>_n<BN>  the GEMM, fmt in {q4s, q8, q40, q40t, q41t,
//                       q50t, q4kt, q6kt}
//   smith_gemm_prep_a_perm + smith_gemm2_<fmt>_m<BM>_n<BN>  the DMA-staged
//                       GEMM for the tile-plane formats (further below)
//
// Workgroup tile BM x BN (128x64 .. 256x256), K in stages of BK=64 (two
// 32-row quantization groups), double-buffered in LDS: while the MFMAs
// consume stage s, the global loads of stage s+1 (A16 rows, weight records)
// are in flight in registers; they are dequantized and stored after the
// MFMAs.  Big tiles give each stage enough MFMA work (0.86 us for 256x256)
// to cover the loads' latency.  A wave owns a 64x64 (64x32 for BN=64) part
// of the tile as 16x16 MFMA tiles.  LDS rows hold 64 K values; their 16-byte
// chunks are XOR-swizzled by the row (128 B stride, 256 * (BM + BN) bytes of
// LDS) for the smaller tiles, and rows are padded by 8 halves instead (144 B
// stride, 288 * (BM + BN) = 147 KB) at 256x256, where measured the swizzle
// did not pay.
// Dequantization (exact products, one f16 rounding per weight):
//   Q4S   w = scale * (nib - zero)   record (g,n) 24 B  (shaders/matmul_q4.metal:24-28)
//   Q8    w = f32(d) * int8          record (g,n) 34 B  (shaders/matmul_q8.metal:40-52)
//   Q40T  w = d * (nib - 8)          tile-major planes  (src/gguf.js:187-197)
//   Q40   same, planes in (g, n) record order
// element k of a group is nibble k (byte k>>1, low nibble first) / byte k.
// Epilogues: 0 store, 1 residual add, 2 SwiGLU on interleaved (gate, up)
// columns: C[m][n/2] = silu(gate) * up.
// Tiles are numbered so the tiles that share a weight tile run on one XCD
// (workgroup id mod 8), keeping that weight tile in one L2.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
#include "gguf_tiles_dev.h"

#define WF_Q4S 0
#define WF_Q8 1
#define WF_Q40T 2
#define WF_Q40 3  // Q4_0 planes in (g, n) order (smith_repack_q4_0)

#define GBK 64
#define GLD 80  // halves per LDS row (64 + 16 pad: 160-byte rows keep the 16-byte reads aligned; 4x fewer bank conflicts than 72)

__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
  _Float16 ha = (_Float16)a, hb = (_Float16)b;
  return (uint32_t)__builtin_bit_cast(uint16_t, ha) | ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
}

// one weight record in registers
struct WRec {
  u32x4 q;         // Q4: 32 nibbles; Q8: int8 0..15
  u32x4 q8b;       // Q8: int8 16..31 (with the 2-byte shift dword)
  uint32_t q8c;
  uint32_t sh;
  float s, z;
  uint32_t h0, h1, p, sp;  // GGUF tile planes (FMT >= GT_Q41): hb words, prm, sup
};

template <int FMT>
__device__ __forceinline__ WRec load_wrec(const uint8_t* __restrict__ B, const uint16_t* __restrict__ D,
                                          uint32_t N, uint32_t G, uint32_t g, uint32_t n) {
  WRec r;
  const bool ok = g < G && n < N;
  const uint32_t gc = g < G ? g : G - 1, nc = n < N ? n : N - 1;
  r.sh = 0;
  r.z = 0.f;
  if (FMT >= GT_Q41) {
    // GGUF tile planes (gguf_tiles.h); a zero prm / sup makes the record 0
    GtW<FMT> w;
    const size_t rec = ((size_t)(nc >> 4) * G + gc) * 16 + (nc & 15);
    gt_load<FMT>(w, B, gt_planes(FMT, N, G), rec, ((size_t)(nc >> 4) * (G / 8) + gc / 8) * 16 + (nc & 15));
    r.q = w.q;
    r.h0 = w.h0;
    r.h1 = w.h1;
    r.p = ok ? w.p : 0u;
    r.sp = ok ? w.sp : 0u;
    r.s = 1.f;
    return r;
  }
  if (FMT == WF_Q4S) {
    const uint8_t* p = B + ((size_t)gc * N + nc) * 24;
    r.q = *(const u32x4*)p;
    const float2 sz = *(const float2*)(p + 16);
    r.s = sz.x;
    r.z = sz.y;
  } else if (FMT == WF_Q40T || FMT == WF_Q40) {
    const size_t rec = FMT == WF_Q40 ? (size_t)gc * N + nc : ((size_t)(nc >> 4) * G + gc) * 16 + (nc & 15);
    r.q = *(const u32x4*)(B + rec * 16);
    r.s = (float)__builtin_bit_cast(_Float16, D[rec]);
    r.z = 8.f;
  } else {
    const uint8_t* p = B + ((size_t)gc * N + nc) * 34;
    r.s = (float)__builtin_bit_cast(_Float16, *(const uint16_t*)p);
    const size_t a = (size_t)(p + 2);
    const uint32_t* w = (const uint32_t*)(p + 2 - (a & 3));  // stays a global pointer (no flat loads)
    r.sh = (uint32_t)(a & 3);
    r.q = (u32x4){w[0], w[1], w[2], w[3]};
    r.q8b = (u32x4){w[4], w[5], w[6], w[7]};
    r.q8c = w[8];
  }
  if (!ok) r.s = 0.f;
  return r;
}

// Q4 records (Q4S, Q4_0: w = s * (q - z)) in packed f16: elements 16h ..
// 16h+15 as 8 f16 pairs, each 8-element chunk in the slot order
// {0,4,1,5,2,6,3,7} (A is prepared in the same order).  Nibbles b and b+4 of
// a dword land in the low mantissa bits of 0x6400 (f16 1024 + q, exact),
// 1024 comes off exactly, and one fma applies the scale and -scale*zero
// (both rounded to f16; the product is exact inside the fma).
__device__ __forceinline__ void q4_pairs(const WRec& r, uint32_t h, uint32_t (&o)[8]) {
  typedef _Float16 h2v __attribute__((ext_vector_type(2)));
  const _Float16 sh = (_Float16)r.s, ch = (_Float16)(-r.s * r.z);
  const h2v s2 = {sh, sh}, c2 = {ch, ch}, k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
  const uint32_t d[2] = {h ? r.q.z : r.q.x, h ? r.q.w : r.q.y};
#pragma unroll
  for (int i = 0; i < 2; i++) {
#pragma unroll
    for (int b = 0; b < 4; b++) {
      const uint32_t u = ((d[i] >> (4 * b)) & 0x000F000Fu) | 0x64006400u;
      const h2v q = __builtin_bit_cast(h2v, u) - k1024;
      o[4 * i + b] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(q, s2, c2));
    }
  }
}

// the 32 dequantized weights of a record as 16 packed f16 pairs (k order; Q4 formats in the slot order of q4_pairs)
template <int FMT>
__device__ __forceinline__ void dequant_wrec(const WRec& r, uint32_t (&o)[16]) {
  if constexpr (FMT >= GT_Q41) {
    GtW<FMT> w;
    w.q = r.q;
    w.h0 = r.h0;
    w.h1 = r.h1;
    w.p = r.p;
    w.sp = r.sp;
    float s0, c0, s1, c1;
    gt_affine<FMT>(w, s0, c0, s1, c1);
#pragma unroll
    for (int e = 0; e < 32; e += 2) {
      const float s = e < 16 ? s0 : s1, c = e < 16 ? c0 : c1;
      o[e / 2] = pack_h2(__builtin_fmaf((float)gt_q<FMT>(w, e), s, c), __builtin_fmaf((float)gt_q<FMT>(w, e + 1), s, c));
    }
    return;
  }
  if (FMT == WF_Q8) {
    const uint32_t d[9] = {r.q.x, r.q.y, r.q.z, r.q.w, r.q8b.x, r.q8b.y, r.q8b.z, r.q8b.w, r.q8c};
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t x = __builtin_amdgcn_alignbyte(d[i + 1], d[i], r.sh);  // int8 4i..4i+3
      const float v0 = (float)(int8_t)(x & 0xFF), v1 = (float)(int8_t)((x >> 8) & 0xFF);
      const float v2 = (float)(int8_t)((x >> 16) & 0xFF), v3 = (float)(int8_t)(x >> 24);
      o[2 * i] = pack_h2(r.s * v0, r.s * v1);
      o[2 * i + 1] = pack_h2(r.s * v2, r.s * v3);
    }
  } else {
    uint32_t a[8], b[8];
    q4_pairs(r, 0, a);
    q4_pairs(r, 1, b);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      o[i] = a[i];
      o[8 + i] = b[i];
    }
  }
}

// elements 16h .. 16h+15 of a record (h = 0 or 1, per thread) as 8 packed f16
// pairs: the half of dequant_wrec a thread stores when two threads share a
// record (same arithmetic, so the same bits)
template <int FMT>
__device__ __forceinline__ void dequant_half(const WRec& r, uint32_t h, uint32_t (&o)[8]) {
  if constexpr (FMT >= GT_Q41) {
    uint32_t full[16];
    dequant_wrec<FMT>(r, full);
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = h ? full[8 + i] : full[i];
  } else if constexpr (FMT == WF_Q8) {
    const uint32_t d[9] = {r.q.x, r.q.y, r.q.z, r.q.w, r.q8b.x, r.q8b.y, r.q8b.z, r.q8b.w, r.q8c};
#pragma unroll
    for (int ii = 0; ii < 4; ii++) {
      // int8 16h + 4ii .. +3 (dwords 4h+ii, 4h+ii+1 of the shifted window)
      const uint32_t lo = h ? d[4 + ii] : d[ii], hi = h ? d[5 + ii] : d[1 + ii];
      const uint32_t x = __builtin_amdgcn_alignbyte(hi, lo, r.sh);
      const float v0 = (float)(int8_t)(x & 0xFF), v1 = (float)(int8_t)((x >> 8) & 0xFF);
      const float v2 = (float)(int8_t)((x >> 16) & 0xFF), v3 = (float)(int8_t)(x >> 24);
      o[2 * ii] = pack_h2(r.s * v0, r.s * v1);
      o[2 * ii + 1] = pack_h2(r.s * v2, r.s * v3);
    }
  } else {
    q4_pairs(r, h, o);
  }
}

// 16-byte chunk position of chunk c (0..7) of LDS row r: with padded rows
// (LD > 64) the identity; unpadded rows (LD == 64) XOR-swizzle the chunk by
// the row so the 16-row MFMA operand reads and the row-wise stores spread
// over the banks
template <int LD>
__device__ __forceinline__ uint32_t swz(uint32_t r, uint32_t c) {
  return LD == 64 ? (c ^ (r & 7)) : c;
}

__device__ __forceinline__ float silu_mul_g(float g, float u) { return g / (1.0f + __expf(-g)) * u; }

template <int FMT, int BM, int BN, int WM, int WN, int LD = GLD>
__device__ __forceinline__ void gemm_body(const _Float16* __restrict__ A16, const uint8_t* __restrict__ B,
                                         const uint16_t* __restrict__ D, float* __restrict__ C, uint32_t M,
                                         uint32_t N, uint32_t K, const float* __restrict__ R, uint32_t epi,
                                         float* __restrict__ ws, uint32_t sps) {
  constexpr int WAVES_N = BN / WN, NT = 64 * (BM / WM) * WAVES_N;
  constexpr int TM = WM / 16, TN = WN / 16;          // 16x16 MFMA tiles per wave
  constexpr int ACH = BM * GBK / 8;                  // 16-byte A chunks per stage
  constexpr int APT = ACH / NT;                      // per thread
  constexpr int NREC = BN * GBK / 32;                // weight records per stage
  constexpr int RPT = NREC >= NT ? NREC / NT : 1;    // records per thread
  constexpr bool HALF = NREC < NT;                   // two threads per record, 16 elements each
  static_assert(ACH % NT == 0, "A chunks must divide evenly");
  static_assert(NREC >= NT ? NREC % NT == 0 : NT == 2 * NREC, "records must divide evenly over the threads");
  __shared__ __attribute__((aligned(16))) _Float16 As[2][BM][LD];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[2][BN][LD];

  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t wm = wave / WAVES_N, wn = wave % WAVES_N;
  const uint32_t G = K / 32;
  const uint32_t MB = (M + BM - 1) / BM, NBk = (N + BN - 1) / BN, T = MB * NBk;
  // XCD-grouped tile order: XCD x (= id % 8) takes tiles [x*T/8, (x+1)*T/8),
  // M-fastest, so its tiles share weight tiles
  uint32_t t = blockIdx.x;
  if (T % 8 == 0) t = (blockIdx.x % 8) * (T / 8) + blockIdx.x / 8;
  const uint32_t nb = t / MB, mb = t % MB;
  const uint32_t m0 = mb * BM, n0 = nb * BN;
  // K split (gridDim.y > 1): this block runs stages [s0, s1) and writes its
  // partial tile to ws[blockIdx.y]; smith_gemm_reduce finishes
  const uint32_t Sall = (K + GBK - 1) / GBK;
  const uint32_t s0 = blockIdx.y * sps < Sall ? blockIdx.y * sps : Sall;
  const uint32_t s1 = s0 + sps < Sall ? s0 + sps : Sall;
  const uint32_t S = s1 - s0;

  struct Regs {
    u32x4 av[APT];
    WRec wr[RPT];
  };
  auto load_stage = [&](Regs& rg, uint32_t s) {
    const uint32_t k0 = s * GBK;
#pragma unroll
    for (int q = 0; q < APT; q++) {
      const uint32_t idx = tid + NT * q, row = idx >> 3, c8 = idx & 7;
      const uint32_t m = m0 + row < M ? m0 + row : M - 1;
      const uint32_t k = k0 + 8 * c8;
      rg.av[q] = k < K ? *(const u32x4*)(A16 + (size_t)m * K + k) : (u32x4){0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int q = 0; q < RPT; q++) {
      const uint32_t idx = HALF ? tid % NREC : tid + NT * q;  // every thread has a record: no branch
      const uint32_t n = idx % BN, gi = idx / BN;
      rg.wr[q] = load_wrec<FMT>(B, D, N, G, 2 * s + gi, n0 + n);
    }
  };
  auto store_stage = [&](const Regs& rg, uint32_t buf) {
#pragma unroll
    for (int q = 0; q < APT; q++) {
      const uint32_t idx = tid + NT * q, row = idx >> 3, c8 = idx & 7;
      *(u32x4*)&As[buf][row][8 * swz<LD>(row, c8)] = rg.av[q];
    }
#pragma unroll
    for (int q = 0; q < RPT; q++) {
      if constexpr (HALF) {
        const uint32_t idx = tid % NREC, h = tid / NREC;
        const uint32_t n = idx % BN, gi = idx / BN;
        uint32_t o[8];
        dequant_half<FMT>(rg.wr[q], h, o);
#pragma unroll
        for (int v = 0; v < 2; v++)
          *(u32x4*)&Bs[buf][n][8 * swz<LD>(n, 4 * gi + 2 * h + v)] =
              (u32x4){o[4 * v], o[4 * v + 1], o[4 * v + 2], o[4 * v + 3]};
      } else {
        const uint32_t idx = tid + NT * q;
        const uint32_t n = idx % BN, gi = idx / BN;
        uint32_t o[16];
        dequant_wrec<FMT>(rg.wr[q], o);
#pragma unroll
        for (int v = 0; v < 4; v++)
          *(u32x4*)&Bs[buf][n][8 * swz<LD>(n, 4 * gi + v)] = (u32x4){o[4 * v], o[4 * v + 1], o[4 * v + 2], o[4 * v + 3]};
      }
    }
  };

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

  const uint32_t r16 = lane & 15, kq = lane >> 4;
  auto mfma_stage = [&](uint32_t buf) {
#pragma unroll
    for (int kk = 0; kk < GBK; kk += 32) {
      half8 af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; i++) {
        const uint32_t row = wm * WM + i * 16 + r16;
        af[i] = *(const half8*)&As[buf][row][8 * swz<LD>(row, kk / 8 + kq)];
      }
#pragma unroll
      for (int j = 0; j < TN; j++) {
        const uint32_t row = wn * WN + j * 16 + r16;
        bf[j] = *(const half8*)&Bs[buf][row][8 * swz<LD>(row, kk / 8 + kq)];
      }
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  };

  Regs r0;
  if (S > 0) {
    load_stage(r0, s0);
    store_stage(r0, 0);
  }
  __syncthreads();
  // steady state without guards (the last stage is peeled off).  (Pinning the
  // loads to the top of the stage with scheduling barriers measured slower:
  // the compiler's interleaving of the dequant work with the MFMAs wins.)
  for (uint32_t s = 0; s + 1 < S; s++) {
    const uint32_t buf = s & 1;
    load_stage(r0, s0 + s + 1);
    mfma_stage(buf);
    store_stage(r0, buf ^ 1);
    __syncthreads();
  }
  if (S > 0) mfma_stage((S - 1) & 1);

  // epilogue: lane (c = lane % 16, kq) holds rows 4kq .. 4kq+3 of column c of each tile
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const uint32_t n = n0 + wn * WN + j * 16 + r16;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const uint32_t m = m0 + wm * WM + i * 16 + 4 * kq + e;
        float v = acc[i][j][e];
        if (gridDim.y > 1) {
          if (m < M && n < N) ws[((size_t)blockIdx.y * M + m) * N + n] = v;
        } else if (epi == 2) {
          const float u = __shfl_down(v, 1);  // column n+1 of the same row
          if (m < M && n + 1 < N && (r16 & 1) == 0) C[(size_t)m * (N / 2) + n / 2] = silu_mul_g(v, u);
        } else if (m < M && n < N) {
          if (epi == 1) v += R[(size_t)m * N + n];
          C[(size_t)m * N + n] = v;
        }
      }
    }
}

#define DEF_GEMM(NAME, FMT, BM, BN, WM, WN, ...)                                                        \
  extern "C" __global__ __launch_bounds__(64 * (BM / WM) * (BN / WN)) void NAME(                            \
      const _Float16* __restrict__ A16, const uint8_t* __restrict__ B, const uint16_t* __restrict__ D,       \
      float* __restrict__ C, uint32_t M, uint32_t N, uint32_t K, const float* __restrict__ R, uint32_t epi,   \
      float* __restrict__ ws, uint32_t sps) {                                                                \
    gemm_body<FMT, BM, BN, WM, WN, ##__VA_ARGS__>(A16, B, D, C, M, N, K, R, epi, ws, sps);            \
  }

// tiles BMxBN: m128_n64 (4 waves of 64x32), m128_n128 (4 waves), m256_n128 (8),
// m256_n256 (16 waves); LDS holds 2 buffers of A and B rows
#define DEF_GEMM_FMT(TAG, FMT)                                             \
  DEF_GEMM(smith_gemm_##TAG##_m128_n64, FMT, 128, 64, 64, 32, 64)           \
  DEF_GEMM(smith_gemm_##TAG##_m128_n128, FMT, 128, 128, 64, 64, 64)         \
  DEF_GEMM(smith_gemm_##TAG##_m256_n128, FMT, 256, 128, 64, 64, 64)         \
  DEF_GEMM(smith_gemm_##TAG##_m256_n256, FMT, 256, 256, 64, 64)

DEF_GEMM_FMT(q4s, WF_Q4S)
DEF_GEMM_FMT(q8, WF_Q8)
DEF_GEMM_FMT(q40t, WF_Q40T)
DEF_GEMM_FMT(q40, WF_Q40)
DEF_GEMM_FMT(q41t, GT_Q41)
DEF_GEMM_FMT(q50t, GT_Q50)
DEF_GEMM_FMT(q4kt, GT_Q4K)
DEF_GEMM_FMT(q6kt, GT_Q6K)

// C = epilogue(sum over the ks K-split partials ws[0..ks) [M][N]), fixed
// order; one thread per output (pair for SwiGLU).
// ---------------------------------------------------------------------------
// gemm2: the same GEMM with the operands staged by direct-to-LDS loads
// (global_load_lds, no registers on the way) into a ring of 3 stages, and
// the weights kept in LDS as their raw records -- dequantized in registers
// right before the MFMAs.  Per stage of 64 K: A rows (f16, 16-byte chunks
// XOR-swizzled by row through the choice of each lane's source), weight
// planes of the tile's BN columns for 2 groups (Q4_0 tiles: 16 B of
// nibbles + 2 B d per record; the other tile formats add their high-bit and
// parameter planes).  The A operand's 8-element chunks are in the slot order
// {0,4,1,5,2,6,3,7} (smith_gemm_prep_a_perm), the order in which a nibble
// dword converts to f16 with 4 bit-inserts (exponent bias 1024 + q for low
// nibbles, 64 + q for high): both operands permuted alike leave the dot
// product unchanged.  Q4_0: w = (h - bias - 8) * d in packed f16 (q - 8
// exact, one rounding).  The loop is unrolled by the ring size so every LDS
// access names its stage buffer at compile time.  (Q4S records take the
// register-staged kernel above: converted per wave here they were slower.)
// ---------------------------------------------------------------------------
template <int BYTES_PER_WAVE>
struct DmaUnit {  // dwordx4 or dword loads splitting a wave's bytes evenly (LDS slot = lane * size)
  static constexpr int U = BYTES_PER_WAVE % 1024 == 0 ? 16 : 4;
  static constexpr int N = BYTES_PER_WAVE / (64 * U);
  static_assert(BYTES_PER_WAVE % (64 * U) == 0 && N >= 1, "stage bytes must split over the waves");
};

typedef __attribute__((address_space(3))) void* lds_ptr_t;

template <int U>
__device__ __forceinline__ void dma(const void* g, lds_ptr_t l) {
  if constexpr (U == 16) __builtin_amdgcn_global_load_lds(g, l, 16, 0, 0);
  else __builtin_amdgcn_global_load_lds(g, l, 4, 0, 0);
}

// Tile-plane formats (Q4_0 tiles and gguf_tiles.h): per stage and 16-column
// tile the weight bytes are contiguous runs in each plane -- nibbles 512 B
// (2 groups x 16 records x 16 B), high bits 32*hb B, record parameters 32*prm
// B, super-block parameters 16*sup B -- so each plane is one DMA segment,
// padded to 256 B (one dword load per lane of a wave).
template <int FMT>
struct GtFmt {
  static constexpr bool TILES = FMT == WF_Q40T || FMT >= GT_Q41;
  static constexpr int F = FMT == WF_Q40T ? GT_Q40 : FMT;  // gguf_tiles.h code
  static constexpr int HB = TILES ? (int)gt_hb_bytes(F) : 0;
  static constexpr int PRM = TILES ? (int)gt_prm_bytes(F) : 0;
  static constexpr int SUP = TILES ? (int)gt_sup_bytes(F) : 0;
};

__device__ __forceinline__ constexpr int pad256(int x) { return (x + 255) / 256 * 256; }

template <int FMT, int BM, int BN, int WM, int WN>
struct G2 {
  using GF = GtFmt<FMT>;
  static constexpr int NW = (BM / WM) * (BN / WN);
  static constexpr int A_BYTES = BM * 128;
  static constexpr int NIB = BN * 32;  // nibbles of 2 groups
  static constexpr int HBY = pad256(BN * 2 * GF::HB);
  static constexpr int PRY = GF::TILES ? pad256(BN * 2 * GF::PRM) : 0;
  static constexpr int SUY = pad256(BN * GF::SUP);
  static constexpr int B_BYTES = NIB + HBY + PRY + SUY;
  using UA = DmaUnit<A_BYTES / NW>;
};

__device__ __forceinline__ constexpr uint32_t vmcnt_imm(uint32_t n) {
  return (n & 0xF) | (0x7u << 4) | (0xFu << 8) | (((n >> 4) & 3u) << 14);
}

// s_waitcnt vmcnt(n) for a wave-uniform n (the immediate must be a constant)
__device__ __forceinline__ void wait_vm(uint32_t n) {
  switch (n) {
#define WV(i) \
  case i: __builtin_amdgcn_s_waitcnt(vmcnt_imm(i)); break;
    WV(0) WV(1) WV(2) WV(3) WV(4) WV(5) WV(6) WV(7) WV(8) WV(9) WV(10) WV(11) WV(12) WV(13) WV(14) WV(15)
    WV(16) WV(17) WV(18) WV(19) WV(20) WV(21) WV(22) WV(23) WV(24) WV(25) WV(26) WV(27) WV(28) WV(29) WV(30)
#undef WV
    default: __builtin_amdgcn_s_waitcnt(vmcnt_imm(0)); break;
  }
}

// DMA instructions (dword, 256 B each) of a padded segment of `bytes` that
// wave w issues: instruction j goes to wave j % NW
template <int NW>
__device__ __forceinline__ constexpr uint32_t seg_count(int bytes, uint32_t w) {
  return (uint32_t)(bytes / 256) > w ? ((uint32_t)(bytes / 256) - w + NW - 1) / NW : 0u;
}

template <int FMT, int BM, int BN, int WM, int WN>
__device__ __forceinline__ void gemm2_body(const _Float16* __restrict__ A16, const uint8_t* __restrict__ B,
                                          const uint16_t* __restrict__ D, float* __restrict__ C, uint32_t M,
                                          uint32_t N, uint32_t K, const float* __restrict__ R, uint32_t epi,
                                          float* __restrict__ ws, uint32_t sps) {
  using P = G2<FMT, BM, BN, WM, WN>;
  using GF = GtFmt<FMT>;
  static_assert(GF::TILES, "tile-plane formats only");
  constexpr int NW = P::NW, WAVES_N = BN / WN;
  constexpr int TM = WM / 16, TN = WN / 16;
  __shared__ __attribute__((aligned(1024))) uint8_t As0[P::A_BYTES], As1[P::A_BYTES], As2[P::A_BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t Bs0[P::B_BYTES], Bs1[P::B_BYTES], Bs2[P::B_BYTES];

  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t wm = wave / WAVES_N, wn = wave % WAVES_N;
  const uint32_t G = K / 32;
  const uint32_t MB = (M + BM - 1) / BM, NBk = (N + BN - 1) / BN, T = MB * NBk;
  uint32_t t = blockIdx.x;
  if (T % 8 == 0) t = (blockIdx.x % 8) * (T / 8) + blockIdx.x / 8;
  const uint32_t nb = t / MB, mb = t % MB;
  const uint32_t m0 = mb * BM, n0 = nb * BN;
  const uint32_t Sall = K / 64;
  const uint32_t s0 = blockIdx.y * sps < Sall ? blockIdx.y * sps : Sall;
  const uint32_t s1 = s0 + sps < Sall ? s0 + sps : Sall;
  const uint32_t S = s1 - s0;
  // plane bases (tile formats): Q4_0 tiles take the d plane from D; the
  // others find their planes after the nibbles (gguf_tiles.h)
  const GtPlanes PL = gt_planes(GF::F, N, G);
  const uint8_t* hbp = B + PL.hb;
  const uint8_t* prp = FMT == WF_Q40T ? (const uint8_t*)D : B + PL.prm;
  const uint8_t* sup = B + PL.sup;
  const uint32_t NT16 = N / 16;
  // this wave's DMA instructions per stage
  const uint32_t cnt = P::UA::N + seg_count<NW>(P::NIB, wave) + seg_count<NW>(P::HBY, wave) +
                       seg_count<NW>(P::PRY, wave) + seg_count<NW>(P::SUY, wave);

  // one padded segment: per 16-column tile a run of TPB bytes at plane +
  // tile_off(tg); lanes past the segment load the last word again (into the
  // pad).  Each lane's source of its j-th instruction is formed once, for
  // stage 0; a stage adds the plane's stride (per-stage address arithmetic
  // was ~11 VALU per instruction in a VALU-bound loop)
  constexpr uint32_t SEGJ = (uint32_t)(P::NIB / 256 + NW - 1) / NW;  // most instructions of any segment per wave
  static_assert((uint32_t)(P::HBY / 256 + NW - 1) / NW <= SEGJ && (uint32_t)(P::PRY / 256 + NW - 1) / NW <= SEGJ &&
                    (uint32_t)(P::SUY / 256 + NW - 1) / NW <= SEGJ,
                "the nibble segment is the longest");
  auto seg_src = [&](const uint8_t* (&src)[SEGJ], int bytes, int TPB, auto src_of) {
#pragma unroll
    for (uint32_t jj = 0; jj < SEGJ; jj++) {
      uint32_t off = (wave + jj * NW) * 256 + lane * 4;
      const uint32_t real = (uint32_t)(BN / 16) * TPB;
      off = off < real ? off : real - 4;
      const uint32_t tt = off / TPB, w = off % TPB;
      uint32_t tg = n0 / 16 + tt;
      tg = tg < NT16 ? tg : NT16 - 1;
      src[jj] = src_of(tg) + w;
      (void)bytes;
    }
  };
  auto segment = [&](uint8_t* dst, int bytes, const uint8_t* const (&src)[SEGJ], size_t stage_off) {
    const uint32_t ni = (uint32_t)bytes / 256;
#pragma unroll
    for (uint32_t jj = 0; jj < SEGJ; jj++) {
      const uint32_t j = wave + jj * NW;
      if (j < ni) dma<4>(src[jj] + stage_off, (lds_ptr_t)(dst + j * 256));
    }
  };
  const uint8_t* srcN[SEGJ];
  const uint8_t* srcH[SEGJ];
  const uint8_t* srcP[SEGJ];
  const uint8_t* srcS[SEGJ];
  {
    seg_src(srcN, P::NIB, 512, [&](uint32_t tg) { return B + ((size_t)tg * G * 16) * 16; });
    if (GF::HB) seg_src(srcH, P::HBY, 32 * GF::HB, [&](uint32_t tg) { return hbp + ((size_t)tg * G * 16) * GF::HB; });
    seg_src(srcP, P::PRY, 32 * GF::PRM, [&](uint32_t tg) { return prp + ((size_t)tg * G * 16) * GF::PRM; });
    if (GF::SUP)
      seg_src(srcS, P::SUY, 16 * GF::SUP, [&](uint32_t tg) { return sup + ((size_t)tg * (G / 8) * 16) * GF::SUP; });
  }

  // DMA of stage s (absolute) into buffers (as, bs)
  auto issue = [&](uint32_t s, uint8_t* as, uint8_t* bs) {
    const uint32_t k0 = s * 64;
#pragma unroll
    for (int q = 0; q < P::UA::N; q++) {
      // this wave's bytes [off, off + 64 U) of the stage's A rows
      const uint32_t off = (wave * P::UA::N + q) * 64 * P::UA::U + lane * P::UA::U;
      const uint32_t row = off / 128, cs = (off % 128) / 16, ci = (off % 16) / 2;  // slot chunk, half within
      const uint32_t c = cs ^ (row & 7);
      const uint32_t m = m0 + row < M ? m0 + row : M - 1;
      dma<P::UA::U>(A16 + (size_t)m * K + k0 + 8 * c + ci, (lds_ptr_t)(as + (wave * P::UA::N + q) * 64 * P::UA::U));
    }
    const size_t g0 = 2 * s;  // a stage is two 32-row groups
    segment(bs, P::NIB, srcN, g0 * 16 * 16);
    if (GF::HB) segment(bs + P::NIB, P::HBY, srcH, g0 * 16 * GF::HB);
    segment(bs + P::NIB + P::HBY, P::PRY, srcP, g0 * 16 * GF::PRM);
    if (GF::SUP) segment(bs + P::NIB + P::HBY + P::PRY, P::SUY, srcS, (g0 / 8) * 16 * GF::SUP);
  };

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
  const uint32_t r16 = lane & 15, kq = lane >> 4;
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));

  auto compute = [&](const uint8_t* as, const uint8_t* bs) {
#pragma unroll
    for (int kk = 0; kk < 2; kk++) {
      half8 af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; i++) {
        const uint32_t row = wm * WM + i * 16 + r16;
        af[i] = *(const half8*)(as + row * 128 + 16 * ((kk * 4 + kq) ^ (row & 7)));
      }
#pragma unroll
      for (int j = 0; j < TN; j++) {
        const uint32_t col = wn * WN + j * 16 + r16;
        u32x4 u;
        {
          const uint32_t tt = col / 16, cc = col % 16;
          const uint32_t ri = (tt * 2 + kk) * 16 + cc;  // record within the stage, tile order
          const uint32_t x = *(const uint32_t*)(bs + ri * 16 + 4 * kq);
          const uint32_t y = x >> 8;
          uint32_t bx = 0x64006400u, by = 0x54005400u, bz = 0x64006400u, bw = 0x54005400u;
          if constexpr (GF::F == GT_Q50) {
            const uint32_t W = *(const uint32_t*)(bs + P::NIB + ri * 4);
            // element 8kq + k: bit 4kq + (k & 3) + 16 (k >> 2) (gguf_tiles.h)
            bx |= ((W >> (4 * kq)) << 4) & 0x00100010u;
            by |= ((W >> (4 * kq + 1)) << 8) & 0x01000100u;
            bz |= ((W >> (4 * kq + 2)) << 4) & 0x00100010u;
            bw |= ((W >> (4 * kq + 3)) << 8) & 0x01000100u;
          } else if constexpr (GF::F == GT_Q6K) {
            const uint2 hw = *(const uint2*)(bs + P::NIB + ri * 8);
            const uint32_t W = kq < 2 ? hw.x : hw.y, cb = 4 * (kq & 1);
            bx |= ((W >> (2 * cb)) << 4) & 0x00300030u;
            by |= ((W >> (2 * cb + 2)) << 8) & 0x03000300u;
            bz |= ((W >> (2 * cb + 4)) << 4) & 0x00300030u;
            bw |= ((W >> (2 * cb + 6)) << 8) & 0x03000300u;
          }
          // w = s*q + c with q = h - bias exact in f16
          h2 sv, cv;
          const uint8_t* prm = bs + P::NIB + P::HBY;
          if constexpr (GF::F == GT_Q40 || GF::F == GT_Q50) {
            const _Float16 d = *(const _Float16*)(prm + ri * 2);
            const _Float16 c = d * (_Float16)(GF::F == GT_Q40 ? -8.0f : -16.0f);  // exact
            sv = (h2){d, d};
            cv = (h2){c, c};
          } else if constexpr (GF::F == GT_Q41) {
            const h2 dm = *(const h2*)(prm + ri * 4);  // (d, m)
            sv = (h2){dm.x, dm.x};
            cv = (h2){dm.y, dm.y};
          } else {  // Q4_K, Q6_K: f32 products of the f16 and the 6-bit / int8 scales, rounded to f16
            float s0f, c0f, s1f, c1f;
            GtW<GF::F> w;
            w.p = *(const uint16_t*)(prm + ri * 2);
            w.sp = GF::SUP == 4 ? *(const uint32_t*)(prm + P::PRY + (tt * 16 + cc) * 4)
                                : *(const uint16_t*)(prm + P::PRY + (tt * 16 + cc) * 2);
            gt_affine<GF::F>(w, s0f, c0f, s1f, c1f);
            const float sf = kq < 2 ? s0f : s1f, cf = kq < 2 ? c0f : c1f;
            sv = (h2){(_Float16)sf, (_Float16)sf};
            cv = (h2){(_Float16)cf, (_Float16)cf};
          }
          const h2 blo = (h2){(_Float16)1024.0f, (_Float16)1024.0f}, bhi = (h2){(_Float16)64.0f, (_Float16)64.0f};
          const h2 v0 = __builtin_elementwise_fma(__builtin_bit_cast(h2, (x & 0x000F000Fu) | bx) - blo, sv, cv);
          const h2 v1 = __builtin_elementwise_fma(__builtin_bit_cast(h2, (x & 0x00F000F0u) | by) - bhi, sv, cv);
          const h2 v2 = __builtin_elementwise_fma(__builtin_bit_cast(h2, (y & 0x000F000Fu) | bz) - blo, sv, cv);
          const h2 v3 = __builtin_elementwise_fma(__builtin_bit_cast(h2, (y & 0x00F000F0u) | bw) - bhi, sv, cv);
          u = (u32x4){__builtin_bit_cast(uint32_t, v0), __builtin_bit_cast(uint32_t, v1),
                      __builtin_bit_cast(uint32_t, v2), __builtin_bit_cast(uint32_t, v3)};
        }
        bf[j] = __builtin_bit_cast(half8, u);
      }
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  };

  // ring: stage s in buffer s % 3; stages s+1 and s+2 in flight while s is used
  if (S > 0) issue(s0, As0, Bs0);
  if (S > 1) issue(s0 + 1, As1, Bs1);
  auto step = [&](uint32_t s, uint8_t* as, uint8_t* bs, uint8_t* an, uint8_t* bn) {
    // this wave's DMA of stage s done (stage s+1 may stay in flight), then all waves'
    wait_vm(s + 1 < S ? cnt : 0u);
    __builtin_amdgcn_s_barrier();
    if (s + 2 < S) issue(s0 + s + 2, an, bn);  // into the buffer stage s-1 used (all waves are past it)
    compute(as, bs);
  };
  for (uint32_t s = 0; s < S; s += 3) {
    step(s, As0, Bs0, As2, Bs2);
    if (s + 1 < S) step(s + 1, As1, Bs1, As0, Bs0);
    if (s + 2 < S) step(s + 2, As2, Bs2, As1, Bs1);
  }

#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const uint32_t n = n0 + wn * WN + j * 16 + r16;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const uint32_t m = m0 + wm * WM + i * 16 + 4 * kq + e;
        float v = acc[i][j][e];
        if (gridDim.y > 1) {
          if (m < M && n < N) ws[((size_t)blockIdx.y * M + m) * N + n] = v;
        } else if (epi == 2) {
          const float u = __shfl_down(v, 1);
          if (m < M && n + 1 < N && (r16 & 1) == 0) C[(size_t)m * (N / 2) + n / 2] = silu_mul_g(v, u);
        } else if (m < M && n < N) {
          if (epi == 1) v += R[(size_t)m * N + n];
          C[(size_t)m * N + n] = v;
        }
      }
    }
}

#define DEF_GEMM2(NAME, FMT, BM, BN, WM, WN)                                                                  \
  extern "C" __global__ __launch_bounds__(64 * (BM / WM) * (BN / WN))                                       \
  __attribute__((amdgpu_waves_per_eu(2))) void NAME(                                                          \
      const _Float16* __restrict__ A16, const uint8_t* __restrict__ B, const uint16_t* __restrict__ D,       \
      float* __restrict__ C, uint32_t M, uint32_t N, uint32_t K, const float* __restrict__ R, uint32_t epi,   \
      float* __restrict__ ws, uint32_t sps) {                                                                \
    gemm2_body<FMT, BM, BN, WM, WN>(A16, B, D, C, M, N, K, R, epi, ws, sps);                                  \
  }
// 128-row tiles: four waves side by side along N, each over all 128 rows,
// so every B fragment is converted once per workgroup (two 64-row waves per
// column converted it twice: gate|up at M = 128 36.7 -> 34.6 us)
#define DEF_GEMM2_FMT(TAG, FMT)                                   \
  DEF_GEMM2(smith_gemm2_##TAG##_m128_n64, FMT, 128, 64, 128, 16)   \
  DEF_GEMM2(smith_gemm2_##TAG##_m128_n128, FMT, 128, 128, 128, 32) \
  DEF_GEMM2(smith_gemm2_##TAG##_m256_n128, FMT, 256, 128, 64, 64) \
  DEF_GEMM2(smith_gemm2_##TAG##_m256_n256, FMT, 256, 256, 64, 64)
DEF_GEMM2_FMT(q40t, WF_Q40T)
DEF_GEMM2_FMT(q41t, GT_Q41)
DEF_GEMM2_FMT(q50t, GT_Q50)
DEF_GEMM2_FMT(q4kt, GT_Q4K)
DEF_GEMM2_FMT(q6kt, GT_Q6K)

template <bool PERM>
__device__ __forceinline__ void prep_a_row(const float* __restrict__ A, const float* __restrict__ gamma, float eps,
                                           _Float16* __restrict__ A16, uint32_t K);

// A16 as smith_gemm_prep_a, with each 8-element chunk in the slot order
// {0,4,1,5,2,6,3,7} of the gemm2 weight conversion.
extern "C" __global__ __launch_bounds__(256) void smith_gemm_prep_a_perm(const float* __restrict__ A,
                                                                        const float* __restrict__ gamma, float eps,
                                                                        _Float16* __restrict__ A16, uint32_t K) {
  prep_a_row<true>(A, gamma, eps, A16, K);
}

#define RED_BATCH 8

// Sum of the K-split partials in split order (deterministic), then the
// epilogue: 2 = SwiGLU of the (gate, up) column pairs, 1 = + residual.
// Four consecutive partials per thread with 16-byte loads when the sizes
// and pointers allow it, else one per thread.
extern "C" __global__ void smith_gemm_reduce(const float* __restrict__ ws, uint32_t ks, float* __restrict__ C,
                                             uint32_t M, uint32_t N, const float* __restrict__ R, uint32_t epi) {
  const size_t MN = (size_t)M * N;
  const size_t nout = epi == 2 ? MN / 2 : MN;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  const bool vec = (MN & 3) == 0 && ((size_t)C & (epi == 2 ? 7 : 15)) == 0 && ((size_t)ws & 15) == 0 &&
                   (epi != 1 || ((size_t)R & 15) == 0);
  if (vec) {
    for (size_t qd = (size_t)blockIdx.x * blockDim.x + threadIdx.x; 4 * qd < MN; qd += stride) {
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      for (uint32_t y0 = 0; y0 < ks; y0 += RED_BATCH) {  // a batch of split reads in flight, summed in order
        float4 t[RED_BATCH];
#pragma unroll
        for (uint32_t b = 0; b < RED_BATCH; b++)
          t[b] = y0 + b < ks ? *(const float4*)(ws + (y0 + b) * MN + 4 * qd) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (uint32_t b = 0; b < RED_BATCH; b++)
          if (y0 + b < ks) {
            v.x += t[b].x;
            v.y += t[b].y;
            v.z += t[b].z;
            v.w += t[b].w;
          }
      }
      if (epi == 2) {  // (gate, up) at columns 2c, 2c+1 of one row
        *(float2*)(C + 2 * qd) = make_float2(silu_mul_g(v.x, v.y), silu_mul_g(v.z, v.w));
      } else {
        if (epi == 1) {
          const float4 r = *(const float4*)(R + 4 * qd);
          v = make_float4(r.x + v.x, r.y + v.y, r.z + v.z, r.w + v.w);
        }
        *(float4*)(C + 4 * qd) = v;
      }
    }
    return;
  }
  for (size_t o = (size_t)blockIdx.x * blockDim.x + threadIdx.x; o < nout; o += stride) {
    if (epi == 2) {
      const size_t i = 2 * o;  // (gate, up) at columns 2c, 2c+1 of one row
      float g = 0.f, u = 0.f;
      for (uint32_t y0 = 0; y0 < ks; y0 += RED_BATCH) {
        float2 t[RED_BATCH];
#pragma unroll
        for (uint32_t b = 0; b < RED_BATCH; b++)
          t[b] = y0 + b < ks ? *(const float2*)(ws + (y0 + b) * MN + i) : make_float2(0.f, 0.f);
#pragma unroll
        for (uint32_t b = 0; b < RED_BATCH; b++)
          if (y0 + b < ks) {
            g += t[b].x;
            u += t[b].y;
          }
      }
      C[o] = silu_mul_g(g, u);
    } else {
      float v = 0.f;
      for (uint32_t y0 = 0; y0 < ks; y0 += RED_BATCH) {
        float t[RED_BATCH];
#pragma unroll
        for (uint32_t b = 0; b < RED_BATCH; b++) t[b] = y0 + b < ks ? ws[(y0 + b) * MN + o] : 0.f;
#pragma unroll
        for (uint32_t b = 0; b < RED_BATCH; b++)
          if (y0 + b < ks) v += t[b];
      }
      C[o] = epi == 1 ? R[o] + v : v;
    }
  }
}

// A16[m][k] = f16(A[m][k] * rms_m * gamma[k]) (gamma != null: RMSNorm,
// rmsnorm.metal:15-47) or f16(A[m][k]).  One row of A (blockIdx.x) to f16
// by 256 threads, in chunks of 8192
// elements: every load of a chunk is issued before the first is used, and a
// row of <= 8192 elements is read once (norm and conversion from registers).
// PERM: each thread takes 8 consecutive elements and writes them in the slot
// order {0,4,1,5,2,6,3,7}; else 4 consecutive elements.  K % 8 == 0.
template <bool PERM>
__device__ __forceinline__ void prep_a_row(const float* __restrict__ A, const float* __restrict__ gamma, float eps,
                                           _Float16* __restrict__ A16, uint32_t K) {
  constexpr uint32_t CH = 8192, U = 8;  // 8 float4 per thread per chunk
  __shared__ float red[4];
  const uint32_t m = blockIdx.x, tid = threadIdx.x;
  const float* a = A + (size_t)m * K;
  _Float16* d = A16 + (size_t)m * K;
  // element offset of float4 u of this thread within a chunk
  auto off = [&](uint32_t u) -> uint32_t { return PERM ? 8 * tid + 2048 * (u / 2) + 4 * (u % 2) : 4 * tid + 1024 * u; };
  float4 v[U];
  auto load = [&](uint32_t base) {
#pragma unroll
    for (uint32_t u = 0; u < U; u++) {
      const uint32_t k = base + off(u);
      v[u] = k < K ? *(const float4*)(a + k) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  auto store = [&](uint32_t base, float rms) {
    float4 g[U];
#pragma unroll
    for (uint32_t u = 0; u < U; u++) {
      const uint32_t k = base + off(u);
      g[u] = gamma && k < K ? *(const float4*)(gamma + k) : make_float4(1.f, 1.f, 1.f, 1.f);
    }
#pragma unroll
    for (uint32_t u = 0; u < U; u++) {
      v[u] = gamma ? make_float4(v[u].x * rms * g[u].x, v[u].y * rms * g[u].y, v[u].z * rms * g[u].z,
                                 v[u].w * rms * g[u].w)
                   : v[u];
    }
#pragma unroll
    for (uint32_t u = 0; u < U; u += PERM ? 2 : 1) {
      const uint32_t k = base + off(u);
      if (k >= K) continue;
      if (PERM) {  // slots (0,4) (1,5) (2,6) (3,7)
        uint4 o;
        o.x = pack_h2(v[u].x, v[u + 1].x);
        o.y = pack_h2(v[u].y, v[u + 1].y);
        o.z = pack_h2(v[u].z, v[u + 1].z);
        o.w = pack_h2(v[u].w, v[u + 1].w);
        *(uint4*)(d + k) = o;
      } else {
        uint2 o;
        o.x = pack_h2(v[u].x, v[u].y);
        o.y = pack_h2(v[u].z, v[u].w);
        *(uint2*)(d + k) = o;
      }
    }
  };
  auto sumsq = [&]() {
    float ss = 0.f;
#pragma unroll
    for (uint32_t u = 0; u < U; u++)
      ss = __builtin_fmaf(v[u].x, v[u].x,
                          __builtin_fmaf(v[u].y, v[u].y, __builtin_fmaf(v[u].z, v[u].z, __builtin_fmaf(v[u].w, v[u].w, ss))));
    return ss;
  };
  load(0);
  float rms = 1.f;
  if (gamma) {
    float ss = sumsq();
    for (uint32_t base = CH; base < K; base += CH) {  // rows past one chunk: a first pass for the norm
      load(base);
      ss += sumsq();
    }
    for (int dd = 32; dd >= 1; dd >>= 1) ss += __shfl_xor(ss, dd);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    rms = 1.0f / __builtin_sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)K + eps);
    if (K > CH) load(0);
  }
  for (uint32_t base = 0; base < K; base += CH) {
    if (base) load(base);
    store(base, rms);
  }
}

// smith_gemm_reduce fused with the next GEMM's activation prep: the K-split
// partials summed in split order with the epilogue (1: + residual, 2:
// SwiGLU of the (gate, up) column pairs) -- the same sums and epilogue as
// smith_gemm_reduce -- stored to C, and the output rows also written as the
// next GEMM's A operand: f16, each 8-element chunk in the slot order
// {0,4,1,5,2,6,3,7} (as smith_gemm_prep_a_perm).  Row length Kn = N (N / 2
// for SwiGLU), Kn % 8 == 0.  reduce_chunk8: one 8-output chunk of row m.
__device__ __forceinline__ void reduce_chunk8(const float* __restrict__ ws, uint32_t ks, size_t MN, uint32_t m,
                                              uint32_t N, const float* __restrict__ R, uint32_t epi, uint32_t k0,
                                              float v[8]) {
  const float* wr = ws + (size_t)m * N;
  if (epi == 2) {
    float4 a[4];
#pragma unroll
    for (int q = 0; q < 4; q++) a[q] = make_float4(0.f, 0.f, 0.f, 0.f);
    for (uint32_t z0 = 0; z0 < ks; z0 += RED_BATCH) {
      float4 t[RED_BATCH][4];
#pragma unroll
      for (uint32_t b = 0; b < RED_BATCH; b++)
#pragma unroll
        for (int q = 0; q < 4; q++)
          t[b][q] = z0 + b < ks ? *(const float4*)(wr + (z0 + b) * MN + 2 * k0 + 4 * q) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (uint32_t b = 0; b < RED_BATCH; b++)
        if (z0 + b < ks)
#pragma unroll
          for (int q = 0; q < 4; q++) {
            a[q].x += t[b][q].x;
            a[q].y += t[b][q].y;
            a[q].z += t[b][q].z;
            a[q].w += t[b][q].w;
          }
    }
#pragma unroll
    for (int q = 0; q < 4; q++) {
      v[2 * q] = silu_mul_g(a[q].x, a[q].y);
      v[2 * q + 1] = silu_mul_g(a[q].z, a[q].w);
    }
  } else {
    float4 a[2] = {make_float4(0.f, 0.f, 0.f, 0.f), make_float4(0.f, 0.f, 0.f, 0.f)};
    for (uint32_t z0 = 0; z0 < ks; z0 += RED_BATCH) {
      float4 t[RED_BATCH][2];
#pragma unroll
      for (uint32_t b = 0; b < RED_BATCH; b++)
#pragma unroll
        for (int q = 0; q < 2; q++)
          t[b][q] = z0 + b < ks ? *(const float4*)(wr + (z0 + b) * MN + k0 + 4 * q) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (uint32_t b = 0; b < RED_BATCH; b++)
        if (z0 + b < ks)
#pragma unroll
          for (int q = 0; q < 2; q++) {
            a[q].x += t[b][q].x;
            a[q].y += t[b][q].y;
            a[q].z += t[b][q].z;
            a[q].w += t[b][q].w;
          }
    }
    if (epi == 1) {
      const float4 r0 = *(const float4*)(R + (size_t)m * N + k0), r1 = *(const float4*)(R + (size_t)m * N + k0 + 4);
      a[0] = make_float4(r0.x + a[0].x, r0.y + a[0].y, r0.z + a[0].z, r0.w + a[0].w);
      a[1] = make_float4(r1.x + a[1].x, r1.y + a[1].y, r1.z + a[1].z, r1.w + a[1].w);
    }
    v[0] = a[0].x; v[1] = a[0].y; v[2] = a[0].z; v[3] = a[0].w;
    v[4] = a[1].x; v[5] = a[1].y; v[6] = a[1].z; v[7] = a[1].w;
  }
}

__device__ __forceinline__ uint4 perm_chunk8(const float v[8]) {
  uint4 o;
  o.x = pack_h2(v[0], v[4]);
  o.y = pack_h2(v[1], v[5]);
  o.z = pack_h2(v[2], v[6]);
  o.w = pack_h2(v[3], v[7]);
  return o;
}

// no norm: one 8-output chunk per thread over the whole M x Kn output
extern "C" __global__ __launch_bounds__(256) void smith_gemm_reduce_perm(
    const float* __restrict__ ws, uint32_t ks, float* __restrict__ C, uint32_t M, uint32_t N,
    const float* __restrict__ R, uint32_t epi, _Float16* __restrict__ A16) {
  const uint32_t Kn = epi == 2 ? N / 2 : N, cpr = Kn / 8;
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)M * cpr) return;
  const uint32_t m = (uint32_t)(idx / cpr), k0 = 8 * (uint32_t)(idx % cpr);
  float v[8];
  reduce_chunk8(ws, ks, (size_t)M * N, m, N, R, epi, k0, v);
  float* cr = C + (size_t)m * Kn + k0;
  *(float4*)cr = make_float4(v[0], v[1], v[2], v[3]);
  *(float4*)(cr + 4) = make_float4(v[4], v[5], v[6], v[7]);
  *(uint4*)(A16 + (size_t)m * Kn + k0) = perm_chunk8(v);
}

// with the next GEMM's RMSNorm (gamma): one row per 512-thread workgroup,
// at most 4 chunks of 8 per thread (Kn <= 16384), kept in registers across
// the row's sum of squares (gamma loaded before it); rsqrt(mean + eps) and
// x * rms * gamma as smith_gemm_prep_a_perm.
#define RP_MAXC 4
#define RP_NT 512
extern "C" __global__ __launch_bounds__(RP_NT) void smith_gemm_reduce_prep(
    const float* __restrict__ ws, uint32_t ks, float* __restrict__ C, uint32_t M, uint32_t N,
    const float* __restrict__ R, uint32_t epi, const float* __restrict__ gamma, float eps,
    _Float16* __restrict__ A16) {
  __shared__ float red[RP_NT / 64];
  const uint32_t m = blockIdx.x, tid = threadIdx.x;
  const uint32_t Kn = epi == 2 ? N / 2 : N;
  float* cr = C + (size_t)m * Kn;
  _Float16* ar = A16 + (size_t)m * Kn;
  float v[RP_MAXC][8], g[RP_MAXC][8];
  float ss = 0.f;
#pragma unroll
  for (int q = 0; q < RP_MAXC; q++) {
    const uint32_t k0 = 8 * (tid + RP_NT * q);
    if (k0 < Kn) {
      const float4 g0 = *(const float4*)(gamma + k0), g1 = *(const float4*)(gamma + k0 + 4);
      g[q][0] = g0.x; g[q][1] = g0.y; g[q][2] = g0.z; g[q][3] = g0.w;
      g[q][4] = g1.x; g[q][5] = g1.y; g[q][6] = g1.z; g[q][7] = g1.w;
      reduce_chunk8(ws, ks, (size_t)M * N, m, N, R, epi, k0, v[q]);
      *(float4*)(cr + k0) = make_float4(v[q][0], v[q][1], v[q][2], v[q][3]);
      *(float4*)(cr + k0 + 4) = make_float4(v[q][4], v[q][5], v[q][6], v[q][7]);
#pragma unroll
      for (int e = 0; e < 8; e++) ss = __builtin_fmaf(v[q][e], v[q][e], ss);
    }
  }
  for (int d = 32; d >= 1; d >>= 1) ss += __shfl_xor(ss, d);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < RP_NT / 64; w++) tot += red[w];
  const float rms = 1.0f / __builtin_sqrtf(tot / (float)Kn + eps);
#pragma unroll
  for (int q = 0; q < RP_MAXC; q++) {
    const uint32_t k0 = 8 * (tid + RP_NT * q);
    if (k0 < Kn) {
      float y[8];
#pragma unroll
      for (int e = 0; e < 8; e++) y[e] = v[q][e] * rms * g[q][e];
      *(uint4*)(ar + k0) = perm_chunk8(y);
    }
  }
}

extern "C" __global__ __launch_bounds__(256) void smith_gemm_prep_a(const float* __restrict__ A,
                                                                   const float* __restrict__ gamma, float eps,
                                                                   _Float16* __restrict__ A16, uint32_t K) {
  prep_a_row<false>(A, gamma, eps, A16, K);
}
