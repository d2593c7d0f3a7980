// smith_kernels.hip -- gfx950 (CDNA4) kernels for SMITH's quantized-weight
// matmul path.  Compiled to a code object (smith_kernels.hsaco) that the
// bridge loads with hipModuleLoad; every kernel is extern "C" so the bridge
// and the generic dispatch API can look it up by name.
//
// Formats (byte-exact with the reference):
//   Q4S  -- quantizeQ4 (src/ops/quantize.js:14-68): record (g,n) at
//           (g*N+n)*24: 16 nibble bytes (element k -> byte k>>1, low nibble
//           for even k), f32 scale at +16, f32 zero at +20;
//           w = scale*(nib - zero)                (shaders/matmul_q4.metal:24-28)
//   Q8   -- matmulQ8 blocks (shaders/matmul_q8.metal:40-52): block (g,n) at
//           (g*N+n)*34: f16 scale at +0, int8[32] at +2; w = f32(scale)*q
//   Q4_0 -- GGUF blocks (src/gguf.js:187-197) after the loader splits them
//           into planes without touching a byte: nibbles nib[(g*N+n)*16..]
//           and f16 scales d[g*N+n]; w = d*(nib - 8), interleaved nibbles.
//
// Decode GEMV (M <= 32) -- the HBM-bound hot path -- on
// v_mfma_f32_16x16x32_f16 with EXACT weights: nibbles / int8 become f16
// integers plus a known per-slot offset with one v_bfi_b32 (or v_perm_b32)
// per pair, using exponent-bias magic numbers (0x6400 -> 1024+q for a low
// nibble, 0x5400 -> 64+q for a high nibble, 1024+(q+128) for int8).
// Activations are split into f16 hi + f16 lo*2048 ("hi/lo", M <= 8) so the
// products keep ~22 bits of each f32 activation, or plain f16 (M > 8).  Per
// 32-K group and activation row the MFMA result P becomes the exact group
// contribution scale * (P - C1 - zero * S), with C1 = sum(a * offset) and
// S = sum(a), accumulated in f32; scale and zero never touch the f16 path.
// (smith_qgemv5 subtracts the offsets from the f16 operands instead -- exact
// -- and needs no C1.)
//   smith_qgemv1_*  M <= 2: activation prep fused (LDS), one kernel per call
//   smith_qgemv5_*  2 < M <= 32: per-wave activation prep, one launch
//   smith_qgemv3_*  2 < M <= 32: activations prepared once by smith_qprep_*
//                   (K % 32 != 0)
//   smith_qgemv4_*  2 < M <= 32: workgroup-shared prep (comparison path)
//   smith_agemv_*   M == 1 on an act (act_frag.h) its producer wrote
// Q4_0 weights for the decode path use tile-major planes (FMT_Q40T): the 16
// columns of a tile are contiguous over all of K, so a wave's records sit at
// fixed offsets from one base address.
// Split-K across workgroups (only when a block does not cover K) is reduced
// deterministically: partials go to a workspace through agent-scope atomic
// RMWs and the last-arriving workgroup of each column block sums them in
// fixed order (the counter self-resets).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "act_frag.h"
#include "splitk.h"

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
#include "gguf_tiles_dev.h"

#define FMT_Q4S 0
#define FMT_Q8 1
#define FMT_Q40 2
#define FMT_Q40T 3  // Q4_0 planes in column-tile-major order (16-column tiles)
__host__ __device__ constexpr bool is_q40(int f) { return f == FMT_Q40 || f == FMT_Q40T; }

// ---------------------------------------------------------------------------
// Reference-semantics kernels (one thread per output element).  They take the
// exact binding of the reference shaders -- A at slot 0, B at 1, C at 2, the
// {M,N,K,groups} u32 struct at 3 -- so the reference's quantize.js dispatch
// (run('matmul_q4', ..., grid {N,M}, group {16,16})) works unchanged through
// the generic encoder API.  The fast path is the smith_qgemv_* family below.
// ---------------------------------------------------------------------------
struct QMatmulParams {
  uint32_t M, N, K, groups;
};

extern "C" __global__ void matmul_q4(const float* __restrict__ A, const uint8_t* __restrict__ B,
                                     float* __restrict__ C, QMatmulParams p) {
  // Same math and accumulation order as shaders/matmul_q4.metal:34-65.
  uint32_t col = blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t row = blockIdx.y * blockDim.y + threadIdx.y;
  if (row >= p.M || col >= p.N) return;
  float acc = 0.0f;
  for (uint32_t g = 0; g < p.groups; g++) {
    const uint8_t* rec = B + ((size_t)g * p.N + col) * 24;
    float scale = *(const float*)(rec + 16);
    float zero = *(const float*)(rec + 20);
    for (uint32_t k = 0; k < 32 && g * 32 + k < p.K; k++) {
      uint8_t b = rec[k >> 1];
      float nib = (float)((k & 1) ? (b >> 4) : (b & 15));
      acc = __fadd_rn(acc, __fmul_rn(A[(size_t)row * p.K + g * 32 + k], __fmul_rn(scale, __fsub_rn(nib, zero))));
    }
  }
  C[(size_t)row * p.N + col] = acc;
}

extern "C" __global__ void matmul_q8(const float* __restrict__ A, const uint8_t* __restrict__ B,
                                     float* __restrict__ C, QMatmulParams p) {
  // Same math and accumulation order as shaders/matmul_q8.metal:20-57.
  uint32_t col = blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t row = blockIdx.y * blockDim.y + threadIdx.y;
  if (row >= p.M || col >= p.N) return;
  float acc = 0.0f;
  for (uint32_t g = 0; g < p.groups; g++) {
    const uint8_t* blk = B + ((size_t)g * p.N + col) * 34;
    uint16_t hbits = (uint16_t)(blk[0] | (blk[1] << 8));
    float scale = (float)__builtin_bit_cast(_Float16, hbits);
    const int8_t* v = (const int8_t*)(blk + 2);
    for (uint32_t k = 0; k < 32 && g * 32 + k < p.K; k++)
      acc = __fadd_rn(acc, __fmul_rn(A[(size_t)row * p.K + g * 32 + k], __fmul_rn(scale, (float)v[k])));
  }
  C[(size_t)row * p.N + col] = acc;
}

// ---------------------------------------------------------------------------
// quantizeQ4 on the GPU, bit-exact with src/ops/quantize.js:14-68.
// One thread per (group, column); f64 arithmetic with JavaScript's Math.max /
// Math.min / Math.round semantics and ToUint8 (NaN -> 0).
// ---------------------------------------------------------------------------
__device__ __forceinline__ double js_max(double a, double b) {
  if (a != a || b != b) return __builtin_nan("");
  if (a == 0.0 && b == 0.0) return __builtin_signbit(a) ? b : a;
  return a > b ? a : b;
}
__device__ __forceinline__ double js_min(double a, double b) {
  if (a != a || b != b) return __builtin_nan("");
  if (a == 0.0 && b == 0.0) return __builtin_signbit(a) ? a : b;
  return a < b ? a : b;
}
__device__ __forceinline__ uint32_t js_round_u8(double x) {
  // Math.round (ties toward +inf) followed by the Uint8Array store; x is
  // NaN or within [0, 15] here.
  if (x != x) return 0u;
  double r = __builtin_floor(x);
  if (__dsub_rn(x, r) >= 0.5) r = r + 1.0;
  return (uint32_t)(int32_t)r;
}

extern "C" __global__ void smith_quantize_q4s(const float* __restrict__ w, uint8_t* __restrict__ out,
                                              uint32_t K, uint32_t N) {
  uint32_t groups = (K + 31) / 32;
  size_t total = (size_t)groups * N;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
    uint32_t g = (uint32_t)(idx / N), col = (uint32_t)(idx % N);
    uint32_t k0 = g * 32;
    uint32_t valid = K - k0 < 32 ? K - k0 : 32;
    double mn = __builtin_inf(), mx = -__builtin_inf();
    for (uint32_t k = 0; k < valid; k++) {
      double v = (double)w[(size_t)(k0 + k) * N + col];
      if (v < mn) mn = v;
      if (v > mx) mx = v;
    }
    double range = __dsub_rn(mx, mn);
    double scale = range > 0 ? __ddiv_rn(range, 15.0) : 1.0;
    double zero = range > 0 ? __ddiv_rn(-mn, scale) : 8.0;
    uint32_t words[6];
#pragma unroll
    for (int d = 0; d < 4; d++) {
      uint32_t word = 0;
#pragma unroll
      for (int j = 0; j < 8; j++) {
        uint32_t k = d * 8 + j;
        double v = k < valid ? (double)w[(size_t)(k0 + k) * N + col] : 0.0;
        double t = __dadd_rn(__ddiv_rn(v, scale), zero);
        uint32_t q = js_round_u8(js_min(15.0, js_max(0.0, t)));
        word |= (q & 15u) << (4 * j);
      }
      words[d] = word;
    }
    words[4] = __float_as_uint(__double2float_rn(scale));
    words[5] = __float_as_uint(__double2float_rn(zero));
    uint32_t* rec = (uint32_t*)(out + idx * 24);
#pragma unroll
    for (int d = 0; d < 6; d++) rec[d] = words[d];
  }
}

// f32 -> f16 bits, IEEE round-to-nearest-even (ggml FP32_TO_FP16).
__device__ __forceinline__ uint16_t f32_to_f16_rne(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// Q8 blocks in matmul_q8.metal's layout, ggml q8_0 rounding: d = amax/127,
// q = roundf(x * (1/d)), scale stored as RNE f16.  Thread per (group, col).
extern "C" __global__ void smith_quantize_q8(const float* __restrict__ w, uint8_t* __restrict__ out,
                                             uint32_t K, uint32_t N) {
  uint32_t groups = (K + 31) / 32;
  size_t total = (size_t)groups * N;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
    uint32_t g = (uint32_t)(idx / N), col = (uint32_t)(idx % N);
    float x[32];
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < 32; k++) {
      uint32_t kk = g * 32 + k;
      x[k] = kk < K ? w[(size_t)kk * N + col] : 0.0f;
      float a = __builtin_fabsf(x[k]);
      amax = a > amax ? a : amax;
    }
    float d = __fdiv_rn(amax, 127.0f);
    float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    uint8_t* blk = out + idx * 34;
    uint16_t h = f32_to_f16_rne(d);
    // 34-byte records are only 2-byte aligned: write as 17 u16 halves.
    uint16_t* hp = (uint16_t*)blk;
    hp[0] = h;
#pragma unroll
    for (int k = 0; k < 32; k += 2) {
      int8_t q0 = (int8_t)__builtin_roundf(__fmul_rn(x[k], id));
      int8_t q1 = (int8_t)__builtin_roundf(__fmul_rn(x[k + 1], id));
      hp[1 + k / 2] = (uint16_t)((uint8_t)q0 | ((uint16_t)(uint8_t)q1 << 8));
    }
  }
}

// GGUF Q4_0 (ggml q4_0 rounding, reference's interleaved nibble order) for a
// row-major f32 [rows, cols] matrix, cols % 32 == 0.  Thread per block.
extern "C" __global__ void smith_quantize_q4_0_rows(const float* __restrict__ x, uint8_t* __restrict__ out,
                                                    uint32_t rows, uint32_t cols) {
  uint32_t bpr = cols / 32;
  size_t total = (size_t)rows * bpr;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
    const float* v = x + idx * 32;  // rows are contiguous, so block idx covers 32 floats
    float amax = 0.0f, mx = 0.0f;
    float xv[32];
#pragma unroll
    for (int i = 0; i < 32; i++) {
      xv[i] = v[i];
      float a = __builtin_fabsf(xv[i]);
      if (amax < a) { amax = a; mx = xv[i]; }
    }
    float d = __fdiv_rn(mx, -8.0f);
    float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    uint16_t* hp = (uint16_t*)(out + idx * 18);
    hp[0] = f32_to_f16_rne(d);
#pragma unroll
    for (int i = 0; i < 32; i += 2) {
      int q0 = (int)(int8_t)__fadd_rn(__fmul_rn(xv[i], id), 8.5f);
      int q1 = (int)(int8_t)__fadd_rn(__fmul_rn(xv[i + 1], id), 8.5f);
      q0 = q0 < 15 ? q0 : 15;
      q1 = q1 < 15 ? q1 : 15;
      ((uint8_t*)hp)[2 + i / 2] = (uint8_t)((q0 & 15) | ((q1 & 15) << 4));
    }
  }
}

// Split GGUF Q4_0 blocks of a weight listed [out=N][in=K] (block (n,g) at
// (n*G+g)*18) into the planar, column-interleaved layout the GEMV reads:
// nib[(g*Nt+col)*16 + 0..15] and d[g*Nt+col] with col = n_off + n*n_stride,
// so several weights can share one buffer (q|k|v side by side, gate/up
// interleaved).  Bytes are moved, never changed.
extern "C" __global__ void smith_repack_q4_0_cols(const uint8_t* __restrict__ src, uint8_t* __restrict__ nib,
                                                  uint16_t* __restrict__ dsc, uint32_t N, uint32_t G,
                                                  uint32_t n_off, uint32_t n_stride, uint32_t Nt) {
  size_t total = (size_t)N * G;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
    uint32_t n = (uint32_t)(idx / G), g = (uint32_t)(idx % G);
    const uint16_t* s = (const uint16_t*)(src + idx * 18);
    size_t o = (size_t)g * Nt + n_off + (size_t)n * n_stride;
    dsc[o] = s[0];
    uint16_t* dn = (uint16_t*)(nib + o * 16);
#pragma unroll
    for (int i = 0; i < 8; i++) dn[i] = s[1 + i];
  }
}

// Same, into the tile-major planes of FMT_Q40T: column col = n_off +
// n*n_stride of tile t = col/16 has record (g, col) at ((t*G + g)*16 + col%16)
// (16 nibble bytes each, f16 scale at the same index of dsc), so one 16-column
// tile is G*256 contiguous nibble bytes.
extern "C" __global__ void smith_repack_q4_0_tiles(const uint8_t* __restrict__ src, uint8_t* __restrict__ nib,
                                                   uint16_t* __restrict__ dsc, uint32_t N, uint32_t G,
                                                   uint32_t n_off, uint32_t n_stride) {
  size_t total = (size_t)N * G;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
    uint32_t n = (uint32_t)(idx / G), g = (uint32_t)(idx % G);
    const uint16_t* s = (const uint16_t*)(src + idx * 18);
    const uint32_t col = n_off + n * n_stride;
    size_t o = ((size_t)(col >> 4) * G + g) * 16 + (col & 15);
    dsc[o] = s[0];
    uint16_t* dn = (uint16_t*)(nib + o * 16);
#pragma unroll
    for (int i = 0; i < 8; i++) dn[i] = s[1 + i];
  }
}

// GGUF Q8_0 blocks of a weight listed [out=N][in=K] into matmulQ8's record
// order (shaders/matmul_q8.metal:40-52): record (g, col) at (g*Nt+col)*34,
// col = n_off + n*n_stride.  34-byte blocks, moved unchanged.
extern "C" __global__ void smith_repack_q8_0_cols(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                  uint32_t N, uint32_t G, uint32_t n_off, uint32_t n_stride,
                                                  uint32_t Nt) {
  size_t total = (size_t)N * G;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
    uint32_t n = (uint32_t)(idx / G), g = (uint32_t)(idx % G);
    const uint16_t* s = (const uint16_t*)(src + idx * 34);
    uint16_t* d = (uint16_t*)(dst + ((size_t)g * Nt + n_off + (size_t)n * n_stride) * 34);
#pragma unroll
    for (int i = 0; i < 17; i++) d[i] = s[i];
  }
}

// ---------------------------------------------------------------------------
// Activation preparation for the MFMA GEMV.
//   frag[(rb*G + g)*64 + lane]  u32x4 = the 8 f16 A-operand values of `lane`
//   cst [(rb*G + g)*16 + vrow]  float2 = (C1, S) of virtual row vrow
// Virtual rows of row block rb: HILO -> vrow r<8 is hi(row rb*8+r), vrow r>=8
// is lo(row rb*8+r-8)*2048; plain -> vrow r is row rb*16+r.  The f16 slots
// of a lane follow the B-operand conversion order of the weight format:
//   Q4 family: elements {0,4,1,5,2,6,3,7} of its 8-K slice, offsets
//              {1024,1024,64,64,1024,1024,64,64}
//   Q8:        elements {0,2,1,3,4,6,5,7}, offset 1152 everywhere
// C1 = sum(a*offset) (+ 8*S folded in for Q4_0, whose zero point is 8).
// Thread per (real row, group, kslice), kslice fastest.
// ---------------------------------------------------------------------------
template <int FMT, bool HILO>
__device__ __forceinline__ void qprep_body(const float* __restrict__ A, u32x4* __restrict__ frag,
                                           float2* __restrict__ cst, uint32_t M, uint32_t K, uint32_t G,
                                           uint32_t RB) {
  const uint32_t rows_per_rb = HILO ? 8 : 16;
  uint32_t tid = blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t kq = tid & 3;
  uint32_t rest = tid >> 2;
  uint32_t g = rest % G;
  uint32_t m = rest / G;  // padded real row, < RB*rows_per_rb
  bool active = m < RB * rows_per_rb;
  // slot -> element within the 8-K slice, and slot offsets
  const int perm_q4[8] = {0, 4, 1, 5, 2, 6, 3, 7};
  const int perm_q8[8] = {0, 2, 1, 3, 4, 6, 5, 7};
  const float off_q4[8] = {1024.f, 1024.f, 64.f, 64.f, 1024.f, 1024.f, 64.f, 64.f};
  float hi_c1 = 0.f, hi_s = 0.f, lo_c1 = 0.f, lo_s = 0.f;
  _Float16 hv[8], lv[8];
  // the slice's 8 elements, loaded together (two 16-byte loads when the
  // slice lies inside an aligned row) before any of them is converted
  float av[8];
  const uint32_t k0 = g * 32 + kq * 8;
  if (active && m < M && k0 + 8 <= K && K % 4 == 0) {
    const float4* ap = (const float4*)(A + (size_t)m * K + k0);
    const float4 x0 = ap[0], x1 = ap[1];
    av[0] = x0.x; av[1] = x0.y; av[2] = x0.z; av[3] = x0.w;
    av[4] = x1.x; av[5] = x1.y; av[6] = x1.z; av[7] = x1.w;
  } else {
#pragma unroll
    for (int e = 0; e < 8; e++) av[e] = (active && m < M && k0 + e < K) ? A[(size_t)m * K + k0 + e] : 0.0f;
  }
#pragma unroll
  for (int j = 0; j < 8; j++) {
    int e = FMT == FMT_Q8 ? perm_q8[j] : perm_q4[j];
    float off = FMT == FMT_Q8 ? 1152.f : off_q4[j];
    float a = av[e];
    _Float16 h = (_Float16)a;
    hv[j] = h;
    float hf = (float)h;
    hi_c1 = __builtin_fmaf(hf, off, hi_c1);
    hi_s += hf;
    if (HILO) {
      _Float16 l = (_Float16)((a - hf) * 2048.0f);
      lv[j] = l;
      float lf = (float)l;
      lo_c1 = __builtin_fmaf(lf, off, lo_c1);
      lo_s += lf;
    }
  }
  // reduce the four K slices of the group (lanes tid^1, tid^2 are the same
  // row/group because kq is the fastest index)
  hi_c1 = add_xor2(add_xor1(hi_c1));
  hi_s = add_xor2(add_xor1(hi_s));
  if (HILO) {
    lo_c1 = add_xor2(add_xor1(lo_c1));
    lo_s = add_xor2(add_xor1(lo_s));
  }
  if (!active) return;
  uint32_t rb = m / rows_per_rb, r = m % rows_per_rb;
  size_t fbase = ((size_t)rb * G + g) * 64;
  size_t cbase = ((size_t)rb * G + g) * 16;
  u32x4 hp;
  hp.x = __builtin_bit_cast(uint32_t, (_Float16 __attribute__((ext_vector_type(2)))){hv[0], hv[1]});
  hp.y = __builtin_bit_cast(uint32_t, (_Float16 __attribute__((ext_vector_type(2)))){hv[2], hv[3]});
  hp.z = __builtin_bit_cast(uint32_t, (_Float16 __attribute__((ext_vector_type(2)))){hv[4], hv[5]});
  hp.w = __builtin_bit_cast(uint32_t, (_Float16 __attribute__((ext_vector_type(2)))){hv[6], hv[7]});
  frag[fbase + r + 16 * kq] = hp;
  float fold = is_q40(FMT) ? 8.0f : 0.0f;
  if (kq == 0) cst[cbase + r] = make_float2(__builtin_fmaf(fold, hi_s, hi_c1), hi_s);
  if (HILO) {
    u32x4 lp;
    lp.x = __builtin_bit_cast(uint32_t, (_Float16 __attribute__((ext_vector_type(2)))){lv[0], lv[1]});
    lp.y = __builtin_bit_cast(uint32_t, (_Float16 __attribute__((ext_vector_type(2)))){lv[2], lv[3]});
    lp.z = __builtin_bit_cast(uint32_t, (_Float16 __attribute__((ext_vector_type(2)))){lv[4], lv[5]});
    lp.w = __builtin_bit_cast(uint32_t, (_Float16 __attribute__((ext_vector_type(2)))){lv[6], lv[7]});
    frag[fbase + r + 8 + 16 * kq] = lp;
    if (kq == 0) cst[cbase + r + 8] = make_float2(__builtin_fmaf(fold, lo_s, lo_c1), lo_s);
  }
}

#define DEF_QPREP(NAME, FMT, HILO)                                                                     \
  extern "C" __global__ __launch_bounds__(256) void NAME(const float* A, u32x4* frag, float2* cst,     \
                                                         uint32_t M, uint32_t K, uint32_t G,           \
                                                         uint32_t RB) {                                \
    qprep_body<FMT, HILO>(A, frag, cst, M, K, G, RB);                                                  \
  }
DEF_QPREP(smith_qprep_q4_hilo, FMT_Q4S, true)
DEF_QPREP(smith_qprep_q4_plain, FMT_Q4S, false)
DEF_QPREP(smith_qprep_q40_hilo, FMT_Q40, true)
DEF_QPREP(smith_qprep_q40_plain, FMT_Q40, false)
DEF_QPREP(smith_qprep_q8_hilo, FMT_Q8, true)
DEF_QPREP(smith_qprep_q8_plain, FMT_Q8, false)

// ---------------------------------------------------------------------------
// Epilogues shared by the GEMVs (the GGUF decode path fuses its elementwise
// ops into the projection that produces their input):
//   EPI_STORE   C[m][n] = v
//   EPI_RESID   C[m][n] = R[m][n] + v            (residual add, gguf_cache.js:159,171)
//   EPI_SWIGLU  columns hold interleaved (gate, up) pairs: C[m][n/2] =
//               silu(v[2j]) * v[2j+1] with silu(g) = g / (1 + exp(-g))
//               (shaders/swiglu.metal:12-21); C has N/2 columns.
// ---------------------------------------------------------------------------
#define EPI_STORE 0u
#define EPI_RESID 1u
#define EPI_SWIGLU 2u

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + __expf(-g)) * u; }

// Cross-workgroup split-K: this workgroup's partials are already in ws
// (agent-scope atomic exchanges); the last-arriving workgroup of the column
// block sums the ksplit partials in fixed order and applies the epilogue.
__device__ __forceinline__ void splitk_finish(float* __restrict__ ws, uint32_t* __restrict__ counters,
                                              float* __restrict__ C, const float* __restrict__ R, uint32_t epi,
                                              uint32_t M, uint32_t N, uint32_t mrows, uint32_t nb, uint32_t BC,
                                              uint32_t NT, uint32_t ksplit, int* s_last) {
  __builtin_amdgcn_s_waitcnt(0);  // every exchange of this thread has been performed
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t prev = __hip_atomic_fetch_add(counters + blockIdx.x, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *s_last = prev == ksplit - 1;
  }
  __syncthreads();
  if (!*s_last) return;
  auto part = [&](uint32_t m, uint32_t n) { return splitk_sum(ws + (size_t)m * N + n, (size_t)M * N, ksplit); };
  if (epi == EPI_SWIGLU) {
    for (uint32_t e = threadIdx.x; e < mrows * BC / 2; e += NT) {
      uint32_t m = e / (BC / 2), n = nb + 2 * (e % (BC / 2));
      if (n >= N) continue;
      C[(size_t)m * (N / 2) + n / 2] = silu_mul(part(m, n), part(m, n + 1));
    }
  } else {
    for (uint32_t e = threadIdx.x; e < mrows * BC; e += NT) {
      uint32_t m = e / BC, n = nb + e % BC;
      if (n >= N) continue;
      float v = part(m, n);
      C[(size_t)m * N + n] = epi == EPI_RESID ? R[(size_t)m * N + n] + v : v;
    }
  }
  if (threadIdx.x == 0)
    __hip_atomic_exchange(counters + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Decode GEMV for M <= 2 with the activation prep fused (no prep launch).
//
// Lane (c = lane%16, j = lane/16) loads the WHOLE weight record of column
// n0+c in group g0+4s+j with 128-bit loads, so the 16 lanes of a lane group
// read 16 consecutive records (one contiguous run).  Step s covers 4 groups
// (one per lane group) x 16 columns with 4 MFMAs: MFMA i consumes nibble
// dword i (K elements 8i..8i+7) of every lane.  The A operand is arranged so
// that MFMA row 4j+u only sees K slice j (lane group j), i.e. row 4j+u of P
// is the dot product of group g0+4s+j alone, and it lands in lane group j of
// the accumulator layout -- the lanes that hold that group's scale and zero.
// Rows u: 0 = hi(row 0), 1 = lo(row 0)*2048, 2 = hi(row 1), 3 = lo(row 1).
//
// The block issues all of its weight loads first, then loads its K range of
// the activations (and, with a fused RMSNorm, the full rows) and converts
// them into those f16 fragments in LDS (plus per-group C1 and S).  WK waves split the
// block's groups (reduced through LDS), WN waves sit side by side along N.
// Grid: x = column blocks of 16*CT*WN, y = K splits of 4*S*WK groups.
// ---------------------------------------------------------------------------
template <int FMT>
struct Rec {
  u32x4 q;        // Q4: 32 nibbles; Q8: raw dwords 0-3 of the record's 36 bytes
  u32x4 q8b;      // Q8: raw dwords 4-7
  uint32_t q8c;   // Q8: raw dword 8
  float s, z;     // Q4S: scale, zero as loaded
  uint32_t sb;    // Q4_0: the f16 scale's raw bits
  bool odd;       // Q8: the record starts at byte 2 of its first dword
  bool ok;        // record inside the weight (else its scale reads as 0)
};

// Every load result stays raw until its use: a select or conversion right
// where a record is loaded makes the wave wait for that load before it can
// issue the loads behind it (vector loads complete in order), and with
// everything converted at the point of use the waits fall where the data
// is needed.
template <int FMT>
__device__ __forceinline__ float rec_scale(const Rec<FMT>& r) {
  if (FMT == FMT_Q40 || FMT == FMT_Q40T)
    return r.ok ? (float)__builtin_bit_cast(_Float16, (uint16_t)r.sb) : 0.f;
  if (FMT == FMT_Q8)
    return r.ok ? (float)__builtin_bit_cast(_Float16, (uint16_t)(r.odd ? (r.q.x >> 16) : (r.q.x & 0xFFFFu))) : 0.f;
  return r.ok ? r.s : 0.f;
}

// Q8: the 8 dwords of int8 0..31.  At an aligned record the f16 scale is
// bytes 0-1 and the int8 start at byte 2; otherwise the scale is bytes 2-3
// and the int8 are raw dwords 1..8.
template <int FMT>
__device__ __forceinline__ void q8_dwords(const Rec<FMT>& r, uint32_t e[8]) {
  const uint32_t w[9] = {r.q.x, r.q.y, r.q.z, r.q.w, r.q8b.x, r.q8b.y, r.q8b.z, r.q8b.w, r.q8c};
#pragma unroll
  for (int q = 0; q < 8; q++) e[q] = r.odd ? w[q + 1] : __builtin_amdgcn_alignbyte(w[q + 1], w[q], 2);
}

template <int FMT>
__device__ __forceinline__ Rec<FMT> load_rec(const uint8_t* __restrict__ B, const uint16_t* __restrict__ D,
                                             uint32_t N, uint32_t G, uint32_t g, uint32_t n) {
  Rec<FMT> r;
  r.ok = g < G && n < N;
  size_t rec = (size_t)(g < G ? g : G - 1) * N + (n < N ? n : N - 1);
  r.z = 0.f;
  if (FMT == FMT_Q4S) {
    const uint8_t* p = B + rec * 24;
    r.q = *(const u32x4*)p;
    float2 sz = *(const float2*)(p + 16);
    r.s = sz.x;
    r.z = sz.y;
  } else if (FMT == FMT_Q40T) {
    // tile-major: the 16 columns of a tile, group after group, contiguous
    uint32_t nn = n < N ? n : N - 1, gg = g < G ? g : G - 1;
    rec = ((size_t)(nn >> 4) * G + gg) * 16 + (nn & 15);
    r.q = *(const u32x4*)(B + rec * 16);
    r.sb = D[rec];
  } else if (FMT == FMT_Q40) {
    r.q = *(const u32x4*)(B + rec * 16);
    r.sb = D[rec];
  } else {
    // the 36 bytes from the dword holding the record's first byte, in two
    // 128-bit loads + one dword (global loads need dword alignment only):
    // 3 load instructions per record (records are 2-byte aligned)
    const uint8_t* p = B + rec * 34;
    const size_t a = (size_t)p;
    // aligned down by pointer arithmetic on p (an integer-to-pointer cast
    // would lose the global address space: flat loads, which also count
    // against every LDS wait)
    const uint32_t* w = (const uint32_t*)(p - (a & 3));
    r.q = *(const u32x4*)w;
    r.q8b = *(const u32x4*)(w + 4);
    r.q8c = w[8];
    r.odd = (a & 3) != 0;
  }
  return r;
}

// Weight k of record (g, n) in f32, read byte by byte (0 outside the
// weight): nibble k in byte k / 2, low nibble first, for Q4S
// scale * (nibble - zero) (shaders/matmul_q4.metal:21-26) and Q4_0
// d * (nibble - 8) (src/gguf.js:187-197); Q8_0 d * int8 k.  Only the f32
// fallback of the GEMVs uses it (few registers, slow), not their MFMA path.
template <int FMT>
__device__ __forceinline__ float weight_at(const uint8_t* __restrict__ B, const uint16_t* __restrict__ D,
                                           uint32_t N, uint32_t G, uint32_t g, uint32_t n, uint32_t k) {
  if (g >= G || n >= N) return 0.f;
  if (FMT == FMT_Q8) {
    const uint8_t* p = B + ((size_t)g * N + n) * 34;
    const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(p[0] | (p[1] << 8)));
    return d * (float)(int8_t)p[2 + k];
  }
  size_t rec = (size_t)g * N + n;
  if (FMT == FMT_Q40T) rec = ((size_t)(n >> 4) * G + g) * 16 + (n & 15);
  const uint8_t* p = B + rec * (FMT == FMT_Q4S ? 24 : 16);
  const uint32_t byte = p[k >> 1];
  const float nib = (float)((k & 1) ? byte >> 4 : byte & 15u);
  if (FMT == FMT_Q4S) return *(const float*)(p + 16) * (nib - *(const float*)(p + 20));
  return (float)__builtin_bit_cast(_Float16, D[rec]) * (nib - 8.0f);
}

__device__ __forceinline__ bool finite_f32(float v) { return __builtin_fabsf(v) < __builtin_inff(); }

// f32 fallback of the GEMVs: sum over k of the groups [g0, g1) (within K)
// of a[m][k] (times rms * gamma[k] with an RMSNorm) * weight k of column n,
// in K order as the reference multiplies.  Taken only for a block sum that
// came out non-finite from the f16 operands (an activation beyond the f16
// range, or an infinite / NaN one); slow and small in registers.
template <int FMT>
__device__ __forceinline__ float f32_block_sum(const float* __restrict__ A, const uint8_t* __restrict__ B,
                                               const uint16_t* __restrict__ D, uint32_t N, uint32_t G, uint32_t K,
                                               uint32_t m, uint32_t n, uint32_t g0, uint32_t g1,
                                               const float* __restrict__ gamma, float rms) {
  const uint32_t k1 = g1 * 32 < K ? g1 * 32 : K;
  float d = 0.f;
#pragma unroll 1
  for (uint32_t k = g0 * 32; k < k1; k++) {
    float x = A[(size_t)m * K + k];
    if (gamma) x = x * rms * gamma[k];
    d = __builtin_fmaf(x, weight_at<FMT>(B, D, N, G, k / 32, n, k % 32), d);
  }
  return d;
}

// (x & mask) | (base & ~mask).  Plain C on purpose: the compiler's hazard
// recognizer does not see VALU work inside inline asm, and a v_bfi_b32
// written by asm into a dead lane of an in-flight MFMA's result was
// overwritten when the MFMA retired.
__device__ __forceinline__ uint32_t bfi(uint32_t mask, uint32_t x, uint32_t base) {
  return (x & mask) | (base & ~mask);
}

// B operand of MFMA i (K elements 8i..8i+7 of the record).
template <int FMT>
__device__ __forceinline__ half8 rec_to_f16(const Rec<FMT>& r, int i) {
  u32x4 u;
  if (FMT == FMT_Q8) {
    const uint32_t w[9] = {r.q.x, r.q.y, r.q.z, r.q.w, r.q8b.x, r.q8b.y, r.q8b.z, r.q8b.w, r.q8c};
    uint32_t x0 = (r.odd ? w[2 * i + 1] : __builtin_amdgcn_alignbyte(w[2 * i + 1], w[2 * i], 2)) ^ 0x80808080u;
    uint32_t x1 = (r.odd ? w[2 * i + 2] : __builtin_amdgcn_alignbyte(w[2 * i + 2], w[2 * i + 1], 2)) ^ 0x80808080u;
    u.x = __builtin_amdgcn_perm(0x64646464u, x0, 0x04020400u);
    u.y = __builtin_amdgcn_perm(0x64646464u, x0, 0x04030401u);
    u.z = __builtin_amdgcn_perm(0x64646464u, x1, 0x04020400u);
    u.w = __builtin_amdgcn_perm(0x64646464u, x1, 0x04030401u);
  } else {
    uint32_t x = i == 0 ? r.q.x : (i == 1 ? r.q.y : (i == 2 ? r.q.z : r.q.w));
    uint32_t y = x >> 8;
    u.x = bfi(0x000F000Fu, x, 0x64006400u);
    u.y = bfi(0x00F000F0u, x, 0x54005400u);
    u.z = bfi(0x000F000Fu, y, 0x64006400u);
    u.w = bfi(0x00F000F0u, y, 0x54005400u);
  }
  return __builtin_bit_cast(half8, u);
}

// PLAIN: the variant for plain matmuls (no RMSNorm prologue, plain store,
// no K split across blocks), without the code of those paths
// Q8C (Q8 records, N % 16 == 0, 16-byte aligned weight): each lane group
// reads the 544 contiguous bytes of its 16 records as 16-byte chunks (the
// records' own 36-byte windows at a 34-byte stride cost ~15 % of HBM rate
// at config 2) and the wave regroups them into records through a private
// LDS slice, which needs no barrier: one wave's LDS accesses run in order.
template <int FMT, int MR, int CT, int WK, int WN, int S, bool PLAIN = false, bool PS = false, bool Q8C = false>
__device__ __forceinline__ void qgemv1_body(const float* __restrict__ A, const uint8_t* __restrict__ B,
                                            const uint16_t* __restrict__ D, float* __restrict__ C,
                                            float* __restrict__ ws, uint32_t* __restrict__ counters,
                                            uint32_t M, uint32_t N, uint32_t K, uint32_t G,
                                            const float* __restrict__ gamma, float eps,
                                            const float* __restrict__ R, uint32_t epi) {
  constexpr int GPW = 4 * S;           // groups per wave (S steps of 4)
  constexpr int KB = GPW * WK;         // groups per block
  constexpr int BC = 16 * CT * WN;     // block columns
  constexpr int NT = 64 * WK * WN;     // threads
  // prep chunks (group, row, mfma slice) of one wave's own GPW groups: each
  // wave converts exactly the activations its MFMAs read, so the fragments
  // need only a wave-level barrier (no workgroup barrier before the MFMAs)
  constexpr int NCHW = GPW * MR * 4;
  constexpr int CPT = (NCHW + 63) / 64;
  __shared__ u32x4 fragL[KB][2 * MR][4];  // [group][row u][mfma i]
  __shared__ float2 cL[KB][MR];           // (C1, S) with hi + lo/2048 folded
  __shared__ float red[WK][MR][BC];
  __shared__ float nred[MR][WK * WN];
  __shared__ int s_last;
  __shared__ u32x4 q8L[Q8C ? WK * WN : 1][Q8C ? 4 * CT : 1][Q8C ? 34 : 1];  // [wave][run][chunk]

  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t wk = wave / WN, wn = wave % WN;
  const uint32_t c = lane & 15, j = lane >> 4;
  const uint32_t n0 = blockIdx.x * BC + wn * 16 * CT;
  const uint32_t gb = blockIdx.y * KB;
  const uint32_t gw = gb + wk * GPW;
  const uint32_t ksplit = PLAIN ? 1u : gridDim.y;
  if (PLAIN) {
    gamma = nullptr;
    R = nullptr;
    epi = EPI_STORE;
  }

  // 1. activation loads (small, cache resident) and the RMSNorm gammas go out
  //    BEFORE the weights: vector loads complete in order, so the prep below
  //    then waits only for these, not for the weight records behind them
  const int perm_q4[8] = {0, 4, 1, 5, 2, 6, 3, 7};
  const int perm_q8[8] = {0, 2, 1, 3, 4, 6, 5, 7};
  const float off_q4[8] = {1024.f, 1024.f, 64.f, 64.f, 1024.f, 1024.f, 64.f, 64.f};
  float av[CPT][8];
  float gv[CPT][8];
  if (gamma) {
#pragma unroll
    for (int cc = 0; cc < CPT; cc++) {
      uint32_t ch = lane + cc * 64;
      uint32_t i = ch & 3, gl = wk * GPW + (ch >> 2) / MR;
      uint32_t k0 = (gb + gl) * 32 + 8 * i;
      bool in = ch < (uint32_t)NCHW && k0 + 8 <= K;
      const float4* gp = (const float4*)(gamma + (in ? k0 : 0));
      float4 g0 = gp[0], g1 = gp[1];
      gv[cc][0] = g0.x; gv[cc][1] = g0.y; gv[cc][2] = g0.z; gv[cc][3] = g0.w;
      gv[cc][4] = g1.x; gv[cc][5] = g1.y; gv[cc][6] = g1.z; gv[cc][7] = g1.w;
    }
  }
#pragma unroll
  for (int cc = 0; cc < CPT; cc++) {
    uint32_t ch = lane + cc * 64;
    uint32_t i = ch & 3, m = (ch >> 2) % MR, gl = wk * GPW + (ch >> 2) / MR;
    uint32_t k0 = (gb + gl) * 32 + 8 * i;
    bool ok = ch < (uint32_t)NCHW && m < M && k0 + 8 <= K;
    if (ok) {
      const float4* ap = (const float4*)(A + (size_t)m * K + k0);
      float4 x0 = ap[0], x1 = ap[1];
      av[cc][0] = x0.x; av[cc][1] = x0.y; av[cc][2] = x0.z; av[cc][3] = x0.w;
      av[cc][4] = x1.x; av[cc][5] = x1.y; av[cc][6] = x1.z; av[cc][7] = x1.w;
    } else {
#pragma unroll
      for (int e = 0; e < 8; e++) {
        uint32_t k = k0 + e;
        av[cc][e] = (ch < (uint32_t)NCHW && m < M && k < K) ? A[(size_t)m * K + k] : 0.f;
      }
    }
  }

  // 2. weights: every record of this wave, all loads in flight.  The
  //    never-taken branches end basic blocks, which the instruction scheduler
  //    does not reorder across (it would otherwise wait for the activation
  //    loads before issuing the last records)
  if (K == 0xFFFFFFFFu) __builtin_amdgcn_s_sleep(1);
  Rec<FMT> wr[S][CT];
  u32x4 q8ch[Q8C ? S : 1][Q8C ? CT : 1][3];
  if constexpr (Q8C) {
    // run (group g, tile ct) = records n0 + 16 ct .. +15 of group g: 34
    // chunks; lane c takes chunks c, c + 16 and (c < 2) c + 32 -- the other
    // lanes repeat chunk c + 16 (the same line, so no extra HBM bytes)
#pragma unroll
    for (int st = 0; st < S; st++)
#pragma unroll
      for (int ct = 0; ct < CT; ct++) {
        const uint32_t g = gw + 4 * st + j, gc = g < G ? g : G - 1;
        const uint32_t nt = n0 + ct * 16 < N ? n0 + ct * 16 : N - 16;  // a tile past N: read in range, scale 0
        const u32x4* run = (const u32x4*)(B + ((size_t)gc * N + nt) * 34);
        q8ch[st][ct][0] = run[c];
        q8ch[st][ct][1] = run[c + 16];
        q8ch[st][ct][2] = run[c < 2 ? c + 32 : c + 16];
      }
  } else {
#pragma unroll
    for (int st = 0; st < S; st++)
#pragma unroll
      for (int ct = 0; ct < CT; ct++) wr[st][ct] = load_rec<FMT>(B, D, N, G, gw + 4 * st + j, n0 + ct * 16 + c);
  }
  if (K == 0xFFFFFFFEu) __builtin_amdgcn_s_sleep(1);

  // 3. optional RMSNorm prologue (gguf_cache.js:121 fused into the projection
  //    that consumes it): every workgroup sums x^2 over its rows' full K
  float nss[MR];
#pragma unroll
  for (int m = 0; m < MR; m++) nss[m] = 0.f;
  if (gamma) {
    // K % 32 == 0 on this path: float4 loads, all of a thread's issued together
#pragma unroll
    for (int m = 0; m < MR; m++)
      if ((uint32_t)m < M) {
        const float4* ar = (const float4*)(A + (size_t)m * K);
        for (uint32_t i = threadIdx.x; i < K / 4; i += NT) {
          float4 v = ar[i];
          nss[m] = __builtin_fmaf(v.x, v.x, __builtin_fmaf(v.y, v.y, __builtin_fmaf(v.z, v.z, __builtin_fmaf(v.w, v.w, nss[m]))));
        }
      }
  }

  // 4. activations -> f16 hi/lo fragments + (C1, S) in LDS
  float rms[MR];
#pragma unroll
  for (int m = 0; m < MR; m++) rms[m] = 1.0f;
  if (gamma) {
#pragma unroll
    for (int m = 0; m < MR; m++) {
      const float v = sum64_lanes(nss[m]);
      if (lane == 0) nred[m][wave] = v;
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < MR; m++) {
      float tot = 0.f;
      for (int w = 0; w < WK * WN; w++) tot += nred[m][w];
      rms[m] = 1.0f / __builtin_sqrtf(tot / (float)K + eps);
    }
#pragma unroll
    for (int cc = 0; cc < CPT; cc++) {
      uint32_t ch = lane + cc * 64;
      uint32_t i = ch & 3, m = (ch >> 2) % MR, gl = wk * GPW + (ch >> 2) / MR;
      uint32_t k0 = (gb + gl) * 32 + 8 * i;
      float r = 0.f;
#pragma unroll
      for (int q = 0; q < MR; q++) r = (uint32_t)q == m ? rms[q] : r;
#pragma unroll
      for (int e = 0; e < 8; e++) av[cc][e] = (k0 + e < K) ? av[cc][e] * r * gv[cc][e] : 0.f;
    }
  }
#pragma unroll
  for (int cc = 0; cc < CPT; cc++) {
    uint32_t ch = lane + cc * 64;
    uint32_t i = ch & 3, m = (ch >> 2) % MR, gl = wk * GPW + (ch >> 2) / MR;
    float c1h = 0.f, sh_ = 0.f, c1l = 0.f, sl = 0.f;
    _Float16 hv[8], lv[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
      int el = FMT == FMT_Q8 ? perm_q8[e] : perm_q4[e];
      float off = FMT == FMT_Q8 ? 1152.f : off_q4[e];
      float a = av[cc][el];
      _Float16 h = (_Float16)a;
      float hf = (float)h;
      _Float16 l = (_Float16)((a - hf) * 2048.0f);
      float lf = (float)l;
      hv[e] = h;
      lv[e] = l;
      c1h = __builtin_fmaf(hf, off, c1h);
      sh_ += hf;
      c1l = __builtin_fmaf(lf, off, c1l);
      sl += lf;
    }
    float c1 = __builtin_fmaf(c1l, 1.0f / 2048.0f, c1h);
    float sm = __builtin_fmaf(sl, 1.0f / 2048.0f, sh_);
    // the four mfma slices of (group, row) are adjacent threads
    c1 = add_xor2(add_xor1(c1));
    sm = add_xor2(add_xor1(sm));
    if (is_q40(FMT)) c1 = __builtin_fmaf(8.0f, sm, c1);
    if (ch < (uint32_t)NCHW) {
      u32x4 hp, lp;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        hp[q] = __builtin_bit_cast(uint32_t, (_Float16 __attribute__((ext_vector_type(2)))){hv[2 * q], hv[2 * q + 1]});
        lp[q] = __builtin_bit_cast(uint32_t, (_Float16 __attribute__((ext_vector_type(2)))){lv[2 * q], lv[2 * q + 1]});
      }
      fragL[gl][2 * m][i] = hp;
      fragL[gl][2 * m + 1][i] = lp;
      if (i == 0) cL[gl][m] = make_float2(c1, sm);
    }
  }
  // LDS operations of one wave complete in order
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // 5. MFMAs: lane (r = lane%16, j) feeds A row r from K slice j only
  const uint32_t r = lane & 15;
  const bool a_active = (r >> 2) == j && (r & 3) < 2 * MR;
  const uint32_t ru = r & 3;  // read by active lanes only
  float acc[CT][MR];
#pragma unroll
  for (int ct = 0; ct < CT; ct++)
#pragma unroll
    for (int m = 0; m < MR; m++) acc[ct][m] = 0.f;
  // A fragments of every step into registers first (PS: each step's right
  // before its MFMAs -- 48 fewer VGPRs, more workgroups resident per CU on
  // the wide matrices).  Only the 2*MR lanes per lane group whose MFMA row
  // carries an activation row read LDS (the exec-masked reads move 1/8 of
  // the bytes a read by all 64 lanes would); the rest hold zeros.
  u32x4 afr[PS ? 1 : S][4];
  if (!PS) {
#pragma unroll
    for (int st = 0; st < S; st++)
#pragma unroll
      for (int i = 0; i < 4; i++) afr[PS ? 0 : st][i] = (u32x4){0u, 0u, 0u, 0u};
    if (a_active) {
#pragma unroll
      for (int st = 0; st < S; st++)
#pragma unroll
        for (int i = 0; i < 4; i++) afr[PS ? 0 : st][i] = fragL[wk * GPW + 4 * st + j][ru][i];
    }
  }
#pragma unroll
  for (int st = 0; st < S; st++) {
    const uint32_t gl = wk * GPW + 4 * st + j;
    half8 af[4];
    if (PS) {
#pragma unroll
      for (int i = 0; i < 4; i++) afr[0][i] = (u32x4){0u, 0u, 0u, 0u};
      if (a_active)
#pragma unroll
        for (int i = 0; i < 4; i++) afr[0][i] = fragL[gl][ru][i];
    }
#pragma unroll
    for (int i = 0; i < 4; i++) af[i] = __builtin_bit_cast(half8, afr[PS ? 0 : st][i]);
    float2 cv[MR];
#pragma unroll
    for (int m = 0; m < MR; m++) cv[m] = cL[gl][m];
    if constexpr (Q8C) {
      // this step's chunks into the wave's slice, then each lane's record:
      // the 9 dwords from the one holding its first byte (byte 34 c of the run)
#pragma unroll
      for (int ct = 0; ct < CT; ct++) {
        u32x4* sl = q8L[wave][j * CT + ct];
        sl[c] = q8ch[st][ct][0];
        sl[c + 16] = q8ch[st][ct][1];
        if (c < 2) sl[c + 32] = q8ch[st][ct][2];
      }
#pragma unroll
      for (int ct = 0; ct < CT; ct++) {
        const uint32_t* w = (const uint32_t*)q8L[wave][j * CT + ct] + ((34 * c) >> 2);
        Rec<FMT>& rr = wr[st][ct];
        rr.q = (u32x4){w[0], w[1], w[2], w[3]};
        rr.q8b = (u32x4){w[4], w[5], w[6], w[7]};
        rr.q8c = w[8];
        rr.odd = (c & 1) != 0;
        const uint32_t g = gw + 4 * st + j, n = n0 + ct * 16 + c;
        rr.ok = g < G && n < N;
        rr.z = 0.f;
      }
    }
#pragma unroll
    for (int ct = 0; ct < CT; ct++) {
      f32x4 p = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < 4; i++)
        p = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], rec_to_f16<FMT>(wr[st][ct], i), p, 0, 0, 0);
      float s = rec_scale(wr[st][ct]), z = wr[st][ct].z;
#pragma unroll
      for (int m = 0; m < MR; m++) {
        float t = __builtin_fmaf(p[2 * m + 1], 1.0f / 2048.0f, p[2 * m]) - cv[m].x;
        if (FMT == FMT_Q4S) t = __builtin_fmaf(-z, cv[m].y, t);
        acc[ct][m] = __builtin_fmaf(s, t, acc[ct][m]);
      }
    }
  }

  // 6. sum the four lane groups (different K groups, same column), then the
  //    WK waves of the block in fixed order
#pragma unroll
  for (int ct = 0; ct < CT; ct++)
#pragma unroll
    for (int m = 0; m < MR; m++) {
      float v = acc[ct][m];
      v = add_xor32(add_xor16(v));
      if (j == 0) red[wk][m][wn * 16 * CT + ct * 16 + c] = v;
    }
  __syncthreads();
  const uint32_t nb = blockIdx.x * BC;
  const uint32_t mrows = M < (uint32_t)MR ? M : MR;
  // a non-finite block sum (an activation beyond the f16 range, |a| >=
  // 65520, or an infinite / NaN one) is recomputed in f32 over the block's
  // K range and stored again over the first store
  auto f32_sum = [&](uint32_t m, uint32_t n) {
    float r = 0.f;
#pragma unroll
    for (int q = 0; q < MR; q++) r = (uint32_t)q == m ? rms[q] : r;
    return f32_block_sum<FMT>(A, B, D, N, G, K, m, n, gb, gb + KB, gamma, r);
  };
  if (ksplit == 1) {
    if (epi == EPI_SWIGLU) {
      for (uint32_t e = threadIdx.x; e < mrows * BC / 2; e += NT) {
        uint32_t m = e / (BC / 2), cc = 2 * (e % (BC / 2)), n = nb + cc;
        float g = 0.f, u = 0.f;
#pragma unroll
        for (int w = 0; w < WK; w++) {
          g += red[w][m][cc];
          u += red[w][m][cc + 1];
        }
        if (n >= N) continue;
        C[(size_t)m * (N / 2) + n / 2] = silu_mul(g, u);
        if (!finite_f32(g) || !finite_f32(u)) C[(size_t)m * (N / 2) + n / 2] = silu_mul(f32_sum(m, n), f32_sum(m, n + 1));
      }
    } else {
      for (uint32_t e = threadIdx.x; e < mrows * BC; e += NT) {
        uint32_t m = e / BC, cc = e % BC, n = nb + cc;
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < WK; w++) v += red[w][m][cc];
        if (n >= N) continue;
        C[(size_t)m * N + n] = epi == EPI_RESID ? R[(size_t)m * N + n] + v : v;
        if (!finite_f32(v)) {
          v = f32_sum(m, n);
          C[(size_t)m * N + n] = epi == EPI_RESID ? R[(size_t)m * N + n] + v : v;
        }
      }
    }
    return;
  }
  for (uint32_t e = threadIdx.x; e < mrows * BC; e += NT) {
    uint32_t m = e / BC, cc = e % BC, n = nb + cc;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < WK; w++) v += red[w][m][cc];
    if (n >= N) continue;
    if (!finite_f32(v)) v = f32_sum(m, n);
    __hip_atomic_exchange((uint32_t*)ws + ((size_t)blockIdx.y * M + m) * N + n, __float_as_uint(v),
                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  splitk_finish(ws, counters, C, R, epi, M, N, mrows, nb, BC, NT, ksplit, &s_last);
}

#define DEF_QGEMV1(NAME, FMT, MR, CT, WK, WN, S, ...)                                                   \
  extern "C" __global__ __launch_bounds__(WK * WN * 64) void NAME(                                       \
      const float* A, const uint8_t* B, const uint16_t* D, float* C, float* ws, uint32_t* counters,      \
      uint32_t M, uint32_t N, uint32_t K, uint32_t G, const float* gamma, float eps, const float* R,     \
      uint32_t epi) {                                                                                    \
    qgemv1_body<FMT, MR, CT, WK, WN, S, ##__VA_ARGS__>(A, B, D, C, ws, counters, M, N, K, G, gamma, eps, R, \
                                                       epi);                                             \
  }

// ---------------------------------------------------------------------------
// Decode GEMV for 2 < M <= 32 (16-row MFMA layout, prepared activations).
//
// Loads are as in the fused kernel (lane (c, j) fetches the whole record of
// column c in group g+j with 128-bit loads); a 4x4 transpose of dwords across
// the four lane groups (v_permlane32_swap + v_permlane16_swap) then gives
// every lane (c, kq) dword kq of each of the four records, i.e. the
// K-slice layout of v_mfma_f32_16x16x32_f16 in which all 16 MFMA rows carry
// activation rows (8 hi/lo rows, or 16 plain rows, per row block).  The
// activation fragments and (C1, S) come from smith_qprep_* (one pass over A
// shared by every workgroup).  Scale / zero of group g+t reach all lanes of a
// column with ds_bpermute from lane group t.
// Grid: x = column blocks of 16*CT*WN, y = K splits of 4*S*WK groups.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void xpose4(uint32_t& x0, uint32_t& x1, uint32_t& x2, uint32_t& x3) {
  // in: lane group j holds X[j][0..3] in (x0..x3); out: lane group i holds X[0..3][i]
  // in (x0..x3), i.e. register t of lane group i = X[t][i].
  auto a = __builtin_amdgcn_permlane32_swap(x0, x2, false, false);
  auto b = __builtin_amdgcn_permlane32_swap(x1, x3, false, false);
  auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
  auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
  x0 = c[0];
  x1 = c[1];
  x2 = d[0];
  x3 = d[1];
}

template <int FMT, int RB, bool HILO, int VPL, int CT, int S, int WK, int WN>
__device__ __forceinline__ void qgemv3_body(const u32x4* __restrict__ frag, const float2* __restrict__ cst,
                                            const uint8_t* __restrict__ B, const uint16_t* __restrict__ D,
                                            float* __restrict__ C, float* __restrict__ ws,
                                            uint32_t* __restrict__ counters, uint32_t M, uint32_t N,
                                            uint32_t G, const float* __restrict__ R, uint32_t epi,
                                            const float* __restrict__ A, uint32_t K) {
  constexpr int GPW = 4 * S;
  constexpr int BC = 16 * CT * WN;
  constexpr int NT = 64 * WK * WN;
  __shared__ float red[WK][RB][16][BC];
  __shared__ int s_last;

  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t wk = wave / WN, wn = wave % WN;
  const uint32_t c = lane & 15, j = lane >> 4;
  const uint32_t n0 = blockIdx.x * BC + wn * 16 * CT;
  const uint32_t ksplit = gridDim.y;
  const uint32_t g0 = (blockIdx.y * WK + wk) * GPW;

  // activation fragments first (small, L2 resident): loads complete in
  // order, so the MFMAs of step st then wait only for the weights up to st
  u32x4 afr[S][4][RB];
  float4 cvv[S][4][RB][(VPL + 1) / 2];
#pragma unroll
  for (int st = 0; st < S; st++)
#pragma unroll
    for (int t = 0; t < 4; t++) {
      uint32_t g = g0 + 4 * st + t;
      g = g < G ? g : G - 1;
#pragma unroll
      for (int rb = 0; rb < RB; rb++) {
        afr[st][t][rb] = frag[((size_t)rb * G + g) * 64 + lane];
        const float4* cp = (const float4*)(cst + ((size_t)rb * G + g) * 16 + j * 4);
#pragma unroll
        for (int h = 0; h < (VPL + 1) / 2; h++) cvv[st][t][rb][h] = cp[h];
      }
    }

  Rec<FMT> wr[S][CT];
#pragma unroll
  for (int st = 0; st < S; st++)
#pragma unroll
    for (int ct = 0; ct < CT; ct++) wr[st][ct] = load_rec<FMT>(B, D, N, G, g0 + 4 * st + j, n0 + ct * 16 + c);

  f32x4 acc[CT][RB];
#pragma unroll
  for (int ct = 0; ct < CT; ct++)
#pragma unroll
    for (int rb = 0; rb < RB; rb++) acc[ct][rb] = (f32x4){0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int st = 0; st < S; st++)
#pragma unroll
    for (int ct = 0; ct < CT; ct++) {
      const Rec<FMT>& rr = wr[st][ct];
      // K-slice operands of the four records after the transpose
      half8 bf[4];
      if (FMT == FMT_Q8) {
        uint32_t e[8];
        q8_dwords(rr, e);
        xpose4(e[0], e[2], e[4], e[6]);
        xpose4(e[1], e[3], e[5], e[7]);
#pragma unroll
        for (int t = 0; t < 4; t++) {
          uint32_t x0 = e[2 * t] ^ 0x80808080u, x1 = e[2 * t + 1] ^ 0x80808080u;
          u32x4 u;
          u.x = __builtin_amdgcn_perm(0x64646464u, x0, 0x04020400u);
          u.y = __builtin_amdgcn_perm(0x64646464u, x0, 0x04030401u);
          u.z = __builtin_amdgcn_perm(0x64646464u, x1, 0x04020400u);
          u.w = __builtin_amdgcn_perm(0x64646464u, x1, 0x04030401u);
          bf[t] = __builtin_bit_cast(half8, u);
        }
      } else {
        uint32_t x[4] = {rr.q.x, rr.q.y, rr.q.z, rr.q.w};
        xpose4(x[0], x[1], x[2], x[3]);
#pragma unroll
        for (int t = 0; t < 4; t++) {
          uint32_t y = x[t] >> 8;
          u32x4 u;
          u.x = (x[t] & 0x000F000Fu) | 0x64006400u;
          u.y = (x[t] & 0x00F000F0u) | 0x54005400u;
          u.z = (y & 0x000F000Fu) | 0x64006400u;
          u.w = (y & 0x00F000F0u) | 0x54005400u;
          bf[t] = __builtin_bit_cast(half8, u);
        }
      }
      // scale / zero of record (group g+t, column c) from lane group t: the
      // same 4x4 lane-group transpose with every register holding the own value
      uint32_t sx[4], zx[4];
#pragma unroll
      for (int t = 0; t < 4; t++) {
        sx[t] = __float_as_uint(rec_scale(rr));
        zx[t] = __float_as_uint(rr.z);
      }
      xpose4(sx[0], sx[1], sx[2], sx[3]);
      if (FMT == FMT_Q4S) xpose4(zx[0], zx[1], zx[2], zx[3]);
#pragma unroll
      for (int t = 0; t < 4; t++) {
        float s = __uint_as_float(sx[t]);
        float z = FMT == FMT_Q4S ? __uint_as_float(zx[t]) : 0.f;
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
          f32x4 p = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, afr[st][t][rb]), bf[t],
                                                           (f32x4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < VPL; i++) {
            float4 c2 = cvv[st][t][rb][i >> 1];
            float c1 = (i & 1) ? c2.z : c2.x, sr = (i & 1) ? c2.w : c2.y;
            float tt = p[i] - c1;
            if (FMT == FMT_Q4S) tt = __builtin_fmaf(-z, sr, tt);
            acc[ct][rb][i] = __builtin_fmaf(s, tt, acc[ct][rb][i]);
          }
        }
      }
    }

#pragma unroll
  for (int ct = 0; ct < CT; ct++)
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
      for (int i = 0; i < 4; i++)
        red[wk][rb][j * 4 + i][wn * 16 * CT + ct * 16 + c] = i < VPL ? acc[ct][rb][i] : 0.f;
  __syncthreads();
  const uint32_t rows_per_rb = HILO ? 8 : 16;
  const uint32_t mrows = M < (uint32_t)(RB * rows_per_rb) ? M : RB * rows_per_rb;
  const uint32_t nb = blockIdx.x * BC;
  auto colsum = [&](uint32_t m, uint32_t cc) {
    uint32_t rb = m / rows_per_rb, rr = m % rows_per_rb;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < WK; w++) {
      if (HILO) v += red[w][rb][rr][cc] + red[w][rb][rr + 8][cc] * (1.0f / 2048.0f);
      else v += red[w][rb][rr][cc];
    }
    return v;
  };
  // a non-finite block sum (an activation beyond the f16 range, |a| >=
  // 65520, or an infinite / NaN one) is recomputed in f32 over the block's
  // K range from the activations the prep read, and stored again
  const uint32_t gb = blockIdx.y * WK * GPW;
  auto f32_sum = [&](uint32_t m, uint32_t n) {
    return f32_block_sum<FMT>(A, B, D, N, G, K, m, n, gb, gb + WK * GPW, nullptr, 1.0f);
  };
  if (ksplit == 1) {
    if (epi == EPI_SWIGLU) {
      for (uint32_t e = threadIdx.x; e < mrows * BC / 2; e += NT) {
        uint32_t m = e / (BC / 2), cc = 2 * (e % (BC / 2)), n = nb + cc;
        if (n >= N) continue;
        const float g = colsum(m, cc), u = colsum(m, cc + 1);
        C[(size_t)m * (N / 2) + n / 2] = silu_mul(g, u);
        if (!finite_f32(g) || !finite_f32(u)) C[(size_t)m * (N / 2) + n / 2] = silu_mul(f32_sum(m, n), f32_sum(m, n + 1));
      }
    } else {
      for (uint32_t e = threadIdx.x; e < mrows * BC; e += NT) {
        uint32_t m = e / BC, cc = e % BC, n = nb + cc;
        if (n >= N) continue;
        float v = colsum(m, cc);
        C[(size_t)m * N + n] = epi == EPI_RESID ? R[(size_t)m * N + n] + v : v;
        if (!finite_f32(v)) {
          v = f32_sum(m, n);
          C[(size_t)m * N + n] = epi == EPI_RESID ? R[(size_t)m * N + n] + v : v;
        }
      }
    }
    return;
  }
  for (uint32_t e = threadIdx.x; e < mrows * BC; e += NT) {
    uint32_t m = e / BC, cc = e % BC, n = nb + cc;
    if (n >= N) continue;
    float v = colsum(m, cc);
    if (!finite_f32(v)) v = f32_sum(m, n);
    __hip_atomic_exchange((uint32_t*)ws + ((size_t)blockIdx.y * M + m) * N + n, __float_as_uint(v),
                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  splitk_finish(ws, counters, C, R, epi, M, N, mrows, nb, BC, NT, ksplit, &s_last);
}

#define DEF_QGEMV3(NAME, FMT, RB, HILO, VPL, CT, S, WK, WN)                                             \
  extern "C" __global__ __launch_bounds__(WK * WN * 64) void NAME(                                       \
      const u32x4* frag, const float2* cst, const uint8_t* B, const uint16_t* D, float* C, float* ws,    \
      uint32_t* counters, uint32_t M, uint32_t N, uint32_t G, const float* R, uint32_t epi, const float* A, \
      uint32_t K) {                                                                                      \
    qgemv3_body<FMT, RB, HILO, VPL, CT, S, WK, WN>(frag, cst, B, D, C, ws, counters, M, N, G, R, epi, A, K); \
  }

// Fused M <= 2 variants, named by the groups one block covers: k64 = 4 waves
// x 4 steps, k96 / k128 / k288 = 8 waves x 3 / 4 / 9 steps (K = 3072, 4096,
// 9216 in one block), k448w16 = 16 waves x 7 steps (K = 14336 in one block,
// plain single-row matmuls only); _c2: two 16-column tiles per wave (wide N); _pl:
// plain matmuls; the _c2 and _pls variants read each step's A operands
// right before its MFMAs (fewer VGPRs: more workgroups per CU, for wide N).
#define DEF_QGEMV1_FMT(TAG, FMT)                                          \
  DEF_QGEMV1(smith_qgemv1_##TAG##_m1_k128, FMT, 1, 1, 8, 1, 4)            \
  DEF_QGEMV1(smith_qgemv1_##TAG##_m1_k128_pl, FMT, 1, 1, 8, 1, 4, true)   \
  DEF_QGEMV1(smith_qgemv1_##TAG##_m1_k128_pls, FMT, 1, 1, 8, 1, 4, true, true) \
  DEF_QGEMV1(smith_qgemv1_##TAG##_m1_k64_pl, FMT, 1, 1, 4, 1, 4, true)    \
  DEF_QGEMV1(smith_qgemv1_##TAG##_m1_k96_pl, FMT, 1, 1, 8, 1, 3, true)    \
  DEF_QGEMV1(smith_qgemv1_##TAG##_m1_k288_pl, FMT, 1, 1, 8, 1, 9, true)   \
  DEF_QGEMV1(smith_qgemv1_##TAG##_m1_k448w16_pl, FMT, 1, 1, 16, 1, 7, true, true) \
  DEF_QGEMV1(smith_qgemv1_##TAG##_m1_k96_c2_pl, FMT, 1, 2, 8, 1, 3, true, true) \
  DEF_QGEMV1(smith_qgemv1_##TAG##_m1_k128_c2_pl, FMT, 1, 2, 8, 1, 4, true, true) \
  DEF_QGEMV1(smith_qgemv1_##TAG##_m1_k64, FMT, 1, 1, 4, 1, 4)             \
  DEF_QGEMV1(smith_qgemv1_##TAG##_m1_k96, FMT, 1, 1, 8, 1, 3)             \
  DEF_QGEMV1(smith_qgemv1_##TAG##_m1_k288, FMT, 1, 1, 8, 1, 9)            \
  DEF_QGEMV1(smith_qgemv1_##TAG##_m1_k96_c2, FMT, 1, 2, 8, 1, 3, false, true) \
  DEF_QGEMV1(smith_qgemv1_##TAG##_m1_k128_c2, FMT, 1, 2, 8, 1, 4, false, true) \
  DEF_QGEMV1(smith_qgemv1_##TAG##_m2_k128, FMT, 2, 1, 8, 1, 4)            \
  DEF_QGEMV1(smith_qgemv1_##TAG##_m2_k64, FMT, 2, 1, 4, 1, 4)             \
  DEF_QGEMV1(smith_qgemv1_##TAG##_m2_k96, FMT, 2, 1, 8, 1, 3)             \
  DEF_QGEMV1(smith_qgemv1_##TAG##_m2_k288, FMT, 2, 1, 8, 1, 9)

// Q8 records read as contiguous 16-byte chunks (plain single-row matmuls
// with N % 16 == 0 on a 16-byte aligned weight)
#define DEF_QGEMV1_Q8C                                                                 \
  DEF_QGEMV1(smith_qgemv1_q8c_m1_k128_pl, FMT_Q8, 1, 1, 8, 1, 4, true, false, true)    \
  DEF_QGEMV1(smith_qgemv1_q8c_m1_k64_pl, FMT_Q8, 1, 1, 4, 1, 4, true, false, true)     \
  DEF_QGEMV1(smith_qgemv1_q8c_m1_k96_pl, FMT_Q8, 1, 1, 8, 1, 3, true, false, true)     \
  DEF_QGEMV1(smith_qgemv1_q8c_m1_k288_pl, FMT_Q8, 1, 1, 8, 1, 9, true, false, true)    \
  DEF_QGEMV1(smith_qgemv1_q8c_m1_k96_c2_pl, FMT_Q8, 1, 2, 8, 1, 3, true, true, true)   \
  DEF_QGEMV1(smith_qgemv1_q8c_m1_k128_c2_pl, FMT_Q8, 1, 2, 8, 1, 4, true, true, true)

// M > 2 row buckets (RB, HILO, VPL): m4 / m8 hi/lo, m16 / m32 plain f16;
// 2 column tiles x 1 step per wave, 8 waves split the block's 32 groups.
#define DEF_QGEMV3_FMT(TAG, FMT)                                          \
  DEF_QGEMV3(smith_qgemv3_##TAG##_m4, FMT, 1, true, 4, 2, 1, 8, 1)        \
  DEF_QGEMV3(smith_qgemv3_##TAG##_m8, FMT, 1, true, 4, 2, 1, 8, 1)        \
  DEF_QGEMV3(smith_qgemv3_##TAG##_m16, FMT, 1, false, 4, 2, 1, 8, 1)      \
  DEF_QGEMV3(smith_qgemv3_##TAG##_m32, FMT, 2, false, 4, 2, 1, 8, 1)      \
  DEF_QGEMV3(smith_qgemv3_##TAG##_m4_c1, FMT, 1, true, 4, 1, 1, 8, 1)     \
  DEF_QGEMV3(smith_qgemv3_##TAG##_m8_c1, FMT, 1, true, 4, 1, 1, 8, 1)     \
  DEF_QGEMV3(smith_qgemv3_##TAG##_m16_c1, FMT, 1, false, 4, 1, 1, 8, 1)   \
  DEF_QGEMV3(smith_qgemv3_##TAG##_m32_c1, FMT, 2, false, 4, 1, 1, 8, 1)

// The four records a lane group holds (groups g..g+3 of one column per
// lane) transposed into MFMA K slices: bf[t] is the B operand of group g+t,
// sv[t] / zv[t] its scale / zero for this lane's column.
template <int FMT>
__device__ __forceinline__ void rec_kslices(const Rec<FMT>& rr, half8 bf[4], uint32_t sv[4], uint32_t zv[4]) {
  if (FMT == FMT_Q8) {
    uint32_t e[8];
    q8_dwords(rr, e);
    xpose4(e[0], e[2], e[4], e[6]);
    xpose4(e[1], e[3], e[5], e[7]);
#pragma unroll
    for (int t = 0; t < 4; t++) {
      uint32_t x0 = e[2 * t] ^ 0x80808080u, x1 = e[2 * t + 1] ^ 0x80808080u;
      u32x4 u;
      u.x = __builtin_amdgcn_perm(0x64646464u, x0, 0x04020400u);
      u.y = __builtin_amdgcn_perm(0x64646464u, x0, 0x04030401u);
      u.z = __builtin_amdgcn_perm(0x64646464u, x1, 0x04020400u);
      u.w = __builtin_amdgcn_perm(0x64646464u, x1, 0x04030401u);
      bf[t] = __builtin_bit_cast(half8, u);
    }
  } else {
    uint32_t x[4] = {rr.q.x, rr.q.y, rr.q.z, rr.q.w};
    xpose4(x[0], x[1], x[2], x[3]);
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const uint32_t y = x[t] >> 8;
      u32x4 u;
      u.x = bfi(0x000F000Fu, x[t], 0x64006400u);
      u.y = bfi(0x00F000F0u, x[t], 0x54005400u);
      u.z = bfi(0x000F000Fu, y, 0x64006400u);
      u.w = bfi(0x00F000F0u, y, 0x54005400u);
      bf[t] = __builtin_bit_cast(half8, u);
    }
  }
  // scale (and zero) of group t for this lane's column: register t after
  // the same transpose of four copies
  const float rs = rec_scale(rr);
  sv[0] = sv[1] = sv[2] = sv[3] = __float_as_uint(rs);
  xpose4(sv[0], sv[1], sv[2], sv[3]);
  zv[0] = zv[1] = zv[2] = zv[3] = 0u;
  if (FMT == FMT_Q4S) {
    zv[0] = zv[1] = zv[2] = zv[3] = __float_as_uint(rr.z);
    xpose4(zv[0], zv[1], zv[2], zv[3]);
  }
}

// ---------------------------------------------------------------------------
// Batched decode GEMV for 2 < M <= 32 in ONE launch (activation prep fused).
//
// Workgroup (column block, K range): its 512 threads first load their share
// of A[rows, K range] (before any weight load: loads complete in order), then
// every wave issues all of its weight records (lane (c, j): the whole record
// of column c in group g+j, as in qgemv1/qgemv3), then the activations become
// MFMA A fragments in LDS -- virtual rows as in smith_qprep (hi/lo for M <= 8,
// plain f16 otherwise; per group and row C1 = sum(a*offset) (+8S for Q4_0)
// and S = sum(a)) -- shared by all waves of the block.  Per step a wave
// transposes its four records' dwords across lane groups (xpose4) into the
// K-slice B layout, so one v_mfma_f32_16x16x32_f16 per (group, row block)
// covers 16 columns x 16 virtual rows; the per-column scale / zero of the four
// groups reach every lane through the same transpose.  WK waves split the
// block's K range (LDS reduction); K splits across workgroups use the
// deterministic split-K finish.
// Grid: x = column blocks of 16*CT*WN, y = K splits of 4*S*WK groups.
// ---------------------------------------------------------------------------
template <int FMT, int RB, bool HILO, int CT, int S, int WK, int WN>
__device__ __forceinline__ void qgemv4_body(const float* __restrict__ A, const uint8_t* __restrict__ B,
                                            const uint16_t* __restrict__ D, float* __restrict__ C,
                                            float* __restrict__ ws, uint32_t* __restrict__ counters,
                                            uint32_t M, uint32_t N, uint32_t K, uint32_t G,
                                            const float* __restrict__ R, uint32_t epi) {
  constexpr int GPW = 4 * S;               // groups per wave
  constexpr int KB = GPW * WK;             // groups per block
  constexpr int BC = 16 * CT * WN;         // block columns
  constexpr int NT = 64 * WK * WN;         // threads
  constexpr int RPB = HILO ? 8 : 16;       // real rows per row block
  constexpr int NITEM = KB * RB * RPB * 4; // prep items (group, rb, row, kslice), kslice fastest
  constexpr int IPT = (NITEM + NT - 1) / NT;
  static_assert(NT % 4 == 0, "prep items of one (group, row) must share a quad of lanes");
  // the wave partials reuse the fragment area once every wave is past its MFMAs
  constexpr size_t FRAG_BYTES = sizeof(u32x4) * KB * RB * 64, RED_BYTES = sizeof(float) * WK * RB * 16 * BC;
  __shared__ __attribute__((aligned(16))) uint8_t smem[FRAG_BYTES > RED_BYTES ? FRAG_BYTES : RED_BYTES];
  __shared__ float4 cstL[KB][RB][8];       // (C1, S) of virtual rows 2q, 2q+1
  __shared__ int s_last;
  u32x4(*fragL)[RB][64] = reinterpret_cast<u32x4(*)[RB][64]>(smem);
  float(*red)[RB][16][BC] = reinterpret_cast<float(*)[RB][16][BC]>(smem);

  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t wk = wave / WN, wn = wave % WN;
  const uint32_t c = lane & 15, j = lane >> 4;
  const uint32_t n0 = blockIdx.x * BC + wn * 16 * CT;
  const uint32_t gb = blockIdx.y * KB;
  const uint32_t gw = gb + wk * GPW;
  const uint32_t ksplit = gridDim.y;

  // 1. activation loads of this block's K range (K % 32 == 0 on this
  //    path): unconditional 16-byte loads from a clamped address, dead
  //    items zeroed where they are converted
  float av[IPT][8];
  bool alive[IPT];
#pragma unroll
  for (int it = 0; it < IPT; it++) {
    const uint32_t item = threadIdx.x + it * NT;
    const uint32_t kq = item & 3, rest = item >> 2;
    const uint32_t r = rest % RPB, rb = (rest / RPB) % RB, gl = rest / (RPB * RB);
    const uint32_t m = rb * RPB + r;
    const uint32_t k0 = (gb + gl) * 32 + 8 * kq;
    alive[it] = item < (uint32_t)NITEM && m < M && k0 < K;
    const float4* ap = (const float4*)(A + (alive[it] ? (size_t)m * K + k0 : 0));
    float4 x0 = ap[0], x1 = ap[1];
    av[it][0] = x0.x; av[it][1] = x0.y; av[it][2] = x0.z; av[it][3] = x0.w;
    av[it][4] = x1.x; av[it][5] = x1.y; av[it][6] = x1.z; av[it][7] = x1.w;
  }

  // 2. weight records of this wave, all loads in flight.  The never-taken
  //    branches on either side end basic blocks, which the instruction
  //    scheduler does not reorder across: it would otherwise interleave the
  //    conversion below (and its wait for the activation loads) with, or
  //    ahead of, the weight loads
  if (K == 0xFFFFFFFFu) __builtin_amdgcn_s_sleep(1);
  Rec<FMT> wr[S][CT];
#pragma unroll
  for (int st = 0; st < S; st++)
#pragma unroll
    for (int ct = 0; ct < CT; ct++) wr[st][ct] = load_rec<FMT>(B, D, N, G, gw + 4 * st + j, n0 + ct * 16 + c);
  if (K == 0xFFFFFFFEu) __builtin_amdgcn_s_sleep(1);

  // 3. activations -> f16 fragments and (C1, S) in LDS
  {
    const int perm_q4[8] = {0, 4, 1, 5, 2, 6, 3, 7};
    const int perm_q8[8] = {0, 2, 1, 3, 4, 6, 5, 7};
    const float off_q4[8] = {1024.f, 1024.f, 64.f, 64.f, 1024.f, 1024.f, 64.f, 64.f};
    const float fold = is_q40(FMT) ? 8.0f : 0.0f;
    float* cst1 = (float*)&cstL[0][0][0];
#pragma unroll
    for (int it = 0; it < IPT; it++) {
      const uint32_t item = threadIdx.x + it * NT;
      const uint32_t kq = item & 3, rest = item >> 2;
      const uint32_t r = rest % RPB, rb = (rest / RPB) % RB, gl = rest / (RPB * RB);
      float c1h = 0.f, sh_ = 0.f, c1l = 0.f, sl = 0.f;
      _Float16 hv[8], lv[8];
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const int el = FMT == FMT_Q8 ? perm_q8[e] : perm_q4[e];
        const float off = FMT == FMT_Q8 ? 1152.f : off_q4[e];
        const float a = alive[it] ? av[it][el] : 0.f;
        const _Float16 h = (_Float16)a;
        const float hf = (float)h;
        hv[e] = h;
        c1h = __builtin_fmaf(hf, off, c1h);
        sh_ += hf;
        if (HILO) {
          const _Float16 l = (_Float16)((a - hf) * 2048.0f);
          const float lf = (float)l;
          lv[e] = l;
          c1l = __builtin_fmaf(lf, off, c1l);
          sl += lf;
        }
      }
      c1h = add_xor2(add_xor1(c1h));
      sh_ = add_xor2(add_xor1(sh_));
      if (HILO) {
        c1l = add_xor2(add_xor1(c1l));
        sl = add_xor2(add_xor1(sl));
      }
      if (item < (uint32_t)NITEM) {
        u32x4 hp, lp;
#pragma unroll
        for (int q = 0; q < 4; q++) {
          hp[q] = __builtin_bit_cast(uint32_t, (_Float16 __attribute__((ext_vector_type(2)))){hv[2 * q], hv[2 * q + 1]});
          if (HILO)
            lp[q] = __builtin_bit_cast(uint32_t, (_Float16 __attribute__((ext_vector_type(2)))){lv[2 * q], lv[2 * q + 1]});
        }
        fragL[gl][rb][r + 16 * kq] = hp;
        if (HILO) fragL[gl][rb][r + 8 + 16 * kq] = lp;
        float* cp = cst1 + ((size_t)gl * RB + rb) * 32;  // 16 virtual rows x (C1, S)
        if (kq == 0) {
          cp[2 * r] = __builtin_fmaf(fold, sh_, c1h);
          cp[2 * r + 1] = sh_;
        }
        if (HILO && kq == 1) {
          cp[2 * (r + 8)] = __builtin_fmaf(fold, sl, c1l);
          cp[2 * (r + 8) + 1] = sl;
        }
      }
    }
  }
  __syncthreads();

  // 4. MFMAs: per step, the four groups' records transposed into K slices
  f32x4 acc[CT][RB];
#pragma unroll
  for (int ct = 0; ct < CT; ct++)
#pragma unroll
    for (int rb = 0; rb < RB; rb++) acc[ct][rb] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int st = 0; st < S; st++) {
    const uint32_t gl0 = wk * GPW + 4 * st;
    half8 af[4][RB];
    float4 cv[4][RB][2];
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
      for (int rb = 0; rb < RB; rb++) {
        af[t][rb] = __builtin_bit_cast(half8, fragL[gl0 + t][rb][lane]);
        cv[t][rb][0] = cstL[gl0 + t][rb][2 * j];
        cv[t][rb][1] = cstL[gl0 + t][rb][2 * j + 1];
      }
#pragma unroll
    for (int ct = 0; ct < CT; ct++) {
      const Rec<FMT>& rr = wr[st][ct];
      half8 bf[4];
      uint32_t sv[4], zv[4];
      rec_kslices<FMT>(rr, bf, sv, zv);
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const float s = __uint_as_float(sv[t]), z = __uint_as_float(zv[t]);
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
          const f32x4 p = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[t][rb], bf[t], (f32x4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
          const float4 c01 = cv[t][rb][0], c23 = cv[t][rb][1];
          const float c1v[4] = {c01.x, c01.z, c23.x, c23.z}, sv4[4] = {c01.y, c01.w, c23.y, c23.w};
#pragma unroll
          for (int i = 0; i < 4; i++) {
            float tt = p[i] - c1v[i];
            if (FMT == FMT_Q4S) tt = __builtin_fmaf(-z, sv4[i], tt);
            acc[ct][rb][i] = __builtin_fmaf(s, tt, acc[ct][rb][i]);
          }
        }
      }
    }
  }

  // 5. the WK waves of the block in fixed order, then the epilogue or the
  //    cross-block split
  __syncthreads();
#pragma unroll
  for (int ct = 0; ct < CT; ct++)
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
      for (int i = 0; i < 4; i++) red[wk][rb][j * 4 + i][wn * 16 * CT + ct * 16 + c] = acc[ct][rb][i];
  __syncthreads();
  const uint32_t mrows = M < (uint32_t)(RB * RPB) ? M : RB * RPB;
  const uint32_t nb = blockIdx.x * BC;
  auto colsum = [&](uint32_t m, uint32_t cc) {
    const uint32_t rb = m / RPB, rr = m % RPB;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < WK; w++) {
      if (HILO) v += red[w][rb][rr][cc] + red[w][rb][rr + 8][cc] * (1.0f / 2048.0f);
      else v += red[w][rb][rr][cc];
    }
    return v;
  };
  if (ksplit == 1) {
    if (epi == EPI_SWIGLU) {
      for (uint32_t e = threadIdx.x; e < mrows * BC / 2; e += NT) {
        const uint32_t m = e / (BC / 2), cc = 2 * (e % (BC / 2)), n = nb + cc;
        if (n < N) C[(size_t)m * (N / 2) + n / 2] = silu_mul(colsum(m, cc), colsum(m, cc + 1));
      }
    } else {
      for (uint32_t e = threadIdx.x; e < mrows * BC; e += NT) {
        const uint32_t m = e / BC, cc = e % BC, n = nb + cc;
        if (n >= N) continue;
        const float v = colsum(m, cc);
        C[(size_t)m * N + n] = epi == EPI_RESID ? R[(size_t)m * N + n] + v : v;
      }
    }
    return;
  }
  for (uint32_t e = threadIdx.x; e < mrows * BC; e += NT) {
    const uint32_t m = e / BC, cc = e % BC, n = nb + cc;
    if (n >= N) continue;
    __hip_atomic_exchange((uint32_t*)ws + ((size_t)blockIdx.y * M + m) * N + n, __float_as_uint(colsum(m, cc)),
                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  splitk_finish(ws, counters, C, R, epi, M, N, mrows, nb, BC, NT, ksplit, &s_last);
}

#define DEF_QGEMV4(NAME, FMT, RB, HILO, CT, S, WK, WN)                                                  \
  extern "C" __global__ __launch_bounds__(WK * WN * 64) void NAME(                                       \
      const float* A, const uint8_t* B, const uint16_t* D, float* C, float* ws, uint32_t* counters,      \
      uint32_t M, uint32_t N, uint32_t K, uint32_t G, const float* R, uint32_t epi) {                    \
    qgemv4_body<FMT, RB, HILO, CT, S, WK, WN>(A, B, D, C, ws, counters, M, N, K, G, R, epi);             \
  }

// Row buckets h8 (M <= 8, hi/lo), p16 (M <= 16), p32 (M <= 32, two row
// blocks); k32 / k16 = groups per block (64 columns per block, 8 waves:
// 2 along K x 4 along N).  (Blocks over all of K = 4096 with 16 columns lost:
// every block then converts the whole activation, 11.7 vs 9.4 us at M = 4.)
#define DEF_QGEMV4_FMT(TAG, FMT)                                         \
  DEF_QGEMV4(smith_qgemv4_##TAG##_h8_k32, FMT, 1, true, 1, 4, 2, 4)      \
  DEF_QGEMV4(smith_qgemv4_##TAG##_h8_k16, FMT, 1, true, 1, 2, 2, 4)      \
  DEF_QGEMV4(smith_qgemv4_##TAG##_h8_k32_n32, FMT, 1, true, 1, 2, 4, 2)  \
  DEF_QGEMV4(smith_qgemv4_##TAG##_h8_k16_n32, FMT, 1, true, 1, 1, 4, 2)  \
  DEF_QGEMV4(smith_qgemv4_##TAG##_p16_k32, FMT, 1, false, 1, 4, 2, 4)    \
  DEF_QGEMV4(smith_qgemv4_##TAG##_p16_k16, FMT, 1, false, 1, 2, 2, 4)    \
  DEF_QGEMV4(smith_qgemv4_##TAG##_p32_k32, FMT, 2, false, 1, 4, 2, 4)    \
  DEF_QGEMV4(smith_qgemv4_##TAG##_p32_k16, FMT, 2, false, 1, 2, 2, 4)

// ---------------------------------------------------------------------------
// Batched decode GEMV for 2 < M <= 16 in ONE launch, each wave preparing
// only the activations its own MFMAs read.
//
// The MFMA scheme is qgemv4's (records transposed into K slices, all 16 MFMA
// rows carrying activation rows: hi rows 0-7 + lo rows 8-15 for M <= 8, or
// 16 plain f16 rows), but the activation prep is qgemv1's: a wave loads the
// MR rows of its own 4*S groups first (before its weight records: loads
// complete in order), converts them into its private slice of LDS and needs
// only a wave barrier before its MFMAs.  A block of WK waves covers 4*S*WK
// groups -- all of K when that fits, so the usual shapes need no cross-block
// reduction.  Lanes whose MFMA row is past the bucket's MR rows feed zeros
// from registers; LDS holds only the MR live rows:
//   fragL[group][kslice][vrow], vrow = m (hi or plain) or MR + m (lo).
// The record operands have their exponent-bias offsets subtracted in f16
// (exact; for Q4_0 its zero point 8 too), so the MFMA yields sum(a * q)
// (Q4_0: sum(a * (q - 8))); Q4S needs the per-(group, row) sums S =
// sum(a) of the f16 operand values for its zero term: for the hi/lo rows
// (M <= 8) formed during the conversion (v_dot2_f32_f16 against ones over a
// lane's 8 values, then the lane quad of the row's four K slices by DPP) and
// kept in LDS, where each lane reads the four of its output rows with one
// broadcast load; for plain rows from one more MFMA per group against a
// ones column, read by every lane with a DPP row broadcast.  The conversion
// is the f16 rounding (v_cvt_pk_f16_f32, and one fused multiply-add per
// element for the lo half) and those sums.
// Grid: x = column blocks of 16*CT, y = K splits of 4*S*WK groups.
// ---------------------------------------------------------------------------

template <int FMT, int MR, bool HILO, int CT, int S, int WK>
__device__ __forceinline__ void qgemv5_body(const float* __restrict__ A, const uint8_t* __restrict__ B,
                                            const uint16_t* __restrict__ D, float* __restrict__ C,
                                            float* __restrict__ ws, uint32_t* __restrict__ counters,
                                            uint32_t M, uint32_t N, uint32_t K, uint32_t G,
                                            const float* __restrict__ R, uint32_t epi) {
  constexpr int GPW = 4 * S;               // groups per wave
  constexpr int KB = GPW * WK;             // groups per block
  constexpr int BC = 16 * CT;              // block columns
  constexpr int NT = 64 * WK;              // threads
  constexpr int RPB = HILO ? 8 : 16;       // activation rows per MFMA row block
  constexpr int RB = (MR + RPB - 1) / RPB; // MFMA row blocks
  static_assert(!HILO || RB == 1, "hi/lo rows fit one row block");
  static_assert(RB <= 2, "at most two row blocks");
  constexpr int VR = HILO ? 2 * MR : MR;   // live virtual rows
  // Q4S: - zero * S; Q4_0's zero point 8 comes off with the f16 offsets
  // (exact), so only Q4S needs the sums
  constexpr bool NEED_S = FMT == FMT_Q4S;
  // hi/lo rows: S formed during the conversion and kept in LDS; plain rows:
  // S from one more MFMA per group against a ones column (same-box A/B: the
  // LDS sums took M = 4 from 6.31 to 5.99 us at 4096 x 4096, but made the
  // plain M = 16 / 32 buckets, with 2-4x the conversion work, 2-6 % slower)
  constexpr bool SUM_LDS = NEED_S && HILO;
  constexpr int NITEM = GPW * MR * 4;      // prep items of a wave (group, row, kslice), kslice fastest
  constexpr int IPT = (NITEM + 63) / 64;
  __shared__ u32x4 fragL[KB][4][VR];
  // per (group, MFMA row) sum of the f16 operand values of that row (the S of
  // the zero term, hi/lo buckets): hi row m at m, lo row m at 8 + m
  __shared__ __attribute__((aligned(16))) float sL[SUM_LDS ? KB : 1][16 * RB];
  // when the fragments and a separate reduction array would not fit the
  // LDS (16 waves x 32 rows), or would keep a second workgroup off the CU
  // while the fragments alone leave room for it (8 waves x 32 rows: 80 /
  // 128 -> 64 KB at 16 / 64 columns), the reduction reuses the fragments
  // after a block barrier
  constexpr size_t RED_BYTES = sizeof(float) * WK * 16 * RB * BC;
  constexpr bool ALIAS = sizeof(fragL) + RED_BYTES > 150 * 1024 ||
                         (sizeof(fragL) + RED_BYTES >= 80 * 1024 && sizeof(fragL) <= 72 * 1024);
  static_assert(!ALIAS || sizeof(fragL) >= RED_BYTES, "reduction fits the fragments");
  __shared__ float red_own[ALIAS ? 1 : WK][ALIAS ? 1 : 16 * RB][BC];
  float(*red)[16 * RB][BC] = ALIAS ? (float(*)[16 * RB][BC])(void*)fragL : (float(*)[16 * RB][BC])red_own;
  __shared__ int s_last;

  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wk = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t c = lane & 15, j = lane >> 4;
  const uint32_t n0 = blockIdx.x * BC;
  const uint32_t gb = blockIdx.y * KB;
  const uint32_t gw = gb + wk * GPW;
  const uint32_t ksplit = gridDim.y;

  // 1. this wave's activations (K % 32 == 0 on this path): unconditional
  //    16-byte loads from a clamped address, dead items zeroed where they
  //    are converted
  float av[IPT][8];
  bool alive[IPT];
#pragma unroll
  for (int it = 0; it < IPT; it++) {
    const uint32_t item = lane + it * 64;
    const uint32_t kq = item & 3, m = (item >> 2) % MR, gl = (item >> 2) / MR;
    const uint32_t k0 = (gw + gl) * 32 + 8 * kq;
    alive[it] = item < (uint32_t)NITEM && m < M && k0 < K;
    const float4* ap = (const float4*)(A + (alive[it] ? (size_t)m * K + k0 : 0));
    float4 x0 = ap[0], x1 = ap[1];
    av[it][0] = x0.x; av[it][1] = x0.y; av[it][2] = x0.z; av[it][3] = x0.w;
    av[it][4] = x1.x; av[it][5] = x1.y; av[it][6] = x1.z; av[it][7] = x1.w;
  }

  // 2. weight records of this wave, all loads in flight.  The never-taken
  //    branches on either side end basic blocks, which the instruction
  //    scheduler does not reorder across: it would otherwise interleave the
  //    conversion below (and its wait for the activation loads) with, or
  //    ahead of, the weight loads
  if (K == 0xFFFFFFFFu) __builtin_amdgcn_s_sleep(1);
  Rec<FMT> wr[S][CT];
#pragma unroll
  for (int st = 0; st < S; st++)
#pragma unroll
    for (int ct = 0; ct < CT; ct++) wr[st][ct] = load_rec<FMT>(B, D, N, G, gw + 4 * st + j, n0 + ct * 16 + c);
  if (K == 0xFFFFFFFEu) __builtin_amdgcn_s_sleep(1);

  // 3. activations -> f16 fragments in this wave's LDS slice, in the slot
  //    order of the record conversion; hi = f16(a), lo = f16((a - hi) * 2048)
  {
    const int perm_q4[8] = {0, 4, 1, 5, 2, 6, 3, 7};
    const int perm_q8[8] = {0, 2, 1, 3, 4, 6, 5, 7};
    typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
    typedef float float2_t __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int it = 0; it < IPT; it++) {
      const uint32_t item = lane + it * 64;
      const uint32_t kq = item & 3, m = (item >> 2) % MR, gl = wk * GPW + (item >> 2) / MR;
      u32x4 hp, lp;
      const half2_t one2 = {(_Float16)1, (_Float16)1};
      float sh = 0.f, sl = 0.f;  // sums of the f16 values (v_dot2_f32_f16 against ones)
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int e0 = FMT == FMT_Q8 ? perm_q8[2 * q] : perm_q4[2 * q];
        const int e1 = FMT == FMT_Q8 ? perm_q8[2 * q + 1] : perm_q4[2 * q + 1];
        const float a0 = alive[it] ? av[it][e0] : 0.f, a1 = alive[it] ? av[it][e1] : 0.f;
        const half2_t h = __builtin_convertvector((float2_t){a0, a1}, half2_t);
        hp[q] = __builtin_bit_cast(uint32_t, h);
        sh = __builtin_amdgcn_fdot2(h, one2, sh, false);
        if (HILO) {
          const float l0 = __builtin_fmaf((float)h[0], -2048.0f, a0 * 2048.0f);
          const float l1 = __builtin_fmaf((float)h[1], -2048.0f, a1 * 2048.0f);
          const half2_t lh = __builtin_convertvector((float2_t){l0, l1}, half2_t);
          lp[q] = __builtin_bit_cast(uint32_t, lh);
          sl = __builtin_amdgcn_fdot2(lh, one2, sl, false);
        }
      }
      if (SUM_LDS) {  // the four K slices of (group, row) sit in one lane quad
        sh = add_xor2(add_xor1(sh));
        if (HILO) sl = add_xor2(add_xor1(sl));
      }
      if (item < (uint32_t)NITEM) {
        fragL[gl][kq][m] = hp;
        if (HILO) fragL[gl][kq][MR + m] = lp;
        if (SUM_LDS && kq == 0) {
          sL[gl][m] = sh;
          if (HILO) sL[gl][8 + m] = sl;
        }
      }
    }
  }
  // LDS operations of one wave complete in order
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // 4. MFMAs.  A operand: lane (r = lane%16, kslice j); MFMA row r of row
  //    block rb is activation row 16 rb + r (plain) or r / r-8 (hi / lo),
  //    live when below MR.
  const uint32_t r = lane & 15;
  const uint32_t rm = HILO ? (r & 7) : r;
  bool a_live[RB];
  uint32_t avr[RB];
#pragma unroll
  for (int rb = 0; rb < RB; rb++) {
    a_live[rb] = 16 * rb + rm < (uint32_t)MR;
    avr[rb] = HILO && r >= 8 ? MR + rm : 16 * rb + rm;
  }
  // The record operands get their exponent-bias offset (1024 / 64 per
  // nibble slot, 1152 per int8) subtracted in f16 -- exact -- so the MFMA
  // sums a * q itself instead of a * (offset + q) with the offset part taken
  // off afterwards in f32, which cancelled ~1e-5 of the result at K = 512
  half8 boff;
  {
    const _Float16 off_q4[8] = {1024, 1024, 64, 64, 1024, 1024, 64, 64};
#pragma unroll
    for (int e = 0; e < 8; e++) boff[e] = FMT == FMT_Q8 ? (_Float16)1152 : off_q4[e] + (is_q40(FMT) ? 8 : 0);
  }
  f32x4 acc[CT][RB];
#pragma unroll
  for (int ct = 0; ct < CT; ct++)
#pragma unroll
    for (int rb = 0; rb < RB; rb++) acc[ct][rb] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int st = 0; st < S; st++) {
    const uint32_t gl0 = wk * GPW + 4 * st;
    half8 af[4][RB];
    float sv4[4][RB][4];
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
      for (int rb = 0; rb < RB; rb++) {
        u32x4 f = (u32x4){0u, 0u, 0u, 0u};
        if (a_live[rb]) f = fragL[gl0 + t][j][avr[rb]];
        af[t][rb] = __builtin_bit_cast(half8, f);
        if (SUM_LDS) {  // S of the lane's output rows 4j .. 4j+3 (same-address reads broadcast)
          const float4 s4 = *(const float4*)&sL[gl0 + t][16 * rb + 4 * j];
          sv4[t][rb][0] = s4.x;
          sv4[t][rb][1] = s4.y;
          sv4[t][rb][2] = s4.z;
          sv4[t][rb][3] = s4.w;
        } else if (NEED_S) {
          half8 bx;
#pragma unroll
          for (int e = 0; e < 8; e++) bx[e] = c == 0 ? (_Float16)1 : (_Float16)0;
          const f32x4 pe = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[t][rb], bx, (f32x4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 4; i++)
            sv4[t][rb][i] = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(pe[i]), 0x150, 0xF, 0xF, false));
        }
      }
#pragma unroll
    for (int ct = 0; ct < CT; ct++) {
      half8 bf[4];
      uint32_t sv[4], zv[4];
      rec_kslices<FMT>(wr[st][ct], bf, sv, zv);
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const float s = __uint_as_float(sv[t]), z = __uint_as_float(zv[t]);
        const half8 bq = bf[t] - boff;  // the integers q (Q4_0: q - 8) themselves
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
          const f32x4 p = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[t][rb], bq, (f32x4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const float tt = NEED_S ? __builtin_fmaf(-z, sv4[t][rb][i], p[i]) : p[i];
            acc[ct][rb][i] = __builtin_fmaf(s, tt, acc[ct][rb][i]);
          }
        }
      }
    }
  }

  // 5. the WK waves of the block in fixed order, then the epilogue or the
  //    cross-block split
  if (ALIAS) __syncthreads();  // every wave is done with the fragments
#pragma unroll
  for (int ct = 0; ct < CT; ct++)
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
      for (int i = 0; i < 4; i++) red[wk][16 * rb + j * 4 + i][ct * 16 + c] = acc[ct][rb][i];
  __syncthreads();
  const uint32_t mrows = M < (uint32_t)MR ? M : MR;
  const uint32_t nb = blockIdx.x * BC;
  auto colsum = [&](uint32_t m, uint32_t cc) {
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < WK; w++) {
      if (HILO) v += red[w][m][cc] + red[w][m + 8][cc] * (1.0f / 2048.0f);
      else v += red[w][m][cc];
    }
    return v;
  };
  // a non-finite block sum (an activation beyond the f16 range, |a| >=
  // 65520, or an infinite / NaN one) is recomputed in f32 over the block's
  // K range and stored again over the first store
  auto f32_sum = [&](uint32_t m, uint32_t n) {
    return f32_block_sum<FMT>(A, B, D, N, G, K, m, n, gb, gb + KB, nullptr, 1.0f);
  };
  if (ksplit == 1) {
    if (epi == EPI_SWIGLU) {
      for (uint32_t e = threadIdx.x; e < mrows * BC / 2; e += NT) {
        const uint32_t m = e / (BC / 2), cc = 2 * (e % (BC / 2)), n = nb + cc;
        if (n >= N) continue;
        const float g = colsum(m, cc), u = colsum(m, cc + 1);
        C[(size_t)m * (N / 2) + n / 2] = silu_mul(g, u);
        if (!finite_f32(g) || !finite_f32(u)) C[(size_t)m * (N / 2) + n / 2] = silu_mul(f32_sum(m, n), f32_sum(m, n + 1));
      }
    } else {
      for (uint32_t e = threadIdx.x; e < mrows * BC; e += NT) {
        const uint32_t m = e / BC, cc = e % BC, n = nb + cc;
        if (n >= N) continue;
        float v = colsum(m, cc);
        C[(size_t)m * N + n] = epi == EPI_RESID ? R[(size_t)m * N + n] + v : v;
        if (!finite_f32(v)) {
          v = f32_sum(m, n);
          C[(size_t)m * N + n] = epi == EPI_RESID ? R[(size_t)m * N + n] + v : v;
        }
      }
    }
    return;
  }
  for (uint32_t e = threadIdx.x; e < mrows * BC; e += NT) {
    const uint32_t m = e / BC, cc = e % BC, n = nb + cc;
    if (n >= N) continue;
    float v = colsum(m, cc);
    if (!finite_f32(v)) v = f32_sum(m, n);
    __hip_atomic_exchange((uint32_t*)ws + ((size_t)blockIdx.y * M + m) * N + n, __float_as_uint(v),
                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  splitk_finish(ws, counters, C, R, epi, M, N, mrows, nb, BC, NT, ksplit, &s_last);
}

#define DEF_QGEMV5(NAME, FMT, MR, HILO, CT, S, WK)                                                      \
  extern "C" __global__ __launch_bounds__(WK * 64) void NAME(                                            \
      const float* A, const uint8_t* B, const uint16_t* D, float* C, float* ws, uint32_t* counters,      \
      uint32_t M, uint32_t N, uint32_t K, uint32_t G, const float* R, uint32_t epi) {                    \
    qgemv5_body<FMT, MR, HILO, CT, S, WK>(A, B, D, C, ws, counters, M, N, K, G, R, epi);                 \
  }

// Row buckets m4 / m8 (hi/lo) and m16 (plain f16).  w16: 16 waves x 2
// steps = 128 groups (all of K <= 4096 in one block), 16 columns; k32: 8
// waves x 1 step, 16 columns (narrow N: K splits fill the chip); k32c4: the
// same K range with 4 column tiles per wave (64 columns: wide N, long K);
// m32_k64c2: 16 waves x 1 step over 64 groups, 32 columns (M = 32)
#define DEF_QGEMV5_FMT(TAG, FMT)                                       \
  DEF_QGEMV5(smith_qgemv5_##TAG##_m4_w16, FMT, 4, true, 1, 2, 16)      \
  DEF_QGEMV5(smith_qgemv5_##TAG##_m8_w16, FMT, 8, true, 1, 2, 16)      \
  DEF_QGEMV5(smith_qgemv5_##TAG##_m16_w16, FMT, 16, false, 1, 2, 16)   \
  DEF_QGEMV5(smith_qgemv5_##TAG##_m4_k32, FMT, 4, true, 1, 1, 8)       \
  DEF_QGEMV5(smith_qgemv5_##TAG##_m8_k32, FMT, 8, true, 1, 1, 8)       \
  DEF_QGEMV5(smith_qgemv5_##TAG##_m16_k32, FMT, 16, false, 1, 1, 8)    \
  DEF_QGEMV5(smith_qgemv5_##TAG##_m4_k32c4, FMT, 4, true, 4, 1, 8)     \
  DEF_QGEMV5(smith_qgemv5_##TAG##_m8_k32c4, FMT, 8, true, 4, 1, 8)     \
  DEF_QGEMV5(smith_qgemv5_##TAG##_m16_k32c4, FMT, 16, false, 4, 1, 8)   \
  DEF_QGEMV5(smith_qgemv5_##TAG##_m32_k32, FMT, 32, false, 1, 1, 8)      \
  DEF_QGEMV5(smith_qgemv5_##TAG##_m32_k32c4, FMT, 32, false, 4, 1, 8)    \
  DEF_QGEMV5(smith_qgemv5_##TAG##_m32_k64c2, FMT, 32, false, 2, 1, 16)


// ---------------------------------------------------------------------------
// Single-row decode GEMV on a prepared activation (act_frag.h) and Q4_0
// weights in tile-major order (FMT_Q40T).  Same MFMA scheme as qgemv1 with
// the activation side reduced to loads: lane (r, j) of a wave feeds A row r
// (r = 4j: hi, 4j+1: lo of group g+j; other rows zero) straight from the act
// buffer, and (C1) of its group from the act's tile sums.  With `norm` the
// result is scaled by rms = 1/sqrt(mean(v^2) + eps) from the act's sums of
// squares (an RMSNorm on the input, gguf_cache.js:121,167).  A block covers
// the whole K (4*S*WK groups >= K/32), so no cross-block reduction.
// Wave 0 finishes its BC columns: sum of the WK partials, rms, epilogue
// (store / residual / SwiGLU), the f32 store (C may be null) and, with
// act_out, the act of the produced vector for the next projection.
// ---------------------------------------------------------------------------
// SRC 0: the input is an act.  SRC 1: the input is the attention output as
// per-split partials (smith_attention_part: (m, l, o[hd]) per head and key
// split, ATTP_STRIDE floats each); the block combines the splits of the
// heads in its K range (softmax weights e^(m_z - M) / L) and converts them
// to the MFMA operand in LDS itself.  No RMSNorm in front (norm == 0).
// Word 3 of a raw buffer resource on gfx9 (CDNA): DATA_FORMAT = 32 bits, no
// swizzle; with stride 0 a lane whose byte offset is >= num_records reads
// zeros without a memory access
#define RSRC_WORD3 0x00020000
#define ATTP_MAXSPLIT 8  // as llama_kernels.hip
#define ATTP_ROWS 32
#define ATTP_STRIDE 132
// NONORM: a variant for callers that never pass a norm (the residual
// projections), without the sum-of-squares loads and the norm code
template <int F, int CT, int S, int WK, int SRC, bool NONORM = false>
__device__ __forceinline__ void agemv_body(const uint8_t* __restrict__ act, const uint8_t* __restrict__ B,
                                           const uint16_t* __restrict__ D, float* __restrict__ C, uint32_t N,
                                           uint32_t K, uint32_t norm, float eps, const float* __restrict__ R,
                                           uint32_t epi, uint8_t* __restrict__ act_out,
                                           const float* __restrict__ gamma_out, float* __restrict__ ws,
                                           uint32_t* __restrict__ counters, const int32_t* __restrict__ pos_ptr,
                                           uint32_t hd, uint32_t bx) {
  constexpr int GPW = 4 * S;
  constexpr int BC = 16 * CT;
  constexpr int GMAX = 4 * S * WK;
  __shared__ u32x4 fragL[8 * GMAX];  // [g][hi/lo][slice]
  __shared__ float red[WK][BC];
  constexpr bool NEED_S = F != FMT_Q40T;  // the affine term needs the group sums S
  constexpr bool HALVES = F == GT_Q6K;    // separate scales for elements 0-15 / 16-31
  __shared__ float c1L[SRC == 1 ? 4 * GMAX : 1];                 // per-part C1 (SRC 1)
  __shared__ float sL[SRC == 1 && NEED_S ? 4 * GMAX : 1];         // per-part S (SRC 1)
  __shared__ float coefL[SRC == 1 ? GMAX : 1][ATTP_MAXSPLIT];    // per-head split weights (SRC 1)
  const uint32_t G = K / 32, T = K / 8;
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wk = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t c = lane & 15, j = lane >> 4;
  const uint32_t n0 = bx * BC;  // bx: this block's column block
  const uint32_t ksplit = gridDim.y;
  const uint32_t gb = blockIdx.y * GMAX;  // first group of this block
  const uint32_t gw = gb + wk * GPW;

  // 1. activation fragments: the act's frag words copied to LDS as they are
  //    (no conversion), group sums C1 from the act's tile sums
  const uint32_t r = lane & 15;
  const bool a_active = (r >> 2) == j && (r & 3) < 2;
  const u32x4* frag = (const u32x4*)act;
  const float* c1p = (const float*)(act + (size_t)K * 4);
  constexpr int NT = 64 * WK;
  constexpr int SPL = (GMAX + 63) / 64;           // float4s of part sums of squares per lane
  float c1[S], c1b[S], sg[S], sgb[S];  // (C1, S) of the group, or of its halves (HALVES)
  float4 ssv[SPL];
  float4 ccv = make_float4(0.f, 0.f, 0.f, 0.f), svv = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int q = 0; q < SPL; q++) ssv[q] = make_float4(0.f, 0.f, 0.f, 0.f);
  // SRC 1: split partials of this block's parts (part = 8 elements)
  constexpr int PPT = SRC == 1 ? (4 * GMAX + NT - 1) / NT : 1;
  float4 oa[PPT][ATTP_MAXSPLIT], ob[PPT][ATTP_MAXSPLIT];
  float mlv[2 * ATTP_MAXSPLIT];
  uint32_t nsplit = 1, h0 = 0;
  // SRC 0: each wave copies the act fragments of its own GPW groups (8 per
  // group: hi/lo x 4 slices) to its LDS slice with coalesced loads; after a
  // wave-level barrier only the lanes whose MFMA row carries an activation
  // row (2 of 16 per lane group) read their operands, the others hold zeros
  constexpr int FPW = (8 * GPW + 63) / 64;  // fragment words per lane
  u32x4 fv[FPW];
  if (SRC == 0) {
#pragma unroll
    for (int q = 0; q < FPW; q++) {
      const uint32_t e = 8 * gw + lane + 64 * q;
      fv[q] = frag[e < 8 * G ? e : 8 * G - 1];  // clamped: branch-free issue
    }
    // the tile sums of the wave's GPW groups: lane l < GPW loads group gw + l
    // once (a per-step load by every lane returned 64 copies of 4 groups'
    // sums: the wave's load data, which the CU returns at 64 B per clock,
    // was then mostly duplicates); handed to the lanes after the weight loads
    // (buffer loads: the other lanes' offsets are out of range, so they
    // fetch nothing and read zeros, with no branch around the load)
    {
      const uint32_t g = gw + lane;
      const uint32_t gc = g < G ? g : G - 1;
      const uint32_t off = lane < (uint32_t)GPW ? 16 * gc : 0x80000000u;
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)c1p, 0, (int)(8 * T), RSRC_WORD3);
      ccv = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
      if (NEED_S) svv = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 4 * T, 0, 0));
    }
    // sums of squares for the RMSNorm (one block covers K; with a K split the
    // finishing block reads them at the end): only wave 0 forms the norm
    if (!NONORM && wk == 0)
#pragma unroll
      for (int q = 0; q < SPL; q++) {  // T % 4 == 0 (K % 32 == 0): 16-byte loads
        const uint32_t t = lane + 64 * q;
        ssv[q] = ((const float4*)(c1p + 2 * T))[t < T / 4 ? t : T / 4 - 1];
      }
  } else {
    const uint32_t T1 = (uint32_t)pos_ptr[0] + 1;
    nsplit = (T1 + ATTP_ROWS - 1) / ATTP_ROWS;
    nsplit = nsplit < ATTP_MAXSPLIT ? nsplit : ATTP_MAXSPLIT;
    const float* parts = (const float*)act;
    h0 = gb * 32 / hd;
    const uint32_t hend = ((gb + GMAX < G ? gb + GMAX : G) * 32 + hd - 1) / hd;
    // buffer loads: threads past the block's heads / parts get out-of-range
    // offsets and fetch nothing (clamped duplicates of the last head's
    // partials made up 40 % of the block's load data: the workgroup's loads
    // return at ~155 GB/s, which bounds this kernel)
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc((void*)parts, 0, 0x7FFFFFFF, RSRC_WORD3);
    {  // (m, l) of head h0 + threadIdx.x (all splits: offsets that waited for the
       // position's split count would put a memory round trip before these loads)
      const bool live = h0 + threadIdx.x < hend;
#pragma unroll
      for (int zz = 0; zz < ATTP_MAXSPLIT; zz++) {
        const uint32_t off =
            live ? (uint32_t)((((h0 + threadIdx.x) * ATTP_MAXSPLIT + zz) * ATTP_STRIDE) * 4) : 0x80000000u;
        const float2 ml = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(prs, off, 0, 0));
        mlv[2 * zz] = ml.x;
        mlv[2 * zz + 1] = ml.y;
      }
    }
#pragma unroll
    for (int q = 0; q < PPT; q++) {
      const uint32_t pl = threadIdx.x + q * NT, pi = 4 * gb + pl;
      const bool live = pl < 4 * GMAX && pi < 4 * G;
      const uint32_t e0 = 8 * pi, hh = e0 / hd, d0 = e0 % hd;
#pragma unroll
      for (int zz = 0; zz < ATTP_MAXSPLIT; zz++) {
        const uint32_t off = live ? (uint32_t)(((hh * ATTP_MAXSPLIT + zz) * ATTP_STRIDE + 4 + d0) * 4) : 0x80000000u;
        oa[q][zz] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(prs, off, 0, 0));
        ob[q][zz] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(prs, off + 16, 0, 0));
      }
    }
  }
  // epilogue operands of wave 0 (residual, next norm's gamma), loaded now so
  // the tail after the reduction has no global load in its dependency chain
  float rv = 0.f, gv = 1.f;
  if (wk == 0) {
    const uint32_t n = n0 + (lane < BC ? lane : 0);
    if (epi == EPI_RESID) rv = R[n < N ? n : N - 1];
    if (act_out && gamma_out) {
      const uint32_t no = epi == EPI_SWIGLU ? N / 2 : N;
      const uint32_t o = (epi == EPI_SWIGLU ? n0 / 2 : n0) + (lane & 31);
      gv = gamma_out[o < no ? o : no - 1];
    }
  }
  // 2. weights (after the small act loads: loads complete in order), then the
  //    LDS copy is published
  // one clamped base per wave; records at fixed offsets (1 KB per step of 4
  // groups, G*256 bytes per tile).  Out-of-range records (ragged N or K) are
  // read clamped and get scale 0.
  u32x4 wq[S][CT];
  uint16_t wd[S][CT];
  GtW<F> gw_[S][CT];
  {
    const uint32_t nt = n0 >> 4, ntl = (N - 1) >> 4;
    const GtPlanes P = gt_planes(F, N, G);
#pragma unroll
    for (int st = 0; st < S; st++)
#pragma unroll
      for (int ct = 0; ct < CT; ct++) {
        const uint32_t g = gw + 4 * st + j, t = nt + ct;
        const uint32_t tc = t < ntl ? t : ntl, gc = g < G ? g : G - 1;
        const size_t rec = ((size_t)tc * G + gc) * 16 + c;
        if (F == FMT_Q40T) {
          wq[st][ct] = *(const u32x4*)(B + rec * 16);
          wd[st][ct] = D[rec];
        } else {
          gt_load<F>(gw_[st][ct], B, P, rec, ((size_t)tc * (G / 8) + gc / 8) * 16 + c);
        }
      }
  }

  float ssum = 0.f;
  if (SRC == 0) {
#pragma unroll
    for (int q = 0; q < FPW; q++) {
      const uint32_t e = lane + 64 * q;
      if (e < 8u * GPW) fragL[8 * wk * GPW + e] = fv[q];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    {  // (C1, S) of group gw + 4 st + j from lane 4 st + j; the empty asm
       // keeps the sums here (hoisted into the load's branch they made the
       // wave wait for the load before issuing its weight loads)
      asm volatile("" : "+v"(ccv.x), "+v"(ccv.y), "+v"(ccv.z), "+v"(ccv.w));
      if (NEED_S) asm volatile("" : "+v"(svv.x), "+v"(svv.y), "+v"(svv.z), "+v"(svv.w));
      const float c1v = HALVES ? ccv.x + ccv.y : (ccv.x + ccv.y) + (ccv.z + ccv.w), c1bv = ccv.z + ccv.w;
      const float sgv = HALVES ? svv.x + svv.y : (svv.x + svv.y) + (svv.z + svv.w), sgbv = svv.z + svv.w;
#pragma unroll
      for (int st = 0; st < S; st++) {
        const int src = 4 * st + (int)j;
        c1[st] = __shfl(c1v, src);
        if (HALVES) c1b[st] = __shfl(c1bv, src);
        if (NEED_S) {
          sg[st] = __shfl(sgv, src);
          if (HALVES) sgb[st] = __shfl(sgbv, src);
        }
      }
    }
    if (!NONORM && ksplit == 1 && wk == 0)
#pragma unroll
      for (int q = 0; q < SPL; q++)
        ssum += lane + 64 * q < T / 4 ? (ssv[q].x + ssv[q].y) + (ssv[q].z + ssv[q].w) : 0.f;
  } else {
    // softmax weights of each head's splits: e^(m_z - M) / sum_z e^(m_z - M) l_z
    if (threadIdx.x < GMAX) {
      float M = -__builtin_inff();
#pragma unroll
      for (int zz = 0; zz < ATTP_MAXSPLIT; zz++)
        if ((uint32_t)zz < nsplit) M = mlv[2 * zz] > M ? mlv[2 * zz] : M;
      float f[ATTP_MAXSPLIT], L = 0.f;
#pragma unroll
      for (int zz = 0; zz < ATTP_MAXSPLIT; zz++) {
        const bool live = (uint32_t)zz < nsplit && mlv[2 * zz] != -__builtin_inff();
        f[zz] = live ? __expf(mlv[2 * zz] - M) : 0.f;
        L = live ? __builtin_fmaf(f[zz], mlv[2 * zz + 1], L) : L;  // unwritten splits may hold anything
      }
#pragma unroll
      for (int zz = 0; zz < ATTP_MAXSPLIT; zz++) coefL[threadIdx.x][zz] = f[zz] / L;
    }
    __syncthreads();
    // combined elements -> f16 hi/lo operand slots + per-part C1 (act_frag.h order)
#pragma unroll
    for (int q = 0; q < PPT; q++) {
      const uint32_t pl = threadIdx.x + q * NT;  // part within the block
      const uint32_t pi = 4 * gb + pl;
      if (pl < 4 * GMAX && pi < 4 * G) {
        const uint32_t hl = 8 * pi / hd - h0;
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = 0.f;
#pragma unroll
        for (int zz = 0; zz < ATTP_MAXSPLIT; zz++) {
          if ((uint32_t)zz >= nsplit) break;  // unwritten splits (never multiply stale memory)
          const float cz = coefL[hl][zz];
          v[0] = __builtin_fmaf(cz, oa[q][zz].x, v[0]);
          v[1] = __builtin_fmaf(cz, oa[q][zz].y, v[1]);
          v[2] = __builtin_fmaf(cz, oa[q][zz].z, v[2]);
          v[3] = __builtin_fmaf(cz, oa[q][zz].w, v[3]);
          v[4] = __builtin_fmaf(cz, ob[q][zz].x, v[4]);
          v[5] = __builtin_fmaf(cz, ob[q][zz].y, v[5]);
          v[6] = __builtin_fmaf(cz, ob[q][zz].z, v[6]);
          v[7] = __builtin_fmaf(cz, ob[q][zz].w, v[7]);
        }
        const int perm[8] = {0, 4, 1, 5, 2, 6, 3, 7};
        _Float16 hv[8], lv[8];
        float c1p_ = 0.f, sp_ = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const float a = v[perm[e]];
          const _Float16 hh = (_Float16)a;
          const float hf = (float)hh;
          const _Float16 ll = (_Float16)((a - hf) * 2048.0f);
          const float lf = (float)ll;
          hv[e] = hh;
          lv[e] = ll;
          const float off = (e & 2) ? 64.0f : 1024.0f;
          c1p_ += __builtin_fmaf(lf * off, 1.0f / 2048.0f, hf * off);
          sp_ += __builtin_fmaf(lf, 1.0f / 2048.0f, hf);
        }
        u32x4 hp, lp;
#pragma unroll
        for (int k = 0; k < 4; k++) {
          hp[k] = __builtin_bit_cast(uint32_t, (_Float16 __attribute__((ext_vector_type(2)))){hv[2 * k], hv[2 * k + 1]});
          lp[k] = __builtin_bit_cast(uint32_t, (_Float16 __attribute__((ext_vector_type(2)))){lv[2 * k], lv[2 * k + 1]});
        }
        const uint32_t gl = pl >> 2, sl = pl & 3;
        fragL[(gl * 2 + 0) * 4 + sl] = hp;
        fragL[(gl * 2 + 1) * 4 + sl] = lp;
        c1L[pl] = __builtin_fmaf(8.0f, sp_, c1p_);
        if (NEED_S) sL[pl] = sp_;
      }
    }
    __syncthreads();
  }
  if (SRC == 1) {
#pragma unroll
    for (int st = 0; st < S; st++) {
      const uint32_t g = gw + 4 * st + j;
      const uint32_t gl = (g < G ? g : G - 1) - gb;
      if (HALVES) {
        c1[st] = c1L[4 * gl] + c1L[4 * gl + 1];
        c1b[st] = c1L[4 * gl + 2] + c1L[4 * gl + 3];
        sg[st] = sL[4 * gl] + sL[4 * gl + 1];
        sgb[st] = sL[4 * gl + 2] + sL[4 * gl + 3];
      } else {
        c1[st] = (c1L[4 * gl] + c1L[4 * gl + 1]) + (c1L[4 * gl + 2] + c1L[4 * gl + 3]);
        if (NEED_S) sg[st] = (sL[4 * gl] + sL[4 * gl + 1]) + (sL[4 * gl + 2] + sL[4 * gl + 3]);
      }
    }
  }

  // 3. MFMAs and the exact per-group post-step
  float acc[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ct++) acc[ct] = 0.f;
#pragma unroll
  for (int st = 0; st < S; st++) {
    // this step's A operands: LDS reads by the active lanes only (the
    // others' rows are zero), just before the MFMAs that take them
    u32x4 afr[4] = {(u32x4){0u, 0u, 0u, 0u}, (u32x4){0u, 0u, 0u, 0u}, (u32x4){0u, 0u, 0u, 0u},
                    (u32x4){0u, 0u, 0u, 0u}};
    {
      const uint32_t g = gw + 4 * st + j;
      if (a_active && g < G)
#pragma unroll
        for (int i = 0; i < 4; i++) afr[i] = fragL[((g - gb) * 2 + (r & 3)) * 4 + i];
    }
#pragma unroll
    for (int ct = 0; ct < CT; ct++) {
      const uint32_t g = gw + 4 * st + j, n = n0 + 16 * ct + c;
      const bool in = g < G && n < N;
      if constexpr (F == FMT_Q40T) {
        f32x4 p = (f32x4){0.f, 0.f, 0.f, 0.f};
        Rec<FMT_Q40T> rr;
        rr.q = wq[st][ct];
#pragma unroll
        for (int i = 0; i < 4; i++)
          p = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, afr[i]),
                                                     rec_to_f16<FMT_Q40T>(rr, i), p, 0, 0, 0);
        const float sc = in ? (float)__builtin_bit_cast(_Float16, wd[st][ct]) : 0.f;
        const float t = __builtin_fmaf(p[1], 1.0f / 2048.0f, p[0]) - c1[st];
        acc[ct] = __builtin_fmaf(sc, t, acc[ct]);
      } else {
        // sum of a*(s*q + c) = s*X + (8s + c)*S with X = P - C1 (C1 carries
        // the +8S of the act): per group, or per 16-element half (Q6_K)
        const GtW<F>& w = gw_[st][ct];
        const u32x4* fa = afr;
        f32x4 p = (f32x4){0.f, 0.f, 0.f, 0.f}, p2 = (f32x4){0.f, 0.f, 0.f, 0.f};
        p = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, fa[0]), gt_to_f16<F, 0>(w), p, 0, 0, 0);
        p = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, fa[1]), gt_to_f16<F, 1>(w), p, 0, 0, 0);
        if (HALVES) {
          p2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, fa[2]), gt_to_f16<F, 2>(w), p2, 0, 0, 0);
          p2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, fa[3]), gt_to_f16<F, 3>(w), p2, 0, 0, 0);
        } else {
          p = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, fa[2]), gt_to_f16<F, 2>(w), p, 0, 0, 0);
          p = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, fa[3]), gt_to_f16<F, 3>(w), p, 0, 0, 0);
        }
        float s0, a0, s1, a1;
        gt_affine<F>(w, s0, a0, s1, a1);
        s0 = in ? s0 : 0.f;
        a0 = in ? a0 : 0.f;
        const float t = __builtin_fmaf(p[1], 1.0f / 2048.0f, p[0]) - c1[st];
        acc[ct] = __builtin_fmaf(s0, t, __builtin_fmaf(__builtin_fmaf(8.0f, s0, a0), sg[st], acc[ct]));
        if (HALVES) {
          s1 = in ? s1 : 0.f;
          a1 = in ? a1 : 0.f;
          const float t2 = __builtin_fmaf(p2[1], 1.0f / 2048.0f, p2[0]) - c1b[st];
          acc[ct] = __builtin_fmaf(s1, t2, __builtin_fmaf(__builtin_fmaf(8.0f, s1, a1), sgb[st], acc[ct]));
        }
      }
    }
  }

  // 4. lane groups (K groups g+j), then the WK waves in fixed order
#pragma unroll
  for (int ct = 0; ct < CT; ct++) {
    float v = acc[ct];
    v = add_xor32(add_xor16(v));
    if (j == 0) red[wk][ct * 16 + c] = v;
  }
  __syncthreads();
  if (wk != 0) return;
  // wave 0: block partial of column n0 + lane (lane < BC)
  float v = 0.f;
  if (lane < BC) {
#pragma unroll
    for (int w = 0; w < WK; w++) v += red[w][lane];
  }
  if (ksplit > 1) {
    // deterministic split-K: partials through agent-scope atomics, the last
    // block of the column block sums them in split order (counter self-resets)
    if (lane < BC && n0 + lane < N)
      __hip_atomic_exchange((uint32_t*)ws + (size_t)blockIdx.y * N + n0 + lane, __float_as_uint(v),
                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    uint32_t prev = 0;
    if (lane == 0)
      prev = __hip_atomic_fetch_add(counters + bx, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    prev = __shfl(prev, 0);
    if (prev != ksplit - 1) return;
    v = 0.f;
    if (lane < BC && n0 + lane < N)
      v = splitk_sum(ws + n0 + lane, N, ksplit);
    if (lane == 0) __hip_atomic_exchange(counters + bx, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (norm)
      for (uint32_t t = lane; t < T; t += 64) ssum += c1p[2 * T + t];
  }
  float rms = 1.0f;
  if (NONORM) norm = 0;
  if (norm) {
    ssum = sum64_lanes(ssum);
    rms = 1.0f / __builtin_sqrtf(ssum / (float)K + eps);
  }
  v *= rms;
  if (epi == EPI_SWIGLU) {
    // lane o < BC/2 takes the interleaved (gate, up) pair of columns 2o, 2o+1
    const float g = __shfl(v, (int)(2 * (lane & 31))), u = __shfl(v, (int)(2 * (lane & 31) + 1));
    if (lane < BC / 2) {
      const uint32_t o = n0 / 2 + lane;
      const bool in = n0 + 2 * lane < N;
      const float y = silu_mul(g, u);
      if (C && in) C[o] = y;
      if (act_out) act_emit8(act_out, N / 2, o, in ? y : 0.f, gv);
    }
  } else if (lane < BC) {
    const uint32_t n = n0 + lane;
    const bool in = n < N;
    if (epi == EPI_RESID) v += rv;
    if (C && in) C[n] = v;
    if (act_out) act_emit8(act_out, N, n, in ? v : 0.f, gv);
  }
}

#define DEF_AGEMV(NAME, F, CT, S, WK, ...)                                                                    \
  extern "C" __global__ __launch_bounds__(WK * 64) void NAME(                                                \
      const uint8_t* __restrict__ act, const uint8_t* __restrict__ B, const uint16_t* __restrict__ D,        \
      float* __restrict__ C, uint32_t N, uint32_t K, uint32_t norm, float eps, const float* __restrict__ R,   \
      uint32_t epi, uint8_t* __restrict__ act_out, const float* __restrict__ gamma_out, float* __restrict__ ws, \
      uint32_t* __restrict__ counters) {                                                                     \
    agemv_body<F, CT, S, WK, 0, ##__VA_ARGS__>(act, B, D, C, N, K, norm, eps, R, epi, act_out, gamma_out, ws, \
                                               counters, nullptr, 0, blockIdx.x);                            \
  }

// o-projection on attention split partials (SRC 1); parts in place of the act
#define DEF_AGEMV_ATT(NAME, F, CT, S, WK)                                                                     \
  extern "C" __global__ __launch_bounds__(WK * 64) void NAME(                                                \
      const float* __restrict__ parts, const int32_t* __restrict__ pos_ptr, uint32_t hd,                     \
      const uint8_t* __restrict__ B, const uint16_t* __restrict__ D, float* __restrict__ C, uint32_t N,       \
      uint32_t K, const float* __restrict__ R, uint32_t epi, uint8_t* __restrict__ act_out,                   \
      const float* __restrict__ gamma_out, float* __restrict__ ws, uint32_t* __restrict__ counters) {        \
    agemv_body<F, CT, S, WK, 1>((const uint8_t*)parts, B, D, C, N, K, 0u, 0.f, R, epi, act_out, gamma_out, ws, \
                             counters, pos_ptr, hd, blockIdx.x);                                             \
  }

// named by the groups one block covers (4*S*WK) and the column tiles per wave;
// a K longer than one block is split over gridDim.y blocks
#define DEF_AGEMV_FMT(TAG, F)                                 \
  DEF_AGEMV(smith_agemv_##TAG##_k32, F, 1, 2, 4)              \
  DEF_AGEMV(smith_agemv_##TAG##_k48, F, 1, 3, 4)              \
  DEF_AGEMV(smith_agemv_##TAG##_k64, F, 1, 4, 4)              \
  DEF_AGEMV(smith_agemv_##TAG##_k72, F, 1, 3, 6)              \
  DEF_AGEMV(smith_agemv_##TAG##_k96, F, 1, 3, 8)              \
  DEF_AGEMV(smith_agemv_##TAG##_k128, F, 1, 4, 8)             \
  DEF_AGEMV(smith_agemv_##TAG##_k144, F, 1, 3, 12)            \
  DEF_AGEMV(smith_agemv_##TAG##_k192, F, 1, 6, 8)             \
  DEF_AGEMV(smith_agemv_##TAG##_k288, F, 1, 9, 8)             \
  DEF_AGEMV(smith_agemv_##TAG##_k96_c2, F, 2, 3, 8)           \
  DEF_AGEMV(smith_agemv_##TAG##_k288_w12, F, 1, 6, 12)        \
  DEF_AGEMV(smith_agemv_##TAG##_k288_w12_nn, F, 1, 6, 12, true) \
  DEF_AGEMV_ATT(smith_agemv_att_##TAG##_k64, F, 1, 4, 4)      \
  DEF_AGEMV_ATT(smith_agemv_att_##TAG##_k96, F, 1, 3, 8)      \
  DEF_AGEMV_ATT(smith_agemv_att_##TAG##_k128, F, 1, 4, 8)     \
  DEF_AGEMV_ATT(smith_agemv_att_##TAG##_k192, F, 1, 6, 8)
// Two tile formats in one launch, for q|k|v projections whose weights differ
// in block type (Q4_K_M keeps attn_v in Q6_K): output columns [0, N1) from
// planes B1 (format F1), [N1, N) from planes B2 (format F2), the same act in;
// plain stores (no epilogue, no act out).  Workgroups choose their half by
// blockIdx.x (uniform); each half keeps its own LDS.
#define DEF_AGEMV2(NAME, F1, F2, CT, S, WK)                                                                   \
  extern "C" __global__ __launch_bounds__(WK * 64) void NAME(                                                \
      const uint8_t* __restrict__ act, const uint8_t* __restrict__ B1, const uint8_t* __restrict__ B2,       \
      float* __restrict__ C, uint32_t N1, uint32_t N, uint32_t K, uint32_t norm, float eps,                  \
      float* __restrict__ ws, uint32_t* __restrict__ counters) {                                             \
    const uint32_t nb1 = N1 / (16 * CT);                                                                     \
    const uint16_t* D1 = F1 == FMT_Q40T ? (const uint16_t*)(B1 + gt_planes(GT_Q40, N1, K / 32).prm)          \
                                        : (const uint16_t*)B1;                                               \
    const uint16_t* D2 = F2 == FMT_Q40T ? (const uint16_t*)(B2 + gt_planes(GT_Q40, N - N1, K / 32).prm)      \
                                        : (const uint16_t*)B2;                                               \
    if (blockIdx.x < nb1)                                                                                    \
      agemv_body<F1, CT, S, WK, 0>(act, B1, D1, C, N1, K, norm, eps, nullptr, 0u, nullptr, nullptr, ws,      \
                                   counters, nullptr, 0, blockIdx.x);                                        \
    else                                                                                                     \
      agemv_body<F2, CT, S, WK, 0>(act, B2, D2, C + N1, N - N1, K, norm, eps, nullptr, 0u, nullptr, nullptr, \
                                   ws + (size_t)gridDim.y * N1, counters + nb1, nullptr, 0, blockIdx.x - nb1); \
  }
#define DEF_AGEMV2_FMT(TAG, F1, F2)                       \
  DEF_AGEMV2(smith_agemv2_##TAG##_k32, F1, F2, 1, 2, 4)   \
  DEF_AGEMV2(smith_agemv2_##TAG##_k48, F1, F2, 1, 3, 4)   \
  DEF_AGEMV2(smith_agemv2_##TAG##_k64, F1, F2, 1, 4, 4)   \
  DEF_AGEMV2(smith_agemv2_##TAG##_k72, F1, F2, 1, 3, 6)   \
  DEF_AGEMV2(smith_agemv2_##TAG##_k96, F1, F2, 1, 3, 8)   \
  DEF_AGEMV2(smith_agemv2_##TAG##_k128, F1, F2, 1, 4, 8)  \
  DEF_AGEMV2(smith_agemv2_##TAG##_k144, F1, F2, 1, 3, 12) \
  DEF_AGEMV2(smith_agemv2_##TAG##_k192, F1, F2, 1, 6, 8)  \
  DEF_AGEMV2(smith_agemv2_##TAG##_k288, F1, F2, 1, 9, 8)

DEF_AGEMV_FMT(q40t, FMT_Q40T)
DEF_AGEMV_FMT(q41t, GT_Q41)
DEF_AGEMV_FMT(q50t, GT_Q50)
DEF_AGEMV_FMT(q4kt, GT_Q4K)
DEF_AGEMV_FMT(q6kt, GT_Q6K)
// the q|k|v type pairs of the llama.cpp K-quant mixes
DEF_AGEMV2_FMT(q4kt_q6kt, GT_Q4K, GT_Q6K)
DEF_AGEMV2_FMT(q4kt_q50t, GT_Q4K, GT_Q50)
DEF_AGEMV2_FMT(q50t_q6kt, GT_Q50, GT_Q6K)
DEF_AGEMV2_FMT(q40t_q6kt, FMT_Q40T, GT_Q6K)
DEF_AGEMV2_FMT(q4kt_q40t, GT_Q4K, FMT_Q40T)

#ifndef SMITH_NO_INSTANCES
DEF_QGEMV3_FMT(q4s, FMT_Q4S)
DEF_QGEMV3_FMT(q8, FMT_Q8)
DEF_QGEMV3_FMT(q40, FMT_Q40)
DEF_QGEMV3_FMT(q40t, FMT_Q40T)
DEF_QGEMV4_FMT(q4s, FMT_Q4S)
DEF_QGEMV4_FMT(q8, FMT_Q8)
DEF_QGEMV4_FMT(q40, FMT_Q40)
DEF_QGEMV4_FMT(q40t, FMT_Q40T)
DEF_QGEMV5_FMT(q4s, FMT_Q4S)
DEF_QGEMV5_FMT(q8, FMT_Q8)
DEF_QGEMV5_FMT(q40, FMT_Q40)
DEF_QGEMV5_FMT(q40t, FMT_Q40T)
DEF_QGEMV1_FMT(q4s, FMT_Q4S)
DEF_QGEMV1_FMT(q8, FMT_Q8)
DEF_QGEMV1_Q8C
DEF_QGEMV1_FMT(q40, FMT_Q40)
DEF_QGEMV1_FMT(q40t, FMT_Q40T)
#endif

// Zero fill (used instead of hipMemsetAsync so the op stays a plain kernel).
extern "C" __global__ void smith_zero_u32(uint32_t* __restrict__ p, uint64_t n) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}
