/*
 * smith_oracle.c -- CPU restatement of SMITH's quantized-weight matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (smith_amd/, include/,
 * the HIP kernels) links, loads or calls this file.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and only as
 * the checker / the timed CPU baseline.
 *
 * Build: make -C oracle   (plain C11, -O2 -ffp-contract=off, no fast-math)
 *
 * Every function names the reference file:line it restates.  Pinning of each
 * function (known answers, invariants, brute force) lives in
 * tests/test_oracle.py; see the table in that file's docstring.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>

#define Q4S_GROUP 32
#define Q4S_BYTES 24 /* 16 nibble bytes + f32 scale + f32 zero */
#define Q8_BYTES 34  /* f16 scale + 32 x int8 */
#define Q4_0_BYTES 18 /* f16 scale + 16 nibble bytes */

/* ---------- JavaScript number semantics used by quantize.js ---------- */

/* Math.max(a, b) for the two-argument case: NaN if either is NaN, and +0
 * preferred over -0. */
static double js_max(double a, double b) {
  if (isnan(a) || isnan(b)) return NAN;
  if (a == 0.0 && b == 0.0) return signbit(a) ? b : a;
  return a > b ? a : b;
}
static double js_min(double a, double b) {
  if (isnan(a) || isnan(b)) return NAN;
  if (a == 0.0 && b == 0.0) return signbit(a) ? a : b;
  return a < b ? a : b;
}
/* Math.round: nearest integer, ties toward +Infinity.  floor(x + 0.5) is NOT
 * this (it is wrong for 0.49999999999999994), so compare the fraction. */
static double js_round(double x) {
  if (isnan(x) || isinf(x)) return x;
  double r = floor(x);
  return (x - r >= 0.5) ? r + 1.0 : r;
}
/* ToUint8 / ToInt32 of a small value: NaN -> 0, else truncate. */
static uint32_t js_to_u32(double x) {
  if (isnan(x) || isinf(x)) return 0;
  return (uint32_t)(int64_t)x;
}

/* ---------- f16 helpers ---------- */

/* fromFloat16, src/gguf.js:398-408 (identical to src/dtype.js:60-79):
 * exact decode of an IEEE half. */
double oracle_from_f16(uint16_t h) {
  int sign = (h >> 15) & 1;
  int e = (h >> 10) & 0x1f;
  int frac = h & 0x3ff;
  double v;
  if (e == 0) {
    if (frac == 0) return sign ? -0.0 : 0.0;
    v = ldexp(1.0, -14) * (frac / 1024.0);
  } else if (e == 31) {
    return frac ? NAN : (sign ? -INFINITY : INFINITY);
  } else {
    v = ldexp(1.0, e - 15) * (1.0 + frac / 1024.0);
  }
  return sign ? -v : v;
}

/* toFloat16, src/dtype.js:29-58: TRUNCATING f32 -> f16 encoder. */
uint16_t oracle_to_f16_trunc(float val) {
  uint32_t bits;
  memcpy(&bits, &val, 4);
  uint32_t sign = (bits >> 31) & 1;
  int e = (bits >> 23) & 0xff;
  uint32_t frac = bits & 0x7fffff;
  if (e == 0xff) return (uint16_t)((sign << 15) | 0x7c00 | (frac ? 0x200 : 0));
  e -= 127;
  if (e > 15) return (uint16_t)((sign << 15) | 0x7c00);
  if (e < -14) {
    if (e < -24) return (uint16_t)(sign << 15);
    frac |= 0x800000;
    int shift = -1 - e;
    frac >>= shift;
    return (uint16_t)((sign << 15) | (frac >> 13));
  }
  return (uint16_t)((sign << 15) | ((uint32_t)(e + 15) << 10) | (frac >> 13));
}

/* IEEE round-to-nearest-even f32 -> f16 (what ggml's FP32_TO_FP16 does).
 * Used by the Q8_0 / Q4_0 quantizers this build defines for the formats the
 * reference only decodes. */
uint16_t oracle_f32_to_f16_rne(float val) {
  uint32_t x;
  memcpy(&x, &val, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520 -> inf */
  if (ax < 0x38800000u) {
    /* result is subnormal (or zero): value / 2^-24, rounded to nearest even */
    if (ax < 0x33000000u) return (uint16_t)sign; /* < 2^-25: rounds to 0 */
    int e = (int)(ax >> 23);
    uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    int shift = 126 - e; /* value = m * 2^(e-150); want units of 2^-24 */
    uint32_t q = m >> (shift);
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t e = ((ax >> 23) - 112u) << 10;
  uint32_t m = ax & 0x7fffffu;
  uint32_t h = e | (m >> 13);
  uint32_t rem = m & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}

/* ---------- Q4S: the reference's quantizeQ4 format ---------- */

/* quantizeQ4, src/ops/quantize.js:14-68.  w is the f32 [K,N] row-major
 * weight; out receives ceil(K/32)*N*24 bytes.  Record (g, col) sits at byte
 * (g*N + col)*24: 16 nibble bytes (element k -> byte k>>1, low nibble when k
 * is even), then the f32 scale, then the f32 zero point.  All arithmetic is
 * f64 as in JS; scale/zero are rounded to f32 on store (Float32Array). */
void oracle_quantize_q4s(const float* w, int64_t K, int64_t N, uint8_t* out) {
  int64_t groups = (K + Q4S_GROUP - 1) / Q4S_GROUP;
  memset(out, 0, (size_t)(groups * N * Q4S_BYTES));
  for (int64_t g = 0; g < groups; g++) {
    int64_t k0 = g * Q4S_GROUP;
    int64_t k1 = k0 + Q4S_GROUP < K ? k0 + Q4S_GROUP : K;
    for (int64_t col = 0; col < N; col++) {
      double mn = INFINITY, mx = -INFINITY;
      for (int64_t k = k0; k < k1; k++) {
        double v = (double)w[k * N + col];
        if (v < mn) mn = v;
        if (v > mx) mx = v;
      }
      double range = mx - mn;
      double scale = range > 0 ? range / 15.0 : 1.0;
      double zero = range > 0 ? -mn / scale : 8.0;
      uint8_t* rec = out + (g * N + col) * Q4S_BYTES;
      int64_t valid = k1 - k0;
      for (int k = 0; k < Q4S_GROUP; k++) {
        double v = k < valid ? (double)w[(k0 + k) * N + col] : 0.0;
        double q = js_round(js_min(15.0, js_max(0.0, v / scale + zero)));
        uint32_t qi = js_to_u32(q);
        if (k & 1) rec[k >> 1] |= (uint8_t)(qi << 4);
        else rec[k >> 1] = (uint8_t)qi;
      }
      float s32 = (float)scale, z32 = (float)zero;
      memcpy(rec + 16, &s32, 4);
      memcpy(rec + 20, &z32, 4);
    }
  }
}

/* dequant_q4, shaders/matmul_q4.metal:24-28, in f32:
 * scale * (float(nibble) - zero).  Writes the [K,N] f32 weight. */
void oracle_dequant_q4s(const uint8_t* q, int64_t K, int64_t N, float* w) {
  for (int64_t k = 0; k < K; k++) {
    int64_t g = k / Q4S_GROUP, kk = k % Q4S_GROUP;
    for (int64_t col = 0; col < N; col++) {
      const uint8_t* rec = q + (g * N + col) * Q4S_BYTES;
      float scale, zero;
      memcpy(&scale, rec + 16, 4);
      memcpy(&zero, rec + 20, 4);
      uint8_t b = rec[kk >> 1];
      uint8_t nib = (kk & 1) ? (b >> 4) : (b & 0x0f);
      float t = (float)nib - zero;
      w[k * N + col] = scale * t;
    }
  }
}

/* ---------- Q8 (matmulQ8's block layout) ---------- */

/* The reference has no Q8 quantizer; matmulQ8 (src/ops/quantize.js:99-118)
 * consumes blocks laid out as shaders/matmul_q8.metal:40-52 reads them:
 * block (g, col) at byte (g*N + col)*34, f16 scale at +0, 32 x int8 at +2.
 * This quantizer follows ggml's published quantize_row_q8_0_ref (ggml
 * v0.0-era, file ggml-quants.c): amax = max|x|; d = amax/127 (f32);
 * id = d ? 1/d : 0; scale stored as round-to-nearest-even f16(d);
 * q = roundf(x*id) (round half away from zero).  Elements k >= K are 0. */
void oracle_quantize_q8(const float* w, int64_t K, int64_t N, uint8_t* out) {
  int64_t groups = (K + 31) / 32;
  for (int64_t g = 0; g < groups; g++) {
    for (int64_t col = 0; col < N; col++) {
      float x[32];
      float amax = 0.0f;
      for (int k = 0; k < 32; k++) {
        int64_t kk = g * 32 + k;
        x[k] = kk < K ? w[kk * N + col] : 0.0f;
        float a = fabsf(x[k]);
        if (a > amax) amax = a;
      }
      float d = amax / 127.0f;
      float id = d != 0.0f ? 1.0f / d : 0.0f;
      uint8_t* blk = out + (g * N + col) * Q8_BYTES;
      uint16_t h = oracle_f32_to_f16_rne(d);
      blk[0] = (uint8_t)(h & 0xff);
      blk[1] = (uint8_t)(h >> 8);
      for (int k = 0; k < 32; k++) {
        float p = x[k] * id;
        blk[2 + k] = (uint8_t)(int8_t)roundf(p);
      }
    }
  }
}

/* matmul_q8 dequant, shaders/matmul_q8.metal:44-52: float(half scale) *
 * float(int8), in f32. */
void oracle_dequant_q8(const uint8_t* q, int64_t K, int64_t N, float* w) {
  for (int64_t k = 0; k < K; k++) {
    int64_t g = k / 32, kk = k % 32;
    for (int64_t col = 0; col < N; col++) {
      const uint8_t* blk = q + (g * N + col) * Q8_BYTES;
      uint16_t h = (uint16_t)(blk[0] | (blk[1] << 8));
      float s = (float)oracle_from_f16(h);
      int8_t v = (int8_t)blk[2 + kk];
      w[k * N + col] = s * (float)v;
    }
  }
}

/* ---------- GGUF Q4_0 / Q8_0 blocks ---------- */

/* dequantQ4_0, src/gguf.js:187-197: block = f16 d, then 16 nibble bytes;
 * element i is the LOW nibble of byte i>>1 when i is even, HIGH when odd
 * (interleaved, unlike llama.cpp).  value = d * (nibble - 8), computed in
 * f64 and stored to Float32Array. */
void oracle_dequant_q4_0_block(const uint8_t* blk, float* out32) {
  double d = oracle_from_f16((uint16_t)(blk[0] | (blk[1] << 8)));
  for (int i = 0; i < 32; i++) {
    uint8_t b = blk[2 + (i >> 1)];
    int nib = (i & 1) ? (b >> 4) : (b & 0x0f);
    out32[i] = (float)(d * (double)(nib - 8));
  }
}

/* dequantQ8_0, src/gguf.js:221-231: f16 d then 32 int8; d * int8 in f64. */
void oracle_dequant_q8_0_block(const uint8_t* blk, float* out32) {
  double d = oracle_from_f16((uint16_t)(blk[0] | (blk[1] << 8)));
  for (int i = 0; i < 32; i++) {
    uint8_t v = blk[2 + i];
    out32[i] = (float)(d * (double)(v > 127 ? (int)v - 256 : (int)v));
  }
}

/* dequantizeTensor, src/gguf.js:343-394, for Q4_0 (type 2) and Q8_0 (type 8):
 * blocks in storage order along the flat tensor; the last block is cut at
 * numElements. */
int oracle_dequantize_tensor(int type, const uint8_t* data, int64_t numel, float* out) {
  int bpb;
  void (*fn)(const uint8_t*, float*);
  if (type == 2) { bpb = Q4_0_BYTES; fn = oracle_dequant_q4_0_block; }
  else if (type == 8) { bpb = Q8_BYTES; fn = oracle_dequant_q8_0_block; }
  else return -1;
  int64_t blocks = (numel + 31) / 32;
  float tmp[32];
  for (int64_t b = 0; b < blocks; b++) {
    fn(data + b * bpb, tmp);
    int64_t cnt = numel - b * 32 < 32 ? numel - b * 32 : 32;
    memcpy(out + b * 32, tmp, (size_t)cnt * 4);
  }
  return 0;
}

/* Q4_0 encoder for the synthetic GGUF files this build writes (the reference
 * has none).  Follows ggml's published quantize_row_q4_0_ref: take the
 * element with the largest magnitude (signed, first one wins); d = max / -8;
 * id = d ? 1/d : 0; q = min(15, (int8)(x*id + 8.5f)); d stored as
 * round-to-nearest-even f16.  Packing uses the reference decoder's
 * interleaved nibble order (element i in byte i>>1, low nibble if even).
 * row points at 32 consecutive weights (k >= K padded with 0). */
void oracle_quantize_q4_0_block(const float* x, uint8_t* blk) {
  float amax = 0.0f, mx = 0.0f;
  for (int i = 0; i < 32; i++) {
    if (amax < fabsf(x[i])) { amax = fabsf(x[i]); mx = x[i]; }
  }
  float d = mx / -8.0f;
  float id = d != 0.0f ? 1.0f / d : 0.0f;
  uint16_t h = oracle_f32_to_f16_rne(d);
  blk[0] = (uint8_t)(h & 0xff);
  blk[1] = (uint8_t)(h >> 8);
  memset(blk + 2, 0, 16);
  for (int i = 0; i < 32; i++) {
    float t = x[i] * id + 8.5f;
    int8_t qi = (int8_t)t;
    int q = qi < 15 ? qi : 15;
    if (i & 1) blk[2 + (i >> 1)] |= (uint8_t)(q << 4);
    else blk[2 + (i >> 1)] |= (uint8_t)q;
  }
}

/* Q8_0 encoder with GGUF block order (32 consecutive elements per block). */
void oracle_quantize_q8_0_block(const float* x, uint8_t* blk) {
  float amax = 0.0f;
  for (int i = 0; i < 32; i++) {
    float a = fabsf(x[i]);
    if (a > amax) amax = a;
  }
  float d = amax / 127.0f;
  float id = d != 0.0f ? 1.0f / d : 0.0f;
  uint16_t h = oracle_f32_to_f16_rne(d);
  blk[0] = (uint8_t)(h & 0xff);
  blk[1] = (uint8_t)(h >> 8);
  for (int i = 0; i < 32; i++) blk[2 + i] = (uint8_t)(int8_t)roundf(x[i] * id);
}

/* Quantize a [rows, cols] f32 matrix row by row into GGUF blocks
 * (type 2 = Q4_0, 8 = Q8_0); cols is padded up to a multiple of 32 with 0. */
int oracle_quantize_rows(int type, const float* x, int64_t rows, int64_t cols, uint8_t* out) {
  int bpb = type == 2 ? Q4_0_BYTES : (type == 8 ? Q8_BYTES : 0);
  if (!bpb) return -1;
  int64_t bpr = (cols + 31) / 32;
  float tmp[32];
  for (int64_t r = 0; r < rows; r++) {
    for (int64_t b = 0; b < bpr; b++) {
      for (int i = 0; i < 32; i++) {
        int64_t c = b * 32 + i;
        tmp[i] = c < cols ? x[r * cols + c] : 0.0f;
      }
      uint8_t* blk = out + (r * bpr + b) * bpb;
      if (type == 2) oracle_quantize_q4_0_block(tmp, blk);
      else oracle_quantize_q8_0_block(tmp, blk);
    }
  }
  return 0;
}

/* ---------- matmul references ---------- */

/* C[M,N] = A[M,K] . W[K,N] with f64 accumulation (the exact value the f32
 * dequantize-then-matmul approximates; matmul_q4.metal:34-65 and
 * matmul_q8.metal:20-57 accumulate the same products in f32). */
void oracle_matmul_f64acc(const float* a, const float* w, int64_t M, int64_t N, int64_t K, float* c) {
  double* acc = (double*)malloc((size_t)N * sizeof(double));
  for (int64_t m = 0; m < M; m++) {
    for (int64_t n = 0; n < N; n++) acc[n] = 0.0;
    for (int64_t k = 0; k < K; k++) {
      double av = a[m * K + k];
      const float* wr = w + k * N;
      for (int64_t n = 0; n < N; n++) acc[n] += av * (double)wr[n];
    }
    for (int64_t n = 0; n < N; n++) c[m * N + n] = (float)acc[n];
  }
  free(acc);
}

/* The reference CPU path as the baseline times it: dequantize the whole
 * weight to f32, then a plain f32 triple loop (k-sequential accumulation,
 * as matmul_q4.metal:47-57 does per output). */
void oracle_matmul_f32(const float* a, const float* w, int64_t M, int64_t N, int64_t K, float* c) {
  for (int64_t m = 0; m < M; m++) {
    float* cr = c + m * N;
    for (int64_t n = 0; n < N; n++) cr[n] = 0.0f;
    for (int64_t k = 0; k < K; k++) {
      float av = a[m * K + k];
      const float* wr = w + k * N;
      for (int64_t n = 0; n < N; n++) cr[n] += av * wr[n];
    }
  }
}

/* matmulQ4 oracle: dequantize Q4S then f64-accumulated matmul. */
void oracle_matmul_q4s(const float* a, const uint8_t* q, int64_t M, int64_t N, int64_t K, float* c) {
  float* w = (float*)malloc((size_t)(K * N) * 4);
  oracle_dequant_q4s(q, K, N, w);
  oracle_matmul_f64acc(a, w, M, N, K, c);
  free(w);
}

/* matmulQ8 oracle: dequantize Q8 then f64-accumulated matmul. */
void oracle_matmul_q8(const float* a, const uint8_t* q, int64_t M, int64_t N, int64_t K, float* c) {
  float* w = (float*)malloc((size_t)(K * N) * 4);
  oracle_dequant_q8(q, K, N, w);
  oracle_matmul_f64acc(a, w, M, N, K, c);
  free(w);
}

/* GGUF Q4_0/Q8_0 weight listed [out=N, in=K] (blocks along K per output
 * row): y[M,N] = A[M,K] . W^T, the transpose gguf_loader.js:243-253 applies
 * for a [out,in] listing.  f64 accumulation. */
int oracle_matmul_gguf(int type, const float* a, const uint8_t* q, int64_t M, int64_t N, int64_t K, float* c) {
  int64_t kp = (K + 31) / 32 * 32;
  float* wt = (float*)malloc((size_t)(N * kp) * 4);
  int bpb = type == 2 ? Q4_0_BYTES : Q8_BYTES;
  for (int64_t n = 0; n < N; n++) {
    if (oracle_dequantize_tensor(type, q + n * (kp / 32) * bpb, kp, wt + n * kp)) { free(wt); return -1; }
  }
  for (int64_t m = 0; m < M; m++) {
    for (int64_t n = 0; n < N; n++) {
      double acc = 0.0;
      for (int64_t k = 0; k < K; k++) acc += (double)a[m * K + k] * (double)wt[n * kp + k];
      c[m * N + n] = (float)acc;
    }
  }
  free(wt);
  return 0;
}
