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
  const int64_t G = (K + 31) / 32;
  float* sc = (float*)malloc((size_t)N * sizeof(float));
  for (int64_t g = 0; g < G; g++) {
    for (int64_t col = 0; col < N; col++) { /* each block's scale once */
      const uint8_t* blk = q + (g * N + col) * Q8_BYTES;
      sc[col] = (float)oracle_from_f16((uint16_t)(blk[0] | (blk[1] << 8)));
    }
    for (int64_t kk = 0; kk < 32 && g * 32 + kk < K; kk++)
      for (int64_t col = 0; col < N; col++)
        w[(g * 32 + kk) * N + col] = sc[col] * (float)(int8_t)q[(g * N + col) * Q8_BYTES + 2 + kk];
  }
  free(sc);
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

/* dequantQ4_1, src/gguf.js:203-215: f16 d, f16 m, 16 nibble bytes
 * (interleaved order as Q4_0); value = d * nibble + m in f64, stored f32. */
void oracle_dequant_q4_1_block(const uint8_t* blk, float* out32) {
  double d = oracle_from_f16((uint16_t)(blk[0] | (blk[1] << 8)));
  double m = oracle_from_f16((uint16_t)(blk[2] | (blk[3] << 8)));
  for (int i = 0; i < 32; i++) {
    uint8_t b = blk[4 + (i >> 1)];
    int nib = (i & 1) ? (b >> 4) : (b & 0x0f);
    out32[i] = (float)(d * (double)nib + m);
  }
}

/* dequantQ5_0, src/gguf.js:238-259: f16 d, a 32-bit little-endian word of
 * fifth bits (bit i for element i), 16 nibble bytes (interleaved order);
 * value = d * ((nibble | bit << 4) - 16) in f64, stored f32. */
void oracle_dequant_q5_0_block(const uint8_t* blk, float* out32) {
  double d = oracle_from_f16((uint16_t)(blk[0] | (blk[1] << 8)));
  uint32_t hb = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8) | ((uint32_t)blk[4] << 16) | ((uint32_t)blk[5] << 24);
  for (int i = 0; i < 32; i++) {
    uint8_t b = blk[6 + (i >> 1)];
    int nib = (i & 1) ? (b >> 4) : (b & 0x0f);
    int q = nib | (int)(((hb >> i) & 1u) << 4);
    out32[i] = (float)(d * (double)(q - 16));
  }
}

/* The 6-bit (scale, min) pair of sub-block i of a Q4_K super-block as the
 * reference unpacks it (src/gguf.js:281-291): i < 4: low 6 bits of bytes i
 * and i+4; i >= 4: scale = (byte[i-4] >> 6) | (low nibble of byte[i+4]) << 2,
 * min = (byte[i] >> 6) | (high nibble of byte[i+4]) << 2.  (The bit order of
 * the i >= 4 case differs from llama.cpp's get_scale_min_k4; the reference's
 * is the one restated.) */
void oracle_q4_k_scale_min(const uint8_t* sc12, int i, int* sc, int* mn) {
  if (i < 4) {
    *sc = sc12[i] & 0x3f;
    *mn = sc12[4 + i] & 0x3f;
  } else {
    *sc = (sc12[i - 4] >> 6) | ((sc12[i + 4] & 0x0f) << 2);
    *mn = (sc12[i] >> 6) | ((sc12[i + 4] >> 4) << 2);
  }
}

/* dequantQ4_K, src/gguf.js:264-305: 256 elements; f16 d, f16 dmin, 12 bytes
 * of packed 6-bit scales/mins, 128 nibble bytes with element j in byte j>>1
 * (low nibble if j even).  sc = f32(d * scale), mn = f32(dmin * min)
 * (Float32Array stores); value = sc * nibble - mn in f64, stored f32. */
void oracle_dequant_q4_k_block(const uint8_t* blk, float* out256) {
  double d = oracle_from_f16((uint16_t)(blk[0] | (blk[1] << 8)));
  double dmin = oracle_from_f16((uint16_t)(blk[2] | (blk[3] << 8)));
  float sc[8], mn[8];
  for (int i = 0; i < 8; i++) {
    int s, m;
    oracle_q4_k_scale_min(blk + 4, i, &s, &m);
    sc[i] = (float)(d * s);
    mn[i] = (float)(dmin * m);
  }
  for (int j = 0; j < 256; j++) {
    uint8_t b = blk[16 + (j >> 1)];
    int nib = (j & 1) ? (b >> 4) : (b & 0x0f);
    out256[j] = (float)((double)sc[j >> 5] * nib - (double)mn[j >> 5]);
  }
}

/* dequantQ6_K, src/gguf.js:309-339: 256 elements; ql[128] (element j: nibble
 * of byte j>>1, low if j even), qh[64] (element j: bits (j&3)*2.. of byte
 * j>>2), int8 scales[16] (one per 16 elements), f16 d at byte 208;
 * value = d * scale * (q - 32) evaluated left to right in f64, stored f32. */
void oracle_dequant_q6_k_block(const uint8_t* blk, float* out256) {
  double d = oracle_from_f16((uint16_t)(blk[208] | (blk[209] << 8)));
  for (int j = 0; j < 256; j++) {
    uint8_t lb = blk[j >> 1];
    int ql = (j & 1) ? (lb >> 4) : (lb & 0x0f);
    int qh = (blk[128 + (j >> 2)] >> ((j & 3) * 2)) & 3;
    int q = ql | (qh << 4);
    int sc = (int8_t)blk[192 + (j >> 4)];
    out256[j] = (float)(d * (double)sc * (double)(q - 32));
  }
}

/* GGML type numbers (src/gguf.js:15-25) and block geometry (:30-41). */
int oracle_block_geometry(int type, int* elems, int* bytes) {
  switch (type) {
    case 0: *elems = 1; *bytes = 4; return 0;     /* F32 */
    case 1: *elems = 1; *bytes = 2; return 0;     /* F16 */
    case 30: *elems = 1; *bytes = 2; return 0;    /* BF16 */
    case 2: *elems = 32; *bytes = 18; return 0;   /* Q4_0 */
    case 3: *elems = 32; *bytes = 20; return 0;   /* Q4_1 */
    case 6: *elems = 32; *bytes = 22; return 0;   /* Q5_0 */
    case 8: *elems = 32; *bytes = 34; return 0;   /* Q8_0 */
    case 12: *elems = 256; *bytes = 144; return 0; /* Q4_K */
    case 14: *elems = 256; *bytes = 210; return 0; /* Q6_K */
    default: return -1;
  }
}

/* dequantizeTensor, src/gguf.js:343-394: F32 as stored, F16 by fromFloat16,
 * BF16 by a 16-bit shift, block types block by block in storage order along
 * the flat tensor with the last block cut at numElements. */
int oracle_dequantize_tensor(int type, const uint8_t* data, int64_t numel, float* out) {
  int be, bb;
  if (oracle_block_geometry(type, &be, &bb)) return -1;
  if (type == 0) { memcpy(out, data, (size_t)numel * 4); return 0; }
  if (type == 1 || type == 30) {
    for (int64_t i = 0; i < numel; i++) {
      uint16_t h = (uint16_t)(data[2 * i] | (data[2 * i + 1] << 8));
      if (type == 1) out[i] = (float)oracle_from_f16(h);
      else { uint32_t u = (uint32_t)h << 16; memcpy(out + i, &u, 4); }
    }
    return 0;
  }
  void (*fn)(const uint8_t*, float*) = 0;
  switch (type) {
    case 2: fn = oracle_dequant_q4_0_block; break;
    case 3: fn = oracle_dequant_q4_1_block; break;
    case 6: fn = oracle_dequant_q5_0_block; break;
    case 8: fn = oracle_dequant_q8_0_block; break;
    case 12: fn = oracle_dequant_q4_k_block; break;
    case 14: fn = oracle_dequant_q6_k_block; break;
  }
  int64_t blocks = (numel + be - 1) / be;
  float tmp[256];
  for (int64_t b = 0; b < blocks; b++) {
    fn(data + b * bb, tmp);
    int64_t cnt = numel - b * be < be ? numel - b * be : be;
    memcpy(out + b * be, tmp, (size_t)cnt * 4);
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

/* Encoders for the other block types, written for this build's synthetic
 * files (the reference has none).  Each packs in the layout the reference's
 * decoder above reads; the rounding choices are this build's. */

static void put_f16(uint8_t* p, float v) {
  uint16_t h = oracle_f32_to_f16_rne(v);
  p[0] = (uint8_t)(h & 0xff);
  p[1] = (uint8_t)(h >> 8);
}
static void put_nib(uint8_t* qs, int i, int q) { qs[i >> 1] |= (uint8_t)((i & 1) ? (q << 4) : q); }
static int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* Q4_1 as ggml's quantize_row_q4_1_ref: d = (max - min) / 15, m = min,
 * q = min(15, (int8)((x - min) / d + 0.5f)). */
void oracle_quantize_q4_1_block(const float* x, uint8_t* blk) {
  float mn = x[0], mx = x[0];
  for (int i = 1; i < 32; i++) { if (x[i] < mn) mn = x[i]; if (x[i] > mx) mx = x[i]; }
  float d = (mx - mn) / 15.0f;
  float id = d != 0.0f ? 1.0f / d : 0.0f;
  put_f16(blk, d);
  put_f16(blk + 2, mn);
  memset(blk + 4, 0, 16);
  for (int i = 0; i < 32; i++) {
    int8_t qi = (int8_t)((x[i] - mn) * id + 0.5f);
    put_nib(blk + 4, i, qi < 15 ? qi : 15);
  }
}

/* Q5_0 as ggml's quantize_row_q5_0_ref: signed extreme max, d = max / -16,
 * q = min(31, (int8)(x / d + 16.5f)); nibble and fifth bit of element i in
 * the reference's order. */
void oracle_quantize_q5_0_block(const float* x, uint8_t* blk) {
  float amax = 0.0f, mx = 0.0f;
  for (int i = 0; i < 32; i++) if (amax < fabsf(x[i])) { amax = fabsf(x[i]); mx = x[i]; }
  float d = mx / -16.0f;
  float id = d != 0.0f ? 1.0f / d : 0.0f;
  put_f16(blk, d);
  uint32_t hb = 0;
  memset(blk + 6, 0, 16);
  for (int i = 0; i < 32; i++) {
    int8_t qi = (int8_t)(x[i] * id + 16.5f);
    int q = qi < 31 ? qi : 31;
    put_nib(blk + 6, i, q & 15);
    hb |= (uint32_t)(q >> 4) << i;
  }
  for (int k = 0; k < 4; k++) blk[2 + k] = (uint8_t)(hb >> (8 * k));
}

/* Q4_K: per 32-element sub-block, step = (max - min) / 15 and offset = -min
 * (min clamped to <= 0); d = max step / 63, dmin = max offset / 63 (f16);
 * 6-bit ints round(step / d), round(offset / dmin); then
 * q = clamp(round((x + dmin*m) / (d*s)), 0, 15) with the stored values. */
void oracle_quantize_q4_k_block(const float* x, uint8_t* blk) {
  float step[8], offs[8], smax = 0.0f, omax = 0.0f;
  for (int i = 0; i < 8; i++) {
    float mn = 0.0f, mx = 0.0f;
    for (int k = 0; k < 32; k++) {
      float v = x[32 * i + k];
      if (k == 0 || v < mn) mn = v;
      if (k == 0 || v > mx) mx = v;
    }
    if (mn > 0.0f) mn = 0.0f;
    step[i] = (mx - mn) / 15.0f;
    offs[i] = -mn;
    if (step[i] > smax) smax = step[i];
    if (offs[i] > omax) omax = offs[i];
  }
  put_f16(blk, smax / 63.0f);
  put_f16(blk + 2, omax / 63.0f);
  float d = (float)oracle_from_f16((uint16_t)(blk[0] | (blk[1] << 8)));
  float dmin = (float)oracle_from_f16((uint16_t)(blk[2] | (blk[3] << 8)));
  uint8_t* s12 = blk + 4;
  memset(s12, 0, 12);
  int S[8], Mi[8];
  for (int i = 0; i < 8; i++) {
    S[i] = d > 0.0f ? clampi((int)roundf(step[i] / d), 0, 63) : 0;
    Mi[i] = dmin > 0.0f ? clampi((int)roundf(offs[i] / dmin), 0, 63) : 0;
    if (i < 4) {
      s12[i] |= (uint8_t)S[i];
      s12[4 + i] |= (uint8_t)Mi[i];
    } else {
      s12[i - 4] |= (uint8_t)((S[i] & 3) << 6);
      s12[i + 4] |= (uint8_t)((S[i] >> 2) | ((Mi[i] >> 2) << 4));
      s12[i] |= (uint8_t)((Mi[i] & 3) << 6);
    }
  }
  memset(blk + 16, 0, 128);
  for (int j = 0; j < 256; j++) {
    float sc = d * (float)S[j >> 5], mn = dmin * (float)Mi[j >> 5];
    int q = sc > 0.0f ? clampi((int)roundf((x[j] + mn) / sc), 0, 15) : 0;
    put_nib(blk + 16, j, q);
  }
}

/* Q6_K: per 16-element sub-block the signed extreme max, scale = max / -32;
 * d = (largest |scale|) / 127 (f16); int8 s = clamp(round(scale / d));
 * q = clamp(round(x / (d*s)), -32, 31) + 32 in the reference's ql/qh order. */
void oracle_quantize_q6_k_block(const float* x, uint8_t* blk) {
  float scl[16], amx = 0.0f;
  for (int i = 0; i < 16; i++) {
    float am = 0.0f, mx = 0.0f;
    for (int k = 0; k < 16; k++) {
      float v = x[16 * i + k];
      if (am < fabsf(v)) { am = fabsf(v); mx = v; }
    }
    scl[i] = mx / -32.0f;
    if (fabsf(scl[i]) > amx) amx = fabsf(scl[i]);
  }
  memset(blk, 0, 210);
  put_f16(blk + 208, amx / 127.0f);
  float d = (float)oracle_from_f16((uint16_t)(blk[208] | (blk[209] << 8)));
  for (int i = 0; i < 16; i++) {
    int s = d > 0.0f ? clampi((int)roundf(scl[i] / d), -128, 127) : 0;
    blk[192 + i] = (uint8_t)(int8_t)s;
    float step = d * (float)s;
    for (int k = 0; k < 16; k++) {
      int j = 16 * i + k;
      int q = step != 0.0f ? clampi((int)roundf(x[j] / step), -32, 31) + 32 : 32;
      put_nib(blk, j, q & 15);
      blk[128 + (j >> 2)] |= (uint8_t)((q >> 4) << ((j & 3) * 2));
    }
  }
}

/* Quantize a [rows, cols] f32 matrix row by row into GGUF blocks of any of
 * the block types above; cols is padded up to a multiple of the block size
 * with 0. */
int oracle_quantize_rows(int type, const float* x, int64_t rows, int64_t cols, uint8_t* out) {
  int be, bb;
  if (oracle_block_geometry(type, &be, &bb) || be == 1) return -1;
  void (*fn)(const float*, uint8_t*) = 0;
  switch (type) {
    case 2: fn = oracle_quantize_q4_0_block; break;
    case 3: fn = oracle_quantize_q4_1_block; break;
    case 6: fn = oracle_quantize_q5_0_block; break;
    case 8: fn = oracle_quantize_q8_0_block; break;
    case 12: fn = oracle_quantize_q4_k_block; break;
    case 14: fn = oracle_quantize_q6_k_block; break;
  }
  int64_t bpr = (cols + be - 1) / be;
  float tmp[256];
  for (int64_t r = 0; r < rows; r++) {
    for (int64_t b = 0; b < bpr; b++) {
      for (int i = 0; i < be; i++) {
        int64_t c = b * be + i;
        tmp[i] = c < cols ? x[r * cols + c] : 0.0f;
      }
      fn(tmp, out + (r * bpr + b) * bb);
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
  int be, bb;
  if (oracle_block_geometry(type, &be, &bb) || be == 1) return -1;
  int64_t kp = (K + be - 1) / be * be;
  float* wt = (float*)malloc((size_t)(N * kp) * 4);
  for (int64_t n = 0; n < N; n++) {
    if (oracle_dequantize_tensor(type, q + n * (kp / be) * bb, kp, wt + n * kp)) { free(wt); return -1; }
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
