// llama_kernels.hip -- gfx950 kernels for the GGUF Llama decode/prefill path
// that loadGGUF(...).generate runs around the quantized GEMVs
// (src/gguf_cache.js:109-265).  Built into its own code object
// (smith_llama.hsaco); every kernel is extern "C".
//
// Positions are read from device memory (pos_ptr) so a whole decode step can
// be captured once as a HIP graph and replayed.
#include <hip/hip_runtime.h>
#include <stdint.h>

// ---------------------------------------------------------------------------
// RMSNorm rows: y = x * rsqrt(mean(x^2) + eps) * gamma
// (shaders/rmsnorm.metal:15-47; one workgroup per row).
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void smith_rmsnorm_rows(const float* __restrict__ x,
                                                                     const float* __restrict__ gamma,
                                                                     float* __restrict__ y, uint32_t rows,
                                                                     uint32_t cols, float eps) {
  __shared__ float red[8];
  uint32_t row = blockIdx.x;
  if (row >= rows) return;
  const float* xr = x + (size_t)row * cols;
  float ss = 0.f;
  for (uint32_t i = threadIdx.x; i < cols; i += blockDim.x) ss = __builtin_fmaf(xr[i], xr[i], ss);
  for (int d = 32; d >= 1; d >>= 1) ss += __shfl_xor(ss, d);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
  for (uint32_t w = 0; w < blockDim.x / 64; w++) tot += red[w];
  float rms = 1.0f / __builtin_sqrtf(tot / (float)cols + eps);
  for (uint32_t i = threadIdx.x; i < cols; i += blockDim.x) y[(size_t)row * cols + i] = xr[i] * rms * gamma[i];
}

// ---------------------------------------------------------------------------
// Embedding gather (autograd.js:308-334): out[r] = E[tokens[r]].
// ---------------------------------------------------------------------------
extern "C" __global__ void smith_embed_rows(const float* __restrict__ E, const int32_t* __restrict__ tokens,
                                            float* __restrict__ out, uint32_t rows, uint32_t dim) {
  uint32_t r = blockIdx.x;
  if (r >= rows) return;
  const float* src = E + (size_t)tokens[r] * dim;
  for (uint32_t i = threadIdx.x; i < dim; i += blockDim.x) out[(size_t)r * dim + i] = src[i];
}

// ---------------------------------------------------------------------------
// RoPE with the reference's WHOLE-ROW indexing (shaders/rope.metal:18-37 as
// gguf_cache.js:130-131 calls it on a [1, dim] projection): element i of a
// row of width W pairs with i + W/2 and uses table entry pos*(W/2) + (i mod
// W/2) of the flat [maxSeqLen, headDim/2] cos/sin tables (ops/rope.js:10-30).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float rope_elem(const float* __restrict__ row, uint32_t W, uint32_t i, uint32_t pos,
                                          const float* __restrict__ cosT, const float* __restrict__ sinT) {
  uint32_t half = W / 2;
  uint32_t p = i < half ? i : i - half;
  float x0 = row[p], x1 = row[p + half];
  size_t t = (size_t)pos * half + p;
  float c = cosT[t], s = sinT[t];
  return i < half ? x0 * c - x1 * s : x0 * s + x1 * c;
}

// ---------------------------------------------------------------------------
// Fused RoPE + KV-cache append + GQA attention, for S query rows at positions
// p0 .. p0+S-1 with p0 = *pos_ptr (gguf_cache.js:128-157 for decode,
// :212-231 for prefill).  qkv rows hold [q | k | v] (ld floats per row).
// Workgroup (h, s): q head h, row s; KV head kvh = h / (nH/nKV) (repeatKV,
// gguf_cache.js:90-105).  Keys of positions < p0 come from the cache; keys of
// p0..p0+s are roped here from the raw k of this launch (so no workgroup
// depends on another); the workgroup with h % (nH/nKV) == 0 writes row s's
// roped k and raw v into the cache.  scale = 1/sqrt(hd) after the dot
// product, softmax with max subtraction, out = P V.  hd <= 128, positions
// p0+S <= maxSeq, 256 threads.
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void smith_attention(
    const float* __restrict__ qkv, uint32_t ld, const int32_t* __restrict__ pos_ptr, uint32_t S, uint32_t nH,
    uint32_t nKV, uint32_t hd, const float* __restrict__ cosT, const float* __restrict__ sinT,
    float* __restrict__ kcache, float* __restrict__ vcache, uint32_t maxSeq, float* __restrict__ out) {
  extern __shared__ float sm[];
  const uint32_t h = blockIdx.x, s = blockIdx.y;
  const uint32_t p0 = (uint32_t)pos_ptr[0];
  const uint32_t pos = p0 + s;
  const uint32_t T = pos + 1;
  const uint32_t rep = nH / nKV, kvh = h / rep;
  const uint32_t Wq = nH * hd, Wk = nKV * hd;
  float* qr = sm;              // [hd]
  float* kn = sm + 128;        // [S][hd] roped new keys of rows 0..s (only 0..s used)
  float* sc = kn + S * 128;    // [T] scores
  __shared__ float red[8];
  __shared__ float stat[2];

  const float* qrow = qkv + (size_t)s * ld;
  for (uint32_t e = threadIdx.x; e < hd; e += blockDim.x) qr[e] = rope_elem(qrow, Wq, h * hd + e, pos, cosT, sinT);
  for (uint32_t idx = threadIdx.x; idx < (s + 1) * hd; idx += blockDim.x) {
    uint32_t r = idx / hd, e = idx % hd;
    kn[r * 128 + e] = rope_elem(qkv + (size_t)r * ld + Wq, Wk, kvh * hd + e, p0 + r, cosT, sinT);
  }
  __syncthreads();
  if (h % rep == 0) {
    const float* vrow = qkv + (size_t)s * ld + Wq + Wk;
    for (uint32_t e = threadIdx.x; e < hd; e += blockDim.x) {
      size_t o = ((size_t)kvh * maxSeq + pos) * hd + e;
      kcache[o] = kn[s * 128 + e];
      vcache[o] = vrow[kvh * hd + e];
    }
  }
  const float scale = 1.0f / __builtin_sqrtf((float)hd);
  // scores: one thread per position
  float mx = -__builtin_inff();
  for (uint32_t t = threadIdx.x; t < T; t += blockDim.x) {
    const float* kr = t < p0 ? kcache + ((size_t)kvh * maxSeq + t) * hd : kn + (t - p0) * 128;
    float d = 0.f;
    for (uint32_t e = 0; e < hd; e++) d = __builtin_fmaf(qr[e], kr[e], d);
    d *= scale;
    sc[t] = d;
    mx = d > mx ? d : mx;
  }
  for (int dd = 32; dd >= 1; dd >>= 1) {
    float o = __shfl_xor(mx, dd);
    mx = o > mx ? o : mx;
  }
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  if (threadIdx.x == 0) {
    float m = red[0];
    for (uint32_t w = 1; w < blockDim.x / 64; w++) m = red[w] > m ? red[w] : m;
    stat[0] = m;
  }
  __syncthreads();
  mx = stat[0];
  float sum = 0.f;
  for (uint32_t t = threadIdx.x; t < T; t += blockDim.x) {
    float e = __expf(sc[t] - mx);
    sc[t] = e;
    sum += e;
  }
  for (int dd = 32; dd >= 1; dd >>= 1) sum += __shfl_xor(sum, dd);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = sum;
  __syncthreads();
  if (threadIdx.x == 0) {
    float tot = 0.f;
    for (uint32_t w = 0; w < blockDim.x / 64; w++) tot += red[w];
    stat[1] = 1.0f / tot;
  }
  __syncthreads();
  const float inv = stat[1];
  // out[e] = sum_t p_t v_t[e]: thread (e, part) over interleaved positions
  const uint32_t parts = blockDim.x / hd;  // hd divides 256 (64 or 128)
  const uint32_t e = threadIdx.x % hd, part = threadIdx.x / hd;
  float acc = 0.f;
  for (uint32_t t = part; t < T; t += parts) {
    float v = t < p0 ? vcache[((size_t)kvh * maxSeq + t) * hd + e]
                     : qkv[(size_t)(t - p0) * ld + Wq + Wk + kvh * hd + e];
    acc = __builtin_fmaf(sc[t], v, acc);
  }
  __syncthreads();
  sc[threadIdx.x] = acc;  // scores are consumed; reuse for the part reduction
  __syncthreads();
  if (part == 0) {
    float v = 0.f;
    for (uint32_t q = 0; q < parts; q++) v += sc[q * hd + e];
    out[(size_t)s * Wq + h * hd + e] = v * inv;
  }
}

// ---------------------------------------------------------------------------
// LM head on the GGUF output.weight as the reference loads it: the flat data
// is read as lmHead[dim][vocab] (gguf_loader.js:240-259 never transposes a
// path that does not end in ".weight"), so for Q4_0 the 32-weight blocks run
// along the VOCAB axis: block (k, vb) at (k*(N/32) + vb)*18 covers
// lmHead[k][32vb .. 32vb+31] = d*(nib - 8) (interleaved nibbles).
// y[n] = sum_k x[k] * lmHead[k][n] for M = 1, optionally with the final
// RMSNorm of x fused (gamma != null).
// Lane (vb = lane/4, sub = lane%4) owns outputs 32vb + 8sub .. +7 of the 16
// blocks a workgroup covers (one dword of nibbles per row k); per row:
// c = x_k * d, 8 fma(c, nibble), and one -8c correction for the lane's 8
// outputs.  8 waves split the workgroup's K range (LDS reduction); K splits
// across workgroups (grid.y) are summed by the last-arriving workgroup.
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(512) void smith_lmhead_q4_0_nb(
    const float* __restrict__ x, const float* __restrict__ gamma, float eps, const uint8_t* __restrict__ W,
    float* __restrict__ y, uint32_t K, uint32_t N, float* __restrict__ ws, uint32_t* __restrict__ counters) {
  __shared__ float xs[8192];
  __shared__ float part[8][512];
  __shared__ float red[8];
  __shared__ int s_last;
  const uint32_t NB = N / 32;
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t vb = blockIdx.x * 16 + lane / 4, sub = lane & 3;
  const uint32_t ksplit = gridDim.y;
  const uint32_t kb = (K + ksplit - 1) / ksplit;
  const uint32_t kb0 = blockIdx.y * kb, kb1 = kb0 + kb < K ? kb0 + kb : K;
  float ss = 0.f;
  for (uint32_t i = threadIdx.x; i < K; i += 512) {
    float v = x[i];
    xs[i] = v;
    ss = __builtin_fmaf(v, v, ss);
  }
  if (gamma) {
    for (int d = 32; d >= 1; d >>= 1) ss += __shfl_xor(ss, d);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float tot = 0.f;
    for (int w = 0; w < 8; w++) tot += red[w];
    float rms = 1.0f / __builtin_sqrtf(tot / (float)K + eps);
    for (uint32_t i = threadIdx.x; i < K; i += 512) xs[i] = xs[i] * rms * gamma[i];
  }
  __syncthreads();
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; i++) acc[i] = 0.f;
  float corr = 0.f;
  const uint32_t kper = (kb1 - kb0 + 7) / 8;
  const uint32_t k0 = kb0 + wave * kper, k1 = k0 + kper < kb1 ? k0 + kper : kb1;
  if (vb < NB) {
    for (uint32_t k = k0; k < k1; k++) {
      const uint8_t* b = W + ((size_t)k * NB + vb) * 18;
      float c = xs[k] * (float)__builtin_bit_cast(_Float16, *(const uint16_t*)b);
      const uint16_t* q = (const uint16_t*)(b + 2 + 4 * sub);  // records are only 2-byte aligned
      uint32_t w = (uint32_t)q[0] | ((uint32_t)q[1] << 16);
      corr += c;
#pragma unroll
      for (int e = 0; e < 8; e++) acc[e] = __builtin_fmaf(c, (float)((w >> (4 * e)) & 15u), acc[e]);
    }
  }
#pragma unroll
  for (int e = 0; e < 8; e++) part[wave][lane * 8 + e] = __builtin_fmaf(-8.0f, corr, acc[e]);
  __syncthreads();
  const uint32_t nb0 = blockIdx.x * 512;
  for (uint32_t o = threadIdx.x; o < 512; o += 512) {
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < 8; w++) v += part[w][o];
    uint32_t n = nb0 + o;
    if (n >= N) continue;
    if (ksplit == 1)
      y[n] = v;
    else
      __hip_atomic_exchange((uint32_t*)ws + (size_t)blockIdx.y * N + n, __float_as_uint(v), __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_AGENT);
  }
  if (ksplit == 1) return;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t prev = __hip_atomic_fetch_add(counters + blockIdx.x, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == ksplit - 1;
  }
  __syncthreads();
  if (!s_last) return;
  for (uint32_t o = threadIdx.x; o < 512; o += 512) {
    uint32_t n = nb0 + o;
    if (n >= N) continue;
    float v = 0.f;
    for (uint32_t sp = 0; sp < ksplit; sp++)
      v += __uint_as_float(__hip_atomic_fetch_add((uint32_t*)ws + (size_t)sp * N + n, 0u, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT));
    y[n] = v;
  }
  if (threadIdx.x == 0)
    __hip_atomic_exchange(counters + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// f32 GEMV on a [K][N] row-major weight (an F32 output.weight read as
// lmHead[dim][vocab]): y[n] = sum_k x[k] W[k][n], optional fused RMSNorm.
// Threads along n (coalesced), 16 waves split K, LDS reduction.
extern "C" __global__ __launch_bounds__(1024) void smith_gemv_f32_kn(const float* __restrict__ x,
                                                                     const float* __restrict__ gamma, float eps,
                                                                     const float* __restrict__ W,
                                                                     float* __restrict__ y, uint32_t K,
                                                                     uint32_t N) {
  __shared__ float xs[8192];
  __shared__ float part[16][64];
  __shared__ float red[16];
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float ss = 0.f;
  for (uint32_t i = threadIdx.x; i < K; i += 1024) {
    float v = x[i];
    xs[i] = v;
    ss = __builtin_fmaf(v, v, ss);
  }
  if (gamma) {
    for (int d = 32; d >= 1; d >>= 1) ss += __shfl_xor(ss, d);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float tot = 0.f;
    for (int w = 0; w < 16; w++) tot += red[w];
    float rms = 1.0f / __builtin_sqrtf(tot / (float)K + eps);
    for (uint32_t i = threadIdx.x; i < K; i += 1024) xs[i] = xs[i] * rms * gamma[i];
  }
  __syncthreads();
  const uint32_t n = blockIdx.x * 64 + lane;
  const uint32_t kper = (K + 15) / 16;
  const uint32_t k0 = wave * kper, k1 = k0 + kper < K ? k0 + kper : K;
  float acc = 0.f;
  if (n < N)
    for (uint32_t k = k0; k < k1; k++) acc = __builtin_fmaf(xs[k], W[(size_t)k * N + n], acc);
  part[wave][lane] = acc;
  __syncthreads();
  if (wave == 0 && n < N) {
    float v = 0.f;
    for (int w = 0; w < 16; w++) v += part[w][lane];
    y[n] = v;
  }
}

// f32 GEMV on an [N][K] row-major weight (weight tying: logits = x . E^T,
// gguf_cache.js:180-181): y[n] = sum_k x[k] E[n][k].  One wave per output.
extern "C" __global__ __launch_bounds__(256) void smith_gemv_f32_nk(const float* __restrict__ x,
                                                                    const float* __restrict__ gamma, float eps,
                                                                    const float* __restrict__ E,
                                                                    float* __restrict__ y, uint32_t K,
                                                                    uint32_t N) {
  __shared__ float xs[8192];
  __shared__ float red[4];
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float ss = 0.f;
  for (uint32_t i = threadIdx.x; i < K; i += 256) {
    float v = x[i];
    xs[i] = v;
    ss = __builtin_fmaf(v, v, ss);
  }
  if (gamma) {
    for (int d = 32; d >= 1; d >>= 1) ss += __shfl_xor(ss, d);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float rms = 1.0f / __builtin_sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)K + eps);
    for (uint32_t i = threadIdx.x; i < K; i += 256) xs[i] = xs[i] * rms * gamma[i];
  }
  __syncthreads();
  for (uint32_t n = blockIdx.x * 4 + wave; n < N; n += gridDim.x * 4) {
    const float* er = E + (size_t)n * K;
    float acc = 0.f;
    for (uint32_t k = lane; k < K; k += 64) acc = __builtin_fmaf(xs[k], er[k], acc);
    for (int d = 32; d >= 1; d >>= 1) acc += __shfl_xor(acc, d);
    if (lane == 0) y[n] = acc;
  }
}

// ---------------------------------------------------------------------------
// Greedy step on device: token = argmax(logits) (generate.js:70-76: the
// first maximum wins), tokens[*count] = token, x = E[token], then *count and
// *pos advance.  One workgroup of 1024 threads.
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(1024) void smith_argmax_embed(const float* __restrict__ logits, uint32_t N,
                                                                      const float* __restrict__ E, uint32_t dim,
                                                                      float* __restrict__ x,
                                                                      int32_t* __restrict__ tokens,
                                                                      int32_t* __restrict__ count,
                                                                      int32_t* __restrict__ pos) {
  __shared__ float bv[16];
  __shared__ int32_t bi[16];
  __shared__ int32_t s_tok;
  float best = -__builtin_inff();
  int32_t bidx = 0x7fffffff;
  for (uint32_t i = threadIdx.x; i < N; i += 1024) {
    float v = logits[i];
    if (v > best) {  // strictly greater: earliest index within this thread
      best = v;
      bidx = (int32_t)i;
    }
  }
  for (int d = 32; d >= 1; d >>= 1) {
    float ov = __shfl_xor(best, d);
    int32_t oi = __shfl_xor(bidx, d);
    if (ov > best || (ov == best && oi < bidx)) {
      best = ov;
      bidx = oi;
    }
  }
  if ((threadIdx.x & 63) == 0) {
    bv[threadIdx.x >> 6] = best;
    bi[threadIdx.x >> 6] = bidx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = bv[0];
    int32_t t = bi[0];
    for (int w = 1; w < 16; w++)
      if (bv[w] > b || (bv[w] == b && bi[w] < t)) {
        b = bv[w];
        t = bi[w];
      }
    if (t == 0x7fffffff) t = 0;  // all NaN: the reference's argmax returns 0
    s_tok = t;
    int32_t c = count[0];
    tokens[c] = t;
    count[0] = c + 1;
  }
  __syncthreads();
  const int32_t t = s_tok;
  for (uint32_t i = threadIdx.x; i < dim; i += 1024) x[i] = E[(size_t)t * dim + i];
  __syncthreads();
  if (threadIdx.x == 0) pos[0] = pos[0] + 1;
}

// Set a device int (graph-capturable replacement for a tiny H2D copy).
extern "C" __global__ void smith_set_i32(int32_t* __restrict__ p, int32_t v) {
  if (threadIdx.x == 0 && blockIdx.x == 0) p[0] = v;
}

// ---------------------------------------------------------------------------
// Seeded N(mean, std) f32 (SplitMix64 -> (0,1] -> Box-Muller in f64, pairs in
// the order of src/tensor.js:129-145): element i of the stream that starts
// at `offset`.  Used to write synthetic GGUF weights on the device.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t splitmix64_at(uint64_t seed, uint64_t i) {
  uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

extern "C" __global__ void smith_randn_f32(float* __restrict__ out, uint64_t n, uint64_t seed, uint64_t offset,
                                           float stdv, float mean) {
  for (uint64_t pi = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; 2 * pi < n;
       pi += (uint64_t)gridDim.x * blockDim.x) {
    uint64_t e = offset + 2 * pi;  // pair index in the stream is e / 2
    double u1 = ((double)(splitmix64_at(seed, e) >> 11) + 1.0) * 0x1.0p-53;
    double u2 = ((double)(splitmix64_at(seed, e + 1) >> 11) + 1.0) * 0x1.0p-53;
    double r = sqrt(-2.0 * log(u1));
    double th = 2.0 * 3.141592653589793 * u2;
    out[2 * pi] = (float)(r * cos(th) * (double)stdv + (double)mean);
    if (2 * pi + 1 < n) out[2 * pi + 1] = (float)(r * sin(th) * (double)stdv + (double)mean);
  }
}
