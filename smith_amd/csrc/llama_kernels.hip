// llama_kernels.hip -- gfx950 kernels for the GGUF Llama decode/prefill path
// that loadGGUF(...).generate runs around the quantized GEMVs
// (src/gguf_cache.js:109-265).  Built into its own code object
// (smith_llama.hsaco); every kernel is extern "C".
//
// Positions are read from device memory (pos_ptr) so a whole decode step can
// be captured once as a HIP graph and replayed.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "act_frag.h"
#include "splitk.h"
#include "gguf_tiles.h"

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

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
                                            float* __restrict__ out, uint32_t rows, uint32_t dim,
                                            uint8_t* __restrict__ act_out, const float* __restrict__ gamma_out) {
  uint32_t r = blockIdx.x;
  if (r >= rows) return;
  const float* src = E + (size_t)tokens[r] * dim;
  for (uint32_t i = threadIdx.x; i < dim; i += blockDim.x) {
    const float v = src[i];
    out[(size_t)r * dim + i] = v;
    if (act_out) act_emit8(act_out, dim, i, v, gamma_out ? gamma_out[i] : 1.0f);  // rows == 1, dim % 32 == 0
  }
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
// Device-side bound of the positions a launch touches: rows p0 .. p0+S-1
// (p0 = *pos_ptr, read on the device) must lie inside the KV cache
// (p0 + S <= maxSeq) and inside the RoPE tables for whole-row indexing of
// rows W wide (entries pos*(W/2) + i, so (p0 + S) * (W/2) <= rope_len).  The
// reference's whole-row RoPE reads past its table for positions with
// pos*(dim/2) >= maxSeqLen*headDim/2 (rope.metal:29-36 as gguf_cache.js:130
// applies it); here such a launch touches neither the tables nor the caches.
// The condition is the same for every workgroup, so all of them leave before
// their first position-dependent access (no barrier or split counter is left
// half-used).  Workgroup (0,0,0) records (code, p0, S) in err -- host-mapped
// memory the bridge reads at its next synchronisation -- unless an earlier
// failure is already recorded there.
// ---------------------------------------------------------------------------
#define POS_ERR_KV_APPEND 1u
#define POS_ERR_ATTENTION 2u
#define POS_ERR_PREFILL 3u
#define POS_ERR_PART 4u

__device__ __forceinline__ bool pos_in_range(int32_t p0i, uint32_t S, uint32_t maxSeq, uint32_t W, uint32_t rope_len,
                                             uint32_t* __restrict__ err, uint32_t code) {
  const uint64_t end = (uint64_t)(uint32_t)p0i + S;
  if (p0i >= 0 && end <= maxSeq && end * (W / 2) <= rope_len) return true;
  if (err && threadIdx.x == 0 && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0 &&
      __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) == 0u) {
    __hip_atomic_store(err + 1, (uint32_t)p0i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(err + 2, S, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(err, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
  return false;
}

// ---------------------------------------------------------------------------
// One key split of one query row, shared by the attention kernels (256
// threads): keys t0 .. t1-1, 32-row K/V tiles staged in LDS; rows t < p0
// come from the caches, rows t >= p0 (this launch's rows) from qkv row
// t - p0 with RoPE.  Each thread's share of a tile (4 float4 of K and of V)
// is loaded into registers one tile ahead, the first tile before `qfill`
// (which writes the roped query to qr) runs, so those loads overlap.
// Softmax per tile runs across lanes (lane l: row l % 32), P.V as thread
// (e, half) over the rows of one parity.  Returns the running (m, l) and
// this thread's o for element e = tid % 128, row parity tid / 128.
// ---------------------------------------------------------------------------
#define ATT_TILE 32

struct AttShared {
  float qr[128] __attribute__((aligned(16)));
  float Kt[ATT_TILE][129];
  float Vt[ATT_TILE][128] __attribute__((aligned(16)));
  float sc[ATT_TILE];
};

template <bool NEW>
__device__ __forceinline__ void att_load_tile(float4 (&kreg)[4], float4 (&vreg)[4], const float* __restrict__ kb,
                                              const float* __restrict__ vb, const float* __restrict__ newk,
                                              uint32_t ld, uint32_t Wk, uint32_t kvh, uint32_t hd, uint32_t p0,
                                              uint32_t tb, uint32_t t1, const float* __restrict__ cosT,
                                              const float* __restrict__ sinT) {
  const uint32_t tid = threadIdx.x, c4n = hd / 4;
  const uint32_t nt = t1 - tb < ATT_TILE ? t1 - tb : ATT_TILE;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t idx = tid + 256 * i, r = idx / c4n, c4 = idx % c4n;
    const uint32_t t = tb + (r < nt ? r : nt - 1);  // rows past nt: copies of a real row (weight 0)
    float4 kv, vv;
    if (!NEW || t < p0) {
      kv = *(const float4*)(kb + (size_t)t * hd + 4 * c4);
      vv = *(const float4*)(vb + (size_t)t * hd + 4 * c4);
    } else {
      const float* kr = newk + (size_t)(t - p0) * ld;
      const uint32_t e0 = kvh * hd + 4 * c4;
      kv = make_float4(rope_elem(kr, Wk, e0, t, cosT, sinT), rope_elem(kr, Wk, e0 + 1, t, cosT, sinT),
                       rope_elem(kr, Wk, e0 + 2, t, cosT, sinT), rope_elem(kr, Wk, e0 + 3, t, cosT, sinT));
      vv = *(const float4*)(kr + Wk + e0);
    }
    kreg[i] = kv;
    vreg[i] = vv;
  }
}

template <bool NEW, class QF>
__device__ __forceinline__ void att_split(AttShared& sh, const float* __restrict__ kb, const float* __restrict__ vb,
                                          const float* __restrict__ newk, uint32_t ld, uint32_t Wk, uint32_t kvh,
                                          uint32_t hd, uint32_t p0, uint32_t t0, uint32_t t1,
                                          const float* __restrict__ cosT, const float* __restrict__ sinT,
                                          float scale, QF qfill, float& m, float& l, float& o) {
  const uint32_t tid = threadIdx.x;
  const uint32_t c4n = hd / 4;
  float4 kreg[4], vreg[4];
  if (t0 < t1) att_load_tile<NEW>(kreg, vreg, kb, vb, newk, ld, Wk, kvh, hd, p0, t0, t1, cosT, sinT);
  qfill();
  const uint32_t e = tid % 128, part = tid / 128;
  m = -__builtin_inff();
  l = 0.f;
  o = 0.f;
  __syncthreads();  // qr visible
  for (uint32_t tb = t0; tb < t1; tb += ATT_TILE) {
    const uint32_t nt = t1 - tb < ATT_TILE ? t1 - tb : ATT_TILE;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t idx = tid + 256 * i, r = idx / c4n, c4 = idx % c4n;
      if (r < ATT_TILE) {
        sh.Kt[r][4 * c4] = kreg[i].x;
        sh.Kt[r][4 * c4 + 1] = kreg[i].y;
        sh.Kt[r][4 * c4 + 2] = kreg[i].z;
        sh.Kt[r][4 * c4 + 3] = kreg[i].w;
        *(float4*)&sh.Vt[r][4 * c4] = vreg[i];
      }
    }
    __syncthreads();
    if (tb + ATT_TILE < t1)  // next tile in flight during this one
      att_load_tile<NEW>(kreg, vreg, kb, vb, newk, ld, Wk, kvh, hd, p0, tb + ATT_TILE, t1, cosT, sinT);
    {
      const uint32_t r = tid / 8, sub = tid % 8;
      float d = 0.f;
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const uint32_t c = sub + 8 * i;
        if (c < hd) d = __builtin_fmaf(sh.qr[c], sh.Kt[r][c], d);
      }
      d += __shfl_xor(d, 1);
      d += __shfl_xor(d, 2);
      d += __shfl_xor(d, 4);
      if (sub == 0) sh.sc[r] = r < nt ? d * scale : -__builtin_inff();
    }
    __syncthreads();
    const float sl = sh.sc[tid & 31];
    float tm = sl;
#pragma unroll
    for (int k = 16; k >= 1; k >>= 1) {
      const float ov = __shfl_xor(tm, k);
      tm = ov > tm ? ov : tm;
    }
    const float mn = tm > m ? tm : m;
    const float alpha = __expf(m - mn);  // first tile: m = -inf -> 0
    const float pl = __expf(sl - mn);    // rows >= nt: exp(-inf) = 0
    float ps = pl;
#pragma unroll
    for (int k = 16; k >= 1; k >>= 1) ps += __shfl_xor(ps, k);
    float acc = 0.f;
#pragma unroll
    for (int rr = 0; rr < ATT_TILE / 2; rr++) {
      const uint32_t row = 2 * rr + part;
      acc = __builtin_fmaf(__shfl(pl, (int)row), sh.Vt[row][e < hd ? e : 0], acc);
    }
    l = l * alpha + ps;
    o = o * alpha + acc;
    m = mn;
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// KV-cache append for S rows at positions p0 .. p0+S-1 (p0 = *pos_ptr):
// kcache[kv][p] = RoPE(k row) (the reference's whole-row indexing), vcache
// [kv][p] = v row (gguf_cache.js:212-231).  Workgroup s, threads over Wk.
// ---------------------------------------------------------------------------
extern "C" __global__ void smith_kv_append(const float* __restrict__ qkv, uint32_t ld, const int32_t* __restrict__ pos_ptr,
                                           uint32_t Wq, uint32_t nKV, uint32_t hd, const float* __restrict__ cosT,
                                           const float* __restrict__ sinT, float* __restrict__ kcache,
                                           float* __restrict__ vcache, uint32_t maxSeq, uint32_t rope_len,
                                           uint32_t* __restrict__ err) {
  const int32_t p0i = pos_ptr[0];
  // bounded by the q row width as well, so a launch sequence that fails in
  // the attention kernel after this one has not appended anything either
  const uint32_t Wmax = Wq > nKV * hd ? Wq : nKV * hd;
  if (!pos_in_range(p0i, gridDim.x, maxSeq, Wmax, rope_len, err, POS_ERR_KV_APPEND)) return;
  const uint32_t s = blockIdx.x, pos = (uint32_t)p0i + s;
  const uint32_t Wk = nKV * hd;
  const float* krow = qkv + (size_t)s * ld + Wq;
  for (uint32_t i = threadIdx.x; i < Wk; i += blockDim.x) {
    const uint32_t kv = i / hd, e = i % hd;
    const size_t o = ((size_t)kv * maxSeq + pos) * hd + e;
    kcache[o] = rope_elem(krow, Wk, i, pos, cosT, sinT);
    vcache[o] = krow[Wk + i];
  }
}

// ---------------------------------------------------------------------------
// Fused RoPE + KV-cache append + GQA attention, for S query rows at positions
// p0 .. p0+S-1 with p0 = *pos_ptr (gguf_cache.js:128-157 for decode,
// :212-231 for prefill).  qkv rows hold [q | k | v] (ld floats per row).
// q head h uses KV head h / (nH/nKV) (repeatKV, gguf_cache.js:90-105);
// scores (q.k) * 1/sqrt(hd), softmax over positions 0..p0+s, out = P V.
//
// Workgroup (h, s, z): query row s, head h, split z of the NSPLIT splits of
// its T = p0+s+1 key rows.  Keys/values of positions < p0 come from the
// cache; those of p0..p0+s are formed here from the raw k (roped) and v of
// this launch's qkv rows, so no workgroup depends on another's writes.  The
// (h % rep == 0, z == 0) workgroup of row s writes row s's roped key and its
// value into the cache.  Each split stages 32-row K and V tiles in LDS with
// 128-bit loads and keeps an online softmax (running max m, sum l, output
// o); partials go to a workspace and the last split to finish (per (h, s),
// agent-scope atomics) combines them: out = sum_z e^(m_z-M) o_z /
// sum_z e^(m_z-M) l_z.  hd <= 128, 256 threads.
// ---------------------------------------------------------------------------
#define ATT_SPLIT 8

template <bool APPENDED>
__device__ __forceinline__ void attention_body(
    const float* __restrict__ qkv, uint32_t ld, const int32_t* __restrict__ pos_ptr, uint32_t S, uint32_t nH,
    uint32_t nKV, uint32_t hd, const float* __restrict__ cosT, const float* __restrict__ sinT,
    float* __restrict__ kcache, float* __restrict__ vcache, uint32_t maxSeq, float* __restrict__ out,
    float* __restrict__ ws, uint32_t* __restrict__ counters, uint8_t* __restrict__ act_out, uint32_t rope_len,
    uint32_t* __restrict__ err) {
  __shared__ AttShared sh;
  __shared__ float ored[2][128];
  __shared__ int s_last;
  const uint32_t h = blockIdx.x, s = blockIdx.y, z = blockIdx.z;
  const uint32_t tid = threadIdx.x;
  const int32_t p0i = pos_ptr[0];
  if (!pos_in_range(p0i, S, maxSeq, nH * hd, rope_len, err, POS_ERR_ATTENTION)) return;
  const uint32_t p0 = (uint32_t)p0i;
  const uint32_t pos = p0 + s;
  const uint32_t T = pos + 1;
  const uint32_t rep = nH / nKV, kvh = h / rep;
  const uint32_t Wq = nH * hd, Wk = nKV * hd;
  const float scale = 1.0f / __builtin_sqrtf((float)hd);
  const float* qrow = qkv + (size_t)s * ld;
  // this split's key rows
  const uint32_t per = (T + ATT_SPLIT - 1) / ATT_SPLIT;
  const uint32_t t0 = z * per, t1 = t0 + per < T ? t0 + per : T;
  const uint32_t e = tid % 128, part = tid / 128;  // output element, row half
  float m, l, o;
  // APPENDED: smith_kv_append already put this launch's rows in the caches
  att_split<!APPENDED>(sh, kcache + (size_t)kvh * maxSeq * hd, vcache + (size_t)kvh * maxSeq * hd, qkv + Wq, ld, Wk, kvh, hd,
            APPENDED ? p0 + S : p0, t0, t1, cosT, sinT, scale,
            [&]() {
              for (uint32_t e2 = tid; e2 < hd; e2 += 256) sh.qr[e2] = rope_elem(qrow, Wq, h * hd + e2, pos, cosT, sinT);
              if (!APPENDED && h % rep == 0 && z == 0) {
                const float* krow = qkv + (size_t)s * ld + Wq;
                for (uint32_t e2 = tid; e2 < hd; e2 += 256) {
                  size_t oo = ((size_t)kvh * maxSeq + pos) * hd + e2;
                  kcache[oo] = rope_elem(krow, Wk, kvh * hd + e2, pos, cosT, sinT);
                  vcache[oo] = krow[Wk + kvh * hd + e2];
                }
              }
            },
            m, l, o);
  // combine the two row halves of this split
  if (e < hd) ored[part][e] = o;
  __syncthreads();
  const size_t slot = ((size_t)s * nH + h) * ATT_SPLIT + z;
  float* wsp = ws + slot * 130;
  if (tid < hd) {
    float v = ored[0][tid] + ored[1][tid];
    __hip_atomic_exchange((uint32_t*)wsp + 2 + tid, __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (tid == 0) {
    __hip_atomic_exchange((uint32_t*)wsp, __float_as_uint(m), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_exchange((uint32_t*)wsp + 1, __float_as_uint(l), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  uint32_t* cnt = counters + (size_t)s * nH + h;
  if (tid == 0) {
    uint32_t prev = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == ATT_SPLIT - 1;
  }
  __syncthreads();
  if (!s_last) return;
  const float* base = ws + ((size_t)s * nH + h) * ATT_SPLIT * 130;
  auto ld32 = [&](const float* p) {
    return __uint_as_float(__hip_atomic_fetch_add((uint32_t*)p, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  };
  __shared__ float mz_s[ATT_SPLIT], wz_s[ATT_SPLIT];
  if (tid < ATT_SPLIT) {
    mz_s[tid] = ld32(base + tid * 130);
    wz_s[tid] = ld32(base + tid * 130 + 1);
  }
  __syncthreads();
  float M = -__builtin_inff();
#pragma unroll
  for (int zz = 0; zz < ATT_SPLIT; zz++) M = mz_s[zz] > M ? mz_s[zz] : M;
  float L = 0.f, wz[ATT_SPLIT];
#pragma unroll
  for (int zz = 0; zz < ATT_SPLIT; zz++) {
    wz[zz] = mz_s[zz] == -__builtin_inff() ? 0.f : __expf(mz_s[zz] - M);
    L = __builtin_fmaf(wz[zz], wz_s[zz], L);
  }
  if (tid < hd) {
    float ov[ATT_SPLIT];
#pragma unroll
    for (int zz = 0; zz < ATT_SPLIT; zz++) ov[zz] = ld32(base + zz * 130 + 2 + tid);
    float v = 0.f;
#pragma unroll
    for (int zz = 0; zz < ATT_SPLIT; zz++) v = __builtin_fmaf(wz[zz], ov[zz], v);
    const float y = v / L;
    out[(size_t)s * Wq + h * hd + tid] = y;
    if (act_out) act_emit8(act_out, Wq, h * hd + tid, y, 1.0f);  // S == 1, hd % 8 == 0
  }
  if (tid == 0) __hip_atomic_exchange(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

#define ATT_ARGS                                                                                              \
  const float *__restrict__ qkv, uint32_t ld, const int32_t *__restrict__ pos_ptr, uint32_t S, uint32_t nH,    \
      uint32_t nKV, uint32_t hd, const float *__restrict__ cosT, const float *__restrict__ sinT,               \
      float *__restrict__ kcache, float *__restrict__ vcache, uint32_t maxSeq, float *__restrict__ out,        \
      float *__restrict__ ws, uint32_t *__restrict__ counters, uint8_t *__restrict__ act_out, uint32_t rope_len, \
      uint32_t *__restrict__ err
// rows' keys formed here from qkv (and appended to the caches)
extern "C" __global__ __launch_bounds__(256) void smith_attention(ATT_ARGS) {
  attention_body<false>(qkv, ld, pos_ptr, S, nH, nKV, hd, cosT, sinT, kcache, vcache, maxSeq, out, ws, counters,
                        act_out, rope_len, err);
}
// every key already in the caches (smith_kv_append ran first)
extern "C" __global__ __launch_bounds__(256) void smith_attention_cached(ATT_ARGS) {
  attention_body<true>(qkv, ld, pos_ptr, S, nH, nKV, hd, cosT, sinT, kcache, vcache, maxSeq, out, ws, counters,
                       act_out, rope_len, err);
}

// ---------------------------------------------------------------------------
// Prefill attention on the f32 matrix cores (flash-attention form of
// flash_attention.js:34-70 / flash_attention.metal, which gguf_cache.js:213
// runs on the prefill rows): S query rows at positions p0 .. p0+S-1, every
// key row 0 .. p0+s already in the caches (smith_kv_append ran first).
// Workgroup (h, qb): head h, query rows 16*qb .. +15 (roped, in LDS).  K and
// V tiles of 64 keys are staged in LDS; wave w takes keys 16w .. 16w+15 of
// every tile, so the four waves split the key range and each keeps its own
// online softmax (running max m, sum l, O) for the 16 rows: S = Q K^T with
// v_mfma_f32_16x16x4_f32 (f32 operands, exact products, f32 sums -- the
// reference's arithmetic type), scale, causal mask, P through LDS into the
// A-operand layout, O += P V on the same MFMA.  At the end the four
// partials are combined in LDS: out = sum_w e^(m_w - M) O_w / sum_w e^(m_w - M) l_w.
// hd % 16 == 0, hd <= 128.
// MFMA 16x16x4 f32 layout: lane (c = lane % 16, j = lane / 16) supplies
// A[row c][k j] and B[k j][col c] and holds D rows 4j .. 4j+3 of column c.
// ---------------------------------------------------------------------------
typedef float f32x4_t __attribute__((ext_vector_type(4)));
#define FA_BQ 16
#define FA_BK 64
#define FA_QS 132  // Q / K row stride (floats): A/B reads of 16 rows x 4 k hit 64 banks
#define FA_VS 144  // V row stride: B reads of 4 keys x 16 columns hit 64 banks
#define FA_PS 20   // P row stride: A reads of 16 rows x 4 keys hit 64 banks

template <int NT>  // head_dim / 16
__device__ __forceinline__ void attention_prefill_body(
    const float* __restrict__ qkv, uint32_t ld, const int32_t* __restrict__ pos_ptr, uint32_t S, uint32_t nH,
    uint32_t nKV, const float* __restrict__ cosT, const float* __restrict__ sinT, const float* __restrict__ kcache,
    const float* __restrict__ vcache, uint32_t maxSeq, float* __restrict__ out, uint32_t rope_len,
    uint32_t* __restrict__ err, _Float16* __restrict__ a16) {
  constexpr uint32_t hd = 16 * NT;
  __shared__ __attribute__((aligned(16))) float Qs[FA_BQ * FA_QS];
  __shared__ __attribute__((aligned(16))) float KV[FA_BK * FA_QS + FA_BK * FA_VS];  // then the waves' O
  __shared__ float Ps[4][16 * FA_PS];
  __shared__ float MLs[4][2][16];
  float* Ks = KV;
  float* Vs = KV + FA_BK * FA_QS;
  const uint32_t h = blockIdx.x, s0 = blockIdx.y * FA_BQ;
  const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const uint32_t c = lane & 15, j = lane >> 4;
  const int32_t p0i = pos_ptr[0];
  if (!pos_in_range(p0i, S, maxSeq, nH * hd, rope_len, err, POS_ERR_PREFILL)) return;
  const uint32_t p0 = (uint32_t)p0i;
  const uint32_t rep = nH / nKV, kvh = h / rep;
  const uint32_t Wq = nH * hd;
  const float scale = 1.0f / __builtin_sqrtf((float)hd);
  const uint32_t nrow = S - s0 < FA_BQ ? S - s0 : FA_BQ;
  const uint32_t Tend = p0 + s0 + nrow;  // keys of the block: 0 .. Tend-1
  const float* kb = kcache + (size_t)kvh * maxSeq * hd;
  const float* vb = vcache + (size_t)kvh * maxSeq * hd;
  constexpr uint32_t c4n = hd / 4;
  constexpr uint32_t TPT = (FA_BK * c4n + 255) / 256;  // float4s of a K (and V) tile per thread
  // K / V tiles staged through registers: tile t+1's loads are in flight
  // while tile t is multiplied (and tile 0's while the queries are roped)
  float4 kr[TPT], vr[TPT];
  auto load_tile = [&](uint32_t t0) {
#pragma unroll
    for (uint32_t q = 0; q < TPT; q++) {
      const uint32_t i = tid + 256 * q, r = i / c4n, c4 = i % c4n, t = t0 + r;
      kr[q] = vr[q] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (i < FA_BK * c4n && t < Tend) {
        kr[q] = *(const float4*)(kb + (size_t)t * hd + 4 * c4);
        vr[q] = *(const float4*)(vb + (size_t)t * hd + 4 * c4);
      }
    }
  };
  load_tile(0);
  // 1. roped queries (whole-row RoPE of the q part of each qkv row); rows past S zero
  for (uint32_t i = tid; i < FA_BQ * hd; i += 256) {
    const uint32_t r = i / hd, e = i % hd;
    float v = 0.f;
    if (r < nrow) v = rope_elem(qkv + (size_t)(s0 + r) * ld, Wq, h * hd + e, p0 + s0 + r, cosT, sinT);
    Qs[r * FA_QS + e] = v;
  }
  f32x4_t o[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) o[t] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
  float m[4], l[4];
#pragma unroll
  for (int r = 0; r < 4; r++) {
    m[r] = -__builtin_inff();
    l[r] = 0.f;
  }
  float* P = Ps[w];
  for (uint32_t t0 = 0; t0 < Tend; t0 += FA_BK) {
    __syncthreads();  // previous tile's K/V reads done (and, first time, Qs written)
    // 2. K and V tile from the registers (rows past Tend zero: their P is 0
    //    and V must be finite), then the next tile's loads
#pragma unroll
    for (uint32_t q = 0; q < TPT; q++) {
      const uint32_t i = tid + 256 * q, r = i / c4n, c4 = i % c4n;
      if (i < FA_BK * c4n) {
        *(float4*)&Ks[r * FA_QS + 4 * c4] = kr[q];
        *(float4*)&Vs[r * FA_VS + 4 * c4] = vr[q];
      }
    }
    if (t0 + FA_BK < Tend) load_tile(t0 + FA_BK);
    __syncthreads();
    const uint32_t k0 = t0 + 16 * w;  // this wave's 16 keys
    if (k0 >= Tend) continue;         // after every row of the block
    // 3. scores of the 16 rows against the wave's 16 keys (two independent
    //    accumulator chains over alternate k steps, summed at the end)
    f32x4_t sc = (f32x4_t){0.f, 0.f, 0.f, 0.f}, sc2 = sc;
#pragma unroll 8
    for (uint32_t kk = 0; kk < hd; kk += 8) {
      sc = __builtin_amdgcn_mfma_f32_16x16x4f32(Qs[c * FA_QS + kk + j], Ks[(16 * w + c) * FA_QS + kk + j], sc, 0, 0,
                                                0);
      sc2 = __builtin_amdgcn_mfma_f32_16x16x4f32(Qs[c * FA_QS + kk + 4 + j], Ks[(16 * w + c) * FA_QS + kk + 4 + j],
                                                 sc2, 0, 0, 0);
    }
    sc += sc2;
    // 4. online softmax per row (row 4j + r: the 16 lanes of group j)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const uint32_t pos = p0 + s0 + 4 * j + r;
      const float sv = k0 + c <= pos ? sc[r] * scale : -__builtin_inff();
      const float v = max16_lanes(sv);
      const float mn = v > m[r] ? v : m[r];  // -inf while every key so far is masked for this row
      const float alpha = m[r] == -__builtin_inff() ? 0.f : __expf(m[r] - mn);
      const float pv = sv == -__builtin_inff() ? 0.f : __expf(sv - mn);
      const float rs = sum16_lanes(pv);
      l[r] = __builtin_fmaf(l[r], alpha, rs);
      m[r] = mn;
#pragma unroll
      for (int t = 0; t < NT; t++) o[t][r] *= alpha;
      P[(4 * j + r) * FA_PS + c] = pv;
    }
    // 5. P (16 rows x 16 keys) read back as the A operand of P V
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
#pragma unroll
    for (uint32_t kk = 0; kk < 16; kk += 4) {
      const float a = P[c * FA_PS + kk + j];
#pragma unroll
      for (int t = 0; t < NT; t++)
        o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, Vs[(16 * w + kk + j) * FA_VS + 16 * t + c], o[t], 0, 0, 0);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");  // P reads done before the next tile's P writes
    __builtin_amdgcn_wave_barrier();
  }
  // 6. combine the waves' partials: out = sum_w e^(m_w - M) O_w / sum_w e^(m_w - M) l_w
  __syncthreads();  // every wave is done with the K/V tile: KV holds the O partials now
  float* Os = KV;
  if (c == 0)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      MLs[w][0][4 * j + r] = m[r];
      MLs[w][1][4 * j + r] = l[r];
    }
#pragma unroll
  for (int r = 0; r < 4; r++)
#pragma unroll
    for (int t = 0; t < NT; t++) Os[(w * 16 + 4 * j + r) * hd + 16 * t + c] = o[t][r];
  __syncthreads();
  for (uint32_t i = tid; i < nrow * hd; i += 256) {
    const uint32_t r = i / hd, e = i % hd;
    float M = MLs[0][0][r];
#pragma unroll
    for (int ww = 1; ww < 4; ww++) M = MLs[ww][0][r] > M ? MLs[ww][0][r] : M;  // finite: key 0 is in wave 0
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int ww = 0; ww < 4; ww++) {
      const float mw = MLs[ww][0][r];
      const float f = mw == -__builtin_inff() ? 0.f : __expf(mw - M);
      den = __builtin_fmaf(f, MLs[ww][1][r], den);
      num = __builtin_fmaf(f, Os[(ww * 16 + r) * hd + e], num);
    }
    out[(size_t)(s0 + r) * Wq + h * hd + e] = num / den;
  }
  if (!a16) return;
  // the rows also as the output projection's f16 GEMM operand: each
  // 8-element chunk in the slot order {0,4,1,5,2,6,3,7} (the order of
  // smith_gemm_prep_a_perm), the same values as above
  for (uint32_t ci = tid; ci < nrow * (hd / 8); ci += 256) {
    const uint32_t r = ci / (hd / 8), e0 = 8 * (ci % (hd / 8));
    float M = MLs[0][0][r];
#pragma unroll
    for (int ww = 1; ww < 4; ww++) M = MLs[ww][0][r] > M ? MLs[ww][0][r] : M;
    float f[4], den = 0.f;
#pragma unroll
    for (int ww = 0; ww < 4; ww++) {
      const float mw = MLs[ww][0][r];
      f[ww] = mw == -__builtin_inff() ? 0.f : __expf(mw - M);
      den = __builtin_fmaf(f[ww], MLs[ww][1][r], den);
    }
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
      float num = 0.f;
#pragma unroll
      for (int ww = 0; ww < 4; ww++) num = __builtin_fmaf(f[ww], Os[(ww * 16 + r) * hd + e0 + e], num);
      v[e] = num / den;
    }
    uint32_t w4[4];
#pragma unroll
    for (int q = 0; q < 4; q++)
      w4[q] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[q]) |
              ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[q + 4]) << 16);
    *(uint4*)(a16 + (size_t)(s0 + r) * Wq + h * hd + e0) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
  }
}

#define DEF_ATT_PREFILL(NT)                                                                                      \
  extern "C" __global__ __launch_bounds__(256) void smith_attention_prefill_hd##NT(                              \
      const float* __restrict__ qkv, uint32_t ld, const int32_t* __restrict__ pos_ptr, uint32_t S, uint32_t nH,   \
      uint32_t nKV, const float* __restrict__ cosT, const float* __restrict__ sinT,                              \
      const float* __restrict__ kcache, const float* __restrict__ vcache, uint32_t maxSeq, float* __restrict__ out, \
      uint32_t rope_len, uint32_t* __restrict__ err, _Float16* __restrict__ a16) {                                \
    attention_prefill_body<NT>(qkv, ld, pos_ptr, S, nH, nKV, cosT, sinT, kcache, vcache, maxSeq, out, rope_len, err, \
                               a16);                                                                             \
  }
// named by head_dim / 16
DEF_ATT_PREFILL(1)
DEF_ATT_PREFILL(2)
DEF_ATT_PREFILL(3)
DEF_ATT_PREFILL(4)
DEF_ATT_PREFILL(5)
DEF_ATT_PREFILL(6)
DEF_ATT_PREFILL(7)
DEF_ATT_PREFILL(8)

// ---------------------------------------------------------------------------
// Single-row decode attention writing per-split partials for the output
// projection to combine (smith_agemv_att_*), so no workgroup of this kernel
// waits for another.  Row position p0 = *pos_ptr, T = p0 + 1 keys in 32-row
// tiles; split count nsplit = min(ATTP_MAXSPLIT, tiles) decided on the device
// (one captured grid serves every position; workgroups past nsplit leave at
// once); split z takes tiles z, z + ATTP_MAXSPLIT, ...  Workgroup (b, z):
// query head h of KV head b % nKV (the rep query heads of a KV head get
// workgroup ids congruent mod nKV, i.e. the same XCD when nKV is a multiple
// of 8, so they share its L2), key split z.
//
// Everything that does not depend on the position is issued at once: the
// split's first K/V tile from the caches (rows 32z .. 32z+31), the q row and
// this KV head's new k / v (with their whole-row RoPE partners), the position
// and the rope row -- cos / sin of the current position for the q and k row
// widths, tagged with that position, written by the previous greedy step
// (smith_argmax_embed) -- so one memory round trip feeds the split.  A rope
// row of another position (or none) falls back to the table.  Cache rows
// past p0 are zeroed in LDS (their weight is 0; the cache may hold anything
// there) and row p0 is this token's roped k and v.  Math as smith_attention
// (1/sqrt(hd) scores, online softmax over the tile); the partial (m, l, o[hd])
// of (h, z) goes to parts[(h*ATTP_MAXSPLIT + z)*ATTP_STRIDE ..] with plain
// stores.  The (h % rep == 0, z == 0) workgroup appends the row's key/value.
// ---------------------------------------------------------------------------
#define ATTP_ROWS 32
#define ATTP_MAXSPLIT 8
#define ATTP_STRIDE 132  // floats per partial: m, l, 2 pad, o[128] (16-byte aligned)
#define ROPE_ROW_HDR 4   // rope row: int32 position tag, 3 pad, then cos_q, sin_q, cos_k, sin_k

struct AttPShared {
  float qr[128] __attribute__((aligned(16)));
  float Kt[ATTP_ROWS][132] __attribute__((aligned(16)));  // 16-byte rows: 4-float reads
  float Vt[ATTP_ROWS][132] __attribute__((aligned(16)));  // padded: rows 2rr, 2rr+1 of a column in other banks
  float sc[ATTP_ROWS] __attribute__((aligned(16)));
};


extern "C" __global__ __launch_bounds__(256) void smith_attention_part(
    const float* __restrict__ qkv, const int32_t* __restrict__ pos_ptr, uint32_t nH, uint32_t nKV, uint32_t hd,
    const float* __restrict__ cosT, const float* __restrict__ sinT, const float* __restrict__ rrow,
    float* __restrict__ kcache, float* __restrict__ vcache, uint32_t maxSeq, float* __restrict__ parts,
    uint32_t rope_len, uint32_t* __restrict__ err) {
  __shared__ AttPShared sh;
  const uint32_t rep = nH / nKV;
  const uint32_t kvh = blockIdx.x % nKV, h = kvh * rep + blockIdx.x / nKV, z = blockIdx.y;
  const uint32_t tid = threadIdx.x, c4n = hd / 4;
  const uint32_t Wq = nH * hd, Wk = nKV * hd, hq = Wq / 2, hk = Wk / 2;
  const float scale = 1.0f / __builtin_sqrtf((float)hd);
  const float* krow = qkv + Wq;
  const float* kb = kcache + (size_t)kvh * maxSeq * hd;
  const float* vb = vcache + (size_t)kvh * maxSeq * hd;

  // 1. loads that need no position
  const int32_t p0i = pos_ptr[0];
  const int32_t tag = rrow ? *(const int32_t*)rrow : -1;
  float4 kreg[4], vreg[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t idx = tid + 256 * i, r = idx / c4n, c4 = idx % c4n;
    uint32_t t = ATTP_ROWS * z + (r < ATTP_ROWS ? r : ATTP_ROWS - 1);
    t = t < maxSeq ? t : maxSeq - 1;
    kreg[i] = *(const float4*)(kb + (size_t)t * hd + 4 * c4);
    vreg[i] = *(const float4*)(vb + (size_t)t * hd + 4 * c4);
  }
  const uint32_t e = tid < hd ? tid : 0;
  const uint32_t iq = h * hd + e, pq = iq < hq ? iq : iq - hq;
  const uint32_t ik = kvh * hd + e, pk = ik < hk ? ik : ik - hk;
  const float q0 = qkv[pq], q1 = qkv[pq + hq];
  const float k0 = krow[pk], k1 = krow[pk + hk];
  const float vnew = krow[Wk + ik];
  float cq = 0.f, sq = 0.f, ck = 0.f, sk = 0.f;
  if (rrow) {
    cq = rrow[ROPE_ROW_HDR + pq];
    sq = rrow[ROPE_ROW_HDR + hq + pq];
    ck = rrow[ROPE_ROW_HDR + Wq + pk];
    sk = rrow[ROPE_ROW_HDR + Wq + hk + pk];
  }

  // 2. the position: split count, RoPE of q and of the new k (rope_elem's
  //    whole-row pairing), the cache append
  if (!pos_in_range(p0i, 1, maxSeq, Wq, rope_len, err, POS_ERR_PART)) return;
  const uint32_t p0 = (uint32_t)p0i, T = p0 + 1;
  const uint32_t ntile = (T + ATTP_ROWS - 1) / ATTP_ROWS;
  const uint32_t nsplit = ntile < ATTP_MAXSPLIT ? ntile : ATTP_MAXSPLIT;
  if (z >= nsplit) return;
  if (tag != p0i) {
    cq = cosT[(size_t)p0 * hq + pq];
    sq = sinT[(size_t)p0 * hq + pq];
    ck = cosT[(size_t)p0 * hk + pk];
    sk = sinT[(size_t)p0 * hk + pk];
  }
  // this token's roped key element tid and value element tid stay in
  // registers: their threads write them into tile row p0 themselves
  const float kr = ik < hk ? k0 * ck - k1 * sk : k0 * sk + k1 * ck;
  if (tid < hd) {
    sh.qr[tid] = iq < hq ? q0 * cq - q1 * sq : q0 * sq + q1 * cq;
    if (h % rep == 0 && z == 0) {
      const size_t oo = ((size_t)kvh * maxSeq + p0) * hd + tid;
      kcache[oo] = kr;
      vcache[oo] = vnew;
    }
  }

  // 3. the split's tiles.  P.V lanes: column ee, rows of parity `part`;
  //    the two parities of a column sit in adjacent lanes
  const uint32_t ee = tid >> 1, part = tid & 1;
  float m = -__builtin_inff(), l = 0.f, o = 0.f;
  for (uint32_t tau = z; tau < ntile; tau += ATTP_MAXSPLIT) {
    const uint32_t tb = ATTP_ROWS * tau;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t idx = tid + 256 * i, r = idx / c4n, c4 = idx % c4n;
      if (r < ATTP_ROWS) {
        const uint32_t t = tb + r;
        float4 kv = kreg[i], vv = vreg[i];
        if (t > p0) kv = vv = make_float4(0.f, 0.f, 0.f, 0.f);
        if (t != p0) {  // row p0: written below by the threads holding its elements
          *(float4*)&sh.Kt[r][4 * c4] = kv;
          *(float4*)&sh.Vt[r][4 * c4] = vv;
        }
      }
    }
    if (tid < hd && p0 >= tb && p0 < tb + ATTP_ROWS) {
      sh.Kt[p0 - tb][tid] = kr;
      sh.Vt[p0 - tb][tid] = vnew;
    }
    __syncthreads();  // the tile (and, first time, qr) visible
    if (tau + ATTP_MAXSPLIT < ntile) {  // the split's next tile in flight during this one
      const uint32_t tn = tb + ATTP_ROWS * ATTP_MAXSPLIT;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t idx = tid + 256 * i, r = idx / c4n, c4 = idx % c4n;
        uint32_t t = tn + (r < ATTP_ROWS ? r : ATTP_ROWS - 1);
        t = t < maxSeq ? t : maxSeq - 1;
        kreg[i] = *(const float4*)(kb + (size_t)t * hd + 4 * c4);
        vreg[i] = *(const float4*)(vb + (size_t)t * hd + 4 * c4);
      }
    }
    {
      // score of row r: lanes (r, sub) take elements 16 sub .. 16 sub + 15
      // (four 16-byte reads of q and of the key row, all issued together)
      const uint32_t r = tid / 8, sub = tid % 8, c0 = 16 * sub;
      // (one wave per SIMD here, so instruction latency is exposed: four
      // independent chains of four FMAs instead of one of sixteen)
      float d = 0.f;
      if (c0 < hd) {
        float4 qv[4], kv[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          qv[i] = *(const float4*)&sh.qr[c0 + 4 * i];
          kv[i] = *(const float4*)&sh.Kt[r][c0 + 4 * i];
        }
        float di[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          di[i] = 0.f;
          if (c0 + 4 * i < hd) {  // hd % 4 == 0
            di[i] = qv[i].x * kv[i].x;
            di[i] = __builtin_fmaf(qv[i].y, kv[i].y, di[i]);
            di[i] = __builtin_fmaf(qv[i].z, kv[i].z, di[i]);
            di[i] = __builtin_fmaf(qv[i].w, kv[i].w, di[i]);
          }
        }
        d = (di[0] + di[1]) + (di[2] + di[3]);
      }
      d = sum8_lanes(d);
      if (sub == 0) sh.sc[r] = tb + r <= p0 ? d * scale : -__builtin_inff();
    }
    __syncthreads();
    // every thread reads the 32 scores (broadcast reads) and forms the
    // tile's max, weights and weight sum itself
    float sv[ATTP_ROWS];
#pragma unroll
    for (int i = 0; i < ATTP_ROWS / 4; i++) {
      const float4 v4 = *(const float4*)&sh.sc[4 * i];
      sv[4 * i] = v4.x;
      sv[4 * i + 1] = v4.y;
      sv[4 * i + 2] = v4.z;
      sv[4 * i + 3] = v4.w;
    }
    const uint32_t ec = ee < hd ? ee : 0;
    float vv[ATTP_ROWS / 2];
#pragma unroll
    for (int rr = 0; rr < ATTP_ROWS / 2; rr++) vv[rr] = sh.Vt[2 * rr + part][ec];
    // the tile's max as a tree (exact in any order)
    float mx[ATTP_ROWS / 2];
#pragma unroll
    for (int i = 0; i < ATTP_ROWS / 2; i++) mx[i] = sv[2 * i + 1] > sv[2 * i] ? sv[2 * i + 1] : sv[2 * i];
#pragma unroll
    for (int i = 0; i < 8; i++) mx[i] = mx[i + 8] > mx[i] ? mx[i + 8] : mx[i];
#pragma unroll
    for (int i = 0; i < 4; i++) mx[i] = mx[i + 4] > mx[i] ? mx[i + 4] : mx[i];
#pragma unroll
    for (int i = 0; i < 2; i++) mx[i] = mx[i + 2] > mx[i] ? mx[i + 2] : mx[i];
    const float tm = mx[1] > mx[0] ? mx[1] : mx[0];
    const float mn = tm > m ? tm : m;
    const float alpha = __expf(m - mn);  // first tile: m = -inf -> 0
    // weights of this lane's parity only; the other parity's sum comes from
    // lane ^ 1.  Two interleaved accumulation chains each.
    // (the parity select on the bits: as `part ? a : b` the compiler turned
    // it into a dynamically indexed read of the score array, in scratch)
    const uint32_t pm = 0u - part;
    float pe[ATTP_ROWS / 2];
#pragma unroll
    for (int rr = 0; rr < ATTP_ROWS / 2; rr++) {
      const uint32_t bits = (__float_as_uint(sv[2 * rr]) & ~pm) | (__float_as_uint(sv[2 * rr + 1]) & pm);
      pe[rr] = __expf(__uint_as_float(bits) - mn);  // masked rows: 0
    }
    float psa = 0.f, psb = 0.f, acca = 0.f, accb = 0.f;
#pragma unroll
    for (int rr = 0; rr < ATTP_ROWS / 2; rr += 2) {
      psa += pe[rr];
      psb += pe[rr + 1];
      acca = __builtin_fmaf(pe[rr], vv[rr], acca);
      accb = __builtin_fmaf(pe[rr + 1], vv[rr + 1], accb);
    }
    const float ps_own = psa + psb, acc = acca + accb;
    const float ps_other = dpp_f32<0xB1>(ps_own);  // every lane active: no DPP under a branch
    const float ps = part ? ps_other + ps_own : ps_own + ps_other;  // even + odd rows
    l = l * alpha + ps;
    o = o * alpha + acc;
    m = mn;
    if (tau + ATTP_MAXSPLIT < ntile) __syncthreads();  // every lane done with the tile before the next
  }
  // the even-row sum plus the odd-row sum of column ee (lane ^ 1)
  const float o_odd = dpp_f32<0xB1>(o);
  float* pp = parts + ((size_t)h * ATTP_MAXSPLIT + z) * ATTP_STRIDE;
  if (part == 0 && ee < hd) pp[4 + ee] = o + o_odd;
  if (tid == 0) {
    pp[0] = m;
    pp[1] = l;
  }
}

// ---------------------------------------------------------------------------
// LM head on the GGUF output.weight as the reference loads it: the flat data
// is read as lmHead[dim][vocab] (gguf_loader.js:240-259 never transposes a
// path that does not end in ".weight"), so for Q4_0 the 32-weight blocks run
// along the VOCAB axis: block (k, vb) at (k*(N/32) + vb)*18 covers
// lmHead[k][32vb .. 32vb+31] = d*(nib - 8), element e in nibble e (byte
// e/2, low nibble first).  smith_repack_lmhead_q4_0 regroups the blocks by
// row octets: record (o = k/8, vb) holds the nibbles of rows 8o .. 8o+7 as
// 128 bytes [quarter q = 0..3][row r = 0..7][the 4 nibble bytes 4q .. 4q+3 of
// block (8o+r, vb)] in a nibble plane, and the 8 scales as 16 bytes in a
// scale plane, both in (o, vb) order.  Lane (vb, q) then reads its 8 outputs'
// nibbles of 8 rows as two 16-byte loads and their scales as one, and a wave
// (16 blocks x 4 quarters) reads 2 KB of contiguous nibbles per row octet.
// K % 8 == 0.
// ---------------------------------------------------------------------------
extern "C" __global__ void smith_repack_lmhead_q4_0(const uint8_t* __restrict__ src, uint8_t* __restrict__ nib,
                                                    uint16_t* __restrict__ dsc, uint32_t K, uint32_t NB) {
  size_t total = (size_t)K * NB;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
    const uint32_t k = (uint32_t)(idx / NB), vb = (uint32_t)(idx % NB);
    const uint16_t* b = (const uint16_t*)(src + idx * 18);
    const size_t rec = (size_t)(k / 8) * NB + vb;
    const uint32_t r = k % 8;
    dsc[rec * 8 + r] = b[0];
#pragma unroll
    for (int q = 0; q < 4; q++)
      *(uint32_t*)(nib + rec * 128 + q * 32 + r * 4) = (uint32_t)b[1 + 2 * q] | ((uint32_t)b[2 + 2 * q] << 16);
  }
}

// Greedy step after the logits (generate.js:70-76 argmax, gguf_cache.js:
// 335-341 append): the token goes to tokens[count], count and the position
// advance, x = E[token] (and its act for the next step's first GEMV), and the
// rope row of the next position is written (cos / sin of the q and k row
// widths, tagged with that position) when the table holds it.
struct GreedyTail {
  const float* E;  // null: no greedy step
  float* x;
  int32_t* tokens;
  int32_t* count;
  int32_t* pos;
  uint8_t* act_out;
  const float* gamma_out;
  const float* cosT;
  const float* sinT;
  float* rrow;
  uint64_t* amx;  // [0] best key, [1] low word: tiles finished (zero between calls)
  uint32_t rope_len, wq, wk, dim;
};

// Order-preserving key of (logit, index) for an unsigned max: larger logits
// win, and among equal logits the smaller index (the reference keeps the
// first maximum).  NaNs never win (key 0); -0 counts as +0.  A NaN at index 0
// gets the largest key: the reference's scan compares against logits[0]
// first and then never moves.  Key 0 and the all-ones key both decode to 0.
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t n) {
  if (v != v) return n == 0 ? ~0ull : 0ull;
  uint32_t u = __float_as_uint(v == 0.f ? 0.f : v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)u << 32) | (uint32_t)(0xFFFFFFFFu - n);
}

__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t wave_max64(uint64_t k) { return max64_lanes(k); }

// The rope row of position np (tag np), written when the tables hold it;
// threads tid, tid + nt, ... of the caller.
__device__ __forceinline__ void rope_row_write(float* __restrict__ rrow, const float* __restrict__ cosT,
                                               const float* __restrict__ sinT, uint32_t rope_len, uint32_t wq,
                                               uint32_t wk, uint32_t np, uint32_t tid, uint32_t nt) {
  const uint32_t hq = wq / 2, hk = wk / 2;
  if (!rrow || (size_t)(np + 1) * hq > rope_len || (size_t)(np + 1) * hk > rope_len) return;
  for (uint32_t i = tid; i < hq + hk; i += nt) {
    const size_t t = i < hq ? (size_t)np * hq + i : (size_t)np * hk + (i - hq);
    const uint32_t o = i < hq ? ROPE_ROW_HDR + i : ROPE_ROW_HDR + wq + (i - hq);
    const uint32_t half = i < hq ? hq : hk;
    rrow[o] = cosT[t];
    rrow[o + half] = sinT[t];
  }
  if (tid == 0) *(int32_t*)rrow = (int32_t)np;
}

// x = E[t] and its act (gamma_out may be null), by NT threads: every load of
// a chunk of CH * NT elements is issued before the first store (the stores
// may alias E as far as the compiler knows, so a load-store loop would take
// one memory round trip per iteration).  dim % 32 == 0 with an act.
template <int NT, int CH>
__device__ __forceinline__ void embed_row(const float* __restrict__ E, int32_t t, uint32_t dim, float* x,
                                          uint8_t* act_out, const float* gamma_out, uint32_t tid) {
  for (uint32_t base = 0; base < dim; base += CH * NT) {
    float ev[CH], gv[CH];
#pragma unroll
    for (int q = 0; q < CH; q++) {
      const uint32_t i = base + tid + NT * q;
      ev[q] = i < dim ? E[(size_t)t * dim + i] : 0.f;
      gv[q] = i < dim && gamma_out ? gamma_out[i] : 1.f;
    }
#pragma unroll
    for (int q = 0; q < CH; q++) {
      const uint32_t i = base + tid + NT * q;
      if (i < dim) {
        x[i] = ev[q];
        if (act_out) act_emit8(act_out, dim, i, ev[q], gv[q]);
      }
    }
  }
}

// y[n] = sum_k x[k] * lmHead[k][n] for M = 1, optionally with the final
// RMSNorm of x fused (gamma != null).  Workgroup (bx, split): 16 blocks of
// 32 outputs, the split's row octets shared by 8 waves (at most 4 octets per
// wave: the host picks splits of <= 256 rows), every load of a wave issued
// at once.  Lane (vb, q) owns outputs 32vb + 8q .. +7; per row c = x_k * d,
// 8 fma(c, nibble) and one -8c correction.  Waves are summed in LDS, splits
// by the last-arriving workgroup of the column tile (agent-scope atomics).
// With a greedy tail (gt.E != null), each tile's finisher publishes the
// argmax key of its 512 logits with one 64-bit atomic max, and the last tile
// to finish runs the greedy step with the winning token.
#define LMH_OCT 4
#define LMH_ROWS (8 * 8 * LMH_OCT)

// The greedy step after an LM head's column tile (one workgroup of 512
// threads, thread tid holds logit v of column n): the tile's best key goes
// into gt.amx with an atomic max, and the last tile to arrive runs the step
// (token append, count / position advance, x = E[token] and its act).  The
// max is a returning atomic, complete (performed at agent scope) before the
// tile counter moves, so no fence is needed.  c0 / p0: count and position
// read at the kernel's start (only this last tile writes them).
__device__ __forceinline__ void greedy_finish(float v, uint32_t n, uint32_t N, const GreedyTail& gt, int32_t c0,
                                              int32_t p0) {
  __shared__ uint64_t kred[8];
  __shared__ int g_last;
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint64_t key = wave_max64(n < N ? argmax_key(v, n) : 0ull);
  if (lane == 0) kred[wave] = key;
  __syncthreads();
  if (tid == 0) {
    uint64_t b = kred[0];
    for (int w = 1; w < 8; w++) b = umax64(b, kred[w]);
    kred[0] = __hip_atomic_fetch_max(gt.amx, b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    const uint32_t prev =
        __hip_atomic_fetch_add((uint32_t*)(gt.amx + 1), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    g_last = prev == gridDim.x - 1;
    if (g_last) {
      kred[1] = __hip_atomic_exchange(gt.amx, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store((uint32_t*)(gt.amx + 1), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
  if (!g_last) return;
  const uint64_t best = kred[1];
  const int32_t t = best == 0 ? 0 : (int32_t)(0xFFFFFFFFu - (uint32_t)best);
  if (tid == 0) {
    gt.tokens[c0] = t;
    gt.count[0] = c0 + 1;
    gt.pos[0] = p0 + 1;
  }
  embed_row<512, 6>(gt.E, t, gt.dim, gt.x, gt.act_out, gt.gamma_out, tid);
}

extern "C" __global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(6))) void smith_lmhead_q4_0_nb(
    const float* __restrict__ x, const float* __restrict__ gamma, float eps, const uint8_t* __restrict__ nib,
    const uint16_t* __restrict__ dsc, float* __restrict__ y, uint32_t K, uint32_t N, float* __restrict__ ws,
    uint32_t* __restrict__ counters, GreedyTail gt) {
  __shared__ float xs[LMH_ROWS];
  __shared__ float part[8][512];
  __shared__ float red[8];
  __shared__ int s_last;
  const uint32_t NB = N / 32;
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t vb0 = blockIdx.x * 16 + lane / 4, qq = lane & 3;
  const uint32_t vb = vb0 < NB ? vb0 : NB - 1;  // clamped; lanes past NB store nothing
  const uint32_t ksplit = gridDim.y;
  const uint32_t KO = K / 8;
  const uint32_t ob = (KO + ksplit - 1) / ksplit;  // octets per split (<= 8 * LMH_OCT)
  const uint32_t os0 = blockIdx.y * ob < KO ? blockIdx.y * ob : KO, os1 = os0 + ob < KO ? os0 + ob : KO;
  const uint32_t ow = (os1 - os0 + 7) / 8;  // octets per wave (<= LMH_OCT)
  const uint32_t o0 = os0 + wave * ow < os1 ? os0 + wave * ow : os1, o1 = o0 + ow < os1 ? o0 + ow : os1;

  // 1. x for the norm (the first 4096 entries; the rest, if any, later),
  //    this split's x / gamma, the weights: all in flight
  float xv[8];
#pragma unroll
  for (int q = 0; q < 8; q++) {
    const uint32_t i = tid + 512 * q;
    xv[q] = i < K ? x[i] : 0.f;
  }
  const uint32_t kx = os0 * 8 + tid;
  const bool xin = tid < LMH_ROWS && kx < os1 * 8;
  const float xsv = xin ? x[kx] : 0.f;
  const float gsv = xin && gamma ? gamma[kx] : 1.f;
  u32x4 wn[LMH_OCT][2], wd[LMH_OCT];
#pragma unroll
  for (int j = 0; j < LMH_OCT; j++) {
    uint32_t oc = o0 + j < o1 ? o0 + j : (o1 > 0 ? o1 - 1 : 0);
    oc = oc < KO ? oc : KO - 1;
    const size_t rec = (size_t)oc * NB + vb;
    const uint8_t* pn = nib + rec * 128 + qq * 32;
    wn[j][0] = *(const u32x4*)pn;
    wn[j][1] = *(const u32x4*)(pn + 16);
    wd[j] = *(const u32x4*)(dsc + rec * 8);
  }

  // the greedy step's count and position (written only by this launch's last
  // workgroup, after every other has finished), and the next position's rope
  // row, which does not depend on the token (workgroup (0, 0))
  int32_t c0 = 0, p0 = 0;
  if (gt.E) {
    c0 = gt.count[0];
    p0 = gt.pos[0];
    if (blockIdx.x == 0 && blockIdx.y == 0)
      rope_row_write(gt.rrow, gt.cosT, gt.sinT, gt.rope_len, gt.wq, gt.wk, (uint32_t)p0 + 1, tid, 512);
  }

  // 2. RMSNorm scale; this split's normalized x into LDS
  float rms = 1.f;
  if (gamma) {
    float ss = 0.f;
#pragma unroll
    for (int q = 0; q < 8; q++) ss = __builtin_fmaf(xv[q], xv[q], ss);
    for (uint32_t i = tid + 4096; i < K; i += 512) ss = __builtin_fmaf(x[i], x[i], ss);
    ss = sum64_lanes(ss);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float tot = 0.f;
    for (int w = 0; w < 8; w++) tot += red[w];
    rms = 1.0f / __builtin_sqrtf(tot / (float)K + eps);
  }
  if (tid < LMH_ROWS) xs[tid] = gamma ? xsv * rms * gsv : xsv;
  __syncthreads();

  // 3. rows
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; i++) acc[i] = 0.f;
  float corr = 0.f;
#pragma unroll
  for (int j = 0; j < LMH_OCT; j++) {
    const uint32_t oc = o0 + j;
#pragma unroll
    for (int r = 0; r < 8; r++) {
      const uint32_t dw = wd[j][r / 2];
      const uint16_t dh = (uint16_t)((r & 1) ? dw >> 16 : dw & 0xFFFFu);
      const float c = oc < o1 ? xs[(oc - os0) * 8 + r] * (float)__builtin_bit_cast(_Float16, dh) : 0.f;
      const uint32_t w = wn[j][r / 4][r % 4];
      const uint32_t ev = w & 0x0F0F0F0Fu, od = (w >> 4) & 0x0F0F0F0Fu;  // nibbles 2j / 2j+1 in byte j
      corr += c;
#pragma unroll
      for (int jb = 0; jb < 4; jb++) {
        acc[2 * jb] = __builtin_fmaf(c, (float)((ev >> (8 * jb)) & 0xFFu), acc[2 * jb]);
        acc[2 * jb + 1] = __builtin_fmaf(c, (float)((od >> (8 * jb)) & 0xFFu), acc[2 * jb + 1]);
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 8; e++) part[wave][lane * 8 + e] = __builtin_fmaf(-8.0f, corr, acc[e]);
  __syncthreads();
  const uint32_t n = blockIdx.x * 512 + tid;
  float v = 0.f;
#pragma unroll
  for (int w = 0; w < 8; w++) v += part[w][tid];
  if (ksplit > 1) {
    if (n < N)
      __hip_atomic_exchange((uint32_t*)ws + (size_t)blockIdx.y * N + n, __float_as_uint(v), __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
      uint32_t prev = __hip_atomic_fetch_add(counters + blockIdx.x, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = prev == ksplit - 1;
    }
    __syncthreads();
    if (!s_last) return;
    if (n < N) v = splitk_sum(ws + n, N, ksplit);
    if (tid == 0)
      __hip_atomic_exchange(counters + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (n < N) y[n] = v;
  if (!gt.E) return;

  greedy_finish(v, n, N, gt, c0, p0);
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
// *pos advance.  With rrow, the rope row of the new position (cos / sin of
// the table rows the whole-row RoPE of a q row (wq wide) and a k row (wk
// wide) reads, tag = the position) is written for the next decode step's
// attention, if the tables (rope_len entries each) reach that far.  One workgroup of 1024 threads;
// every thread's logits loads go out together with the count / position
// loads, so the only dependent round trip is the embedding row.
// ---------------------------------------------------------------------------
#define AMX_BATCH 32
extern "C" __global__ __launch_bounds__(1024) void smith_argmax_embed(
    const float* __restrict__ logits, uint32_t N, const float* __restrict__ E, uint32_t dim, float* __restrict__ x,
    int32_t* __restrict__ tokens, int32_t* __restrict__ count, int32_t* __restrict__ pos,
    uint8_t* __restrict__ act_out, const float* __restrict__ gamma_out, const float* __restrict__ cosT,
    const float* __restrict__ sinT, uint32_t rope_len, uint32_t wq, uint32_t wk, float* __restrict__ rrow) {
  __shared__ float bv[16];
  __shared__ int32_t bi[16];
  __shared__ int32_t s_tok;
  const int32_t c0 = count[0], p = pos[0];
  float best = -__builtin_inff();
  int32_t bidx = 0x7fffffff;
  // thread t scans indices t, t + 1024, ... in increasing order
  for (uint32_t i0 = threadIdx.x; i0 < N; i0 += AMX_BATCH * 1024) {
    float v[AMX_BATCH];
#pragma unroll
    for (int u = 0; u < AMX_BATCH; u++) {
      const uint32_t i = i0 + 1024 * u;
      v[u] = logits[i < N ? i : N - 1];
    }
#pragma unroll
    for (int u = 0; u < AMX_BATCH; u++) {
      const uint32_t i = i0 + 1024 * u;
      if (i < N && v[u] > best) {  // strictly greater: earliest index within this thread
        best = v[u];
        bidx = (int32_t)i;
      }
    }
  }
  // the next position's rope row (independent of the token)
  rope_row_write(rrow, cosT, sinT, rope_len, wq, wk, (uint32_t)p + 1, threadIdx.x, 1024);
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
    if (logits[0] != logits[0]) t = 0;  // the reference's scan never moves past a NaN at index 0
    s_tok = t;
    tokens[c0] = t;
    count[0] = c0 + 1;
  }
  __syncthreads();
  const int32_t t = s_tok;
  embed_row<1024, 4>(E, t, dim, x, act_out, gamma_out, threadIdx.x);
  if (threadIdx.x == 0) pos[0] = p + 1;
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

// ---------------------------------------------------------------------------
// LM head on a Q6_K output.weight read as lmHead[K=dim][N=vocab] (256-element
// blocks along vocab, dequantQ6_K, src/gguf.js:309-339).  Planes of one
// buffer (offsets below), in row octets (K % 8 == 0): per (octet k/8,
// 32-column group vb, quarter sub) the 4 low-nibble bytes of the quarter's 8
// outputs for the octet's 8 rows (32 B) and their 2 high-bit bytes (16 B:
// element e's 2 bits at bit 2e) -- the block's ql / qh bytes of that group,
// moved, so a lane reads 8 rows of its outputs in three 16-byte loads and a
// wave 2 KB of contiguous nibbles; the int8 scales transposed to [N/16][K] and
// the f16 d to [N/256][K] (16 / 8 rows per 16-byte load).  Same structure as
// smith_lmhead_q4_0_nb: lane (vb, sub) owns outputs 32vb + 8sub .. +7; per
// row c = x_k * d * scale, 8 fma(c, q) and one -32c correction.
// ---------------------------------------------------------------------------
__host__ __device__ inline void lmh6_offsets(uint32_t K, uint32_t N, size_t* hb, size_t* sc, size_t* d, size_t* total) {
  const size_t KN = (size_t)K * N;
  *hb = gt_align(KN / 2);
  *sc = gt_align(*hb + KN / 4);
  *d = gt_align(*sc + KN / 16);
  *total = gt_align(*d + KN / 256 * 2);
}

extern "C" __global__ void smith_repack_lmhead_q6_k(const uint8_t* __restrict__ src, uint8_t* __restrict__ planes,
                                                    uint32_t K, uint32_t N) {
  size_t ohb, osc, od, tot;
  lmh6_offsets(K, N, &ohb, &osc, &od, &tot);
  const uint32_t NB = N / 256, NB32 = N / 32;
  const size_t total = (size_t)K * NB;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
    const uint32_t k = (uint32_t)(idx / NB), vb = (uint32_t)(idx % NB);
    const uint8_t* b = src + idx * 210;
    for (int i8 = 0; i8 < 8; i8++) {
      const size_t g = ((size_t)(k / 8) * NB32 + vb * 8 + i8) * 4;  // (octet, group) quarter 0
      for (int q = 0; q < 16; q++) planes[(g + q / 4) * 32 + (k % 8) * 4 + q % 4] = b[16 * i8 + q];
      for (int q = 0; q < 8; q++) planes[ohb + (g + q / 2) * 16 + (k % 8) * 2 + q % 2] = b[128 + 8 * i8 + q];
    }
    for (int t = 0; t < 16; t++) planes[osc + ((size_t)vb * 16 + t) * K + k] = b[192 + t];
    ((uint16_t*)(planes + od))[(size_t)vb * K + k] = (uint16_t)(b[208] | (b[209] << 8));
  }
}

#define LMH_BATCH 16  // rows per batch of loads

// two workgroups per CU (<= 128 VGPRs): three rounds of one did not hide the
// batch load latency
extern "C" __global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void smith_lmhead_q6_k_nb(
    const float* __restrict__ x, const float* __restrict__ gamma, float eps, const uint8_t* __restrict__ planes,
    float* __restrict__ y, uint32_t K, uint32_t N, float* __restrict__ ws, uint32_t* __restrict__ counters,
    GreedyTail gt) {
  __shared__ float xs[8192];
  __shared__ float part[8][512];
  __shared__ float red[8];
  __shared__ int s_last;
  size_t ohb, osc, od, tot;
  lmh6_offsets(K, N, &ohb, &osc, &od, &tot);
  const uint8_t* nib = planes;
  const uint16_t* hbp = (const uint16_t*)(planes + ohb);
  const int8_t* scp = (const int8_t*)(planes + osc);
  const uint16_t* dp = (const uint16_t*)(planes + od);
  const uint32_t NB = N / 32;
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t vb0 = blockIdx.x * 16 + lane / 4, sub = lane & 3;
  const uint32_t vb = vb0 < NB ? vb0 : NB - 1;  // clamped; lanes past NB store nothing
  const uint32_t v16 = 2 * vb + sub / 2, v256 = vb / 8;
  const uint32_t ksplit = gridDim.y;
  // split and wave row counts are multiples of 16 (K % 16 == 0): aligned 16-byte scale loads
  const uint32_t kb = ((K + ksplit - 1) / ksplit + 15) / 16 * 16;
  const uint32_t kb0 = blockIdx.y * kb < K ? blockIdx.y * kb : K, kb1 = kb0 + kb < K ? kb0 + kb : K;
  const uint32_t kper = ((kb1 - kb0 + 7) / 8 + 15) / 16 * 16;
  const uint32_t k0 = kb0 + wave * kper < kb1 ? kb0 + wave * kper : kb1;
  const uint32_t k1 = k0 + kper < kb1 ? k0 + kper : kb1;

  float xv[16], gvv[16];
#pragma unroll
  for (int q = 0; q < 16; q++) {
    const uint32_t i = threadIdx.x + 512 * q;
    xv[q] = i < K ? x[i] : 0.f;
    gvv[q] = gamma && i < K ? gamma[i] : 1.f;
  }
  // a batch's raw loads (the 16-bit high-bit words stay packed until use:
  // both batches' registers live at once)
  uint4 wn[LMH_BATCH / 4], wh[LMH_BATCH / 8];
  uint4 ws8, wd[2];
  // kbase is a multiple of 16 below k1, and k1 a multiple of 16: both octets
  // of a batch lie inside the wave's rows
  auto load_batch = [&](uint32_t kbase) {
#pragma unroll
    for (int oc = 0; oc < LMH_BATCH / 8; oc++) {
      const size_t g = ((size_t)(kbase / 8 + oc) * NB + vb) * 4 + sub;
      wn[2 * oc] = *(const uint4*)(nib + g * 32);
      wn[2 * oc + 1] = *(const uint4*)(nib + g * 32 + 16);
      wh[oc] = *(const uint4*)((const uint8_t*)hbp + g * 16);
    }
    const uint32_t kc = kbase < K ? kbase : K - 16;  // K % 16 == 0
    ws8 = *(const uint4*)(scp + (size_t)v16 * K + kc);
    wd[0] = *(const uint4*)(dp + (size_t)v256 * K + kc);
    wd[1] = *(const uint4*)(dp + (size_t)v256 * K + kc + 8);
  };
  if (k0 < k1) load_batch(k0);

  // the greedy step's count and position (written only by this launch's last
  // workgroup) and the next position's rope row (workgroup (0, 0))
  int32_t c0 = 0, p0 = 0;
  if (gt.E) {
    c0 = gt.count[0];
    p0 = gt.pos[0];
    if (blockIdx.x == 0 && blockIdx.y == 0)
      rope_row_write(gt.rrow, gt.cosT, gt.sinT, gt.rope_len, gt.wq, gt.wk, (uint32_t)p0 + 1, threadIdx.x, 512);
  }

  float ss = 0.f;
#pragma unroll
  for (int q = 0; q < 16; q++) ss = __builtin_fmaf(xv[q], xv[q], ss);
  float rms = 1.f;
  if (gamma) {
    for (int d = 32; d >= 1; d >>= 1) ss += __shfl_xor(ss, d);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float tot2 = 0.f;
    for (int w = 0; w < 8; w++) tot2 += red[w];
    rms = 1.0f / __builtin_sqrtf(tot2 / (float)K + eps);
  }
#pragma unroll
  for (int q = 0; q < 16; q++) {
    const uint32_t i = threadIdx.x + 512 * q;
    if (i < K) xs[i] = gamma ? xv[q] * rms * gvv[q] : xv[q];
  }
  __syncthreads();

  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; i++) acc[i] = 0.f;
  float corr = 0.f;
  for (uint32_t kb16 = k0; kb16 < k1; kb16 += LMH_BATCH) {
    uint4 cn[LMH_BATCH / 4], ch[LMH_BATCH / 8];
#pragma unroll
    for (int q = 0; q < LMH_BATCH / 4; q++) cn[q] = wn[q];
#pragma unroll
    for (int q = 0; q < LMH_BATCH / 8; q++) ch[q] = wh[q];
    const uint4 cs = ws8, cd0 = wd[0], cd1 = wd[1];
    if (kb16 + LMH_BATCH < k1) load_batch(kb16 + LMH_BATCH);
#pragma unroll
    for (int r = 0; r < LMH_BATCH; r++) {
      const uint32_t k = kb16 + r;
      const uint32_t sw = (&cs.x)[r / 4];
      const int8_t sc = (int8_t)((sw >> (8 * (r % 4))) & 0xFFu);
      const uint32_t dw = r < 8 ? (&cd0.x)[r / 2] : (&cd1.x)[(r - 8) / 2];
      const uint16_t dh = (uint16_t)((r & 1) ? dw >> 16 : dw & 0xFFFFu);
      const float c = k < k1 ? xs[k] * ((float)__builtin_bit_cast(_Float16, dh) * (float)sc) : 0.f;
      const uint32_t w = (&cn[r / 4].x)[r % 4];
      const uint32_t hw = (&ch[r / 8].x)[(r % 8) / 2];
      const uint32_t h = (r & 1) ? hw >> 16 : hw & 0xFFFFu;
      corr += c;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const uint32_t q = ((w >> (4 * e)) & 0xFu) | (((h >> (2 * e)) & 3u) << 4);
        acc[e] = __builtin_fmaf(c, (float)q, acc[e]);
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 8; e++) part[wave][lane * 8 + e] = __builtin_fmaf(-32.0f, corr, acc[e]);
  __syncthreads();
  const uint32_t nb0 = blockIdx.x * 512;
  const uint32_t o = threadIdx.x, n = nb0 + o;
  float v = 0.f;
#pragma unroll
  for (int w = 0; w < 8; w++) v += part[w][o];
  if (ksplit > 1) {
    if (n < N)
      __hip_atomic_exchange((uint32_t*)ws + (size_t)blockIdx.y * N + n, __float_as_uint(v), __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
      uint32_t prev = __hip_atomic_fetch_add(counters + blockIdx.x, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = prev == ksplit - 1;
    }
    __syncthreads();
    if (!s_last) return;
    if (n < N) v = splitk_sum(ws + n, N, ksplit);
    if (threadIdx.x == 0)
      __hip_atomic_exchange(counters + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (n < N) y[n] = v;
  if (gt.E) greedy_finish(v, n, N, gt, c0, p0);
}

// ---------------------------------------------------------------------------
// GGUF weights [out=N rows, in=K] of Q4_0 / Q4_1 / Q5_0 / Q4_K / Q6_K blocks
// -> the tile planes of gguf_tiles.h.  Values are moved, never changed: the
// same integers, f16 fields and 6-bit / int8 scales the reference's decoders
// read (src/gguf.js:187-339), at the record of column n_off + n * n_stride of
// an N_total-column buffer (q|k|v side by side, gate/up interleaved).
// One thread per (row, 32-element group).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

template <int F>
__device__ __forceinline__ void repack_gguf_tiles(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                  uint32_t N, uint32_t G, uint32_t n_off, uint32_t n_stride,
                                                  uint32_t N_total) {
  const GtPlanes P = gt_planes(F, N_total, G);
  const size_t total = (size_t)N * G;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
    const uint32_t n = (uint32_t)(idx / G), g = (uint32_t)(idx % G);
    const uint32_t col = n_off + n * n_stride;
    const size_t rec = ((size_t)(col >> 4) * G + g) * 16 + (col & 15);
    const uint32_t sb = g >> 3, i8 = g & 7;  // super-block and sub-block (Q4_K / Q6_K)
    const uint8_t* blk;
    const uint8_t* qs;
    if (F == GT_Q41) blk = src + idx * 20, qs = blk + 4;
    else if (F == GT_Q50) blk = src + idx * 22, qs = blk + 6;
    else if (F == GT_Q4K) blk = src + ((size_t)n * (G / 8) + sb) * 144, qs = blk + 16 + 16 * i8;
    else if (F == GT_Q6K) blk = src + ((size_t)n * (G / 8) + sb) * 210, qs = blk + 16 * i8;
    else blk = src + idx * 18, qs = blk + 2;
    uint32_t w[4];
#pragma unroll
    for (int d = 0; d < 4; d++)
      w[d] = (uint32_t)qs[4 * d] | ((uint32_t)qs[4 * d + 1] << 8) | ((uint32_t)qs[4 * d + 2] << 16) |
             ((uint32_t)qs[4 * d + 3] << 24);
    *(uint4*)(dst + rec * 16) = make_uint4(w[0], w[1], w[2], w[3]);
    if (F == GT_Q50) {
      const uint32_t hb = ld_u16(blk + 2) | (ld_u16(blk + 4) << 16);  // bit e: element e
      uint32_t W = 0;
#pragma unroll
      for (int e = 0; e < 32; e++) {
        const int i = e >> 3, k = e & 7;
        W |= ((hb >> e) & 1u) << (4 * i + (k & 3) + 16 * (k >> 2));
      }
      *(uint32_t*)(dst + P.hb + rec * 4) = W;
    }
    if (F == GT_Q6K) {
      const uint8_t* qh = blk + 128 + 8 * i8;  // elements 32*i8 .. +31: 2 bits each, 4 per byte
      uint32_t W0 = 0, W1 = 0;
#pragma unroll
      for (int e = 0; e < 32; e++) {
        const int i = e >> 3, k = e & 7;
        const uint32_t v = (qh[e >> 2] >> (2 * (e & 3))) & 3u;
        const uint32_t pos = 2 * (4 * (i & 1) + (k & 3)) + 16 * (k >> 2);
        if (i < 2) W0 |= v << pos;
        else W1 |= v << pos;
      }
      *(uint2*)(dst + P.hb + rec * 8) = make_uint2(W0, W1);
    }
    if (F == GT_Q41) {
      *(uint32_t*)(dst + P.prm + rec * 4) = ld_u16(blk) | (ld_u16(blk + 2) << 16);
    } else if (F == GT_Q4K) {
      // 6-bit (scale, min) of sub-block i8 as src/gguf.js:281-291 unpacks them
      const uint8_t* s12 = blk + 4;
      uint32_t sc, mn;
      if (i8 < 4) {
        sc = s12[i8] & 0x3Fu;
        mn = s12[4 + i8] & 0x3Fu;
      } else {
        sc = (uint32_t)(s12[i8 - 4] >> 6) | ((uint32_t)(s12[i8 + 4] & 0x0F) << 2);
        mn = (uint32_t)(s12[i8] >> 6) | ((uint32_t)(s12[i8 + 4] >> 4) << 2);
      }
      *(uint16_t*)(dst + P.prm + rec * 2) = (uint16_t)(sc | (mn << 8));
    } else if (F == GT_Q6K) {
      *(uint16_t*)(dst + P.prm + rec * 2) = (uint16_t)ld_u16(blk + 192 + 2 * i8);
    } else {
      *(uint16_t*)(dst + P.prm + rec * 2) = (uint16_t)ld_u16(blk);
    }
    if (gt_super(F) && i8 == 0) {
      const size_t srec = ((size_t)(col >> 4) * (G / 8) + sb) * 16 + (col & 15);
      if (F == GT_Q4K) *(uint32_t*)(dst + P.sup + srec * 4) = ld_u16(blk) | (ld_u16(blk + 2) << 16);
      else *(uint16_t*)(dst + P.sup + srec * 2) = (uint16_t)ld_u16(blk + 208);
    }
  }
}

#define DEF_REPACK_GT(NAME, F)                                                                                  \
  extern "C" __global__ void NAME(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, uint32_t N,      \
                                  uint32_t G, uint32_t n_off, uint32_t n_stride, uint32_t N_total) {           \
    repack_gguf_tiles<F>(src, dst, N, G, n_off, n_stride, N_total);                                           \
  }
DEF_REPACK_GT(smith_repack_gt_q40, GT_Q40)
DEF_REPACK_GT(smith_repack_gt_q41, GT_Q41)
DEF_REPACK_GT(smith_repack_gt_q50, GT_Q50)
DEF_REPACK_GT(smith_repack_gt_q4k, GT_Q4K)
DEF_REPACK_GT(smith_repack_gt_q6k, GT_Q6K)

// ---------------------------------------------------------------------------
// dequantizeTensor (src/gguf.js:343-394) on the device: element idx of a flat
// tensor from its block, evaluated as the reference does -- f64 products
// and sums of the exactly decoded f16 fields and integers, one rounding to
// f32 (Float32Array store).  F16 by exact conversion, BF16 by a 16-bit shift
// (F32 needs no kernel).  One thread per element.
// ---------------------------------------------------------------------------
__device__ __forceinline__ double f16_to_f64(uint32_t h) { return (double)(float)__builtin_bit_cast(_Float16, (uint16_t)h); }

template <int T>
__device__ __forceinline__ float dequant_elem(const uint8_t* __restrict__ src, size_t idx) {
  if (T == 1) return (float)__builtin_bit_cast(_Float16, (uint16_t)ld_u16(src + 2 * idx));
  if (T == 30) return __uint_as_float(ld_u16(src + 2 * idx) << 16);
  const uint32_t be = (T == 12 || T == 14) ? 256 : 32;
  const uint32_t bb = T == 2 ? 18 : (T == 3 ? 20 : (T == 6 ? 22 : (T == 8 ? 34 : (T == 12 ? 144 : 210))));
  const uint8_t* blk = src + (idx / be) * bb;
  const uint32_t j = (uint32_t)(idx % be);
  auto nib = [&](const uint8_t* qs) { const uint8_t b = qs[j >> 1]; return (int)((j & 1) ? (b >> 4) : (b & 15)); };
  if (T == 2) return (float)(f16_to_f64(ld_u16(blk)) * (double)(nib(blk + 2) - 8));
  if (T == 3) return (float)(f16_to_f64(ld_u16(blk)) * (double)nib(blk + 4) + f16_to_f64(ld_u16(blk + 2)));
  if (T == 6) {
    const uint32_t hb = ld_u16(blk + 2) | (ld_u16(blk + 4) << 16);
    return (float)(f16_to_f64(ld_u16(blk)) * (double)((nib(blk + 6) | (int)(((hb >> j) & 1u) << 4)) - 16));
  }
  if (T == 8) return (float)(f16_to_f64(ld_u16(blk)) * (double)(int8_t)blk[2 + j]);
  if (T == 12) {
    const uint32_t i = j >> 5;
    const uint8_t* s12 = blk + 4;
    uint32_t sc, mn;
    if (i < 4) {
      sc = s12[i] & 0x3Fu;
      mn = s12[4 + i] & 0x3Fu;
    } else {
      sc = (uint32_t)(s12[i - 4] >> 6) | ((uint32_t)(s12[i + 4] & 0x0F) << 2);
      mn = (uint32_t)(s12[i] >> 6) | ((uint32_t)(s12[i + 4] >> 4) << 2);
    }
    const float scf = (float)(f16_to_f64(ld_u16(blk)) * (double)sc);
    const float mnf = (float)(f16_to_f64(ld_u16(blk + 2)) * (double)mn);
    return (float)((double)scf * (double)nib(blk + 16) - (double)mnf);
  }
  // Q6_K
  const int q = nib(blk) | (int)(((blk[128 + (j >> 2)] >> (2 * (j & 3))) & 3u) << 4);
  return (float)(f16_to_f64(ld_u16(blk + 208)) * (double)(int8_t)blk[192 + (j >> 4)] * (double)(q - 32));
}

#define DEF_DEQUANT(NAME, T)                                                                                   \
  extern "C" __global__ void NAME(const uint8_t* __restrict__ src, float* __restrict__ dst, uint64_t numel) { \
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < numel;                              \
         idx += (size_t)gridDim.x * blockDim.x)                                                               \
      dst[idx] = dequant_elem<T>(src, idx);                                                                    \
  }
DEF_DEQUANT(smith_dequantize_f16, 1)
DEF_DEQUANT(smith_dequantize_bf16, 30)
DEF_DEQUANT(smith_dequantize_q4_0, 2)
DEF_DEQUANT(smith_dequantize_q4_1, 3)
DEF_DEQUANT(smith_dequantize_q5_0, 6)
DEF_DEQUANT(smith_dequantize_q8_0, 8)
DEF_DEQUANT(smith_dequantize_q4_k, 12)
DEF_DEQUANT(smith_dequantize_q6_k, 14)
