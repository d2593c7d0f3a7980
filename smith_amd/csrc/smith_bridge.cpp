// smith_bridge.cpp -- libsmith.so: the C-ABI HIP bridge (include/smith.h).
//
// Replaces native/gpu_bridge.m (Objective-C + Metal).  Design differences,
// all deliberate for MI355X:
//   * buffers are hipMalloc device memory; the host reaches them with explicit
//     copies (no unified-memory views);
//   * kernels come from a gfx950 code object loaded with hipModuleLoad (or
//     hipRTC for smith_compile_source) and are looked up by name;
//   * one stream per context; encoders enqueue, end_sync/end_timed wait;
//   * op-level entry points (smith_matmul_q4, ...) pick the kernel variant
//     and launch geometry here, so a host language needs one FFI call per op.
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <algorithm>
#include <chrono>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <atomic>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/smith.h"
#include "gguf_tiles.h"

namespace {

struct Library {
  hipModule_t mod = nullptr;
  std::unordered_map<std::string, hipFunction_t> fns;
};

struct Pipeline {
  hipFunction_t fn;
  std::string name;
};

struct Ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  hipEvent_t t0 = nullptr, t1 = nullptr;
  std::string err;
  std::vector<Library*> libs;
  Library* ops = nullptr;
  std::vector<Pipeline*> pipelines;
  uint64_t allocated = 0;
  // op scratch: prepared activations, split-K partials, split-K counters
  void* prep = nullptr;
  size_t prep_bytes = 0;
  float* ws = nullptr;
  size_t ws_bytes = 0;
  uint32_t* counters = nullptr;
  uint64_t* amx = nullptr;  // greedy LM head: best key, tiles finished (zero between calls)
  size_t counters_n = 0;
  void* normbuf = nullptr;
  size_t normbuf_bytes = 0;
  void* a16 = nullptr;  // f16 activations of the GEMM path
  size_t a16_bytes = 0;
  // smith_prep_next: the next GEMM's K-split reduce also writes its output
  // as the A operand of the GEMM after it (a16_* say which one it fits)
  bool next_pending = false;
  const float* next_gamma = nullptr;
  float next_eps = 0.f;
  const float* a16_src = nullptr;
  const float* a16_gamma = nullptr;
  float a16_eps = 0.f;
  uint32_t a16_M = 0, a16_K = 0;
  void* att_ws = nullptr;
  size_t att_ws_bytes = 0;
  uint32_t* att_cnt = nullptr;
  size_t att_cnt_n = 0;
  bool capturing = false;
  // set while an entry point that must not allocate runs on the static
  // scratch (its name, for the error when a region is too small)
  const char* no_alloc = nullptr;
  // device-side position bound failures (attention, KV append): host-mapped
  // words {code, p0, S} the kernels store into, read at every synchronising
  // call (pos_err_host) and passed to kernels as pos_err_dev
  uint32_t* pos_err_host = nullptr;
  uint32_t* pos_err_dev = nullptr;
  // scratch buffers replaced by bigger ones: a captured graph may still name
  // them, so they are freed only with the context
  std::vector<void*> retired;
  // per-launch HIP event pairs of op-level kernels while profiling is on
  bool profile = false;
  struct Rec {
    std::string name;
    hipEvent_t a, b;
  };
  std::vector<Rec> recs;
  std::vector<hipEvent_t> event_pool;
};

struct BufInfo {
  Ctx* ctx;
  uint64_t bytes;
};

std::mutex g_mu;
std::unordered_map<void*, BufInfo> g_bufs;

int fail(Ctx* c, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (c) c->err = buf;
  return -1;
}

#define HIPCHK(c, expr)                                                                 \
  do {                                                                                  \
    hipError_t e_ = (expr);                                                             \
    if (e_ != hipSuccess) return fail((c), "%s: %s", #expr, hipGetErrorString(e_));     \
  } while (0)

double now_s() {
  using namespace std::chrono;
  return duration<double>(steady_clock::now().time_since_epoch()).count();
}

int set_device(Ctx* c) {
  HIPCHK(c, hipSetDevice(c->device));
  return 0;
}

int lookup(Ctx* c, Library* lib, const char* name, hipFunction_t* out) {
  if (!lib) return fail(c, "smith: no code object loaded (call smith_load_library first)");
  auto it = lib->fns.find(name);
  if (it != lib->fns.end()) {
    *out = it->second;
    return 0;
  }
  hipFunction_t f;
  hipError_t e = hipModuleGetFunction(&f, lib->mod, name);
  if (e != hipSuccess) return fail(c, "smith: kernel '%s' not found in code object", name);
  lib->fns[name] = f;
  *out = f;
  return 0;
}

hipEvent_t pooled_event(Ctx* c) {
  if (!c->event_pool.empty()) {
    hipEvent_t e = c->event_pool.back();
    c->event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

// Op kernels may live in any loaded code object (smith_kernels.hsaco,
// smith_llama.hsaco, ...): first match in load order wins.
int find_kernel(Ctx* c, const char* name, hipFunction_t* out) {
  if (c->libs.empty()) return fail(c, "smith: no code object loaded (call smith_load_library first)");
  for (Library* lib : c->libs) {
    auto it = lib->fns.find(name);
    if (it != lib->fns.end()) {
      *out = it->second;
      return 0;
    }
    hipFunction_t f;
    if (hipModuleGetFunction(&f, lib->mod, name) == hipSuccess) {
      lib->fns[name] = f;
      *out = f;
      return 0;
    }
  }
  return fail(c, "smith: kernel '%s' not found in any loaded code object", name);
}

// The smith_prep_next hint and the prepared f16 operand it leads to belong to
// the one call that follows: gemm() and the prefill attention read them
// before their first launch and set them after their last, so every other
// launch and every copy into device memory drops them here.
void drop_hints(Ctx* c) {
  c->next_pending = false;
  c->a16_src = nullptr;
}

int launch(Ctx* c, const char* name, dim3 grid, dim3 block, void** args, unsigned shmem = 0) {
  drop_hints(c);
  hipFunction_t f;
  if (find_kernel(c, name, &f)) return -1;
  hipEvent_t ea = nullptr, eb = nullptr;
  if (c->profile) {
    ea = pooled_event(c);
    eb = pooled_event(c);
    if (ea && eb) HIPCHK(c, hipEventRecord(ea, c->stream));
  }
  HIPCHK(c, hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z, shmem, c->stream,
                                  args, nullptr));
  if (c->profile && ea && eb) {
    HIPCHK(c, hipEventRecord(eb, c->stream));
    c->recs.push_back(Ctx::Rec{name, ea, eb});
  }
  return 0;
}

// Zero fresh device memory on the context's stream and wait for it.  A plain
// hipMemset runs on the null stream, which the context's non-blocking stream
// is not ordered after: a kernel enqueued next could read the counters
// before they are zero, and a counter that never reaches its "last arrival"
// value is never reset by the kernels, so every later call would go wrong.
int zero_now(Ctx* c, void* p, size_t bytes) {
  HIPCHK(c, hipMemsetAsync(p, 0, bytes, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return 0;
}

// Grow-only device scratch owned by the context.  Growing waits for the
// stream so no enqueued kernel still uses the old allocation.
int ensure(Ctx* c, void** p, size_t* have, size_t need) {
  if (need <= *have) return 0;
  if (c->no_alloc)
    return fail(c, "%s: needs a %zu-byte scratch region, the static scratch region holds %zu bytes (use the "
                "allocating entry point for this size)", c->no_alloc, need, *have);
  if (c->capturing)
    return fail(c, "smith: scratch of %zu bytes needed while capturing a graph; run the op once before capture",
                need);
  HIPCHK(c, hipStreamSynchronize(c->stream));
  if (*p) c->retired.push_back(*p);  // a captured graph may still use it
  *p = nullptr;
  *have = 0;
  size_t sz = (need + 0xFFFFF) & ~(size_t)0xFFFFF;
  HIPCHK(c, hipMalloc(p, sz));
  *have = sz;
  c->allocated += sz;  // the device's allocated size counts the op scratch too
  return 0;
}

// Called after the stream has drained: reports (once) a position bound
// failure that a kernel recorded on the device since the last check.
int check_pos_err(Ctx* c) {
  volatile uint32_t* e = c->pos_err_host;
  if (!e || e[0] == 0) return 0;
  static const char* who[] = {"?", "smith_kv_append", "smith_attention", "smith_attention (prefill)",
                              "smith_attention_parts"};
  const uint32_t code = e[0], p0 = e[1], S = e[2];
  e[1] = e[2] = 0;
  e[0] = 0;
  return fail(c, "%s: positions %d .. %d lie outside the KV cache or the whole-row RoPE table (device bound "
              "check); the launch read and wrote no cache or table entry",
              who[code < 5 ? code : 0], (int32_t)p0, (int32_t)(p0 + S) - 1);
}

int ensure_counters(Ctx* c, size_t n) {
  if (n <= c->counters_n) return 0;
  if (c->no_alloc)
    return fail(c, "%s: needs %zu split-K counters, the static scratch holds %zu", c->no_alloc, n, c->counters_n);
  if (c->capturing) return fail(c, "smith: split-K counters needed while capturing a graph; run the op once first");
  HIPCHK(c, hipStreamSynchronize(c->stream));
  if (c->counters) c->retired.push_back(c->counters);  // a captured graph may still use them
  c->counters = nullptr;
  c->counters_n = 0;
  size_t cap = std::max<size_t>(n, 4096);
  HIPCHK(c, hipMalloc((void**)&c->counters, cap * sizeof(uint32_t)));
  c->allocated += cap * sizeof(uint32_t);
  // counters start at zero once; the kernel's last workgroup resets its own
  if (zero_now(c, c->counters, cap * sizeof(uint32_t))) return -1;
  c->counters_n = cap;
  return 0;
}

int ensure_amx(Ctx* c) {
  if (c->amx) return 0;
  if (c->capturing) return fail(c, "smith: greedy LM head state needed while capturing a graph; run the op once first");
  HIPCHK(c, hipMalloc((void**)&c->amx, 2 * sizeof(uint64_t)));
  c->allocated += 2 * sizeof(uint64_t);
  if (zero_now(c, c->amx, 2 * sizeof(uint64_t))) return -1;
  return 0;
}

// Kernel argument of smith_lmhead_q4_0_nb (same layout as the device struct).
struct GreedyTail {
  const float* E;
  float* x;
  int32_t* tokens;
  int32_t* count;
  int32_t* pos;
  void* act_out;
  const float* gamma_out;
  const float* cosT;
  const float* sinT;
  float* rrow;
  uint64_t* amx;
  uint32_t rope_len, wq, wk, dim;
};

enum Fmt { FQ4S = 0, FQ8 = 1, FQ40 = 2, FQ40T = 3, FQ41T = 4, FQ50T = 5, FQ4KT = 6, FQ6KT = 7 };

const char* fmt_tag(Fmt f) {
  static const char* tags[] = {"q4s", "q8", "q40", "q40t", "q41t", "q50t", "q4kt", "q6kt"};
  return tags[f];
}

// M > 2 with K % 32 != 0: prepare the activations once (smith_qprep_*), then
// the 16-row MFMA GEMV (smith_qgemv3_*).  Buckets must match DEF_QGEMV3_FMT.
struct Epi {
  const float* gamma = nullptr;  // RMSNorm of the activation rows first
  float eps = 0.f;
  const float* resid = nullptr;  // out = resid + y
  uint32_t mode = 0;             // 0 store, 1 residual, 2 SwiGLU on (gate, up) column pairs
};

int qgemv3_chunk(Ctx* c, Fmt fmt, const float* a, const void* B, const void* D, float* out, uint32_t M,
                 uint32_t N, uint32_t K, uint32_t G, const Epi& ep) {
  const char* tag = fmt_tag(fmt);
  const char* ptag = fmt == FQ4S ? "q4" : (fmt == FQ8 ? "q8" : "q40");  // Q4_0 layouts share one prep
  uint32_t bucket = M <= 4 ? 4 : (M <= 8 ? 8 : (M <= 16 ? 16 : 32));
  bool hilo = bucket <= 8;
  uint32_t RB = bucket == 32 ? 2 : 1;
  size_t frag_bytes = (size_t)RB * G * 64 * 16;
  size_t cst_bytes = (size_t)RB * G * 16 * 8;
  if (ensure(c, &c->prep, &c->prep_bytes, frag_bytes + cst_bytes)) return -1;
  void* frag = c->prep;
  void* cst = (char*)c->prep + frag_bytes;
  if (ep.gamma) {
    // RMSNorm rows into a context buffer, then GEMV on the normalized rows
    if (ensure(c, &c->normbuf, &c->normbuf_bytes, (size_t)M * K * sizeof(float))) return -1;
    const float* pa = a;
    const float* pg = ep.gamma;
    void* py = c->normbuf;
    uint32_t pr = M, pc = K;
    float pe = ep.eps;
    void* nargs[] = {&pa, &pg, &py, &pr, &pc, &pe};
    if (launch(c, "smith_rmsnorm_rows", dim3(M), dim3(256), nargs)) return -1;
    a = (const float*)c->normbuf;
  }
  char name[64];
  snprintf(name, sizeof name, "smith_qprep_%s_%s", ptag, hilo ? "hilo" : "plain");
  uint64_t threads = (uint64_t)RB * (hilo ? 8 : 16) * G * 4;
  {
    const float* pa = a;
    uint32_t pM = M, pK = K, pG = G, pRB = RB;
    void* args[] = {&pa, &frag, &cst, &pM, &pK, &pG, &pRB};
    if (launch(c, name, dim3((unsigned)((threads + 255) / 256)), dim3(256), args)) return -1;
  }
  // 32 columns per block (CT=2, S=1, WK=8), or 16 (the _c1 variants) when
  // 32-column blocks would leave CUs idle (e.g. N = 1024: 128 -> 256 blocks)
  const uint32_t kb = 32, nthreads = 512;
  const uint32_t ksplit = (G + kb - 1) / kb;
  const bool c1 = (uint64_t)((N + 31) / 32) * ksplit < 256;
  const uint32_t bc = c1 ? 16 : 32;
  uint32_t gx = (N + bc - 1) / bc;
  if (ksplit > 1) {
    if (ensure(c, (void**)&c->ws, &c->ws_bytes, (size_t)ksplit * M * N * sizeof(float))) return -1;
    if (ensure_counters(c, gx)) return -1;
  }
  snprintf(name, sizeof name, "smith_qgemv3_%s_m%u%s", tag, bucket, c1 ? "_c1" : "");
  const void* pB = B;
  const void* pD = D;
  float* pC = out;
  float* pws = c->ws;
  uint32_t* pcnt = c->counters;
  uint32_t pM = M, pN = N, pG = G;
  const float* pR = ep.resid;
  uint32_t pepi = ep.mode;
  const float* pA = a;  // the rows the prep read (normalised when ep.gamma): the f32 fallback's input
  uint32_t pK = K;
  void* args[] = {&frag, &cst, &pB, &pD, &pC, &pws, &pcnt, &pM, &pN, &pG, &pR, &pepi, &pA, &pK};
  return launch(c, name, dim3(gx, ksplit), dim3(nthreads), args);
}

// 2 < M <= 32 in one launch (smith_qgemv4_*): each workgroup converts its K
// range of the activations into MFMA fragments in LDS.  64 columns per
// block; 32 groups per block unless that leaves fewer than ~200 blocks.
int qgemv4_chunk(Ctx* c, Fmt fmt, const float* a, const void* B, const void* D, float* out, uint32_t M,
                 uint32_t N, uint32_t K, uint32_t G, const Epi& ep) {
  const char* tag = fmt_tag(fmt);
  const char* rows = M <= 8 ? "h8" : (M <= 16 ? "p16" : "p32");
  if (ep.gamma) {
    if (ensure(c, &c->normbuf, &c->normbuf_bytes, (size_t)M * K * sizeof(float))) return -1;
    const float* pa = a;
    const float* pg = ep.gamma;
    void* py = c->normbuf;
    uint32_t pr = M, pc = K;
    float pe = ep.eps;
    void* nargs[] = {&pa, &pg, &py, &pr, &pc, &pe};
    if (launch(c, "smith_rmsnorm_rows", dim3(M), dim3(256), nargs)) return -1;
    a = (const float*)c->normbuf;
  }
  static const int force_kb = [] {
    const char* e = getenv("SMITH_QGEMV4_KB");
    return e ? atoi(e) : 0;
  }();
  // 64 columns per block; 32-column blocks (the _n32 variants, M <= 8) when
  // even 16-group K splits leave fewer than ~200 blocks (e.g. N = 1024)
  const bool n32 = M <= 8 && (uint64_t)((N + 63) / 64) * ((G + 15) / 16) < 200;
  const uint32_t bc = n32 ? 32 : 64;
  const uint32_t gx = (N + bc - 1) / bc;
  uint32_t kb = force_kb == 16 ? 16 : 32;
  if (kb == 32 && (uint64_t)gx * ((G + 31) / 32) < 200) kb = 16;
  const uint32_t ksplit = (G + kb - 1) / kb;
  if (ksplit > 1) {
    if (ensure(c, (void**)&c->ws, &c->ws_bytes, (size_t)ksplit * M * N * sizeof(float))) return -1;
    if (ensure_counters(c, gx)) return -1;
  }
  char name[64];
  snprintf(name, sizeof name, "smith_qgemv4_%s_%s_k%u%s", tag, rows, kb, n32 ? "_n32" : "");
  const float* pa = a;
  const void* pB = B;
  const void* pD = D;
  float* pC = out;
  float* pws = c->ws;
  uint32_t* pcnt = c->counters;
  uint32_t pM = M, pN = N, pK = K, pG = G;
  const float* pR = ep.resid;
  uint32_t pepi = ep.mode;
  void* args[] = {&pa, &pB, &pD, &pC, &pws, &pcnt, &pM, &pN, &pK, &pG, &pR, &pepi};
  return launch(c, name, dim3(gx, ksplit), dim3(512), args);
}

// 2 < M <= 32 in one launch (smith_qgemv5_*): each wave converts the
// activations of its own groups (K % 32 == 0).  Whole K (<= 128 groups) per
// block when 16-column blocks give 128..320 workgroups (M <= 16); M = 32
// runs 16 waves over 64-group K ranges and 32 columns when that gives
// 192..320 workgroups (a 2-way K split at 4096 x 4096); narrower outputs
// split K into 32-group ranges; wider ones (or longer K) use 64-column
// blocks over 32-group ranges.
int qgemv5_chunk(Ctx* c, Fmt fmt, const float* a, const void* B, const void* D, float* out, uint32_t M,
                 uint32_t N, uint32_t K, uint32_t G, const Epi& ep) {
  const char* tag = fmt_tag(fmt);
  const uint32_t bucket = M <= 4 ? 4 : (M <= 8 ? 8 : (M <= 16 ? 16 : 32));
  if (ep.gamma) {
    if (ensure(c, &c->normbuf, &c->normbuf_bytes, (size_t)M * K * sizeof(float))) return -1;
    const float* pa = a;
    const float* pg = ep.gamma;
    void* py = c->normbuf;
    uint32_t pr = M, pc = K;
    float pe = ep.eps;
    void* nargs[] = {&pa, &pg, &py, &pr, &pc, &pe};
    if (launch(c, "smith_rmsnorm_rows", dim3(M), dim3(256), nargs)) return -1;
    a = (const float*)c->normbuf;
  }
  const uint32_t nb16 = (N + 15) / 16;
  const char* var;
  uint32_t gx, ksplit, threads;
  if (bucket <= 16 && G <= 128 && nb16 >= 128 && nb16 <= 320) {
    var = "w16", gx = nb16, ksplit = 1, threads = 1024;
  } else if (bucket == 32 && (N + 31) / 32 * ((G + 63) / 64) >= 192 &&
             (uint64_t)((N + 31) / 32) * ((G + 63) / 64) <= 320) {
    var = "k64c2", gx = (N + 31) / 32, ksplit = (G + 63) / 64, threads = 1024;
  } else if (nb16 < 128) {
    var = "k32", gx = nb16, ksplit = (G + 31) / 32, threads = 512;
  } else {
    var = "k32c4", gx = (N + 63) / 64, ksplit = (G + 31) / 32, threads = 512;
  }
  if (ksplit > 1) {
    if (ensure(c, (void**)&c->ws, &c->ws_bytes, (size_t)ksplit * M * N * sizeof(float))) return -1;
    if (ensure_counters(c, gx)) return -1;
  }
  char name[64];
  snprintf(name, sizeof name, "smith_qgemv5_%s_m%u_%s", tag, bucket, var);
  const float* pa = a;
  const void* pB = B;
  const void* pD = D;
  float* pC = out;
  float* pws = c->ws;
  uint32_t* pcnt = c->counters;
  uint32_t pM = M, pN = N, pK = K, pG = G;
  const float* pR = ep.resid;
  uint32_t pepi = ep.mode;
  void* args[] = {&pa, &pB, &pD, &pC, &pws, &pcnt, &pM, &pN, &pK, &pG, &pR, &pepi};
  return launch(c, name, dim3(gx, ksplit), dim3(threads), args);
}

// M <= 2: the fused kernel (activation prep in LDS, whole records per lane,
// K split across the waves of a block; a cross-block split only when one
// block's 64/128 groups do not cover K).
int qgemv1_chunk(Ctx* c, Fmt fmt, const float* a, const void* B, const void* D, float* out, uint32_t M,
                 uint32_t N, uint32_t K, uint32_t G, const Epi& ep) {
  const char* tag = fmt_tag(fmt);
  // block K coverage (groups): the smallest variant that covers K in one
  // block, else 128 with a cross-block split
  uint32_t kb = G <= 64 ? 64 : (G <= 96 ? 96 : (G <= 128 ? 128 : (G <= 288 ? 288 : 128)));
  uint32_t threads = kb == 64 ? 256 : 512;
  // plain single-row matmuls with 288 < G <= 448 and ~one 16-column tile
  // per CU: 16 waves x 7 steps cover K in one block, no split-K finish
  // (N = 4096, K = 14336: Q4S 13.2 -> 10.9 us, Q4_0 tiles 12.2 -> 9.4 us;
  // at N = 2048 / 1024 the 4-way split over more workgroups stays faster)
  const uint32_t nt16 = (N + 15) / 16;
  const bool k448 = M == 1 && (fmt == FQ4S || fmt == FQ40 || fmt == FQ40T) && G > 288 && G <= 448 &&
                    nt16 >= 224 && nt16 <= 320 && !ep.gamma && !ep.resid && ep.mode == 0;
  if (k448) kb = 448, threads = 1024;
  // wide outputs (N >= 8192): two column tiles per wave halve the workgroup
  // count, and both the c2 and the _pls variants read each step's A operands
  // just before its MFMAs, which frees 48 VGPRs for more resident workgroups
  // (N = 14336: Q4S 10.3 -> 9.5 us, Q8 14.6 -> 13.7 us; Q4_0 tiles keep one
  // tile per wave: 8.7 -> 8.3 us)
  const bool wide = M == 1 && (kb == 96 || kb == 128) && N >= 8192;
  const bool q40 = fmt == FQ40 || fmt == FQ40T;
  bool c2 = wide && !q40;
  uint32_t gx = c2 ? (N + 31) / 32 : (N + 15) / 16;
  uint32_t ksplit = (G + kb - 1) / kb;
  if (ksplit > 1) {
    if (ensure(c, (void**)&c->ws, &c->ws_bytes, (size_t)ksplit * M * N * sizeof(float))) return -1;
    if (ensure_counters(c, gx)) return -1;
  }
  // plain single-row matmuls (no norm, plain store, one block per column
  // tile): the variants without the code of the other paths
  const bool plain = M == 1 && ksplit == 1 && !ep.gamma && !ep.resid && ep.mode == 0;
  const bool pls = plain && wide && q40 && kb == 128;
  // plain Q8 matmuls whose 16-column record runs are whole and 16-byte
  // aligned read them as contiguous chunks (config 2: 13.7 -> ~12 us)
  const bool q8c = plain && fmt == FQ8 && M == 1 && N % (c2 ? 32 : 16) == 0 && ((uintptr_t)B & 15) == 0;
  char name[64];
  snprintf(name, sizeof name, "smith_qgemv1_%s_m%u_k%u%s%s%s", q8c ? "q8c" : tag, M, kb, c2 ? "_c2" : "",
           k448 ? "w16" : "", pls ? "_pls" : (plain ? "_pl" : ""));
  const float* pa = a;
  const void* pB = B;
  const void* pD = D;
  float* pC = out;
  float* pws = c->ws;
  uint32_t* pcnt = c->counters;
  uint32_t pM = M, pN = N, pK = K, pG = G;
  const float* pg = ep.gamma;
  float pe = ep.eps;
  const float* pR = ep.resid;
  uint32_t pepi = ep.mode;
  void* args[] = {&pa, &pB, &pD, &pC, &pws, &pcnt, &pM, &pN, &pK, &pG, &pg, &pe, &pR, &pepi};
  return launch(c, name, dim3(gx, ksplit), dim3(threads), args);
}

// M >= GEMM_MIN_M: f16 activations (RMSNorm fused into their conversion),
// weights dequantized to f16 in LDS, MFMA GEMM with f32 accumulation.
const uint32_t GEMM_MIN_M = 64;

int gemm(Ctx* c, Fmt fmt, const float* a, const void* B, const void* D, float* out, uint32_t M, uint32_t N,
         uint32_t K, const Epi& ep) {
  // A operand already written by the previous GEMM's fused reduce (same
  // source rows, norm and shape; only the permuted layout is written)
  const bool want_next = c->next_pending;
  c->next_pending = false;
  const bool pre = c->a16_src && c->a16_src == a && c->a16_gamma == ep.gamma &&
                   (!ep.gamma || c->a16_eps == ep.eps) && c->a16_M == M && c->a16_K == K &&
                   c->a16_bytes >= (size_t)M * K * 2;
  c->a16_src = nullptr;
  if (ensure(c, &c->a16, &c->a16_bytes, (size_t)M * K * 2)) return -1;
  // tile-plane formats (Q4_0 tiles, Q4_1, Q5_0, Q4_K, Q6_K) with K % 64 == 0:
  // the DMA-staged kernels (smith_gemm2_*),
  // whose A operand is in the permuted slot order.  (On Q4S records the f32
  // in-register dequantisation, repeated by the waves sharing a weight
  // fragment, made them slower at config-4 sizes: 487 vs 331 us.)
  static const bool gemm2_on = [] {
    const char* e = getenv("SMITH_GEMM2");
    return !(e && e[0] == '0');
  }();
  const bool g2 = gemm2_on && (fmt == FQ40T || fmt >= FQ41T) && K % 64 == 0;
  {
    const float* pa = a;
    const float* pg = ep.gamma;
    float pe = ep.eps;
    void* pd = c->a16;
    uint32_t pK = K;
    void* args[] = {&pa, &pg, &pe, &pd, &pK};
    // the DMA-staged kernels and the register-staged Q4S / Q4_0 ones take A
    // in the permuted slot order of their packed-f16 weight conversion
    const bool perm = g2 || fmt == FQ4S || fmt == FQ40 || fmt == FQ40T;
    if (!(pre && perm) && launch(c, perm ? "smith_gemm_prep_a_perm" : "smith_gemm_prep_a", dim3(M), dim3(256), args))
      return -1;
  }
  // tile choice: the biggest tile that still gives about one tile per CU
  // (bigger tiles carry more MFMA work per K stage to cover load latency);
  // small grids split K across workgroups (partials reduced after)
  auto ntiles = [&](uint32_t bm, uint32_t bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
  uint32_t bm = 128, bn = 64;
  if (ntiles(256, 256) >= 256) bm = 256, bn = 256;
  else if (ntiles(256, 128) >= 200) bm = 256, bn = 128;
  else if (ntiles(128, 128) >= 256) bm = 128, bn = 128;
  if (g2 && M <= 128) bn = ntiles(128, 128) >= 128 ? 128 : 64;
  if (g2 && bm == 256 && bn == 256) bn = 128;  // 256x256 spills registers on the high-bit formats
  // M >= 256 on the register-staged kernel: 256x256 tiles (one 1024-thread
  // workgroup per CU) and enough K splits to fill one wave of workgroups,
  // each split at least 8 stages -- measured best at config 4 (M = 512:
  // 123 -> 114 us at K = 4096, 191 -> 110 us at K = 14336; M = 2048,
  // K = 14336: 411 -> 359 us; M = 2048, K = 4096 unchanged)
  const bool big = !g2 && M >= 256;
  if (big) bm = bn = 256;
  const uint32_t tiles = ntiles(bm, bn);
  const uint32_t S = (K + 63) / 64;
  uint32_t ks = 1;
  if (big) {
    ks = std::max<uint32_t>(1, std::min<uint32_t>(256 / tiles, S / 8));
  } else if (g2 && bm == 128 && tiles < 512) {
    // about 450 workgroups, at least 6 stages per split (measured at M = 128)
    ks = std::min<uint32_t>(std::max<uint32_t>(1, (448 + tiles / 2) / tiles), std::max<uint32_t>(1, S / 6));
  } else if (bm == 128 && bn == 64 && tiles < 512) {
    ks = std::min<uint32_t>((512 + tiles - 1) / tiles, std::max<uint32_t>(1, S / 8));
  }
  const uint32_t sps = (S + ks - 1) / ks;
  ks = (S + sps - 1) / sps;
  if (ks > 1 && ensure(c, (void**)&c->ws, &c->ws_bytes, (size_t)ks * M * N * sizeof(float))) return -1;
  const uint32_t threads = 64 * (bm / 64) * (bn / (bn >= 128 ? 64 : 32));
  char name[64];
  snprintf(name, sizeof name, "smith_gemm%s_%s_m%u_n%u", g2 ? "2" : "", fmt_tag(fmt), bm, bn);
  const void* pA = c->a16;
  const void* pB = B;
  const void* pD = D;
  float* pC = out;
  uint32_t pM = M, pN = N, pK = K, pepi = ep.mode, psps = sps;
  const float* pR = ep.resid;
  float* pws = c->ws;
  void* args[] = {&pA, &pB, &pD, &pC, &pM, &pN, &pK, &pR, &pepi, &pws, &psps};
  if (launch(c, name, dim3(tiles, ks), dim3(threads), args)) return -1;
  if (ks == 1) return 0;
  const float* cws = c->ws;
  uint32_t pks = ks;
  const uint32_t Kn = ep.mode == 2 ? N / 2 : N;
  if (want_next && (ep.mode == 1 || ep.mode == 2) && Kn % 8 == 0 && (!c->next_gamma || Kn <= 16384) &&
      ((uintptr_t)out & 15) == 0 &&
      (ep.mode != 1 || ((uintptr_t)ep.resid & 15) == 0) && (!c->next_gamma || ((uintptr_t)c->next_gamma & 15) == 0)) {
    // the reduce also writes the rows as the next GEMM's (permuted) A operand
    // into the f16 scratch, whose GEMM has finished reading it by then
    if (ensure(c, &c->a16, &c->a16_bytes, (size_t)M * Kn * 2)) return -1;
    const float* pg = c->next_gamma;
    float pe = c->next_eps;
    void* pa = c->a16;
    if (pg) {
      void* fargs[] = {&cws, &pks, &pC, &pM, &pN, &pR, &pepi, &pg, &pe, &pa};
      if (launch(c, "smith_gemm_reduce_prep", dim3(M), dim3(512), fargs)) return -1;
    } else {
      void* fargs[] = {&cws, &pks, &pC, &pM, &pN, &pR, &pepi, &pa};
      const uint64_t chunks = (uint64_t)M * (Kn / 8);
      if (launch(c, "smith_gemm_reduce_perm", dim3((unsigned)((chunks + 255) / 256)), dim3(256), fargs)) return -1;
    }
    c->a16_src = out;
    c->a16_gamma = c->next_gamma;
    c->a16_eps = c->next_eps;
    c->a16_M = M;
    c->a16_K = Kn;
    return 0;
  }
  void* rargs[] = {&cws, &pks, &pC, &pM, &pN, &pR, &pepi};
  const size_t per = (size_t)M * N % 4 == 0 ? (size_t)M * N / 4 : (size_t)M * N / (ep.mode == 2 ? 2 : 1);
  return launch(c, "smith_gemm_reduce", dim3((unsigned)std::min<size_t>((per + 255) / 256, 65536)), dim3(256), rargs);
}

int qmatmul(Ctx* c, Fmt fmt, const float* a, const void* B, const void* D, float* out, uint32_t M,
            uint32_t N, uint32_t K, uint32_t G, const Epi& ep = Epi()) {
  if (set_device(c)) return -1;
  if (M == 0 || N == 0) return 0;
  if (ep.mode == 2 && N % 2) return fail(c, "smith: SwiGLU epilogue needs an even column count (got %u)", N);
  if (M >= GEMM_MIN_M && K % 32 == 0) return gemm(c, fmt, a, B, D, out, M, N, K, ep);
  c->next_pending = false;  // the GEMV path has no K-split reduce to fuse
  c->a16_src = nullptr;
  const uint32_t nout = ep.mode == 2 ? N / 2 : N;
  for (uint32_t m0 = 0; m0 < M; m0 += 32) {
    uint32_t mc = std::min<uint32_t>(32, M - m0);
    const float* am = a + (size_t)m0 * K;
    float* om = out + (size_t)m0 * nout;
    Epi e = ep;
    if (e.resid) e.resid += (size_t)m0 * N;
    // SMITH_QGEMV=3 / 4 / 5 forces one of the M > 2 paths (comparisons)
    static const int vq = [] {
      const char* e = getenv("SMITH_QGEMV");
      return e ? atoi(e) : 0;
    }();
    // the one-launch kernels read the activations in 32-element groups
    // (K % 32 != 0 prepares them once, smith_qprep_*, for smith_qgemv3_*).
    // At 32 rows the one-launch kernel also wins on the wide shapes once its
    // 64-column blocks fit two per CU (14336 x 4096 Q4S: 27.0 us for prep +
    // qgemv3 -> 23.8 us; 4096 x 14336: 29.4 -> 27.4 us)
    const bool v3 = K % 32 != 0 || vq == 3;
    const bool v5 = !v3 && vq != 4;
    int rc = mc <= 2 ? qgemv1_chunk(c, fmt, am, B, D, om, mc, N, K, G, e)
                     : (v3 ? qgemv3_chunk(c, fmt, am, B, D, om, mc, N, K, G, e)
                           : (v5 ? qgemv5_chunk(c, fmt, am, B, D, om, mc, N, K, G, e)
                                 : qgemv4_chunk(c, fmt, am, B, D, om, mc, N, K, G, e)));
    if (rc) return -1;
  }
  return 0;
}

struct Slot {
  bool is_buf = false;
  void* ptr = nullptr;
  std::vector<uint8_t> bytes;
};

}  // namespace

struct SmithEncoder {
  Ctx* ctx;
  Pipeline* pipe = nullptr;
  std::map<uint32_t, Slot> slots;
  uint64_t shmem = 0;
  bool timed_started = false;
  hipEvent_t ev0 = nullptr;
  double submit_s = 0;
  bool failed = false;
};

// Static device scratch of smith_matmul_q4_noalloc (for callers that cannot
// allocate: code under HIP graph capture, serving loops, harnesses that
// forbid hipMalloc).  Each GPU the library runs on holds its own copy until
// the process ends.  Host code never passes `scratch` itself to a kernel (in
// host code the name is a host-side stand-in, not a device address): the
// device address comes from hipGetSymbolAddress, once per device at set-up,
// into g_scratch_dev[device].
//   [0, 64 KiB)            split-K counters (16384 x u32; zero at load and
//                          after every launch: each kernel's last workgroup
//                          resets the counters it used)
//   [64 KiB, +4 MiB)       activation fragments (M > 8 GEMV prep; f16 A of
//                          the M >= 64 GEMM)
//   [4 MiB + 64 KiB, 32 MiB)  split-K partials
constexpr size_t NOALLOC_BYTES = 32u << 20;
constexpr size_t NOALLOC_CNT_BYTES = 64u << 10;
constexpr size_t NOALLOC_PREP_BYTES = 4u << 20;
static __device__ __align__(256) uint8_t scratch[NOALLOC_BYTES];
constexpr int NOALLOC_MAX_DEVICES = 64;
static void* g_scratch_dev[NOALLOC_MAX_DEVICES];
// set while a host thread enqueues work on that device's static scratch: a
// second thread's call fails instead of sharing the counters (work of two
// streams that overlaps on the GPU after enqueueing is not detected)
static std::atomic<bool> g_scratch_busy[NOALLOC_MAX_DEVICES];

// Once per device, with that device current: the device address of its copy
// of `scratch`, and its counter region cleared (outside any capture).
static int noalloc_setup(Ctx* c) {
  if (c->device < 0 || c->device >= NOALLOC_MAX_DEVICES)
    return fail(c, "smith: device %d beyond the static scratch table", c->device);
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_scratch_dev[c->device]) return 0;
  void* ptr = nullptr;
  HIPCHK(c, hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
  HIPCHK(c, hipMemset(ptr, 0, NOALLOC_CNT_BYTES));
  HIPCHK(c, hipDeviceSynchronize());
  g_scratch_dev[c->device] = ptr;
  return 0;
}

extern "C" {

// ---------------- lifecycle ----------------
void* smith_init(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return nullptr;
  Ctx* c = new Ctx();
  if (hipSetDevice(0) != hipSuccess || hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess ||
      hipEventCreate(&c->t0) != hipSuccess || hipEventCreate(&c->t1) != hipSuccess ||
      hipHostMalloc((void**)&c->pos_err_host, 256, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess ||
      hipHostGetDevicePointer((void**)&c->pos_err_dev, c->pos_err_host, 0) != hipSuccess) {
    if (c->pos_err_host) (void)hipHostFree(c->pos_err_host);
    delete c;
    return nullptr;
  }
  memset(c->pos_err_host, 0, 256);
  if (noalloc_setup(c)) {
    (void)hipHostFree(c->pos_err_host);
    delete c;
    return nullptr;
  }
  return c;
}

void smith_destroy(void* ctx) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return;
  (void)hipSetDevice(c->device);
  (void)hipStreamSynchronize(c->stream);
  {
    std::lock_guard<std::mutex> lk(g_mu);
    for (auto it = g_bufs.begin(); it != g_bufs.end();) {
      if (it->second.ctx == c) {
        (void)hipFree(it->first);
        it = g_bufs.erase(it);
      } else {
        ++it;
      }
    }
  }
  if (c->prep) (void)hipFree(c->prep);
  if (c->normbuf) (void)hipFree(c->normbuf);
  if (c->a16) (void)hipFree(c->a16);
  if (c->att_ws) (void)hipFree(c->att_ws);
  if (c->att_cnt) (void)hipFree(c->att_cnt);
  if (c->ws) (void)hipFree(c->ws);
  if (c->counters) (void)hipFree(c->counters);
  if (c->amx) (void)hipFree(c->amx);
  for (void* r : c->retired) (void)hipFree(r);
  for (auto& r : c->recs) {
    (void)hipEventDestroy(r.a);
    (void)hipEventDestroy(r.b);
  }
  for (hipEvent_t e : c->event_pool) (void)hipEventDestroy(e);
  for (Pipeline* p : c->pipelines) delete p;
  for (Library* l : c->libs) {
    (void)hipModuleUnload(l->mod);
    delete l;
  }
  (void)hipEventDestroy(c->t0);
  (void)hipEventDestroy(c->t1);
  (void)hipStreamDestroy(c->stream);
  if (c->pos_err_host) (void)hipHostFree(c->pos_err_host);
  delete c;
}

const char* smith_last_error(void* ctx) {
  Ctx* c = (Ctx*)ctx;
  return c ? c->err.c_str() : "smith: null context";
}

void smith_free(void* p) { free(p); }

// ---------------- device info ----------------
char* smith_device_name(void* ctx) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return nullptr;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, c->device) != hipSuccess) return nullptr;
  std::string s = std::string(prop.name) + " (" + prop.gcnArchName + ")";
  return strdup(s.c_str());
}

uint64_t smith_max_threadgroup_memory(void* ctx) {
  Ctx* c = (Ctx*)ctx;
  hipDeviceProp_t prop;
  if (!c || hipGetDeviceProperties(&prop, c->device) != hipSuccess) return 0;
  return prop.sharedMemPerBlock;
}

uint64_t smith_max_threads_per_threadgroup(void* ctx) {
  Ctx* c = (Ctx*)ctx;
  hipDeviceProp_t prop;
  if (!c || hipGetDeviceProperties(&prop, c->device) != hipSuccess) return 0;
  return prop.maxThreadsPerBlock;
}

// ---------------- buffers ----------------
void* smith_alloc(void* ctx, uint64_t bytes, uint32_t mode) {
  (void)mode;
  Ctx* c = (Ctx*)ctx;
  if (!c) return nullptr;
  if (set_device(c)) return nullptr;
  // round up and pad so vector loads of a buffer's last record never leave
  // the allocation
  uint64_t sz = ((bytes ? bytes : 1) + 255) / 256 * 256 + 256;
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, sz);
  if (e != hipSuccess) {
    fail(c, "smith: failed to allocate %llu bytes: %s", (unsigned long long)bytes, hipGetErrorString(e));
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(g_mu);
  g_bufs[p] = BufInfo{c, bytes};
  c->allocated += bytes;
  return p;
}

void* smith_buffer_contents(void* buffer) {
  (void)buffer;
  return nullptr;
}

uint64_t smith_buffer_length(void* buffer) {
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_bufs.find(buffer);
  return it == g_bufs.end() ? 0 : it->second.bytes;
}

int64_t smith_buffer_retain_count(void* buffer) {
  std::lock_guard<std::mutex> lk(g_mu);
  return g_bufs.count(buffer) ? 1 : 0;
}

void smith_release_buffer(void* buffer) {
  Ctx* c = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_bufs.find(buffer);
    if (it == g_bufs.end()) return;
    c = it->second.ctx;
    c->allocated -= it->second.bytes;
    g_bufs.erase(it);
  }
  // work already enqueued may still read the buffer
  (void)hipSetDevice(c->device);
  (void)hipStreamSynchronize(c->stream);
  (void)hipFree(buffer);
}

uint64_t smith_allocated_size(void* ctx) {
  Ctx* c = (Ctx*)ctx;
  return c ? c->allocated : 0;
}

int64_t smith_test_release(void* ctx) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  // bytes freed by the release (gpu_bridge.m: after_alloc - after_release)
  void* p = smith_alloc(ctx, 1 << 20, SMITH_SHARED);
  if (!p) return -1;
  uint64_t mid = c->allocated;
  smith_release_buffer(p);
  return (int64_t)(mid - c->allocated);
}

int64_t smith_test_release_after_use(void* ctx) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  void* p = smith_alloc(ctx, 1 << 20, SMITH_SHARED);
  if (!p) return -1;
  if (hipMemsetAsync(p, 0, 1 << 20, c->stream) != hipSuccess || hipStreamSynchronize(c->stream) != hipSuccess) {
    smith_release_buffer(p);
    return -1;
  }
  uint64_t mid = c->allocated;
  smith_release_buffer(p);
  return (int64_t)(mid - c->allocated);
}

int smith_copy_h2d(void* ctx, void* dst, uint64_t off, const void* src, uint64_t bytes) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  drop_hints(c);
  if (set_device(c)) return -1;
  if (!bytes) return 0;
  HIPCHK(c, hipMemcpyAsync((char*)dst + off, src, bytes, hipMemcpyHostToDevice, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return 0;
}

int smith_copy_d2h(void* ctx, void* dst, const void* src, uint64_t off, uint64_t bytes) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (set_device(c)) return -1;
  if (!bytes) return 0;
  HIPCHK(c, hipMemcpyAsync(dst, (const char*)src + off, bytes, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  if (check_pos_err(c)) return -1;
  return 0;
}

int smith_copy_d2d(void* ctx, void* dst, uint64_t doff, const void* src, uint64_t soff, uint64_t bytes) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  drop_hints(c);
  if (set_device(c)) return -1;
  if (!bytes) return 0;
  HIPCHK(c, hipMemcpyAsync((char*)dst + doff, (const char*)src + soff, bytes, hipMemcpyDeviceToDevice, c->stream));
  return 0;
}

int smith_copy_2d(void* ctx, void* dst, uint64_t dpitch, const void* src, uint64_t spitch, uint64_t width,
                  uint64_t rows) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (!rows || !width) return 0;
  if (!dst || !src || width > dpitch || width > spitch) return fail(c, "smith_copy_2d: bad pitches or buffers");
  drop_hints(c);
  if (set_device(c)) return -1;
  HIPCHK(c, hipMemcpy2DAsync(dst, dpitch, src, spitch, width, rows, hipMemcpyDeviceToDevice, c->stream));
  return 0;
}

int smith_fill_zero(void* ctx, void* buffer, uint64_t bytes) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (set_device(c)) return -1;
  if (!bytes) return 0;
  if (bytes % 4) return fail(c, "smith_fill_zero: byte count %llu is not a multiple of 4", (unsigned long long)bytes);
  uint64_t n = bytes / 4;
  void* p = buffer;
  void* args[] = {&p, &n};
  uint64_t blocks = std::min<uint64_t>((n + 255) / 256, 65536);
  return launch(c, "smith_zero_u32", dim3((unsigned)blocks), dim3(256), args);
}

int smith_prep_next(void* ctx, const float* gamma, float eps) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  c->next_pending = true;
  c->next_gamma = gamma;
  c->next_eps = eps;
  return 0;
}

int smith_sync(void* ctx) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (set_device(c)) return -1;
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return check_pos_err(c);
}

// ---------------- code objects ----------------
void* smith_load_library(void* ctx, const char* path) {
  Ctx* c = (Ctx*)ctx;
  if (!c || !path) return nullptr;
  if (set_device(c)) return nullptr;
  hipModule_t m;
  hipError_t e = hipModuleLoad(&m, path);
  if (e != hipSuccess) {
    fail(c, "smith: failed to load code object at %s: %s", path, hipGetErrorString(e));
    return nullptr;
  }
  Library* lib = new Library();
  lib->mod = m;
  c->libs.push_back(lib);
  if (!c->ops) c->ops = lib;
  return lib;
}

void* smith_compile_source(void* ctx, const char* source, char** error_out) {
  Ctx* c = (Ctx*)ctx;
  if (error_out) *error_out = nullptr;
  if (!c || !source) return nullptr;
  if (set_device(c)) return nullptr;
  hiprtcProgram prog;
  if (hiprtcCreateProgram(&prog, source, "smith_rtc.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS) {
    if (error_out) *error_out = strdup("hiprtcCreateProgram failed");
    return nullptr;
  }
  // no packed-f32 VALU instructions, as for the library's own code objects
  const char* opts[] = {"--offload-arch=gfx950", "-O3", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
  hiprtcResult r = hiprtcCompileProgram(prog, 6, opts);
  if (r != HIPRTC_SUCCESS) {
    size_t n = 0;
    hiprtcGetProgramLogSize(prog, &n);
    std::string log(n + 1, '\0');
    if (n) hiprtcGetProgramLog(prog, &log[0]);
    if (error_out) *error_out = strdup(log.c_str());
    fail(c, "smith: hipRTC compile failed");
    hiprtcDestroyProgram(&prog);
    return nullptr;
  }
  size_t code_sz = 0;
  hiprtcGetCodeSize(prog, &code_sz);
  std::vector<char> code(code_sz);
  hiprtcGetCode(prog, code.data());
  hiprtcDestroyProgram(&prog);
  hipModule_t m;
  hipError_t e = hipModuleLoadData(&m, code.data());
  if (e != hipSuccess) {
    if (error_out) *error_out = strdup(hipGetErrorString(e));
    return nullptr;
  }
  Library* lib = new Library();
  lib->mod = m;
  c->libs.push_back(lib);
  return lib;
}

void* smith_create_pipeline(void* ctx, void* library, const char* fn_name) {
  Ctx* c = (Ctx*)ctx;
  if (!c || !library || !fn_name) return nullptr;
  hipFunction_t f;
  if (lookup(c, (Library*)library, fn_name, &f)) return nullptr;
  Pipeline* p = new Pipeline{f, fn_name};
  c->pipelines.push_back(p);
  return p;
}

// ---------------- encoded dispatch ----------------
SmithEncoder* smith_begin(void* ctx) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return nullptr;
  SmithEncoder* e = new SmithEncoder();
  e->ctx = c;
  return e;
}

void smith_set_buffer(SmithEncoder* enc, void* buffer, uint32_t index) {
  if (!enc) return;
  Slot& s = enc->slots[index];
  s.is_buf = true;
  s.ptr = buffer;
  s.bytes.clear();
}

void smith_set_bytes(SmithEncoder* enc, const void* data, uint32_t length, uint32_t index) {
  if (!enc) return;
  Slot& s = enc->slots[index];
  s.is_buf = false;
  s.ptr = nullptr;
  s.bytes.assign((const uint8_t*)data, (const uint8_t*)data + length);
}

void smith_set_pipeline(SmithEncoder* enc, void* pipeline) {
  if (enc) enc->pipe = (Pipeline*)pipeline;
}

void smith_set_threadgroup_memory(SmithEncoder* enc, uint64_t length, uint32_t index) {
  (void)index;  // HIP has one dynamic LDS block per workgroup: lengths add up
  if (enc) enc->shmem += length;
}

void smith_dispatch(SmithEncoder* enc, uint64_t gx, uint64_t gy, uint64_t gz, uint64_t bx, uint64_t by,
                    uint64_t bz) {
  if (!enc) return;
  Ctx* c = enc->ctx;
  if (!enc->pipe) {
    fail(c, "smith_dispatch: no pipeline set");
    enc->failed = true;
    return;
  }
  if (!bx) bx = 1;
  if (!by) by = 1;
  if (!bz) bz = 1;
  if (bx * by * bz > 1024) {
    fail(c, "smith_dispatch: workgroup of %llu threads exceeds 1024", (unsigned long long)(bx * by * bz));
    enc->failed = true;
    return;
  }
  if (!gx || !gy || !gz) return;  // empty grid: nothing to run
  std::vector<uint8_t> blob;
  for (auto& kv : enc->slots) {
    const Slot& s = kv.second;
    size_t align = s.is_buf ? 8 : (s.bytes.size() % 8 == 0 ? 8 : 4);
    size_t off = (blob.size() + align - 1) / align * align;
    if (s.is_buf) {
      blob.resize(off + 8);
      memcpy(blob.data() + off, &s.ptr, 8);
    } else {
      blob.resize(off + s.bytes.size());
      memcpy(blob.data() + off, s.bytes.data(), s.bytes.size());
    }
  }
  size_t blob_sz = blob.size();
  void* extra[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, blob.data(), HIP_LAUNCH_PARAM_BUFFER_SIZE, &blob_sz,
                   HIP_LAUNCH_PARAM_END};
  if (set_device(c)) {
    enc->failed = true;
    return;
  }
  if (!enc->timed_started) {
    enc->timed_started = true;
    enc->submit_s = now_s();
    if (hipEventCreate(&enc->ev0) == hipSuccess) (void)hipEventRecord(enc->ev0, c->stream);
  }
  drop_hints(c);
  hipError_t e = hipModuleLaunchKernel(enc->pipe->fn, (unsigned)((gx + bx - 1) / bx), (unsigned)((gy + by - 1) / by),
                                       (unsigned)((gz + bz - 1) / bz), (unsigned)bx, (unsigned)by, (unsigned)bz,
                                       (unsigned)enc->shmem, c->stream, nullptr, extra);
  if (e != hipSuccess) {
    fail(c, "smith_dispatch(%s): %s", enc->pipe->name.c_str(), hipGetErrorString(e));
    enc->failed = true;
  }
}

void smith_end_sync(SmithEncoder* enc) {
  if (!enc) return;
  (void)hipSetDevice(enc->ctx->device);
  // void in the reference too: a failure of the enqueued work is left in
  // smith_last_error
  const hipError_t e = hipStreamSynchronize(enc->ctx->stream);
  if (e != hipSuccess) fail(enc->ctx, "smith_end_sync: %s", hipGetErrorString(e));
  if (enc->ev0) (void)hipEventDestroy(enc->ev0);
  delete enc;
}

void* smith_end_async(SmithEncoder* enc) {
  if (!enc) return nullptr;
  hipEvent_t ev;
  void* token = nullptr;
  if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) == hipSuccess) {
    (void)hipEventRecord(ev, enc->ctx->stream);
    token = (void*)ev;
  }
  if (enc->ev0) (void)hipEventDestroy(enc->ev0);
  delete enc;
  return token;
}

void smith_wait(void* token) {
  if (!token) return;
  hipEvent_t ev = (hipEvent_t)token;
  (void)hipEventSynchronize(ev);
  (void)hipEventDestroy(ev);
}

SmithTiming* smith_end_timed(SmithEncoder* enc) {
  if (!enc) return nullptr;
  Ctx* c = enc->ctx;
  SmithTiming* t = (SmithTiming*)calloc(1, sizeof(SmithTiming));
  (void)hipSetDevice(c->device);
  hipEvent_t ev1 = nullptr;
  if (enc->ev0 && hipEventCreate(&ev1) == hipSuccess) {
    (void)hipEventRecord(ev1, c->stream);
    const hipError_t e = hipEventSynchronize(ev1);
    if (e != hipSuccess) fail(c, "smith_end_timed: %s", hipGetErrorString(e));
    float ms = 0.f;
    (void)hipEventElapsedTime(&ms, enc->ev0, ev1);
    t->gpu_ms = ms;
    (void)hipEventDestroy(ev1);
  } else {
    const hipError_t e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) fail(c, "smith_end_timed: %s", hipGetErrorString(e));
  }
  t->gpu_end = now_s();
  t->gpu_start = enc->timed_started ? enc->submit_s : t->gpu_end;
  if (enc->ev0) (void)hipEventDestroy(enc->ev0);
  delete enc;
  return t;
}

void smith_dispatch_sync(void* ctx, void* pipeline, void** buffers, uint32_t* indices, uint32_t count,
                         const void* params, uint32_t params_length, uint32_t params_index, uint64_t gx,
                         uint64_t gy, uint64_t gz, uint64_t bx, uint64_t by, uint64_t bz) {
  SmithEncoder* e = smith_begin(ctx);
  if (!e) return;
  smith_set_pipeline(e, pipeline);
  for (uint32_t i = 0; i < count; i++) smith_set_buffer(e, buffers[i], indices[i]);
  if (params && params_length) smith_set_bytes(e, params, params_length, params_index);
  smith_dispatch(e, gx, gy, gz, bx, by, bz);
  smith_end_sync(e);
}

// ---------------- op-level entry points ----------------
int smith_quantize_q4(void* ctx, const float* w, void* out, uint32_t K, uint32_t N) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (set_device(c)) return -1;
  uint64_t total = (uint64_t)((K + 31) / 32) * N;
  if (!total) return 0;
  uint32_t pK = K, pN = N;
  void* args[] = {&w, &out, &pK, &pN};
  return launch(c, "smith_quantize_q4s", dim3((unsigned)std::min<uint64_t>((total + 255) / 256, 1 << 20)),
                dim3(256), args);
}

int smith_quantize_q8(void* ctx, const float* w, void* out, uint32_t K, uint32_t N) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (set_device(c)) return -1;
  uint64_t total = (uint64_t)((K + 31) / 32) * N;
  if (!total) return 0;
  uint32_t pK = K, pN = N;
  void* args[] = {&w, &out, &pK, &pN};
  return launch(c, "smith_quantize_q8", dim3((unsigned)std::min<uint64_t>((total + 255) / 256, 1 << 20)),
                dim3(256), args);
}

int smith_quantize_q4_0(void* ctx, const float* x, void* out, uint32_t rows, uint32_t cols) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (cols % 32) return fail(c, "smith_quantize_q4_0: cols %u is not a multiple of 32", cols);
  if (set_device(c)) return -1;
  uint64_t total = (uint64_t)rows * (cols / 32);
  if (!total) return 0;
  uint32_t pr = rows, pc = cols;
  void* args[] = {&x, &out, &pr, &pc};
  return launch(c, "smith_quantize_q4_0_rows", dim3((unsigned)std::min<uint64_t>((total + 255) / 256, 1 << 20)),
                dim3(256), args);
}

int smith_repack_q4_0(void* ctx, const void* blocks, void* nib, void* d, uint32_t N, uint32_t K) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (K % 32) return fail(c, "smith_repack_q4_0: K %u is not a multiple of 32", K);
  if (set_device(c)) return -1;
  uint32_t G = K / 32;
  uint64_t total = (uint64_t)N * G;
  if (!total) return 0;
  uint32_t pN = N, pG = G, po = 0, ps = 1, pt = N;
  void* args[] = {&blocks, &nib, &d, &pN, &pG, &po, &ps, &pt};
  return launch(c, "smith_repack_q4_0_cols", dim3((unsigned)std::min<uint64_t>((total + 255) / 256, 1 << 20)),
                dim3(256), args);
}

int smith_matmul_q4(void* ctx, const float* a, const void* wq, float* out, uint32_t M, uint32_t N, uint32_t K,
                    uint32_t groups) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (groups != (K + 31) / 32)
    return fail(c, "matmulQ4: groups %u does not match ceil(K/32) for K=%u", groups, K);
  return qmatmul(c, FQ4S, a, wq, nullptr, out, M, N, K, groups);
}

int smith_matmul_q4_noalloc(void* ctx, const float* a, const void* wq, float* out, uint32_t M, uint32_t N,
                            uint32_t K, uint32_t groups) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (groups != (K + 31) / 32)
    return fail(c, "matmulQ4: groups %u does not match ceil(K/32) for K=%u", groups, K);
  if (set_device(c)) return -1;
  uint8_t* base = (uint8_t*)g_scratch_dev[c->device];
  if (!base) return fail(c, "smith_matmul_q4_noalloc: static scratch not set up on device %d", c->device);
  // run the allocating entry point's kernels on the static regions: every
  // ensure() below finds its region big enough or fails (no_alloc set)
  struct Saved {
    void* prep; size_t prep_bytes; void* a16; size_t a16_bytes; float* ws; size_t ws_bytes;
    uint32_t* counters; size_t counters_n;
  } sv = {c->prep, c->prep_bytes, c->a16, c->a16_bytes, c->ws, c->ws_bytes, c->counters, c->counters_n};
  c->counters = (uint32_t*)base;
  c->counters_n = NOALLOC_CNT_BYTES / sizeof(uint32_t);
  c->prep = c->a16 = base + NOALLOC_CNT_BYTES;
  c->prep_bytes = c->a16_bytes = NOALLOC_PREP_BYTES;
  c->ws = (float*)(base + NOALLOC_CNT_BYTES + NOALLOC_PREP_BYTES);
  c->ws_bytes = NOALLOC_BYTES - NOALLOC_CNT_BYTES - NOALLOC_PREP_BYTES;
  if (g_scratch_busy[c->device].exchange(true))
    return fail(c, "smith_matmul_q4_noalloc: another call is enqueueing on device %d's static scratch", c->device);
  // the context's prepared-operand hint names its own f16 buffer, not the
  // static region: dropped before and after
  drop_hints(c);
  c->no_alloc = "smith_matmul_q4_noalloc";
  const int rc = qmatmul(c, FQ4S, a, wq, nullptr, out, M, N, K, groups);
  c->no_alloc = nullptr;
  drop_hints(c);
  g_scratch_busy[c->device].store(false);
  c->prep = sv.prep, c->prep_bytes = sv.prep_bytes, c->a16 = sv.a16, c->a16_bytes = sv.a16_bytes;
  c->ws = sv.ws, c->ws_bytes = sv.ws_bytes, c->counters = sv.counters, c->counters_n = sv.counters_n;
  return rc;
}

int smith_matmul_q8(void* ctx, const float* a, const void* wq, float* out, uint32_t M, uint32_t N, uint32_t K,
                    uint32_t groups) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (groups != (K + 31) / 32)
    return fail(c, "matmulQ8: groups %u does not match ceil(K/32) for K=%u", groups, K);
  return qmatmul(c, FQ8, a, wq, nullptr, out, M, N, K, groups);
}

int smith_matmul_q4_0(void* ctx, const float* a, const void* nib, const void* d, float* out, uint32_t M,
                      uint32_t N, uint32_t K) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (K % 32) return fail(c, "smith_matmul_q4_0: K %u is not a multiple of 32", K);
  return qmatmul(c, FQ40, a, nib, d, out, M, N, K, K / 32);
}


// ---------------- GGUF decode path ----------------
int smith_repack_q4_0_into(void* ctx, const void* blocks, void* nib, void* d, uint32_t N, uint32_t K, uint32_t n_off,
                           uint32_t n_stride, uint32_t N_total) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (K % 32) return fail(c, "smith_repack_q4_0_into: K %u is not a multiple of 32", K);
  if ((uint64_t)n_off + (uint64_t)(N ? N - 1 : 0) * n_stride >= N_total && N)
    return fail(c, "smith_repack_q4_0_into: columns exceed N_total=%u", N_total);
  if (set_device(c)) return -1;
  uint32_t G = K / 32;
  uint64_t total = (uint64_t)N * G;
  if (!total) return 0;
  uint32_t pN = N, pG = G, po = n_off, ps = n_stride, pt = N_total;
  void* args[] = {&blocks, &nib, &d, &pN, &pG, &po, &ps, &pt};
  return launch(c, "smith_repack_q4_0_cols", dim3((unsigned)std::min<uint64_t>((total + 255) / 256, 1 << 20)),
                dim3(256), args);
}

int smith_repack_q8_0_into(void* ctx, const void* blocks, void* dst, uint32_t N, uint32_t K, uint32_t n_off,
                           uint32_t n_stride, uint32_t N_total) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (K % 32) return fail(c, "smith_repack_q8_0_into: K %u is not a multiple of 32", K);
  if ((uint64_t)n_off + (uint64_t)(N ? N - 1 : 0) * n_stride >= N_total && N)
    return fail(c, "smith_repack_q8_0_into: columns exceed N_total=%u", N_total);
  if (set_device(c)) return -1;
  uint32_t G = K / 32;
  uint64_t total = (uint64_t)N * G;
  if (!total) return 0;
  uint32_t pN = N, pG = G, po = n_off, ps = n_stride, pt = N_total;
  void* args[] = {&blocks, &dst, &pN, &pG, &po, &ps, &pt};
  return launch(c, "smith_repack_q8_0_cols", dim3((unsigned)std::min<uint64_t>((total + 255) / 256, 1 << 20)),
                dim3(256), args);
}

int smith_linear_q4_0(void* ctx, const float* x, const void* nib, const void* d, float* out, uint32_t M, uint32_t N,
                      uint32_t K, const float* norm_gamma, float eps, const float* resid, uint32_t epilogue) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (K % 32) return fail(c, "smith_linear_q4_0: K %u is not a multiple of 32", K);
  if (epilogue > 2) return fail(c, "smith_linear_q4_0: unknown epilogue %u", epilogue);
  if (epilogue == 1 && !resid) return fail(c, "smith_linear_q4_0: residual epilogue without a residual buffer");
  Epi e;
  e.gamma = norm_gamma;
  e.eps = eps;
  e.resid = epilogue == 1 ? resid : nullptr;
  e.mode = epilogue;
  return qmatmul(c, FQ40, x, nib, d, out, M, N, K, K / 32, e);
}

int smith_repack_q4_0_t_into(void* ctx, const void* blocks, void* nib, void* d, uint32_t N, uint32_t K,
                             uint32_t n_off, uint32_t n_stride, uint32_t N_total) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (K % 32) return fail(c, "smith_repack_q4_0_t_into: K %u is not a multiple of 32", K);
  if (N_total % 16) return fail(c, "smith_repack_q4_0_t_into: N_total %u is not a multiple of 16", N_total);
  if ((uint64_t)n_off + (uint64_t)(N ? N - 1 : 0) * n_stride >= N_total && N)
    return fail(c, "smith_repack_q4_0_t_into: columns exceed N_total=%u", N_total);
  if (set_device(c)) return -1;
  uint32_t G = K / 32;
  uint64_t total = (uint64_t)N * G;
  if (!total) return 0;
  uint32_t pN = N, pG = G, po = n_off, ps = n_stride;
  void* args[] = {&blocks, &nib, &d, &pN, &pG, &po, &ps};
  return launch(c, "smith_repack_q4_0_tiles", dim3((unsigned)std::min<uint64_t>((total + 255) / 256, 1 << 20)),
                dim3(256), args);
}

int smith_linear_q4_0_t(void* ctx, const float* x, const void* nib, const void* d, float* out, uint32_t M,
                        uint32_t N, uint32_t K, const float* norm_gamma, float eps, const float* resid,
                        uint32_t epilogue) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (K % 32) return fail(c, "smith_linear_q4_0_t: K %u is not a multiple of 32", K);
  if (N % 16) return fail(c, "smith_linear_q4_0_t: N %u is not a multiple of 16", N);
  if (epilogue > 2) return fail(c, "smith_linear_q4_0_t: unknown epilogue %u", epilogue);
  if (epilogue == 1 && !resid) return fail(c, "smith_linear_q4_0_t: residual epilogue without a residual buffer");
  Epi e;
  e.gamma = norm_gamma;
  e.eps = eps;
  e.resid = epilogue == 1 ? resid : nullptr;
  e.mode = epilogue;
  return qmatmul(c, FQ40T, x, nib, d, out, M, N, K, K / 32, e);
}

namespace {

// single-row GEMV on an act (smith_agemv_<fmt>_k*); B/D as the format takes
// them (Q4_0: nib and d planes; other tile formats: the plane buffer twice)
int act_gemv(Ctx* c, const char* fn, Fmt fmt, const void* act_in, int norm, float eps, const void* B, const void* D,
             float* out, uint32_t N, uint32_t K, const float* resid, uint32_t epilogue, void* act_out,
             const float* gamma_out) {
  if (!act_in) return fail(c, "%s: no input act", fn);
  if (K % 32 || !K) return fail(c, "%s: K %u is not a positive multiple of 32", fn, K);
  if (N % 16 || !N) return fail(c, "%s: N %u is not a positive multiple of 16", fn, N);
  if (epilogue > 2) return fail(c, "%s: unknown epilogue %u", fn, epilogue);
  if (epilogue == 1 && !resid) return fail(c, "%s: residual epilogue without a residual buffer", fn);
  const uint32_t nout = epilogue == 2 ? N / 2 : N;
  if (act_out && nout % 32) return fail(c, "%s: act output needs %u %% 32 == 0", fn, nout);
  if (set_device(c)) return -1;
  // smallest block K coverage that holds all K groups (no split), else 288
  // groups per block and a K split across blocks
  static const uint32_t kbs[] = {32, 48, 64, 72, 96, 128, 144, 192, 288};
  const uint32_t G = K / 32;
  uint32_t kb = 288;
  for (uint32_t v : kbs)
    if (v >= G) {
      kb = v;
      break;
    }
  const uint32_t ksplit = (G + kb - 1) / kb;
  const uint32_t threads = kb == 32 || kb == 48 || kb == 64 ? 256 : (kb == 72 ? 384 : (kb == 144 ? 768 : 512));
  const uint32_t gx = N / 16;
  if (ksplit > 1) {
    if (ensure(c, (void**)&c->ws, &c->ws_bytes, (size_t)ksplit * N * sizeof(float))) return -1;
    if (ensure_counters(c, gx)) return -1;
  }
  char name[64];
  snprintf(name, sizeof name, "smith_agemv_%s_k%u", fmt_tag(fmt), kb);
  // K = 9216 (down projection): 12 waves of 6 steps instead of 8 of 9;
  // 256 < N/16 <= 512 column tiles (the fused q|k|v at dim 3072): two tiles
  // per wave, so the blocks fit one round on the 256 CUs instead of leaving
  // 1.25 per CU (config-5 decode 948 -> 973-980 tok/s with both).  Q4_K also
  // on the wider gate|up (1152 column tiles: Q4_K_M decode 873 -> 882
  // tok/s; Q4_0 there measured 1010 -> 998, so it keeps one tile per wave)
  uint32_t gxx = gx, thr = threads;
  if (kb == 288) {
    // without a norm (the down projection): the variant that has no norm code
    strncat(name, norm ? "_w12" : "_w12_nn", sizeof name - strlen(name) - 1);
    thr = 768;
  } else if (kb == 96 && gx > 256 && gx % 2 == 0 && (gx <= 512 || fmt == FQ4KT)) {
    strncat(name, "_c2", sizeof name - strlen(name) - 1);
    gxx = gx / 2;
  }
  float* pws = c->ws;
  uint32_t* pcnt = c->counters;
  uint32_t pN = N, pK = K, pnorm = norm ? 1u : 0u, pepi = epilogue;
  const float* pR = epilogue == 1 ? resid : nullptr;
  void* args[] = {&act_in, &B, &D, &out, &pN, &pK, &pnorm, &eps, &pR, &pepi, &act_out, &gamma_out, &pws, &pcnt};
  return launch(c, name, dim3(gxx, ksplit), dim3(thr), args);
}

// o-projection on attention split partials (smith_agemv_att_<fmt>_k*)
int attn_gemv(Ctx* c, const char* fn, Fmt fmt, const float* parts, const int32_t* pos_ptr, uint32_t head_dim,
              const void* B, const void* D, float* out, uint32_t N, uint32_t K, const float* resid,
              uint32_t epilogue, void* act_out, const float* gamma_out) {
  if (!parts || !pos_ptr) return fail(c, "%s: no attention partials", fn);
  if (!head_dim || head_dim > 128 || head_dim % 32 || K % head_dim)
    return fail(c, "%s: head_dim %u unsupported for K %u", fn, head_dim, K);
  if (K % 32 || !K) return fail(c, "%s: K %u is not a positive multiple of 32", fn, K);
  if (N % 16 || !N) return fail(c, "%s: N %u is not a positive multiple of 16", fn, N);
  if (epilogue > 2) return fail(c, "%s: unknown epilogue %u", fn, epilogue);
  if (epilogue == 1 && !resid) return fail(c, "%s: residual epilogue without a residual buffer", fn);
  const uint32_t nout = epilogue == 2 ? N / 2 : N;
  if (act_out && nout % 32) return fail(c, "%s: act output needs %u %% 32 == 0", fn, nout);
  if (set_device(c)) return -1;
  static const uint32_t kbs[] = {64, 96, 128, 192};
  const uint32_t G = K / 32;
  uint32_t kb = 192;
  for (uint32_t v : kbs)
    if (v >= G) {
      kb = v;
      break;
    }
  const uint32_t ksplit = (G + kb - 1) / kb;
  const uint32_t threads = kb == 64 ? 256 : 512;
  const uint32_t gx = N / 16;
  if (ksplit > 1) {
    if (ensure(c, (void**)&c->ws, &c->ws_bytes, (size_t)ksplit * N * sizeof(float))) return -1;
    if (ensure_counters(c, gx)) return -1;
  }
  char name[64];
  snprintf(name, sizeof name, "smith_agemv_att_%s_k%u", fmt_tag(fmt), kb);
  float* pws = c->ws;
  uint32_t* pcnt = c->counters;
  uint32_t pN = N, pK = K, phd = head_dim, pepi = epilogue;
  const float* pR = epilogue == 1 ? resid : nullptr;
  void* args[] = {&parts, &pos_ptr, &phd, &B, &D, &out, &pN, &pK, &pR, &pepi, &act_out, &gamma_out, &pws, &pcnt};
  return launch(c, name, dim3(gx, ksplit), dim3(threads), args);
}

// GGML type -> tile format, with the shape rules of the tile planes
int tiles_fmt(Ctx* c, const char* fn, uint32_t type, uint32_t N, uint32_t K, Fmt* fmt) {
  const int f = gt_of_ggml((int)type);
  if (f < 0) return fail(c, "%s: GGML type %u has no tile layout (Q4_0, Q4_1, Q5_0, Q4_K, Q6_K)", fn, type);
  const uint32_t kq = gt_super(f) ? 256 : 32;
  if (!K || K % kq) return fail(c, "%s: K %u is not a positive multiple of %u for GGML type %u", fn, K, kq, type);
  if (!N || N % 16) return fail(c, "%s: N %u is not a positive multiple of 16", fn, N);
  *fmt = (Fmt)f;
  return 0;
}

// (B, D) kernel arguments of a tile-plane buffer
void tiles_bd(Fmt fmt, const void* planes, uint32_t N, uint32_t K, const void** B, const void** D) {
  *B = planes;
  *D = fmt == FQ40T ? (const void*)((const char*)planes + gt_planes(GT_Q40, N, K / 32).prm) : planes;
}

}  // namespace

int smith_linear_q4_0_t_act(void* ctx, const void* act_in, int norm, float eps, const void* nib, const void* d,
                            float* out, uint32_t N, uint32_t K, const float* resid, uint32_t epilogue,
                            void* act_out, const float* gamma_out) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  return act_gemv(c, "smith_linear_q4_0_t_act", FQ40T, act_in, norm, eps, nib, d, out, N, K, resid, epilogue,
                  act_out, gamma_out);
}

int smith_linear_q8(void* ctx, const float* x, const void* wq, float* out, uint32_t M, uint32_t N, uint32_t K,
                    const float* norm_gamma, float eps, const float* resid, uint32_t epilogue) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (K % 32) return fail(c, "smith_linear_q8: K %u is not a multiple of 32 (GGUF Q8_0 rows)", K);
  if (epilogue > 2) return fail(c, "smith_linear_q8: unknown epilogue %u", epilogue);
  if (epilogue == 1 && !resid) return fail(c, "smith_linear_q8: residual epilogue without a residual buffer");
  Epi e;
  e.gamma = norm_gamma;
  e.eps = eps;
  e.resid = epilogue == 1 ? resid : nullptr;
  e.mode = epilogue;
  return qmatmul(c, FQ8, x, wq, nullptr, out, M, N, K, (K + 31) / 32, e);
}

int smith_rmsnorm(void* ctx, const float* x, const float* gamma, float* out, uint32_t rows, uint32_t cols, float eps) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (set_device(c)) return -1;
  if (!rows || !cols) return 0;
  void* args[] = {&x, &gamma, &out, &rows, &cols, &eps};
  return launch(c, "smith_rmsnorm_rows", dim3(rows), dim3(256), args);
}

int smith_embed(void* ctx, const float* E, const int32_t* tokens, float* out, uint32_t rows, uint32_t dim,
                void* act_out, const float* gamma_out) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (act_out && (rows != 1 || dim % 32))
    return fail(c, "smith_embed: an act output needs one row and dim %% 32 == 0 (rows %u, dim %u)", rows, dim);
  if (set_device(c)) return -1;
  if (!rows) return 0;
  void* args[] = {&E, &tokens, &out, &rows, &dim, &act_out, &gamma_out};
  return launch(c, "smith_embed_rows", dim3(rows), dim3(256), args);
}

int smith_attention(void* ctx, const float* qkv, uint32_t ld, const int32_t* pos_ptr, uint32_t S, uint32_t n_heads,
                    uint32_t n_kv_heads, uint32_t head_dim, const float* rope_cos, const float* rope_sin,
                    uint32_t rope_len, float* kcache, float* vcache, uint32_t max_seq, float* out, void* act_out) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (act_out && (S != 1 || head_dim % 8 || (n_heads * head_dim) % 32))
    return fail(c, "smith_attention: an act output needs one row, head_dim %% 8 == 0 and heads*head_dim %% 32 == 0");
  if (!n_kv_heads || n_heads % n_kv_heads)
    return fail(c, "smith_attention: %u heads not a multiple of %u kv heads", n_heads, n_kv_heads);
  if (head_dim > 128 || head_dim % 4) return fail(c, "smith_attention: head_dim %u unsupported (<= 128, % 4)", head_dim);
  if (!rope_cos || !rope_sin || !kcache || !vcache || !qkv || !pos_ptr || !out)
    return fail(c, "smith_attention: null buffer");
  if (set_device(c)) return -1;
  const bool want_next = c->next_pending && !c->next_gamma;  // smith_prep_next: no norm before the output projection
  c->next_pending = false;
  c->a16_src = nullptr;
  if (!S) return 0;
  uint32_t* perr = c->pos_err_dev;
  if (S > 1 && head_dim % 16 == 0) {
    // prompt rows: rope + append every row's key/value, then flash attention
    // on the f32 matrix cores over the caches (16 query rows per workgroup,
    // its four waves splitting the keys)
    uint32_t Wq = n_heads * head_dim;
    void* aargs[] = {&qkv, &ld, &pos_ptr, &Wq, &n_kv_heads, &head_dim, &rope_cos, &rope_sin, &kcache, &vcache,
                     &max_seq, &rope_len, &perr};
    if (launch(c, "smith_kv_append", dim3(S), dim3(256), aargs)) return -1;
    // with the hint the rows are also written as the output projection's f16
    // operand (its GEMM then skips the activation prep)
    void* pa = nullptr;
    if (want_next && S >= GEMM_MIN_M && Wq % 32 == 0) {
      if (ensure(c, &c->a16, &c->a16_bytes, (size_t)S * Wq * 2)) return -1;
      pa = c->a16;
    }
    void* fargs[] = {&qkv, &ld, &pos_ptr, &S, &n_heads, &n_kv_heads, &rope_cos, &rope_sin,
                     &kcache, &vcache, &max_seq, &out, &rope_len, &perr, &pa};
    char name[48];
    snprintf(name, sizeof name, "smith_attention_prefill_hd%u", head_dim / 16);
    if (launch(c, name, dim3(n_heads, (S + 15) / 16), dim3(256), fargs)) return -1;
    if (pa) {
      c->a16_src = out;
      c->a16_gamma = nullptr;
      c->a16_eps = 0.f;
      c->a16_M = S;
      c->a16_K = Wq;
    }
    return 0;
  }
  const uint32_t nsplit = 8;  // ATT_SPLIT in llama_kernels.hip
  size_t slots = (size_t)S * n_heads;
  if (ensure(c, &c->att_ws, &c->att_ws_bytes, slots * nsplit * 130 * sizeof(float))) return -1;
  if (slots > c->att_cnt_n) {
    if (c->capturing) return fail(c, "smith_attention: counters needed while capturing; run once first");
    HIPCHK(c, hipStreamSynchronize(c->stream));
    if (c->att_cnt) c->retired.push_back(c->att_cnt);  // a captured graph may still use them
    c->att_cnt = nullptr;
    c->att_cnt_n = 0;
    size_t cap = std::max<size_t>(slots, 4096);
    HIPCHK(c, hipMalloc((void**)&c->att_cnt, cap * sizeof(uint32_t)));
    c->allocated += cap * sizeof(uint32_t);
    if (zero_now(c, c->att_cnt, cap * sizeof(uint32_t))) return -1;
    c->att_cnt_n = cap;
  }
  void* pws = c->att_ws;
  uint32_t* pcnt = c->att_cnt;
  uint32_t appended = 0;
  if (S > 1) {
    // prompt rows: rope + append every row's key/value first, so the
    // attention workgroups read all keys from the caches
    uint32_t Wq = n_heads * head_dim;
    void* aargs[] = {&qkv, &ld, &pos_ptr, &Wq, &n_kv_heads, &head_dim, &rope_cos, &rope_sin, &kcache, &vcache,
                     &max_seq, &rope_len, &perr};
    if (launch(c, "smith_kv_append", dim3(S), dim3(256), aargs)) return -1;
    appended = 1;
  }
  void* args[] = {&qkv, &ld, &pos_ptr, &S, &n_heads, &n_kv_heads, &head_dim, &rope_cos, &rope_sin,
                  &kcache, &vcache, &max_seq, &out, &pws, &pcnt, &act_out, &rope_len, &perr};
  return launch(c, appended ? "smith_attention_cached" : "smith_attention", dim3(n_heads, S, nsplit), dim3(256),
                args);
}

int smith_attention_parts(void* ctx, const float* qkv, const int32_t* pos_ptr, uint32_t n_heads, uint32_t n_kv_heads,
                          uint32_t head_dim, const float* rope_cos, const float* rope_sin, uint32_t rope_len,
                          const float* rope_row, float* kcache, float* vcache, uint32_t max_seq, float* parts) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (!n_kv_heads || n_heads % n_kv_heads)
    return fail(c, "smith_attention_parts: %u heads not a multiple of %u kv heads", n_heads, n_kv_heads);
  if (head_dim > 128 || head_dim % 32)
    return fail(c, "smith_attention_parts: head_dim %u unsupported (<= 128, %% 32)", head_dim);
  if (set_device(c)) return -1;
  if ((n_heads * head_dim) % 2 || (n_kv_heads * head_dim) % 2)
    return fail(c, "smith_attention_parts: q / k row widths must be even (RoPE pairs)");
  uint32_t* perr = c->pos_err_dev;
  void* args[] = {&qkv, &pos_ptr, &n_heads, &n_kv_heads, &head_dim, &rope_cos, &rope_sin, &rope_row,
                  &kcache, &vcache, &max_seq, &parts, &rope_len, &perr};
  return launch(c, "smith_attention_part", dim3(n_heads, 8), dim3(256), args);  // ATTP_MAXSPLIT splits
}

int smith_linear_q4_0_t_attn(void* ctx, const float* parts, const int32_t* pos_ptr, uint32_t head_dim,
                             const void* nib, const void* d, float* out, uint32_t N, uint32_t K, const float* resid,
                             uint32_t epilogue, void* act_out, const float* gamma_out) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  return attn_gemv(c, "smith_linear_q4_0_t_attn", FQ40T, parts, pos_ptr, head_dim, nib, d, out, N, K, resid,
                   epilogue, act_out, gamma_out);
}

uint64_t smith_gguf_tiles_bytes(uint32_t ggml_type, uint32_t N, uint32_t K) {
  const int f = gt_of_ggml((int)ggml_type);
  if (f < 0 || !N || N % 16 || !K || K % (gt_super(f) ? 256u : 32u)) return 0;
  return gt_planes(f, N, K / 32).total;
}

int smith_repack_gguf_tiles_into(void* ctx, uint32_t ggml_type, const void* blocks, void* planes, uint32_t N,
                                 uint32_t K, uint32_t n_off, uint32_t n_stride, uint32_t N_total) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  Fmt fmt;
  if (tiles_fmt(c, "smith_repack_gguf_tiles_into", ggml_type, N_total, K, &fmt)) return -1;
  if (!blocks || !planes) return fail(c, "smith_repack_gguf_tiles_into: null buffer");
  if (N && (uint64_t)n_off + (uint64_t)(N - 1) * n_stride >= N_total)
    return fail(c, "smith_repack_gguf_tiles_into: columns exceed N_total=%u", N_total);
  if (set_device(c)) return -1;
  const uint32_t G = K / 32;
  const uint64_t total = (uint64_t)N * G;
  if (!total) return 0;
  static const char* names[] = {"", "", "", "smith_repack_gt_q40", "smith_repack_gt_q41", "smith_repack_gt_q50",
                                "smith_repack_gt_q4k", "smith_repack_gt_q6k"};
  uint32_t pN = N, pG = G, po = n_off, ps = n_stride, pT = N_total;
  void* args[] = {&blocks, &planes, &pN, &pG, &po, &ps, &pT};
  return launch(c, names[fmt], dim3((unsigned)std::min<uint64_t>((total + 255) / 256, 1 << 20)), dim3(256), args);
}

int smith_linear_gguf_tiles(void* ctx, uint32_t ggml_type, const float* x, const void* planes, float* out,
                            uint32_t M, uint32_t N, uint32_t K, const float* norm_gamma, float eps, const float* resid,
                            uint32_t epilogue) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  Fmt fmt;
  if (tiles_fmt(c, "smith_linear_gguf_tiles", ggml_type, N, K, &fmt)) return -1;
  if (epilogue > 2) return fail(c, "smith_linear_gguf_tiles: unknown epilogue %u", epilogue);
  if (epilogue == 1 && !resid) return fail(c, "smith_linear_gguf_tiles: residual epilogue without a residual buffer");
  const void *B, *D;
  tiles_bd(fmt, planes, N, K, &B, &D);
  Epi e;
  e.gamma = norm_gamma;
  e.eps = eps;
  e.resid = epilogue == 1 ? resid : nullptr;
  e.mode = epilogue;
  if (fmt == FQ40T) return qmatmul(c, FQ40T, x, B, D, out, M, N, K, K / 32, e);
  // the other tile formats: every row count on the MFMA GEMM (single rows
  // of the decode step take the act path, smith_linear_gguf_tiles_act)
  if (set_device(c)) return -1;
  if (M == 0) return 0;
  return gemm(c, fmt, x, B, D, out, M, N, K, e);
}

int smith_linear_gguf_tiles_act(void* ctx, uint32_t ggml_type, const void* act_in, int norm, float eps,
                                const void* planes, float* out, uint32_t N, uint32_t K, const float* resid,
                                uint32_t epilogue, void* act_out, const float* gamma_out) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  Fmt fmt;
  if (tiles_fmt(c, "smith_linear_gguf_tiles_act", ggml_type, N, K, &fmt)) return -1;
  const void *B, *D;
  tiles_bd(fmt, planes, N, K, &B, &D);
  return act_gemv(c, "smith_linear_gguf_tiles_act", fmt, act_in, norm, eps, B, D, out, N, K, resid, epilogue,
                  act_out, gamma_out);
}

int smith_linear_gguf_tiles_attn(void* ctx, uint32_t ggml_type, const float* parts, const int32_t* pos_ptr,
                                 uint32_t head_dim, const void* planes, float* out, uint32_t N, uint32_t K,
                                 const float* resid, uint32_t epilogue, void* act_out, const float* gamma_out) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  Fmt fmt;
  if (tiles_fmt(c, "smith_linear_gguf_tiles_attn", ggml_type, N, K, &fmt)) return -1;
  const void *B, *D;
  tiles_bd(fmt, planes, N, K, &B, &D);
  return attn_gemv(c, "smith_linear_gguf_tiles_attn", fmt, parts, pos_ptr, head_dim, B, D, out, N, K, resid,
                   epilogue, act_out, gamma_out);
}

namespace {
const char* pair_tag(Fmt f1, Fmt f2) {
  static const struct { Fmt a, b; const char* tag; } pairs[] = {
      {FQ4KT, FQ6KT, "q4kt_q6kt"}, {FQ4KT, FQ50T, "q4kt_q50t"}, {FQ50T, FQ6KT, "q50t_q6kt"},
      {FQ40T, FQ6KT, "q40t_q6kt"}, {FQ4KT, FQ40T, "q4kt_q40t"}};
  for (const auto& p : pairs)
    if (p.a == f1 && p.b == f2) return p.tag;
  return nullptr;
}
}  // namespace

int smith_gguf_tiles_pair_ok(uint32_t type1, uint32_t type2) {
  const int f1 = gt_of_ggml((int)type1), f2 = gt_of_ggml((int)type2);
  return f1 >= 0 && f2 >= 0 && pair_tag((Fmt)f1, (Fmt)f2) ? 1 : 0;
}

int smith_linear_gguf_tiles_pair_act(void* ctx, uint32_t type1, const void* planes1, uint32_t N1, uint32_t type2,
                                     const void* planes2, uint32_t N2, const void* act_in, int norm, float eps,
                                     float* out, uint32_t K) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  const char* fn = "smith_linear_gguf_tiles_pair_act";
  Fmt f1, f2;
  if (tiles_fmt(c, fn, type1, N1, K, &f1) || tiles_fmt(c, fn, type2, N2, K, &f2)) return -1;
  const char* tag = pair_tag(f1, f2);
  if (!tag) return fail(c, "%s: no kernel for the GGML type pair (%u, %u)", fn, type1, type2);
  if (!act_in || !planes1 || !planes2 || !out) return fail(c, "%s: null buffer", fn);
  if (set_device(c)) return -1;
  static const uint32_t kbs[] = {32, 48, 64, 72, 96, 128, 144, 192, 288};
  const uint32_t G = K / 32, N = N1 + N2;
  uint32_t kb = 288;
  for (uint32_t v : kbs)
    if (v >= G) {
      kb = v;
      break;
    }
  const uint32_t ksplit = (G + kb - 1) / kb;
  const uint32_t threads = kb == 32 || kb == 48 || kb == 64 ? 256 : (kb == 72 ? 384 : (kb == 144 ? 768 : 512));
  const uint32_t gx = N / 16;
  if (ksplit > 1) {
    if (ensure(c, (void**)&c->ws, &c->ws_bytes, (size_t)ksplit * N * sizeof(float))) return -1;
    if (ensure_counters(c, gx)) return -1;
  }
  char name[64];
  snprintf(name, sizeof name, "smith_agemv2_%s_k%u", tag, kb);
  float* pws = c->ws;
  uint32_t* pcnt = c->counters;
  uint32_t pN1 = N1, pN = N, pK = K, pnorm = norm ? 1u : 0u;
  void* args[] = {&act_in, &planes1, &planes2, &out, &pN1, &pN, &pK, &pnorm, &eps, &pws, &pcnt};
  return launch(c, name, dim3(gx, ksplit), dim3(threads), args);
}

int smith_dequantize_gguf(void* ctx, uint32_t ggml_type, const void* src, float* dst, uint64_t numel) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (!numel) return 0;
  if (!src || !dst) return fail(c, "smith_dequantize_gguf: null buffer");
  if (set_device(c)) return -1;
  if (ggml_type == 0) {
    HIPCHK(c, hipMemcpyAsync(dst, src, numel * 4, hipMemcpyDeviceToDevice, c->stream));
    return 0;
  }
  const char* name = nullptr;
  switch (ggml_type) {
    case 1: name = "smith_dequantize_f16"; break;
    case 30: name = "smith_dequantize_bf16"; break;
    case 2: name = "smith_dequantize_q4_0"; break;
    case 3: name = "smith_dequantize_q4_1"; break;
    case 6: name = "smith_dequantize_q5_0"; break;
    case 8: name = "smith_dequantize_q8_0"; break;
    case 12: name = "smith_dequantize_q4_k"; break;
    case 14: name = "smith_dequantize_q6_k"; break;
    default: return fail(c, "smith_dequantize_gguf: GGML type %u cannot be dequantized", ggml_type);
  }
  uint64_t pn = numel;
  void* args[] = {&src, &dst, &pn};
  return launch(c, name, dim3((unsigned)std::min<uint64_t>((numel + 255) / 256, 1 << 20)), dim3(256), args);
}

int smith_repack_lmhead_q4_0(void* ctx, const void* blocks, void* nib, void* d, uint32_t K, uint32_t N) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (N % 32) return fail(c, "smith_repack_lmhead_q4_0: vocab %u is not a multiple of 32", N);
  if (set_device(c)) return -1;
  uint32_t NB = N / 32;
  uint64_t total = (uint64_t)K * NB;
  if (!total) return 0;
  void* args[] = {&blocks, &nib, &d, &K, &NB};
  return launch(c, "smith_repack_lmhead_q4_0", dim3((unsigned)std::min<uint64_t>((total + 255) / 256, 1 << 20)),
                dim3(256), args);
}

static int lmhead_q4_0(Ctx* c, const char* who, const float* x, const float* norm_gamma, float eps,
                       const void* nib, const void* d, float* y, uint32_t K, uint32_t N, GreedyTail gt) {
  if (N % 32) return fail(c, "%s: vocab %u is not a multiple of 32", who, N);
  if (K > 8192 || K % 8 || !K) return fail(c, "%s: dim %u unsupported (8..8192, %% 8)", who, K);
  if (set_device(c)) return -1;
  uint32_t gx = (N / 32 + 15) / 16;
  // splits of <= 256 rows: at most 4 row octets per wave, all loads in flight at once
  uint32_t ksplit = std::max<uint32_t>(1, (K + 255) / 256);
  if (ksplit > 1) {
    if (ensure(c, (void**)&c->ws, &c->ws_bytes, (size_t)ksplit * N * sizeof(float))) return -1;
    if (ensure_counters(c, gx)) return -1;
  }
  float* pws = c->ws;
  uint32_t* pcnt = c->counters;
  void* args[] = {&x, &norm_gamma, &eps, &nib, &d, &y, &K, &N, &pws, &pcnt, &gt};
  return launch(c, "smith_lmhead_q4_0_nb", dim3(gx, ksplit), dim3(512), args);
}

int smith_lmhead_q4_0_nb(void* ctx, const float* x, const float* norm_gamma, float eps, const void* nib,
                         const void* d, float* y, uint32_t K, uint32_t N) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  GreedyTail gt{};
  return lmhead_q4_0(c, "smith_lmhead_q4_0_nb", x, norm_gamma, eps, nib, d, y, K, N, gt);
}

int smith_lmhead_q4_0_greedy(void* ctx, const float* x, const float* norm_gamma, float eps, const void* nib,
                             const void* d, float* logits, uint32_t K, uint32_t N, const float* E, float* x_out,
                             int32_t* tokens, int32_t* count, int32_t* pos, void* act_out, const float* gamma_out,
                             const float* rope_cos, const float* rope_sin, uint32_t rope_len, uint32_t wq,
                             uint32_t wk, float* rope_row) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (!E || !x_out || !tokens || !count || !pos)
    return fail(c, "smith_lmhead_q4_0_greedy: embedding, x, tokens, count and position are required");
  if (act_out && K % 32) return fail(c, "smith_lmhead_q4_0_greedy: an act output needs dim %% 32 == 0 (dim %u)", K);
  if (rope_row && (!rope_cos || !rope_sin || wq % 2 || wk % 2))
    return fail(c, "smith_lmhead_q4_0_greedy: a rope row needs both tables and even row widths");
  if (set_device(c) || ensure_amx(c)) return -1;
  GreedyTail gt{E, x_out, tokens, count, pos, act_out, gamma_out, rope_cos, rope_sin, rope_row, c->amx,
                rope_len, wq, wk, K};
  return lmhead_q4_0(c, "smith_lmhead_q4_0_greedy", x, norm_gamma, eps, nib, d, logits, K, N, gt);
}

uint64_t smith_lmhead_q6_k_bytes(uint32_t K, uint32_t N) {
  if (!K || !N || N % 256) return 0;
  const size_t KN = (size_t)K * N;
  size_t hb = gt_align(KN / 2), sc = gt_align(hb + KN / 4), d = gt_align(sc + KN / 16);
  return gt_align(d + KN / 256 * 2);
}

int smith_repack_lmhead_q6_k(void* ctx, const void* blocks, void* planes, uint32_t K, uint32_t N) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (N % 256 || !N) return fail(c, "smith_repack_lmhead_q6_k: vocab %u is not a multiple of 256", N);
  if (K % 8) return fail(c, "smith_repack_lmhead_q6_k: dim %u is not a multiple of 8 (row octets)", K);
  if (set_device(c)) return -1;
  uint64_t total = (uint64_t)K * (N / 256);
  if (!total) return 0;
  void* args[] = {&blocks, &planes, &K, &N};
  return launch(c, "smith_repack_lmhead_q6_k", dim3((unsigned)std::min<uint64_t>((total + 255) / 256, 1 << 20)),
                dim3(256), args);
}

static int lmhead_q6_k(Ctx* c, const char* who, const float* x, const float* norm_gamma, float eps,
                       const void* planes, float* y, uint32_t K, uint32_t N, GreedyTail gt) {
  if (N % 256 || !N) return fail(c, "%s: vocab %u is not a multiple of 256", who, N);
  if (K > 8192 || K % 16 || !K) return fail(c, "%s: dim %u unsupported (16..8192, %% 16)", who, K);
  if (set_device(c)) return -1;
  uint32_t gx = (N / 32 + 15) / 16;
  uint32_t ksplit = std::max<uint32_t>(1, std::min<uint32_t>((K + 255) / 256, 64));
  if (ksplit > 1) {
    if (ensure(c, (void**)&c->ws, &c->ws_bytes, (size_t)ksplit * N * sizeof(float))) return -1;
    if (ensure_counters(c, gx)) return -1;
  }
  float* pws = c->ws;
  uint32_t* pcnt = c->counters;
  void* args[] = {&x, &norm_gamma, &eps, &planes, &y, &K, &N, &pws, &pcnt, &gt};
  return launch(c, "smith_lmhead_q6_k_nb", dim3(gx, ksplit), dim3(512), args);
}

int smith_lmhead_q6_k_nb(void* ctx, const float* x, const float* norm_gamma, float eps, const void* planes, float* y,
                         uint32_t K, uint32_t N) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  GreedyTail gt{};
  return lmhead_q6_k(c, "smith_lmhead_q6_k_nb", x, norm_gamma, eps, planes, y, K, N, gt);
}

int smith_lmhead_q6_k_greedy(void* ctx, const float* x, const float* norm_gamma, float eps, const void* planes,
                             float* logits, uint32_t K, uint32_t N, const float* E, float* x_out, int32_t* tokens,
                             int32_t* count, int32_t* pos, void* act_out, const float* gamma_out,
                             const float* rope_cos, const float* rope_sin, uint32_t rope_len, uint32_t wq,
                             uint32_t wk, float* rope_row) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (!E || !x_out || !tokens || !count || !pos)
    return fail(c, "smith_lmhead_q6_k_greedy: embedding, x, tokens, count and position are required");
  if (act_out && K % 32) return fail(c, "smith_lmhead_q6_k_greedy: an act output needs dim %% 32 == 0 (dim %u)", K);
  if (rope_row && (!rope_cos || !rope_sin || wq % 2 || wk % 2))
    return fail(c, "smith_lmhead_q6_k_greedy: a rope row needs both tables and even row widths");
  if (set_device(c) || ensure_amx(c)) return -1;
  GreedyTail gt{E, x_out, tokens, count, pos, act_out, gamma_out, rope_cos, rope_sin, rope_row, c->amx,
                rope_len, wq, wk, K};
  return lmhead_q6_k(c, "smith_lmhead_q6_k_greedy", x, norm_gamma, eps, planes, logits, K, N, gt);
}

int smith_gemv_f32(void* ctx, const float* x, const float* norm_gamma, float eps, const float* W, float* y,
                   uint32_t K, uint32_t N, int w_is_nk) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (K > 8192) return fail(c, "smith_gemv_f32: K %u exceeds 8192", K);
  if (set_device(c)) return -1;
  void* args[] = {&x, &norm_gamma, &eps, &W, &y, &K, &N};
  if (w_is_nk) return launch(c, "smith_gemv_f32_nk", dim3(std::min<uint32_t>((N + 3) / 4, 2048)), dim3(256), args);
  return launch(c, "smith_gemv_f32_kn", dim3((N + 63) / 64), dim3(1024), args);
}

int smith_argmax_embed(void* ctx, const float* logits, uint32_t N, const float* E, uint32_t dim, float* x,
                       int32_t* tokens, int32_t* count, int32_t* pos, void* act_out, const float* gamma_out,
                       const float* rope_cos, const float* rope_sin, uint32_t rope_len, uint32_t wq, uint32_t wk,
                       float* rope_row) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (act_out && dim % 32) return fail(c, "smith_argmax_embed: an act output needs dim %% 32 == 0 (dim %u)", dim);
  if (set_device(c)) return -1;
  if (rope_row && (!rope_cos || !rope_sin || wq % 2 || wk % 2))
    return fail(c, "smith_argmax_embed: a rope row needs both tables and even row widths");
  void* args[] = {&logits, &N, &E, &dim, &x, &tokens, &count, &pos, &act_out, &gamma_out,
                  &rope_cos, &rope_sin, &rope_len, &wq, &wk, &rope_row};
  return launch(c, "smith_argmax_embed", dim3(1), dim3(1024), args);
}

int smith_set_i32(void* ctx, int32_t* p, int32_t v) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (set_device(c)) return -1;
  void* args[] = {&p, &v};
  return launch(c, "smith_set_i32", dim3(1), dim3(64), args);
}

int smith_randn(void* ctx, float* out, uint64_t n, uint64_t seed, uint64_t offset, float stdv, float mean) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (offset % 2) return fail(c, "smith_randn: offset must be even (Box-Muller pairs)");
  if (set_device(c)) return -1;
  if (!n) return 0;
  void* args[] = {&out, &n, &seed, &offset, &stdv, &mean};
  uint64_t pairs = (n + 1) / 2;
  return launch(c, "smith_randn_f32", dim3((unsigned)std::min<uint64_t>((pairs + 255) / 256, 65536)), dim3(256),
                args);
}

// ---------------- HIP graphs ----------------
int smith_graph_begin(void* ctx) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (set_device(c)) return -1;
  if (c->profile) return fail(c, "smith_graph_begin: kernel profiling must be off while capturing");
  HIPCHK(c, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
  c->capturing = true;
  return 0;
}

void* smith_graph_end(void* ctx) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return nullptr;
  c->capturing = false;
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(c->stream, &g);
  if (e != hipSuccess || !g) {
    fail(c, "smith_graph_end: %s", hipGetErrorString(e));
    return nullptr;
  }
  hipGraphExec_t ge = nullptr;
  e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) {
    fail(c, "smith_graph_end: instantiate: %s", hipGetErrorString(e));
    return nullptr;
  }
  return (void*)ge;
}

int smith_graph_launch(void* ctx, void* graph) {
  Ctx* c = (Ctx*)ctx;
  if (!c || !graph) return -1;
  if (set_device(c)) return -1;
  HIPCHK(c, hipGraphLaunch((hipGraphExec_t)graph, c->stream));
  return 0;
}

void smith_graph_destroy(void* graph) {
  if (graph) (void)hipGraphExecDestroy((hipGraphExec_t)graph);
}

// ---------------- timing ----------------
int smith_profile_kernels(void* ctx, int enable) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  c->profile = enable != 0;
  return 0;
}

int smith_profile_read(void* ctx, const char* prefix, double* total_ms, uint64_t* count) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (set_device(c)) return -1;
  HIPCHK(c, hipStreamSynchronize(c->stream));
  size_t plen = prefix ? strlen(prefix) : 0;
  double tot = 0.0;
  uint64_t n = 0;
  std::vector<Ctx::Rec> keep;
  for (auto& r : c->recs) {
    if (plen && r.name.compare(0, plen, prefix) != 0) {
      keep.push_back(r);
      continue;
    }
    float ms = 0.f;
    HIPCHK(c, hipEventElapsedTime(&ms, r.a, r.b));
    tot += ms;
    n++;
    c->event_pool.push_back(r.a);
    c->event_pool.push_back(r.b);
  }
  c->recs.swap(keep);
  if (total_ms) *total_ms = tot;
  if (count) *count = n;
  return 0;
}

int smith_timer_start(void* ctx) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (set_device(c)) return -1;
  HIPCHK(c, hipEventRecord(c->t0, c->stream));
  return 0;
}

double smith_timer_stop(void* ctx) {
  Ctx* c = (Ctx*)ctx;
  if (!c) return -1;
  if (set_device(c)) return -1;
  if (hipEventRecord(c->t1, c->stream) != hipSuccess || hipEventSynchronize(c->t1) != hipSuccess)
    return fail(c, "smith_timer_stop: event failure");
  float ms = 0.f;
  if (hipEventElapsedTime(&ms, c->t0, c->t1) != hipSuccess) return fail(c, "smith_timer_stop: elapsed failure");
  return ms;
}

}  // extern "C"
