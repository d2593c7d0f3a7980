// Bench-only host helper (libsmith_bench.so): times the floor kernels of
// bench_floor.hip the way bench.py times the product's steps -- `steps`
// launches, launch i reading buffer i % nbufs, captured once as a HIP graph
// on a stream of its own, replayed once untimed, then once between two HIP
// events.  The buffers are device pointers of the same device (allocated by
// the product library).  Not part of the product ABI (include/smith.h).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

namespace {
std::string g_err;
hipModule_t g_mod = nullptr;
std::string g_mod_path;

int fail(const char* what, hipError_t e) {
  g_err = std::string(what) + ": " + hipGetErrorString(e);
  return -1;
}
}  // namespace

#define CHK(expr)                                  \
  do {                                             \
    hipError_t e_ = (expr);                        \
    if (e_ != hipSuccess) return fail(#expr, e_);  \
  } while (0)

extern "C" {

const char* smith_bench_error(void) { return g_err.c_str(); }

// Per-launch microseconds of kernel `name` from code object `hsaco`:
// args (bufs[i % nbufs], n, out), grid x block threads.
int smith_bench_floor(const char* hsaco, const char* name, void* const* bufs, uint32_t nbufs, uint64_t n, void* out,
                      uint32_t grid, uint32_t block, uint32_t steps, double* us) {
  if (!hsaco || !name || !bufs || !nbufs || !steps || !us || !grid || !block) {
    g_err = "smith_bench_floor: bad arguments";
    return -1;
  }
  if (!g_mod || g_mod_path != hsaco) {
    CHK(hipModuleLoad(&g_mod, hsaco));
    g_mod_path = hsaco;
  }
  hipFunction_t f;
  CHK(hipModuleGetFunction(&f, g_mod, name));
  hipStream_t s;
  CHK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  hipGraph_t g = nullptr;
  hipGraphExec_t ge = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  int rc = -1;
  do {
    if (hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal) != hipSuccess) break;
    bool ok = true;
    for (uint32_t i = 0; i < steps && ok; i++) {
      void* p = bufs[i % nbufs];
      uint64_t pn = n;
      void* po = out;
      void* args[] = {&p, &pn, &po};
      ok = hipModuleLaunchKernel(f, grid, 1, 1, block, 1, 1, 0, s, args, nullptr) == hipSuccess;
    }
    const hipError_t ec = hipStreamEndCapture(s, &g);
    if (!ok || ec != hipSuccess) {
      g_err = "smith_bench_floor: capture failed";
      break;
    }
    if (hipGraphInstantiate(&ge, g, nullptr, nullptr, 0) != hipSuccess) {
      g_err = "smith_bench_floor: instantiate failed";
      break;
    }
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) break;
    if (hipGraphLaunch(ge, s) != hipSuccess || hipStreamSynchronize(s) != hipSuccess) break;  // warm
    if (hipEventRecord(e0, s) != hipSuccess || hipGraphLaunch(ge, s) != hipSuccess ||
        hipEventRecord(e1, s) != hipSuccess || hipEventSynchronize(e1) != hipSuccess)
      break;
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, e0, e1) != hipSuccess) break;
    *us = ms * 1e3 / steps;
    rc = 0;
  } while (false);
  if (rc && g_err.empty()) g_err = "smith_bench_floor: HIP call failed";
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (ge) (void)hipGraphExecDestroy(ge);
  if (g) (void)hipGraphDestroy(g);
  (void)hipStreamSynchronize(s);
  (void)hipStreamDestroy(s);
  return rc;
}
}
