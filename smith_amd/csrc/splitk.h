// splitk.h -- the read side of the deterministic cross-workgroup split-K
// reduction shared by the GEMV, LM head and GEMM kernels: the partials of
// the other workgroups (possibly on other XCDs, written with agent-scope
// atomics) are read with agent-scope atomics too, up to 16 in flight at
// once, and summed in split order -- the same sum as a serial loop, with one
// memory round trip per 16 splits instead of one per split.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define SPLITK_BATCH 16

// sum over sp < ksplit of the float at p + sp * stride
__device__ __forceinline__ float splitk_sum(const float* p, size_t stride, uint32_t ksplit) {
  uint32_t* q = (uint32_t*)p;
  float v = 0.f;
  for (uint32_t sp = 0; sp < ksplit; sp += SPLITK_BATCH) {
    float x[SPLITK_BATCH];
#pragma unroll
    for (int i = 0; i < SPLITK_BATCH; i++)
      x[i] = sp + i < ksplit
                 ? __uint_as_float(__hip_atomic_fetch_add(q + (size_t)(sp + i) * stride, 0u, __ATOMIC_RELAXED,
                                                          __HIP_MEMORY_SCOPE_AGENT))
                 : 0.f;
#pragma unroll
    for (int i = 0; i < SPLITK_BATCH; i++)
      if (sp + i < ksplit) v += x[i];
  }
  return v;
}
