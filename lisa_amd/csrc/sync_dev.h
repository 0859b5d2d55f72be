// Hand-off between workgroups of one launch (device helpers).
//
// A producer workgroup stores its data write-through (sc1: to the device's
// coherence point, no L2 write-back needed), waits for those stores, then
// stores a 64-bit flag holding the launch's tag; a consumer polls the flags
// with sc1 loads and reads the data with sc1 loads.  The tag is unique per
// dispatch (the AQL packet's dispatch id on its queue, mixed with the queue's
// address), so flags left by earlier launches never match and nothing is
// ever reset.  Waits are bounded: one that gives up sets *err.  A consumer
// only waits for workgroups dispatched before it or alongside it (the callers
// order their blocks so), so the waits end.
#pragma once
#include "lisaq_common.h"

namespace lisaq {

extern "C" __device__ uint64_t lisaq_dispatch_id() __asm("llvm.amdgcn.dispatch.id");

__device__ __forceinline__ uint64_t launch_tag() {
  return lisaq_dispatch_id() * 0x9E3779B97F4A7C15ull ^ (uint64_t)(uintptr_t)__builtin_amdgcn_queue_ptr();
}

// cache policy of the write-through stores and the coherent loads
constexpr int kSc1 = 16;

// polls of a wait before it gives up (each ~1-2 us: uncached loads plus a
// sleep); a wait only ends this way if the dispatch order assumption fails
constexpr int kSpinMax = 200000;

__device__ __forceinline__ void store_flag(uint64_t* f, uint64_t tag) {
  __hip_atomic_store(f, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// every thread of the workgroup: wait until flags[0, n) all hold tag
__device__ __forceinline__ void wait_flags(const uint64_t* f, int n, uint64_t tag, uint32_t* err) {
  for (int it = 0;; ++it) {
    int pend = 0;
    for (int i = (int)threadIdx.x; i < n; i += (int)blockDim.x)
      pend |= __hip_atomic_load(f + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != tag;
    if (!__syncthreads_or(pend)) return;
    if (it == kSpinMax) {
      if (threadIdx.x == 0) __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
    __builtin_amdgcn_s_sleep(4);  // (1: 12.2 us, 4: 12.3, 10: 12.5 at the decode MoE, T = 1)
  }
}

}  // namespace lisaq
