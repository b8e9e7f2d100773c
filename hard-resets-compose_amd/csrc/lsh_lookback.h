// Decoupled look-back across workgroups: coherent cross-XCD values and flags (shared by the LIF and
// ALIF look-back adjoints).
#pragma once
#include "lsh_common.h"

namespace lsh {

// Cross-workgroup values are written and read with agent-scope relaxed atomics (coherent
// vector loads/stores that bypass the non-coherent L2 of each XCD) instead of release/acquire
// fences, which would write back or invalidate a whole L2 per hand-off.  Ordering: a producer
// waits for its value stores to be acknowledged (s_waitcnt) before storing the flag; a consumer
// issues its value loads only after the flag load has returned non-zero.
__device__ __forceinline__ float ld_coh(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void publish_flag(int* f, int v) {
  __builtin_amdgcn_s_waitcnt(0);  // this wave's value stores are acknowledged
  if (__lane_id() == 0) __hip_atomic_store(f, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// flag of (segment, block) -> value seen by the whole wave
__device__ __forceinline__ int flag_wait(int* f, unsigned int* timeouts) {
  for (int it = 0; it < (1 << 22); ++it) {
    int v = __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    v = __builtin_amdgcn_readfirstlane(v);
    if (v != 0) return v;
    __builtin_amdgcn_s_sleep(2);
  }
  if (__lane_id() == 0) atomicAdd(timeouts, 1u);
  return -1;
}

}  // namespace lsh
