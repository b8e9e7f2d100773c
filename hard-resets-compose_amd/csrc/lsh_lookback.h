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

// Deterministic look-back.  Segments are grouped in runs of LB_GROUP; the first segment of each
// run (seg % LB_GROUP == 0) is its anchor.  The value at the end of segment `seg` is the
// composition of the published maps of the segments after it up to the next anchor
// B = (seg / LB_GROUP + 1) * LB_GROUP, in ascending order, applied to the anchor's published
// inclusive value (to 0 past the last segment).  An anchor publishes its inclusive value
// (flag 2) once it has its own end value, every other segment its map (flag 1) before it looks
// back.  Which operands meet in which order is fixed by the segment index alone, so the result
// has the same bits on every run (a look-back that stops at the first inclusive value it finds
// depends on which workgroup finished first).  The anchors form one chain of NSEG / LB_GROUP
// hand-offs; every other wait is on segments of the same run.  A workgroup only waits for
// segments with smaller tickets (running or done), so every wait ends; each is bounded anyway
// and a give-up is counted.
//
// The operands are fetched by all waves of the workgroup in parallel (lb_fetch: wave w waits for
// and loads the operands k = w, w + W, ... into LDS), then one wave composes them (lb_compose),
// so the look-back costs about one flag latency and one load latency, and no wave holds more
// than one operand in registers.
constexpr int LB_GROUP = 16;

__device__ __forceinline__ bool lb_is_anchor(int seg) { return seg % LB_GROUP == 0; }

// Operands of segment seg's look-back: k = 0 .. lb_count(seg) - 1 is segment seg + 1 + k, a map
// (P, Q) below the next anchor, the anchor's inclusive value (in P) at the anchor itself.
__device__ __forceinline__ int lb_next_anchor(int seg) { return (seg / LB_GROUP + 1) * LB_GROUP; }
__device__ __forceinline__ int lb_count(int seg, int NSEG) {
  const int B = lb_next_anchor(seg);
  return (B < NSEG ? B : NSEG - 1) - seg;
}

// Called by every wave w of W (all lanes): waits for and loads operands w, w + W, ... of
// segment seg for this lane's column `col` into sP[k][lane] / sQ[k][lane] (LDS, [LB_GROUP][64]).
// aP, aQ: published segment maps (value at start = Q + P * value at end), inc: published
// inclusive values, all [NSEG][N]; fl: flags [NSEG][NB]; nb: this workgroup's neuron block.
__device__ __forceinline__ void lb_fetch(int seg, int NSEG, int NB, int nb, int64_t N, int64_t col,
                                         int w, int W, const float* aP, const float* aQ,
                                         const float* inc, int* fl, float (*sP)[64],
                                         float (*sQ)[64], unsigned int* timeouts) {
  const int B = lb_next_anchor(seg);
  const int cnt = lb_count(seg, NSEG);
  const int lane = (int)__lane_id();
  for (int k = w; k < cnt; k += W) {
    const int j = seg + 1 + k;
    int* const f = fl + (size_t)j * NB + nb;
    bool ok = false;
    for (int it = 0; it < (1 << 22); ++it) {
      int v = __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      v = __builtin_amdgcn_readfirstlane(v);
      if (v != 0) {
        ok = true;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    if (!ok) {
      if (lane == 0) atomicAdd(timeouts, 1u);
      sP[k][lane] = 0.0f;  // not valid; the counted give-up says so
      sQ[k][lane] = 0.0f;
    } else if (j < B) {
      sP[k][lane] = ld_coh(aP + (size_t)j * N + col);
      sQ[k][lane] = ld_coh(aQ + (size_t)j * N + col);
    } else {
      sP[k][lane] = ld_coh(inc + (size_t)j * N + col);
    }
  }
}

// After a barrier that follows lb_fetch: the value at the end of segment seg (one wave).
__device__ __forceinline__ float lb_compose(int seg, int NSEG, const float (*sP)[64],
                                            const float (*sQ)[64]) {
  const int B = lb_next_anchor(seg);
  const int cnt = lb_count(seg, NSEG);
  const int lane = (int)__lane_id();
  float Pa = 1.0f, Qa = 0.0f;
  for (int k = 0; k < cnt; ++k) {
    if (seg + 1 + k < B) {
      Qa = Qa + Pa * sQ[k][lane];
      Pa = Pa * sP[k][lane];
    } else {
      return Qa + Pa * sP[k][lane];  // the anchor's inclusive value
    }
  }
  return Qa;  // past the last segment: the value there is 0
}

}  // namespace lsh
