// Capacity-K piecewise chunk map of the hard-reset LIF step: construction (one input at a
// time) and evaluation.  Shared by the standalone build kernel and the fused scans.
//
// A map covering steps 1..L is  M(u) = A*u + B            if u < xd[n-1] (or n == 0)
//                                      cd[k]               k = #{i < n : xd[i] > u}
// with breakpoints xd[0] > xd[1] > ... (appended in this order) and constants cd[i]
// (fast.py:86-91; exact.py:64-131).  Breakpoint z of step j is the preimage of the threshold
// under the affine part so far, z = (theta - x - beta*B) / (beta*A) (+-inf when the
// denominator underflows to 0, fast.py:94-99), kept iff z < xmin and z <= hi
// (triton_lif.py:760); the reference's extra condition xmin > lo is applied afterwards by
// truncation (see k_lif_build).
#pragma once
#include "lsh_common.h"

namespace lsh {

template <int KMAX>
struct MapBuilder {
  float A, B, xmin;
  float xd[KMAX], cd[KMAX];
  int cnt;   // breakpoints stored
  int wcnt;  // wave-uniform upper bound of cnt (bounds the per-slot loops)
  bool ovf;  // a (K+1)-th breakpoint appeared

  __device__ __forceinline__ void init() {
    A = 1.0f;
    B = 0.0f;
    xmin = INFINITY;
    cnt = 0;
    wcnt = 0;
    ovf = false;
#pragma unroll
    for (int i = 0; i < KMAX; ++i) {
      xd[i] = INFINITY;
      cd[i] = 0.0f;
    }
  }

  // One step with input x (triton_lif.py:752-769): push every constant through the step,
  // then append the step's breakpoint, then advance the affine part.
  // wcnt is the same on every lane (it only grows through a ballot), so it is read as a scalar:
  // constants are pushed in groups of 8 slots behind one scalar branch per group (a slot above
  // a lane's cnt holds no breakpoint yet and is overwritten when one is added), and the
  // insertion, which few steps need, is skipped by the whole wave when no lane inserts.
  __device__ __forceinline__ void step(float x, float beta, float theta, float u_r, float hi, int K) {
    const int wc = __builtin_amdgcn_readfirstlane(wcnt);
    constexpr int G = KMAX < 8 ? KMAX : 8;
#pragma unroll
    for (int g = 0; g < KMAX; g += G) {
      if (g < wc) {
#pragma unroll
        for (int i = g; i < g + G; ++i) {
          const float v = lif_v(cd[i], x, beta);
          cd[i] = v >= theta ? u_r : v;
        }
      }
    }
    const float num = (theta - x) - beta * B;
    const float den = beta * A;
    const float z = den == 0.0f ? (num > 0.0f ? INFINITY : -INFINITY) : num / den;
    bool nw = (z < xmin) && (z <= hi);
    if (nw && cnt >= K) ovf = true;
    nw = nw && (cnt < K);
    if (__ballot(nw) != 0ull) {
#pragma unroll
      for (int i = 0; i < KMAX; ++i) {
        const bool put = nw && (i == cnt);
        xd[i] = put ? z : xd[i];
        cd[i] = put ? u_r : cd[i];
      }
      if (__ballot(nw && cnt == wc) != 0ull) ++wcnt;
    }
    cnt += nw ? 1 : 0;
    xmin = nw ? z : xmin;
    A = beta * A;
    B = lif_v(B, x, beta);
  }
};

}  // namespace lsh
