// Shared device helpers for the MI355X (gfx950) hard-reset LIF / ALIF scan kernels.
//
// Numerics contract (every kernel in this library):
//   * one canonical step arithmetic, two IEEE round-to-nearest operations:
//       v = fl(fl(beta * u) + x);  s = v >= theta;  u' = s ? u_r : v
//     (triton_lif.py:21-25 `_step`, fast.py:76-79).  No FMA contraction anywhere
//     (built with -ffp-contract=off and the pragma below), so the serial
//     kernel, the scan's replay, the overflow fallback and the map constants
//     execute the identical instruction sequence and a plain fp32 CPU loop
//     reproduces every bit.
//   * fp32 denormals are kept (built with -fno-gpu-flush-denormals-to-zero).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#pragma clang fp contract(off)

namespace lsh {

constexpr int WAVE = 64;

// Waves per workgroup of the single-pass (fused) kernels, where each wave owns one chunk of a
// round: 4 when there are enough 64-neuron blocks to give every CU several workgroups, more
// chunks in flight per workgroup when there are few.  wmax is what the kernel's registers allow
// (16 waves of a workgroup need <= 128 VGPRs per lane, 8 waves <= 256).
inline int fused_waves(int64_t nblocks, int wmax) {
  const int w = nblocks >= 512 ? 4 : (nblocks >= 128 ? 8 : 16);
  return w < wmax ? w : wmax;
}

// LIF membrane update before the threshold test (triton_lif.py:22).
__device__ __forceinline__ float lif_v(float u, float x, float beta) {
  return __fadd_rn(__fmul_rn(beta, u), x);
}

// One affine-reset step (triton_affine.py:20-24): u' = s ? fl(fl(gamma*v) + delta) : v.
__device__ __forceinline__ float aff_step(float u, float x, float beta, float theta, float gamma,
                                          float delta, bool& s) {
  const float v = __fadd_rn(__fmul_rn(beta, u), x);
  s = v >= theta;
  return s ? __fadd_rn(__fmul_rn(gamma, v), delta) : v;
}

// One hard-reset LIF step; returns the new state and writes the spike.
__device__ __forceinline__ float lif_step(float u, float x, float beta, float theta, float u_r,
                                          bool& s) {
  const float v = lif_v(u, x, beta);
  s = v >= theta;
  return s ? u_r : v;
}

// The value of v in lane `lane` (wave-uniform), for walks with one wave per neuron.
__device__ __forceinline__ float lane_f(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// L serial LIF steps of column n from row r0, for a walk with one wave per neuron (every lane
// holds the same state u): the rows are read 64 at a time, one per lane, the next 64 (index
// clamped to the last row) while a block is walked, and each step takes its input from its lane.
// The same step arithmetic as the replay.
__device__ __forceinline__ float wave_serial_rows(const float* __restrict__ I, int64_t N,
                                                  int64_t n, int64_t r0, int64_t L, float u,
                                                  float beta, float theta, float u_r) {
  const int lane = threadIdx.x & 63;
  const float* Ip = I + (size_t)r0 * N + n;
  float xv = Ip[(size_t)min<int64_t>(lane, L - 1) * N];
  for (int64_t t0 = 0; t0 < L; t0 += 64) {
    const float xn = Ip[(size_t)min<int64_t>(t0 + 64 + lane, L - 1) * N];
    if (L - t0 >= 64) {
#pragma unroll 16
      for (int j = 0; j < 64; ++j) {
        bool s;
        u = lif_step(u, lane_f(xv, j), beta, theta, u_r, s);
      }
    } else {
      for (int j = 0; j < (int)(L - t0); ++j) {
        bool s;
        u = lif_step(u, lane_f(xv, j), beta, theta, u_r, s);
      }
    }
    xv = xn;
  }
  return u;
}

// Neuron of workgroup b for kernels with one wave per neuron: eight contiguous ranges, range x
// on the workgroups b with b % 8 == x.  Consecutive workgroups go to the eight XCDs in turn,
// so each XCD's L2 then holds the cache lines (32 neurons a line) of its own neurons.
__device__ __forceinline__ int64_t xcd_neuron(int64_t b, int64_t N) {
  const int64_t q = N / 8, rem = N % 8, x = b % 8;
  return x * q + (x < rem ? x : rem) + b / 8;
}

// 1 / (1 + exp(-z)), the logistic sigmoid of every surrogate.  LSH_FAST_SURROGATE (default)
// takes the hardware exponential and reciprocal (a few ulp; the reference's Triton path also
// uses approximate exp and division) instead of the library expf and a correctly rounded
// division: adjoints move by <= 2e-7 relative and run 1-2.5 % faster (cfg2 recomputing adjoint
// 0.605 -> 0.598 ms, cfg4 serial adjoint 36.6 -> 35.7 ms); gradients are compared within a
// tolerance either way.
#ifndef LSH_FAST_SURROGATE
#define LSH_FAST_SURROGATE 1
#endif
__device__ __forceinline__ float sigmoid_neg_exact(float z) { return 1.0f / (1.0f + expf(-z)); }
__device__ __forceinline__ float sigmoid_neg(float z) {
#if LSH_FAST_SURROGATE
  return __builtin_amdgcn_rcpf(1.0f + __expf(-z));
#else
  return 1.0f / (1.0f + expf(-z));
#endif
}

// Surrogate derivative alpha*sig*(1-sig), sig = 1/(1+exp(-alpha*(v-theta)))
// (triton_lif.py:45-46).
__device__ __forceinline__ float surrogate(float v, float theta, float alpha) {
  const float sig = sigmoid_neg(alpha * (v - theta));
  return alpha * sig * (1.0f - sig);
}

// Streaming (non-temporal) accesses: U, S and Lam are written once and not
// re-read by the same kernel, so they should not evict the inputs from L2/MALL.
template <typename T>
__device__ __forceinline__ void st_nt(T* p, T v) { __builtin_nontemporal_store(v, p); }
template <typename T>
__device__ __forceinline__ T ld_nt(const T* p) { return __builtin_nontemporal_load(p); }

// Row access with a wave-uniform row pointer and a 32-bit per-lane byte offset, so the
// compiler can address with an SGPR base + VGPR offset instead of a 64-bit VGPR pair per
// access (fewer VGPRs and address instructions in the unrolled time loops).
__device__ __forceinline__ float ld_row(const float* __restrict__ row, unsigned boff) {
  return *reinterpret_cast<const float*>(reinterpret_cast<const char*>(row) + boff);
}
__device__ __forceinline__ void st_row_nt(float* __restrict__ row, unsigned boff, float v) {
  __builtin_nontemporal_store(v, reinterpret_cast<float*>(reinterpret_cast<char*>(row) + boff));
}

// Raw buffer access (CDNA3/4): a 128-bit SGPR descriptor for a wave-uniform base address,
// one per-lane VGPR byte offset shared by every access, and a wave-uniform SGPR byte offset
// per time row.  The unrolled time loops then need no per-access address registers.
// Descriptor word 3 (0x00020000) is the gfx9-family raw-buffer format (32-bit data).  The
// record count is left at its maximum: callers keep every access in bounds themselves.
// Cache policy of the streaming row loads: 2 = nt (non-temporal, the streaming hint; the rows
// are read once per pass).  Measured at cfg2: adjoint 0.622 -> 0.606-0.612 ms, forward ~1.5%
// faster than with the default policy 0, same bits.
#ifndef LSH_LD_POLICY
#define LSH_LD_POLICY 2
#endif

struct Buf {
  __amdgpu_buffer_rsrc_t r;
  __device__ __forceinline__ explicit Buf(const void* base)
      : r(__builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)0xffffffff,
                                            0x00020000)) {}
  __device__ __forceinline__ float ld(unsigned voff, unsigned soff) const {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, LSH_LD_POLICY));
  }
  // non-temporal store (cache policy bit 1 = nt on gfx94x/gfx950)
  __device__ __forceinline__ void st_nt(unsigned voff, unsigned soff, float v) const {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, voff, soff, 2);
  }
};

// Wave-level reductions (wave64).
// f(j, p[j*stride]) for j = 0..n-1 in order, loading the rows in tiles of D with the next
// tile's loads issued before the current tile is consumed (serial fallbacks and repairs run
// one dependent chain per lane; without this every step waits for its own load).  The next
// tile's loads are issued on every tile (the last tile reloads itself): behind a branch the
// compiler could not tell whether they were issued, and its wait for the current tile would
// then cover them too.
template <int D, class F>
__device__ __forceinline__ void stream_rows(const float* __restrict__ p, size_t stride, int64_t n,
                                            F&& f) {
  const int64_t nt = n / D;
  float a[D];
  if (nt > 0) {
#pragma unroll
    for (int k = 0; k < D; ++k) a[k] = p[(size_t)k * stride];
  }
  for (int64_t t = 0; t < nt; ++t) {
    float b[D];
    const int64_t tn = t + 1 < nt ? t + 1 : t;
#pragma unroll
    for (int k = 0; k < D; ++k) b[k] = p[(size_t)(tn * D + k) * stride];
#pragma unroll
    for (int k = 0; k < D; ++k) f(t * D + k, a[k]);
#pragma unroll
    for (int k = 0; k < D; ++k) a[k] = b[k];
  }
  for (int64_t j = nt * D; j < n; ++j) f(j, p[(size_t)j * stride]);
}

// f(j, p[j*stride], q[j*stride]) for j = 0, 1, ... in order until f returns true or j = n;
// returns whether f stopped the walk.  Rows of p and q are loaded in tiles of D with the next
// tile's loads in flight, as stream_rows.  f may store to q's row j (it has been read).
template <int D, class F>
__device__ __forceinline__ bool stream_rows_until(const float* __restrict__ p,
                                                  const float* q, size_t stride,
                                                  int64_t n, F&& f) {
  const int64_t nt = n / D;
  float a[D], c[D];
  if (nt > 0) {
#pragma unroll
    for (int k = 0; k < D; ++k) {
      a[k] = p[(size_t)k * stride];
      c[k] = q[(size_t)k * stride];
    }
  }
  for (int64_t t = 0; t < nt; ++t) {
    float b[D], d[D];
    const int64_t tn = t + 1 < nt ? t + 1 : t;  // issued on every tile, as in stream_rows
#pragma unroll
    for (int k = 0; k < D; ++k) {
      b[k] = p[(size_t)(tn * D + k) * stride];
      d[k] = q[(size_t)(tn * D + k) * stride];
    }
    bool stop = false;
#pragma unroll
    for (int k = 0; k < D; ++k)
      if (!stop) stop = f(t * D + k, a[k], c[k]);
    if (stop) return true;
#pragma unroll
    for (int k = 0; k < D; ++k) {
      a[k] = b[k];
      c[k] = d[k];
    }
  }
  for (int64_t j = nt * D; j < n; ++j)
    if (f(j, p[(size_t)j * stride], q[(size_t)j * stride])) return true;
  return false;
}

// Ballot of a bool over the active lanes: the lanes' compare mask itself (__ballot(int) goes
// through a 0/1 value in a VGPR and a compare, two VALU instructions more).
__device__ __forceinline__ unsigned long long wave_ballot(bool p) {
  return __builtin_amdgcn_ballot_w64(p);
}

__device__ __forceinline__ int wave_max_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, WAVE));
  return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
  return v;
}
__device__ __forceinline__ unsigned long long wave_sum_u64(unsigned long long v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
  return v;
}

__device__ __forceinline__ bool same_bits(float a, float b) {
  return __float_as_uint(a) == __float_as_uint(b);
}

}  // namespace lsh
