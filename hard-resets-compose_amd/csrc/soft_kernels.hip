// Soft-reset LIF adjoint for MI355X (gfx950).  Reference: lifscan/triton_soft.py:214-221
// (soft_adjoint_fft), lifscan/triton_lif.py:1052-1069 and :1139-1210 (soft serial adjoints),
// lifscan/fit.py:93-149 (LIFSoftFn, LIFSoftScanFn).
//
// With the reset u = v - theta*s detached, du_t/dv_t = 1 and the adjoint is the constant-
// coefficient recurrence
//     lam_t = b_t + beta*lam_{t+1},   b_t = gS_t*alpha*sg_t*(1 - sg_t),  sg_t = sigmoid(alpha*(v_t - theta))
// (b_t in fp32 as the reference forms it).  The reference solves it by a float64 FFT convolution
// with beta^k; here it is solved directly in float64 (the convolution's exact value), stored as
// fp32: one reverse sweep per (chunk, neuron) lane, chunks chained by a sequential carry of
// float64 chunk offsets when T is long against N.  v_t comes from V, or is recomputed as
// fl(fl(beta*u_{t-1}) + x_t) from I, u0, U, the forward's own arithmetic.
// The soft-reset forward is the affine reset with gamma = 1, delta = -theta (affine_kernels.hip):
// fl(fl(1*v) + (-theta)) = fl(v - theta), the reference's single rounding.
#include "lsh_abi.h"
#include "lsh_common.h"

namespace lsh {

__device__ __forceinline__ float soft_b(float v, float gs, float theta, float alpha) {
  // the float64 adjoint (soft_adjoint_fft) keeps the library exp and the rounded division
  const float sg = sigmoid_neg_exact(alpha * (v - theta));
  return gs * alpha * sg * (1.0f - sg);
}

// COMPOSE: Q[m] = the chunk's offset (lam at its start for lam = 0 after its end).
// Otherwise: replay from lam_end[m] (0 for the last chunk / a single segment), store Lam, and
// with PS sum lam_t*u_{t-1} in fp64 (lam as stored) into one partials row per block.
template <bool FROM_V, bool COMPOSE, bool PS>
__global__ __launch_bounds__(64) void k_soft_bwd(const float* __restrict__ I,
                                                 const float* __restrict__ u0,
                                                 const float* __restrict__ U,
                                                 const float* __restrict__ V,
                                                 const float* __restrict__ GS,
                                                 const double* __restrict__ lam_end,
                                                 float* __restrict__ Lam, double* __restrict__ Q,
                                                 double* __restrict__ partials, int64_t N,
                                                 int64_t Ls, int NB, double beta, float beta32,
                                                 float theta, float alpha) {
  static_assert(!PS || (!FROM_V && !COMPOSE), "dbeta sums need u_{t-1}, in the replay");
  constexpr int D = 8;
  const int64_t m = blockIdx.x / NB;
  const int nb = (int)(blockIdx.x - m * NB);
  const int64_t n = (int64_t)nb * WAVE + threadIdx.x;
  double acc = 0.0;
  if (n < N) {
    double lam = (!COMPOSE && lam_end) ? lam_end[m * N + n] : 0.0;
    const int64_t t0 = m * Ls;
    const float u0n = FROM_V ? 0.0f : u0[n];
    auto row = [&](int64_t t) { return (size_t)t * (size_t)N + (size_t)n; };
    auto vb = [&](int64_t t, float& up) -> float {  // b_t, and u_{t-1}
      const size_t o = row(t);
      float v;
      if (FROM_V) {
        up = 0.0f;
        v = V[o];
      } else {
        up = t > 0 ? U[o - N] : u0n;
        v = lif_v(up, I[o], beta32);
      }
      return soft_b(v, GS[o], theta, alpha);
    };
    auto step = [&](int64_t t, float b, float up) {
      lam = (double)b + beta * lam;
      if (!COMPOSE) {
        const float l32 = (float)lam;
        st_nt(Lam + row(t), l32);
        if (PS) acc += (double)l32 * (double)up;
      }
    };
    const int64_t nt = Ls / D;
    // rows not covered by whole tiles (the top ones) first
    for (int64_t t = t0 + Ls - 1; t >= t0 + nt * D; --t) {
      float up;
      const float b = vb(t, up);
      step(t, b, up);
    }
    if (nt > 0) {
      float bb[D], uu[D];
#pragma unroll
      for (int k = 0; k < D; ++k) bb[k] = vb(t0 + (nt - 1) * D + k, uu[k]);
      for (int64_t g = nt - 1; g >= 0; --g) {
        float bn[D], un[D];
        if (g > 0) {
#pragma unroll
          for (int k = 0; k < D; ++k) bn[k] = vb(t0 + (g - 1) * D + k, un[k]);
        }
#pragma unroll
        for (int k = D - 1; k >= 0; --k) step(t0 + g * D + k, bb[k], uu[k]);
        if (g > 0) {
#pragma unroll
          for (int k = 0; k < D; ++k) {
            bb[k] = bn[k];
            uu[k] = un[k];
          }
        }
      }
    }
    if (COMPOSE) Q[m * N + n] = lam;
  }
  if (PS) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, WAVE);
    if (threadIdx.x == 0) partials[blockIdx.x] = acc;
  }
}

// Reverse carry over chunks: lam_end[m] = lam after chunk m; lam <- Q[m] + beta^C*lam.  The
// chunk offsets do not depend on lam, so they are loaded 8 chunks ahead.
__global__ __launch_bounds__(64) void k_soft_bwd_carry(const double* __restrict__ Q,
                                                       double* __restrict__ lam_end, int64_t N,
                                                       int M, double betaC) {
  constexpr int D = 8;
  const int64_t n = (int64_t)blockIdx.x * WAVE + threadIdx.x;
  if (n >= N) return;
  auto row = [&](int m) { return (size_t)m * (size_t)N + (size_t)n; };
  double lam = 0.0;
  int m = M - 1;
  for (; m >= D - 1; m -= D) {
    double q[D];
#pragma unroll
    for (int k = 0; k < D; ++k) q[k] = Q[row(m - k)];
#pragma unroll
    for (int k = 0; k < D; ++k) {
      lam_end[row(m - k)] = lam;
      lam = q[k] + betaC * lam;
    }
  }
  for (; m >= 0; --m) {
    lam_end[row(m)] = lam;
    lam = Q[row(m)] + betaC * lam;
  }
}

static int soft_bwd_check(int64_t T, int64_t N, int C) {
  if (T < 0 || N < 0 || N > (int64_t)1 << 31) return LSH_ERR_SHAPE;
  if (C < 1) return LSH_ERR_SHAPE;
  if (T % C != 0) return LSH_ERR_DIVISIBILITY;
  if ((T / C) * ((N + WAVE - 1) / WAVE) > ((int64_t)1 << 31) - 1) return LSH_ERR_SHAPE;
  return LSH_OK;
}

template <bool FROM_V, bool COMPOSE, bool PS>
static void launch_soft(const float* I, const float* u0, const float* U, const float* V,
                        const float* GS, const double* lam_end, float* Lam, double* Q,
                        double* partials, int64_t N, int64_t Ls, int64_t M, double beta,
                        float theta, float alpha, hipStream_t st) {
  const int NB = (int)((N + WAVE - 1) / WAVE);
  hipLaunchKernelGGL((k_soft_bwd<FROM_V, COMPOSE, PS>), dim3((unsigned)(M * NB)), dim3(WAVE), 0, st,
                     I, u0, U, V, GS, lam_end, Lam, Q, partials, N, Ls, NB, beta, (float)beta,
                     theta, alpha);
}

template <bool FROM_V, bool PS>
static int soft_bwd(const float* I, const float* u0, const float* U, const float* V,
                    const float* GS, float* Lam, double* partials, int64_t T, int64_t N,
                    double beta, float theta, float alpha, int C, void* ws, hipStream_t st) {
  const int64_t M = T / C;
  if (M == 1) {
    launch_soft<FROM_V, false, PS>(I, u0, U, V, GS, nullptr, Lam, nullptr, partials, N, T, 1, beta,
                                   theta, alpha, st);
    return LSH_OK;
  }
  const size_t mn = align_up((size_t)M * (size_t)N * 8, 256);
  char* w = static_cast<char*>(ws) + kWsHeaderBytes;
  double* Q = reinterpret_cast<double*>(w);
  double* LE = reinterpret_cast<double*>(w + mn);
  double betaC = 1.0;
  for (int j = 0; j < C; ++j) betaC *= beta;
  launch_soft<FROM_V, true, false>(I, u0, U, V, GS, nullptr, nullptr, Q, nullptr, N, C, M, beta,
                                   theta, alpha, st);
  hipLaunchKernelGGL(k_soft_bwd_carry, dim3((unsigned)((N + WAVE - 1) / WAVE)), dim3(WAVE), 0, st, Q,
                     LE, N, (int)M, betaC);
  launch_soft<FROM_V, false, PS>(I, u0, U, V, GS, LE, Lam, nullptr, partials, N, C, M, beta, theta,
                                 alpha, st);
  return LSH_OK;
}

}  // namespace lsh

using namespace lsh;

extern "C" size_t lsh_soft_bwd_workspace(int64_t T, int64_t N, int C) {
  if (soft_bwd_check(T, N, C) != LSH_OK) return 0;
  const int64_t M = T / C;
  if (M <= 1) return kWsHeaderBytes;
  return kWsHeaderBytes + 2 * align_up((size_t)M * (size_t)N * 8, 256);
}

extern "C" int64_t lsh_soft_bwd_partials(int64_t T, int64_t N, int C) {
  if (soft_bwd_check(T, N, C) != LSH_OK) return -1;
  return (T / C) * ((N + WAVE - 1) / WAVE);
}

extern "C" int lsh_soft_bwd(const float* I, const float* u0, const float* U, const float* V,
                            const float* GS, float* Lam, double* partials, int64_t T, int64_t N,
                            double beta, float theta, float alpha, int C, void* ws,
                            size_t ws_bytes, void* stream) {
  const bool from_v = V != nullptr;
  if (bad_ptr(GS) || bad_ptr(Lam)) return LSH_ERR_ARG;
  if (!from_v && (bad_ptr(I) || bad_ptr(u0) || bad_ptr(U))) return LSH_ERR_ARG;
  if (from_v && partials) return LSH_ERR_ARG;  // dbeta needs u_{t-1}
  const int rc = soft_bwd_check(T, N, C);
  if (rc != LSH_OK) return rc;
  if (T / C > 1 && (bad_ptr(ws) || ws_bytes < lsh_soft_bwd_workspace(T, N, C) ||
                    (reinterpret_cast<uintptr_t>(ws) & 255u) != 0))
    return LSH_ERR_WORKSPACE;
  if (T == 0 || N == 0) return LSH_OK;
  hipStream_t st = (hipStream_t)stream;
  int r;
  if (from_v)
    r = soft_bwd<true, false>(I, u0, U, V, GS, Lam, nullptr, T, N, beta, theta, alpha, C, ws, st);
  else if (partials)
    r = soft_bwd<false, true>(I, u0, U, V, GS, Lam, partials, T, N, beta, theta, alpha, C, ws, st);
  else
    r = soft_bwd<false, false>(I, u0, U, V, GS, Lam, nullptr, T, N, beta, theta, alpha, C, ws, st);
  if (r != LSH_OK) return r;
  LSH_CHECK_LAUNCH();
  return LSH_OK;
}
