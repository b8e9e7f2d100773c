// Wave-specialised serial sweeps for few neurons (MI355X, gfx950).
//
// A serial recurrence over T steps for one block of 64 neurons is one chain of dependent steps.
// Run by a single wave, every instruction of a step (loads, address arithmetic, the surrogate's
// exp and division, stores) issues from that wave at 4 cycles per wave64 VALU instruction, so
// with few neurons the sweep is bound by one wave's issue rate while the rest of its CU idles.
// Here one workgroup per 64 neurons splits the work by role:
//   * PIPE_P producer waves load the inputs of a tile of PIPE_D rows one tile ahead, compute the
//     per-step coefficients (everything that does not depend on the recurrence) into an LDS
//     double buffer, and store the outputs of the tile the consumer finished one round earlier;
//   * one consumer wave (raised issue priority) runs only the recurrence, through LDS.
// One barrier per tile hands the buffers over.  The per-step arithmetic is the serial kernels'
// (same operations, same order, no contraction), so every output is bit-identical to theirs.
#include "lsh_abi.h"
#include "lsh_common.h"

namespace lsh {

// Every serial sweep of the library's serial entry points runs here, at every neuron count.
// Measured on MI355X (LIF adjoint, one wave -> pipe): N = 1024, T = 2^20: 172 -> 36.6 ms;
// N = 16384, T = 4096: 0.71 -> 0.26 ms; N = 65536, T = 4096: 1.13 -> 1.06 ms.

#ifndef LSH_PIPE_D
#define LSH_PIPE_D 64
#endif
// rows per tile of the adjoint, a multiple of 16 (LDS: 2 x D x 64 x 12 B).  96 rows measured
// 3 % faster at N = 1024, T = 2^20 (34.6 vs 35.7 ms) and no better at N = 16384.
constexpr int PIPE_D = LSH_PIPE_D;
constexpr int PIPE_P = 15;  // producer waves (16 waves per workgroup)
constexpr int PIPE_R = (PIPE_D + PIPE_P - 1) / PIPE_P;  // rows per producer per tile
// Rows per tile of the forward (LDS: 2 x D x 64 x 8 B = 128 KB).  Each tile costs a fixed
// ~0.35 us (barrier, load latency) besides ~14 ns per row at N = 1024: 32-row tiles were 28 %
// slower than 64-row ones, which longer tiles amortise further.
#ifndef LSH_PIPE_FD
#define LSH_PIPE_FD 128
#endif
constexpr int PIPE_FD = LSH_PIPE_FD;
constexpr int PIPE_FR = (PIPE_FD + PIPE_P - 1) / PIPE_P;

__device__ __forceinline__ int64_t pipe_tile_lo(int64_t T, int64_t k) {
  const int64_t hi = T - k * PIPE_D;
  return hi > PIPE_D ? hi - PIPE_D : 0;
}
__device__ __forceinline__ int pipe_tile_rows(int64_t T, int64_t k) {
  const int64_t hi = T - k * PIPE_D;
  return (int)(hi > PIPE_D ? PIPE_D : hi);
}

// Serial hard-reset LIF adjoint lam_t = b_t + a_t*lam_{t+1}, lam_T = 0 (triton_lif.py:54-72
// serial_bwd_kernel, :1088-1135 bwd_tiled_pf_kernel): tiles from the end of time, coefficients
// as k_lif_bwd's (v = fl(fl(beta*u_{t-1}) + x_t), sg = surrogate'(v - theta), J = 1 - s_t
// (+ (u_r - v)*sg when the reset is not detached), a = beta*J, b = gs*sg + J*gu).
template <bool DETACH, bool HAS_GU>
__global__ __launch_bounds__(WAVE*(PIPE_P + 1)) void k_lif_bwd_pipe(
    const float* __restrict__ I, const float* __restrict__ u0, const float* __restrict__ U,
    const float* __restrict__ S, const float* __restrict__ GS, const float* __restrict__ GU,
    float* __restrict__ Lam, int64_t N, int64_t T, float beta, float theta, float u_r,
    float alpha) {
  constexpr int D = PIPE_D, P = PIPE_P, R = PIPE_R;
  __shared__ float2 sAB[2][D][WAVE];
  __shared__ float sL[2][D][WAVE];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const unsigned lane = threadIdx.x % WAVE;
  const int64_t nb0 = (int64_t)blockIdx.x * WAVE;
  const bool valid = nb0 + lane < N;
  const unsigned ln = valid ? lane : (unsigned)(N - 1 - nb0);
  const unsigned lb = ln * 4u, sb = lane * 4u;
  const int64_t ntiles = (T + D - 1) / D;

  if (w == 0) {  // consumer: tile k - 1 in round k
    __builtin_amdgcn_s_setprio(3);
    float lam = 0.0f;
    for (int64_t k = 0; k <= ntiles + 1; ++k) {
      if (k >= 1 && k <= ntiles) {
        const int buf = (int)((k - 1) & 1);
        const int nr = pipe_tile_rows(T, k - 1);
        if (nr == D) {
#pragma unroll
          for (int g = D - 16; g >= 0; g -= 16) {
            float2 ab[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) ab[i] = sAB[buf][g + i][lane];
#pragma unroll
            for (int i = 15; i >= 0; --i) {
              lam = ab[i].y + ab[i].x * lam;
              sL[buf][g + i][lane] = lam;
            }
          }
        } else {
          for (int j = nr - 1; j >= 0; --j) {
            const float2 ab = sAB[buf][j][lane];
            lam = ab.y + ab.x * lam;
            sL[buf][j][lane] = lam;
          }
        }
      }
      __syncthreads();
    }
    return;
  }

  // producers: coefficients of tile k and the stores of tile k - 2 in round k
  const int p = w - 1;
  const float u0n = u0[nb0 + ln];
  float xr[R], sr[R], gr[R], hr[R], pr[R];
  auto load = [&](int64_t k) {
    const int64_t lo = pipe_tile_lo(T, k);
    const int nr = pipe_tile_rows(T, k);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int j = p + r * P;
      if (j < nr) {
        const int64_t t = lo + j;
        const size_t row = (size_t)t * (size_t)N + (size_t)nb0;
        xr[r] = ld_row(I + row, lb);
        sr[r] = ld_row(S + row, lb);
        gr[r] = ld_row(GS + row, lb);
        hr[r] = HAS_GU ? ld_row(GU + row, lb) : 0.0f;
        pr[r] = t > 0 ? ld_row(U + row - N, lb) : u0n;
      }
    }
  };
  if (ntiles > 0) load(0);
  for (int64_t k = 0; k <= ntiles + 1; ++k) {
    if (k < ntiles) {
      float x[R], s[R], g[R], h[R], up[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        x[r] = xr[r];
        s[r] = sr[r];
        g[r] = gr[r];
        h[r] = hr[r];
        up[r] = pr[r];
      }
      if (k + 1 < ntiles) load(k + 1);
      const int buf = (int)(k & 1);
      const int nr = pipe_tile_rows(T, k);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int j = p + r * P;
        if (j < nr) {
          const float v = lif_v(up[r], x[r], beta);
          const float sg = surrogate(v, theta, alpha);
          float J = 1.0f - s[r];
          if (!DETACH) J = J + (u_r - v) * sg;
          const float a = beta * J;
          const float bb = HAS_GU ? g[r] * sg + J * h[r] : g[r] * sg;
          sAB[buf][j][lane] = make_float2(a, bb);
        }
      }
    }
    if (k >= 2 && valid) {
      const int buf = (int)(k & 1);  // tile k - 2 has the parity of k
      const int64_t lo = pipe_tile_lo(T, k - 2);
      const int nr = pipe_tile_rows(T, k - 2);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int j = p + r * P;
        if (j < nr) st_row_nt(Lam + (size_t)(lo + j) * (size_t)N + (size_t)nb0, sb, sL[buf][j][lane]);
      }
    }
    __syncthreads();
  }
}

// The two serial forwards' steps: hard reset (triton_lif.py:21-25) and affine reset
// (triton_affine.py:20-24), with the one-wave kernels' arithmetic (lif_step, aff_step).
// spike(u, x): the step's threshold decision from the state before it, with the step's own
// operations (the producers recompute S with it).
struct LifStep {
  float beta, theta, u_r;
  __device__ __forceinline__ float operator()(float u, float x, bool& s) const {
    return lif_step(u, x, beta, theta, u_r, s);
  }
  __device__ __forceinline__ bool spike(float u, float x) const { return lif_v(u, x, beta) >= theta; }
};
struct AffStep {
  float beta, theta, gamma, delta;
  __device__ __forceinline__ float operator()(float u, float x, bool& s) const {
    return aff_step(u, x, beta, theta, gamma, delta, s);
  }
  __device__ __forceinline__ bool spike(float u, float x) const { return lif_v(u, x, beta) >= theta; }
};

// Serial forward from u0 (triton_lif.py:30-39 serial_fwd_kernel, :460-466
// serial_forward_tiled; triton_affine.py:143-162): tiles in time order; the consumer runs the
// step and writes u per step (and each tile's entry state), the producers stage I into LDS one
// tile ahead and store U, S of the tile finished one round earlier, recomputing each spike
// from the state before it and their own loaded rows (kept two rounds in registers) with the
// step's operations, so the consumer's chain carries no spike-to-float select.
template <class Step>
__global__ __launch_bounds__(WAVE*(PIPE_P + 1)) void k_serial_fwd_pipe(
    const float* __restrict__ I, const float* __restrict__ u0, float* __restrict__ U,
    float* __restrict__ S, int64_t N, int64_t T, Step step) {
  constexpr int D = PIPE_FD, P = PIPE_P, R = PIPE_FR;
  __shared__ float sX[2][D][WAVE];
  __shared__ float sU[2][D][WAVE];
  __shared__ float sEntry[2][WAVE];  // u before row 0 of the tile in the same buffer
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const unsigned lane = threadIdx.x % WAVE;
  const int64_t nb0 = (int64_t)blockIdx.x * WAVE;
  const bool valid = nb0 + lane < N;
  const unsigned ln = valid ? lane : (unsigned)(N - 1 - nb0);
  const unsigned lb = ln * 4u, sb = lane * 4u;
  const int64_t ntiles = (T + D - 1) / D;
  auto rows = [&](int64_t k) { return (int)(T - k * D > D ? D : T - k * D); };

  if (w == 0) {  // consumer: tile k - 1 in round k
    __builtin_amdgcn_s_setprio(3);
    float u = u0[nb0 + ln];
    for (int64_t k = 0; k <= ntiles + 1; ++k) {
      if (k >= 1 && k <= ntiles) {
        const int buf = (int)((k - 1) & 1);
        const int nr = rows(k - 1);
        sEntry[buf][lane] = u;
        if (nr == D) {
#pragma unroll
          for (int g = 0; g < D; g += 16) {
            float x[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) x[i] = sX[buf][g + i][lane];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              bool sp;
              u = step(u, x[i], sp);
              sU[buf][g + i][lane] = u;
            }
          }
        } else {
          for (int j = 0; j < nr; ++j) {
            bool sp;
            u = step(u, sX[buf][j][lane], sp);
            sU[buf][j][lane] = u;
          }
        }
      }
      __syncthreads();
    }
    return;
  }

  // producers: I of tile k into LDS (loaded one round ahead) and U, S of tile k - 2 in round k;
  // xr: the rows of the tile being loaded; at the start of round k, x1 and x2 hold this
  // producer's rows of tiles k - 1 and k - 2
  const int p = w - 1;
  float xr[R], x1[R], x2[R];
#pragma unroll
  for (int r = 0; r < R; ++r) xr[r] = x1[r] = x2[r] = 0.0f;
  auto load = [&](int64_t k) {
    const int nr = rows(k);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int j = p + r * P;
      if (j < nr) xr[r] = ld_row(I + (size_t)(k * D + j) * (size_t)N + (size_t)nb0, lb);
    }
  };
  if (ntiles > 0) load(0);
  for (int64_t k = 0; k <= ntiles + 1; ++k) {
    float xk[R];  // this producer's rows of tile k
#pragma unroll
    for (int r = 0; r < R; ++r) xk[r] = xr[r];
    if (k < ntiles) {
      const int buf = (int)(k & 1);
      const int nr = rows(k);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int j = p + r * P;
        if (j < nr) sX[buf][j][lane] = xr[r];
      }
      if (k + 1 < ntiles) load(k + 1);
    }
    if (k >= 2 && valid) {
      const int buf = (int)(k & 1);
      const int nr = rows(k - 2);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int j = p + r * P;
        if (j < nr) {
          const size_t row = (size_t)((k - 2) * D + j) * (size_t)N + (size_t)nb0;
          const float u = sU[buf][j][lane];
          const float up = j == 0 ? sEntry[buf][lane] : sU[buf][j - 1][lane];
          st_row_nt(U + row, sb, u);
          st_row_nt(S + row, sb, step.spike(up, x2[r]) ? 1.0f : 0.0f);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      x2[r] = x1[r];
      x1[r] = xk[r];
    }
    __syncthreads();
  }
}

void lif_serial_fwd_pipe(const float* I, const float* u0, float* U, float* S, int64_t N, int64_t T,
                         float beta, float theta, float u_r, hipStream_t st) {
  const int NB = (int)((N + WAVE - 1) / WAVE);
  hipLaunchKernelGGL((k_serial_fwd_pipe<LifStep>), dim3((unsigned)NB), dim3(WAVE * (PIPE_P + 1)), 0,
                     st, I, u0, U, S, N, T, LifStep{beta, theta, u_r});
}

void aff_serial_fwd_pipe(const float* I, const float* u0, float* U, float* S, int64_t N, int64_t T,
                         float beta, float theta, float gamma, float delta, hipStream_t st) {
  const int NB = (int)((N + WAVE - 1) / WAVE);
  hipLaunchKernelGGL((k_serial_fwd_pipe<AffStep>), dim3((unsigned)NB), dim3(WAVE * (PIPE_P + 1)), 0,
                     st, I, u0, U, S, N, T, AffStep{beta, theta, gamma, delta});
}

template <bool DETACH, bool HAS_GU>
static void launch_lif_bwd_pipe(const float* I, const float* u0, const float* U, const float* S,
                                const float* GS, const float* GU, float* Lam, int64_t N, int64_t T,
                                float beta, float theta, float u_r, float alpha, hipStream_t st) {
  const int NB = (int)((N + WAVE - 1) / WAVE);
  hipLaunchKernelGGL((k_lif_bwd_pipe<DETACH, HAS_GU>), dim3((unsigned)NB), dim3(WAVE * (PIPE_P + 1)),
                     0, st, I, u0, U, S, GS, GU, Lam, N, T, beta, theta, u_r, alpha);
}

void lif_serial_bwd_pipe(const float* I, const float* u0, const float* U, const float* S,
                         const float* GS, const float* GU, float* Lam, int64_t N, int64_t T,
                         float beta, float theta, float u_r, float alpha, bool detach,
                         hipStream_t st) {
  const bool gu = GU != nullptr;
  if (detach && gu)
    launch_lif_bwd_pipe<true, true>(I, u0, U, S, GS, GU, Lam, N, T, beta, theta, u_r, alpha, st);
  else if (detach)
    launch_lif_bwd_pipe<true, false>(I, u0, U, S, GS, GU, Lam, N, T, beta, theta, u_r, alpha, st);
  else if (gu)
    launch_lif_bwd_pipe<false, true>(I, u0, U, S, GS, GU, Lam, N, T, beta, theta, u_r, alpha, st);
  else
    launch_lif_bwd_pipe<false, false>(I, u0, U, S, GS, GU, Lam, N, T, beta, theta, u_r, alpha, st);
}

}  // namespace lsh
