// Single-pass fused scans for MI355X: one workgroup owns a block of 64 neurons and walks
// the time axis in rounds of W chunks, one chunk per wave.  Inputs are read from HBM once;
// everything that crosses chunks (maps, chunk ends, affine aggregates) goes through LDS, so
// no workgroup waits on another one.
//
// Forward (exact, i.e. the reference's two-level scan with repair run to convergence,
// triton_lif.py:782-817):
//   1. each wave loads its chunk's C inputs into registers and builds the chunk's
//      capacity-K map (the same fold as triton_lif.py:737-779, hi-pruned) into LDS;
//   2. each wave evaluates the maps of the earlier chunks of the round, from the round's
//      exact entry state, to a speculative entry state, and replays its chunk (compute only)
//      to a speculative exit state;
//   3. exact exit states are handed from wave to wave through an LDS flag chain: a wave whose
//      speculative entry equals the exact one (bit for bit) passes its speculative exit on at
//      once, otherwise it replays from the exact entry first;
//   4. every wave replays its chunk from the exact entry once more, storing U and S.
//   The stored trajectory is therefore the serial recurrence bit for bit; the maps decide
//   only how long the hand-off chain waits.
// Backward (the affine scan of triton_lif.py:512-526 in one pass): each wave turns its chunk
// into per-step coefficients (a_t, b_t) kept in registers, composes them to (P, Q) in LDS,
// takes the adjoint at its chunk end from the later chunks' aggregates, and replays.
#include "lsh_abi.h"
#include "lsh_common.h"
#include "lsh_map.h"

namespace lsh {

// Bounded LDS spin: waits until *flag == want.  The chain cannot deadlock (wave 0 never
// waits), so the bound only guarantees termination if that reasoning were ever broken.
__device__ __forceinline__ bool lds_wait(int* flag, int want) {
  for (int it = 0; it < (1 << 24); ++it) {
    if (__hip_atomic_load(flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) == want) return true;
    __builtin_amdgcn_s_sleep(1);
  }
  return false;
}

// SO (starts only): U is [M, N] and receives each chunk's exact entry state instead of the
// trajectory, S as usual; the adjoint recomputes the trajectory from those states
// (k_lif_bwd_fused<..., RC = true>), so the forward writes 4 B per neuron-step instead of 8.
template <int KMAX, int C, int W, bool SPEC, bool SO = false>
__global__ __launch_bounds__(WAVE* W) void k_lif_fwd_fused(const float* __restrict__ I,
                                                           const float* __restrict__ u0,
                                                           float* __restrict__ U,
                                                           float* __restrict__ S, WsHeader* hdr,
                                                           int64_t N, int M, int K, float beta,
                                                           float theta, float u_r) {
  constexpr int KL = SPEC ? KMAX : 1;
  __shared__ float sA[W][WAVE], sB[W][WAVE];
  __shared__ float sXd[W][KL][WAVE], sCd[W][KL][WAVE];
  __shared__ int sCnt[W][WAVE];
  __shared__ float sEnd[W][WAVE];
  __shared__ float sStart[WAVE];
  __shared__ int sFlag[W];

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const unsigned lane = threadIdx.x % WAVE;
  const int64_t nb0 = (int64_t)blockIdx.x * WAVE;
  const bool valid = nb0 + lane < N;
  // inactive lanes of the last block read a valid column and store nothing
  const unsigned ln = valid ? lane : (unsigned)(N - 1 - nb0);
  const unsigned lb = ln * 4u, sb = lane * 4u;  // load / store byte offsets within a row
  const float* __restrict__ Ib = I + nb0;
  float* __restrict__ Ub = U + nb0;
  float* __restrict__ Sb = S + nb0;
  const float hi = fmaxf(u0[nb0 + ln], fmaxf(theta, u_r));
  if (w == 0) sStart[lane] = u0[nb0 + ln];
  if (lane == 0) sFlag[w] = 0;
  __syncthreads();

  unsigned long long fixups = 0, unknown = 0;
  unsigned int timeouts = 0;
  const int rounds = (M + W - 1) / W;
  const unsigned rstride = (unsigned)(N * 4);  // bytes per time row (C*N*4 < 2^31 checked on host)
  // Without speculation the round's inputs are loaded one round ahead (xn), so the loads of
  // round r+1 are in flight during round r's hand-off chain (barriers wait on LDS only).
  float x[C], xn[SPEC ? 1 : C];
  if (!SPEC && w < M) {
    const Buf bi(Ib + (size_t)w * C * N);
#pragma unroll
    for (int j = 0; j < C; ++j) x[j] = bi.ld(lb, j * rstride);
  }
  for (int r = 0; r < rounds; ++r) {
    const int m = r * W + w;
    const bool active = m < M;  // wave-uniform
    const size_t row0 = (size_t)m * C;
    if (!SPEC && m + W < M) {
      const Buf bn(Ib + (row0 + (size_t)W * C) * N);
#pragma unroll
      for (int j = 0; j < C; ++j) xn[j] = bn.ld(lb, j * rstride);
    }
    if (active) {
      if (SPEC) {
        const Buf bi(Ib + row0 * N);
#pragma unroll
        for (int j = 0; j < C; ++j) x[j] = bi.ld(lb, j * rstride);
        MapBuilder<KMAX> mb;
        mb.init();
#pragma unroll
        for (int j = 0; j < C; ++j) mb.step(x[j], beta, theta, u_r, hi, K);
        sA[w][lane] = mb.A;
        sB[w][lane] = mb.B;
        sCnt[w][lane] = mb.cnt | (mb.ovf ? (1 << 16) : 0);
#pragma unroll
        for (int i = 0; i < KL; ++i) {
          sXd[w][i][lane] = mb.xd[i];
          sCd[w][i][lane] = mb.cd[i];
        }
      }
    }
    __syncthreads();
    float e = 0.0f;
    if (active) {
      // (2) speculative entry through the earlier chunks' maps, speculative exit
      float u_spec = sStart[lane];
      bool known = SPEC;
      float e_spec = 0.0f;
      if (SPEC) {
        for (int v = 0; v < w; ++v) {
          const int cw = sCnt[v][lane];
          const int cnt = cw & 0xffff;
          int k = 0;
#pragma unroll
          for (int i = 0; i < KL; ++i) k += (i < cnt && sXd[v][i][lane] > u_spec) ? 1 : 0;
          float cval = 0.0f;
#pragma unroll
          for (int i = 0; i < KL; ++i) cval = (i == k) ? sCd[v][i][lane] : cval;
          if (k == cnt) {
            if (cw >> 16) known = false;  // overflowed map, state below its stored pieces
            u_spec = __fadd_rn(__fmul_rn(sA[v][lane], u_spec), sB[v][lane]);
          } else {
            u_spec = cval;
          }
        }
        e_spec = u_spec;
#pragma unroll
        for (int j = 0; j < C; ++j) {
          bool s;
          e_spec = lif_step(e_spec, x[j], beta, theta, u_r, s);
        }
      }
      // (3) exact entry from the previous wave of the chain
      float start;
      if (w == 0) {
        start = sStart[lane];
      } else {
        if (!lds_wait(&sFlag[w - 1], r + 1)) ++timeouts;
        start = sEnd[w - 1][lane];
      }
      const bool hit = known && same_bits(u_spec, start);
      if (hit) {
        e = e_spec;
      } else {
        e = start;
#pragma unroll
        for (int j = 0; j < C; ++j) {
          bool s;
          e = lif_step(e, x[j], beta, theta, u_r, s);
        }
      }
      sEnd[w][lane] = e;
      if (lane == 0)
        __hip_atomic_store(&sFlag[w], r + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
      fixups += (SPEC && known && !hit && valid) ? 1ull : 0ull;
      unknown += (SPEC && !known && valid) ? 1ull : 0ull;
      // (4) the stored trajectory, from the exact entry
      if (valid && SO) {
        U[(size_t)m * N + nb0 + lane] = start;
        const Buf bs(Sb + row0 * N);
        float u = start;
#pragma unroll
        for (int j = 0; j < C; ++j) {
          bool s;
          u = lif_step(u, x[j], beta, theta, u_r, s);
          bs.st_nt(sb, j * rstride, s ? 1.0f : 0.0f);
        }
      } else if (valid) {
        const Buf bu(Ub + row0 * N), bs(Sb + row0 * N);
        float u = start;
#pragma unroll
        for (int j = 0; j < C; ++j) {
          bool s;
          u = lif_step(u, x[j], beta, theta, u_r, s);
          bu.st_nt(sb, j * rstride, u);
          bs.st_nt(sb, j * rstride, s ? 1.0f : 0.0f);
        }
      }
    }
    __syncthreads();
    const int last = min(W, M - r * W) - 1;
    if (w == last) sStart[lane] = e;
    __syncthreads();
    if (!SPEC && m + W < M) {
#pragma unroll
      for (int j = 0; j < C; ++j) x[j] = xn[j];
    }
  }
  fixups = wave_sum_u64(fixups);
  unknown = wave_sum_u64(unknown);
  if (lane == 0 && hdr != nullptr) {  // the starts-only forward may run without counters
    if (fixups) atomicAdd(&hdr->fused_fixups, fixups);
    if (unknown) atomicAdd(&hdr->fused_unknown, unknown);
    if (timeouts) atomicAdd(&hdr->spin_timeouts, timeouts);
  }
}

// PS (detached, no GU) also sums parameter gradients in fp64 (u_{t-1} and the spike bits of
// the chunk stay in registers) and writes one partials row per workgroup:
//   PS == 1, hard reset (fit.py:43-47): sum lam_t*u_{t-1}, sum gs_t*sg_t, sum s_t*lam_{t+1};
//   PS == 2, affine reset u <- gamma*v + delta (triton_affine.py:229-242), `u_r` carrying
//            gamma (a detached reset needs no u_r): J_t = s_t ? gamma : 1, and the sums
//            lam_t*u_{t-1}, s_t*v_t*lam_{t+1}, s_t*lam_{t+1}.  a_t = beta*J_t follows from
//            the spike bit, so v_t takes the registers a_t would.
// RC (recompute, detached, no GU): U is the [M, N] array of chunk entry states written by the
// SO forward and S is not read; the wave replays its chunk's forward from the entry state in
// registers (the forward's own arithmetic, so u_{t-1} and s_t are the forward's bits) while it
// forms the coefficients: 8 B read per neuron-step instead of 16.
template <int C, int W, bool DETACH, bool HAS_GU, int PS = 0, bool RC = false>
__global__ __launch_bounds__(WAVE* W) void k_lif_bwd_fused(
    const float* __restrict__ I, const float* __restrict__ u0, const float* __restrict__ U,
    const float* __restrict__ S, const float* __restrict__ GS, const float* __restrict__ GU,
    float* __restrict__ Lam, double* __restrict__ partials, int64_t N, int M, float beta,
    float theta, float u_r, float alpha) {
  static_assert(!PS || (DETACH && !HAS_GU && C <= 64), "parameter sums: detached, no GU");
  static_assert(!RC || (DETACH && !HAS_GU && PS != 2), "recompute: hard reset, detached, no GU");
  constexpr bool AFF = PS == 2;
  __shared__ float sP[W][WAVE], sQ[W][WAVE];
  __shared__ float sLam[WAVE];
  __shared__ double sAcc[PS ? W : 1][3];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const unsigned lane = threadIdx.x % WAVE;
  const int64_t nb0 = (int64_t)blockIdx.x * WAVE;
  const bool valid = nb0 + lane < N;
  const unsigned ln = valid ? lane : (unsigned)(N - 1 - nb0);
  const unsigned lb = ln * 4u, sb = lane * 4u;
  const float* __restrict__ Ib = I + nb0;
  const float* __restrict__ Sb = S + nb0;
  const float* __restrict__ Gb = GS + nb0;
  const float* __restrict__ Hb = HAS_GU ? GU + nb0 : nullptr;
  const float* __restrict__ Ub = U + nb0;
  float* __restrict__ Lb = Lam + nb0;
  const float u0n = u0[nb0 + ln];
  double acc_b = 0.0, acc_t = 0.0, acc_r = 0.0;
  const float gbeta = beta * u_r;  // AFF: beta*gamma
  if (w == 0) sLam[lane] = 0.0f;
  __syncthreads();
  const int rounds = (M + W - 1) / W;
  for (int r = 0; r < rounds; ++r) {
    const int m = M - 1 - (r * W + w);  // wave 0 holds the latest chunk of the round
    const bool active = m >= 0;
    float a[AFF ? 1 : C], b[C];
    float upk[PS ? C : 1];
    float vpk[AFF ? C : 1];
    unsigned long long sbits = 0;
    float lam = 0.0f;
    const size_t row0 = (size_t)(active ? m : 0) * C;
    const unsigned rstride = (unsigned)(N * 4);
    if (active) {
      const Buf bi(Ib + row0 * N), bs_(Sb + row0 * N), bg(Gb + row0 * N), bp(Ub + row0 * N);
      // state before the chunk's first step: the previous chunk's last U row, or u0 (RC: the
      // stored entry state of the chunk)
      const float up0 = RC ? U[(size_t)m * N + nb0 + ln]
                           : (row0 > 0 ? ld_row(Ub + (row0 - 1) * N, lb) : u0n);
      float ur = up0;  // RC: the recomputed state
#pragma unroll
      for (int j = 0; j < C; ++j) {
        const unsigned so = j * rstride;
        const float x = bi.ld(lb, so);
        float s, up;
        if constexpr (RC) {
          up = ur;
          bool sb_;
          ur = lif_step(ur, x, beta, theta, u_r, sb_);
          s = sb_ ? 1.0f : 0.0f;
        } else {
          s = bs_.ld(lb, so);
        }
        const float gs = bg.ld(lb, so);
        if constexpr (!RC) up = j == 0 ? up0 : bp.ld(lb, so - rstride);
        const float v = lif_v(up, x, beta);
        const float sg = surrogate(v, theta, alpha);
        float J = 1.0f - s;
        if (!DETACH) J = J + (u_r - v) * sg;
        if constexpr (!AFF) a[j] = beta * J;
        b[j] = HAS_GU ? gs * sg + J * Buf(Hb + row0 * N).ld(lb, so) : gs * sg;
        if (PS) {
          upk[j] = up;
          if (s != 0.0f) sbits |= 1ull << j;
          if (PS == 1 && valid) acc_t += (double)b[j];
          if constexpr (AFF) vpk[j] = v;
        }
      }
      float P = 1.0f, Q = 0.0f;
#pragma unroll
      for (int j = C - 1; j >= 0; --j) {
        if constexpr (AFF) {
          const float aa = ((sbits >> j) & 1ull) ? gbeta : beta;
          Q = b[j] + aa * Q;
          P = aa * P;
        } else {
          Q = b[j] + a[j] * Q;
          P = a[j] * P;
        }
      }
      sP[w][lane] = P;
      sQ[w][lane] = Q;
    }
    __syncthreads();
    if (active) {
      lam = sLam[lane];
      for (int v = 0; v < w; ++v) lam = sQ[v][lane] + sP[v][lane] * lam;
      const Buf bl(Lb + row0 * N);
#pragma unroll
      for (int j = C - 1; j >= 0; --j) {
        const float lam_next = lam;
        if constexpr (AFF)
          lam = b[j] + (((sbits >> j) & 1ull) ? gbeta : beta) * lam;
        else
          lam = b[j] + a[j] * lam;
        if (valid) {
          bl.st_nt(sb, j * rstride, lam);
          if (PS) {
            acc_b += (double)lam * (double)upk[j];
            if ((sbits >> j) & 1ull) {
              acc_r += (double)lam_next;
              if constexpr (AFF) acc_t += (double)vpk[j] * (double)lam_next;
            }
          }
        }
      }
    }
    __syncthreads();
    const int last = min(W, M - r * W) - 1;
    if (w == last) sLam[lane] = lam;
    __syncthreads();
  }
  if (PS) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      acc_b += __shfl_xor(acc_b, o, WAVE);
      acc_t += __shfl_xor(acc_t, o, WAVE);
      acc_r += __shfl_xor(acc_r, o, WAVE);
    }
    if (lane == 0) {
      sAcc[w][0] = acc_b;
      sAcc[w][1] = acc_t;
      sAcc[w][2] = acc_r;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      double tb = 0.0, tt = 0.0, tr = 0.0;
      for (int v = 0; v < W; ++v) {
        tb += sAcc[v][0];
        tt += sAcc[v][1];
        tr += sAcc[v][2];
      }
      double* out = partials + (size_t)blockIdx.x * 3;
      out[0] = tb;
      out[1] = tt;
      out[2] = tr;
    }
  }
}

// ---------------------------------------------------------------------------------------
template <int KMAX, int C, int W, bool SPEC, bool SO = false>
static void launch_fwd_fused(const float* I, const float* u0, float* U, float* S, WsHeader* h,
                             int64_t N, int M, int K, float beta, float theta, float u_r,
                             hipStream_t st) {
  const int NB = (int)((N + WAVE - 1) / WAVE);
  hipLaunchKernelGGL((k_lif_fwd_fused<KMAX, C, W, SPEC, SO>), dim3((unsigned)NB), dim3(WAVE * W), 0,
                     st, I, u0, U, S, h, N, M, K, beta, theta, u_r);
}

// The chunked-serial exact forward (no maps) writing S and the chunk entry states only.
template <int C>
static void fwd_starts_c(const float* I, const float* u0, float* STARTS, float* S, WsHeader* h,
                         int64_t N, int M, float beta, float theta, float u_r, hipStream_t st) {
  constexpr int WMAX = C <= 32 ? 16 : (C == 64 ? 8 : 4);
  const int W = fused_waves((N + WAVE - 1) / WAVE, WMAX);
  if constexpr (WMAX >= 16) {
    if (W == 16) {
      launch_fwd_fused<1, C, 16, false, true>(I, u0, STARTS, S, h, N, M, 1, beta, theta, u_r, st);
      return;
    }
  }
  if constexpr (WMAX >= 8) {
    if (W == 8) {
      launch_fwd_fused<1, C, 8, false, true>(I, u0, STARTS, S, h, N, M, 1, beta, theta, u_r, st);
      return;
    }
  }
  launch_fwd_fused<1, C, 4, false, true>(I, u0, STARTS, S, h, N, M, 1, beta, theta, u_r, st);
}

template <int C, bool SPEC>
static int fwd_fused_k(const float* I, const float* u0, float* U, float* S, WsHeader* h, int64_t N,
                       int M, int K, float beta, float theta, float u_r, hipStream_t st) {
  if (!SPEC) {
    // registers allow 16 waves up to C = 32, 8 at C = 64
    constexpr int WMAX = C <= 32 ? 16 : (C == 64 ? 8 : 4);
    const int W = fused_waves((N + WAVE - 1) / WAVE, WMAX);
    if constexpr (WMAX >= 16) {
      if (W == 16) {
        launch_fwd_fused<1, C, 16, false>(I, u0, U, S, h, N, M, K, beta, theta, u_r, st);
        return LSH_OK;
      }
    }
    if constexpr (WMAX >= 8) {
      if (W == 8) {
        launch_fwd_fused<1, C, 8, false>(I, u0, U, S, h, N, M, K, beta, theta, u_r, st);
        return LSH_OK;
      }
    }
    launch_fwd_fused<1, C, 4, false>(I, u0, U, S, h, N, M, K, beta, theta, u_r, st);
  } else if (K <= 4) {  // map speculation keeps the maps of a round in LDS: 4 waves
    launch_fwd_fused<4, C, 4, true>(I, u0, U, S, h, N, M, K, beta, theta, u_r, st);
  } else if (K <= 8) {
    launch_fwd_fused<8, C, 4, true>(I, u0, U, S, h, N, M, K, beta, theta, u_r, st);
  } else if (K <= 16) {
    launch_fwd_fused<16, C, 4, true>(I, u0, U, S, h, N, M, K, beta, theta, u_r, st);
  } else {
    return LSH_ERR_SHAPE;
  }
  return LSH_OK;
}

template <bool SPEC>
static int fwd_fused(const float* I, const float* u0, float* U, float* S, WsHeader* h, int64_t N,
                     int M, int C, int K, float beta, float theta, float u_r, hipStream_t st) {
  switch (C) {
    case 16: return fwd_fused_k<16, SPEC>(I, u0, U, S, h, N, M, K, beta, theta, u_r, st);
    case 32: return fwd_fused_k<32, SPEC>(I, u0, U, S, h, N, M, K, beta, theta, u_r, st);
    case 64: return fwd_fused_k<64, SPEC>(I, u0, U, S, h, N, M, K, beta, theta, u_r, st);
    case 128: return fwd_fused_k<128, SPEC>(I, u0, U, S, h, N, M, K, beta, theta, u_r, st);
    default: return LSH_ERR_SHAPE;
  }
}

template <int C, int W, bool DETACH, bool HAS_GU>
static void launch_bwd_fused(const float* I, const float* u0, const float* U, const float* S,
                             const float* GS, const float* GU, float* Lam, int64_t N, int M,
                             float beta, float theta, float u_r, float alpha, hipStream_t st) {
  const int NB = (int)((N + WAVE - 1) / WAVE);
  hipLaunchKernelGGL((k_lif_bwd_fused<C, W, DETACH, HAS_GU>), dim3((unsigned)NB), dim3(WAVE * W), 0,
                     st, I, u0, U, S, GS, GU, Lam, nullptr, N, M, beta, theta, u_r, alpha);
}

template <int C, int W>
static void bwd_fused_cw(const float* I, const float* u0, const float* U, const float* S,
                         const float* GS, const float* GU, float* Lam, int64_t N, int M, float beta,
                         float theta, float u_r, float alpha, bool detach, hipStream_t st) {
  if (detach) {
    if (GU)
      launch_bwd_fused<C, W, true, true>(I, u0, U, S, GS, GU, Lam, N, M, beta, theta, u_r, alpha, st);
    else
      launch_bwd_fused<C, W, true, false>(I, u0, U, S, GS, GU, Lam, N, M, beta, theta, u_r, alpha, st);
  } else {
    if (GU)
      launch_bwd_fused<C, W, false, true>(I, u0, U, S, GS, GU, Lam, N, M, beta, theta, u_r, alpha, st);
    else
      launch_bwd_fused<C, W, false, false>(I, u0, U, S, GS, GU, Lam, N, M, beta, theta, u_r, alpha,
                                           st);
  }
}

template <int C>
static void bwd_fused_c(const float* I, const float* u0, const float* U, const float* S,
                        const float* GS, const float* GU, float* Lam, int64_t N, int M, float beta,
                        float theta, float u_r, float alpha, bool detach, hipStream_t st) {
  // registers allow 16 waves at C = 16, 8 at C = 32
  constexpr int WMAX = C == 16 ? 16 : (C == 32 ? 8 : 4);
  const int W = fused_waves((N + WAVE - 1) / WAVE, WMAX);
  if constexpr (WMAX >= 16) {
    if (W == 16) {
      bwd_fused_cw<C, 16>(I, u0, U, S, GS, GU, Lam, N, M, beta, theta, u_r, alpha, detach, st);
      return;
    }
  }
  if constexpr (WMAX >= 8) {
    if (W == 8) {
      bwd_fused_cw<C, 8>(I, u0, U, S, GS, GU, Lam, N, M, beta, theta, u_r, alpha, detach, st);
      return;
    }
  }
  bwd_fused_cw<C, 4>(I, u0, U, S, GS, GU, Lam, N, M, beta, theta, u_r, alpha, detach, st);
}

// Recomputing adjoint (RC): chunk entry states instead of U and S; ps 0 plain, ps 1 with the
// fit.py parameter sums.
template <int C, int W>
static void launch_bwd_rc(const float* I, const float* STARTS, const float* GS, float* Lam,
                          double* partials, int64_t N, int M, float beta, float theta, float u_r,
                          float alpha, hipStream_t st) {
  const int NB = (int)((N + WAVE - 1) / WAVE);
  if (partials)
    hipLaunchKernelGGL((k_lif_bwd_fused<C, W, true, false, 1, true>), dim3((unsigned)NB),
                       dim3(WAVE * W), 0, st, I, STARTS, STARTS, nullptr, GS, nullptr, Lam, partials,
                       N, M, beta, theta, u_r, alpha);
  else
    hipLaunchKernelGGL((k_lif_bwd_fused<C, W, true, false, 0, true>), dim3((unsigned)NB),
                       dim3(WAVE * W), 0, st, I, STARTS, STARTS, nullptr, GS, nullptr, Lam, nullptr,
                       N, M, beta, theta, u_r, alpha);
}

template <int C>
static void bwd_rc_c(const float* I, const float* STARTS, const float* GS, float* Lam,
                     double* partials, int64_t N, int M, float beta, float theta, float u_r,
                     float alpha, hipStream_t st) {
  // registers as the plain adjoint (with the sums as the parameter variant)
  constexpr int WMAX = C == 16 ? 16 : (C == 32 ? 8 : 4);
  const int wmax = partials ? (C <= 32 ? 8 : 4) : WMAX;
  const int W = fused_waves((N + WAVE - 1) / WAVE, wmax);
  if constexpr (WMAX >= 16) {
    if (W == 16) {
      launch_bwd_rc<C, 16>(I, STARTS, GS, Lam, partials, N, M, beta, theta, u_r, alpha, st);
      return;
    }
  }
  if constexpr (WMAX >= 8) {
    if (W == 8) {
      launch_bwd_rc<C, 8>(I, STARTS, GS, Lam, partials, N, M, beta, theta, u_r, alpha, st);
      return;
    }
  }
  launch_bwd_rc<C, 4>(I, STARTS, GS, Lam, partials, N, M, beta, theta, u_r, alpha, st);
}

template <int C, int W>
static void launch_param_fused(const float* I, const float* u0, const float* U, const float* S,
                               const float* GS, float* Lam, double* partials, int64_t N, int M,
                               float beta, float theta, float u_r, float alpha, int ps,
                               hipStream_t st) {
  const int NB = (int)((N + WAVE - 1) / WAVE);
  if (ps == 2)
    hipLaunchKernelGGL((k_lif_bwd_fused<C, W, true, false, 2>), dim3((unsigned)NB), dim3(WAVE * W), 0,
                       st, I, u0, U, S, GS, nullptr, Lam, partials, N, M, beta, theta, u_r, alpha);
  else
    hipLaunchKernelGGL((k_lif_bwd_fused<C, W, true, false, 1>), dim3((unsigned)NB), dim3(WAVE * W), 0,
                       st, I, u0, U, S, GS, nullptr, Lam, partials, N, M, beta, theta, u_r, alpha);
}

template <int C>
static void param_fused_c(const float* I, const float* u0, const float* U, const float* S,
                          const float* GS, float* Lam, double* partials, int64_t N, int M, float beta,
                          float theta, float u_r, float alpha, int ps, hipStream_t st) {
  // u_{t-1} kept per step: 8 waves up to C = 32
  constexpr int WMAX = C <= 32 ? 8 : 4;
  const int W = fused_waves((N + WAVE - 1) / WAVE, WMAX);
  if constexpr (WMAX >= 8) {
    if (W == 8) {
      launch_param_fused<C, 8>(I, u0, U, S, GS, Lam, partials, N, M, beta, theta, u_r, alpha, ps, st);
      return;
    }
  }
  launch_param_fused<C, 4>(I, u0, U, S, GS, Lam, partials, N, M, beta, theta, u_r, alpha, ps, st);
}

int lif_param_bwd_fused(const float* I, const float* u0, const float* U, const float* S,
                        const float* GS, float* Lam, double* partials, int64_t T, int64_t N,
                        float beta, float theta, float u_r, float alpha, int C, int ps,
                        hipStream_t st) {
  if (T < 0 || N < 0 || N > (int64_t)1 << 31) return LSH_ERR_SHAPE;
  if (C != 16 && C != 32 && C != 64) return LSH_ERR_SHAPE;
  if (T % C != 0) return LSH_ERR_DIVISIBILITY;
  if ((uint64_t)N * (uint64_t)C * 4u >= ((uint64_t)1 << 32)) return LSH_ERR_SHAPE;
  if (T == 0 || N == 0) return LSH_OK;
  const int M = (int)(T / C);
  switch (C) {
    case 16:
      param_fused_c<16>(I, u0, U, S, GS, Lam, partials, N, M, beta, theta, u_r, alpha, ps, st);
      break;
    case 32:
      param_fused_c<32>(I, u0, U, S, GS, Lam, partials, N, M, beta, theta, u_r, alpha, ps, st);
      break;
    default:
      param_fused_c<64>(I, u0, U, S, GS, Lam, partials, N, M, beta, theta, u_r, alpha, ps, st);
      break;
  }
  LSH_CHECK_LAUNCH();
  return LSH_OK;
}

}  // namespace lsh

using namespace lsh;

extern "C" size_t lsh_lif_scan_exact_workspace(void) { return kWsHeaderBytes; }

static int exact_fwd(bool spec, const float* I, const float* u0, float* U, float* S, int64_t T,
                     int64_t N, float beta, float theta, float u_r, int C, int K, void* ws,
                     size_t ws_bytes, void* stream) {
  if (bad_ptr(I) || bad_ptr(u0) || bad_ptr(U) || bad_ptr(S) || bad_ptr(ws)) return LSH_ERR_ARG;
  if (T < 0 || N < 0 || N > (int64_t)1 << 31 || K < 1 || K > 16) return LSH_ERR_SHAPE;
  if (C != 16 && C != 32 && C != 64 && C != 128) return LSH_ERR_SHAPE;
  if (T % C != 0) return LSH_ERR_DIVISIBILITY;
  // per-lane + per-row buffer byte offsets within one chunk must stay below 2^32
  if ((uint64_t)N * (uint64_t)C * 4u >= ((uint64_t)1 << 32)) return LSH_ERR_SHAPE;
  if (ws_bytes < kWsHeaderBytes || (reinterpret_cast<uintptr_t>(ws) & 255u) != 0)
    return LSH_ERR_WORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  WsHeader* h = reinterpret_cast<WsHeader*>(ws);
  hipLaunchKernelGGL(k_ws_header_reset, dim3(1), dim3(64), 0, st, h);
  if (T > 0 && N > 0) {
    const int rc = spec ? fwd_fused<true>(I, u0, U, S, h, N, (int)(T / C), C, K, beta, theta, u_r, st)
                        : fwd_fused<false>(I, u0, U, S, h, N, (int)(T / C), C, K, beta, theta, u_r, st);
    if (rc != LSH_OK) return rc;
  }
  LSH_CHECK_LAUNCH();
  return LSH_OK;
}

extern "C" int lsh_lif_scan_exact_fwd(const float* I, const float* u0, float* U, float* S,
                                      int64_t T, int64_t N, float beta, float theta, float u_r,
                                      int C, int K, void* ws, size_t ws_bytes, void* stream) {
  return exact_fwd(true, I, u0, U, S, T, N, beta, theta, u_r, C, K, ws, ws_bytes, stream);
}

extern "C" int lsh_lif_chunked_serial_fwd(const float* I, const float* u0, float* U, float* S,
                                          int64_t T, int64_t N, float beta, float theta, float u_r,
                                          int C, void* ws, size_t ws_bytes, void* stream) {
  return exact_fwd(false, I, u0, U, S, T, N, beta, theta, u_r, C, 1, ws, ws_bytes, stream);
}

extern "C" int lsh_lif_scan_exact_fwd_starts(const float* I, const float* u0, float* STARTS,
                                             float* S, int64_t T, int64_t N, float beta,
                                             float theta, float u_r, int C, void* ws,
                                             size_t ws_bytes, void* stream) {
  if (bad_ptr(I) || bad_ptr(u0) || bad_ptr(STARTS) || bad_ptr(S)) return LSH_ERR_ARG;
  if (T < 0 || N < 0 || N > (int64_t)1 << 31) return LSH_ERR_SHAPE;
  if (C != 16 && C != 32 && C != 64) return LSH_ERR_SHAPE;
  if (T % C != 0) return LSH_ERR_DIVISIBILITY;
  if ((uint64_t)N * (uint64_t)C * 4u >= ((uint64_t)1 << 32)) return LSH_ERR_SHAPE;
  // ws NULL: no counters.  Otherwise the kernel adds its counters (spin_timeouts) to the
  // header without clearing it first: no reset launch precedes the forward, and a header the
  // caller cleared once accumulates over many calls.
  if (ws != nullptr &&
      (ws_bytes < kWsHeaderBytes || (reinterpret_cast<uintptr_t>(ws) & 255u) != 0))
    return LSH_ERR_WORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  WsHeader* h = reinterpret_cast<WsHeader*>(ws);
  if (T > 0 && N > 0) {
    const int M = (int)(T / C);
    switch (C) {
      case 16: fwd_starts_c<16>(I, u0, STARTS, S, h, N, M, beta, theta, u_r, st); break;
      case 32: fwd_starts_c<32>(I, u0, STARTS, S, h, N, M, beta, theta, u_r, st); break;
      default: fwd_starts_c<64>(I, u0, STARTS, S, h, N, M, beta, theta, u_r, st); break;
    }
  }
  LSH_CHECK_LAUNCH();
  return LSH_OK;
}

extern "C" int lsh_lif_scan_fused_bwd_starts(const float* I, const float* STARTS, const float* GS,
                                             float* Lam, double* partials, int64_t T, int64_t N,
                                             float beta, float theta, float u_r, float alpha, int C,
                                             void* stream) {
  if (bad_ptr(I) || bad_ptr(STARTS) || bad_ptr(GS) || bad_ptr(Lam)) return LSH_ERR_ARG;
  if (T < 0 || N < 0 || N > (int64_t)1 << 31) return LSH_ERR_SHAPE;
  if (C != 16 && C != 32 && C != 64) return LSH_ERR_SHAPE;
  if (T % C != 0) return LSH_ERR_DIVISIBILITY;
  if ((uint64_t)N * (uint64_t)C * 4u >= ((uint64_t)1 << 32)) return LSH_ERR_SHAPE;
  if (T == 0 || N == 0) return LSH_OK;
  hipStream_t st = (hipStream_t)stream;
  const int M = (int)(T / C);
  switch (C) {
    case 16: bwd_rc_c<16>(I, STARTS, GS, Lam, partials, N, M, beta, theta, u_r, alpha, st); break;
    case 32: bwd_rc_c<32>(I, STARTS, GS, Lam, partials, N, M, beta, theta, u_r, alpha, st); break;
    default: bwd_rc_c<64>(I, STARTS, GS, Lam, partials, N, M, beta, theta, u_r, alpha, st); break;
  }
  LSH_CHECK_LAUNCH();
  return LSH_OK;
}

extern "C" int lsh_lif_scan_fused_bwd(const float* I, const float* u0, const float* U,
                                      const float* S, const float* GS, const float* GU, float* Lam,
                                      int64_t T, int64_t N, float beta, float theta, float u_r,
                                      float alpha, int detach, int C, void* stream) {
  if (bad_ptr(I) || bad_ptr(u0) || bad_ptr(U) || bad_ptr(S) || bad_ptr(GS) || bad_ptr(Lam))
    return LSH_ERR_ARG;
  if (T < 0 || N < 0 || N > (int64_t)1 << 31) return LSH_ERR_SHAPE;
  if (C != 16 && C != 32 && C != 64) return LSH_ERR_SHAPE;
  if (T % C != 0) return LSH_ERR_DIVISIBILITY;
  // per-lane + per-row buffer byte offsets within one chunk must stay below 2^32
  if ((uint64_t)N * (uint64_t)C * 4u >= ((uint64_t)1 << 32)) return LSH_ERR_SHAPE;
  if (T == 0 || N == 0) return LSH_OK;
  hipStream_t st = (hipStream_t)stream;
  const int M = (int)(T / C);
  const bool d = detach != 0;
  switch (C) {
    case 16: bwd_fused_c<16>(I, u0, U, S, GS, GU, Lam, N, M, beta, theta, u_r, alpha, d, st); break;
    case 32: bwd_fused_c<32>(I, u0, U, S, GS, GU, Lam, N, M, beta, theta, u_r, alpha, d, st); break;
    default: bwd_fused_c<64>(I, u0, U, S, GS, GU, Lam, N, M, beta, theta, u_r, alpha, d, st); break;
  }
  LSH_CHECK_LAUNCH();
  return LSH_OK;
}
