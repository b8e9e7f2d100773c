// Single-pass affine-scan adjoint for few neurons (MI355X, gfx950): decoupled look-back across
// workgroups.  Reference: triton_lif.py:512-526 (scan_backward_tiled), :43-50 (_coef).
//
//   lam_t = b_t + a_t * lam_{t+1},  lam_T = 0,   dI_t = lam_t
//
// The single-pass kernel of lif_fused.hip gives one workgroup all of T for 64 neurons, which
// leaves most of the chip idle when there are few neurons.  Here a workgroup owns one segment
// of W*C steps of 64 neurons (wave w: one chunk of C steps, wave 0 the latest), and
// workgroups take segments latest-first through a ticket counter:
//   1. every wave loads its chunk once (I, U_{t-1}, S, GS[, GU]) into registers and composes
//      its affine map (P, Q);
//   2. wave 0 composes the segment map;
//   3. wave 0 takes lam at its segment end from the later segments' published maps and an
//      anchor's inclusive value, in an order fixed by the segment index (lb_value_at_end: the
//      same bits on every run); an anchor then publishes its inclusive value (lam at the
//      segment start, flag 2), every other segment has published its map (flag 1) before;
//   4. every wave takes lam at its chunk end from the later chunks of the segment and replays,
//      storing dI.
// A workgroup only waits for segments whose tickets are smaller than its own, i.e. for
// workgroups already running, so the waits end; each is bounded all the same (a give-up is
// counted in the header and the result is then not valid).  Flags and aggregates cross XCDs;
// they go through coherent vector atomics only (see ld_coh / st_coh / publish_flag).
#include <mutex>

#include "lsh_abi.h"
#include "lsh_common.h"
#include "lsh_lookback.h"

namespace lsh {

__global__ __launch_bounds__(64) void k_fill_i32(int* __restrict__ p, int64_t n, int v) {
  const int64_t i = (int64_t)blockIdx.x * WAVE + threadIdx.x;
  if (i < n) p[i] = v;
}

void fill_i32_launch(int* p, int64_t n, int v, hipStream_t st) {
  if (n > 0)
    hipLaunchKernelGGL(k_fill_i32, dim3((unsigned)((n + WAVE - 1) / WAVE)), dim3(WAVE), 0, st, p, n, v);
}

// PS (detached, no GU): parameter sums in fp64, one partials row per workgroup (tile), as
// k_lif_bwd_fused: PS == 1 the hard reset's (fit.py:43-47), PS == 2 the affine reset's
// (triton_affine.py:229-242) with `u_r` carrying gamma.
template <int C, int W, bool DETACH, bool HAS_GU, int PS = 0>
__global__ __launch_bounds__(WAVE* W) void k_lif_bwd_lookback(
    const float* __restrict__ I, const float* __restrict__ u0, const float* __restrict__ U,
    const float* __restrict__ S, const float* __restrict__ GS, const float* __restrict__ GU,
    float* __restrict__ Lam, float* __restrict__ aggP, float* __restrict__ aggQ,
    float* __restrict__ incl, int* __restrict__ flags, WsHeader* hdr, double* __restrict__ partials,
    int64_t N, int NB, int NSEG, float beta, float theta, float u_r, float alpha) {
  static_assert(!PS || (DETACH && !HAS_GU && C <= 64), "parameter sums: detached, no GU");
  constexpr bool AFF = PS == 2;
  __shared__ float sP[W][WAVE], sQ[W][WAVE];
  __shared__ float sLamEnd[WAVE];
  __shared__ float sLbP[LB_GROUP][WAVE], sLbQ[LB_GROUP][WAVE];
  __shared__ double sAcc[PS ? W : 1][3];
  __shared__ int sTicket;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const unsigned lane = threadIdx.x % WAVE;
  if (threadIdx.x == 0) sTicket = (int)atomicAdd(&hdr->ticket, 1u);
  __syncthreads();
  const int t = sTicket;
  const int nb = t % NB;
  const int seg = NSEG - 1 - t / NB;  // latest segments first
  const int64_t nb0 = (int64_t)nb * WAVE;
  const bool valid = nb0 + lane < N;
  const unsigned ln = valid ? lane : (unsigned)(N - 1 - nb0);
  const unsigned lb = ln * 4u, sb = lane * 4u;
  const unsigned rstride = (unsigned)(N * 4);
  const size_t row0 = ((size_t)seg * W + (W - 1 - w)) * C;  // wave 0 holds the latest chunk
  const float u0n = u0[nb0 + ln];

  // 1. coefficients of the chunk and its map
  float a[AFF ? 1 : C], b[C];
  float upk[PS ? C : 1];
  float vpk[AFF ? C : 1];
  unsigned long long sbits = 0;
  const float gbeta = beta * u_r;  // AFF: beta*gamma
  double acc_b = 0.0, acc_t = 0.0, acc_r = 0.0;
  {
    const Buf bi(I + nb0 + row0 * N), bs(S + nb0 + row0 * N), bg(GS + nb0 + row0 * N);
    const Buf bp(U + nb0 + row0 * N);
    const float up0 = row0 > 0 ? ld_row(U + nb0 + (row0 - 1) * N, lb) : u0n;
#pragma unroll
    for (int j = 0; j < C; ++j) {
      const unsigned so = j * rstride;
      const float x = bi.ld(lb, so);
      const float s = bs.ld(lb, so);
      const float gs = bg.ld(lb, so);
      const float up = j == 0 ? up0 : bp.ld(lb, so - rstride);
      const float v = lif_v(up, x, beta);
      const float sg = surrogate(v, theta, alpha);
      float J = 1.0f - s;
      if (!DETACH) J = J + (u_r - v) * sg;
      if constexpr (!AFF) a[j] = beta * J;
      b[j] = HAS_GU ? gs * sg + J * Buf(GU + nb0 + row0 * N).ld(lb, so) : gs * sg;
      if (PS) {
        upk[j] = up;
        if (s != 0.0f) sbits |= 1ull << j;
        if (PS == 1 && valid) acc_t += (double)b[j];
        if constexpr (AFF) vpk[j] = v;
      }
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
  __syncthreads();

  // 2. segment map (wave 0); a segment that is not an anchor publishes it now
  const bool anchor = lb_is_anchor(seg);
  const size_t so = (size_t)seg * N + nb0 + lane;
  int* const myflag = flags + (size_t)seg * NB + nb;
  float Ps = 1.0f, Qs = 0.0f;  // lam_start(seg) = Qs + Ps * lam_end(seg)
  if (w == 0) {
    for (int v = 0; v < W; ++v) {
      Qs = sQ[v][lane] + sP[v][lane] * Qs;
      Ps = sP[v][lane] * Ps;
    }
    if (!anchor) {
      if (valid) {
        st_coh(aggP + so, Ps);
        st_coh(aggQ + so, Qs);
      }
      publish_flag(myflag, 1);
    }
  }
  // 3. look-back: every wave fetches operands, wave 0 composes them in a fixed order; an anchor
  //    publishes its inclusive value
  lb_fetch(seg, NSEG, NB, nb, N, nb0 + ln, w, W, aggP, aggQ, incl, flags, sLbP, sLbQ,
           &hdr->spin_timeouts);
  __syncthreads();
  if (w == 0) {
    const float lam_end = lb_compose(seg, NSEG, sLbP, sLbQ);
    if (anchor) {
      if (valid) st_coh(incl + so, Qs + Ps * lam_end);
      publish_flag(myflag, 2);
    }
    sLamEnd[lane] = lam_end;
  }
  __syncthreads();

  // 4. replay of every chunk from lam at its end
  float lam = sLamEnd[lane];
  for (int v = 0; v < w; ++v) lam = sQ[v][lane] + sP[v][lane] * lam;
  const Buf bl(Lam + nb0 + row0 * N);
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
      double* out = partials + ((size_t)seg * NB + nb) * 3;
      out[0] = tb;
      out[1] = tt;
      out[2] = tr;
    }
  }
}

template <int C, int W, bool DETACH, bool HAS_GU, int PS = 0>
static void launch_lookback(const float* I, const float* u0, const float* U, const float* S,
                            const float* GS, const float* GU, float* Lam, char* ws, int64_t N,
                            int NSEG, float beta, float theta, float u_r, float alpha,
                            hipStream_t st, double* partials = nullptr) {
  const int NB = (int)((N + WAVE - 1) / WAVE);
  const size_t sn = align_up((size_t)NSEG * (size_t)N * 4, 256);
  float* aggP = reinterpret_cast<float*>(ws + kWsHeaderBytes);
  float* aggQ = reinterpret_cast<float*>(ws + kWsHeaderBytes + sn);
  float* incl = reinterpret_cast<float*>(ws + kWsHeaderBytes + 2 * sn);
  int* flags = reinterpret_cast<int*>(ws + kWsHeaderBytes + 3 * sn);
  const int64_t nflags = (int64_t)NSEG * NB;
  hipLaunchKernelGGL(k_ws_header_reset, dim3(1), dim3(64), 0, st, reinterpret_cast<WsHeader*>(ws));
  hipLaunchKernelGGL(k_fill_i32, dim3((unsigned)((nflags + WAVE - 1) / WAVE)), dim3(WAVE), 0, st,
                     flags, nflags, 0);
  hipLaunchKernelGGL((k_lif_bwd_lookback<C, W, DETACH, HAS_GU, PS>), dim3((unsigned)nflags),
                     dim3(WAVE * W), 0, st, I, u0, U, S, GS, GU, Lam, aggP, aggQ, incl, flags,
                     reinterpret_cast<WsHeader*>(ws), partials, N, NB, NSEG, beta, theta, u_r,
                     alpha);
}

template <int C, int W>
static void lookback_cw(const float* I, const float* u0, const float* U, const float* S,
                        const float* GS, const float* GU, float* Lam, char* ws, int64_t N, int NSEG,
                        float beta, float theta, float u_r, float alpha, bool detach,
                        hipStream_t st) {
  if (detach) {
    if (GU)
      launch_lookback<C, W, true, true>(I, u0, U, S, GS, GU, Lam, ws, N, NSEG, beta, theta, u_r,
                                        alpha, st);
    else
      launch_lookback<C, W, true, false>(I, u0, U, S, GS, GU, Lam, ws, N, NSEG, beta, theta, u_r,
                                         alpha, st);
  } else {
    if (GU)
      launch_lookback<C, W, false, true>(I, u0, U, S, GS, GU, Lam, ws, N, NSEG, beta, theta, u_r,
                                         alpha, st);
    else
      launch_lookback<C, W, false, false>(I, u0, U, S, GS, GU, Lam, ws, N, NSEG, beta, theta, u_r,
                                          alpha, st);
  }
}

}  // namespace lsh

using namespace lsh;

// Segment = 256 steps: 16 waves of 16 steps (C = 16) or 8 waves of 32 steps (C = 32).
static constexpr int kLookbackSeg = 256;

extern "C" size_t lsh_lif_scan_lookback_bwd_workspace(int64_t T, int64_t N) {
  if (T < 0 || N < 0 || T % kLookbackSeg != 0) return 0;
  const int64_t NSEG = T / kLookbackSeg;
  const int64_t NB = (N + WAVE - 1) / WAVE;
  const size_t sn = align_up((size_t)NSEG * (size_t)N * 4, 256);
  return kWsHeaderBytes + 3 * sn + align_up((size_t)NSEG * (size_t)NB * 4, 256);
}

extern "C" int lsh_lif_scan_lookback_bwd(const float* I, const float* u0, const float* U,
                                         const float* S, const float* GS, const float* GU,
                                         float* Lam, int64_t T, int64_t N, float beta, float theta,
                                         float u_r, float alpha, int detach, int C, void* ws,
                                         size_t ws_bytes, void* stream) {
  if (bad_ptr(I) || bad_ptr(u0) || bad_ptr(U) || bad_ptr(S) || bad_ptr(GS) || bad_ptr(Lam) ||
      bad_ptr(ws))
    return LSH_ERR_ARG;
  if (T < 0 || N < 0 || N > (int64_t)1 << 31) return LSH_ERR_SHAPE;
  if (C != 16 && C != 32) return LSH_ERR_SHAPE;
  if (T % kLookbackSeg != 0) return LSH_ERR_DIVISIBILITY;
  if ((uint64_t)N * (uint64_t)C * 4u >= ((uint64_t)1 << 32)) return LSH_ERR_SHAPE;
  if (ws_bytes < lsh_lif_scan_lookback_bwd_workspace(T, N) ||
      (reinterpret_cast<uintptr_t>(ws) & 255u) != 0)
    return LSH_ERR_WORKSPACE;
  const int64_t NSEG = T / kLookbackSeg;
  const int64_t NB = (N + WAVE - 1) / WAVE;
  if (NSEG * NB > ((int64_t)1 << 31) - 1) return LSH_ERR_SHAPE;
  if (T == 0 || N == 0) return LSH_OK;
  hipStream_t st = (hipStream_t)stream;
  char* w = static_cast<char*>(ws);
  if (C == 16)
    lookback_cw<16, 16>(I, u0, U, S, GS, GU, Lam, w, N, (int)NSEG, beta, theta, u_r, alpha,
                        detach != 0, st);
  else
    lookback_cw<32, 8>(I, u0, U, S, GS, GU, Lam, w, N, (int)NSEG, beta, theta, u_r, alpha,
                       detach != 0, st);
  LSH_CHECK_LAUNCH();
  return LSH_OK;
}

// ---------------------------------------------------------------------------------------
// The look-back adjoint without a workspace argument (lsh_lif_scan_lookback_bwd_noalloc), for
// callers that cannot allocate: its workspace (header, segment aggregates, flags) is `scratch`,
// a static device array that every device the library runs on holds until the process ends.
// The array's name is a host-side stand-in in host code: its device address is taken once per
// device with hipGetSymbolAddress (with that device current) and kept in g_scratch_ptr, and only
// that address reaches kernels.  The header and the flags are cleared by kernels at every call
// (no memset node), so the array needs no initial contents.
static __device__ __align__(256) unsigned char scratch[LSH_NOALLOC_SCRATCH_BYTES];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[64];  // per device; set on the first call on that device

static void* scratch_address() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

extern "C" int lsh_lif_scan_lookback_bwd_noalloc(const float* I, const float* u0, const float* U,
                                                 const float* S, const float* GS, const float* GU,
                                                 float* Lam, int64_t T, int64_t N, float beta,
                                                 float theta, float u_r, float alpha, int detach,
                                                 int C, void* stream) {
  if (bad_ptr(I) || bad_ptr(u0) || bad_ptr(U) || bad_ptr(S) || bad_ptr(GS) || bad_ptr(Lam))
    return LSH_ERR_ARG;
  if (T < 0 || N < 0 || N > (int64_t)1 << 31) return LSH_ERR_SHAPE;
  if (C != 16 && C != 32) return LSH_ERR_SHAPE;
  if (T % kLookbackSeg != 0) return LSH_ERR_DIVISIBILITY;
  if (lsh_lif_scan_lookback_bwd_workspace(T, N) > (size_t)LSH_NOALLOC_SCRATCH_BYTES)
    return LSH_ERR_SCRATCH;
  void* ws = scratch_address();
  if (ws == nullptr) return LSH_ERR_HIP;
  return lsh_lif_scan_lookback_bwd(I, u0, U, S, GS, GU, Lam, T, N, beta, theta, u_r, alpha, detach,
                                   C, ws, (size_t)LSH_NOALLOC_SCRATCH_BYTES, stream);
}

int lsh::lif_param_bwd_lookback(const float* I, const float* u0, const float* U, const float* S,
                                const float* GS, float* Lam, double* partials, void* ws,
                                size_t ws_bytes, int64_t T, int64_t N, float beta, float theta,
                                float u_r, float alpha, int ps, hipStream_t st) {
  if (bad_ptr(ws)) return LSH_ERR_ARG;
  if (T < 0 || N < 0 || N > (int64_t)1 << 31) return LSH_ERR_SHAPE;
  if (T % kLookbackSeg != 0) return LSH_ERR_DIVISIBILITY;
  if (ws_bytes < lsh_lif_scan_lookback_bwd_workspace(T, N) ||
      (reinterpret_cast<uintptr_t>(ws) & 255u) != 0)
    return LSH_ERR_WORKSPACE;
  const int64_t NSEG = T / kLookbackSeg;
  if (NSEG * ((N + WAVE - 1) / WAVE) > ((int64_t)1 << 31) - 1) return LSH_ERR_SHAPE;
  if (T == 0 || N == 0) return LSH_OK;
  if (ps == 2)
    launch_lookback<16, 16, true, false, 2>(I, u0, U, S, GS, nullptr, Lam, static_cast<char*>(ws), N,
                                            (int)NSEG, beta, theta, u_r, alpha, st, partials);
  else
    launch_lookback<16, 16, true, false, 1>(I, u0, U, S, GS, nullptr, Lam, static_cast<char*>(ws), N,
                                            (int)NSEG, beta, theta, u_r, alpha, st, partials);
  LSH_CHECK_LAUNCH();
  return LSH_OK;
}
