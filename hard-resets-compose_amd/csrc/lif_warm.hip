// Converged exact forward for few neurons and long sequences by warm-started chunks (MI355X,
// gfx950).
//
// With few neurons the time axis must supply the parallelism: T is cut into M = T/C chunks
// and every (chunk, 64-neuron block) is one wave.  A hard-reset trajectory forgets its start
// at every spike (the state becomes u_r whatever it was), so two trajectories driven by the
// same inputs become bit-identical from the first step at which both spike, and stay so.
// The entry state of chunk m is therefore predicted by running the recurrence over the W rows
// before the chunk from u_r (from u0, exactly, when those rows reach row 0): the prediction is
// the true state unless the true trajectory and the warm-up never spiked together within W
// steps.  This is the hard-reset LIF analogue of the reference's ALIF warm predictor
// (triton_alif.py:75-92 alif_warm_kernel, :276-285 alif_warm_predict).
//
//   k_lif_fwd_warm  per (chunk, block): W warm-up steps (read only), then the chunk's C steps
//                   from the prediction, writing U, S, STARTS[m] (the prediction) and
//                   ENDS[m] (the replayed exit);
//   k_lif_count_missed  the predictions that differ from the predecessor's replayed exit;
//   k_lif_repair_wide   one repair round over all chunks at once: each missed chunk is replayed
//                   from its predecessor's exit, stopping as soon as it meets the trajectory
//                   already stored for it, so a wrong prediction costs only the steps until the
//                   two trajectories coalesce;
//   k_lif_repair    (lif_kernels.hip) the device repair of the two-level scan, with the same
//                   early stop, until no chunk's start differs from its predecessor's exit.
//
// The result is the serial recurrence bit for bit (the repair's fixed point is the serial
// trajectory; M rounds always reach it), the result of scan_forward_v3 (triton_lif.py:782-817)
// with repair >= T/C.  Traffic: I read over W + C rows per chunk (the warm-up rows are the
// previous chunk's, read at the same time by that chunk's wave, so mostly from cache), U and S
// written once: 12 B per neuron-step from HBM when the re-read hits.  No chunk maps, no carry.
#include "lsh_abi.h"
#include "lsh_common.h"

namespace lsh {

// Rows per register tile of the warm-up and of the replay (loads of the next tile in flight
// while the current one is computed).
constexpr int WARM_D = 16;

__global__ __launch_bounds__(64) void k_lif_fwd_warm(const float* __restrict__ I,
                                                     const float* __restrict__ u0,
                                                     float* __restrict__ U, float* __restrict__ S,
                                                     float* __restrict__ starts,
                                                     float* __restrict__ ends, int64_t N, int C,
                                                     int W, int NB, float beta, float theta,
                                                     float u_r) {
  const int64_t m = blockIdx.x / NB;
  const int nb = (int)(blockIdx.x - m * NB);
  const int64_t n = (int64_t)nb * WAVE + threadIdx.x;
  if (n >= N) return;  // no barriers below: lanes past N simply leave
  const int64_t t0 = m * (int64_t)C;
  // warm-up rows [t0 - w, t0): from u0 when they reach row 0 (an exact start), else from u_r
  const int64_t w = t0 < (int64_t)W ? t0 : (int64_t)W;
  float u = (w == t0) ? u0[n] : u_r;
  stream_rows<WARM_D>(I + (size_t)(t0 - w) * N + n, (size_t)N, w, [&](int64_t, float x) {
    bool s;
    u = lif_step(u, x, beta, theta, u_r, s);
  });
  starts[(size_t)m * N + n] = u;
  // the chunk from the prediction (the replay of the two-level scan)
  const size_t base = (size_t)t0 * (size_t)N + (size_t)n;
  const float* __restrict__ Ip = I + base;
  float* __restrict__ Up = U + base;
  float* __restrict__ Sp = S + base;
  stream_rows<WARM_D>(Ip, (size_t)N, C, [&](int64_t j, float x) {
    bool s;
    u = lif_step(u, x, beta, theta, u_r, s);
    st_nt(Up + (size_t)j * N, u);
    st_nt(Sp + (size_t)j * N, s ? 1.0f : 0.0f);
  });
  ends[(size_t)m * N + n] = u;
}

// Chunk entries m >= 1 whose prediction differs from the predecessor's replayed exit, added to
// the header's fused_fixups (one atomic per wave).
__global__ __launch_bounds__(64) void k_lif_count_missed(const float* __restrict__ starts,
                                                         const float* __restrict__ ends,
                                                         WsHeader* hdr, int64_t N, int NB) {
  const int64_t m = blockIdx.x / NB + 1;
  const int nb = (int)(blockIdx.x % NB);
  const int64_t n = (int64_t)nb * WAVE + threadIdx.x;
  const bool miss = n < N && ends[(size_t)(m - 1) * N + n] != starts[(size_t)m * N + n];
  const unsigned long long b = __ballot(miss);
  if (threadIdx.x == 0 && b) atomicAdd(&hdr->fused_fixups, (unsigned long long)__popcll(b));
}

// One repair round over every (chunk, block) at once, before the per-block repair: each chunk
// m >= 1 whose start differs from its predecessor's exit is replayed from that exit, stopping
// where it meets the trajectory stored for it (the early stop of k_lif_repair).  With many
// missed predictions this spreads their replays over the whole chip instead of one workgroup
// per 64 neurons.  A chunk may read its predecessor's exit before or after the predecessor's
// own replay in this round rewrites it; either way it replays a consistent trajectory from the
// value it read and records that value as its start, and the per-block repair that follows
// checks every chunk again, so the result is the same fixed point (the serial recurrence).
__global__ __launch_bounds__(64) void k_lif_repair_wide(const float* __restrict__ I,
                                                        float* __restrict__ U,
                                                        float* __restrict__ S,
                                                        float* __restrict__ starts,
                                                        float* ends, int64_t N, int C, int NB,
                                                        float beta, float theta, float u_r) {
  const int64_t m = blockIdx.x / NB + 1;
  const int nb = (int)(blockIdx.x % NB);
  const int64_t n = (int64_t)nb * WAVE + threadIdx.x;
  if (n >= N) return;
  const float prev = __builtin_nontemporal_load(ends + (size_t)(m - 1) * N + n);
  if (prev == starts[(size_t)m * N + n]) return;
  starts[(size_t)m * N + n] = prev;
  float u = prev;
  const size_t base = (size_t)m * C * N + n;
  const bool met = stream_rows_until<16>(
      I + base, U + base, (size_t)N, C, [&](int64_t j, float x, float u_old) {
        bool s;
        u = lif_step(u, x, beta, theta, u_r, s);
        U[base + (size_t)j * N] = u;
        S[base + (size_t)j * N] = s ? 1.0f : 0.0f;
        return same_bits(u, u_old);
      });
  if (!met) ends[(size_t)m * N + n] = u;
}

static int warm_check(int64_t T, int64_t N, int C, int W) {
  if (T < 0 || N < 0 || N > ((int64_t)1 << 31) || C < 1 || W < 0) return LSH_ERR_SHAPE;
  if (T % C != 0) return LSH_ERR_DIVISIBILITY;
  if ((T / C) * ((N + WAVE - 1) / WAVE) > ((int64_t)1 << 31) - 1) return LSH_ERR_SHAPE;
  if ((T / C) * ((N + WAVE - 1) / WAVE) * WAVE > ((int64_t)1 << 31) - 1) return LSH_ERR_SHAPE;
  return LSH_OK;
}

struct WarmLayout {
  size_t STARTS, ENDS, LIST0, LIST1, total;
};

static WarmLayout warm_layout(int64_t T, int64_t N, int C) {
  const int64_t M = T / C;
  const size_t mn = (size_t)M * (size_t)N * 4;
  const size_t nb = (size_t)((N + WAVE - 1) / WAVE);
  WarmLayout L;
  Carver c;
  L.STARTS = c.take(mn);
  L.ENDS = c.take(mn);
  L.LIST0 = c.take(nb * (size_t)M * WAVE * 4);
  L.LIST1 = c.take(nb * (size_t)M * WAVE * 4);
  L.total = c.off;
  return L;
}

}  // namespace lsh

using namespace lsh;

extern "C" size_t lsh_lif_scan_warm_workspace(int64_t T, int64_t N, int C) {
  if (warm_check(T, N, C, 0) != LSH_OK) return 0;
  return warm_layout(T, N, C).total;
}

extern "C" int lsh_lif_scan_warm_fwd(const float* I, const float* u0, float* U, float* S,
                                     int64_t T, int64_t N, float beta, float theta, float u_r,
                                     int C, int W, void* ws, size_t ws_bytes, void* stream) {
  if (bad_ptr(I) || bad_ptr(u0) || bad_ptr(U) || bad_ptr(S) || bad_ptr(ws)) return LSH_ERR_ARG;
  const int rc = warm_check(T, N, C, W);
  if (rc != LSH_OK) return rc;
  const WarmLayout L = warm_layout(T, N, C);
  if (ws_bytes < L.total || (reinterpret_cast<uintptr_t>(ws) & 255u) != 0) return LSH_ERR_WORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  char* w = static_cast<char*>(ws);
  WsHeader* h = reinterpret_cast<WsHeader*>(w);
  hipLaunchKernelGGL(k_ws_header_reset, dim3(1), dim3(64), 0, st, h);
  if (T == 0 || N == 0) {
    LSH_CHECK_LAUNCH();
    return LSH_OK;
  }
  const int M = (int)(T / C);
  const int NB = (int)((N + WAVE - 1) / WAVE);
  float* starts = reinterpret_cast<float*>(w + L.STARTS);
  float* ends = reinterpret_cast<float*>(w + L.ENDS);
  hipLaunchKernelGGL(k_lif_fwd_warm, dim3((unsigned)((int64_t)M * NB)), dim3(WAVE), 0, st, I, u0,
                     U, S, starts, ends, N, C, W, NB, beta, theta, u_r);
  // The per-block repair counts the missed predictions, so count them here first (the wide
  // round fixes most of them before that repair looks).
  if (M > 1) {
    hipLaunchKernelGGL(k_lif_count_missed, dim3((unsigned)((int64_t)(M - 1) * NB)), dim3(WAVE), 0,
                       st, starts, ends, h, N, NB);
    hipLaunchKernelGGL(k_lif_repair_wide, dim3((unsigned)((int64_t)(M - 1) * NB)), dim3(WAVE), 0,
                       st, I, U, S, starts, ends, N, C, NB, beta, theta, u_r);
  }
  lif_repair_launch(I, U, S, starts, ends, reinterpret_cast<int*>(w + L.LIST0),
                    reinterpret_cast<int*>(w + L.LIST1), h, N, M, C, (int64_t)M, beta, theta, u_r,
                    st);
  LSH_CHECK_LAUNCH();
  return LSH_OK;
}
