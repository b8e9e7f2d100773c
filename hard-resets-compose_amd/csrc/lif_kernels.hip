// Hard-reset LIF kernels for MI355X (gfx950): serial / replay forward, serial /
// replay adjoint, chunk-map build, carry, on-device repair, affine-scan backward.
//
// Layout: I, U, S, GS, GU, Lam are time-major [T, N] fp32 (element (t, n) at
// t*N + n).  One lane owns one neuron; a wave64 covers 64 consecutive neurons,
// so every time row is one contiguous 256-byte access per wave.  Per-chunk
// arrays are [M, N] and map slots [M, K, N] (neuron-contiguous, coalesced).
#include <cstdlib>
#include <mutex>

#include "lsh_abi.h"
#include "lsh_common.h"

namespace lsh {

// ---------------------------------------------------------------------------------------
// workspace header reset: clears the counters and advances the look-back epoch.
__global__ void k_ws_header_reset(WsHeader* h) {
  unsigned int* w = reinterpret_cast<unsigned int*>(h);
  const int epoch_word = (int)(offsetof(WsHeader, epoch) / 4);
  const int t = threadIdx.x;
  if (t < (int)(sizeof(WsHeader) / 4) && t != epoch_word) w[t] = 0u;
  if (t == 0) h->epoch = h->epoch + 1u;
}

// ---------------------------------------------------------------------------------------
// Forward over a segment of Ls steps from a given start state, D-step register tiles with
// the next tile's loads in flight while the current tile is computed.
//   serial forward: one segment (M = 1, Ls = T, starts = u0);
//   scan replay   : M = T / C segments of Ls = C steps, starts = carried chunk entries.
// Follows triton_lif.py:354-379 (fwd_tiled_kernel) and :152-165 (replay_kernel).
// Rows per tile of the carries' exact fallbacks (converged calls).  Measured at cfg2, beta 0.99,
// the whole map scan at C 32 / 64 / 128: 16 rows 2.44 / 2.04 / 1.20 ms, 32 rows 2.36 / 1.84 /
// 1.21 ms (64 rows: more than a 32-step chunk, which then loads row by row).  Loading the next
// chunk's first rows while a chunk's last ones are walked (overflows come in runs) was slower,
// 2.78 / 2.28 ms: the rows kept across chunks cost the carries their registers.
constexpr int kFbRows = 32;
// done (or null): one flag per (chunk, 64-neuron block), set where the carry has already
// replayed the block's chunk from its start (U, S and the end written); those blocks return.
template <int D>
__global__ __launch_bounds__(64) void k_lif_fwd(const float* __restrict__ I,
                                                const float* __restrict__ starts,
                                                float* __restrict__ U, float* __restrict__ S,
                                                float* __restrict__ ends, int64_t N, int64_t Ls,
                                                int NB, float beta, float theta, float u_r,
                                                const int* __restrict__ done = nullptr) {
  if (done && done[blockIdx.x] != 0) return;
  const int64_t m = blockIdx.x / NB;
  const int nb = (int)(blockIdx.x - m * NB);
  const int64_t n = (int64_t)nb * WAVE + threadIdx.x;
  if (n >= N) return;
  float u = starts[m * N + n];
  const size_t base = (size_t)m * (size_t)Ls * (size_t)N + (size_t)n;
  const float* __restrict__ Ip = I + base;
  float* __restrict__ Up = U + base;
  float* __restrict__ Sp = S + base;
  const int64_t nt = Ls / D;
  float xa[D];
  if (nt > 0) {
#pragma unroll
    for (int j = 0; j < D; ++j) xa[j] = Ip[(size_t)j * N];
  }
  for (int64_t b = 0; b < nt; ++b) {
    float xb[D];
    const bool more = b + 1 < nt;
    if (more) {
      const float* __restrict__ In = Ip + (size_t)(b + 1) * D * N;
#pragma unroll
      for (int j = 0; j < D; ++j) xb[j] = In[(size_t)j * N];
    }
    float* __restrict__ Ub = Up + (size_t)b * D * N;
    float* __restrict__ Sb = Sp + (size_t)b * D * N;
#pragma unroll
    for (int j = 0; j < D; ++j) {
      bool s;
      u = lif_step(u, xa[j], beta, theta, u_r, s);
      st_nt(Ub + (size_t)j * N, u);
      st_nt(Sb + (size_t)j * N, s ? 1.0f : 0.0f);
    }
    if (more) {
#pragma unroll
      for (int j = 0; j < D; ++j) xa[j] = xb[j];
    }
  }
  for (int64_t t = nt * D; t < Ls; ++t) {
    bool s;
    u = lif_step(u, Ip[(size_t)t * N], beta, theta, u_r, s);
    st_nt(Up + (size_t)t * N, u);
    st_nt(Sp + (size_t)t * N, s ? 1.0f : 0.0f);
  }
  if (ends) ends[m * N + n] = u;
}

// ---------------------------------------------------------------------------------------
// Reverse sweep of the adjoint over a segment of Ls steps.
//   COMPOSE = false: lam_t = b_t + a_t*lam_{t+1} from lam_end (or 0), writes Lam
//                    (triton_lif.py:383-418 bwd_tiled_kernel, :1088-1127 bwd_tiled_pf_kernel);
//   COMPOSE = true : composes the segment's affine map lam_start = P*lam_end + Q
//                    (triton_lif.py:422-457 bwd_chunk_tiled_kernel).
// Coefficients (triton_lif.py:43-50 _coef): v = beta*u_{t-1} + x_t, sg = surrogate'(v-theta),
// J = 1 - s_t (+ (u_r - v)*sg when the reset is not detached), a = beta*J, b = gs*sg + J*gu.
// PS (detached, no GU): PS == 1, the replay also sums the parameter gradients of
// fit.py:43-47 in fp64 and writes one partials row per block: sum lam_t*u_{t-1},
// sum gs_t*sg_t, sum s_t*lam_{t+1}.  PS == 2, the affine reset u <- gamma*v + delta
// (triton_affine.py:229-242) with `u_r` carrying gamma: J_t = s_t ? gamma : 1 (compose and
// replay), and the replay's sums lam_t*u_{t-1}, s_t*v_t*lam_{t+1}, s_t*lam_{t+1}.
template <int D, bool COMPOSE, bool DETACH, bool HAS_GU, int PS>
__global__ __launch_bounds__(64) void k_lif_bwd(
    const float* __restrict__ I, const float* __restrict__ u0, const float* __restrict__ U,
    const float* __restrict__ S, const float* __restrict__ GS, const float* __restrict__ GU,
    const float* __restrict__ lam_end, float* __restrict__ Lam, float* __restrict__ PA,
    float* __restrict__ PB, double* __restrict__ partials, int64_t N, int64_t Ls, int NB,
    float beta, float theta, float u_r, float alpha) {
  static_assert(!PS || (DETACH && !HAS_GU), "parameter sums: detached, no GU");
  static_assert(PS != 1 || !COMPOSE, "hard-reset sums: replay only");
  constexpr bool AFF = PS == 2;
  constexpr bool SUMS = PS != 0 && !COMPOSE;
  const float gbeta = beta * u_r;  // AFF: beta*gamma
  const int64_t m = blockIdx.x / NB;
  const int nb = (int)(blockIdx.x - m * NB);
  const int64_t n = (int64_t)nb * WAVE + threadIdx.x;
  double acc_b = 0.0, acc_t = 0.0, acc_r = 0.0;
  auto finish = [&]() {
    if (!SUMS) return;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      acc_b += __shfl_xor(acc_b, o, WAVE);
      acc_t += __shfl_xor(acc_t, o, WAVE);
      acc_r += __shfl_xor(acc_r, o, WAVE);
    }
    if (threadIdx.x == 0) {
      double* out = partials + (size_t)blockIdx.x * 3;
      out[0] = acc_b;
      out[1] = acc_t;
      out[2] = acc_r;
    }
  };
  if (n >= N) {
    finish();
    return;
  }
  const float u0n = u0[n];
  float lam = (!COMPOSE && lam_end) ? lam_end[m * N + n] : 0.0f;
  float P = 1.0f, Q = 0.0f;
  const int64_t t_begin = m * Ls;
  const int64_t nt = Ls / D;

  auto coef = [&](float up, float x, float s, float gs, float gu, float& a, float& bb, float& v) {
    v = lif_v(up, x, beta);
    const float sg = surrogate(v, theta, alpha);
    float J = 1.0f - s;
    if (!DETACH) J = J + (u_r - v) * sg;
    a = AFF ? (s != 0.0f ? gbeta : beta) : beta * J;
    bb = HAS_GU ? gs * sg + J * gu : gs * sg;
  };
  auto uprev = [&](int64_t t) -> float { return t > 0 ? U[(size_t)(t - 1) * N + n] : u0n; };
  // one step of the replay: lam_{t+1} -> lam_t (bb = gs*sg when PS)
  auto replay = [&](size_t o, float up, float s, float a, float bb, float v) {
    const float lam_next = lam;
    lam = bb + a * lam;
    st_nt(Lam + o, lam);
    if (SUMS) {
      acc_b += (double)lam * (double)up;
      if (PS == 1) acc_t += (double)bb;
      if (AFF) acc_t += s != 0.0f ? (double)v * (double)lam_next : 0.0;
      acc_r += s != 0.0f ? (double)lam_next : 0.0;
    }
  };

  // the highest `rem` steps first (segment lengths that are not a multiple of D)
  for (int64_t t = t_begin + Ls - 1; t >= t_begin + nt * D; --t) {
    const size_t o = (size_t)t * N + n;
    float a, bb, v;
    const float up = uprev(t), s = S[o];
    coef(up, I[o], s, GS[o], HAS_GU ? GU[o] : 0.0f, a, bb, v);
    if (COMPOSE) {
      Q = bb + a * Q;
      P = a * P;
    } else {
      replay(o, up, s, a, bb, v);
    }
  }
  if (nt == 0) {
    if (COMPOSE) {
      PA[m * N + n] = P;
      PB[m * N + n] = Q;
    }
    finish();
    return;
  }
  float xa[D], sa[D], ga[D], ha[D], pa[D];
  auto load_tile = [&](int64_t b, float* x, float* s, float* g, float* h, float* p) {
    const int64_t t0 = t_begin + b * D;
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const size_t o = (size_t)(t0 + j) * N + n;
      x[j] = I[o];
      s[j] = S[o];
      g[j] = GS[o];
      h[j] = HAS_GU ? GU[o] : 0.0f;
      p[j] = uprev(t0 + j);
    }
  };
  load_tile(nt - 1, xa, sa, ga, ha, pa);
  for (int64_t b = nt - 1; b >= 0; --b) {
    float xb[D], sb[D], gb[D], hb[D], pb[D];
    const bool more = b > 0;
    if (more) load_tile(b - 1, xb, sb, gb, hb, pb);
    const int64_t t0 = t_begin + b * D;
#pragma unroll
    for (int jj = 0; jj < D; ++jj) {
      const int j = D - 1 - jj;
      float a, bb, v;
      coef(pa[j], xa[j], sa[j], ga[j], ha[j], a, bb, v);
      if (COMPOSE) {
        Q = bb + a * Q;
        P = a * P;
      } else {
        replay((size_t)(t0 + j) * N + n, pa[j], sa[j], a, bb, v);
      }
    }
    if (more) {
#pragma unroll
      for (int j = 0; j < D; ++j) {
        xa[j] = xb[j];
        sa[j] = sb[j];
        ga[j] = gb[j];
        ha[j] = hb[j];
        pa[j] = pb[j];
      }
    }
  }
  if (COMPOSE) {
    PA[m * N + n] = P;
    PB[m * N + n] = Q;
  }
  finish();
}

// Reverse carry over chunk aggregates: LamEnd[m] = lam_{(m+1)C}; lam <- Q + P*lam
// (triton_lif.py:198-208 bwd_carry_kernel).
__global__ __launch_bounds__(64) void k_lif_bwd_carry(const float* __restrict__ PA,
                                                      const float* __restrict__ PB,
                                                      float* __restrict__ lam_end, int64_t N,
                                                      int M) {
  const int64_t n = (int64_t)blockIdx.x * WAVE + threadIdx.x;
  if (n >= N) return;
  float lam = 0.0f;
  for (int m = M - 1; m >= 0; --m) {
    const size_t o = (size_t)m * N + n;
    lam_end[o] = lam;
    lam = PB[o] + PA[o] * lam;
  }
}

// ---------------------------------------------------------------------------------------
// Chunk-map build.  Per (chunk, neuron), one pass over the chunk's C inputs computes
//   (a) the min-affine envelope map l -> min(c, a*l + b) of l -> min(u_r, beta*l + x)
//       (triton_lif.py:699-719 env_chunk_kernel; lemma paper/main.tex:266-272), and
//   (b) the piecewise map u_start -> u_end with capacity KMAX: affine part (A, B), breakpoints
//       appended in descending order with their constants (triton_lif.py:737-779
//       build3_kernel; fast.py:148-183).
// The reference prunes a new breakpoint z unless z < xmin, z <= hi and xmin > lo, where lo
// is the envelope bound of the chunk entry.  That bound depends on the preceding chunks, so
// this pass prunes with hi only and records whether a (K+1)-th breakpoint appeared.  The
// breakpoints form one descending sequence either way, so the reference's map is the prefix
// of this one up to and including the first breakpoint <= lo, and its overflow flag is
// "a (K+1)-th breakpoint appeared and all K stored ones are > lo"; the carry applies that
// truncation once lo is known (k_lif_carry), which removes the separate envelope pass.
template <int KMAX, int D>
__global__ __launch_bounds__(64) void k_lif_build(
    const float* __restrict__ I, const float* __restrict__ u0, float* __restrict__ EC,
    float* __restrict__ EA, float* __restrict__ EB, float* __restrict__ MA, float* __restrict__ MB,
    int* __restrict__ CNT, int* __restrict__ OVFRAW, float* __restrict__ MX, float* __restrict__ MC,
    int64_t N, int C, int NB, int K, float beta, float theta, float u_r,
    float* __restrict__ XT = nullptr, float* __restrict__ CT = nullptr) {
  const int64_t m = blockIdx.x / NB;
  const int nb = (int)(blockIdx.x - m * NB);
  const int64_t n = (int64_t)nb * WAVE + threadIdx.x;
  const bool valid = n < N;
  const int64_t nn = valid ? n : 0;  // invalid lanes run on neuron 0 and store nothing
  const float hi = fmaxf(u0[nn], fmaxf(theta, u_r));
  // the envelope's affine part (a, b) starts at (1, 0) and takes the step of the map's affine
  // part (A, B) (a <- beta*a, b <- fl(fl(beta*b) + x)), so it is (A, B) itself: only its
  // constant c is carried apart
  float ec = INFINITY;
  float A = 1.0f, B = 0.0f, xmin = INFINITY;
  int cnt = 0;
  bool ovf = false;
  int wcnt = 0;  // wave-uniform upper bound of cnt
  // the lane's breakpoints newest first (register r holds breakpoint cnt-1-r): a new one shifts
  // the others up by one register with a select on the lane's (wave-uniform mask) add flag,
  // where writing it at register cnt would take a per-register compare with cnt as well; the
  // stores below put them back in insertion order
  float xd[KMAX], cd[KMAX];
#pragma unroll
  for (int i = 0; i < KMAX; ++i) {
    xd[i] = INFINITY;
    cd[i] = 0.0f;
  }
  const float* __restrict__ Ip = I + (size_t)m * C * N + nn;

  auto step = [&](float x) {
    // (a) envelope constant
    ec = fminf(u_r, lif_v(ec, x, beta));
    // (b) existing constants pushed through the step (same arithmetic as the serial step).
    // wcnt is the same on every lane (it grows through a ballot): slots go in groups of 8
    // behind one scalar branch per group, with no per-slot masks; a slot above a lane's cnt
    // holds no breakpoint yet and is overwritten when one is added, so updating it is harmless.
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
    // preimage of the threshold under the affine part: beta*(A*u + B) + x >= theta
    const float num = (theta - x) - beta * B;
    const float den = beta * A;
    const float z = den == 0.0f ? (num > 0.0f ? INFINITY : -INFINITY) : num / den;
    // the tests as wave masks (each a compare's own result; a combination of per-lane bools
    // would be ballotted through a 0/1 value and another compare)
    const unsigned long long nw0m = wave_ballot(z < xmin) & wave_ballot(z <= hi);
    const unsigned long long fullm = wave_ballot(cnt >= K);
    if (__builtin_amdgcn_inverse_ballot_w64(nw0m & fullm)) ovf = true;
    const unsigned long long nwm = nw0m & ~fullm;
    const bool nw = __builtin_amdgcn_inverse_ballot_w64(nwm);
    if (nwm != 0ull) {  // few steps add a breakpoint anywhere in the wave
      // registers above wc hold no breakpoint in any lane (+inf, shifted onto +inf), so the
      // shift stops at wc's group
#pragma unroll
      for (int g = KMAX - G; g >= 0; g -= G) {
        if (g <= wc) {
#pragma unroll
          for (int i = g + G - 1; i >= g; --i) {
            xd[i] = nw ? (i == 0 ? z : xd[i - 1]) : xd[i];
            cd[i] = nw ? (i == 0 ? u_r : cd[i - 1]) : cd[i];
          }
        }
      }
      if ((nwm & wave_ballot(cnt == wc)) != 0ull) ++wcnt;
    }
    cnt += nw ? 1 : 0;
    xmin = nw ? z : xmin;
    A = beta * A;
    B = lif_v(B, x, beta);
  };

  const int nt = C / D;
  float xa[D];
  if (nt > 0) {
#pragma unroll
    for (int j = 0; j < D; ++j) xa[j] = Ip[(size_t)j * N];
  }
  for (int b = 0; b < nt; ++b) {
    float xb[D];
    const bool more = b + 1 < nt;
    if (more) {
      const float* __restrict__ In = Ip + (size_t)(b + 1) * D * N;
#pragma unroll
      for (int j = 0; j < D; ++j) xb[j] = In[(size_t)j * N];
    }
#pragma unroll
    for (int j = 0; j < D; ++j) step(xa[j]);
    if (more) {
#pragma unroll
      for (int j = 0; j < D; ++j) xa[j] = xb[j];
    }
  }
  for (int t = nt * D; t < C; ++t) step(Ip[(size_t)t * N]);

  if (!valid) return;
  const size_t o = (size_t)m * N + n;
  EC[o] = ec;
  EA[o] = A;
  EB[o] = B;
  MA[o] = A;
  MB[o] = B;
  CNT[o] = cnt;
  OVFRAW[o] = ovf ? 1 : 0;
  // register r goes to slot cnt-1-r (insertion order, breakpoints descending) below cnt and to
  // slot r above it (+inf and unused constants), each slot written once
#pragma unroll
  for (int r = 0; r < KMAX; ++r) {
    if (r < K) {
      const int sl = r < cnt ? cnt - 1 - r : r;
      const size_t os = ((size_t)m * K + sl) * N + n;
      MX[os] = xd[r];
      MC[os] = cd[r];
    }
  }
  if (XT) {  // a neuron's K slots contiguous ([M, N, K]), for walks with one wave per neuron
#pragma unroll
    for (int r = 0; r < KMAX; ++r) {
      if (r < K) {
        const int sl = r < cnt ? cnt - 1 - r : r;
        const size_t ot = ((size_t)m * N + n) * K + sl;
        XT[ot] = xd[r];
        CT[ot] = cd[r];
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// Sequential carry over the M chunks of each neuron (triton_lif.py:579-606 carry2_kernel,
// :723-733 env_carry_kernel):
//   Lo[m] = l - 1e-5*(|l| + 1), l <- min(c, a*l + b)         (envelope bound of chunk entry)
//   (or one caller-given bound per neuron: the v1/v2 scans prune with the loose global
//    state_bounds, triton_lif.py:238-243, :262-295, :609-642)
//   map m truncated at the first breakpoint <= Lo[m] (see k_lif_build), overflow if none
//   Starts[m] = u;  u <- (#{xd > u} == n) ? A*u + B : cd[#{xd > u}]
//   overflowed map: u <- C serial steps from u (same arithmetic as the replay)
// Accumulates the overflow count and kept-breakpoint sum / max for the stats.
template <int KMAX>
__global__ __launch_bounds__(64) void k_lif_carry(
    const float* __restrict__ I, const float* __restrict__ u0, const float* __restrict__ EC,
    const float* __restrict__ EA, const float* __restrict__ EB, const float* __restrict__ MA,
    const float* __restrict__ MB, const int* __restrict__ CNT, const int* __restrict__ OVFRAW,
    const float* __restrict__ MX, const float* __restrict__ MC,
    const float* __restrict__ lo_neuron, float* __restrict__ LO, int* __restrict__ MN,
    int* __restrict__ OVF, float* __restrict__ starts, WsHeader* hdr, int64_t N, int M, int C,
    int K, float beta, float theta, float u_r, float* __restrict__ U, float* __restrict__ S,
    float* __restrict__ ends, int* __restrict__ done) {
  const int64_t n = (int64_t)blockIdx.x * WAVE + threadIdx.x;
  const bool valid = n < N;
  unsigned long long ovf_acc = 0, pcs_acc = 0;
  int pmax = 0;
  if (valid) {
    const float margin = 1e-5f;
    float l = u0[n];
    float u = l;
    for (int m = 0; m < M; ++m) {
      const size_t o = (size_t)m * N + n;
      const float lo = lo_neuron ? lo_neuron[n] : l - margin * (fabsf(l) + 1.0f);
      LO[o] = lo;
      l = fminf(EC[o], __fadd_rn(__fmul_rn(EA[o], l), EB[o]));
      starts[o] = u;
      const int cnt = CNT[o];
      const bool ovfr = OVFRAW[o] != 0;
      float xd[KMAX], cd[KMAX];
#pragma unroll
      for (int i = 0; i < KMAX; ++i) {
        if (i < K) {
          const size_t os = ((size_t)m * K + i) * N + n;
          xd[i] = MX[os];
          cd[i] = MC[os];
        } else {
          xd[i] = -INFINITY;
          cd[i] = 0.0f;
        }
      }
      int gt = 0;
#pragma unroll
      for (int i = 0; i < KMAX; ++i) gt += (i < cnt && xd[i] > lo) ? 1 : 0;
      const int ne = min(cnt, gt + 1);
      const bool ovf = ovfr && gt == cnt;
      MN[o] = ne;
      OVF[o] = ovf ? 1 : 0;
      int k = 0;
#pragma unroll
      for (int i = 0; i < KMAX; ++i) k += (i < ne && xd[i] > u) ? 1 : 0;
      float cval = 0.0f;
#pragma unroll
      for (int i = 0; i < KMAX; ++i) cval = (i == k) ? cd[i] : cval;
      float nu = (k == ne) ? __fadd_rn(__fmul_rn(MA[o], u), MB[o]) : cval;
      if (done) {
        // converged result only (done given): when any lane overflows, every lane of the wave
        // replays the chunk from its start and carries that exact exit; U, S and the end are
        // written here and the replay skips the block
        const bool fb = __ballot(ovf) != 0ull;
        if (fb) {
          float w = u;
          const size_t base = (size_t)m * C * N + n;
          stream_rows<kFbRows>(I + base, (size_t)N, C, [&](int64_t j, float x) {
            bool s;
            w = lif_step(w, x, beta, theta, u_r, s);
            st_nt(U + base + (size_t)j * N, w);
            st_nt(S + base + (size_t)j * N, s ? 1.0f : 0.0f);
          });
          ends[o] = w;
          nu = w;
        }
        if (threadIdx.x == 0) done[(size_t)m * gridDim.x + blockIdx.x] = fb ? 1 : 0;
      } else if (ovf) {  // rare: serial fallback through this chunk
        float w = u;
        stream_rows<16>(I + (size_t)m * C * N + n, (size_t)N, C, [&](int64_t, float x) {
          bool s;
          w = lif_step(w, x, beta, theta, u_r, s);
        });
        nu = w;
      }
      u = nu;
      ovf_acc += ovf ? 1ull : 0ull;
      pcs_acc += (unsigned long long)ne;
      pmax = max(pmax, ne);
    }
  }
  ovf_acc = wave_sum_u64(ovf_acc);
  pcs_acc = wave_sum_u64(pcs_acc);
  pmax = wave_max_i(pmax);
  if (threadIdx.x == 0) {
    atomicAdd(&hdr->ovf_count, ovf_acc);
    atomicAdd(&hdr->pieces_sum, pcs_acc);
    atomicMax(&hdr->pieces_max, (unsigned int)pmax);
  }
}

// The same carry with one wave per neuron, for few neurons (where one lane per neuron leaves
// one or two waves on the chip to walk every chunk with a memory latency each).  The chunks go
// in windows of 64: lane j holds the scalars (envelope map, A, B, count, raw overflow) of the
// window's chunk j, and a map takes a row of RW lanes (RW = 16 for K <= 16, 32 for K <= 32):
// VGPR g holds chunks (64/RW)g + r, lane RW*r + s the breakpoint and constant of slot s of
// chunk (64/RW)g + r.  The next window's loads are issued, unconditionally with clamped
// indices, before the current one is walked, so the walk waits on memory once per 64 chunks.
// Per chunk, the counts #{xd > lo} and #{xd > u} are ballots over the chunk's row, the
// constant is read from lane RW*r + k, and the four
// per-chunk outputs collect in lane c, stored once per window.  The overflow fallback reads
// 64 steps at a time, one per lane, and walks them with lane reads.  Results are the same as
// k_lif_carry's: the same operations on the same values, only distributed over lanes.
template <int RW>
struct LifCarryWindow {
  float ec, ea, eb, ma, mb;  // lane j: chunk j of the window
  int cnt, ovfr;
  float xd[RW], cd[RW];  // VGPR g, lane RW*r + s: slot s of chunk (64/RW)*g + r
};

template <int RW>
__global__ __launch_bounds__(64) void k_lif_carry_wave(
    const float* __restrict__ I, const float* __restrict__ u0, const float* __restrict__ EC,
    const float* __restrict__ EA, const float* __restrict__ EB, const float* __restrict__ MA,
    const float* __restrict__ MB, const int* __restrict__ CNT, const int* __restrict__ OVFRAW,
    const float* __restrict__ MX, const float* __restrict__ MC,
    const float* __restrict__ lo_neuron, float* __restrict__ LO, int* __restrict__ MN,
    int* __restrict__ OVF, float* __restrict__ starts, WsHeader* hdr, int64_t N, int M, int C,
    int K, float beta, float theta, float u_r) {
  const int64_t n = xcd_neuron(blockIdx.x, N);
  const int lane = threadIdx.x;
  constexpr int CPV = 64 / RW;  // chunks per VGPR
  const int row = lane / RW, slot = lane % RW;
  const int sl = min(slot, K - 1);
  auto load = [&](int w, LifCarryWindow<RW>& d) {
    const size_t o = (size_t)min(w * 64 + lane, M - 1) * N + n;
    d.ec = EC[o];
    d.ea = EA[o];
    d.eb = EB[o];
    d.ma = MA[o];
    d.mb = MB[o];
    d.cnt = CNT[o];
    d.ovfr = OVFRAW[o];
#pragma unroll
    for (int g = 0; g < RW; ++g) {
      const size_t os = ((size_t)min(w * 64 + CPV * g + row, M - 1) * K + sl) * N + n;
      d.xd[g] = MX[os];
      d.cd[g] = MC[os];
    }
  };
  const float margin = 1e-5f;
  const float lo_n = lo_neuron ? lo_neuron[n] : 0.0f;
  float l = u0[n];
  float u = l;
  unsigned long long ovf_acc = 0, pcs_acc = 0;
  int pmax = 0;
  const int NW = (M + 63) / 64;
  LifCarryWindow<RW> cur, nxt;
  load(0, cur);
  for (int w = 0; w < NW; ++w) {
    load(min(w + 1, NW - 1), nxt);
    const int nc = min(64, M - w * 64);
    float lo_o = 0.0f, st_o = 0.0f;
    int mn_o = 0, ovf_o = 0;
#pragma unroll
    for (int g = 0; g < RW; ++g) {
      for (int r = 0; r < CPV; ++r) {
        const int c = CPV * g + r;
        if (c >= nc) break;
        const float ec = lane_f(cur.ec, c), ea = lane_f(cur.ea, c), eb = lane_f(cur.eb, c);
        const int cnt = __builtin_amdgcn_readlane(cur.cnt, c);
        const bool ovfr = __builtin_amdgcn_readlane(cur.ovfr, c) != 0;
        const float lo = lo_neuron ? lo_n : l - margin * (fabsf(l) + 1.0f);
        l = fminf(ec, __fadd_rn(__fmul_rn(ea, l), eb));
        const bool in_row = row == r;
        const int gt = __popcll(wave_ballot(in_row && slot < cnt && cur.xd[g] > lo));
        const int ne = min(cnt, gt + 1);
        const bool ovf = ovfr && gt == cnt;
        const int k = __popcll(wave_ballot(in_row && slot < ne && cur.xd[g] > u));
        const float cval = lane_f(cur.cd[g], RW * r + min(k, RW - 1));
        float nu = (k == ne)
                       ? __fadd_rn(__fmul_rn(lane_f(cur.ma, c), u), lane_f(cur.mb, c))
                       : cval;
        if (lane == c) {
          lo_o = lo;
          st_o = u;
          mn_o = ne;
          ovf_o = ovf ? 1 : 0;
        }
        if (ovf)  // rare: serial fallback through this chunk
          nu = wave_serial_rows(I, N, n, (int64_t)(w * 64 + c) * C, C, u, beta, theta, u_r);
        u = nu;
        ovf_acc += ovf ? 1ull : 0ull;
        pcs_acc += (unsigned long long)ne;
        pmax = max(pmax, ne);
      }
    }
    if (lane < nc) {
      const size_t o = (size_t)(w * 64 + lane) * N + n;
      LO[o] = lo_o;
      starts[o] = st_o;
      MN[o] = mn_o;
      OVF[o] = ovf_o;
    }
    cur = nxt;
  }
  if (lane == 0) {
    atomicAdd(&hdr->ovf_count, ovf_acc);
    atomicAdd(&hdr->pieces_sum, pcs_acc);
    atomicMax(&hdr->pieces_max, (unsigned int)pmax);
  }
}

// The same carry with its map reads staged through LDS, for long chunk sequences (many M, few
// neurons), where the one-wave carry above waits a full memory latency per chunk.  A workgroup
// of 4 waves owns 64 neurons: waves 1-3 load the next R chunks' maps (7 + 2K rows of 64 lanes
// each) into one LDS buffer while wave 0 runs the sequential carry over the R chunks already
// in the other buffer; one barrier per stage.  Results are the same as k_lif_carry's.
template <int KMAX>
struct CarryStage {
  static constexpr int ROWS = 7 + 2 * KMAX;                 // EC EA EB MA MB CNT OVFRAW, MX[K], MC[K]
  static constexpr int R = (64 * 1024) / (ROWS * WAVE * 4);  // chunks per stage (<= 64 KB per buffer)
};

template <int KMAX>
__global__ __launch_bounds__(256) void k_lif_carry_staged(
    const float* __restrict__ I, const float* __restrict__ u0, const float* __restrict__ EC,
    const float* __restrict__ EA, const float* __restrict__ EB, const float* __restrict__ MA,
    const float* __restrict__ MB, const int* __restrict__ CNT, const int* __restrict__ OVFRAW,
    const float* __restrict__ MX, const float* __restrict__ MC,
    const float* __restrict__ lo_neuron, float* __restrict__ LO, int* __restrict__ MN,
    int* __restrict__ OVF, float* __restrict__ starts, WsHeader* hdr, int64_t N, int M, int C,
    int K, float beta, float theta, float u_r, float* __restrict__ U, float* __restrict__ S,
    float* __restrict__ ends, int* __restrict__ done) {
  using CS = CarryStage<KMAX>;
  constexpr int ROWS = CS::ROWS, R = CS::R;
  __shared__ float sbuf[2][R * ROWS][WAVE];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const int lane = threadIdx.x % WAVE;
  const int64_t n = (int64_t)blockIdx.x * WAVE + lane;
  const bool valid = n < N;
  const int64_t nn = valid ? n : N - 1;
  const int stages = (M + R - 1) / R;
  // stage s into buffer s & 1 by the loader waves 1-3, chunks w - 1, w + 2, ... of the stage:
  // every load of all of a wave's chunks is issued before the first LDS write (indices clamped
  // into the arrays, so none sits behind a branch), so a stage costs one memory latency; the
  // rows past the map's count are never read
  constexpr int CPL = (R + 2) / 3;  // chunks per loader wave
  auto load_stage = [&](int s) {
    const int m0 = s * R;
    const int nch = min(R, M - m0);
    float v[CPL][ROWS];
#pragma unroll
    for (int t = 0; t < CPL; ++t) {
      const int c = w - 1 + 3 * t;
      const size_t mc = (size_t)min(m0 + c, M - 1);
      const size_t o = mc * N + nn;
      const size_t os = mc * K * N + nn;
      v[t][0] = EC[o];
      v[t][1] = EA[o];
      v[t][2] = EB[o];
      v[t][3] = MA[o];
      v[t][4] = MB[o];
      v[t][5] = __int_as_float(CNT[o]);
      v[t][6] = __int_as_float(OVFRAW[o]);
#pragma unroll
      for (int i = 0; i < KMAX; ++i) {
        const size_t oi = os + (size_t)min(i, K - 1) * N;
        v[t][7 + i] = MX[oi];
        v[t][7 + KMAX + i] = MC[oi];
      }
    }
#pragma unroll
    for (int t = 0; t < CPL; ++t) {
      const int c = w - 1 + 3 * t;
      if (c < nch) {
        float* dst = &sbuf[s & 1][c * ROWS][0];
#pragma unroll
        for (int r = 0; r < ROWS; ++r) dst[r * WAVE + lane] = v[t][r];
      }
    }
  };
  if (w >= 1) load_stage(0);
  __syncthreads();

  unsigned long long ovf_acc = 0, pcs_acc = 0;
  int pmax = 0;
  const float margin = 1e-5f;
  const float lo_n = lo_neuron ? lo_neuron[nn] : 0.0f;
  float l = u0[nn];
  float u = l;
  for (int s = 0; s < stages; ++s) {
    if (w >= 1) {
      if (s + 1 < stages) load_stage(s + 1);
    } else {
      const int m0 = s * R;
      const int nch = min(R, M - m0);
      for (int c = 0; c < nch; ++c) {
        const int m = m0 + c;
        const float* row = &sbuf[s & 1][c * ROWS][0];
        auto rd = [&](int r) { return row[r * WAVE + lane]; };
        const size_t o = (size_t)m * N + nn;
        const float lo = lo_neuron ? lo_n : l - margin * (fabsf(l) + 1.0f);
        l = fminf(rd(0), __fadd_rn(__fmul_rn(rd(1), l), rd(2)));
        const int cnt = __float_as_int(rd(5));
        const bool ovfr = __float_as_int(rd(6)) != 0;
        float xd[KMAX], cd[KMAX];
#pragma unroll
        for (int i = 0; i < KMAX; ++i) {
          xd[i] = i < K ? rd(7 + i) : -INFINITY;
          cd[i] = i < K ? rd(7 + KMAX + i) : 0.0f;
        }
        int gt = 0;
#pragma unroll
        for (int i = 0; i < KMAX; ++i) gt += (i < cnt && xd[i] > lo) ? 1 : 0;
        const int ne = min(cnt, gt + 1);
        const bool ovf = ovfr && gt == cnt;
        int k = 0;
#pragma unroll
        for (int i = 0; i < KMAX; ++i) k += (i < ne && xd[i] > u) ? 1 : 0;
        float cval = 0.0f;
#pragma unroll
        for (int i = 0; i < KMAX; ++i) cval = (i == k) ? cd[i] : cval;
        float nu = (k == ne) ? __fadd_rn(__fmul_rn(rd(3), u), rd(4)) : cval;
        if (valid) {
          LO[o] = lo;
          starts[o] = u;
          MN[o] = ne;
          OVF[o] = ovf ? 1 : 0;
        }
        if (done) {  // as in k_lif_carry: the whole wave replays, the replay skips the block
          const bool fb = __ballot(ovf) != 0ull;
          if (fb) {
            float wv = u;
            const size_t base = (size_t)m * C * N + nn;
            stream_rows<kFbRows>(I + base, (size_t)N, C, [&](int64_t j, float x) {
              bool sp;
              wv = lif_step(wv, x, beta, theta, u_r, sp);
              if (valid) {
                st_nt(U + base + (size_t)j * N, wv);
                st_nt(S + base + (size_t)j * N, sp ? 1.0f : 0.0f);
              }
            });
            if (valid) ends[o] = wv;
            nu = wv;
          }
          if (lane == 0) done[(size_t)m * gridDim.x + blockIdx.x] = fb ? 1 : 0;
        } else if (ovf) {  // rare: serial fallback through this chunk
          float wv = u;
          stream_rows<16>(I + (size_t)m * C * N + nn, (size_t)N, C, [&](int64_t, float x) {
            bool sp;
            wv = lif_step(wv, x, beta, theta, u_r, sp);
          });
          nu = wv;
        }
        u = nu;
        if (valid) {
          ovf_acc += ovf ? 1ull : 0ull;
          pcs_acc += (unsigned long long)ne;
          pmax = max(pmax, ne);
        }
      }
    }
    __syncthreads();
  }
  if (w == 0) {
    ovf_acc = wave_sum_u64(ovf_acc);
    pcs_acc = wave_sum_u64(pcs_acc);
    pmax = wave_max_i(pmax);
    if (lane == 0) {
      atomicAdd(&hdr->ovf_count, ovf_acc);
      atomicAdd(&hdr->pieces_sum, pcs_acc);
      atomicMax(&hdr->pieces_max, (unsigned int)pmax);
    }
  }
}

// ---------------------------------------------------------------------------------------
// On-device repair (triton_lif.py:804-811): Jacobi rounds
//   Starts[m] <- (m == 0 ? u0 : Ends[m-1]); replay the chunks whose start changed
// until nothing changes or `R` rounds ran.  Neurons are independent, so one workgroup owns
// the M chunks of 64 neurons and runs the rounds with workgroup barriers only, with no host
// synchronization.  Only chunks whose start changed are replayed, and only successors of
// chunks whose end changed are re-checked, through two work lists of (chunk, lane) entries.
// Round r gives the same states as the reference's r-th full re-replay; the round count
// (max over neurons) is the reference's repair_iters.
__global__ __launch_bounds__(256) void k_lif_repair(const float* __restrict__ I,
                                                    float* __restrict__ U, float* __restrict__ S,
                                                    float* __restrict__ starts,
                                                    float* __restrict__ ends, int* __restrict__ list0,
                                                    int* __restrict__ list1, WsHeader* hdr,
                                                    int64_t N, int M, int C, int64_t R,
                                                    float beta, float theta, float u_r) {
  __shared__ int s_nd, s_nc;
  const int nb = blockIdx.x;
  const int tid = threadIdx.x;
  const size_t cap = (size_t)M * WAVE;
  int* __restrict__ dl = list0 + (size_t)nb * cap;  // dirty chunks of the current round
  int* __restrict__ cl = list1 + (size_t)nb * cap;  // successors of chunks whose end changed
  if (tid == 0) s_nd = 0;
  __syncthreads();
  for (int e = tid + WAVE; e < M * WAVE; e += blockDim.x) {
    const int m = e / WAVE;
    const int64_t n = (int64_t)nb * WAVE + (e % WAVE);
    if (n < N && ends[(size_t)(m - 1) * N + n] != starts[(size_t)m * N + n]) {
      dl[atomicAdd(&s_nd, 1)] = e;
    }
  }
  __syncthreads();
  int64_t rounds = 0;
  while (true) {
    const int nd = s_nd;
    if (nd == 0 || rounds >= R) break;
    ++rounds;
    for (int i = tid; i < nd; i += blockDim.x) {
      const int e = dl[i];
      const int m = e / WAVE;
      const int64_t n = (int64_t)nb * WAVE + (e % WAVE);
      starts[(size_t)m * N + n] = ends[(size_t)(m - 1) * N + n];
    }
    __syncthreads();
    if (tid == 0) s_nc = 0;
    __syncthreads();
    for (int i = tid; i < nd; i += blockDim.x) {
      const int e = dl[i];
      const int m = e / WAVE;
      const int64_t n = (int64_t)nb * WAVE + (e % WAVE);
      float u = starts[(size_t)m * N + n];
      const size_t base = (size_t)m * C * N + n;
      // U holds this chunk's replay from its previous start.  Once the new trajectory has
      // the same state bits at some step, every later step is the same too (the step is a
      // function of the state and the input), so the replay stops there and the chunk's end
      // is unchanged: exact, and the round gives the same states as a full re-replay.
      const bool met = stream_rows_until<16>(
          I + base, U + base, (size_t)N, C, [&](int64_t j, float x, float u_old) {
            bool s;
            u = lif_step(u, x, beta, theta, u_r, s);
            U[base + (size_t)j * N] = u;
            S[base + (size_t)j * N] = s ? 1.0f : 0.0f;
            return same_bits(u, u_old);
          });
      const size_t oe = (size_t)m * N + n;
      if (!met && u != ends[oe]) {
        ends[oe] = u;
        if (m + 1 < M) cl[atomicAdd(&s_nc, 1)] = e + WAVE;
      }
    }
    __syncthreads();
    if (tid == 0) s_nd = 0;
    __syncthreads();
    const int nc = s_nc;
    for (int i = tid; i < nc; i += blockDim.x) {
      const int e = cl[i];
      const int m = e / WAVE;
      const int64_t n = (int64_t)nb * WAVE + (e % WAVE);
      if (ends[(size_t)(m - 1) * N + n] != starts[(size_t)m * N + n]) dl[atomicAdd(&s_nd, 1)] = e;
    }
    __syncthreads();
  }
  if (tid == 0) atomicMax(&hdr->repair_iters, (unsigned int)rounds);
}

// The repair run to convergence without its round count: one wave per 64 neurons walks the
// chunks in order, carrying each lane's exact exit of the chunk before.  Chunk 0 was replayed
// from u0, so its end is exact; a chunk whose carried start has the bits of that exit was
// replayed exactly and keeps its end; any other chunk is replayed from the exit, lanes masked,
// until the new trajectory meets the stored one (from there on the two are the same, so the
// stored end holds) or the chunk ends (then the new state is the exit).  By induction U and S
// are the serial recurrence, as after the Jacobi rounds, but a run of d consecutive wrong
// starts costs one pass over them instead of d rounds.  Starts and ends are read PF chunks
// ahead; they are not written (the converged result is U and S).
// gate: when not null, the pass runs only if *gate != 0 (the segmented repair's last round
// still rewrote a segment's last end, so its rounds may not have converged).
template <int PF>
__global__ __launch_bounds__(64) void k_lif_repair_ordered(const float* __restrict__ I,
                                                           float* __restrict__ U,
                                                           float* __restrict__ S,
                                                           const float* __restrict__ starts,
                                                           const float* __restrict__ ends,
                                                           int64_t N, int M, int C, float beta,
                                                           float theta, float u_r,
                                                           const int* gate = nullptr) {
  if (gate != nullptr && __builtin_nontemporal_load(gate) == 0) return;
  const int64_t n = (int64_t)blockIdx.x * WAVE + threadIdx.x;
  const bool valid = n < N;
  const int64_t nc = valid ? n : N - 1;  // tail lanes read a valid column and never replay
  float ue = ends[nc];
  float st[PF], en[PF];
#pragma unroll
  for (int k = 0; k < PF; ++k) {
    const size_t o = (size_t)min(1 + k, M - 1) * N + nc;
    st[k] = starts[o];
    en[k] = ends[o];
  }
  for (int m = 1; m < M; ++m) {
    const float s0 = st[0], e0 = en[0];
#pragma unroll
    for (int k = 0; k + 1 < PF; ++k) {
      st[k] = st[k + 1];
      en[k] = en[k + 1];
    }
    {
      const size_t o = (size_t)min(m + PF, M - 1) * N + nc;
      st[PF - 1] = starts[o];
      en[PF - 1] = ends[o];
    }
    const bool dirty = valid && !same_bits(ue, s0);
    if (__ballot(dirty) == 0ull) {
      ue = e0;
      continue;
    }
    if (dirty) {
      float u = ue;
      const size_t base = (size_t)m * C * N + n;
      const bool met = stream_rows_until<16>(
          I + base, U + base, (size_t)N, C, [&](int64_t j, float x, float u_old) {
            bool s;
            u = lif_step(u, x, beta, theta, u_r, s);
            U[base + (size_t)j * N] = u;
            S[base + (size_t)j * N] = s ? 1.0f : 0.0f;
            return same_bits(u, u_old);
          });
      ue = met ? e0 : u;
    } else {
      ue = e0;
    }
  }
}

// The same ordered walk over segments of R chunks at once, for few neurons: one wave per 64
// neurons walking all M chunks leaves a few waves on the chip, and the Jacobi rounds run one
// workgroup per 64 neurons.  Launch r is one round over every (segment, 64 neurons): segment g
// covers chunks m0 = 1 + g R .. m1 - 1 and starts from the stored end of chunk m0 - 1; a
// chunk whose start differs from the carried exit gets that exit as its start and is
// replayed (lanes masked) until it meets its stored trajectory, and its end is rewritten when
// the replay ran to the chunk's end.  After round r every segment is consistent with the end
// it read before it, and segments 0 .. r - 1 are exact (segment r - 1 read the exact end of
// segment r - 2, which round r did not change), so S rounds give the serial recurrence; a
// round in which no segment rewrote its last chunk's end leaves every boundary as the next
// segment read it, so later rounds find nothing to do: flags[r] records whether round r
// rewrote one, and round r + 1 returns at once when it did not.  The launcher runs at most
// kRepairSegRounds rounds and then the whole ordered walk, gated on the last round's flag.  A segment may read its
// boundary before or after the segment before it rewrites it in the same round; either way it
// walks a consistent trajectory from the value it read, and the next round compares again.
// flags[0 .. S] are zero before round 0.
template <int PF>
__global__ __launch_bounds__(64) void k_lif_repair_seg(const float* __restrict__ I,
                                                       float* __restrict__ U, float* __restrict__ S,
                                                       float* __restrict__ starts,
                                                       float* __restrict__ ends, int* flags,
                                                       int64_t N, int M, int C, int R, int NB,
                                                       int round, float beta, float theta,
                                                       float u_r) {
  if (round > 0 && __builtin_nontemporal_load(flags + round - 1) == 0) return;
  const int g = (int)(blockIdx.x / NB);
  const int nb = (int)(blockIdx.x - (int64_t)g * NB);
  const int m0 = 1 + g * R;
  const int m1 = min(M, m0 + R);
  if (m0 >= M) return;
  const int64_t n = (int64_t)nb * WAVE + threadIdx.x;
  const bool valid = n < N;
  const int64_t nc = valid ? n : N - 1;  // tail lanes read a valid column and never replay
  float ue = ends[(size_t)(m0 - 1) * N + nc];
  if (round > 0 && __ballot(valid && !same_bits(ue, starts[(size_t)m0 * N + nc])) == 0ull)
    return;  // consistent with its boundary since the last round
  float st[PF], en[PF];
#pragma unroll
  for (int k = 0; k < PF; ++k) {
    const size_t o = (size_t)min(m0 + k, m1 - 1) * N + nc;
    st[k] = starts[o];
    en[k] = ends[o];
  }
  bool last_changed = false;
  for (int m = m0; m < m1; ++m) {
    const float s0 = st[0], e0 = en[0];
#pragma unroll
    for (int k = 0; k + 1 < PF; ++k) {
      st[k] = st[k + 1];
      en[k] = en[k + 1];
    }
    {
      const size_t o = (size_t)min(m + PF, m1 - 1) * N + nc;
      st[PF - 1] = starts[o];
      en[PF - 1] = ends[o];
    }
    const bool dirty = valid && !same_bits(ue, s0);
    if (__ballot(dirty) == 0ull) {
      // after round 0 the segment is consistent from chunk to chunk, and a later round only
      // changes a run from its start: the first chunk that needs nothing ends that run
      if (round > 0) break;
      ue = e0;
      continue;
    }
    if (dirty) {
      const size_t oc = (size_t)m * N + n;
      starts[oc] = ue;
      float u = ue;
      const size_t base = (size_t)m * C * N + n;
      const bool met = stream_rows_until<16>(
          I + base, U + base, (size_t)N, C, [&](int64_t j, float x, float u_old) {
            bool s;
            u = lif_step(u, x, beta, theta, u_r, s);
            U[base + (size_t)j * N] = u;
            S[base + (size_t)j * N] = s ? 1.0f : 0.0f;
            return same_bits(u, u_old);
          });
      if (met) {
        ue = e0;
      } else {
        ue = u;
        if (!same_bits(u, e0)) {
          ends[oc] = u;
          if (m == m1 - 1) last_changed = true;
        }
      }
    } else {
      ue = e0;
    }
  }
  if (m1 < M && __ballot(last_changed) != 0ull && threadIdx.x == 0) atomicOr(flags + round, 1);
}

// ---------------------------------------------------------------------------------------
// host-side launch helpers
template <int D>
static void launch_fwd(const float* I, const float* starts, float* U, float* S, float* ends,
                       int64_t N, int64_t Ls, int64_t M, float beta, float theta, float u_r,
                       hipStream_t st, const int* done = nullptr) {
  const int NB = (int)((N + WAVE - 1) / WAVE);
  hipLaunchKernelGGL(k_lif_fwd<D>, dim3((unsigned)(M * NB)), dim3(WAVE), 0, st, I, starts, U, S,
                     ends, N, Ls, NB, beta, theta, u_r, done);
}

static void launch_fwd_auto(const float* I, const float* starts, float* U, float* S, float* ends,
                            int64_t N, int64_t Ls, int64_t M, float beta, float theta, float u_r,
                            hipStream_t st, const int* done = nullptr) {
  if (Ls >= 32)
    launch_fwd<16>(I, starts, U, S, ends, N, Ls, M, beta, theta, u_r, st, done);
  else
    launch_fwd<4>(I, starts, U, S, ends, N, Ls, M, beta, theta, u_r, st, done);
}

template <bool COMPOSE, bool DETACH, bool HAS_GU, int PS = 0>
static void launch_bwd3(const float* I, const float* u0, const float* U, const float* S,
                        const float* GS, const float* GU, const float* lam_end, float* Lam, float* PA,
                        float* PB, int64_t N, int64_t Ls, int64_t M, float beta, float theta,
                        float u_r, float alpha, hipStream_t st, double* partials = nullptr) {
  const int NB = (int)((N + WAVE - 1) / WAVE);
  if (M == 1 && !COMPOSE && PS == 0 && !lam_end) {
    // the serial adjoint with few neurons: producer and consumer waves (serial_pipe.hip)
    lif_serial_bwd_pipe(I, u0, U, S, GS, GU, Lam, N, Ls, beta, theta, u_r, alpha, DETACH, st);
    return;
  }
  if (M == 1 && !COMPOSE) {
    // one segment: the serial adjoint, latency-bound with few neurons -> 16 steps in flight
    hipLaunchKernelGGL((k_lif_bwd<16, COMPOSE, DETACH, HAS_GU, PS>), dim3((unsigned)NB), dim3(WAVE), 0,
                       st, I, u0, U, S, GS, GU, lam_end, Lam, PA, PB, partials, N, Ls, NB, beta, theta,
                       u_r, alpha);
    return;
  }
  constexpr int D = 4;
  hipLaunchKernelGGL((k_lif_bwd<D, COMPOSE, DETACH, HAS_GU, PS>), dim3((unsigned)(M * NB)), dim3(WAVE),
                     0, st, I, u0, U, S, GS, GU, lam_end, Lam, PA, PB, partials, N, Ls, NB, beta,
                     theta, u_r, alpha);
}

template <bool COMPOSE>
static void launch_bwd(const float* I, const float* u0, const float* U, const float* S,
                       const float* GS, const float* GU, const float* lam_end, float* Lam, float* PA,
                       float* PB, int64_t N, int64_t Ls, int64_t M, float beta, float theta,
                       float u_r, float alpha, bool detach, hipStream_t st) {
  const bool has_gu = GU != nullptr;
  if (detach) {
    if (has_gu)
      launch_bwd3<COMPOSE, true, true>(I, u0, U, S, GS, GU, lam_end, Lam, PA, PB, N, Ls, M, beta,
                                       theta, u_r, alpha, st);
    else
      launch_bwd3<COMPOSE, true, false>(I, u0, U, S, GS, GU, lam_end, Lam, PA, PB, N, Ls, M, beta,
                                        theta, u_r, alpha, st);
  } else {
    if (has_gu)
      launch_bwd3<COMPOSE, false, true>(I, u0, U, S, GS, GU, lam_end, Lam, PA, PB, N, Ls, M, beta,
                                        theta, u_r, alpha, st);
    else
      launch_bwd3<COMPOSE, false, false>(I, u0, U, S, GS, GU, lam_end, Lam, PA, PB, N, Ls, M, beta,
                                         theta, u_r, alpha, st);
  }
}

void v3_layout_fill(int64_t T, int64_t N, int C, int K, lsh_v3_layout* L) {
  const int64_t M = T / C;
  const size_t mn = (size_t)M * (size_t)N * 4;
  const size_t nb = (size_t)((N + WAVE - 1) / WAVE);
  Carver c;
  L->EC = c.take(mn);
  L->EA = c.take(mn);
  L->EB = c.take(mn);
  L->MA = c.take(mn);
  L->MB = c.take(mn);
  L->CNT = c.take(mn);
  L->OVFRAW = c.take(mn);
  L->MX = c.take(mn * (size_t)K);
  L->MC = c.take(mn * (size_t)K);
  L->LO = c.take(mn);
  L->MN = c.take(mn);
  L->OVF = c.take(mn);
  L->STARTS = c.take(mn);
  L->ENDS = c.take(mn);
  L->LIST0 = c.take(nb * (size_t)M * WAVE * 4);
  L->LIST1 = c.take(nb * (size_t)M * WAVE * 4);
  L->total = c.off;
}

template <int KMAX>
static void launch_build(const float* I, const float* u0, char* ws, const lsh_v3_layout& L,
                         int64_t N, int M, int C, int K, float beta, float theta, float u_r,
                         hipStream_t st, float* XT = nullptr, float* CT = nullptr) {
  const int NB = (int)((N + WAVE - 1) / WAVE);
  auto F = [&](size_t off) { return reinterpret_cast<float*>(ws + off); };
  auto Iq = [&](size_t off) { return reinterpret_cast<int*>(ws + off); };
  if (C >= 16)
    hipLaunchKernelGGL((k_lif_build<KMAX, 8>), dim3((unsigned)(M * NB)), dim3(WAVE), 0, st, I, u0,
                       F(L.EC), F(L.EA), F(L.EB), F(L.MA), F(L.MB), Iq(L.CNT), Iq(L.OVFRAW), F(L.MX),
                       F(L.MC), N, C, NB, K, beta, theta, u_r, XT, CT);
  else
    hipLaunchKernelGGL((k_lif_build<KMAX, 1>), dim3((unsigned)(M * NB)), dim3(WAVE), 0, st, I, u0,
                       F(L.EC), F(L.EA), F(L.EB), F(L.MA), F(L.MB), Iq(L.CNT), Iq(L.OVFRAW), F(L.MX),
                       F(L.MC), N, C, NB, K, beta, theta, u_r, XT, CT);
}

// The carry over the M chunk maps from u0 (the envelope seed and the first start).
// Exact fallbacks (RP given: only where the result is the converged one, the serial
// recurrence): a lane carry whose wave runs the serial fallback for an overflowed lane runs it
// for all its lanes, which then carry the exact exit instead of the map's, and writes U, S and
// the end of that chunk as the replay would; one flag per (chunk, 64-neuron block) in
// RP->done, which the replay reads, tells it which blocks are done.  The same steps cost nothing
// more in the other lanes; at cfg2, beta 0.99 (28-73 % of the chunks overflow at K 8), most
// blocks are then replayed once, inside the carry, and their starts are exact, so the repair
// finds little left.  Returns whether the flags were written (the one-wave-per-neuron carry
// for few neurons keeps the plain fallback).
struct ReplayInto {
  float *U, *S, *ends;
  int* done;
};
constexpr int kStagedCarryMaxBlocks = 256;  // one staged block per CU of the MI355X

template <int KMAX>
static bool launch_carry(const float* I, const float* u0, const float* lo_neuron, char* ws,
                         const lsh_v3_layout& L, int64_t N, int M, int C, int K, float beta,
                         float theta, float u_r, hipStream_t st, const ReplayInto* RP) {
  float* rU = RP ? RP->U : nullptr;
  float* rS = RP ? RP->S : nullptr;
  float* rE = RP ? RP->ends : nullptr;
  int* rD = RP ? RP->done : nullptr;
  const int NB = (int)((N + WAVE - 1) / WAVE);
  auto F = [&](size_t off) { return reinterpret_cast<float*>(ws + off); };
  auto Iq = [&](size_t off) { return reinterpret_cast<int*>(ws + off); };
// Most neurons for the one-wave-per-neuron carry.  Measured on MI355X, the map scan (build,
// carry, replay; x ~ N(0.15, 0.4^2), beta 0.99, C 256, K 16) against the staged carry: N = 128,
// T = 65536 0.47 -> 0.22 ms; N = 1024, T = 65536 0.70 -> 0.50 ms; N = 2048, T = 65536 1.04 ->
// 0.90 ms; N = 2048, T = 16384 0.29 -> 0.32 ms at C 256 (64 chunks) but 0.36 -> 0.33 ms at C 128
// (128 chunks), so above 1024 neurons it takes 128 chunks or more; N = 4096, T = 65536 1.69 ->
// 2.01 ms (K 8, with 3 % overflowed chunks: 3.68 -> 1.95 ms); N = 16384, T = 16384 1.48 -> 2.29.
#ifndef LSH_LIF_CARRY_WAVE_MAX_N
#define LSH_LIF_CARRY_WAVE_MAX_N 2048
#endif
  if (KMAX <= 32 && N <= LSH_LIF_CARRY_WAVE_MAX_N && (N <= 1024 || M >= 128)) {
    // few neurons: one wave per neuron, a chunk map on a row of 16 lanes (K <= 16) or 32
    hipLaunchKernelGGL((k_lif_carry_wave<KMAX <= 16 ? 16 : 32>), dim3((unsigned)N), dim3(WAVE), 0, st, I, u0, F(L.EC),
                       F(L.EA), F(L.EB), F(L.MA), F(L.MB), Iq(L.CNT), Iq(L.OVFRAW), F(L.MX),
                       F(L.MC), lo_neuron, F(L.LO), Iq(L.MN), Iq(L.OVF), F(L.STARTS),
                       reinterpret_cast<WsHeader*>(ws), N, M, C, K, beta, theta, u_r);
    return false;
  }
  // The staged carry's LDS (two stages of R chunk maps, ~130 KB at K 8) leaves one block per CU,
  // so beyond one block per CU its walks run in rounds while the lane carry keeps every walk
  // resident.  Measured at cfg2 (N 65536, 1024 blocks), the map scan at C 32 / 64 (K 8): beta
  // 0.9 1.97 / 1.50 -> 1.72 / 1.33 ms, beta 0.99 2.34 / 1.85 -> 1.49 / 1.29 ms with the lane carry.
  if (M >= 4 * CarryStage<KMAX>::R && KMAX <= 32 && NB <= kStagedCarryMaxBlocks) {
    // long chunk sequences: map reads staged through LDS by three loader waves
    hipLaunchKernelGGL((k_lif_carry_staged<KMAX>), dim3((unsigned)NB), dim3(256), 0, st, I, u0,
                       F(L.EC), F(L.EA), F(L.EB), F(L.MA), F(L.MB), Iq(L.CNT), Iq(L.OVFRAW), F(L.MX),
                       F(L.MC), lo_neuron, F(L.LO), Iq(L.MN), Iq(L.OVF), F(L.STARTS),
                       reinterpret_cast<WsHeader*>(ws), N, M, C, K, beta, theta, u_r, rU, rS, rE,
                       rD);
    return rD != nullptr;
  }
  hipLaunchKernelGGL((k_lif_carry<KMAX>), dim3((unsigned)NB), dim3(WAVE), 0, st, I, u0, F(L.EC),
                     F(L.EA), F(L.EB), F(L.MA), F(L.MB), Iq(L.CNT), Iq(L.OVFRAW), F(L.MX), F(L.MC),
                     lo_neuron, F(L.LO), Iq(L.MN), Iq(L.OVF), F(L.STARTS),
                     reinterpret_cast<WsHeader*>(ws), N, M, C, K, beta, theta, u_r, rU, rS, rE, rD);
  return rD != nullptr;
}

template <int KMAX>
static bool launch_build_carry(const float* I, const float* u0, const float* lo_neuron, char* ws,
                               const lsh_v3_layout& L, int64_t N, int M, int C, int K, float beta,
                               float theta, float u_r, hipStream_t st, const ReplayInto* RP) {
  launch_build<KMAX>(I, u0, ws, L, N, M, C, K, beta, theta, u_r, st);
  return launch_carry<KMAX>(I, u0, lo_neuron, ws, L, N, M, C, K, beta, theta, u_r, st, RP);
}

static bool lif_carry_launch(const float* I, const float* u0, char* ws, const lsh_v3_layout& L,
                             int64_t N, int M, int C, int K, float beta, float theta, float u_r,
                             hipStream_t st, const ReplayInto* RP) {
  if (K <= 4) return launch_carry<4>(I, u0, nullptr, ws, L, N, M, C, K, beta, theta, u_r, st, RP);
  if (K <= 8) return launch_carry<8>(I, u0, nullptr, ws, L, N, M, C, K, beta, theta, u_r, st, RP);
  if (K <= 16) return launch_carry<16>(I, u0, nullptr, ws, L, N, M, C, K, beta, theta, u_r, st, RP);
  if (K <= 32) return launch_carry<32>(I, u0, nullptr, ws, L, N, M, C, K, beta, theta, u_r, st, RP);
  return launch_carry<64>(I, u0, nullptr, ws, L, N, M, C, K, beta, theta, u_r, st, RP);
}

// One non-blocking side stream per device (default priority), created on first use on the
// current device and kept until the process ends.
static hipStream_t side_stream() {
  static std::mutex mu;
  static hipStream_t streams[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  if (streams[dev] == nullptr &&
      hipStreamCreateWithFlags(&streams[dev], hipStreamNonBlocking) != hipSuccess)
    streams[dev] = nullptr;
  return streams[dev];
}

// Build kernel alone (used by the three-level scan).
int lif_build_t_launch(const float* I, const float* u0, char* ws, const lsh_v3_layout& L,
                       int64_t N, int M, int C, int K, float beta, float theta, float u_r,
                       hipStream_t st, float* XT, float* CT);
int lif_build_launch(const float* I, const float* u0, char* ws, const lsh_v3_layout& L, int64_t N,
                     int M, int C, int K, float beta, float theta, float u_r, hipStream_t st) {
  return lif_build_t_launch(I, u0, ws, L, N, M, C, K, beta, theta, u_r, st, nullptr, nullptr);
}

// The same, also writing the maps' slots transposed ([M, N, K]) into XT, CT when given.
int lif_build_t_launch(const float* I, const float* u0, char* ws, const lsh_v3_layout& L,
                       int64_t N, int M, int C, int K, float beta, float theta, float u_r,
                       hipStream_t st, float* XT, float* CT) {
  if (K <= 4) launch_build<4>(I, u0, ws, L, N, M, C, K, beta, theta, u_r, st, XT, CT);
  else if (K <= 8) launch_build<8>(I, u0, ws, L, N, M, C, K, beta, theta, u_r, st, XT, CT);
  else if (K <= 16) launch_build<16>(I, u0, ws, L, N, M, C, K, beta, theta, u_r, st, XT, CT);
  else if (K <= 32) launch_build<32>(I, u0, ws, L, N, M, C, K, beta, theta, u_r, st, XT, CT);
  else launch_build<64>(I, u0, ws, L, N, M, C, K, beta, theta, u_r, st, XT, CT);
  return LSH_OK;
}

// Replay of every chunk from its carried start (but the blocks flagged in done, which the
// carry replayed), then the device repair rounds.
void lif_replay_repair_done_launch(const float* I, float* U, float* S, float* starts, float* ends,
                                   int* list0, int* list1, WsHeader* hdr, int64_t N, int M, int C,
                                   int64_t repair, float beta, float theta, float u_r,
                                   hipStream_t st, const int* done) {
  launch_fwd_auto(I, starts, U, S, ends, N, C, M, beta, theta, u_r, st, done);
  lif_repair_launch(I, U, S, starts, ends, list0, list1, hdr, N, M, C, repair, beta, theta, u_r,
                    st);
}

void lif_replay_repair_launch(const float* I, const float* u0, float* U, float* S, float* starts,
                              float* ends, int* list0, int* list1, WsHeader* hdr, int64_t N, int M,
                              int C, int64_t repair, float beta, float theta, float u_r,
                              hipStream_t st) {
  lif_replay_repair_done_launch(I, U, S, starts, ends, list0, list1, hdr, N, M, C, repair, beta,
                                theta, u_r, st, nullptr);
}

// The segmented ordered repair (k_lif_repair_seg): from this many chunks, with fewer neurons
// than the ordered pass needs; at most kRepairSegRounds rounds, then the ordered walk over all
// chunks if the last round still changed a boundary (a run of wrong starts across more
// segment boundaries than that).  LSH_REPAIR_SEG=0 in the environment turns it off (the
// Jacobi rounds run instead), for measurements.
constexpr int kRepairSegMinM = 1024;
constexpr int kRepairSegMinR = 64;
constexpr int kRepairSegRounds = 32;

static int env_int(const char* name, int dflt) {
  const char* e = getenv(name);
  return e && e[0] ? atoi(e) : dflt;
}

static bool repair_seg_enabled() {
  static const bool on = env_int("LSH_REPAIR_SEG", 1) != 0;
  return on;
}

// Segments of kRepairSegMinR chunks (LSH_REPAIR_SEG_R overrides it, for measurements).
// Measured on MI355X (beta 0.99, x ~ N(0.012, 0.08^2), N 1024, T 2^20; the v4 pipeline at the
// reference default / the map scan at C 64): segments of 4, 8, 16, 64 chunks 26.9 / 23.7,
// 26.1 / 22.8, 25.4 / 22.4, 24.9 / 22.0 ms against 85.9 / 82.6 with the Jacobi rounds: the
// first round replays about as much as the replay itself (43 % of the starts are wrong, and a
// wave walks a chunk until its last lane meets the stored trajectory), whatever the segment.
// With 256 chunks (N 128 / 1024, T 65536, C 256) the Jacobi rounds were 2-4 % faster, so the
// segments start at kRepairSegMinM chunks.
static int repair_seg_count(int NB, int M) {
  static const int r = max(1, env_int("LSH_REPAIR_SEG_R", kRepairSegMinR));
  (void)NB;
  return max((M - 1) / r, 1);
}

// The device repair rounds alone, after a replay that wrote U, S and ends from starts.
void lif_repair_launch(const float* I, float* U, float* S, float* starts, float* ends, int* list0,
                       int* list1, WsHeader* hdr, int64_t N, int M, int C, int64_t repair,
                       float beta, float theta, float u_r, hipStream_t st) {
  if (repair < 0 && M > 1) {
    // To convergence without the round count.  The ordered pass costs about 3-4 us per 16-row
    // batch of each chunk where some lane of a wave is dirty, walked chunk after chunk; the
    // Jacobi rounds cost per round but work on many chunks at once.  Measured on MI355X at
    // beta = 0.99, x ~ N(0.012, 0.08^2) (every pair equal to the serial recurrence): N = 65536,
    // T = 4096: C = 32 8.78 -> 3.52 ms, C = 64 5.02 -> 3.31, C = 128 2.59 -> 2.32, C = 256
    // 1.58 vs 1.65 (Jacobi); N = 8192: C = 32 1.15 -> 0.85, C = 128 0.47 vs 0.75 (Jacobi);
    // N = 1024, T = 65536, C = 256: 3.63 vs 5.77 (Jacobi, 16 waves).
    // (segments of the ordered walk did not pay with many neurons: N = 65536, T = 4096,
    // beta 0.99, C 32, 1024 waves walking 128 chunks each 3.39 ms, 4096 to 16384 waves in
    // segments of 8 or 16 chunks 3.84-4.34 ms; the walk is bound by the replays, not by waves)
    const int NB = (int)((N + WAVE - 1) / WAVE);
    if ((N >= 4096 && M >= 64) || (N >= 32768 && M >= 32)) {
      hipLaunchKernelGGL(k_lif_repair_ordered<8>, dim3((unsigned)NB), dim3(WAVE), 0, st, I, U,
                         S, starts, ends, N, M, C, beta, theta, u_r, (const int*)nullptr);
      return;
    }
    if (M >= kRepairSegMinM && repair_seg_enabled()) {
      // few neurons, many chunks: the ordered walk over segments, one round per launch
      const int SG = repair_seg_count(NB, M);
      const int R = (M - 1 + SG - 1) / SG;
      const int rounds = min(SG, kRepairSegRounds);
      fill_i32_launch(list0, rounds, 0, st);
      for (int r = 0; r < rounds; ++r)
        hipLaunchKernelGGL(k_lif_repair_seg<8>, dim3((unsigned)((int64_t)SG * NB)), dim3(WAVE), 0,
                           st, I, U, S, starts, ends, list0, N, M, C, R, NB, r, beta, theta, u_r);
      if (rounds < SG)
        hipLaunchKernelGGL(k_lif_repair_ordered<8>, dim3((unsigned)NB), dim3(WAVE), 0, st, I, U,
                           S, starts, ends, N, M, C, beta, theta, u_r,
                           (const int*)(list0 + rounds - 1));
      return;
    }
    repair = M;
  }
  if (repair > 0 && M > 1) {
    // Round r makes the starts of chunks 0..r exact, so M rounds always converge; the cap
    // only bounds the work when NaN inputs make the comparison fail forever.
    const int64_t rounds = repair < (int64_t)M ? repair : (int64_t)M;
    const int NB = (int)((N + WAVE - 1) / WAVE);
    hipLaunchKernelGGL(k_lif_repair, dim3((unsigned)NB), dim3(256), 0, st, I, U, S, starts, ends,
                       list0, list1, hdr, N, M, C, rounds, beta, theta, u_r);
  }
}

}  // namespace lsh

using namespace lsh;

// ---------------------------------------------------------------------------------------
// C ABI
extern "C" int lsh_abi_version(void) { return LSH_ABI_VERSION; }
extern "C" const char* lsh_arch(void) { return "gfx950"; }
extern "C" const char* lsh_status_string(int status) {
  switch (status) {
    case LSH_OK: return "ok";
    case LSH_ERR_ARG: return "invalid argument (null pointer or bad scalar)";
    case LSH_ERR_SHAPE: return "unsupported shape (T, N, C, K or G out of range)";
    case LSH_ERR_DIVISIBILITY: return "T must be divisible by the chunk length (and M by G)";
    case LSH_ERR_WORKSPACE: return "workspace too small or not 256-byte aligned";
    case LSH_ERR_HIP: return "HIP launch/runtime error";
    case LSH_ERR_SCRATCH: return "problem larger than the static scratch array of the _noalloc entry";
    default: return "unknown status";
  }
}

extern "C" int lsh_lif_serial_fwd(const float* I, const float* u0, float* U, float* S, int64_t T,
                                  int64_t N, float beta, float theta, float u_r, void* stream) {
  if (bad_ptr(I) || bad_ptr(u0) || bad_ptr(U) || bad_ptr(S)) return LSH_ERR_ARG;
  if (T < 0 || N < 0 || N > (int64_t)1 << 31) return LSH_ERR_SHAPE;
  if (T == 0 || N == 0) return LSH_OK;
  hipStream_t st = (hipStream_t)stream;
  lif_serial_fwd_pipe(I, u0, U, S, N, T, beta, theta, u_r, st);
  LSH_CHECK_LAUNCH();
  return LSH_OK;
}

extern "C" int lsh_lif_serial_bwd(const float* I, const float* u0, const float* U, const float* S,
                                  const float* GS, const float* GU, float* Lam, int64_t T,
                                  int64_t N, float beta, float theta, float u_r, float alpha,
                                  int detach, void* stream) {
  if (bad_ptr(I) || bad_ptr(u0) || bad_ptr(U) || bad_ptr(S) || bad_ptr(GS) || bad_ptr(Lam))
    return LSH_ERR_ARG;
  if (T < 0 || N < 0 || N > (int64_t)1 << 31) return LSH_ERR_SHAPE;
  if (T == 0 || N == 0) return LSH_OK;
  launch_bwd<false>(I, u0, U, S, GS, GU, nullptr, Lam, nullptr, nullptr, N, T, 1, beta, theta, u_r,
                    alpha, detach != 0, (hipStream_t)stream);
  LSH_CHECK_LAUNCH();
  return LSH_OK;
}

static int v3_check(int64_t T, int64_t N, int C, int K) {
  if (T < 0 || N < 0 || N > (int64_t)1 << 31) return LSH_ERR_SHAPE;
  if (C < 1 || K < 1 || K > 64) return LSH_ERR_SHAPE;
  if (T % C != 0) return LSH_ERR_DIVISIBILITY;
  if ((T / C) * ((N + WAVE - 1) / WAVE) > ((int64_t)1 << 31) - 1) return LSH_ERR_SHAPE;
  return LSH_OK;
}

extern "C" int lsh_lif_scan_v3_layout(int64_t T, int64_t N, int C, int K, lsh_v3_layout* out) {
  if (bad_ptr(out)) return LSH_ERR_ARG;
  const int rc = v3_check(T, N, C, K);
  if (rc != LSH_OK) return rc;
  v3_layout_fill(T, N, C, K, out);
  return LSH_OK;
}

extern "C" size_t lsh_lif_scan_v3_workspace(int64_t T, int64_t N, int C, int K) {
  if (v3_check(T, N, C, K) != LSH_OK) return 0;
  lsh_v3_layout L;
  v3_layout_fill(T, N, C, K, &L);
  return L.total;
}

static int scan2_fwd(const float* I, const float* u0, const float* lo_neuron, float* U, float* S,
                     int64_t T, int64_t N, float beta, float theta, float u_r, int C, int K,
                     int64_t repair, void* ws, size_t ws_bytes, void* stream) {
  if (bad_ptr(I) || bad_ptr(u0) || bad_ptr(U) || bad_ptr(S) || bad_ptr(ws)) return LSH_ERR_ARG;
  if (repair < -1) return LSH_ERR_ARG;
  int rc = v3_check(T, N, C, K);
  if (rc != LSH_OK) return rc;
  lsh_v3_layout L;
  v3_layout_fill(T, N, C, K, &L);
  if (ws_bytes < L.total || (reinterpret_cast<uintptr_t>(ws) & 255u) != 0) return LSH_ERR_WORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  char* w = static_cast<char*>(ws);
  hipLaunchKernelGGL(k_ws_header_reset, dim3(1), dim3(64), 0, st, reinterpret_cast<WsHeader*>(w));
  if (T == 0 || N == 0) {
    LSH_CHECK_LAUNCH();
    return LSH_OK;
  }
  const int M = (int)(T / C);
  // converged without statistics (repair -1): exact fallbacks replayed inside the carry, the
  // block flags in the second repair list (the Jacobi rounds refill their lists from scratch)
  const ReplayInto rp{U, S, reinterpret_cast<float*>(w + L.ENDS), reinterpret_cast<int*>(w + L.LIST1)};
  const ReplayInto* RP = repair < 0 ? &rp : nullptr;
  bool done = false;
  if (K <= 4)
    done = launch_build_carry<4>(I, u0, lo_neuron, w, L, N, M, C, K, beta, theta, u_r, st, RP);
  else if (K <= 8)
    done = launch_build_carry<8>(I, u0, lo_neuron, w, L, N, M, C, K, beta, theta, u_r, st, RP);
  else if (K <= 16)
    done = launch_build_carry<16>(I, u0, lo_neuron, w, L, N, M, C, K, beta, theta, u_r, st, RP);
  else if (K <= 32)
    done = launch_build_carry<32>(I, u0, lo_neuron, w, L, N, M, C, K, beta, theta, u_r, st, RP);
  else
    done = launch_build_carry<64>(I, u0, lo_neuron, w, L, N, M, C, K, beta, theta, u_r, st, RP);
  lif_replay_repair_done_launch(
      I, U, S, reinterpret_cast<float*>(w + L.STARTS), reinterpret_cast<float*>(w + L.ENDS),
      reinterpret_cast<int*>(w + L.LIST0), reinterpret_cast<int*>(w + L.LIST1),
      reinterpret_cast<WsHeader*>(w), N, M, C, repair, beta, theta, u_r, st,
      done ? reinterpret_cast<const int*>(w + L.LIST1) : nullptr);
  LSH_CHECK_LAUNCH();
  return LSH_OK;
}

extern "C" int lsh_lif_scan_v3_fwd(const float* I, const float* u0, float* U, float* S, int64_t T,
                                   int64_t N, float beta, float theta, float u_r, int C, int K,
                                   int64_t repair, void* ws, size_t ws_bytes, void* stream) {
  return scan2_fwd(I, u0, nullptr, U, S, T, N, beta, theta, u_r, C, K, repair, ws, ws_bytes,
                   stream);
}

// The converged two-level scan in P pieces of T/P steps (consecutive chunks).  Piece p's maps
// depend only on its rows of I and on the pruning bound max(u0, theta, u_r), which bounds every
// state of every piece (after one step a state is below theta or equal to u_r), so they are
// the maps of the unsplit scan; the builds run back to back on a side stream.  On the caller's
// stream, piece p waits for its build, then carries, replays and repairs to convergence from
// the last row of U of piece p-1 (u0 for piece 0): each piece is the serial recurrence from
// an exact start, so U and S are the serial recurrence.  The memory-bound replays overlap the
// VALU-bound builds of the later pieces.
static constexpr int kMaxPieces = 64;

// The fork/join events of the pieces path, per device, created on the first call that needs
// them and kept until the process ends (no create/destroy per call).  A call holds its device's
// lock while it records and waits on them, so calls from several host threads do not mix their
// records (a wait takes the event's most recent record at the time it is enqueued).
struct PiecesEvents {
  std::mutex mu;
  hipEvent_t ev[kMaxPieces + 1] = {};
  int made = 0;
};

static PiecesEvents* pieces_events(int P) {
  static PiecesEvents per_dev[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  PiecesEvents* pe = &per_dev[dev];
  std::lock_guard<std::mutex> lock(pe->mu);
  while (pe->made <= P) {
    if (hipEventCreateWithFlags(&pe->ev[pe->made], hipEventDisableTiming) != hipSuccess)
      return nullptr;
    ++pe->made;
  }
  return pe;
}

static int pieces_check(int64_t T, int64_t N, int C, int K, int P, lsh_v3_layout* L,
                        size_t* piece_bytes) {
  if (P < 1 || P > kMaxPieces || C < 1) return LSH_ERR_SHAPE;
  if (T % ((int64_t)C * P) != 0) return LSH_ERR_DIVISIBILITY;
  const int rc = v3_check(T / P, N, C, K);
  if (rc != LSH_OK) return rc;
  v3_layout_fill(T / P, N, C, K, L);
  *piece_bytes = align_up(L->total, 256);
  return LSH_OK;
}

extern "C" size_t lsh_lif_scan_v3_pieces_workspace(int64_t T, int64_t N, int C, int K, int P) {
  lsh_v3_layout L;
  size_t pb = 0;
  if (pieces_check(T, N, C, K, P, &L, &pb) != LSH_OK) return 0;
  return (size_t)P * pb;
}

extern "C" int lsh_lif_scan_v3_pieces_fwd(const float* I, const float* u0, float* U, float* S,
                                          int64_t T, int64_t N, float beta, float theta,
                                          float u_r, int C, int K, int P, void* ws,
                                          size_t ws_bytes, void* stream) {
  if (bad_ptr(I) || bad_ptr(u0) || bad_ptr(U) || bad_ptr(S) || bad_ptr(ws)) return LSH_ERR_ARG;
  lsh_v3_layout L;
  size_t pb = 0;
  const int rc = pieces_check(T, N, C, K, P, &L, &pb);
  if (rc != LSH_OK) return rc;
  if (ws_bytes < (size_t)P * pb || (reinterpret_cast<uintptr_t>(ws) & 255u) != 0)
    return LSH_ERR_WORKSPACE;
  if (T == 0 || N == 0) return LSH_OK;
  hipStream_t st = (hipStream_t)stream;
  hipStream_t side = st;  // the caller's stream may be the null stream (handle 0)
  if (P > 1 && (side = side_stream()) == nullptr) return LSH_ERR_HIP;
  char* w = static_cast<char*>(ws);
  const int64_t Tp = T / P;
  const int Mp = (int)(Tp / C);
  PiecesEvents* pe = pieces_events(P);
  if (pe == nullptr) return LSH_ERR_HIP;
  bool ok = true;
  {
    std::lock_guard<std::mutex> lock(pe->mu);
    hipEvent_t* ev = pe->ev;
    // fork: the builds start after the work already queued on the caller's stream
    ok = hipEventRecord(ev[P], st) == hipSuccess && hipStreamWaitEvent(side, ev[P], 0) == hipSuccess;
    for (int p = 0; ok && p < P; ++p) {
      char* wp = w + (size_t)p * pb;
      hipLaunchKernelGGL(k_ws_header_reset, dim3(1), dim3(64), 0, side,
                         reinterpret_cast<WsHeader*>(wp));
      lif_build_launch(I + (size_t)p * Tp * N, u0, wp, L, N, Mp, C, K, beta, theta, u_r, side);
      ok = hipEventRecord(ev[p], side) == hipSuccess;
    }
    for (int p = 0; ok && p < P; ++p) {
      ok = hipStreamWaitEvent(st, ev[p], 0) == hipSuccess;
      if (!ok) break;
      char* wp = w + (size_t)p * pb;
      const size_t r0 = (size_t)p * Tp * N;
      const float* up = p == 0 ? u0 : U + r0 - N;
      const ReplayInto rp{U + r0, S + r0, reinterpret_cast<float*>(wp + L.ENDS),
                          reinterpret_cast<int*>(wp + L.LIST1)};
      const bool done = lif_carry_launch(I + r0, up, wp, L, N, Mp, C, K, beta, theta, u_r, st, &rp);
      lif_replay_repair_done_launch(
          I + r0, U + r0, S + r0, reinterpret_cast<float*>(wp + L.STARTS),
          reinterpret_cast<float*>(wp + L.ENDS), reinterpret_cast<int*>(wp + L.LIST0),
          reinterpret_cast<int*>(wp + L.LIST1), reinterpret_cast<WsHeader*>(wp), N, Mp, C, Mp, beta,
          theta, u_r, st, done ? reinterpret_cast<const int*>(wp + L.LIST1) : nullptr);
    }
  }
  if (!ok) return LSH_ERR_HIP;
  LSH_CHECK_LAUNCH();
  return LSH_OK;
}

extern "C" int lsh_lif_scan_lo_fwd(const float* I, const float* u0, const float* lo, float* U,
                                   float* S, int64_t T, int64_t N, float beta, float theta,
                                   float u_r, int C, int K, int64_t repair, void* ws,
                                   size_t ws_bytes, void* stream) {
  if (bad_ptr(lo)) return LSH_ERR_ARG;
  return scan2_fwd(I, u0, lo, U, S, T, N, beta, theta, u_r, C, K, repair, ws, ws_bytes, stream);
}

extern "C" int lsh_scan_stats_read(const void* ws, int64_t chunk_neurons, int64_t super_neurons,
                                   int alif, lsh_scan_stats* out, void* stream) {
  if (bad_ptr(ws) || bad_ptr(out) || chunk_neurons < 0 || super_neurons < 0) return LSH_ERR_ARG;
  WsHeader h;
  hipStream_t st = (hipStream_t)stream;
  if (hipMemcpyAsync(&h, ws, sizeof(h), hipMemcpyDeviceToHost, st) != hipSuccess) return LSH_ERR_HIP;
  if (hipStreamSynchronize(st) != hipSuccess) return LSH_ERR_HIP;
  const double cn = chunk_neurons > 0 ? (double)chunk_neurons : 1.0;
  const double sn = super_neurons > 0 ? (double)super_neurons : 1.0;
  out->repair_iters = (int64_t)h.repair_iters;
  out->overflow_frac = (double)h.ovf_count / cn;
  if (alif == 2) {  // affine reset: pieces kept, no +1
    out->mean_pieces = (double)h.pieces_sum / cn;
    out->max_pieces = (int64_t)h.pieces_max;
    out->miss_frac = 0.0;
    out->mean_lines = 0.0;
  } else if (alif) {
    const unsigned long long miss = ((unsigned long long)h.miss_count_hi << 32) | h.miss_count_lo;
    out->mean_pieces = (double)h.alif_pieces_sum / cn;
    out->max_pieces = (int64_t)h.alif_pieces_max;
    out->miss_frac = (double)miss / cn;
    out->mean_lines = (double)h.lines_sum / cn;
  } else {
    out->mean_pieces = (double)h.pieces_sum / cn + 1.0;
    out->max_pieces = (int64_t)h.pieces_max + 1;
    out->miss_frac = 0.0;
    out->mean_lines = 0.0;
  }
  out->fused_fixups = (int64_t)h.fused_fixups;
  out->fused_unknown = (int64_t)h.fused_unknown;
  out->spin_timeouts = (int64_t)h.spin_timeouts;
  out->super_overflow_frac = (double)h.super_ovf_count / sn;
  out->super_mean_pieces = (double)h.super_pieces_sum / sn + 1.0;
  out->super_max_pieces = (int64_t)h.super_pieces_max + 1;
  return LSH_OK;
}

static int bwd_check(int64_t T, int64_t N, int C) {
  if (T < 0 || N < 0 || N > (int64_t)1 << 31) return LSH_ERR_SHAPE;
  if (C < 1) return LSH_ERR_SHAPE;
  if (T % C != 0) return LSH_ERR_DIVISIBILITY;
  if ((T / C) * ((N + WAVE - 1) / WAVE) > ((int64_t)1 << 31) - 1) return LSH_ERR_SHAPE;
  return LSH_OK;
}

extern "C" size_t lsh_lif_scan_bwd_workspace(int64_t T, int64_t N, int C) {
  if (bwd_check(T, N, C) != LSH_OK) return 0;
  const size_t mn = (size_t)(T / C) * (size_t)N * 4;
  return kWsHeaderBytes + 3 * align_up(mn, 256);
}

extern "C" int lsh_lif_scan_bwd(const float* I, const float* u0, const float* U, const float* S,
                                const float* GS, const float* GU, float* Lam, int64_t T, int64_t N,
                                float beta, float theta, float u_r, float alpha, int detach, int C,
                                void* ws, size_t ws_bytes, void* stream) {
  if (bad_ptr(I) || bad_ptr(u0) || bad_ptr(U) || bad_ptr(S) || bad_ptr(GS) || bad_ptr(Lam) ||
      bad_ptr(ws))
    return LSH_ERR_ARG;
  const int rc = bwd_check(T, N, C);
  if (rc != LSH_OK) return rc;
  if (ws_bytes < lsh_lif_scan_bwd_workspace(T, N, C) ||
      (reinterpret_cast<uintptr_t>(ws) & 255u) != 0)
    return LSH_ERR_WORKSPACE;
  if (T == 0 || N == 0) return LSH_OK;
  hipStream_t st = (hipStream_t)stream;
  const int64_t M = T / C;
  const size_t mn = align_up((size_t)M * (size_t)N * 4, 256);
  char* w = static_cast<char*>(ws) + kWsHeaderBytes;
  float* PA = reinterpret_cast<float*>(w);
  float* PB = reinterpret_cast<float*>(w + mn);
  float* LE = reinterpret_cast<float*>(w + 2 * mn);
  launch_bwd<true>(I, u0, U, S, GS, GU, nullptr, nullptr, PA, PB, N, C, M, beta, theta, u_r, alpha,
                   detach != 0, st);
  hipLaunchKernelGGL(k_lif_bwd_carry, dim3((unsigned)((N + WAVE - 1) / WAVE)), dim3(WAVE), 0, st, PA,
                     PB, LE, N, (int)M);
  launch_bwd<false>(I, u0, U, S, GS, GU, LE, Lam, nullptr, nullptr, N, C, M, beta, theta, u_r,
                    alpha, detach != 0, st);
  LSH_CHECK_LAUNCH();
  return LSH_OK;
}

extern "C" int64_t lsh_lif_param_partials(int64_t T, int64_t N, int mode, int C) {
  if (T < 0 || N < 0 || mode < 0 || mode > 3) return -1;
  const int64_t NB = (N + WAVE - 1) / WAVE;
  if (mode == 3) return T % 256 == 0 ? (T / 256) * NB : -1;  // look-back: one row per tile
  if (mode != 1) return NB;
  if (C < 1 || T % C != 0) return -1;
  return (T / C) * NB;
}

// The detached adjoint with parameter sums; ps 1: hard reset (fit.py), ps 2: affine reset
// with `ur_or_gamma` = gamma (triton_affine.py:229-242).
template <int PS>
static int param_bwd(const float* I, const float* u0, const float* U, const float* S,
                     const float* GS, float* Lam, double* partials, int64_t T, int64_t N, float beta,
                     float theta, float ur_or_gamma, float alpha, int mode, int C, void* ws,
                     size_t ws_bytes, void* stream) {
  if (bad_ptr(I) || bad_ptr(u0) || bad_ptr(U) || bad_ptr(S) || bad_ptr(GS) || bad_ptr(Lam) ||
      bad_ptr(partials))
    return LSH_ERR_ARG;
  if (T < 0 || N < 0 || N > (int64_t)1 << 31) return LSH_ERR_SHAPE;
  if (mode < 0 || mode > 3) return LSH_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  const float g = ur_or_gamma;
  if (mode == 3)
    return lif_param_bwd_lookback(I, u0, U, S, GS, Lam, partials, ws, ws_bytes, T, N, beta, theta, g,
                                  alpha, PS, st);
  if (mode == 0) {
    if (T == 0 || N == 0) return LSH_OK;
    launch_bwd3<false, true, false, PS>(I, u0, U, S, GS, nullptr, nullptr, Lam, nullptr, nullptr, N, T,
                                        1, beta, theta, g, alpha, st, partials);
    LSH_CHECK_LAUNCH();
    return LSH_OK;
  }
  if (mode == 2)
    return lif_param_bwd_fused(I, u0, U, S, GS, Lam, partials, T, N, beta, theta, g, alpha, C, PS,
                               st);
  const int rc = bwd_check(T, N, C);
  if (rc != LSH_OK) return rc;
  if (bad_ptr(ws) || ws_bytes < lsh_lif_scan_bwd_workspace(T, N, C) ||
      (reinterpret_cast<uintptr_t>(ws) & 255u) != 0)
    return LSH_ERR_WORKSPACE;
  if (T == 0 || N == 0) return LSH_OK;
  const int64_t M = T / C;
  const size_t mn = align_up((size_t)M * (size_t)N * 4, 256);
  char* w = static_cast<char*>(ws) + kWsHeaderBytes;
  float* PA = reinterpret_cast<float*>(w);
  float* PB = reinterpret_cast<float*>(w + mn);
  float* LE = reinterpret_cast<float*>(w + 2 * mn);
  // the compose pass needs the affine reset's J, not the sums
  launch_bwd3<true, true, false, PS == 2 ? 2 : 0>(I, u0, U, S, GS, nullptr, nullptr, nullptr, PA, PB,
                                                  N, C, M, beta, theta, g, alpha, st);
  hipLaunchKernelGGL(k_lif_bwd_carry, dim3((unsigned)((N + WAVE - 1) / WAVE)), dim3(WAVE), 0, st, PA,
                     PB, LE, N, (int)M);
  launch_bwd3<false, true, false, PS>(I, u0, U, S, GS, nullptr, LE, Lam, nullptr, nullptr, N, C, M,
                                      beta, theta, g, alpha, st, partials);
  LSH_CHECK_LAUNCH();
  return LSH_OK;
}

extern "C" int lsh_lif_param_bwd(const float* I, const float* u0, const float* U, const float* S,
                                 const float* GS, float* Lam, double* partials, int64_t T, int64_t N,
                                 float beta, float theta, float u_r, float alpha, int mode, int C,
                                 void* ws, size_t ws_bytes, void* stream) {
  return param_bwd<1>(I, u0, U, S, GS, Lam, partials, T, N, beta, theta, u_r, alpha, mode, C, ws,
                      ws_bytes, stream);
}

extern "C" int lsh_aff_bwd(const float* I, const float* u0, const float* U, const float* S,
                           const float* GS, float* Lam, double* partials, int64_t T, int64_t N,
                           float beta, float theta, float gamma, float alpha, int mode, int C,
                           void* ws, size_t ws_bytes, void* stream) {
  if (!(gamma >= 0.0f && gamma <= 1.0f)) return LSH_ERR_ARG;
  return param_bwd<2>(I, u0, U, S, GS, Lam, partials, T, N, beta, theta, gamma, alpha, mode, C, ws,
                      ws_bytes, stream);
}
