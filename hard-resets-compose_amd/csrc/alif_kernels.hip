// Adaptive-threshold LIF (ALIF) kernels for MI355X (gfx950).  Reference: lifscan/triton_alif.py.
//
//   v = fl(fl(beta*u) + x);  s = v >= fl(theta0 + w);  u' = s ? u_r : v;
//   w' = s ? fl(fl(rho*w) + q) : fl(rho*w)                          (triton_alif.py:26-31)
//
// Forward: serial / replay (k_alif_fwd), warm-up predictor (k_alif_warm), and the exact
// box scan: chunk maps over an entry box [lu, hu) x [lw, hw] (k_alif_build), verified carry
// with serial fallback (k_alif_carry), replay, Jacobi repair on device (k_alif_repair).
// Backward: the adjoint as two affine recurrences (triton_alif.py:361-365)
//   lw_{t-1} = (rho - q*sg_t)*lw_t - sg_t*g_t        LW[t] = lw_t = dL/dw_t
//   lv_t     = (1 - s_t)*beta*lv_{t+1} + sg_t*(g_t + q*lw_t)   LV[t] = dL/dv_t = dL/dI_t
// solved serially, as chunked two-level scans, or in one fused pass.
//
// Map layout (workspace): per-chunk scalars [M, N]; line and piece slots [M, N, K]
// (slot-contiguous, so the 32 lanes of one neuron store 128 contiguous bytes).  Only the slots
// below the line and piece counts are written; the others keep whatever the workspace held.
#include "lsh_abi.h"
#include "lsh_common.h"
#include "lsh_lookback.h"

namespace lsh {

__device__ __forceinline__ float alif_step(float u, float& w, float x, float beta, float rho,
                                           float q, float theta0, float u_r, bool& s) {
  const float v = lif_v(u, x, beta);
  s = v >= theta0 + w;
  const float rw = rho * w;
  w = s ? rw + q : rw;
  return s ? u_r : v;
}

// The four parameters from device memory, [beta, rho, q, theta0] as fp32, for callers that keep
// them on the device (a 0-d tensor per parameter): no device-to-host read before the launch.
__device__ __forceinline__ void alif_params_from(const float* __restrict__ p, float& beta,
                                                 float& rho, float& q, float& theta0) {
  beta = p[0];
  rho = p[1];
  q = p[2];
  theta0 = p[3];
}

// numpy-style min/max (a NaN operand gives NaN), as the oracle evaluates them
__device__ __forceinline__ float nmin(float a, float b) {
  return (a != a) ? a : ((b != b) ? b : (a < b ? a : b));
}
__device__ __forceinline__ float nmax(float a, float b) {
  return (a != a) ? a : ((b != b) ? b : (a > b ? a : b));
}

// ---------------------------------------------------------------------------------------
// Serial / replay forward over segments of Ls steps from (su, sw) (triton_alif.py:46-71).
template <int D>
__global__ __launch_bounds__(64) void k_alif_fwd(const float* __restrict__ I,
                                                 const float* __restrict__ su,
                                                 const float* __restrict__ sw, float* __restrict__ U,
                                                 float* __restrict__ W, float* __restrict__ S,
                                                 float* __restrict__ eu, float* __restrict__ ew,
                                                 int64_t N, int64_t Ls, int NB, float beta, float rho,
                                                 float q, float theta0, float u_r,
                                                 const float* __restrict__ dpar,
                                                 const int* __restrict__ mstar) {
  if (dpar) alif_params_from(dpar, beta, rho, q, theta0);
  const int64_t m = blockIdx.x / NB;
  const int nb = (int)(blockIdx.x - m * NB);
  const int64_t n = (int64_t)nb * WAVE + threadIdx.x;
  if (n >= N) return;
  if (mstar && m >= mstar[n]) return;  // a start that a later serial pass replaces
  float u = su[m * N + n], w = sw[m * N + n];
  const size_t base = (size_t)m * (size_t)Ls * (size_t)N + (size_t)n;
  const float* __restrict__ Ip = I + base;
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
#pragma unroll
      for (int j = 0; j < D; ++j) xb[j] = Ip[(size_t)((b + 1) * D + j) * N];
    }
#pragma unroll
    for (int j = 0; j < D; ++j) {
      bool s;
      u = alif_step(u, w, xa[j], beta, rho, q, theta0, u_r, s);
      const size_t o = base + (size_t)(b * D + j) * N;
      st_nt(U + o, u);
      st_nt(W + o, w);
      st_nt(S + o, s ? 1.0f : 0.0f);
    }
    if (more) {
#pragma unroll
      for (int j = 0; j < D; ++j) xa[j] = xb[j];
    }
  }
  for (int64_t t = nt * D; t < Ls; ++t) {
    bool s;
    u = alif_step(u, w, Ip[(size_t)t * N], beta, rho, q, theta0, u_r, s);
    const size_t o = base + (size_t)t * N;
    st_nt(U + o, u);
    st_nt(W + o, w);
    st_nt(S + o, s ? 1.0f : 0.0f);
  }
  if (eu) {
    eu[m * N + n] = u;
    ew[m * N + n] = w;
  }
}

// Warm-up predictor (triton_alif.py:75-92): chunk m simulates chunks max(m-Wn,0)..m-1.
__global__ __launch_bounds__(64) void k_alif_warm(const float* __restrict__ I,
                                                  const float* __restrict__ u0,
                                                  const float* __restrict__ w0,
                                                  const float* __restrict__ UI,
                                                  const float* __restrict__ WI, float* __restrict__ WP,
                                                  int64_t N, int NB, int C, int Wn, float u_init,
                                                  float w_init, float beta, float rho, float q,
                                                  float theta0, float u_r) {
  const int64_t m = blockIdx.x / NB;
  const int nb = (int)(blockIdx.x - m * NB);
  const int64_t n = (int64_t)nb * WAVE + threadIdx.x;
  if (n >= N) return;
  const int64_t s0 = m - Wn > 0 ? m - Wn : 0;
  float u, w;
  if (s0 == 0) {
    u = u0[n];
    w = w0[n];
  } else if (UI) {
    u = UI[s0 * N + n];
    w = WI[s0 * N + n];
  } else {
    u = u_init;
    w = w_init;
  }
  for (int64_t t = s0 * C; t < m * C; ++t) {
    bool s;
    u = alif_step(u, w, I[(size_t)t * N + n], beta, rho, q, theta0, u_r, s);
  }
  WP[m * N + n] = w;
}

// Chunk envelope maps (triton_lif.py:699-719) and the sequential carry to per-chunk lower
// bounds (:723-733): the hard-reset envelope also bounds ALIF potentials from below.
__global__ __launch_bounds__(64) void k_env_chunks(const float* __restrict__ I,
                                                   float* __restrict__ EC, float* __restrict__ EA,
                                                   float* __restrict__ EB, int64_t N, int NB, int C,
                                                   float beta, float u_r) {
  const int64_t m = blockIdx.x / NB;
  const int nb = (int)(blockIdx.x - m * NB);
  const int64_t n = (int64_t)nb * WAVE + threadIdx.x;
  if (n >= N) return;
  float c = INFINITY, a = 1.0f, b = 0.0f;
  const float* __restrict__ Ip = I + (size_t)m * C * N + n;
  for (int j = 0; j < C; ++j) {
    const float x = Ip[(size_t)j * N];
    c = fminf(u_r, lif_v(c, x, beta));
    a = beta * a;
    b = lif_v(b, x, beta);
  }
  EC[m * N + n] = c;
  EA[m * N + n] = a;
  EB[m * N + n] = b;
}

// The chunk maps are read in tiles of kEnvD chunks, the next tile's loads (indices clamped to
// M - 1, so every load is issued) in flight while a tile is folded: with few neurons one wave
// walks all M chunks, and a load per chunk would cost a memory latency each.
constexpr int kEnvD = 16;
__global__ __launch_bounds__(64) void k_env_carry(const float* __restrict__ u0,
                                                  const float* __restrict__ EC,
                                                  const float* __restrict__ EA,
                                                  const float* __restrict__ EB,
                                                  float* __restrict__ LO, int64_t N, int M) {
  const int64_t n = (int64_t)blockIdx.x * WAVE + threadIdx.x;
  if (n >= N || M <= 0) return;
  const float margin = 1e-5f;
  float l = u0[n];
  float ec[kEnvD], ea[kEnvD], eb[kEnvD];
  auto load = [&](int m0, float* c, float* a, float* b) {
#pragma unroll
    for (int k = 0; k < kEnvD; ++k) {
      const size_t o = (size_t)min(m0 + k, M - 1) * N + n;
      c[k] = EC[o];
      a[k] = EA[o];
      b[k] = EB[o];
    }
  };
  load(0, ec, ea, eb);
  for (int m0 = 0; m0 < M; m0 += kEnvD) {
    float nc[kEnvD], na[kEnvD], nbb[kEnvD];
    load(m0 + kEnvD, nc, na, nbb);
#pragma unroll
    for (int k = 0; k < kEnvD; ++k) {
      if (m0 + k < M) {
        LO[(size_t)(m0 + k) * N + n] = l - margin * (fabsf(l) + 1.0f);
        l = fminf(ec[k], __fadd_rn(__fmul_rn(ea[k], l), eb[k]));
      }
    }
#pragma unroll
    for (int k = 0; k < kEnvD; ++k) {
      ec[k] = nc[k];
      ea[k] = na[k];
      eb[k] = nbb[k];
    }
  }
}

// Entry box of every chunk (triton_alif.py:315-318), from the prediction Wp (Wp[0] = w0):
// lw = max(Wp - dw, 0), hw = Wp + dw, hu = max(theta0 + hw/rho, u_r) + 1e-5(|.| + 1).
__global__ __launch_bounds__(64) void k_alif_box(const float* __restrict__ Wpred,
                                                 const float* __restrict__ w0,
                                                 float* __restrict__ LW, float* __restrict__ HW,
                                                 float* __restrict__ HU, int64_t N, int NB,
                                                 float dw, float rho, float theta0, float u_r) {
  const int64_t m = blockIdx.x / NB;
  const int nb = (int)(blockIdx.x - m * NB);
  const int64_t n = (int64_t)nb * WAVE + threadIdx.x;
  if (n >= N) return;
  const size_t o = (size_t)m * N + n;
  const float wp = m == 0 ? w0[n] : Wpred[o];
  LW[o] = nmax(wp - dw, 0.0f);
  const float hw = wp + dw;
  HW[o] = hw;
  float hu = nmax(theta0 + hw / rho, u_r);
  HU[o] = hu + 1e-5f * (fabsf(hu) + 1.0f);
}

// ---------------------------------------------------------------------------------------
// Box-scan chunk map (triton_alif.py:96-186).  One neuron per 16-lane row of a wave (four
// neurons a wave, a DPP row each): slot s of the neuron's first-spike lines (< K1) and of its
// post-spike pieces (< K2) sits in lane s & 15 of its row, register s >> 4, so a neuron's 32
// slots take two registers per lane and the second is touched only while some neuron of the
// wave holds more than 16 pieces (or lines).  Steps go in tiles of TS:
//  0. the per-neuron line quantities of the tile, which do not depend on the pieces, are
//     computed once per neuron into the wave's own LDS rows (no workgroup barrier): (a) the
//     row's lane 0 runs the sequential recurrences A_j = beta*A, B_j = fl(fl(beta*B) + x_j)
//     and R_j = rho^j; (b) lane i of the row divides for steps 2i and 2i + 1, sj = R_j/A_j,
//     cj = (theta0 - B_j)/A_j, whi_j = min(hw, (hu - cj)/sj), (lu - cj)/sj; (c) the running
//     max wlo_j is a prefix over the row (DPP), and the line's values at wlo_j and whi_j are
//     kept for the dominance test.  Same operations as the serial formulation, so the same
//     bits.  The next tile's inputs are loaded while a tile is processed.
//  1. per step every piece is advanced; pieces cut by the threshold are split and the list
//     compacted: exclusive prefix sum of the output counts over the neuron's slots (DPP row
//     shifts within its row, register 0's total added to register 1's), every output slot's
//     source through an LDS scatter, the sources' fields read from their lanes of the row
//     (every piece first takes the uncut update in place; a split rebuilds the cut neurons'
//     fields from the updated ones, v, rho*of and the cut point z).  The split runs
//     for all neurons of a block of BLK neurons when any of them has a cut (the reference's
//     Triton block): a wave decides for blocks of up to 4 neurons with one ballot; blocks of 8
//     or 16 (a workgroup of 2 or 4 waves) agree through LDS.
//  2. the step's first-spike line u0 >= sj*w0 + cj is added unless an existing line dominates
//     it on [wlo, whi]; its post-spike piece x in [cx*wlo + q, cx*whi + q] (widened) is added.
// Neurons per workgroup: 16 (4 waves) for blocks of up to 4, else one block.
template <int BLK>
struct AlifBuildShape {
  static constexpr int NPW = BLK >= 8 ? BLK : 16;  // neurons per workgroup
  static constexpr int NW = NPW / 4;               // waves per workgroup
};
// Inclusive prefix sum of c over each 16-lane row (DPP row shifts; lanes shifted in from outside
// the row read 0).
__device__ __forceinline__ int row_prefix16(int c) {
  c += __builtin_amdgcn_update_dpp(0, c, 0x111, 0xF, 0xF, true);  // row_shr:1
  c += __builtin_amdgcn_update_dpp(0, c, 0x112, 0xF, 0xF, true);  // row_shr:2
  c += __builtin_amdgcn_update_dpp(0, c, 0x114, 0xF, 0xF, true);  // row_shr:4
  c += __builtin_amdgcn_update_dpp(0, c, 0x118, 0xF, 0xF, true);  // row_shr:8
  return c;
}

// The lanes (a wave-wide mask) of the blocks of BLK neurons, one neuron a 16-lane row, in which
// the ballot b has a lane set.  Wave-uniform arithmetic on the ballot, turned back into a
// per-lane flag by the caller with inverse_ballot.
template <int BLK>
__device__ __forceinline__ unsigned long long block_lanes(unsigned long long b) {
  if (BLK >= 4) return b != 0ull ? ~0ull : 0ull;
  const unsigned lo = (unsigned)b, hi = (unsigned)(b >> 32);
  unsigned mlo, mhi;
  if (BLK == 2) {
    mlo = lo != 0u ? 0xffffffffu : 0u;
    mhi = hi != 0u ? 0xffffffffu : 0u;
  } else {
    mlo = ((lo & 0xffffu) != 0u ? 0xffffu : 0u) | ((lo >> 16) != 0u ? 0xffff0000u : 0u);
    mhi = ((hi & 0xffffu) != 0u ? 0xffffu : 0u) | ((hi >> 16) != 0u ? 0xffff0000u : 0u);
  }
  return ((unsigned long long)mhi << 32) | mlo;
}

// Broadcast of lane L of each 16-lane row to the row (DPP row_newbcast).
template <int L>
__device__ __forceinline__ float row_bcast(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x150 + L, 0xF, 0xF, false));
}

// x of the lane before in the row (DPP row_shr:1); fill for the row's first lane.
__device__ __forceinline__ float row_shr1_fill(float x, float fill) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(__float_as_int(fill), __float_as_int(x), 0x111, 0xF, 0xF, false));
}

// Inclusive prefix of nmax over each 16-lane row in lane order (DPP row shifts; lanes shifted
// in from outside the row contribute -inf), the earlier operand first.
__device__ __forceinline__ float row_prefix_nmax16(float x) {
  const int fill = __float_as_int(-INFINITY);
  x = nmax(__int_as_float(__builtin_amdgcn_update_dpp(fill, __float_as_int(x), 0x111, 0xF, 0xF, false)), x);
  x = nmax(__int_as_float(__builtin_amdgcn_update_dpp(fill, __float_as_int(x), 0x112, 0xF, 0xF, false)), x);
  x = nmax(__int_as_float(__builtin_amdgcn_update_dpp(fill, __float_as_int(x), 0x114, 0xF, 0xF, false)), x);
  x = nmax(__int_as_float(__builtin_amdgcn_update_dpp(fill, __float_as_int(x), 0x118, 0xF, 0xF, false)), x);
  return x;
}

constexpr int kAlifTS = 32;   // steps per tile (LDS: 5 x 16 neurons x 33 floats)

// Waves per SIMD the build is compiled for (registers <= 512 / WPE per lane).  Measured at cfg5
// (N 16384, T 4096, BN 4, dw 0.1q / 0.3q) with the per-wave tile phases: 6 (80 VGPRs) 1.68 /
// 2.13 ms, 7 (72 VGPRs, more spilled) 1.88 / 2.32 ms.  The kernel is bound by instruction issue
// (at cfg5 7321 VALU and 5127 scalar instructions per wave; the VALU ones at 4 cycles each fill
// 89 % of the SIMDs' cycles over the launch, the rest waits on the chains between compares, mask
// logic and selects), so a seventh wave hides little and its extra spills cost instructions.
#ifndef LSH_ALIF_BUILD_WPE
#define LSH_ALIF_BUILD_WPE 6
#endif
template <int BLK>
__global__ __launch_bounds__(WAVE * AlifBuildShape<BLK>::NW)
__attribute__((amdgpu_waves_per_eu(LSH_ALIF_BUILD_WPE))) void k_alif_build(
    const float* __restrict__ I, const float* __restrict__ LU, const float* __restrict__ HU,
    const float* __restrict__ LWb, const float* __restrict__ HWb, float* __restrict__ MA,
    float* __restrict__ MB, int* __restrict__ NL, int* __restrict__ NP, int* __restrict__ OVF,
    float* __restrict__ LS, float* __restrict__ LC, float* __restrict__ LX, int* __restrict__ POWN,
    float* __restrict__ PXL, float* __restrict__ PXR, float* __restrict__ PU, float* __restrict__ PA,
    float* __restrict__ POF, int64_t N, int NBLK, int C, int K1, int K2, float beta, float rho,
    float q, float theta0, float u_r) {
  constexpr int NPW = AlifBuildShape<BLK>::NPW;
  constexpr int NW = AlifBuildShape<BLK>::NW;
  constexpr int GW = BLK > 4 ? BLK / 4 : 1;  // waves per split-decision block (> 1: all of them)
  static_assert(GW == 1 || GW == NW, "a split-decision block wider than a wave is one workgroup");
  constexpr int TS = kAlifTS;
  static_assert(TS == 32, "phase (b, c) gives each lane of a row two steps of the tile");
  // one padding column per row: the neurons of a wave read the same step of different rows
  // (and the row leaders of phase (a) walk rows in step), which a 32-float row stride would
  // put on one bank
  constexpr int TSP = TS + 1;
  // a wave's tile rows: its four neurons (rows 4 wv .. 4 wv + 3), written and read by that wave
  // only, so the tile phases need no workgroup barrier
  __shared__ float sX[NPW][TSP], sS[NPW][TSP], sC[NPW][TSP], sHi[NPW][TSP], sLo[NPW][TSP];
  __shared__ float sR[NPW][TSP];                     // rho^j
  __shared__ float sLwl[NPW][TSP], sLwh[NPW][TSP];  // sj*wlo + cj, sj*whi + cj
  __shared__ int s_cut[2][NW];               // per-step split flags (blocks wider than a wave)
  __shared__ int sD[NW][4][32];              // output slot -> (source slot << 1) | spiking part
  const int64_t m = blockIdx.x / NBLK;
  const int blk = (int)(blockIdx.x - m * NBLK);
  const int tid = threadIdx.x;
  const int wv = tid / WAVE;
  const int lane = tid % WAVE;
  const int g = lane >> 4;         // neuron of this lane within the wave (its DPP row)
  const int i = lane & 15;         // slot i (register 0) and 16 + i (register 1)
  const int rowb = lane & 48;      // the row's first lane
  const int ln = wv * 4 + g;       // neuron of this lane within the workgroup
  const int64_t n = (int64_t)blk * NPW + ln;
  const bool valid_n = n < N;
  const int64_t nn = valid_n ? n : N - 1;
  const size_t o = (size_t)m * N + nn;
  const unsigned long long vmask = __ballot(valid_n);  // lanes of neurons < N
  // the neuron's entry box, in every lane of its row; pW: the running max of the lower w bound
  const float lu_n = LU[o], hu_n = HU[o], hw_n = HWb[o];
  float pW = LWb[o];
  float pA = 1.0f, pB = 0.0f, pR = 1.0f;  // the chunk's recurrences, in the row's lane 0
  // lines and pieces: index [r] is slot 16 r + i
  float ls[2] = {0.0f, 0.0f}, lc[2] = {INFINITY, INFINITY}, lx[2] = {0.0f, 0.0f};
  int pown[2] = {-1, -1};
  float pxl[2] = {INFINITY, INFINITY}, pxr[2] = {INFINITY, INFINITY}, pu[2] = {0.0f, 0.0f};
  float pa[2] = {1.0f, 1.0f}, pof[2] = {0.0f, 0.0f};
  int nl = 0, npc = 0;
  int ovf = 0;
  // inputs of the row's neuron: lane i holds steps 2i and 2i + 1 of a tile, the next tile's
  // loaded while a tile is processed
  const float* __restrict__ Icol = I + (size_t)m * C * N + nn;
  const int k0 = 2 * i, k1 = 2 * i + 1;
  float xq0 = 0.0f, xq1 = 0.0f;
  {
    const int ts = min(TS, C);
    if (k0 < ts) xq0 = Icol[(size_t)k0 * N];
    if (k1 < ts) xq1 = Icol[(size_t)k1 * N];
  }
  int kstep = 0;  // steps done in this chunk (parity of the split flags)
  for (int j0 = 0; j0 < C; j0 += TS) {
    const int ts = min(TS, C - j0);
    // (a0) the tile's inputs to the wave's rows; the next tile's loads issued
    if (k0 < ts) sX[ln][k0] = xq0;
    if (k1 < ts) sX[ln][k1] = xq1;
    if (j0 + TS < C) {
      const int tn = min(TS, C - j0 - TS);
      if (k0 < tn) xq0 = Icol[(size_t)(j0 + TS + k0) * N];
      if (k1 < tn) xq1 = Icol[(size_t)(j0 + TS + k1) * N];
    }
    __builtin_amdgcn_wave_barrier();
    // (a) the sequential recurrences A_j = beta*A, B_j = fl(fl(beta*B) + x_j), R_j = rho^j, by
    // the row's lane 0 (same operations as the serial formulation, so the same bits)
    if (i == 0) {
      for (int k = 0; k < ts; ++k) {
        const float x = sX[ln][k];
        pA = beta * pA;
        pB = lif_v(pB, x, beta);
        sS[ln][k] = pA;  // A_j, replaced by sj in (b)
        sC[ln][k] = pB;  // B_j, replaced by cj in (b)
        sR[ln][k] = pR;
        pR = rho * pR;
      }
    }
    __builtin_amdgcn_wave_barrier();
    // (b) divisions, lane i of a row for steps 2i and 2i + 1: sj = R_j/A_j, cj = (theta0 -
    // B_j)/A_j, whi_j = min(hw, (hu - cj)/sj), and the candidate (lu - cj)/sj of the running max
    float sj0 = 0.0f, cj0 = 0.0f, hi0 = 0.0f, cd0 = -INFINITY;
    float sj1 = 0.0f, cj1 = 0.0f, hi1 = 0.0f, cd1 = -INFINITY;
    if (k0 < ts) {
      const float Aj = sS[ln][k0];
      sj0 = sR[ln][k0] / Aj;
      cj0 = (theta0 - sC[ln][k0]) / Aj;
      hi0 = nmin(hw_n, (hu_n - cj0) / sj0);
      cd0 = (lu_n - cj0) / sj0;
    }
    if (k1 < ts) {
      const float Aj = sS[ln][k1];
      sj1 = sR[ln][k1] / Aj;
      cj1 = (theta0 - sC[ln][k1]) / Aj;
      hi1 = nmin(hw_n, (hu_n - cj1) / sj1);
      cd1 = (lu_n - cj1) / sj1;
    }
    // (c) the running max wlo before each step, pW folded with the candidates of the steps
    // before it: a prefix over the row in step order (DPP row shifts, earlier operand first).
    // nmax returns its later operand on ties and its earliest NaN, so any grouping gives the
    // sequential fold's bits.
    const float incl = row_prefix_nmax16(nmax(cd0, cd1));
    const float excl = row_shr1_fill(incl, -INFINITY);  // the candidates of steps < 2i
    const float wlo0 = nmax(pW, excl);
    const float wlo1 = nmax(pW, nmax(excl, cd0));
    if (k0 < ts) {
      sS[ln][k0] = sj0;
      sC[ln][k0] = cj0;
      sHi[ln][k0] = hi0;
      sLo[ln][k0] = wlo0;
      sLwl[ln][k0] = sj0 * wlo0 + cj0;  // the step's line at both ends of its w range
      sLwh[ln][k0] = sj0 * hi0 + cj0;
    }
    if (k1 < ts) {
      sS[ln][k1] = sj1;
      sC[ln][k1] = cj1;
      sHi[ln][k1] = hi1;
      sLo[ln][k1] = wlo1;
      sLwl[ln][k1] = sj1 * wlo1 + cj1;
      sLwh[ln][k1] = sj1 * hi1 + cj1;
    }
    pW = nmax(pW, row_bcast<15>(incl));
    __builtin_amdgcn_wave_barrier();
    for (int k = 0; k < ts; ++k) {
      // the step's input and line quantities, read before the piece stage so that their LDS
      // latency overlaps it
      const float x = sX[ln][k];
      const float wlo = sLo[ln][k], whi = sHi[ln][k];
      const float lwl = sLwl[ln][k], lwh = sLwh[ln][k];
      // does any neuron of the wave hold pieces in register 1 (slots 16..31)?
      const bool hi_p = wave_ballot(npc > 16) != 0ull;
      // 1. advance the post-spike pieces; a piece spikes for x <= (v - theta0 - pof)/pa.  Every
      // piece first takes the update of an uncut piece, in place; a split below rebuilds the
      // fields of the cut neurons from these updated fields and from v, rho*pof and z.  Slots
      // from npc on hold no piece: their tests are false, and their (u, a, of), advanced with
      // the others, are never read (a slot that receives a piece gets every field written).
      // The tests are kept as wave masks (a lane's test is its bit): a mask is the compare's
      // own result, where a per-lane bool combined with another is turned into a 0/1 value
      // and compared again for each ballot and each use in another block.
      const float v0 = lif_v(pu[0], x, beta);
      const float rr0 = (v0 - theta0) - pof[0];
      const float pa0 = pa[0];
      const unsigned long long va0m = wave_ballot(i < npc);
      const unsigned long long es0m = va0m & wave_ballot(rr0 > pa0 * pxl[0]);
      const unsigned long long en0m = va0m & wave_ballot(rr0 < pa0 * pxr[0]);
      const bool es0 = __builtin_amdgcn_inverse_ballot_w64(es0m);
      const bool en0 = __builtin_amdgcn_inverse_ballot_w64(en0m);
      const float ro0 = rho * pof[0];
      pu[0] = es0 ? u_r : v0;
      pof[0] = es0 ? ro0 + q : ro0;
      pa[0] = rho * pa0;
      unsigned long long cb = es0m & en0m;
      unsigned long long es1m = 0ull, en1m = 0ull;
      float v1, rr1, pa1, ro1;  // read only where hi_p
      if (hi_p) {
        v1 = lif_v(pu[1], x, beta);
        rr1 = (v1 - theta0) - pof[1];
        pa1 = pa[1];
        const unsigned long long va1m = wave_ballot(16 + i < npc);
        es1m = va1m & wave_ballot(rr1 > pa1 * pxl[1]);
        en1m = va1m & wave_ballot(rr1 < pa1 * pxr[1]);
        const bool es1_ = __builtin_amdgcn_inverse_ballot_w64(es1m);
        ro1 = rho * pof[1];
        pu[1] = es1_ ? u_r : v1;
        pof[1] = es1_ ? ro1 + q : ro1;
        pa[1] = rho * pa1;
        cb |= es1m & en1m;
      }
      const bool es1 = __builtin_amdgcn_inverse_ballot_w64(es1m);
      const bool en1 = __builtin_amdgcn_inverse_ballot_w64(en1m);
      unsigned long long cutm;  // lanes of the neurons whose block has a cut
      if (GW == 1) {
        cutm = block_lanes<BLK>(cb);
      } else {
        // one barrier per step: the flags of step k + 2 reuse this step's buffer only after the
        // barrier of step k + 1, which every wave passes after reading this step's flags
        const int par = kstep & 1;
        if (lane == 0) s_cut[par][wv] = cb != 0ull ? 1 : 0;
        __syncthreads();
        int any = 0;
#pragma unroll
        for (int kk = 0; kk < GW; ++kk) any |= s_cut[par][kk];
        cutm = any != 0 ? ~0ull : 0ull;
      }
      ++kstep;
      if (cutm != 0ull) {
        // split and compaction for the neurons whose block has a cut
        const bool cut = __builtin_amdgcn_inverse_ballot_w64(cutm);
        const float z0 = rr0 / pa0;
        const float z1 = hi_p ? rr1 / pa1 : 0.0f;
        const int nout0 = (es0 ? 1 : 0) + (en0 ? 1 : 0);
        const int nout1 = (es1 ? 1 : 0) + (en1 ? 1 : 0);
        // inclusive prefix sums over the row's 16 lanes (DPP row shifts), the row's totals
        const int incl0 = row_prefix16(nout0);
        const int tot0 = __shfl(incl0, rowb + 15, WAVE);
        int incl1 = 0, tot1 = 0;
        if (hi_p) {
          incl1 = row_prefix16(nout1);
          tot1 = __shfl(incl1, rowb + 15, WAVE);
        }
        const int p0 = incl0 - nout0;
        const int p1 = tot0 + incl1 - nout1;
        const int ntot = tot0 + tot1;
        const int n_new = min(ntot, K2);
        // every output slot learns its source through an LDS scatter (same-wave LDS accesses
        // complete in order, so the reads below see these writes); the sources' fields come
        // from their lanes of the same row by cross-lane reads
        int* dsc = sD[wv][g];
        if (cut) {
          if (nout0 >= 1 && p0 < K2) dsc[p0] = (i << 1) | (es0 ? 1 : 0);
          if (nout0 == 2 && p0 + 1 < K2) dsc[p0 + 1] = i << 1;
          if (nout1 >= 1 && p1 < K2) dsc[p1] = ((16 + i) << 1) | (es1 ? 1 : 0);
          if (nout1 == 2 && p1 + 1 < K2) dsc[p1 + 1] = (16 + i) << 1;
          if (ntot > K2) ovf = 1;
        }
        __builtin_amdgcn_wave_barrier();
        const bool hi_o = wave_ballot(cut && n_new > 16) != 0ull;
        // every gather first, then each field replaced once: a kept part of source piece s has
        // bounds from s's and z, u = u_r (spiking part) or v_s, a = rho*a_s (s's updated a),
        // of = rho*of_s (+ q for the spiking part)
        auto gather = [&](float f0, const float& f1, int sl, bool s1) {  // f1 read where hi_p
          const float a0 = __shfl(f0, sl, WAVE);
          const float a1 = hi_p ? __shfl(f1, sl, WAVE) : 0.0f;
          return s1 ? a1 : a0;
        };
        auto gather_i = [&](int f0, int f1, int sl, bool s1) {
          const int a0 = __shfl(f0, sl, WAVE);
          const int a1 = hi_p ? __shfl(f1, sl, WAVE) : 0;
          return s1 ? a1 : a0;
        };
        const bool keep0 = cut && i < n_new;
        const int src0 = keep0 ? dsc[i] : 0;
        const int idx0 = (src0 >> 1) & 31;
        const bool iss0 = (src0 & 1) != 0;
        const int sl0 = rowb + (idx0 & 15);
        const bool s10 = idx0 >= 16;
        const float g0xl = gather(pxl[0], pxl[1], sl0, s10), g0xr = gather(pxr[0], pxr[1], sl0, s10);
        const float g0z = gather(z0, z1, sl0, s10), g0v = gather(v0, v1, sl0, s10);
        const float g0a = gather(pa[0], pa[1], sl0, s10), g0r = gather(ro0, ro1, sl0, s10);
        const int g0w = gather_i(pown[0], pown[1], sl0, s10);
        bool keep1 = false, iss1 = false;
        float g1xl = 0.0f, g1xr = 0.0f, g1z = 0.0f, g1v = 0.0f, g1a = 0.0f, g1r = 0.0f;
        int g1w = 0;
        if (hi_o) {
          keep1 = cut && 16 + i < n_new;
          const int src1 = keep1 ? dsc[16 + i] : 0;
          const int idx1 = (src1 >> 1) & 31;
          iss1 = (src1 & 1) != 0;
          const int sl1 = rowb + (idx1 & 15);
          const bool s11 = idx1 >= 16;
          g1xl = gather(pxl[0], pxl[1], sl1, s11);
          g1xr = gather(pxr[0], pxr[1], sl1, s11);
          g1z = gather(z0, z1, sl1, s11);
          g1v = gather(v0, v1, sl1, s11);
          g1a = gather(pa[0], pa[1], sl1, s11);
          g1r = gather(ro0, ro1, sl1, s11);
          g1w = gather_i(pown[0], pown[1], sl1, s11);
        }
        pxl[0] = cut ? (keep0 ? (iss0 ? g0xl : nmax(g0xl, g0z)) : INFINITY) : pxl[0];
        pxr[0] = cut ? (keep0 ? (iss0 ? nmin(g0xr, g0z) : g0xr) : INFINITY) : pxr[0];
        pu[0] = cut ? (keep0 ? (iss0 ? u_r : g0v) : 0.0f) : pu[0];
        pa[0] = cut ? (keep0 ? g0a : 1.0f) : pa[0];
        pof[0] = cut ? (keep0 ? (iss0 ? g0r + q : g0r) : 0.0f) : pof[0];
        pown[0] = cut ? (keep0 ? g0w : -1) : pown[0];
        if (hi_o || hi_p) {
          pxl[1] = cut ? (keep1 ? (iss1 ? g1xl : nmax(g1xl, g1z)) : INFINITY) : pxl[1];
          pxr[1] = cut ? (keep1 ? (iss1 ? nmin(g1xr, g1z) : g1xr) : INFINITY) : pxr[1];
          pu[1] = cut ? (keep1 ? (iss1 ? u_r : g1v) : 0.0f) : pu[1];
          pa[1] = cut ? (keep1 ? g1a : 1.0f) : pa[1];
          pof[1] = cut ? (keep1 ? (iss1 ? g1r + q : g1r) : 0.0f) : pof[1];
          pown[1] = cut ? (keep1 ? g1w : -1) : pown[1];
        }
        // reads of this step's sources and slots precede the next step's writes to them
        __builtin_amdgcn_wave_barrier();
        npc = cut ? n_new : npc;
      }
      // 2. first-spike line of this step: added unless a line dominates it on [wlo, whi].  A
      // step has a candidate line (wlo < whi) in some row of the wave on about a fifth of the
      // steps at cfg5, so the dominance tests run only then.
      const unsigned long long candm = wave_ballot(wlo < whi) & vmask;
      unsigned long long newm = 0ull;
      if (candm != 0ull) {
        const bool hi_l = wave_ballot(nl > 16) != 0ull;
        unsigned long long bl = wave_ballot(i < nl) & wave_ballot(ls[0] * wlo + lc[0] <= lwl) &
                                wave_ballot(ls[0] * whi + lc[0] <= lwh);
        if (hi_l)
          bl |= wave_ballot(16 + i < nl) & wave_ballot(ls[1] * wlo + lc[1] <= lwl) &
                wave_ballot(ls[1] * whi + lc[1] <= lwh);
        newm = candm & ~block_lanes<1>(bl);
      }
      if (newm != 0ull) {
        // the new line goes to slot nl and its piece to slot npc, written by selects on both
        // registers so the slots stay in registers; the whole block is skipped on the (most)
        // steps where no row of the wave adds a line
        const bool newc = __builtin_amdgcn_inverse_ballot_w64(newm);
        const float sj = sS[ln][k], cj = sC[ln][k];
        const float cx = sR[ln][k] * rho;
        const bool putl = newc && nl < K1 && i == (nl & 15);
        const bool l1 = nl >= 16;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const bool pl = putl && (r == 1) == l1;
          ls[r] = pl ? sj : ls[r];
          lc[r] = pl ? cj : lc[r];
          lx[r] = pl ? cx : lx[r];
        }
        if (newc && nl >= K1) ovf = 1;
        const float xlo = cx * wlo + q;
        const float xhi = cx * whi + q;
        const float pd = 4e-7f * (fabsf(xhi) + 1.0f);
        const bool putp = newc && npc < K2 && i == (npc & 15);
        const bool p1 = npc >= 16;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const bool pp = putp && (r == 1) == p1;
          pxl[r] = pp ? xlo - pd : pxl[r];
          pxr[r] = pp ? xhi + pd : pxr[r];
          pu[r] = pp ? u_r : pu[r];
          pa[r] = pp ? 1.0f : pa[r];
          pof[r] = pp ? 0.0f : pof[r];
          pown[r] = pp ? nl : pown[r];
        }
        if (newc && npc >= K2) ovf = 1;
        nl = newc ? min(nl + 1, K1) : nl;
        npc = newc ? min(npc + 1, K2) : npc;
      }
    }
    __builtin_amdgcn_wave_barrier();  // the tile's rows are rewritten next
  }
  if (!valid_n) return;
  if (i == 0) {
    MA[o] = pA;
    MB[o] = pB;
    NL[o] = nl;
    NP[o] = npc;
    OVF[o] = ovf;
  }
  // only the populated slots are stored (the carry reads every slot but uses only those below
  // the counts): with 7 lines and 10 pieces a neuron on average, a third of the map bytes
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int slot = 16 * r + i;
    if (slot < K1 && slot < nl) {
      const size_t os = o * K1 + slot;
      LS[os] = ls[r];
      LC[os] = lc[r];
      LX[os] = lx[r];
    }
    if (slot < K2 && slot < npc) {
      const size_t os = o * K2 + slot;
      POWN[os] = pown[r];
      PXL[os] = pxl[r];
      PXR[os] = pxr[r];
      PU[os] = pu[r];
      PA[os] = pa[r];
      POF[os] = pof[r];
    }
  }
}

// 16 serial ALIF steps of a row's neuron: lane i of the 16-lane row holds the input of step i
// in xb, and each step takes its input from that lane by a row broadcast (no load per step).
template <int L = 0>
__device__ __forceinline__ void alif_row_block16(float xb, float& u, float& w, float beta,
                                                 float rho, float q, float theta0, float u_r) {
  if constexpr (L < 16) {
    bool s;
    u = alif_step(u, w, row_bcast<L>(xb), beta, rho, q, theta0, u_r, s);
    alif_row_block16<L + 1>(xb, u, w, beta, rho, q, theta0, u_r);
  }
}

// One chunk's map as the carry reads it (one neuron per 16-lane row, slot s in lane s & 15,
// register s >> 4): the per-neuron header, every slot below K1 / K2 (the slots past the line
// and piece counts hold no map; each use is masked by the counts, so their loads need not
// wait for the header).  The serial fallback reads its inputs in groups of kCarryXB * 16 steps
// (lane i of a row: step 16 b + i in register b).
constexpr int kCarryXB = 8;
constexpr int kCarryWaves = 4;  // waves per workgroup
// Neurons per wave: a wave runs the serial fallback when any of its neurons misses, so with
// few neurons (an idle chip) one neuron a wave (its four rows replicating it) cuts the
// fallbacks; with many, four a wave keep the instruction count per neuron low.  Measured on
// MI355X (lsnn, free mean 1.0, previous-iterate prediction, dw 0.1q, no repair; carry / box
// scan): N 16 0.41 / 0.64 ms against 0.66 / 0.89 with four a wave, N 128 0.33 / 0.77 against
// 0.63 / 1.08, N 512 0.59 / 1.65 against 0.86 / 1.93, N 1024 0.61 / 2.52 against 0.84 / 2.79;
// N 2048 0.54 / 2.44 against 0.48 / 2.37, N 4096 0.54 / 2.39 against 0.32 / 2.19, cfg5 (walking
// every chunk) 1.06 against 0.36 ms carry.  Two a wave was between the two at every size.
#ifndef LSH_ALIF_CARRY_NPW1_MAX_N
#define LSH_ALIF_CARRY_NPW1_MAX_N 1024
#endif
constexpr int64_t kCarryNpw1MaxN = LSH_ALIF_CARRY_NPW1_MAX_N;
struct AlifCarryMap {
  float ma, mb, lu, hu, lw, hw;
  int nl, npc, ovf;
  float ls[2], lc[2], lx[2], pl[2], pr[2], pu[2], pa[2], po[2];
  int pw[2];
};

// Verified carry (triton_alif.py:214-252): the first line that fires gives the first spike
// step and x = lx*w + q; the unique piece of that line containing x gives (u, w) at the
// chunk end.  Out of box, overflow or not exactly one piece: the chunk runs serially.
// One neuron per 16-lane row (four a wave, sixteen a workgroup): slot s of the lines and
// pieces in lane s & 15, register s >> 4, as the build keeps them; a serial fallback runs for
// the lanes of the neurons that need it, once per chunk for the wave.  The maps are read
// PD chunks ahead of the chunk that uses them into a ring of PD + 1 register sets, the chunk
// loop unrolled by the ring's length so that no set is copied (a copy would wait for the loads
// into it).  PD = 1 is what runs: on MI355X 2 and 3 were no faster with 1024 neurons (256
// waves) and slower with 16384 (the extra registers cost waves).  With C a
// multiple of 16 the fallback takes its inputs from registers by row broadcasts (loaded when
// a fallback starts, each later group of 128 steps while the one before is replayed), else it
// streams them row by row.  The fallback's first inputs are not part of the ring: loading them
// with every map cost 8 % to 11 % at 16 to 1024 neurons (N = 16, T = 65536: 0.578 -> 0.516
// ms) for the 4 % to 30 % of chunks that fall back.  Workgroups of neighbouring neurons go to
// one XCD (blockIdx b -> group (b % 8) * per + b / 8), so they share its L2 for the inputs and
// the per-neuron arrays.  The statistics are summed per workgroup before the atomics.
template <int PD, int NPW>
__global__ __launch_bounds__(WAVE * kCarryWaves) void k_alif_carry(
    const float* __restrict__ I, const float* __restrict__ u0, const float* __restrict__ w0,
    const float* __restrict__ LU, const float* __restrict__ HU, const float* __restrict__ LWb,
    const float* __restrict__ HWb, const float* __restrict__ MA, const float* __restrict__ MB,
    const int* __restrict__ NL, const int* __restrict__ NP, const int* __restrict__ OVF,
    const float* __restrict__ LS, const float* __restrict__ LC, const float* __restrict__ LX,
    const int* __restrict__ POWN, const float* __restrict__ PXL, const float* __restrict__ PXR,
    const float* __restrict__ PU, const float* __restrict__ PA, const float* __restrict__ POF,
    float* __restrict__ SU, float* __restrict__ SW, int* __restrict__ MISS,
    int* __restrict__ MSTAR, WsHeader* hdr, int64_t N, int M, int C, int K1, int K2, float beta,
    float rho, float q, float theta0, float u_r, float rhoC, int stop_at_mstar) {
  __shared__ unsigned long long s_acc[kCarryWaves][4];
  __shared__ int s_max[kCarryWaves];
  static_assert(NPW == 1 || NPW == 4, "neurons per wave");
  const int64_t ngroups = (N + NPW * kCarryWaves - 1) / (NPW * kCarryWaves);
  const int64_t per = gridDim.x / 8;
  const int64_t grp = (int64_t)(blockIdx.x % 8) * per + blockIdx.x / 8;
  if (grp >= ngroups) return;  // the whole workgroup (the grid is rounded up to 8 per XCD)
  const int wv = threadIdx.x / WAVE;
  const int lane = threadIdx.x % WAVE;
  const int g = lane >> 4;
  const int i = lane & 15;
  const int rowb = lane & 48;
  // NPW neurons a wave: with one, the four rows hold the same neuron (same loads, same steps,
  // so the same results) and row 0 stores and counts
  const int64_t n = grp * (NPW * kCarryWaves) + wv * NPW + (g % NPW);
  const bool lead = g < NPW;
  const bool valid_n = n < N;
  const int64_t nn = valid_n ? n : N - 1;
  const bool xdpp = (C & 15) == 0;  // the fallback's inputs in registers
  const int nb = C >> 4;            // blocks of 16 steps a chunk (xdpp)
  float u = u0[nn], w = w0[nn];
  // mstar: the first chunk whose start came through a map (so it agrees with the serial
  // recurrence only to rounding); the starts before it came from (u0, w0) through serial
  // replays only, so they are the serial recurrence's states
  int mstar = M;
  unsigned long long miss_acc = 0, ovf_acc = 0, lines_acc = 0, pcs_acc = 0;
  int pmax = 0;
  // the first set bit of this row's part of a wave ballot, or -1
  auto row_first = [&](unsigned long long b) {
    const unsigned int r = (unsigned int)(b >> rowb) & 0xffffu;
    return r ? __builtin_ctz(r) : -1;
  };
  auto row_count = [&](unsigned long long b) {
    return __builtin_popcount((unsigned int)(b >> rowb) & 0xffffu);
  };
  // Every load is issued unconditionally, its index clamped into the arrays (chunk <= M - 1,
  // slot <= K - 1, row <= C - 1; the extra values are never used), so that the compiler knows
  // how many loads were issued after each one and waits for the ring set in use only.
  auto load_map = [&](int m, AlifCarryMap& d) {
    const size_t o = (size_t)min(m, M - 1) * N + nn;
    d.ma = MA[o];
    d.mb = MB[o];
    d.lu = LU[o];
    d.hu = HU[o];
    d.lw = LWb[o];
    d.hw = HWb[o];
    d.nl = NL[o];
    d.npc = NP[o];
    d.ovf = OVF[o];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int sl = min(16 * r + i, K1 - 1), sp = min(16 * r + i, K2 - 1);
      d.ls[r] = LS[o * K1 + sl];
      d.lc[r] = LC[o * K1 + sl];
      d.lx[r] = LX[o * K1 + sl];
      d.pw[r] = POWN[o * K2 + sp];
      d.pl[r] = PXL[o * K2 + sp];
      d.pr[r] = PXR[o * K2 + sp];
      d.pu[r] = PU[o * K2 + sp];
      d.pa[r] = PA[o * K2 + sp];
      d.po[r] = POF[o * K2 + sp];
    }
  };
  // a ring of PD + 1 maps: chunk m in mr[m % (PD + 1)]
  AlifCarryMap mr[PD + 1];
#pragma unroll
  for (int k = 0; k < PD; ++k) load_map(k, mr[k]);
  bool done = false;
  for (int m0 = 0; m0 < M && !done; m0 += PD + 1) {
#pragma unroll
  for (int ph = 0; ph <= PD; ++ph) {
    const int m = m0 + ph;
    if (m >= M) {
      done = true;
      break;
    }
    load_map(m + PD, mr[(ph + PD) % (PD + 1)]);  // the set of chunk m - 1
    const AlifCarryMap& hc = mr[ph];
    const AlifCarryMap& sc = mr[ph];
    const size_t o = (size_t)m * N + nn;
    if (valid_n && lead && i == 0) {
      SU[o] = u;
      SW[o] = w;
    }
    const int nl = hc.nl, npc = hc.npc, ovf = hc.ovf;
    // the first line that fires
    const unsigned long long f0 = __ballot(i < nl && u >= sc.ls[0] * w + sc.lc[0]);
    const unsigned long long f1 = __ballot(16 + i < nl && u >= sc.ls[1] * w + sc.lc[1]);
    const int a0 = row_first(f0), a1 = row_first(f1);
    const int first = a0 >= 0 ? a0 : (a1 >= 0 ? 16 + a1 : K1);
    const bool none_ = first == K1;
    const int fl = rowb + (first & 15);
    const float lx0 = __shfl(sc.lx[0], fl, WAVE), lx1 = __shfl(sc.lx[1], fl, WAVE);  // all lanes
    const float lxf = none_ ? 0.0f : (first >= 16 ? lx1 : lx0);
    const float xq = lxf * w + q;
    // the pieces of that line containing x
    const bool h0 = i < npc && sc.pw[0] == first && sc.pl[0] <= xq && xq < sc.pr[0];
    const bool h1 = 16 + i < npc && sc.pw[1] == first && sc.pl[1] <= xq && xq < sc.pr[1];
    const unsigned long long hm0 = __ballot(h0), hm1 = __ballot(h1);
    const int nh = row_count(hm0) + row_count(hm1);
    const int b0 = row_first(hm0), b1 = row_first(hm1);
    const int hs = b0 >= 0 ? b0 : (b1 >= 0 ? 16 + b1 : 0);  // the first hit slot
    const int hl = rowb + (hs & 15);
    const float pu0 = __shfl(sc.pu[0], hl, WAVE), pu1 = __shfl(sc.pu[1], hl, WAVE);
    const float pw0 = __shfl(sc.pa[0] * xq + sc.po[0], hl, WAVE);
    const float pw1 = __shfl(sc.pa[1] * xq + sc.po[1], hl, WAVE);
    const float mu = nh ? (hs >= 16 ? pu1 : pu0) : 0.0f;
    const float mw = nh ? (hs >= 16 ? pw1 : pw0) : 0.0f;
    float nu = none_ ? __fadd_rn(__fmul_rn(hc.ma, u), hc.mb) : mu;
    float nw = none_ ? rhoC * w : mw;
    const bool inbox = (u >= hc.lu) && (u < hc.hu) && (w >= hc.lw) && (w <= hc.hw);
    const bool bad = !inbox || ovf != 0 || (!none_ && nh != 1);
    if (valid_n && lead && i == 0) MISS[o] = bad ? 1 : 0;
    if (__ballot(bad) != 0ull) {
      float uu = u, ww = w;
      if (xdpp) {
        // groups of 128 steps; the next group's inputs loaded while one is replayed (every
        // lane runs the steps: the row broadcasts read lanes of rows that may not need them)
        const float* xp = I + (size_t)m * C * N + nn;
        float xa[kCarryXB];
#pragma unroll
        for (int b = 0; b < kCarryXB; ++b) xa[b] = xp[(size_t)min(16 * b + i, C - 1) * N];
        for (int g0 = 0; g0 < nb; g0 += kCarryXB) {
          // issued for every group (rows clamped into the chunk, the extra values unused), so
          // the wait for this group's inputs does not cover them
          float xn[kCarryXB];
#pragma unroll
          for (int b = 0; b < kCarryXB; ++b)
            xn[b] = xp[(size_t)min(16 * (g0 + kCarryXB + b) + i, C - 1) * N];
#pragma unroll
          for (int b = 0; b < kCarryXB; ++b)
            if (g0 + b < nb) alif_row_block16(xa[b], uu, ww, beta, rho, q, theta0, u_r);
#pragma unroll
          for (int b = 0; b < kCarryXB; ++b) xa[b] = xn[b];
        }
      } else if (bad) {
        stream_rows<4>(I + (size_t)m * C * N + nn, (size_t)N, C, [&](int64_t, float x) {
          bool s;
          uu = alif_step(uu, ww, x, beta, rho, q, theta0, u_r, s);
        });
      }
      if (bad) {
        nu = uu;
        nw = ww;
      }
    }
    u = nu;
    w = nw;
    if (!bad && mstar == M) mstar = m + 1;
    if (valid_n && lead && i == 0) {
      miss_acc += bad ? 1ull : 0ull;
      ovf_acc += ovf ? 1ull : 0ull;
      lines_acc += (unsigned long long)nl;
      pcs_acc += (unsigned long long)npc;
      pmax = max(pmax, npc);
    }
    // repair to convergence: past every neuron's MSTAR the starts are replaced by the serial
    // pass, so the wave stops (the statistics then cover the chunks it walked)
    if (stop_at_mstar && __ballot(valid_n && mstar == M) == 0ull) {
      done = true;
      break;
    }
  }
  }
  if (valid_n && lead && i == 0) MSTAR[nn] = mstar;
  miss_acc = wave_sum_u64(miss_acc);
  ovf_acc = wave_sum_u64(ovf_acc);
  lines_acc = wave_sum_u64(lines_acc);
  pcs_acc = wave_sum_u64(pcs_acc);
  pmax = wave_max_i(pmax);
  if (lane == 0) {
    s_acc[wv][0] = miss_acc;
    s_acc[wv][1] = ovf_acc;
    s_acc[wv][2] = lines_acc;
    s_acc[wv][3] = pcs_acc;
    s_max[wv] = pmax;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < kCarryWaves; ++k) {
      miss_acc += s_acc[k][0];
      ovf_acc += s_acc[k][1];
      lines_acc += s_acc[k][2];
      pcs_acc += s_acc[k][3];
      pmax = max(pmax, s_max[k]);
    }
    const unsigned long long old_lo =
        atomicAdd(&hdr->miss_count_lo, (unsigned int)(miss_acc & 0xffffffffull));
    const unsigned int carry = (old_lo + (miss_acc & 0xffffffffull)) > 0xffffffffull ? 1u : 0u;
    atomicAdd(&hdr->miss_count_hi, (unsigned int)(miss_acc >> 32) + carry);
    atomicAdd(&hdr->ovf_count, ovf_acc);
    atomicAdd(&hdr->lines_sum, lines_acc);
    atomicAdd(&hdr->alif_pieces_sum, pcs_acc);
    atomicMax(&hdr->alif_pieces_max, (unsigned int)pmax);
  }
}

// Jacobi repair of (u, w) chunk starts, as k_lif_repair (triton_alif.py:342-348).
__global__ __launch_bounds__(256) void k_alif_repair(
    const float* __restrict__ I, float* __restrict__ U, float* __restrict__ W,
    float* __restrict__ S, float* __restrict__ su, float* __restrict__ sw, float* __restrict__ eu,
    float* __restrict__ ew, int* __restrict__ list0, int* __restrict__ list1, WsHeader* hdr,
    int64_t N, int M, int C, int64_t R, float beta, float rho, float q, float theta0, float u_r) {
  __shared__ int s_nd, s_nc;
  const int nb = blockIdx.x;
  const int tid = threadIdx.x;
  const size_t cap = (size_t)M * WAVE;
  int* __restrict__ dl = list0 + (size_t)nb * cap;
  int* __restrict__ cl = list1 + (size_t)nb * cap;
  auto differs = [&](int m, int64_t n) {
    const size_t a = (size_t)(m - 1) * N + n, b = (size_t)m * N + n;
    return eu[a] != su[b] || ew[a] != sw[b];
  };
  if (tid == 0) s_nd = 0;
  __syncthreads();
  for (int e = tid + WAVE; e < M * WAVE; e += blockDim.x) {
    const int m = e / WAVE;
    const int64_t n = (int64_t)nb * WAVE + (e % WAVE);
    if (n < N && differs(m, n)) dl[atomicAdd(&s_nd, 1)] = e;
  }
  __syncthreads();
  int64_t rounds = 0;
  while (true) {
    const int nd = s_nd;
    if (nd == 0 || rounds >= R) break;
    ++rounds;
    for (int k = tid; k < nd; k += blockDim.x) {
      const int e = dl[k];
      const int m = e / WAVE;
      const int64_t n = (int64_t)nb * WAVE + (e % WAVE);
      su[(size_t)m * N + n] = eu[(size_t)(m - 1) * N + n];
      sw[(size_t)m * N + n] = ew[(size_t)(m - 1) * N + n];
    }
    __syncthreads();
    if (tid == 0) s_nc = 0;
    __syncthreads();
    for (int k = tid; k < nd; k += blockDim.x) {
      const int e = dl[k];
      const int m = e / WAVE;
      const int64_t n = (int64_t)nb * WAVE + (e % WAVE);
      float u = su[(size_t)m * N + n], w = sw[(size_t)m * N + n];
      const size_t base = (size_t)m * C * N + n;
      stream_rows<16>(I + base, (size_t)N, C, [&](int64_t j, float x) {
        bool s;
        u = alif_step(u, w, x, beta, rho, q, theta0, u_r, s);
        U[base + (size_t)j * N] = u;
        W[base + (size_t)j * N] = w;
        S[base + (size_t)j * N] = s ? 1.0f : 0.0f;
      });
      const size_t oe = (size_t)m * N + n;
      if (u != eu[oe] || w != ew[oe]) {
        eu[oe] = u;
        ew[oe] = w;
        if (m + 1 < M) cl[atomicAdd(&s_nc, 1)] = e + WAVE;
      }
    }
    __syncthreads();
    if (tid == 0) s_nd = 0;
    __syncthreads();
    const int nc = s_nc;
    for (int k = tid; k < nc; k += blockDim.x) {
      const int e = cl[k];
      const int m = e / WAVE;
      const int64_t n = (int64_t)nb * WAVE + (e % WAVE);
      if (differs(m, n)) dl[atomicAdd(&s_nd, 1)] = e;
    }
    __syncthreads();
  }
  if (tid == 0) atomicMax(&hdr->repair_iters, (unsigned int)rounds);
}

// ---------------------------------------------------------------------------------------
// Backward.  Per step t: up = u_{t-1}, wp = w_{t-1} (u0, w0 at t = 0),
// sg = alpha*sig*(1-sig), sig = 1/(1 + exp(-alpha*((beta*up + x - theta0) - wp)))
// (triton_alif.py:367-370).
__device__ __forceinline__ float alif_sg(float up, float wp, float x, float beta, float theta0,
                                         float alpha) {
  const float v = lif_v(up, x, beta);
  const float sig = sigmoid_neg(alpha * ((v - theta0) - wp));
  return alpha * sig * (1.0f - sig);
}

// Parameter-gradient sums of ALIFFn.backward (triton_alif.py:541-554), accumulated in fp64
// while the adjoint is swept: b = sum LV*u_{t-1} (dbeta), r = sum LW*w_{t-1} (drho),
// q = sum LW*S (dq), t = sum sg*(g + q*LW) (-dtheta0).
struct ParamAcc {
  double b = 0.0, r = 0.0, q = 0.0, t = 0.0;
  __device__ __forceinline__ void add(float lv, float up, float lw, float wp, float s, float sg,
                                      float d) {
    b += (double)lv * (double)up;
    r += (double)lw * (double)wp;
    q += (double)lw * (double)s;
    t += (double)sg * (double)d;
  }
  // one chunk's four sums formed in fp32 (fma per term), added here in fp64
  __device__ __forceinline__ void add_chunk(float cb, float cr, float cq, float ct) {
    b += (double)cb;
    r += (double)cr;
    q += (double)cq;
    t += (double)ct;
  }
  __device__ __forceinline__ void wave_sum() {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      b += __shfl_xor(b, o, WAVE);
      r += __shfl_xor(r, o, WAVE);
      q += __shfl_xor(q, o, WAVE);
      t += __shfl_xor(t, o, WAVE);
    }
  }
  __device__ __forceinline__ void store(double* out) const {
    out[0] = b;
    out[1] = r;
    out[2] = q;
    out[3] = t;
  }
};

// Reverse sweep over segments of Ls steps (triton_alif.py:374-440 PASS 0-3):
//   PASS 0: compose the lw maps (P, Q)        PASS 1: lw replay from LamEnd, writes LW
//   PASS 2: compose the lv maps (reads LW)    PASS 3: lv replay from LamEnd, writes LV
// PASS 1 of the first segment also writes lw_{-1} = dL/dw0 to DW0 (if given); PASS 3 with PS
// writes the block's parameter sums to partials[blockIdx.x].
template <int PASS, bool PS>
__global__ __launch_bounds__(64) void k_alif_bwd(
    const float* __restrict__ I, const float* __restrict__ u0, const float* __restrict__ w0,
    const float* __restrict__ U, const float* __restrict__ W, const float* __restrict__ S,
    const float* __restrict__ GS, float* __restrict__ LW, float* __restrict__ LV,
    float* __restrict__ PA_, float* __restrict__ PB_, const float* __restrict__ lam_end,
    float* __restrict__ DW0, double* __restrict__ partials, int64_t N, int64_t Ls, int NB,
    float beta, float rho, float q, float theta0, float alpha, const float* __restrict__ dpar) {
  if (dpar) alif_params_from(dpar, beta, rho, q, theta0);
  const int64_t m = blockIdx.x / NB;
  const int nb = (int)(blockIdx.x - m * NB);
  const int64_t n = (int64_t)nb * WAVE + threadIdx.x;
  ParamAcc acc;
  if (n < N) {
    const float u0n = u0[n], w0n = w0[n];
    float lam = (PASS == 1 || PASS == 3) ? lam_end[m * N + n] : 0.0f;
    float P = 1.0f, Q = 0.0f;
    const int64_t t0 = m * Ls;
    for (int64_t t = t0 + Ls - 1; t >= t0; --t) {
      const size_t o = (size_t)t * N + n;
      const float up = t > 0 ? U[o - N] : u0n;
      const float wp = t > 0 ? W[o - N] : w0n;
      const float x = I[o], s = S[o], gs = GS[o];
      const float sg = alif_sg(up, wp, x, beta, theta0, alpha);
      if (PASS == 0) {
        const float a = rho - q * sg;
        P = a * P;
        Q = a * Q - sg * gs;
      } else if (PASS == 1) {
        st_nt(LW + o, lam);
        lam = (rho - q * sg) * lam - sg * gs;
      } else if (PASS == 2) {
        const float a = (1.0f - s) * beta;
        P = a * P;
        Q = a * Q + sg * (gs + q * LW[o]);
      } else {
        const float lw = LW[o];
        const float d = gs + q * lw;
        lam = (1.0f - s) * beta * lam + sg * d;
        st_nt(LV + o, lam);
        if (PS) acc.add(lam, up, lw, wp, s, sg, d);
      }
    }
    if (PASS == 0 || PASS == 2) {
      PA_[m * N + n] = P;
      PB_[m * N + n] = Q;
    }
    if (PASS == 1 && m == 0 && DW0) DW0[n] = lam;
  }
  if (PS) {
    acc.wave_sum();
    if (threadIdx.x == 0) acc.store(partials + (size_t)blockIdx.x * 4);
  }
}

// The fused serial sweep of both recurrences (triton_alif.py:444-487:
//   d = g + q*lw;  lv = (1-s)*beta*lv + sg*d;  LW[t] = lw;  LV[t] = lv;  lw <- rho*lw - sg*d,
// DW0 = lw_{-1}, partials = the block's parameter sums) with wave roles (as serial_pipe.hip):
// one workgroup per 64 neurons,
// ALIF_PIPE_P producer waves and one consumer wave, tiles of ALIF_PIPE_D rows from the end of
// time in an LDS double buffer.  Producers load the inputs one tile ahead, write (sg_t, g_t,
// (1 - s_t)*beta) per row, and store LV (and LW) of the tile the consumer finished one round
// earlier, adding the parameter sums there with the (u_{t-1}, w_{t-1}, s_t, sg_t) they kept;
// the consumer runs d = g + q*lw, lv = ((1-s)*beta)*lv + sg*d, lw = rho*lw - sg*d, one step
// after another in the reference's order.
constexpr int ALIF_PIPE_D = 32;
constexpr int ALIF_PIPE_P = 15;

// Serial ALIF forward from (u0, w0) with the same wave roles (triton_alif.py:35-42,
// :263-273): the consumer runs alif_step through LDS and writes (u, w) per step and each tile's
// entry state; the producers stage I one tile ahead and store U, W, S of the tile finished one
// round earlier, recomputing s_t = (fl(fl(beta*u_{t-1}) + x_t) >= theta0 + w_{t-1}) with the
// consumer's own operations from the rows they loaded (kept two rounds in registers), so the
// consumer's chain carries no spike-to-float select; bit-identical to k_alif_fwd.
#ifndef LSH_ALIF_FPIPE_D
#define LSH_ALIF_FPIPE_D 64  // rows per tile (LDS: 2 x D x 64 x (4 + 8) B)
#endif
constexpr int ALIF_FPIPE_D = LSH_ALIF_FPIPE_D;

//
// With mstar (the box scan's repair to convergence): the rows from chunk c0 on, c0 the least
// mstar of the block's neurons, from the exact exits (eu, ew) of chunk c0 - 1 (which the replay
// of the chunks below mstar wrote); rows before c0 C are left as they are.
__global__ __launch_bounds__(WAVE*(ALIF_PIPE_P + 1)) void k_alif_fwd_pipe(
    const float* __restrict__ I, const float* __restrict__ u0, const float* __restrict__ w0,
    float* __restrict__ U, float* __restrict__ W, float* __restrict__ S, int64_t N, int64_t T,
    float beta, float rho, float q, float theta0, float u_r, const float* __restrict__ dpar,
    const int* __restrict__ mstar, const float* __restrict__ eu, const float* __restrict__ ew,
    int C) {
  if (dpar) alif_params_from(dpar, beta, rho, q, theta0);
  constexpr int D = ALIF_FPIPE_D, P = ALIF_PIPE_P, R = (D + P - 1) / P;
  __shared__ float sX[2][D][WAVE];
  __shared__ float2 sUW[2][D][WAVE];
  __shared__ float2 sEntry[2][WAVE];  // (u, w) before row 0 of the tile in the same buffer
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const unsigned lane = threadIdx.x % WAVE;
  const int64_t nb0 = (int64_t)blockIdx.x * WAVE;
  const bool valid = nb0 + lane < N;
  const unsigned ln = valid ? lane : (unsigned)(N - 1 - nb0);
  const unsigned lb = ln * 4u, sb = lane * 4u;
  // first chunk of the block's pass (the same in every wave of the block)
  int c0 = 0;
  if (mstar) c0 = -wave_max_i(-(valid ? mstar[nb0 + lane] : 0x7fffffff));
  const int64_t row0 = (int64_t)c0 * C;
  const int64_t Tr = T > row0 ? T - row0 : 0;
  const int64_t ntiles = (Tr + D - 1) / D;
  auto rows = [&](int64_t k) { return (int)(Tr - k * D > D ? D : Tr - k * D); };

  if (w == 0) {  // consumer: tile k - 1 in round k
    __builtin_amdgcn_s_setprio(3);
    const bool from_exit = c0 > 0 && ntiles > 0;
    const size_t oe = from_exit ? (size_t)(c0 - 1) * (size_t)N + (size_t)(nb0 + ln) : 0;
    float u = from_exit ? eu[oe] : u0[nb0 + ln], ww = from_exit ? ew[oe] : w0[nb0 + ln];
    for (int64_t k = 0; k <= ntiles + 1; ++k) {
      if (k >= 1 && k <= ntiles) {
        const int buf = (int)((k - 1) & 1);
        const int nr = rows(k - 1);
        sEntry[buf][lane] = make_float2(u, ww);
        auto step = [&](int j, float x) {
          bool sp;
          u = alif_step(u, ww, x, beta, rho, q, theta0, u_r, sp);
          sUW[buf][j][lane] = make_float2(u, ww);
        };
        if (nr == D) {
#pragma unroll
          for (int g = 0; g < D; g += 16) {
            float x[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) x[i] = sX[buf][g + i][lane];
#pragma unroll
            for (int i = 0; i < 16; ++i) step(g + i, x[i]);
          }
        } else {
          for (int j = 0; j < nr; ++j) step(j, sX[buf][j][lane]);
        }
      }
      __syncthreads();
    }
    return;
  }

  const int p = w - 1;
  // xr: the rows of the tile being loaded; at the start of round k, x1 and x2 hold this
  // producer's rows of tiles k - 1 and k - 2
  float xr[R], x1[R], x2[R];
#pragma unroll
  for (int r = 0; r < R; ++r) xr[r] = x1[r] = x2[r] = 0.0f;
  auto load = [&](int64_t k) {
    const int nr = rows(k);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int j = p + r * P;
      if (j < nr) xr[r] = ld_row(I + (size_t)(row0 + k * D + j) * (size_t)N + (size_t)nb0, lb);
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
          const size_t row = (size_t)(row0 + (k - 2) * D + j) * (size_t)N + (size_t)nb0;
          const float2 o = sUW[buf][j][lane];
          const float2 pr = j == 0 ? sEntry[buf][lane] : sUW[buf][j - 1][lane];
          const bool sp = lif_v(pr.x, x2[r], beta) >= theta0 + pr.y;
          st_row_nt(U + row, sb, o.x);
          st_row_nt(W + row, sb, o.y);
          st_row_nt(S + row, sb, sp ? 1.0f : 0.0f);
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

template <bool WLW, bool PS>
__global__ __launch_bounds__(WAVE*(ALIF_PIPE_P + 1)) void k_alif_bwd_pipe(
    const float* __restrict__ I, const float* __restrict__ u0, const float* __restrict__ w0,
    const float* __restrict__ U, const float* __restrict__ W, const float* __restrict__ S,
    const float* __restrict__ GS, float* __restrict__ LW, float* __restrict__ LV,
    float* __restrict__ DW0, double* __restrict__ partials, int64_t N, int64_t T, float beta,
    float rho, float q, float theta0, float alpha, const float* __restrict__ dpar) {
  if (dpar) alif_params_from(dpar, beta, rho, q, theta0);
  constexpr int D = ALIF_PIPE_D, P = ALIF_PIPE_P, R = (D + P - 1) / P;
  __shared__ float4 sIn[2][D][WAVE];   // sg, g, (1 - s)*beta
  __shared__ float4 sOut[2][D][WAVE];  // lv_t, lw_t (before the step), d_t
  __shared__ double sAcc[P][4];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const unsigned lane = threadIdx.x % WAVE;
  const int64_t nb0 = (int64_t)blockIdx.x * WAVE;
  const bool valid = nb0 + lane < N;
  const unsigned ln = valid ? lane : (unsigned)(N - 1 - nb0);
  const unsigned lb = ln * 4u, sb = lane * 4u;
  const int64_t ntiles = (T + D - 1) / D;
  const int64_t rounds = (ntiles + 3) & ~(int64_t)1;  // >= ntiles + 2, even
  auto tile_lo = [&](int64_t k) { const int64_t hi = T - k * D; return hi > D ? hi - D : (int64_t)0; };
  auto tile_rows = [&](int64_t k) { const int64_t hi = T - k * D; return (int)(hi > D ? D : hi); };

  if (w == 0) {  // consumer: tile k - 1 in round k
    __builtin_amdgcn_s_setprio(3);
    float lw = 0.0f, lv = 0.0f;
    for (int64_t k = 0; k < rounds; ++k) {
      if (k >= 1 && k <= ntiles) {
        const int buf = (int)((k - 1) & 1);
        const int nr = tile_rows(k - 1);
        auto step = [&](int j, const float4 in) {
          const float d = in.y + q * lw;
          const float lw_old = lw;
          lv = in.z * lv + in.x * d;
          lw = rho * lw - in.x * d;
          sOut[buf][j][lane] = make_float4(lv, lw_old, d, 0.0f);
        };
        if (nr == D) {
#pragma unroll
          for (int g = D - 8; g >= 0; g -= 8) {
            float4 in[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) in[i] = sIn[buf][g + i][lane];
#pragma unroll
            for (int i = 7; i >= 0; --i) step(g + i, in[i]);
          }
        } else {
          for (int j = nr - 1; j >= 0; --j) step(j, sIn[buf][j][lane]);
        }
      }
      __syncthreads();
    }
    if (DW0 && valid) DW0[nb0 + lane] = lw;
  } else {  // producers: inputs of tile k, outputs of tile k - 2 in round k
    const int p = w - 1;
    const float u0n = u0[nb0 + ln], w0n = w0[nb0 + ln];
    float xr[R], sr[R], gr[R], ur[R], wr[R];
    float keep0[4][PS ? R : 1], keep1[4][PS ? R : 1];  // (up, wp, s, sg) of the tiles in flight
    ParamAcc acc;
    auto load = [&](int64_t k) {
      const int64_t lo = tile_lo(k);
      const int nr = tile_rows(k);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int j = p + r * P;
        if (j < nr) {
          const int64_t t = lo + j;
          const size_t row = (size_t)t * (size_t)N + (size_t)nb0;
          xr[r] = ld_row(I + row, lb);
          sr[r] = ld_row(S + row, lb);
          gr[r] = ld_row(GS + row, lb);
          ur[r] = t > 0 ? ld_row(U + row - N, lb) : u0n;
          wr[r] = t > 0 ? ld_row(W + row - N, lb) : w0n;
        }
      }
    };
    // tile k's kept values land where tile k - 2's were: use those first
    auto round = [&](int64_t k, float(&keep)[4][PS ? R : 1]) {
      if (k >= 2 && k - 2 < ntiles && valid) {
        const int buf = (int)(k & 1);
        const int64_t lo = tile_lo(k - 2);
        const int nr = tile_rows(k - 2);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int j = p + r * P;
          if (j < nr) {
            const float4 o = sOut[buf][j][lane];
            const size_t row = (size_t)(lo + j) * (size_t)N + (size_t)nb0;
            if (WLW) st_row_nt(LW + row, sb, o.y);
            st_row_nt(LV + row, sb, o.x);
            if constexpr (PS) acc.add(o.x, keep[0][r], o.y, keep[1][r], keep[2][r], keep[3][r], o.z);
          }
        }
      }
      if (k < ntiles) {
        float x[R], sv[R], g[R], up[R], wp[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          x[r] = xr[r];
          sv[r] = sr[r];
          g[r] = gr[r];
          up[r] = ur[r];
          wp[r] = wr[r];
        }
        if (k + 1 < ntiles) load(k + 1);
        const int buf = (int)(k & 1);
        const int nr = tile_rows(k);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int j = p + r * P;
          if (j < nr) {
            const float sg = alif_sg(up[r], wp[r], x[r], beta, theta0, alpha);
            sIn[buf][j][lane] = make_float4(sg, g[r], (1.0f - sv[r]) * beta, 0.0f);
            if constexpr (PS) {
              keep[0][r] = up[r];
              keep[1][r] = wp[r];
              keep[2][r] = sv[r];
              keep[3][r] = sg;
            }
          }
        }
      }
      __syncthreads();
    };
    if (ntiles > 0) load(0);
    for (int64_t k = 0; k < rounds; k += 2) {
      round(k, keep0);
      round(k + 1, keep1);
    }
    if constexpr (PS) {
      acc.wave_sum();
      if (lane == 0) acc.store(sAcc[p]);
    }
  }
  if constexpr (PS) {
    __syncthreads();
    if (threadIdx.x == 0) {
      ParamAcc tot;
      for (int v = 0; v < P; ++v) {
        tot.b += sAcc[v][0];
        tot.r += sAcc[v][1];
        tot.q += sAcc[v][2];
        tot.t += sAcc[v][3];
      }
      tot.store(partials + (size_t)blockIdx.x * 4);
    }
  }
}

// Single-pass two-scan adjoint: one workgroup of W waves owns 64 neurons and walks the time
// axis backwards in rounds of W chunks.  Each wave keeps its chunk's (sg_t, g_t, s_t) in
// registers, composes the lw recurrence into (P1, Q1), takes lw at its chunk end from the
// later chunks through LDS, replays lw (kept in registers), composes the lv recurrence
// (which reads lw_t) into (P2, Q2), takes lv at its chunk end the same way and replays lv.
// WLW: write LW.  PS: also keep u_{t-1}, w_{t-1} and sum the parameter gradients (each
// chunk's in fp32, the chunks in fp64; one partials row per workgroup).  DW0 (if given)
// receives lw_{-1} from the first chunk.
// RC: S is not read and U, W only at the row before each chunk; the chunk's u_{t-1}, w_{t-1}
// and s_t are recomputed with the forward's own step (alif_step, reset value u_r) from that
// entry state, which gives the stored bits when U, W, S come from one serial trajectory.  The
// adjoint arithmetic is unchanged, so the outputs equal the stored-state variant's bit for bit.
template <int C, int WV, bool WLW, bool PS, bool RC = false>
__global__ __launch_bounds__(WAVE* WV) void k_alif_bwd_fused(
    const float* __restrict__ I, const float* __restrict__ u0, const float* __restrict__ w0,
    const float* __restrict__ U, const float* __restrict__ W, const float* __restrict__ S,
    const float* __restrict__ GS, float* __restrict__ LW, float* __restrict__ LV,
    float* __restrict__ DW0, double* __restrict__ partials, int64_t N, int M, float beta,
    float rho, float q, float theta0, float alpha, float u_r, const float* __restrict__ dpar) {
  if (dpar) alif_params_from(dpar, beta, rho, q, theta0);
  // the two recurrences' chunk aggregates in separate arrays and the lv carry double-buffered
  // by round parity, so a round needs two barriers: round r + 1 writes nothing that a wave
  // still in round r reads (every reader passes one of the two barriers first)
  __shared__ float sP1[WV][WAVE], sQ1[WV][WAVE], sP2[WV][WAVE], sQ2[WV][WAVE];
  __shared__ float sLw[WAVE], sLv[2][WAVE];
  __shared__ double sAcc[WV][4];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const unsigned lane = threadIdx.x % WAVE;
  const int64_t nb0 = (int64_t)blockIdx.x * WAVE;
  const bool valid = nb0 + lane < N;
  const unsigned ln = valid ? lane : (unsigned)(N - 1 - nb0);
  const unsigned lb = ln * 4u, sb = lane * 4u;
  const unsigned rstride = (unsigned)(N * 4);
  const float u0n = u0[nb0 + ln], w0n = w0[nb0 + ln];
  ParamAcc acc;
  if (w == 0) {
    sLw[lane] = 0.0f;
    sLv[0][lane] = 0.0f;
  }
  __syncthreads();
  const int rounds = (M + WV - 1) / WV;
  for (int r = 0; r < rounds; ++r) {
    const int par = r & 1;
    const int m = M - 1 - (r * WV + w);
    const bool active = m >= 0;
    const size_t row0 = (size_t)(active ? m : 0) * C;
    float sg[C], g[C], s1[C], lwv[C];
    float upv[PS ? C : 1], wpv[PS ? C : 1];
    float lw_end = 0.0f, lv_end = 0.0f;
    if (active && RC) {
      const Buf bi(I + nb0 + row0 * N), bg(GS + nb0 + row0 * N);
      float up = row0 > 0 ? ld_row(U + nb0 + (row0 - 1) * N, lb) : u0n;
      float wp = row0 > 0 ? ld_row(W + nb0 + (row0 - 1) * N, lb) : w0n;
      float xv[C];
#pragma unroll
      for (int j = 0; j < C; ++j) {
        const unsigned so = j * rstride;
        xv[j] = bi.ld(lb, so);
        g[j] = bg.ld(lb, so);
      }
#pragma unroll
      for (int j = 0; j < C; ++j) {
        sg[j] = alif_sg(up, wp, xv[j], beta, theta0, alpha);
        if (PS) {
          upv[j] = up;
          wpv[j] = wp;
        }
        bool sp;
        up = alif_step(up, wp, xv[j], beta, rho, q, theta0, u_r, sp);
        s1[j] = sp ? 0.0f : 1.0f;
      }
    } else if (active) {
      const Buf bi(I + nb0 + row0 * N), bs(S + nb0 + row0 * N), bg(GS + nb0 + row0 * N);
      const Buf bu(U + nb0 + row0 * N), bw(W + nb0 + row0 * N);
      const float up0 = row0 > 0 ? ld_row(U + nb0 + (row0 - 1) * N, lb) : u0n;
      const float wp0 = row0 > 0 ? ld_row(W + nb0 + (row0 - 1) * N, lb) : w0n;
#pragma unroll
      for (int j = 0; j < C; ++j) {
        const unsigned so = j * rstride;
        const float up = j == 0 ? up0 : bu.ld(lb, so - rstride);
        const float wp = j == 0 ? wp0 : bw.ld(lb, so - rstride);
        sg[j] = alif_sg(up, wp, bi.ld(lb, so), beta, theta0, alpha);
        g[j] = bg.ld(lb, so);
        s1[j] = 1.0f - bs.ld(lb, so);
        if (PS) {
          upv[j] = up;
          wpv[j] = wp;
        }
      }
    }
    if (active) {
      float P = 1.0f, Q = 0.0f;
#pragma unroll
      for (int j = C - 1; j >= 0; --j) {
        const float a = rho - q * sg[j];
        P = a * P;
        Q = a * Q - sg[j] * g[j];
      }
      sP1[w][lane] = P;
      sQ1[w][lane] = Q;
    }
    __syncthreads();
    if (active) {
      float lam = sLw[lane];
      for (int v = 0; v < w; ++v) lam = sQ1[v][lane] + sP1[v][lane] * lam;
#pragma unroll
      for (int j = C - 1; j >= 0; --j) {
        lwv[j] = lam;
        lam = (rho - q * sg[j]) * lam - sg[j] * g[j];
      }
      lw_end = lam;
      if (m == 0 && DW0 && valid) DW0[nb0 + lane] = lam;
    }
    if (active) {
      float P = 1.0f, Q = 0.0f;
#pragma unroll
      for (int j = C - 1; j >= 0; --j) {
        const float a = s1[j] * beta;
        P = a * P;
        Q = a * Q + sg[j] * (g[j] + q * lwv[j]);
      }
      sP2[w][lane] = P;
      sQ2[w][lane] = Q;
    }
    __syncthreads();
    if (active) {
      float lam = sLv[par][lane];
      for (int v = 0; v < w; ++v) lam = sQ2[v][lane] + sP2[v][lane] * lam;
      const Buf bo(LW + nb0 + row0 * N), bv(LV + nb0 + row0 * N);
      float cb = 0.0f, cr = 0.0f, cq = 0.0f, ct = 0.0f;  // PS: this chunk's sums
#pragma unroll
      for (int j = C - 1; j >= 0; --j) {
        const float d = g[j] + q * lwv[j];
        lam = s1[j] * beta * lam + sg[j] * d;
        if (valid) {
          if (WLW) bo.st_nt(sb, j * rstride, lwv[j]);
          bv.st_nt(sb, j * rstride, lam);
        }
        if (PS) {
          cb = fmaf(lam, upv[j], cb);
          cr = fmaf(lwv[j], wpv[j], cr);
          cq += s1[j] == 0.0f ? lwv[j] : 0.0f;
          ct = fmaf(sg[j], d, ct);
        }
      }
      if (PS && valid) acc.add_chunk(cb, cr, cq, ct);
      lv_end = lam;
    }
    // the carries into the next round (its readers are past the next round's first barrier)
    const int last = min(WV, M - r * WV) - 1;
    if (w == last) {
      sLw[lane] = lw_end;
      sLv[par ^ 1][lane] = lv_end;
    }
  }
  if (PS) {
    acc.wave_sum();
    if (lane == 0) acc.store(sAcc[w]);
    __syncthreads();
    if (threadIdx.x == 0) {
      ParamAcc tot;
      for (int v = 0; v < WV; ++v) {
        tot.b += sAcc[v][0];
        tot.r += sAcc[v][1];
        tot.q += sAcc[v][2];
        tot.t += sAcc[v][3];
      }
      tot.store(partials + (size_t)blockIdx.x * 4);
    }
  }
}

// ALIF adjoint for few neurons: both recurrences of k_alif_bwd_fused in one pass, segments of
// ALIF_LB_W chunks of ALIF_LB_C steps chained across workgroups by decoupled look-back (as the LIF
// adjoint in lif_lookback.hip), once for lw and then for lv:
//   1. every wave loads its chunk once (I, u_{t-1}, w_{t-1}, S, GS) and keeps (sg, g, 1 - s);
//   2. lw: chunk maps (a = rho - q*sg, b = -sg*g) -> segment map; wave 0 takes lw at its segment
//      end from the later segments' published maps and an anchor's inclusive value in an order
//      fixed by the segment index (lb_value_at_end, lsh_lookback.h: the same bits on every run;
//      non-anchors publish their map first, anchors their value at the start afterwards); every
//      wave replays lw from its chunk end (kept in registers);
//   3. lv: the same with a = (1 - s)*beta, b = sg*(g + q*lw), then the replay stores LV (and LW)
//      and sums the parameter gradients (fp32 per chunk, fp64 per workgroup).
// Workgroups take (segment, block) tiles latest segment first through a ticket counter and wait
// only for tiles with smaller tickets, which are running or done: every wait ends (and is
// bounded; a give-up is counted in the header).  The same waves per workgroup with and without
// the sums, so dI does not depend on whether the parameters need a gradient.  RC: as in
// k_alif_bwd_fused, S is not read and U, W only at the row before each chunk (the chunk's states
// recomputed with alif_step from there; the same bits as the stored variant).
constexpr int ALIF_LB_C = 16;
constexpr int ALIF_LB_W = 8;
constexpr int ALIF_LB_SEG = ALIF_LB_C * ALIF_LB_W;

template <bool WLW, bool PS, bool RC = false>
__global__ __launch_bounds__(WAVE* ALIF_LB_W) void k_alif_bwd_lookback(
    const float* __restrict__ I, const float* __restrict__ u0, const float* __restrict__ w0,
    const float* __restrict__ U, const float* __restrict__ W, const float* __restrict__ S,
    const float* __restrict__ GS, float* __restrict__ LW, float* __restrict__ LV,
    float* __restrict__ DW0, double* __restrict__ partials, float* __restrict__ agg,
    int* __restrict__ flags, WsHeader* hdr, int64_t N, int NB, int NSEG, float beta, float rho,
    float q, float theta0, float alpha, float u_r, const float* __restrict__ dpar) {
  if (dpar) alif_params_from(dpar, beta, rho, q, theta0);
  constexpr int C = ALIF_LB_C, WV = ALIF_LB_W;
  __shared__ float sP[WV][WAVE], sQ[WV][WAVE];
  __shared__ float sEnd[WAVE];
  __shared__ float sLbP[LB_GROUP][WAVE], sLbQ[LB_GROUP][WAVE];
  __shared__ double sAcc[WV][4];
  __shared__ int sTicket;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const unsigned lane = threadIdx.x % WAVE;
  if (threadIdx.x == 0) sTicket = (int)atomicAdd(&hdr->ticket, 1u);
  __syncthreads();
  const int tk = sTicket;
  const int nb = tk % NB;
  const int seg = NSEG - 1 - tk / NB;  // latest segments first
  const int64_t nb0 = (int64_t)nb * WAVE;
  const bool valid = nb0 + lane < N;
  const unsigned ln = valid ? lane : (unsigned)(N - 1 - nb0);
  const unsigned lb = ln * 4u, sb = lane * 4u;
  const unsigned rstride = (unsigned)(N * 4);
  const size_t row0 = ((size_t)seg * WV + (WV - 1 - w)) * C;  // wave 0 holds the latest chunk
  const size_t sn = (size_t)NSEG * (size_t)N;
  const size_t so = (size_t)seg * N + nb0 + lane;

  // 1. the chunk's per-step quantities
  float sg[C], g[C], s1[C], lwv[C];
  float upv[PS ? C : 1], wpv[PS ? C : 1];
  if constexpr (RC) {
    const Buf bi(I + nb0 + row0 * N), bg(GS + nb0 + row0 * N);
    float up = row0 > 0 ? ld_row(U + nb0 + (row0 - 1) * N, lb) : u0[nb0 + ln];
    float wp = row0 > 0 ? ld_row(W + nb0 + (row0 - 1) * N, lb) : w0[nb0 + ln];
    float xv[C];
#pragma unroll
    for (int j = 0; j < C; ++j) {
      xv[j] = bi.ld(lb, j * rstride);
      g[j] = bg.ld(lb, j * rstride);
    }
#pragma unroll
    for (int j = 0; j < C; ++j) {
      sg[j] = alif_sg(up, wp, xv[j], beta, theta0, alpha);
      if (PS) {
        upv[j] = up;
        wpv[j] = wp;
      }
      bool sp;
      up = alif_step(up, wp, xv[j], beta, rho, q, theta0, u_r, sp);
      s1[j] = sp ? 0.0f : 1.0f;
    }
  } else {
    const Buf bi(I + nb0 + row0 * N), bs(S + nb0 + row0 * N), bg(GS + nb0 + row0 * N);
    const Buf bu(U + nb0 + row0 * N), bw(W + nb0 + row0 * N);
    const float up0 = row0 > 0 ? ld_row(U + nb0 + (row0 - 1) * N, lb) : u0[nb0 + ln];
    const float wp0 = row0 > 0 ? ld_row(W + nb0 + (row0 - 1) * N, lb) : w0[nb0 + ln];
#pragma unroll
    for (int j = 0; j < C; ++j) {
      const unsigned o = j * rstride;
      const float up = j == 0 ? up0 : bu.ld(lb, o - rstride);
      const float wp = j == 0 ? wp0 : bw.ld(lb, o - rstride);
      sg[j] = alif_sg(up, wp, bi.ld(lb, o), beta, theta0, alpha);
      g[j] = bg.ld(lb, o);
      s1[j] = 1.0f - bs.ld(lb, o);
      if (PS) {
        upv[j] = up;
        wpv[j] = wp;
      }
    }
  }

  // The look-back of one phase (its aggregates agg[phase][0..2] = P, Q, inclusive; its flags
  // flags[phase]) over the chunk maps in sP/sQ: wave 0 composes the segment map and, outside
  // an anchor, publishes it; every wave fetches look-back operands; wave 0 composes them in a
  // fixed order (lsh_lookback.h) to the value at this segment's end (sEnd) and, at an anchor,
  // publishes the value at its start.
  const bool anchor = lb_is_anchor(seg);
  int* const myflag0 = flags + (size_t)seg * NB + nb;
  float Ps = 1.0f, Qs = 0.0f;  // value at segment start = Qs + Ps * value at segment end
  auto look_back = [&](int phase) {
    float* aP = agg + (size_t)phase * 3 * sn;
    float* aQ = aP + sn;
    float* inc = aQ + sn;
    int* fl = flags + (size_t)phase * NSEG * NB;
    int* const myflag = myflag0 + (size_t)phase * NSEG * NB;
    if (w == 0) {
      Ps = 1.0f;
      Qs = 0.0f;
      for (int v = 0; v < WV; ++v) {
        Qs = sQ[v][lane] + sP[v][lane] * Qs;
        Ps = sP[v][lane] * Ps;
      }
      if (!anchor) {
        if (valid) {
          st_coh(aP + so, Ps);
          st_coh(aQ + so, Qs);
        }
        publish_flag(myflag, 1);
      }
    }
    lb_fetch(seg, NSEG, NB, nb, N, nb0 + ln, w, WV, aP, aQ, inc, fl, sLbP, sLbQ,
             &hdr->spin_timeouts);
    __syncthreads();
    if (w == 0) {
      const float end = lb_compose(seg, NSEG, sLbP, sLbQ);
      if (anchor) {
        if (valid) st_coh(inc + so, Qs + Ps * end);
        publish_flag(myflag, 2);
      }
      sEnd[lane] = end;
    }
  };

  // 2. lw
  {
    float P = 1.0f, Q = 0.0f;
#pragma unroll
    for (int j = C - 1; j >= 0; --j) {
      const float a = rho - q * sg[j];
      P = a * P;
      Q = a * Q - sg[j] * g[j];
    }
    sP[w][lane] = P;
    sQ[w][lane] = Q;
  }
  __syncthreads();
  look_back(0);
  __syncthreads();
  {
    float lam = sEnd[lane];
    for (int v = 0; v < w; ++v) lam = sQ[v][lane] + sP[v][lane] * lam;
#pragma unroll
    for (int j = C - 1; j >= 0; --j) {
      lwv[j] = lam;
      lam = (rho - q * sg[j]) * lam - sg[j] * g[j];
    }
    if (row0 == 0 && DW0 && valid) DW0[nb0 + lane] = lam;
  }
  __syncthreads();

  // 3. lv
  {
    float P = 1.0f, Q = 0.0f;
#pragma unroll
    for (int j = C - 1; j >= 0; --j) {
      const float a = s1[j] * beta;
      P = a * P;
      Q = a * Q + sg[j] * (g[j] + q * lwv[j]);
    }
    sP[w][lane] = P;
    sQ[w][lane] = Q;
  }
  __syncthreads();
  look_back(1);
  __syncthreads();
  ParamAcc acc;
  {
    float lam = sEnd[lane];
    for (int v = 0; v < w; ++v) lam = sQ[v][lane] + sP[v][lane] * lam;
    const Buf bo(LW + nb0 + row0 * N), bv(LV + nb0 + row0 * N);
    float cb = 0.0f, cr = 0.0f, cq = 0.0f, ct = 0.0f;
#pragma unroll
    for (int j = C - 1; j >= 0; --j) {
      const float d = g[j] + q * lwv[j];
      lam = s1[j] * beta * lam + sg[j] * d;
      if (valid) {
        if (WLW) bo.st_nt(sb, j * rstride, lwv[j]);
        bv.st_nt(sb, j * rstride, lam);
      }
      if (PS) {
        cb = fmaf(lam, upv[j], cb);
        cr = fmaf(lwv[j], wpv[j], cr);
        cq += s1[j] == 0.0f ? lwv[j] : 0.0f;
        ct = fmaf(sg[j], d, ct);
      }
    }
    if (PS && valid) acc.add_chunk(cb, cr, cq, ct);
  }
  if constexpr (PS) {
    acc.wave_sum();
    if (lane == 0) acc.store(sAcc[w]);
    __syncthreads();
    if (threadIdx.x == 0) {
      ParamAcc tot;
      for (int v = 0; v < WV; ++v) {
        tot.b += sAcc[v][0];
        tot.r += sAcc[v][1];
        tot.q += sAcc[v][2];
        tot.t += sAcc[v][3];
      }
      tot.store(partials + ((size_t)seg * NB + nb) * 4);
    }
  }
}

__global__ __launch_bounds__(64) void k_rev_carry(const float* __restrict__ PA_,
                                                  const float* __restrict__ PB_,
                                                  float* __restrict__ lam_end, int64_t N, int M) {
  const int64_t n = (int64_t)blockIdx.x * WAVE + threadIdx.x;
  if (n >= N) return;
  float lam = 0.0f;
  for (int m = M - 1; m >= 0; --m) {
    const size_t o = (size_t)m * N + n;
    lam_end[o] = lam;
    lam = PB_[o] + PA_[o] * lam;
  }
}

static void alif_scan_layout(int64_t T, int64_t N, int C, int K1, int K2, lsh_alif_layout* L) {
  const int64_t M = T / C;
  const size_t mn = (size_t)M * (size_t)N * 4;
  const size_t nb = (size_t)((N + WAVE - 1) / WAVE);
  Carver c;
  L->EC = c.take(mn);
  L->EA = c.take(mn);
  L->EB = c.take(mn);
  L->LU = c.take(mn);
  L->HU = c.take(mn);
  L->LW = c.take(mn);
  L->HW = c.take(mn);
  L->MA = c.take(mn);
  L->MB = c.take(mn);
  L->NL = c.take(mn);
  L->NP = c.take(mn);
  L->OVF = c.take(mn);
  L->LS = c.take(mn * (size_t)K1);
  L->LC = c.take(mn * (size_t)K1);
  L->LX = c.take(mn * (size_t)K1);
  L->POWN = c.take(mn * (size_t)K2);
  L->PXL = c.take(mn * (size_t)K2);
  L->PXR = c.take(mn * (size_t)K2);
  L->PU = c.take(mn * (size_t)K2);
  L->PA = c.take(mn * (size_t)K2);
  L->POF = c.take(mn * (size_t)K2);
  L->SU = c.take(mn);
  L->SW = c.take(mn);
  L->EU = c.take(mn);
  L->EW = c.take(mn);
  L->MISS = c.take(mn);
  L->MSTAR = c.take((size_t)N * 4);
  L->LIST0 = c.take(nb * (size_t)M * WAVE * 4);
  L->LIST1 = c.take(nb * (size_t)M * WAVE * 4);
  L->total = c.off;
}

static int alif_scan_check(int64_t T, int64_t N, int C, int K1, int K2, int block) {
  if (T < 0 || N < 0 || N > (int64_t)1 << 31) return LSH_ERR_SHAPE;
  if (C < 1 || K1 < 1 || K1 > 32 || K2 < 1 || K2 > 32 || (K2 & (K2 - 1)) != 0) return LSH_ERR_SHAPE;
  if (block != 1 && block != 2 && block != 4 && block != 8 && block != 16) return LSH_ERR_SHAPE;
  if (T % C != 0) return LSH_ERR_DIVISIBILITY;
  if ((T / C) * ((N + WAVE - 1) / WAVE) > ((int64_t)1 << 31) - 1) return LSH_ERR_SHAPE;
  return LSH_OK;
}

template <int BLK>
static void launch_alif_build(const float* I, char* w, const lsh_alif_layout& L, int64_t N, int M,
                              int C, int K1, int K2, float beta, float rho, float q, float theta0,
                              float u_r, hipStream_t st) {
  constexpr int NPW = AlifBuildShape<BLK>::NPW;
  const int NBLK = (int)((N + NPW - 1) / NPW);
  auto F = [&](size_t off) { return reinterpret_cast<float*>(w + off); };
  auto Iq = [&](size_t off) { return reinterpret_cast<int*>(w + off); };
  hipLaunchKernelGGL((k_alif_build<BLK>), dim3((unsigned)((int64_t)M * NBLK)),
                     dim3(WAVE * AlifBuildShape<BLK>::NW), 0, st,
                     I, F(L.LU), F(L.HU), F(L.LW), F(L.HW), F(L.MA), F(L.MB), Iq(L.NL), Iq(L.NP),
                     Iq(L.OVF), F(L.LS), F(L.LC), F(L.LX), Iq(L.POWN), F(L.PXL), F(L.PXR), F(L.PU),
                     F(L.PA), F(L.POF), N, NBLK, C, K1, K2, beta, rho, q, theta0, u_r);
}

template <int D>
static void launch_alif_fwd(const float* I, const float* su, const float* sw, float* U, float* W,
                            float* S, float* eu, float* ew, int64_t N, int64_t Ls, int64_t M,
                            float beta, float rho, float q, float theta0, float u_r, hipStream_t st,
                            const float* dpar = nullptr, const int* mstar = nullptr) {
  const int NB = (int)((N + WAVE - 1) / WAVE);
  hipLaunchKernelGGL(k_alif_fwd<D>, dim3((unsigned)(M * NB)), dim3(WAVE), 0, st, I, su, sw, U, W, S,
                     eu, ew, N, Ls, NB, beta, rho, q, theta0, u_r, dpar, mstar);
}

}  // namespace lsh

using namespace lsh;

extern "C" int lsh_alif_serial_fwd(const float* I, const float* u0, const float* w0, float* U,
                                   float* W, float* S, int64_t T, int64_t N, float beta, float rho,
                                   float q, float theta0, float u_r, void* stream) {
  if (bad_ptr(I) || bad_ptr(u0) || bad_ptr(w0) || bad_ptr(U) || bad_ptr(W) || bad_ptr(S))
    return LSH_ERR_ARG;
  if (T < 0 || N < 0 || N > (int64_t)1 << 31) return LSH_ERR_SHAPE;
  if (T == 0 || N == 0) return LSH_OK;
  const int NB = (int)((N + WAVE - 1) / WAVE);
  hipLaunchKernelGGL(k_alif_fwd_pipe, dim3((unsigned)NB), dim3(WAVE * (ALIF_PIPE_P + 1)), 0,
                     (hipStream_t)stream, I, u0, w0, U, W, S, N, T, beta, rho, q, theta0, u_r,
                     nullptr, nullptr, nullptr, nullptr, 1);
  LSH_CHECK_LAUNCH();
  return LSH_OK;
}

extern "C" int lsh_alif_serial_fwd_dparams(const float* I, const float* u0, const float* w0,
                                           float* U, float* W, float* S, int64_t T, int64_t N,
                                           const float* params, float u_r, void* stream) {
  if (bad_ptr(I) || bad_ptr(u0) || bad_ptr(w0) || bad_ptr(U) || bad_ptr(W) || bad_ptr(S) ||
      bad_ptr(params))
    return LSH_ERR_ARG;
  if (T < 0 || N < 0 || N > (int64_t)1 << 31) return LSH_ERR_SHAPE;
  if (T == 0 || N == 0) return LSH_OK;
  const int NB = (int)((N + WAVE - 1) / WAVE);
  hipLaunchKernelGGL(k_alif_fwd_pipe, dim3((unsigned)NB), dim3(WAVE * (ALIF_PIPE_P + 1)), 0,
                     (hipStream_t)stream, I, u0, w0, U, W, S, N, T, 0.0f, 0.0f, 0.0f, 0.0f, u_r,
                     params, nullptr, nullptr, nullptr, 1);
  LSH_CHECK_LAUNCH();
  return LSH_OK;
}

extern "C" int lsh_alif_warm_predict(const float* I, const float* u0, const float* w0,
                                     const float* UI, const float* WI, float* WP, int64_t T,
                                     int64_t N, int C, int Wn, float u_init, float w_init,
                                     float beta, float rho, float q, float theta0, float u_r,
                                     void* stream) {
  if (bad_ptr(I) || bad_ptr(u0) || bad_ptr(w0) || bad_ptr(WP)) return LSH_ERR_ARG;
  if ((UI == nullptr) != (WI == nullptr)) return LSH_ERR_ARG;
  if (T < 0 || N < 0 || C < 1 || Wn < 0 || N > (int64_t)1 << 31) return LSH_ERR_SHAPE;
  const int64_t M = T / C;
  if (M == 0 || N == 0) return LSH_OK;
  const int NB = (int)((N + WAVE - 1) / WAVE);
  hipLaunchKernelGGL(k_alif_warm, dim3((unsigned)(M * NB)), dim3(WAVE), 0, (hipStream_t)stream, I, u0,
                     w0, UI, WI, WP, N, NB, C, Wn, u_init, w_init, beta, rho, q, theta0, u_r);
  LSH_CHECK_LAUNCH();
  return LSH_OK;
}

extern "C" int lsh_alif_scan_layout(int64_t T, int64_t N, int C, int K1, int K2,
                                    lsh_alif_layout* out) {
  if (bad_ptr(out)) return LSH_ERR_ARG;
  const int rc = alif_scan_check(T, N, C, K1, K2, 1);
  if (rc != LSH_OK) return rc;
  alif_scan_layout(T, N, C, K1, K2, out);
  return LSH_OK;
}

extern "C" size_t lsh_alif_scan_workspace(int64_t T, int64_t N, int C, int K1, int K2) {
  if (alif_scan_check(T, N, C, K1, K2, 1) != LSH_OK) return 0;
  lsh_alif_layout L;
  alif_scan_layout(T, N, C, K1, K2, &L);
  return L.total;
}

extern "C" int lsh_alif_scan_fwd(const float* I, const float* u0, const float* w0,
                                 const float* Wpred, float dw, float* U, float* W, float* S,
                                 int64_t T, int64_t N, float beta, float rho, float q, float theta0,
                                 float u_r, float rhoC, int C, int K1, int K2, int block,
                                 int64_t repair, void* ws, size_t ws_bytes,
                                 void* const* phase_events, void* stream) {
  if (bad_ptr(I) || bad_ptr(u0) || bad_ptr(w0) || bad_ptr(Wpred) || bad_ptr(U) || bad_ptr(W) ||
      bad_ptr(S) || bad_ptr(ws))
    return LSH_ERR_ARG;
  if (repair < -1) return LSH_ERR_ARG;
  const int rc = alif_scan_check(T, N, C, K1, K2, block);
  if (rc != LSH_OK) return rc;
  lsh_alif_layout L;
  alif_scan_layout(T, N, C, K1, K2, &L);
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
  auto F = [&](size_t off) { return reinterpret_cast<float*>(w + off); };
  auto Iq = [&](size_t off) { return reinterpret_cast<int*>(w + off); };
  auto mark = [&](int k) {
    if (phase_events && phase_events[k]) (void)hipEventRecord((hipEvent_t)phase_events[k], st);
  };
  mark(0);
  hipLaunchKernelGGL(k_env_chunks, dim3((unsigned)((int64_t)M * NB)), dim3(WAVE), 0, st, I, F(L.EC),
                     F(L.EA), F(L.EB), N, NB, C, beta, u_r);
  hipLaunchKernelGGL(k_env_carry, dim3((unsigned)NB), dim3(WAVE), 0, st, u0, F(L.EC), F(L.EA),
                     F(L.EB), F(L.LU), N, M);
  mark(1);  // the entry box belongs to the build phase, as in the reference (triton_alif.py:314-329)
  hipLaunchKernelGGL(k_alif_box, dim3((unsigned)((int64_t)M * NB)), dim3(WAVE), 0, st, Wpred, w0,
                     F(L.LW), F(L.HW), F(L.HU), N, NB, dw, rho, theta0, u_r);
  switch (block) {
    case 1: launch_alif_build<1>(I, w, L, N, M, C, K1, K2, beta, rho, q, theta0, u_r, st); break;
    case 2: launch_alif_build<2>(I, w, L, N, M, C, K1, K2, beta, rho, q, theta0, u_r, st); break;
    case 4: launch_alif_build<4>(I, w, L, N, M, C, K1, K2, beta, rho, q, theta0, u_r, st); break;
    case 8: launch_alif_build<8>(I, w, L, N, M, C, K1, K2, beta, rho, q, theta0, u_r, st); break;
    default: launch_alif_build<16>(I, w, L, N, M, C, K1, K2, beta, rho, q, theta0, u_r, st); break;
  }
  mark(2);
  // workgroups of 16 neurons, the grid rounded up to a multiple of 8 (one share per XCD)
  const int npw = N <= kCarryNpw1MaxN ? 1 : 4;
  const int64_t carry_groups = (N + npw * kCarryWaves - 1) / (npw * kCarryWaves);
  auto carry = npw == 1 ? k_alif_carry<1, 1> : k_alif_carry<1, 4>;
  hipLaunchKernelGGL(carry, dim3((unsigned)(8 * ((carry_groups + 7) / 8))),
                     dim3(WAVE * kCarryWaves), 0, st, I, u0, w0,
                     F(L.LU), F(L.HU), F(L.LW), F(L.HW), F(L.MA), F(L.MB), Iq(L.NL), Iq(L.NP),
                     Iq(L.OVF), F(L.LS), F(L.LC), F(L.LX), Iq(L.POWN), F(L.PXL), F(L.PXR), F(L.PU),
                     F(L.PA), F(L.POF), F(L.SU), F(L.SW), Iq(L.MISS), Iq(L.MSTAR), h, N, M, C, K1,
                     K2, beta, rho, q, theta0, u_r, rhoC, repair == -1 && M > 1 ? 1 : 0);
  mark(3);
  // repair to convergence: the replay covers the chunks whose starts are the serial states
  // (below mstar), and one serial pass per block of 64 neurons runs from the block's least
  // mstar on, from the exact exit before it (the converged Jacobi rounds' result)
  const bool chain = repair == -1 && M > 1;
  launch_alif_fwd<16>(I, F(L.SU), F(L.SW), U, W, S, F(L.EU), F(L.EW), N, C, M, beta, rho, q, theta0,
                      u_r, st, nullptr, chain ? Iq(L.MSTAR) : nullptr);
  mark(4);
  if (chain) {
    hipLaunchKernelGGL(k_alif_fwd_pipe, dim3((unsigned)NB), dim3(WAVE * (ALIF_PIPE_P + 1)), 0, st,
                       I, u0, w0, U, W, S, N, T, beta, rho, q, theta0, u_r, nullptr, Iq(L.MSTAR),
                       F(L.EU), F(L.EW), C);
  } else if (repair > 0 && M > 1) {
    const int64_t rounds = repair < (int64_t)M ? repair : (int64_t)M;
    hipLaunchKernelGGL(k_alif_repair, dim3((unsigned)NB), dim3(256), 0, st, I, U, W, S, F(L.SU),
                       F(L.SW), F(L.EU), F(L.EW), Iq(L.LIST0), Iq(L.LIST1), h, N, M, C, rounds, beta,
                       rho, q, theta0, u_r);
  }
  LSH_CHECK_LAUNCH();
  return LSH_OK;
}

extern "C" size_t lsh_alif_bwd_workspace(int64_t T, int64_t N, int C) {
  if (T < 0 || N < 0 || C < 1 || T % C != 0) return 0;
  const size_t mn = (size_t)(T / C) * (size_t)N * 4;
  return kWsHeaderBytes + 3 * align_up(mn, 256);
}

extern "C" size_t lsh_alif_bwd_lookback_workspace(int64_t T, int64_t N) {
  if (T < 0 || N < 0 || T % ALIF_LB_SEG != 0) return 0;
  const size_t sn = (size_t)(T / ALIF_LB_SEG) * (size_t)N;
  const size_t nf = (size_t)(T / ALIF_LB_SEG) * (size_t)((N + WAVE - 1) / WAVE);
  return kWsHeaderBytes + align_up(6 * sn * 4, 256) + align_up(2 * nf * 4, 256);
}

extern "C" int64_t lsh_alif_bwd_partials(int64_t T, int64_t N, int mode, int C) {
  if (T < 0 || N < 0 || mode < 0 || mode > 3) return -1;
  const int64_t NB = (N + WAVE - 1) / WAVE;
  if (mode == 3) return T % ALIF_LB_SEG == 0 ? (T / ALIF_LB_SEG) * NB : -1;
  if (mode != 1) return NB;
  if (C < 1 || T % C != 0) return -1;
  return (T / C) * NB;
}

template <int C, int W, bool WLW, bool PS, bool RC>
static void launch_alif_fused_w(const float* I, const float* u0, const float* w0, const float* U,
                                const float* W_, const float* S, const float* GS, float* LW,
                                float* LV, float* DW0, double* partials, int64_t N, int M, int NB,
                                float beta, float rho, float q, float theta0, float alpha,
                                float u_r, hipStream_t st, const float* dpar) {
  hipLaunchKernelGGL((k_alif_bwd_fused<C, W, WLW, PS, RC>), dim3((unsigned)NB), dim3(WAVE * W), 0, st,
                     I, u0, w0, U, W_, S, GS, LW, LV, DW0, partials, N, M, beta, rho, q, theta0,
                     alpha, u_r, dpar);
}

// RC (recompute the states) keeps the stored-state variant's wave count, so both sum the
// chunks in the same order.
template <int C, bool WLW, bool PS, bool RC = false>
static void launch_alif_fused(const float* I, const float* u0, const float* w0, const float* U,
                              const float* W, const float* S, const float* GS, float* LW, float* LV,
                              float* DW0, double* partials, int64_t N, int M, int NB, float beta,
                              float rho, float q, float theta0, float alpha, hipStream_t st,
                              const float* dpar, float u_r = 0.0f) {
  // registers allow 16 waves at C = 16 without the parameter sums, 4 at C = 32 with them, else 8
  constexpr int WMAX = (C == 16 && !PS) ? 16 : ((C == 32 && PS) ? 4 : 8);
  const int nw = fused_waves(NB, WMAX);
  if constexpr (WMAX >= 16) {
    if (nw == 16) {
      launch_alif_fused_w<C, 16, WLW, PS, RC>(I, u0, w0, U, W, S, GS, LW, LV, DW0, partials, N, M, NB,
                                              beta, rho, q, theta0, alpha, u_r, st, dpar);
      return;
    }
  }
  if (nw == 8)
    launch_alif_fused_w<C, 8, WLW, PS, RC>(I, u0, w0, U, W, S, GS, LW, LV, DW0, partials, N, M, NB,
                                           beta, rho, q, theta0, alpha, u_r, st, dpar);
  else
    launch_alif_fused_w<C, 4, WLW, PS, RC>(I, u0, w0, U, W, S, GS, LW, LV, DW0, partials, N, M, NB,
                                           beta, rho, q, theta0, alpha, u_r, st, dpar);
}

template <bool WLW, bool PS>
static void launch_alif_serial_bwd(const float* I, const float* u0, const float* w0, const float* U,
                                   const float* W, const float* S, const float* GS, float* LW,
                                   float* LV, float* DW0, double* partials, int64_t N, int64_t T,
                                   int NB, float beta, float rho, float q, float theta0, float alpha,
                                   hipStream_t st, const float* dpar) {
  hipLaunchKernelGGL((k_alif_bwd_pipe<WLW, PS>), dim3((unsigned)NB), dim3(WAVE * (ALIF_PIPE_P + 1)),
                     0, st, I, u0, w0, U, W, S, GS, LW, LV, DW0, partials, N, T, beta, rho, q,
                     theta0, alpha, dpar);
}

// The look-back single pass (mode 3): header reset, flags cleared, one workgroup per (segment,
// 64-neuron block).  Shapes and the workspace are checked by the caller.
template <bool RC>
static void alif_lookback_launch(const float* I, const float* U, const float* W, const float* S,
                                 const float* GS, const float* u0, const float* w0, float* LV,
                                 float* LW, float* DW0, double* partials, int64_t T, int64_t N,
                                 float beta, float rho, float q, float theta0, float u_r, float alpha,
                                 const float* dpar, void* ws, hipStream_t st) {
  const int NB = (int)((N + WAVE - 1) / WAVE);
  const int NSEG = (int)(T / ALIF_LB_SEG);
  const size_t sn = (size_t)NSEG * (size_t)N;
  char* wsb = static_cast<char*>(ws);
  WsHeader* hdr = reinterpret_cast<WsHeader*>(wsb);
  float* agg = reinterpret_cast<float*>(wsb + kWsHeaderBytes);
  int* flags = reinterpret_cast<int*>(wsb + kWsHeaderBytes + align_up(6 * sn * 4, 256));
  hipLaunchKernelGGL(k_ws_header_reset, dim3(1), dim3(64), 0, st, hdr);
  fill_i32_launch(flags, 2 * (int64_t)NSEG * NB, 0, st);
  const bool wlw = LW != nullptr, ps = partials != nullptr;
#define LSH_LB(WL, P)                                                                              \
  hipLaunchKernelGGL((k_alif_bwd_lookback<WL, P, RC>), dim3((unsigned)((int64_t)NSEG * NB)),       \
                     dim3(WAVE * ALIF_LB_W), 0, st, I, u0, w0, U, W, S, GS, LW, LV, DW0, partials,  \
                     agg, flags, hdr, N, NB, NSEG, beta, rho, q, theta0, alpha, u_r, dpar)
  if (wlw && ps)
    LSH_LB(true, true);
  else if (wlw)
    LSH_LB(true, false);
  else if (ps)
    LSH_LB(false, true);
  else
    LSH_LB(false, false);
#undef LSH_LB
}

static int alif_bwd(const float* I, const float* U, const float* W, const float* S,
                    const float* GS, const float* u0, const float* w0, float* LV, float* LW,
                    float* DW0, double* partials, int64_t T, int64_t N, float beta, float rho,
                    float q, float theta0, float alpha, const float* dpar, int mode, int C, void* ws,
                    size_t ws_bytes, void* stream) {
  if (bad_ptr(I) || bad_ptr(U) || bad_ptr(W) || bad_ptr(S) || bad_ptr(GS) || bad_ptr(u0) ||
      bad_ptr(w0) || bad_ptr(LV))
    return LSH_ERR_ARG;
  if (T < 0 || N < 0 || N > (int64_t)1 << 31) return LSH_ERR_SHAPE;
  if (mode < 0 || mode > 3) return LSH_ERR_ARG;
  if (mode == 1 && bad_ptr(LW)) return LSH_ERR_ARG;  // the chunked scans keep LW in between
  if (mode == 3) {  // look-back single pass (few neurons)
    if (T % ALIF_LB_SEG != 0) return LSH_ERR_DIVISIBILITY;
    if ((uint64_t)N * (uint64_t)ALIF_LB_C * 4u >= ((uint64_t)1 << 32)) return LSH_ERR_SHAPE;
    if ((T / ALIF_LB_SEG) * ((N + WAVE - 1) / WAVE) > ((int64_t)1 << 31) - 1) return LSH_ERR_SHAPE;
    if (bad_ptr(ws) || ws_bytes < lsh_alif_bwd_lookback_workspace(T, N) ||
        (reinterpret_cast<uintptr_t>(ws) & 255u) != 0)
      return LSH_ERR_WORKSPACE;
  }
  if (T == 0 || N == 0) return LSH_OK;
  hipStream_t st = (hipStream_t)stream;
  const int NB = (int)((N + WAVE - 1) / WAVE);
  const bool wlw = LW != nullptr, ps = partials != nullptr;
  if (mode == 3) {
    alif_lookback_launch<false>(I, U, W, S, GS, u0, w0, LV, LW, DW0, partials, T, N, beta, rho, q,
                                theta0, 0.0f, alpha, dpar, ws, st);
    LSH_CHECK_LAUNCH();
    return LSH_OK;
  }
  if (mode == 0) {
    if (wlw && ps)
      launch_alif_serial_bwd<true, true>(I, u0, w0, U, W, S, GS, LW, LV, DW0, partials, N, T, NB, beta,
                                         rho, q, theta0, alpha, st, dpar);
    else if (wlw)
      launch_alif_serial_bwd<true, false>(I, u0, w0, U, W, S, GS, LW, LV, DW0, partials, N, T, NB,
                                          beta, rho, q, theta0, alpha, st, dpar);
    else if (ps)
      launch_alif_serial_bwd<false, true>(I, u0, w0, U, W, S, GS, LW, LV, DW0, partials, N, T, NB,
                                          beta, rho, q, theta0, alpha, st, dpar);
    else
      launch_alif_serial_bwd<false, false>(I, u0, w0, U, W, S, GS, LW, LV, DW0, partials, N, T, NB,
                                           beta, rho, q, theta0, alpha, st, dpar);
    LSH_CHECK_LAUNCH();
    return LSH_OK;
  }
  if (C < 1) return LSH_ERR_SHAPE;
  if (T % C != 0) return LSH_ERR_DIVISIBILITY;
  const int M = (int)(T / C);
  if (mode == 2) {  // single pass
    if (C != 16 && C != 32) return LSH_ERR_SHAPE;
    if ((uint64_t)N * (uint64_t)C * 4u >= ((uint64_t)1 << 32)) return LSH_ERR_SHAPE;
#define LSH_FUSED(CC)                                                                              \
  do {                                                                                             \
    if (wlw && ps)                                                                                 \
      launch_alif_fused<CC, true, true>(I, u0, w0, U, W, S, GS, LW, LV, DW0, partials, N, M, NB,   \
                                        beta, rho, q, theta0, alpha, st, dpar);                    \
    else if (wlw)                                                                                  \
      launch_alif_fused<CC, true, false>(I, u0, w0, U, W, S, GS, LW, LV, DW0, partials, N, M, NB,  \
                                         beta, rho, q, theta0, alpha, st, dpar);                   \
    else if (ps)                                                                                   \
      launch_alif_fused<CC, false, true>(I, u0, w0, U, W, S, GS, LW, LV, DW0, partials, N, M, NB,  \
                                         beta, rho, q, theta0, alpha, st, dpar);                   \
    else                                                                                           \
      launch_alif_fused<CC, false, false>(I, u0, w0, U, W, S, GS, LW, LV, DW0, partials, N, M, NB, \
                                          beta, rho, q, theta0, alpha, st, dpar);                  \
  } while (0)
    if (C == 16)
      LSH_FUSED(16);
    else
      LSH_FUSED(32);
#undef LSH_FUSED
    LSH_CHECK_LAUNCH();
    return LSH_OK;
  }
  // chunked two-level scans (triton_alif.py:510-521)
  if (bad_ptr(ws) || ws_bytes < lsh_alif_bwd_workspace(T, N, C) ||
      (reinterpret_cast<uintptr_t>(ws) & 255u) != 0)
    return LSH_ERR_WORKSPACE;
  const size_t mn = align_up((size_t)M * (size_t)N * 4, 256);
  char* w = static_cast<char*>(ws) + kWsHeaderBytes;
  float* PA_ = reinterpret_cast<float*>(w);
  float* PB_ = reinterpret_cast<float*>(w + mn);
  float* LE = reinterpret_cast<float*>(w + 2 * mn);
  const dim3 g((unsigned)((int64_t)M * NB)), b(WAVE), gc((unsigned)NB);
  hipLaunchKernelGGL((k_alif_bwd<0, false>), g, b, 0, st, I, u0, w0, U, W, S, GS, LW, LV, PA_, PB_,
                     nullptr, nullptr, nullptr, N, C, NB, beta, rho, q, theta0, alpha, dpar);
  hipLaunchKernelGGL(k_rev_carry, gc, b, 0, st, PA_, PB_, LE, N, M);
  hipLaunchKernelGGL((k_alif_bwd<1, false>), g, b, 0, st, I, u0, w0, U, W, S, GS, LW, LV, PA_, PB_, LE,
                     DW0, nullptr, N, C, NB, beta, rho, q, theta0, alpha, dpar);
  hipLaunchKernelGGL((k_alif_bwd<2, false>), g, b, 0, st, I, u0, w0, U, W, S, GS, LW, LV, PA_, PB_,
                     nullptr, nullptr, nullptr, N, C, NB, beta, rho, q, theta0, alpha, dpar);
  hipLaunchKernelGGL(k_rev_carry, gc, b, 0, st, PA_, PB_, LE, N, M);
  if (ps)
    hipLaunchKernelGGL((k_alif_bwd<3, true>), g, b, 0, st, I, u0, w0, U, W, S, GS, LW, LV, PA_, PB_,
                       LE, nullptr, partials, N, C, NB, beta, rho, q, theta0, alpha, dpar);
  else
    hipLaunchKernelGGL((k_alif_bwd<3, false>), g, b, 0, st, I, u0, w0, U, W, S, GS, LW, LV, PA_, PB_,
                       LE, nullptr, nullptr, N, C, NB, beta, rho, q, theta0, alpha, dpar);
  LSH_CHECK_LAUNCH();
  return LSH_OK;
}

extern "C" int lsh_alif_bwd(const float* I, const float* U, const float* W, const float* S,
                            const float* GS, const float* u0, const float* w0, float* LV,
                            float* LW, float* DW0, double* partials, int64_t T, int64_t N,
                            float beta, float rho, float q, float theta0, float alpha, int mode,
                            int C, void* ws, size_t ws_bytes, void* stream) {
  return alif_bwd(I, U, W, S, GS, u0, w0, LV, LW, DW0, partials, T, N, beta, rho, q, theta0, alpha,
                  nullptr, mode, C, ws, ws_bytes, stream);
}

extern "C" int lsh_alif_bwd_dparams(const float* I, const float* U, const float* W,
                                    const float* S, const float* GS, const float* u0,
                                    const float* w0, float* LV, float* LW, float* DW0,
                                    double* partials, int64_t T, int64_t N, const float* params,
                                    float alpha, int mode, int C, void* ws, size_t ws_bytes,
                                    void* stream) {
  if (bad_ptr(params)) return LSH_ERR_ARG;
  return alif_bwd(I, U, W, S, GS, u0, w0, LV, LW, DW0, partials, T, N, 0.0f, 0.0f, 0.0f, 0.0f,
                  alpha, params, mode, C, ws, ws_bytes, stream);
}

// Single-pass adjoint with the states recomputed from the rows before each chunk (RC above);
// params (if given) is the device vector [beta, rho, q, theta0] read in place of the floats.
extern "C" int lsh_alif_bwd_recompute(const float* I, const float* U, const float* W,
                                      const float* GS, const float* u0, const float* w0, float* LV,
                                      float* LW, float* DW0, double* partials, int64_t T, int64_t N,
                                      const float* params, float beta, float rho, float q,
                                      float theta0, float u_r, float alpha, int mode, int C,
                                      void* ws, size_t ws_bytes, void* stream) {
  if (bad_ptr(I) || bad_ptr(U) || bad_ptr(W) || bad_ptr(GS) || bad_ptr(u0) || bad_ptr(w0) ||
      bad_ptr(LV))
    return LSH_ERR_ARG;
  if (T < 0 || N < 0 || N > (int64_t)1 << 31) return LSH_ERR_SHAPE;
  if (mode != 2 && mode != 3) return LSH_ERR_ARG;
  if (mode == 3) {
    if (T % ALIF_LB_SEG != 0) return LSH_ERR_DIVISIBILITY;
    if ((uint64_t)N * (uint64_t)ALIF_LB_C * 4u >= ((uint64_t)1 << 32)) return LSH_ERR_SHAPE;
    if ((T / ALIF_LB_SEG) * ((N + WAVE - 1) / WAVE) > ((int64_t)1 << 31) - 1) return LSH_ERR_SHAPE;
    if (bad_ptr(ws) || ws_bytes < lsh_alif_bwd_lookback_workspace(T, N) ||
        (reinterpret_cast<uintptr_t>(ws) & 255u) != 0)
      return LSH_ERR_WORKSPACE;
    if (T == 0 || N == 0) return LSH_OK;
    alif_lookback_launch<true>(I, U, W, nullptr, GS, u0, w0, LV, LW, DW0, partials, T, N, beta, rho,
                               q, theta0, u_r, alpha, params, ws, (hipStream_t)stream);
    LSH_CHECK_LAUNCH();
    return LSH_OK;
  }
  if (C != 16 && C != 32) return LSH_ERR_SHAPE;
  if (T % C != 0) return LSH_ERR_DIVISIBILITY;
  if ((uint64_t)N * (uint64_t)C * 4u >= ((uint64_t)1 << 32)) return LSH_ERR_SHAPE;
  if (T == 0 || N == 0) return LSH_OK;
  hipStream_t st = (hipStream_t)stream;
  const int NB = (int)((N + WAVE - 1) / WAVE);
  const int M = (int)(T / C);
  const bool wlw = LW != nullptr, ps = partials != nullptr;
  const float* S = nullptr;  // not read
  const float* dpar = params;
#define LSH_FUSED_RC(CC)                                                                           \
  do {                                                                                             \
    if (wlw && ps)                                                                                 \
      launch_alif_fused<CC, true, true, true>(I, u0, w0, U, W, S, GS, LW, LV, DW0, partials, N, M, \
                                              NB, beta, rho, q, theta0, alpha, st, dpar, u_r);     \
    else if (wlw)                                                                                  \
      launch_alif_fused<CC, true, false, true>(I, u0, w0, U, W, S, GS, LW, LV, DW0, partials, N,   \
                                               M, NB, beta, rho, q, theta0, alpha, st, dpar, u_r); \
    else if (ps)                                                                                   \
      launch_alif_fused<CC, false, true, true>(I, u0, w0, U, W, S, GS, LW, LV, DW0, partials, N,   \
                                               M, NB, beta, rho, q, theta0, alpha, st, dpar, u_r); \
    else                                                                                           \
      launch_alif_fused<CC, false, false, true>(I, u0, w0, U, W, S, GS, LW, LV, DW0, partials, N,  \
                                                M, NB, beta, rho, q, theta0, alpha, st, dpar,      \
                                                u_r);                                              \
  } while (0)
  if (C == 16)
    LSH_FUSED_RC(16);
  else
    LSH_FUSED_RC(32);
#undef LSH_FUSED_RC
  LSH_CHECK_LAUNCH();
  return LSH_OK;
}
