// Three-level exact scan for long sequences (reference: triton_lif.py:935-983,
// scan_forward_v4): chunk maps are composed in groups of G into super-chunk maps of capacity
// K2, the carry runs over the M/G super maps, then inside every super map in parallel, then
// every chunk is replayed.  Sequential depth ~ C + G (compose) + M/G + G + C instead of
// C + M + C.
//
// Kernels (one lane per neuron, one wave per 64 neurons):
//   k_lif_env_lo      sequential over chunks (three loads a chunk, tile-prefetched): the
//                     envelope bound Lo[m] of every chunk entry;
//   k_lif_trunc       per (chunk, neuron): the reference's lo-pruned map (breakpoint count,
//                     overflow flag) by truncating the hi-pruned map of k_lif_build;
//   k_lif_compose     per (super, neuron): G-1 compositions (triton_lif.py:829-899);
//   k_map_carry       sequential over super maps with overflow-to-serial fallback
//                     (triton_lif.py:579-606 with K = K2 and fallback length C*G);
//   k_lif_carry_inner per (super, neuron): G chunk-map evaluations (triton_lif.py:903-932).
#include <algorithm>

#include "lsh_abi.h"
#include "lsh_common.h"

namespace lsh {

// Map evaluation (triton_lif.py:592-599): k = #{i < n : xd[i] > u}; k == n -> A*u + B,
// else cd[k].
template <int KMAX>
__device__ __forceinline__ float eval_slots(const float* xd, const float* cd, int n, float A,
                                            float B, float u) {
  int k = 0;
#pragma unroll
  for (int i = 0; i < KMAX; ++i) k += (i < n && xd[i] > u) ? 1 : 0;
  float c = 0.0f;
#pragma unroll
  for (int i = 0; i < KMAX; ++i) c = (i == k) ? cd[i] : c;
  return k == n ? __fadd_rn(__fmul_rn(A, u), B) : c;
}

// Serial fallback over L steps of column n from row r0 (same step arithmetic as the replay).
__device__ __forceinline__ float serial_rows(const float* __restrict__ I, int64_t N, int64_t n,
                                             int64_t r0, int64_t L, float u, float beta,
                                             float theta, float u_r) {
  stream_rows<16>(I + (size_t)r0 * N + n, (size_t)N, L, [&](int64_t, float x) {
    bool s;
    u = lif_step(u, x, beta, theta, u_r, s);
  });
  return u;
}

// Envelope bound of every chunk entry (triton_lif.py:723-733):
//   LO[m] = l - 1e-5(|l| + 1),  l <- min(EC[m], EA[m]*l + EB[m]),  l = u0 at m = 0.
// Sequential over the chunks of a neuron but only three loads a chunk, issued in tiles of D
// ahead of their use.
template <int D>
__global__ __launch_bounds__(64) void k_lif_env_lo(const float* __restrict__ u0,
                                                   const float* __restrict__ EC,
                                                   const float* __restrict__ EA,
                                                   const float* __restrict__ EB,
                                                   float* __restrict__ LO, int64_t N, int M) {
  const int64_t n = (int64_t)blockIdx.x * WAVE + threadIdx.x;
  if (n >= N) return;
  const float margin = 1e-5f;
  float l = u0[n];
  auto step = [&](int m, float c, float a, float b) {
    LO[(size_t)m * N + n] = l - margin * (fabsf(l) + 1.0f);
    l = fminf(c, __fadd_rn(__fmul_rn(a, l), b));
  };
  const int nt = M / D;
  float ca[D], aa[D], ba[D];
  auto load = [&](int t, float* c, float* a, float* b) {
#pragma unroll
    for (int k = 0; k < D; ++k) {
      const size_t o = (size_t)(t * D + k) * N + n;
      c[k] = EC[o];
      a[k] = EA[o];
      b[k] = EB[o];
    }
  };
  if (nt > 0) load(0, ca, aa, ba);
  for (int t = 0; t < nt; ++t) {
    float cb[D], ab[D], bb[D];
    const bool more = t + 1 < nt;
    if (more) load(t + 1, cb, ab, bb);
#pragma unroll
    for (int k = 0; k < D; ++k) step(t * D + k, ca[k], aa[k], ba[k]);
    if (more) {
#pragma unroll
      for (int k = 0; k < D; ++k) {
        ca[k] = cb[k];
        aa[k] = ab[k];
        ba[k] = bb[k];
      }
    }
  }
  for (int m = nt * D; m < M; ++m) {
    const size_t o = (size_t)m * N + n;
    step(m, EC[o], EA[o], EB[o]);
  }
}

// Truncation of every hi-only chunk map at its entry bound (in parallel over chunks and
// neurons): the reference's map is the prefix up to the first breakpoint <= LO, and it
// overflowed iff a (K+1)-th breakpoint appeared and all K stored ones are > LO.  A block of
// 64 neurons takes every MB-th chunk (grid NB x MB), so the header counters see one atomic per
// block rather than one per chunk.
template <int KMAX>
__global__ __launch_bounds__(64) void k_lif_trunc(const float* __restrict__ LO,
                                                  const int* __restrict__ CNT,
                                                  const int* __restrict__ OVFRAW,
                                                  const float* __restrict__ MX,
                                                  int* __restrict__ MN, int* __restrict__ OVF,
                                                  WsHeader* hdr, int64_t N, int NB, int M, int MB,
                                                  int K) {
  const int nb = blockIdx.x % NB;
  const int mb = blockIdx.x / NB;
  const int64_t n = (int64_t)nb * WAVE + threadIdx.x;
  unsigned long long ovf_acc = 0, pcs_acc = 0;
  int pmax = 0;
  if (n < N && mb < M) {
    // a chunk's loads do not wait for its count (every slot is read, the index clamped below
    // K; the count masks the compares), and the next chunk's are issued before this one is
    // counted (the last chunk reloads itself), so the walk waits on one load latency a chunk
    struct Row {
      float lo;
      int cnt, ovr;
      float x[KMAX];
    };
    auto load = [&](int m, Row& r) {
      const size_t o = (size_t)m * N + n;
      r.lo = LO[o];
      r.cnt = CNT[o];
      r.ovr = OVFRAW[o];
#pragma unroll
      for (int i = 0; i < KMAX; ++i) r.x[i] = MX[((size_t)m * K + min(i, K - 1)) * N + n];
    };
    Row cur, nxt;
    load(mb, cur);
    for (int m = mb; m < M; m += MB) {
      load(m + MB < M ? m + MB : m, nxt);
      int gt = 0;
#pragma unroll
      for (int i = 0; i < KMAX; ++i) gt += (i < K && i < cur.cnt && cur.x[i] > cur.lo) ? 1 : 0;
      const int ne = min(cur.cnt, gt + 1);
      const bool ovf = cur.ovr != 0 && gt == cur.cnt;
      const size_t o = (size_t)m * N + n;
      MN[o] = ne;
      OVF[o] = ovf ? 1 : 0;
      ovf_acc += ovf ? 1ull : 0ull;
      pcs_acc += (unsigned long long)ne;
      pmax = max(pmax, ne);
      cur = nxt;
    }
  }
  ovf_acc = wave_sum_u64(ovf_acc);
  pcs_acc = wave_sum_u64(pcs_acc);
  pmax = wave_max_i(pmax);
  if (threadIdx.x == 0) {
    if (ovf_acc) atomicAdd(&hdr->ovf_count, ovf_acc);
    atomicAdd(&hdr->pieces_sum, pcs_acc);
    atomicMax(&hdr->pieces_max, (unsigned int)pmax);
  }
}

template <int KMAX, int K2MAX>
__global__ __launch_bounds__(64) void k_lif_compose(
    const float* __restrict__ MA, const float* __restrict__ MB, const int* __restrict__ MN,
    const int* __restrict__ OVF, const float* __restrict__ MX, const float* __restrict__ MC,
    const float* __restrict__ LO, const float* __restrict__ u0, float* __restrict__ SA,
    float* __restrict__ SB, int* __restrict__ SN, int* __restrict__ SOVF, float* __restrict__ SX,
    float* __restrict__ SC, WsHeader* hdr, int64_t N, int NB, int G, int K, int K2, float theta,
    float u_r) {
  const int64_t s = blockIdx.x / NB;
  const int nb = (int)(blockIdx.x - s * NB);
  const int64_t n = (int64_t)nb * WAVE + threadIdx.x;
  const bool valid = n < N;
  const int64_t nn = valid ? n : N - 1;
  const int64_t m0 = s * G;
  const float lo = LO[(size_t)m0 * N + nn];
  const float hi = fmaxf(u0[nn], fmaxf(theta, u_r));
  float A = MA[(size_t)m0 * N + nn], B = MB[(size_t)m0 * N + nn];
  int nH = MN[(size_t)m0 * N + nn];
  int ov = OVF[(size_t)m0 * N + nn];
  float X[K2MAX], Cc[K2MAX];
#pragma unroll
  for (int i = 0; i < K2MAX; ++i) {
    const bool in = i < K && i < K2;
    X[i] = in ? MX[((size_t)m0 * K + i) * N + nn] : INFINITY;
    Cc[i] = in ? MC[((size_t)m0 * K + i) * N + nn] : 0.0f;
  }
  float xmin = INFINITY;
#pragma unroll
  for (int i = 0; i < K2MAX; ++i) xmin = (i < nH) ? fminf(xmin, X[i]) : xmin;
  // the wave's largest slot counts, as scalars (the guards below are then scalar branches, where
  // a lane-reduced value in a vector register would make each one an exec-mask update)
  int wnH = __builtin_amdgcn_readfirstlane(wave_max_i(nH));
  for (int jj = 1; jj < G; ++jj) {
    const int64_t m = m0 + jj;
    const size_t o = (size_t)m * N + nn;
    const float Ag = MA[o], Bg = MB[o];
    const int ng = MN[o];
    ov |= OVF[o];
    const int wng = __builtin_amdgcn_readfirstlane(wave_max_i(ng));
    float yd[KMAX], dd[KMAX];
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
      if (j < wng) {
        yd[j] = MX[((size_t)m * K + j) * N + nn];
        dd[j] = MC[((size_t)m * K + j) * N + nn];
      } else {
        yd[j] = INFINITY;
        dd[j] = 0.0f;
      }
    }
    // (1) the left map's constants pushed through the right map: c = #{j < ng : yd[j] > C}, a
    // prefix of the strictly descending breakpoints, so the constant dd[c] is the one after the
    // last breakpoint above C (dd[0] if none), picked up in the same pass
#pragma unroll
    for (int i = 0; i < K2MAX; ++i) {
      if (i < wnH) {
        int c = 0;
        float gc = dd[0];
#pragma unroll
        for (int j = 0; j < KMAX; ++j) {
          if (j < wng) {
            const bool gt = j < ng && yd[j] > Cc[i];
            c += gt ? 1 : 0;
            if (j + 1 < KMAX) gc = gt ? dd[j + 1] : gc;
          }
        }
        Cc[i] = (c == ng) ? __fadd_rn(__fmul_rn(Ag, Cc[i]), Bg) : gc;
      }
    }
    // (2) the right map's breakpoints pulled back through the left map's affine part
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
      if (j < wng) {
        const float num = yd[j] - B;
        const float z = A == 0.0f ? (num > 0.0f ? INFINITY : -INFINITY) : num / A;
        bool nw = (j < ng) && (z < xmin) && (z <= hi) && (xmin > lo);
        if (nw && nH >= K2) ov = 1;
        nw = nw && (nH < K2);
        if (__ballot(nw) != 0ull) {  // skipped where no lane of the wave keeps the breakpoint
#pragma unroll
          for (int i = 0; i < K2MAX; ++i) {
            if (i <= wnH) {
              const bool put = nw && (i == nH);
              X[i] = put ? z : X[i];
              Cc[i] = put ? dd[j] : Cc[i];
            }
          }
          if (__ballot(nw && nH == wnH) != 0ull) ++wnH;
          nH += nw ? 1 : 0;
          xmin = nw ? z : xmin;
        }
      }
    }
    // (3) affine parts
    B = __fadd_rn(__fmul_rn(Ag, B), Bg);
    A = Ag * A;
  }
  unsigned long long so = 0, sp = 0;
  int smax = 0;
  if (valid) {
    const size_t o = (size_t)s * N + n;
    SA[o] = A;
    SB[o] = B;
    SN[o] = nH;
    SOVF[o] = ov;
#pragma unroll
    for (int i = 0; i < K2MAX; ++i) {
      if (i < K2) {
        SX[((size_t)s * K2 + i) * N + n] = X[i];
        SC[((size_t)s * K2 + i) * N + n] = Cc[i];
      }
    }
    so = ov ? 1ull : 0ull;
    sp = (unsigned long long)nH;
    smax = nH;
  }
  so = wave_sum_u64(so);
  sp = wave_sum_u64(sp);
  smax = wave_max_i(smax);
  if (threadIdx.x == 0) {
    atomicAdd(&hdr->super_ovf_count, so);
    atomicAdd(&hdr->super_pieces_sum, sp);
    atomicMax(&hdr->super_pieces_max, (unsigned int)smax);
  }
}

// The same composition with one wave per neuron, for few neurons (one lane per neuron gives
// M/G * N/64 waves, 128 at N = 128 and M/G = 64, each composing its slots one after another).
// A wave takes SPW consecutive super maps of one neuron; lane i holds slot i of the composed
// map (K2 <= 64) and of the chunk map being composed.  (1) pushes every kept constant through
// the right map at once (its count over the right map's breakpoints, read from their lanes, then
// a lane shuffle for the constant); (2) walks the right map's breakpoints in order, as wave-
// uniform values, appending the accepted ones in lane nH; the next chunk map's loads (indices
// clamped into the group) are issued before the current one is composed.  The same operations
// on the same values as k_lif_compose, so the same bits; the statistics take one atomic per
// wave.
__global__ __launch_bounds__(64) void k_lif_compose_wave(
    const float* __restrict__ MA, const float* __restrict__ MB, const int* __restrict__ MN,
    const int* __restrict__ OVF, const float* __restrict__ MX, const float* __restrict__ MC,
    const float* __restrict__ LO, const float* __restrict__ u0, float* __restrict__ SA,
    float* __restrict__ SB, int* __restrict__ SN, int* __restrict__ SOVF, float* __restrict__ SX,
    float* __restrict__ SC, WsHeader* hdr, int64_t N, int M2, int SPW, int G, int K, int K2,
    float theta, float u_r) {
  const int64_t b = blockIdx.x;
  const int64_t n = xcd_neuron(b % N, N);
  const int s0 = (int)(b / N) * SPW;
  const int lane = threadIdx.x;
  const int sl = min(lane, K - 1);
  const float hi = fmaxf(u0[n], fmaxf(theta, u_r));
  unsigned long long so = 0, sp = 0;
  int smax = 0;
  struct Chunk {
    float a, b, yd, dd;
    int cnt, ovf;
  };
  auto load = [&](int64_t m, Chunk& d) {
    const size_t o = (size_t)m * N + n;
    d.a = MA[o];
    d.b = MB[o];
    d.cnt = MN[o];
    d.ovf = OVF[o];
    const size_t os = ((size_t)m * K + sl) * N + n;
    d.yd = MX[os];
    d.dd = MC[os];
  };
  const int s1 = min(s0 + SPW, M2);
  for (int s = s0; s < s1; ++s) {
    const int64_t m0 = (int64_t)s * G;
    const float lo = LO[(size_t)m0 * N + n];
    Chunk h, nx;
    load(m0, h);
    load(m0 + min(1, G - 1), nx);
    float A = h.a, B = h.b;
    int nH = h.cnt;
    int ov = h.ovf;
    float X = lane < K ? h.yd : INFINITY;
    float Cc = lane < K ? h.dd : 0.0f;
    float xmin = INFINITY;
    for (int i = 0; i < nH; ++i) xmin = fminf(xmin, lane_f(X, i));
    for (int jj = 1; jj < G; ++jj) {
      const Chunk g = nx;
      load(m0 + min(jj + 1, G - 1), nx);
      const int ng = g.cnt;
      ov |= g.ovf;
      // (1) the left map's constants pushed through the right map
      int c = 0;
      for (int j = 0; j < ng; ++j) c += lane_f(g.yd, j) > Cc ? 1 : 0;
      const float gc = __shfl(g.dd, min(c, 63));
      if (lane < nH) Cc = (c == ng) ? __fadd_rn(__fmul_rn(g.a, Cc), g.b) : gc;
      // (2) the right map's breakpoints pulled back through the left map's affine part
      for (int j = 0; j < ng; ++j) {
        const float dj = lane_f(g.dd, j);
        const float num = lane_f(g.yd, j) - B;
        const float z = A == 0.0f ? (num > 0.0f ? INFINITY : -INFINITY) : num / A;
        bool nw = (z < xmin) && (z <= hi) && (xmin > lo);
        if (nw && nH >= K2) ov = 1;
        nw = nw && (nH < K2);
        if (nw) {
          if (lane == nH) {
            X = z;
            Cc = dj;
          }
          ++nH;
          xmin = z;
        }
      }
      // (3) affine parts
      B = __fadd_rn(__fmul_rn(g.a, B), g.b);
      A = g.a * A;
    }
    const size_t o = (size_t)s * N + n;
    if (lane == 0) {
      SA[o] = A;
      SB[o] = B;
      SN[o] = nH;
      SOVF[o] = ov;
    }
    if (lane < K2) {
      SX[((size_t)s * K2 + lane) * N + n] = X;
      SC[((size_t)s * K2 + lane) * N + n] = Cc;
    }
    so += ov ? 1ull : 0ull;
    sp += (unsigned long long)nH;
    smax = max(smax, nH);
  }
  if (lane == 0) {
    atomicAdd(&hdr->super_ovf_count, so);
    atomicAdd(&hdr->super_pieces_sum, sp);
    atomicMax(&hdr->super_pieces_max, (unsigned int)smax);
  }
}

// The chunk maps behind the super maps (truncated counts and overflow flags, as the inner
// carry reads them), for the fallback of an overflowed super map; walk = 0: serial steps.
// ChunkMaps::walk, the fallback of an overflowed super map: 0 its C*G serial steps, 1 the walk
// over its G chunk maps, kSuperAsStored none: the map as stored (converged calls only, where
// the repair replaces a start it got wrong).
constexpr int kSuperAsStored = 2;
struct ChunkMaps {
  const float* MA;
  const float* MB;
  const int* MN;
  const int* OVF;
  const float* MX;
  const float* MC;
  int K, G, C, walk;
  const float* XT;  // the slots transposed ([M, N, K]) for the one-wave walk, or null
  const float* CT;
};

template <int KMAX>
struct SuperMap {
  float xd[KMAX], cd[KMAX], a, b;
  int cnt, ovf;
};

// The G chunk maps of super map s evaluated in turn from u, as k_lif_carry_inner evaluates
// them (an overflowed chunk map runs its C steps serially): the fallback of an overflowed super
// map that costs G map evaluations instead of C*G steps.
template <int KW>
__device__ __forceinline__ float walk_chunk_maps(const float* __restrict__ I, const ChunkMaps& cm,
                                                 int64_t N, int64_t n, int64_t s, float u,
                                                 float beta, float theta, float u_r) {
  for (int jj = 0; jj < cm.G; ++jj) {
    const int64_t m = s * cm.G + jj;
    const size_t o = (size_t)m * N + n;
    float xd[KW], cd[KW];
#pragma unroll
    for (int i = 0; i < KW; ++i) {
      xd[i] = i < cm.K ? cm.MX[((size_t)m * cm.K + i) * N + n] : INFINITY;
      cd[i] = i < cm.K ? cm.MC[((size_t)m * cm.K + i) * N + n] : 0.0f;
    }
    float nu = eval_slots<KW>(xd, cd, cm.MN[o], cm.MA[o], cm.MB[o], u);
    if (cm.OVF[o]) nu = serial_rows(I, N, n, m * cm.C, cm.C, u, beta, theta, u_r);
    u = nu;
  }
  return u;
}

// Sequential carry over pre-pruned maps (n and ovf final); an overflowed map falls back to its
// L serial steps, or, with chunk maps given (cm.walk), to the walk over its G chunk maps.  The maps are read one ahead into a ring of two register sets (the loop unrolled by two, so no
// set is copied), every load unconditional with its index clamped into the arrays (map <= M -
// 1, slot <= K - 1; eval_slots masks the slots past the count): the compiler's wait for the map
// in use then leaves the next map's loads in flight.  Lanes past N repeat neuron N - 1 and store
// nothing.
template <int KMAX, int KW>
__global__ __launch_bounds__(64) void k_map_carry(
    const float* __restrict__ I, const float* __restrict__ u0, const float* __restrict__ MA,
    const float* __restrict__ MB, const int* __restrict__ MN, const int* __restrict__ OVF,
    const float* __restrict__ MX, const float* __restrict__ MC, float* __restrict__ starts,
    int64_t N, int M, int K, int64_t L, float beta, float theta, float u_r, ChunkMaps cm) {
  const int64_t n = (int64_t)blockIdx.x * WAVE + threadIdx.x;
  const bool valid = n < N;
  const int64_t nn = valid ? n : N - 1;
  if (M <= 0) return;
  float u = u0[nn];
  auto load = [&](int m, SuperMap<KMAX>& d) {
    const size_t mc = (size_t)min(m, M - 1);
    const size_t o = mc * N + nn;
    d.a = MA[o];
    d.b = MB[o];
    d.cnt = MN[o];
    d.ovf = OVF[o];
#pragma unroll
    for (int i = 0; i < KMAX; ++i) {
      const size_t os = (mc * K + min(i, K - 1)) * N + nn;
      d.xd[i] = MX[os];
      d.cd[i] = MC[os];
    }
  };
  SuperMap<KMAX> mr[2];
  load(0, mr[0]);
  for (int m0 = 0; m0 < M; m0 += 2) {
#pragma unroll
    for (int ph = 0; ph < 2; ++ph) {
      const int m = m0 + ph;
      if (m >= M) break;
      load(m + 1, mr[ph ^ 1]);
      const SuperMap<KMAX>& d = mr[ph];
      if (valid) starts[(size_t)m * N + nn] = u;
      float nu = eval_slots<KMAX>(d.xd, d.cd, d.cnt, d.a, d.b, u);
      if (d.ovf && cm.walk != kSuperAsStored)
        nu = cm.walk ? walk_chunk_maps<KW>(I, cm, N, nn, m, u, beta, theta, u_r)
                     : serial_rows(I, N, nn, (int64_t)m * L, L, u, beta, theta, u_r);
      u = nu;
    }
  }
}

// The two sequential walks above with one wave per neuron, for few neurons: one lane per
// neuron leaves one or two waves on the chip, each waiting on memory for every chunk or super
// map.  The maps go in windows of 64: lane j holds the scalars of the window's map j, the next
// window's loads are issued (indices clamped, so every load is issued) before the current one
// is walked, and the per-map outputs collect in lane c, stored once per window.  The
// operations and values are those of k_lif_env_lo and k_map_carry, so the bits are the same.
//
// Envelope bounds: l walks the window's envelope maps read from their lanes.
__global__ __launch_bounds__(64) void k_lif_env_lo_wave(const float* __restrict__ u0,
                                                        const float* __restrict__ EC,
                                                        const float* __restrict__ EA,
                                                        const float* __restrict__ EB,
                                                        float* __restrict__ LO, int64_t N, int M) {
  if (M <= 0) return;
  const int64_t n = xcd_neuron(blockIdx.x, N);
  const int lane = threadIdx.x;
  const float margin = 1e-5f;
  float l = u0[n];
  auto load = [&](int w, float& c, float& a, float& b) {
    const size_t o = (size_t)min(w * 64 + lane, M - 1) * N + n;
    c = EC[o];
    a = EA[o];
    b = EB[o];
  };
  const int NW = (M + 63) / 64;
  float c0, a0, b0;
  load(0, c0, a0, b0);
  for (int w = 0; w < NW; ++w) {
    float c1, a1, b1;
    load(min(w + 1, NW - 1), c1, a1, b1);
    const int nc = min(64, M - w * 64);
    // lane c keeps chunk c's entry bound l; the margin is applied to the window at once
    float l_o = 0.0f;
    auto step = [&](int c) {
      l_o = lane == c ? l : l_o;
      l = fminf(lane_f(c0, c), __fadd_rn(__fmul_rn(lane_f(a0, c), l), lane_f(b0, c)));
    };
    if (nc == 64) {  // a full window, unrolled so that the lane reads run ahead of the chain
#pragma unroll 16
      for (int c = 0; c < 64; ++c) step(c);
    } else {
      for (int c = 0; c < nc; ++c) step(c);
    }
    if (lane < nc) LO[(size_t)(w * 64 + lane) * N + n] = l_o - margin * (fabsf(l_o) + 1.0f);
    c0 = c1;
    a0 = a1;
    b0 = b1;
  }
}

// Super-map carry with one wave per neuron (K2 <= 64): for K2 <= 32 VGPR g holds super maps 2g
// and 2g + 1 of the window, lane 32h + s slot s of map 2g + h; for K2 <= 64 VGPR g holds map g on
// the whole wave.  k = #{s < n : xd[s] > u} is a ballot over the map's lanes and the constant a
// lane read.  An overflowed map reads its L rows 64 at a time, one per lane.
struct SuperWindow {
  float a, b;  // lane j: map j of the window
  int cnt, ovf;
  float xd[32], cd[32];  // VGPR g, lane RW h + s: slot s of map SPR g + h (k_map_carry_wave<RW>)
};

// The G chunk maps of super map s from u, with one wave per neuron (walk_chunk_maps's values):
// batches of 16 chunk maps, VGPR v of a batch holding chunks v*CPV .. v*CPV + CPV - 1 on rows of
// RW lanes (slot i of chunk b in lane (b % CPV) RW + i) and the chunk scalars on lanes 0-15;
// every load of a batch is issued before its first evaluation.
template <int RW>
__device__ __forceinline__ float wave_walk_chunk_maps(const float* __restrict__ I, const ChunkMaps& cm,
                                                      int64_t N, int64_t n, int64_t s, float u,
                                                      float beta, float theta, float u_r) {
  constexpr int CPV = 64 / RW;  // chunks per VGPR
  constexpr int NV = 16 / CPV;  // VGPRs per batch of 16 chunks
  const int lane = threadIdx.x & 63;
  const int row = lane / RW, slot = lane % RW;
  const int sl = min(slot, cm.K - 1);
  const int64_t c0 = s * cm.G;  // first chunk of the super map
  for (int j0 = 0; j0 < cm.G; j0 += 16) {
    const int nb = min(16, cm.G - j0);
    float xv[NV], cv[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const size_t m = (size_t)(c0 + j0 + min(v * CPV + row, nb - 1));
      if (cm.XT) {  // a chunk's slots in one segment: one line per row of the load
        xv[v] = cm.XT[(m * N + n) * cm.K + sl];
        cv[v] = cm.CT[(m * N + n) * cm.K + sl];
      } else {  // one line per lane
        xv[v] = cm.MX[(m * cm.K + sl) * N + n];
        cv[v] = cm.MC[(m * cm.K + sl) * N + n];
      }
    }
    const size_t ms = (size_t)(c0 + j0 + min(lane, nb - 1)) * N + n;
    const float av = cm.MA[ms], bv = cm.MB[ms];
    const int cntv = cm.MN[ms], ovfv = cm.OVF[ms];
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      for (int h = 0; h < CPV; ++h) {
        const int b = v * CPV + h;
        if (b >= nb) break;
        const int cnt = __builtin_amdgcn_readlane(cntv, b);
        const int k = __popcll(__ballot(row == h && slot < cnt && xv[v] > u));
        float nu = k == cnt ? __fadd_rn(__fmul_rn(lane_f(av, b), u), lane_f(bv, b))
                            : lane_f(cv[v], h * RW + min(k, RW - 1));
        if (__builtin_amdgcn_readlane(ovfv, b) != 0)
          nu = wave_serial_rows(I, N, n, (c0 + j0 + b) * cm.C, cm.C, u, beta, theta, u_r);
        u = nu;
      }
    }
  }
  return u;
}

// RW lanes a super map (RW = 32 for K2 <= 32: two maps a register and windows of 64 maps;
// RW = 64 for K2 <= 64: one map a register and windows of 32).
template <int RW>
__global__ __launch_bounds__(64) void k_map_carry_wave(
    const float* __restrict__ I, const float* __restrict__ u0, const float* __restrict__ MA,
    const float* __restrict__ MB, const int* __restrict__ MN, const int* __restrict__ OVF,
    const float* __restrict__ MX, const float* __restrict__ MC, float* __restrict__ starts,
    int64_t N, int M, int K, int64_t L, float beta, float theta, float u_r, ChunkMaps cm) {
  static_assert(RW == 32 || RW == 64, "a super map takes a half or a whole wave");
  constexpr int SPR = WAVE / RW;  // super maps a register
  constexpr int WS = 32 * SPR;    // super maps a window
  if (M <= 0) return;
  const int64_t n = xcd_neuron(blockIdx.x, N);
  const int lane = threadIdx.x;
  const int half = lane / RW, slot = lane % RW;
  const int sl = min(slot, K - 1);
  auto load = [&](int w, SuperWindow& d) {
    const size_t o = (size_t)min(w * WS + lane, M - 1) * N + n;
    d.a = MA[o];
    d.b = MB[o];
    d.cnt = MN[o];
    d.ovf = OVF[o];
#pragma unroll
    for (int g = 0; g < 32; ++g) {
      const size_t os = ((size_t)min(w * WS + SPR * g + half, M - 1) * K + sl) * N + n;
      d.xd[g] = MX[os];
      d.cd[g] = MC[os];
    }
  };
  float u = u0[n];
  const int NW = (M + WS - 1) / WS;
  SuperWindow cur, nxt;
  load(0, cur);
  for (int w = 0; w < NW; ++w) {
    load(min(w + 1, NW - 1), nxt);
    const int nc = min(WS, M - w * WS);
    float st_o = 0.0f;
#pragma unroll
    for (int g = 0; g < 32; ++g) {
      for (int h = 0; h < SPR; ++h) {
        const int c = SPR * g + h;
        if (c >= nc) break;
        const int cnt = __builtin_amdgcn_readlane(cur.cnt, c);
        const int k = __popcll(__ballot(half == h && slot < cnt && cur.xd[g] > u));
        float nu = k == cnt ? __fadd_rn(__fmul_rn(lane_f(cur.a, c), u), lane_f(cur.b, c))
                            : lane_f(cur.cd[g], RW * h + min(k, RW - 1));
        if (lane == c) st_o = u;
        if (cm.walk != kSuperAsStored && __builtin_amdgcn_readlane(cur.ovf, c) != 0) {
          // fallback through the map
          const int64_t sm = (int64_t)w * WS + c;
          if (!cm.walk)
            nu = wave_serial_rows(I, N, n, sm * L, L, u, beta, theta, u_r);
          else if (cm.K <= 16)
            nu = wave_walk_chunk_maps<16>(I, cm, N, n, sm, u, beta, theta, u_r);
          else
            nu = wave_walk_chunk_maps<32>(I, cm, N, n, sm, u, beta, theta, u_r);
        }
        u = nu;
      }
    }
    if (lane < nc) starts[(size_t)(w * WS + lane) * N + n] = st_o;
    cur = nxt;
  }
}

// done (converged calls only; else null): as the v3 lane carries, a wave whose chunk
// overflows in any lane replays that chunk for all its lanes from their starts, writing U, S
// and the end, and flags the (chunk, 64-neuron block) for the replay to skip; every later
// chunk of the group then starts from the exact state of the group's start.
template <int KMAX>
__global__ __launch_bounds__(64) void k_lif_carry_inner(
    const float* __restrict__ I, const float* __restrict__ sstarts, const float* __restrict__ MA,
    const float* __restrict__ MB, const int* __restrict__ MN, const int* __restrict__ OVF,
    const float* __restrict__ MX, const float* __restrict__ MC, float* __restrict__ starts,
    int64_t N, int NB, int G, int C, int K, float beta, float theta, float u_r,
    float* __restrict__ U, float* __restrict__ S, float* __restrict__ ends,
    int* __restrict__ done) {
  const int64_t s = blockIdx.x / NB;
  const int nb = (int)(blockIdx.x - s * NB);
  const int64_t n = (int64_t)nb * WAVE + threadIdx.x;
  if (n >= N) return;
  float u = sstarts[(size_t)s * N + n];
  for (int jj = 0; jj < G; ++jj) {
    const int64_t m = s * G + jj;
    const size_t o = (size_t)m * N + n;
    starts[o] = u;
    float xd[KMAX], cd[KMAX];
#pragma unroll
    for (int i = 0; i < KMAX; ++i) {
      xd[i] = i < K ? MX[((size_t)m * K + i) * N + n] : INFINITY;
      cd[i] = i < K ? MC[((size_t)m * K + i) * N + n] : 0.0f;
    }
    float nu = eval_slots<KMAX>(xd, cd, MN[o], MA[o], MB[o], u);
    const bool ovf = OVF[o] != 0;
    if (done) {
      const bool fb = __ballot(ovf) != 0ull;
      if (fb) {
        float w = u;
        const size_t base = (size_t)m * C * N + n;
        stream_rows<32>(I + base, (size_t)N, C, [&](int64_t j, float x) {
          bool sp;
          w = lif_step(w, x, beta, theta, u_r, sp);
          st_nt(U + base + (size_t)j * N, w);
          st_nt(S + base + (size_t)j * N, sp ? 1.0f : 0.0f);
        });
        ends[o] = w;
        nu = w;
      }
      if (threadIdx.x == 0) done[(size_t)m * NB + nb] = fb ? 1 : 0;
    } else if (ovf) {
      nu = serial_rows(I, N, n, m * C, C, u, beta, theta, u_r);
    }
    u = nu;
  }
}

// ---------------------------------------------------------------------------------------
// entry point plumbing (the build, replay and repair kernels live in lif_kernels.hip)
int lif_build_t_launch(const float* I, const float* u0, char* ws, const lsh_v3_layout& L,
                       int64_t N, int M, int C, int K, float beta, float theta, float u_r,
                       hipStream_t st, float* XT, float* CT);
int lif_build_launch(const float* I, const float* u0, char* ws, const lsh_v3_layout& L, int64_t N,
                     int M, int C, int K, float beta, float theta, float u_r, hipStream_t st);
void lif_replay_repair_done_launch(const float* I, float* U, float* S, float* starts, float* ends,
                                   int* list0, int* list1, WsHeader* hdr, int64_t N, int M, int C,
                                   int64_t repair, float beta, float theta, float u_r,
                                   hipStream_t st, const int* done);
void lif_replay_repair_launch(const float* I, const float* u0, float* U, float* S, float* starts,
                              float* ends, int* list0, int* list1, WsHeader* hdr, int64_t N, int M,
                              int C, int64_t repair, float beta, float theta, float u_r,
                              hipStream_t st);

static int kcap(int k) { return k <= 4 ? 4 : k <= 8 ? 8 : k <= 16 ? 16 : k <= 32 ? 32 : 64; }

// Most neurons for the one-wave-per-neuron envelope walk, composition and super-map carry.
#ifndef LSH_V4_WAVE_MAX_N
#define LSH_V4_WAVE_MAX_N 2048
#endif

template <int KMAX, int K2MAX>
static void launch_compose(char* w, const lsh_v4_layout& L, const float* u0, int64_t N, int M2,
                           int G, int K, int K2, float theta, float u_r, hipStream_t st) {
  const int NB = (int)((N + WAVE - 1) / WAVE);
  auto F = [&](size_t off) { return reinterpret_cast<float*>(w + off); };
  auto Iq = [&](size_t off) { return reinterpret_cast<int*>(w + off); };
  if (N <= LSH_V4_WAVE_MAX_N && K2 <= 64 && (int64_t)M2 * NB <= 256) {
    // few neurons and few super maps (the lane kernel would leave three quarters of the SIMDs
    // idle): one wave per neuron and SPW super maps, about 2048 waves in all
    const int SPW = (int)std::max<int64_t>(1, ((int64_t)M2 * N + 2047) / 2048);
    const int64_t nblk = N * (((int64_t)M2 + SPW - 1) / SPW);
    hipLaunchKernelGGL(k_lif_compose_wave, dim3((unsigned)nblk), dim3(WAVE), 0, st, F(L.v3.MA),
                       F(L.v3.MB), Iq(L.v3.MN), Iq(L.v3.OVF), F(L.v3.MX), F(L.v3.MC), F(L.v3.LO),
                       u0, F(L.SA), F(L.SB), Iq(L.SN), Iq(L.SOVF), F(L.SX), F(L.SC),
                       reinterpret_cast<WsHeader*>(w), N, M2, SPW, G, K, K2, theta, u_r);
    return;
  }
  hipLaunchKernelGGL((k_lif_compose<KMAX, K2MAX>), dim3((unsigned)((int64_t)M2 * NB)), dim3(WAVE), 0,
                     st, F(L.v3.MA), F(L.v3.MB), Iq(L.v3.MN), Iq(L.v3.OVF), F(L.v3.MX), F(L.v3.MC),
                     F(L.v3.LO), u0, F(L.SA), F(L.SB), Iq(L.SN), Iq(L.SOVF), F(L.SX), F(L.SC),
                     reinterpret_cast<WsHeader*>(w), N, NB, G, K, K2, theta, u_r);
}

template <int KMAX>
static int launch_compose_k2(char* w, const lsh_v4_layout& L, const float* u0, int64_t N, int M2,
                             int G, int K, int K2, float theta, float u_r, hipStream_t st) {
  switch (kcap(K2)) {
    case 4: if (KMAX <= 4) { launch_compose<KMAX, 4>(w, L, u0, N, M2, G, K, K2, theta, u_r, st); return LSH_OK; } break;
    case 8: if (KMAX <= 8) { launch_compose<KMAX, 8>(w, L, u0, N, M2, G, K, K2, theta, u_r, st); return LSH_OK; } break;
    case 16: if (KMAX <= 16) { launch_compose<KMAX, 16>(w, L, u0, N, M2, G, K, K2, theta, u_r, st); return LSH_OK; } break;
    case 32: if (KMAX <= 32) { launch_compose<KMAX, 32>(w, L, u0, N, M2, G, K, K2, theta, u_r, st); return LSH_OK; } break;
    default: launch_compose<KMAX, 64>(w, L, u0, N, M2, G, K, K2, theta, u_r, st); return LSH_OK;
  }
  return LSH_ERR_SHAPE;
}

template <int KMAX>
static void launch_chunk_kernels(const float* I, const float* u0, char* w, const lsh_v4_layout& L,
                                 int64_t N, int M, int G, int C, int K, float beta, float theta,
                                 float u_r, hipStream_t st) {
  const int NB = (int)((N + WAVE - 1) / WAVE);
  auto F = [&](size_t off) { return reinterpret_cast<float*>(w + off); };
  auto Iq = [&](size_t off) { return reinterpret_cast<int*>(w + off); };
  if (N <= LSH_V4_WAVE_MAX_N)
    hipLaunchKernelGGL(k_lif_env_lo_wave, dim3((unsigned)N), dim3(WAVE), 0, st, u0, F(L.v3.EC),
                       F(L.v3.EA), F(L.v3.EB), F(L.v3.LO), N, M);
  else
    hipLaunchKernelGGL((k_lif_env_lo<16>), dim3((unsigned)NB), dim3(WAVE), 0, st, u0, F(L.v3.EC),
                       F(L.v3.EA), F(L.v3.EB), F(L.v3.LO), N, M);
  // ~8192 blocks in all: enough to fill the chip, few header atomics
  const int MB = (int)std::max<int64_t>(1, std::min<int64_t>(M, 8192 / NB));
  hipLaunchKernelGGL((k_lif_trunc<KMAX>), dim3((unsigned)((int64_t)MB * NB)), dim3(WAVE), 0, st,
                     F(L.v3.LO), Iq(L.v3.CNT), Iq(L.v3.OVFRAW), F(L.v3.MX), Iq(L.v3.MN), Iq(L.v3.OVF),
                     reinterpret_cast<WsHeader*>(w), N, NB, M, MB, K);
}

// done: converged calls only (see k_lif_carry_inner), else null.
template <int KMAX>
static void launch_inner(const float* I, char* w, const lsh_v4_layout& L, int64_t N, int M2, int G,
                         int C, int K, float beta, float theta, float u_r, hipStream_t st,
                         float* U, float* S, int* done) {
  const int NB = (int)((N + WAVE - 1) / WAVE);
  auto F = [&](size_t off) { return reinterpret_cast<float*>(w + off); };
  auto Iq = [&](size_t off) { return reinterpret_cast<int*>(w + off); };
  hipLaunchKernelGGL((k_lif_carry_inner<KMAX>), dim3((unsigned)((int64_t)M2 * NB)), dim3(WAVE), 0, st,
                     I, F(L.SSTARTS), F(L.v3.MA), F(L.v3.MB), Iq(L.v3.MN), Iq(L.v3.OVF), F(L.v3.MX),
                     F(L.v3.MC), F(L.v3.STARTS), N, NB, G, C, K, beta, theta, u_r, U, S,
                     F(L.v3.ENDS), done);
}

template <int K2MAX, int KW>
static void launch_super_carry_lanes(const float* I, const float* u0, char* w, const lsh_v4_layout& L,
                                     int64_t N, int M2, int K2, int64_t Lsteps, float beta,
                                     float theta, float u_r, const ChunkMaps& cm, hipStream_t st) {
  const int NB = (int)((N + WAVE - 1) / WAVE);
  auto F = [&](size_t off) { return reinterpret_cast<float*>(w + off); };
  auto Iq = [&](size_t off) { return reinterpret_cast<int*>(w + off); };
  hipLaunchKernelGGL((k_map_carry<K2MAX, KW>), dim3((unsigned)NB), dim3(WAVE), 0, st, I, u0, F(L.SA),
                     F(L.SB), Iq(L.SN), Iq(L.SOVF), F(L.SX), F(L.SC), F(L.SSTARTS), N, M2, K2,
                     Lsteps, beta, theta, u_r, cm);
}

// walk != 0: an overflowed super map walks its G chunk maps; else its C*G steps run serially
// (the reference's rule, triton_lif.py:958-963).
template <int K2MAX>
static void launch_super_carry(const float* I, const float* u0, char* w, const lsh_v4_layout& L,
                               int64_t N, int M2, int K2, int G, int C, int K, int walk,
                               float beta, float theta, float u_r, hipStream_t st) {
  auto F = [&](size_t off) { return reinterpret_cast<float*>(w + off); };
  auto Iq = [&](size_t off) { return reinterpret_cast<int*>(w + off); };
  const bool xt = L.XT != L.CT;  // the transposed slots exist (a wave per neuron)
  const ChunkMaps cm{F(L.v3.MA), F(L.v3.MB), Iq(L.v3.MN), Iq(L.v3.OVF), F(L.v3.MX), F(L.v3.MC),
                     K, G, C, walk, xt ? F(L.XT) : nullptr, xt ? F(L.CT) : nullptr};
  const int64_t Lsteps = (int64_t)C * G;
  if (K2 <= 64 && N <= LSH_V4_WAVE_MAX_N) {
    auto kern = K2 <= 32 ? k_map_carry_wave<32> : k_map_carry_wave<64>;
    hipLaunchKernelGGL(kern, dim3((unsigned)N), dim3(WAVE), 0, st, I, u0, F(L.SA), F(L.SB),
                       Iq(L.SN), Iq(L.SOVF), F(L.SX), F(L.SC), F(L.SSTARTS), N, M2, K2, Lsteps,
                       beta, theta, u_r, cm);
    return;
  }
  // the chunk maps' slot capacity (K <= K2)
  if (K <= 4)
    launch_super_carry_lanes<K2MAX, 4>(I, u0, w, L, N, M2, K2, Lsteps, beta, theta, u_r, cm, st);
  else if (K <= 8 || K2MAX <= 4)
    launch_super_carry_lanes<K2MAX, (K2MAX < 8 ? K2MAX : 8)>(I, u0, w, L, N, M2, K2, Lsteps, beta,
                                                             theta, u_r, cm, st);
  else if (K <= 16 || K2MAX <= 8)
    launch_super_carry_lanes<K2MAX, (K2MAX < 16 ? K2MAX : 16)>(I, u0, w, L, N, M2, K2, Lsteps, beta,
                                                               theta, u_r, cm, st);
  else
    launch_super_carry_lanes<K2MAX, (K2MAX < 32 ? K2MAX : 32)>(I, u0, w, L, N, M2, K2, Lsteps, beta,
                                                               theta, u_r, cm, st);
}

void v3_layout_fill(int64_t T, int64_t N, int C, int K, lsh_v3_layout* L);

static int v4_check(int64_t T, int64_t N, int C, int G, int K, int K2) {
  if (T < 0 || N < 0 || N > (int64_t)1 << 31) return LSH_ERR_SHAPE;
  if (C < 1 || G < 1 || K < 1 || K > 32 || K2 < 1 || K2 > 64 || K > K2) return LSH_ERR_SHAPE;
  if (T % C != 0 || (T / C) % G != 0) return LSH_ERR_DIVISIBILITY;
  if ((T / C) * ((N + WAVE - 1) / WAVE) > ((int64_t)1 << 31) - 1) return LSH_ERR_SHAPE;
  return LSH_OK;
}

static void v4_layout(int64_t T, int64_t N, int C, int G, int K, int K2, lsh_v4_layout* L) {
  v3_layout_fill(T, N, C, K, &L->v3);
  const int64_t M2 = (T / C) / G;
  const size_t sn = (size_t)M2 * (size_t)N * 4;
  Carver c;
  c.off = L->v3.total;
  L->SA = c.take(sn);
  L->SB = c.take(sn);
  L->SN = c.take(sn);
  L->SOVF = c.take(sn);
  L->SX = c.take(sn * (size_t)K2);
  L->SC = c.take(sn * (size_t)K2);
  L->SSTARTS = c.take(sn);
  // the chunk maps' slots transposed, for the one-wave super carry's walk over an overflowed
  // super map's chunk maps (a chunk's slots then share cache lines instead of one line each)
  const size_t xt = N <= LSH_V4_WAVE_MAX_N ? (size_t)(T / C) * (size_t)N * (size_t)K * 4 : 0;
  L->XT = c.take(xt);
  L->CT = c.take(xt);
  L->total = c.off;
}

}  // namespace lsh

using namespace lsh;

extern "C" int lsh_lif_scan_v4_layout(int64_t T, int64_t N, int C, int G, int K, int K2,
                                      lsh_v4_layout* out) {
  if (bad_ptr(out)) return LSH_ERR_ARG;
  const int rc = v4_check(T, N, C, G, K, K2);
  if (rc != LSH_OK) return rc;
  v4_layout(T, N, C, G, K, K2, out);
  return LSH_OK;
}

extern "C" size_t lsh_lif_scan_v4_workspace(int64_t T, int64_t N, int C, int G, int K, int K2) {
  if (v4_check(T, N, C, G, K, K2) != LSH_OK) return 0;
  lsh_v4_layout L;
  v4_layout(T, N, C, G, K, K2, &L);
  return L.total;
}

extern "C" int lsh_lif_scan_v4_fwd(const float* I, const float* u0, float* U, float* S, int64_t T,
                                   int64_t N, float beta, float theta, float u_r, int C, int G,
                                   int K, int K2, int super_walk, int64_t repair, void* ws,
                                   size_t ws_bytes, void* stream) {
  if (bad_ptr(I) || bad_ptr(u0) || bad_ptr(U) || bad_ptr(S) || bad_ptr(ws)) return LSH_ERR_ARG;
  if (repair < -1 || super_walk < 0 || super_walk > kSuperAsStored) return LSH_ERR_ARG;
  if (super_walk == kSuperAsStored && repair != -1) return LSH_ERR_ARG;
  const int walk = super_walk;
  const int rc = v4_check(T, N, C, G, K, K2);
  if (rc != LSH_OK) return rc;
  lsh_v4_layout L;
  v4_layout(T, N, C, G, K, K2, &L);
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
  const int M2 = M / G;
  const bool xt = walk == 1 && L.XT != L.CT;  // transposed slots for the one-wave walk
  int r = lif_build_t_launch(I, u0, w, L.v3, N, M, C, K, beta, theta, u_r, st,
                             xt ? reinterpret_cast<float*>(w + L.XT) : nullptr,
                             xt ? reinterpret_cast<float*>(w + L.CT) : nullptr);
  if (r != LSH_OK) return r;
  switch (kcap(K)) {
    case 4:
      launch_chunk_kernels<4>(I, u0, w, L, N, M, G, C, K, beta, theta, u_r, st);
      r = launch_compose_k2<4>(w, L, u0, N, M2, G, K, K2, theta, u_r, st);
      break;
    case 8:
      launch_chunk_kernels<8>(I, u0, w, L, N, M, G, C, K, beta, theta, u_r, st);
      r = launch_compose_k2<8>(w, L, u0, N, M2, G, K, K2, theta, u_r, st);
      break;
    case 16:
      launch_chunk_kernels<16>(I, u0, w, L, N, M, G, C, K, beta, theta, u_r, st);
      r = launch_compose_k2<16>(w, L, u0, N, M2, G, K, K2, theta, u_r, st);
      break;
    default:
      launch_chunk_kernels<32>(I, u0, w, L, N, M, G, C, K, beta, theta, u_r, st);
      r = launch_compose_k2<32>(w, L, u0, N, M2, G, K, K2, theta, u_r, st);
      break;
  }
  if (r != LSH_OK) return r;
  switch (kcap(K2)) {
    case 4: launch_super_carry<4>(I, u0, w, L, N, M2, K2, G, C, K, walk, beta, theta, u_r, st); break;
    case 8: launch_super_carry<8>(I, u0, w, L, N, M2, K2, G, C, K, walk, beta, theta, u_r, st); break;
    case 16: launch_super_carry<16>(I, u0, w, L, N, M2, K2, G, C, K, walk, beta, theta, u_r, st); break;
    case 32: launch_super_carry<32>(I, u0, w, L, N, M2, K2, G, C, K, walk, beta, theta, u_r, st); break;
    default: launch_super_carry<64>(I, u0, w, L, N, M2, K2, G, C, K, walk, beta, theta, u_r, st); break;
  }
  // converged without statistics (repair -1): exact fallbacks in the inner carry, the block
  // flags in the second repair list (the Jacobi rounds refill their lists from scratch)
  int* done = repair < 0 ? reinterpret_cast<int*>(w + L.v3.LIST1) : nullptr;
  switch (kcap(K)) {
    case 4: launch_inner<4>(I, w, L, N, M2, G, C, K, beta, theta, u_r, st, U, S, done); break;
    case 8: launch_inner<8>(I, w, L, N, M2, G, C, K, beta, theta, u_r, st, U, S, done); break;
    case 16: launch_inner<16>(I, w, L, N, M2, G, C, K, beta, theta, u_r, st, U, S, done); break;
    default: launch_inner<32>(I, w, L, N, M2, G, C, K, beta, theta, u_r, st, U, S, done); break;
  }
  lif_replay_repair_done_launch(I, U, S, reinterpret_cast<float*>(w + L.v3.STARTS),
                                reinterpret_cast<float*>(w + L.v3.ENDS),
                                reinterpret_cast<int*>(w + L.v3.LIST0),
                                reinterpret_cast<int*>(w + L.v3.LIST1), h, N, M, C, repair, beta,
                                theta, u_r, st, done);
  LSH_CHECK_LAUNCH();
  return LSH_OK;
}
