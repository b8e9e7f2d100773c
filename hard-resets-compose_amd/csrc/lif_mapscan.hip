// Associative carry of the two-level exact scan (MI355X, gfx950): the chunk maps of a neuron are
// composed with a parallel prefix instead of being evaluated one after another.
//
// The chunk map of the hard-reset LIF over C steps (triton_lif.py:737-779, fast.py:86-91) is
//   M(u) = A*u + B             if u < xd[n-1] (or n == 0)
//          cd[k]               k = #{i < n : xd[i] > u}
// and maps compose: H then g is again such a map (triton_lif.py:864-892 compose_group_kernel,
// exact.py:108-131): H's constants pushed through g, g's breakpoints pulled back through H's
// affine part (kept if below H's smallest breakpoint, <= hi, while that one is above the
// domain's lower bound lo), A = Ag*A, B = Ag*B + Bg.  The min-affine envelope maps
// l -> min(c, a*l + b) of every chunk compose too: (c2, a2, b2) after (c1, a1, b1) is
// (min(c2, a2*c1 + b2), a2*a1, a2*b1 + b2) for a2 >= 0 (beta >= 0).
//
// k_map_scan: one workgroup per neuron, one chunk per lane, tiles of 64*WG chunks:
//   1. every lane loads its chunk's envelope map; an inclusive scan inside each wave (DPP:
//      row_shr 1, 2, 4, 8 within 16-lane rows, then row_bcast:15 into rows 1 and 3 and
//      row_bcast:31 into rows 2 and 3) and the wave totals in LDS give every chunk's entry
//      bound LO = l - 1e-5(|l| + 1) (triton_lif.py:723-733);
//   2. every lane truncates its hi-pruned chunk map at LO (k_lif_build's single-read build;
//      capacity overflow if all K stored breakpoints are above LO);
//   3. the same DPP scan composes the truncated maps, segmented at overflowed chunks (an
//      overflowed chunk starts a segment whose map is applied to that chunk's exit); wave 0
//      composes the wave totals the same way.  A map's breakpoint/constant slots live in LDS
//      (one region per lane, two buffers; breakpoints and constants in separate arrays, so a
//      wave's access to one slot of 64 regions is 64 consecutive 4-byte words, one per bank:
//      the float2 slots of an earlier layout stalled 47 % of the LDS cycles on bank
//      conflicts, this one 1 %), so DPP moves only a map's scalars and the address of its
//      slots, and a composition reads the other map's slots from LDS with binary searches
//      over the descending breakpoints;
//   4. chunk starts: without overflowed chunks in the tile, every lane evaluates its prefix map
//      at the tile's entry state at once; otherwise the overflowed chunks are run serially in
//      order (C steps of the recurrence from their start) and each segment is evaluated after
//      its head.  A composition that exceeds the slot capacity sends the tile to a sequential
//      evaluation of its chunk maps (the carry of k_lif_carry).
// The starts are predictions (rounding of the composed affine parts may differ from the chunk by
// chunk evaluation); the replay and the device repair of the two-level scan (lif_kernels.hip)
// then make U and S the serial recurrence bit for bit.
#include "lsh_abi.h"
#include "lsh_common.h"

namespace lsh {

constexpr int MS_KS = 32;  // breakpoint capacity of a composed map
constexpr int MS_WG = 4;   // most waves per workgroup (chunks per tile = 64 * WG); the slot
                           // buffers take 2 x WG x 64 lanes x KS x 8 B = 128 KB of LDS

// A scanned element: a map over a run of chunks and the domain's lower bound; its slots
// (breakpoint, constant) are (px, pc)[base + i*stride], i < n, breakpoints descending.
//   HEAD: the run contains an overflowed chunk; the map takes the exit state of the last one.
//   BAD : a composition in the run exceeded MS_KS breakpoints (the map is incomplete).
constexpr int MS_HEAD = 1, MS_BAD = 2;

struct SMap {
  float A, B, lo;
  int n, flags, base, stride;
};

// #{i < n : px[base + i*stride] > u} for descending breakpoints (binary search).  The
// breakpoints and the constants are separate arrays, so the searches read 4 bytes a lane.
__device__ __forceinline__ int ms_count_gt(const float* px, int base, int stride, int n,
                                           float u) {
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (px[base + mid * stride] > u) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

// Map evaluation (triton_lif.py:592-599): k = #{xd > u}; k == n -> A*u + B, else cd[k].
__device__ __forceinline__ float ms_eval(const float* px, const float* pc, const SMap& f, float u) {
  const int k = ms_count_gt(px, f.base, f.stride, f.n, u);
  return k == f.n ? __fadd_rn(__fmul_rn(f.A, u), f.B) : pc[f.base + k * f.stride];
}

// g <- g after H (H first), the result's slots written at (ob, os), unless g already starts
// at an overflowed chunk (then g is kept).  Returns whether it composed.  Counting g's
// breakpoints with compares over registers instead of the binary searches was slower on
// MI355X (cfg4, C 2048: 1.21 against 0.87 ms): the searches' LDS waits are not what the kernel
// waits on.
__device__ __forceinline__ bool ms_compose(float* px, float* pc, const SMap& H, SMap& g, int ob,
                                           int os, float hi) {
  if (g.flags & MS_HEAD) return false;
  // (1) H's breakpoints, with H's constants pushed through g
  float xmin = INFINITY;
  for (int i = 0; i < H.n; ++i) {
    const float hx = px[H.base + i * H.stride], hc = pc[H.base + i * H.stride];
    const int c = ms_count_gt(px, g.base, g.stride, g.n, hc);
    const float v = c == g.n ? __fadd_rn(__fmul_rn(g.A, hc), g.B) : pc[g.base + c * g.stride];
    px[ob + i * os] = hx;
    pc[ob + i * os] = v;
    xmin = hx;
  }
  // (2) g's breakpoints pulled back through H's affine part (kept below H's smallest
  // breakpoint, <= hi, while that one is above the domain's lower bound)
  int rn = H.n;
  int flags = H.flags | (g.flags & MS_BAD);
  for (int j = 0; j < g.n; ++j) {
    const float gx = px[g.base + j * g.stride];
    const float num = __fsub_rn(gx, H.B);
    const float z = H.A == 0.0f ? (num > 0.0f ? INFINITY : -INFINITY) : num / H.A;
    if ((z < xmin) && (z <= hi) && (xmin > H.lo)) {
      if (rn >= MS_KS) {
        flags |= MS_BAD;
      } else {
        px[ob + rn * os] = z;
        pc[ob + rn * os] = pc[g.base + j * g.stride];
        ++rn;
        xmin = z;
      }
    }
  }
  const float A = __fmul_rn(g.A, H.A);
  const float B = __fadd_rn(__fmul_rn(g.A, H.B), g.B);
  g = SMap{A, B, H.lo, rn, flags, ob, os};
  return true;
}

// One level of the wave scan: the element of the DPP source lane (CTRL, row mask RM) composed
// before this lane's.  (ob0, ob1) are this lane's two slot regions (stride os); `cur` tells
// which one holds its element.
template <int CTRL, int RM>
__device__ __forceinline__ void ms_level(float* px, float* pc, SMap& f, bool active, int& cur,
                                         int ob0, int ob1, int os, float hi) {
  auto mvf = [](float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, RM, 0xF, false));
  };
  auto mvi = [](int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, RM, 0xF, false); };
  const SMap H{mvf(f.A), mvf(f.B), mvf(f.lo), mvi(f.n), mvi(f.flags), mvi(f.base), mvi(f.stride)};
  const int got = mvi(1);
  const int ob = cur == 0 ? ob1 : ob0;
  if (got && active && ms_compose(px, pc, H, f, ob, os, hi)) cur ^= 1;
  // the next level reads what this one wrote (one wave: LDS accesses complete in order)
  __builtin_amdgcn_wave_barrier();
}

// Inclusive scan of a wave's elements in lane order, segmented at heads.
__device__ __forceinline__ void ms_wave_scan(float* px, float* pc, SMap& f, bool active, int& cur,
                                             int ob0, int ob1, int os, float hi) {
  __builtin_amdgcn_wave_barrier();
  ms_level<0x111, 0xF>(px, pc, f, active, cur, ob0, ob1, os, hi);  // row_shr:1
  ms_level<0x112, 0xF>(px, pc, f, active, cur, ob0, ob1, os, hi);  // row_shr:2
  ms_level<0x114, 0xF>(px, pc, f, active, cur, ob0, ob1, os, hi);  // row_shr:4
  ms_level<0x118, 0xF>(px, pc, f, active, cur, ob0, ob1, os, hi);  // row_shr:8
  ms_level<0x142, 0xA>(px, pc, f, active, cur, ob0, ob1, os, hi);  // row_bcast:15 -> rows 1, 3
  ms_level<0x143, 0xC>(px, pc, f, active, cur, ob0, ob1, os, hi);  // row_bcast:31 -> rows 2, 3
}

// Envelope maps l -> min(c, a*l + b): (c, a, b) after (c1, a1, b1).
struct Env {
  float c, a, b;
};
__device__ __forceinline__ Env env_after(const Env& e1, const Env& e2) {
  return {fminf(e2.c, __fadd_rn(__fmul_rn(e2.a, e1.c), e2.b)), __fmul_rn(e2.a, e1.a),
          __fadd_rn(__fmul_rn(e2.a, e1.b), e2.b)};
}
__device__ __forceinline__ float env_apply(const Env& e, float l) {
  return fminf(e.c, __fadd_rn(__fmul_rn(e.a, l), e.b));
}
template <int CTRL, int RM>
__device__ __forceinline__ void env_level(Env& e) {
  auto mv = [](float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, RM, 0xF, false));
  };
  const Env h = {mv(e.c), mv(e.a), mv(e.b)};
  if (__builtin_amdgcn_update_dpp(0, 1, CTRL, RM, 0xF, false)) e = env_after(h, e);
}
__device__ __forceinline__ void env_wave_scan(Env& e) {
  env_level<0x111, 0xF>(e);
  env_level<0x112, 0xF>(e);
  env_level<0x114, 0xF>(e);
  env_level<0x118, 0xF>(e);
  env_level<0x142, 0xA>(e);
  env_level<0x143, 0xC>(e);
}

// Exit of chunk m from u by C serial steps (the overflow fallback; same step as the replay).
__device__ __forceinline__ float ms_serial(const float* __restrict__ I, int64_t N, int64_t n,
                                           int64_t m, int C, float u, float beta, float theta,
                                           float u_r) {
  stream_rows<16>(I + (size_t)m * C * N + n, (size_t)N, C, [&](int64_t, float x) {
    bool s;
    u = lif_step(u, x, beta, theta, u_r, s);
  });
  return u;
}

__device__ __forceinline__ int wave_or_flags(int f) {
  return (__ballot(f & MS_HEAD) ? MS_HEAD : 0) | (__ballot(f & MS_BAD) ? MS_BAD : 0);
}

// LDS layout (one float per slot, breakpoints in px and constants in pc at the same index):
// the in-wave slot regions [buf][wave][slot][lane], then the totals scan's regions
// [buf][slot][lane] for lanes 0..MS_WG-2 of wave 0.
constexpr int MS_POOL_WAVE = 2 * MS_WG * MS_KS * WAVE;
constexpr int MS_POOL = MS_POOL_WAVE + 2 * MS_KS * MS_WG;

__global__ __launch_bounds__(WAVE* MS_WG) void k_map_scan(
    const float* __restrict__ I, const float* __restrict__ u0, const float* __restrict__ EC,
    const float* __restrict__ EA, const float* __restrict__ EB, const float* __restrict__ MA,
    const float* __restrict__ MB, const int* __restrict__ CNT, const int* __restrict__ OVFRAW,
    const float* __restrict__ MX, const float* __restrict__ MC, float* __restrict__ LO,
    int* __restrict__ MN, int* __restrict__ OVF, float* __restrict__ starts, WsHeader* hdr,
    int64_t N, int M, int C, int K, float beta, float theta, float u_r) {
  __shared__ float px[MS_POOL], pc[MS_POOL];
  __shared__ SMap sTot[MS_WG];  // wave totals, then the exclusive prefixes of the waves
  __shared__ Env sEnv[MS_WG];
  __shared__ float sLo[MS_WG * WAVE];
  __shared__ float sAfter[MS_WG * WAVE];
  __shared__ float sState, sEnvIn;  // the tile's entry state and entry envelope
  __shared__ int sFlags;
  const int WG = blockDim.x / WAVE;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const int lane = threadIdx.x % WAVE;
  // neurons spread over the XCDs in contiguous ranges (workgroups go round-robin over the 8
  // XCDs), so neighbours that share cache lines of the maps run on the same L2: the grid has
  // 8 * per workgroups and workgroup b takes neuron (b % 8) * per + b / 8, which covers
  // 0 .. 8 * per - 1 once each
  const int64_t per = gridDim.x / 8;
  const int64_t b = blockIdx.x;
  const int64_t n = (b % 8) * per + b / 8;
  if (n >= N) return;  // the whole workgroup: no barrier is skipped by a part of it
  const float hi = fmaxf(u0[n], fmaxf(theta, u_r));
  const float margin = 1e-5f;
  // this lane's two slot regions
  const int ob0 = (0 * MS_WG + w) * MS_KS * WAVE + lane;
  const int ob1 = (1 * MS_WG + w) * MS_KS * WAVE + lane;
  if (threadIdx.x == 0) {
    sState = u0[n];
    sEnvIn = u0[n];
  }
  unsigned long long ovf_acc = 0, pcs_acc = 0;
  int pmax = 0;
  const int tile = WAVE * WG;
  for (int m0 = 0; m0 < M; m0 += tile) {
    __syncthreads();  // the previous tile's exit state and envelope are in LDS
    const int64_t m = (int64_t)m0 + threadIdx.x;
    const bool valid = m < M;
    const size_t o = (size_t)(valid ? m : 0) * N + n;
    // 1. envelope bounds of the chunk entries
    Env e = valid ? Env{EC[o], EA[o], EB[o]} : Env{INFINITY, 1.0f, 0.0f};
    env_wave_scan(e);
    if (lane == WAVE - 1) sEnv[w] = e;
    if (threadIdx.x == 0) sFlags = 0;
    __syncthreads();
    float lw = sEnvIn;
    for (int v = 0; v < w; ++v) lw = env_apply(sEnv[v], lw);
    const float l_exit = env_apply(e, lw);
    const float l_prev = __shfl_up(l_exit, 1, WAVE);
    const float l_in = lane == 0 ? lw : l_prev;
    const float lo = l_in - margin * (fabsf(l_in) + 1.0f);
    sLo[threadIdx.x] = lo;
    // 2. the chunk's map truncated at its entry bound (capacity overflow: a head), into this
    //    lane's region 0
    int ne = 0;
    bool ovf = false;
    SMap f{1.0f, 0.0f, lo, 0, 0, ob0, WAVE};
    int cur = 0;
    if (valid) {
      const int cnt = CNT[o];
      const size_t os = (size_t)(valid ? m : 0) * K * N + n;
      // every slot's loads issued before the first is used (K is the same on every lane; the
      // slots past the count are loaded too, so no load waits for it), then the count's prefix
      // goes to LDS
      float xs[MS_KS], cs[MS_KS];
#pragma unroll
      for (int i = 0; i < MS_KS; ++i) {
        if (i < K) {
          xs[i] = MX[os + (size_t)i * N];
          cs[i] = MC[os + (size_t)i * N];
        }
      }
      int gt = 0;
#pragma unroll
      for (int i = 0; i < MS_KS; ++i) {
        if (i < K && i < cnt) {
          px[ob0 + i * WAVE] = xs[i];
          pc[ob0 + i * WAVE] = cs[i];
          gt += xs[i] > lo ? 1 : 0;
        }
      }
      ne = min(cnt, gt + 1);
      ovf = OVFRAW[o] != 0 && gt == cnt;
      if (ovf) {  // a head: the identity applied to the chunk's (serial) exit
        f.flags = MS_HEAD;
        f.lo = -INFINITY;
      } else {
        f.A = MA[o];
        f.B = MB[o];
        f.n = ne;
      }
      LO[o] = lo;
      MN[o] = ne;
      OVF[o] = ovf ? 1 : 0;
      ovf_acc += ovf ? 1ull : 0ull;
      pcs_acc += (unsigned long long)ne;
      pmax = max(pmax, ne);
    }
    // 3. inclusive segmented scan inside the wave; wave totals to LDS
    ms_wave_scan(px, pc, f, true, cur, ob0, ob1, WAVE, hi);
    if (lane == WAVE - 1) sTot[w] = f;
    const int fl = wave_or_flags(f.flags);
    if (lane == 0 && fl) atomicOr(&sFlags, fl);
    __syncthreads();
    // exclusive prefixes of the waves: wave 0 scans the totals of waves 0..WG-2 (lane j holds
    // waves 0..j afterwards, its slots in the totals regions) and stores it as wave j+1's prefix
    if (w == 0 && WG > 1) {
      const bool act = lane < WG - 1;
      SMap t = act ? sTot[lane] : SMap{1.0f, 0.0f, -INFINITY, 0, 0, 0, 1};
      int tcur = 1;  // the first composition writes region 0
      const int tb0 = MS_POOL_WAVE + lane;
      const int tb1 = MS_POOL_WAVE + MS_KS * MS_WG + lane;
      ms_wave_scan(px, pc, t, act, tcur, tb0, tb1, MS_WG, hi);
      const int tf = wave_or_flags(act ? t.flags : 0);
      if (lane == 0 && tf) atomicOr(&sFlags, tf);
      if (act) sTot[lane + 1] = t;  // all reads of sTot above came first (one wave, in order)
    }
    __syncthreads();
    const int tflags = sFlags;
    const float s_in = sState;
    if (threadIdx.x == 0 && tflags != 0)  // tiles that leave the parallel evaluation (statistics)
      atomicAdd((tflags & MS_BAD) ? &hdr->fused_unknown : &hdr->fused_fixups, 1ull);
    if (tflags == 0) {
      // 4a. no overflowed chunk, every composition complete: all chunks at once
      const float s_w = (w == 0) ? s_in : ms_eval(px, pc, sTot[w], s_in);
      sAfter[threadIdx.x] = valid ? ms_eval(px, pc, f, s_w) : 0.0f;
    } else if ((tflags & MS_BAD) == 0) {
      // 4b. overflowed chunks (heads): waves in order, the heads of each wave in order; a head
      // runs its chunk serially from the exit of the chunk before it
      for (int v = 0; v < WG; ++v) {
        if (w == v) {
          const float s_w = (v == 0) ? s_in : sAfter[v * WAVE - 1];
          unsigned long long hm = __ballot(valid && ovf);
          float after = (f.flags & MS_HEAD) ? 0.0f : ms_eval(px, pc, f, s_w);
          while (hm) {
            const int h = __builtin_ctzll(hm);
            hm &= hm - 1;
            const float sh = h == 0 ? s_w : __shfl(after, h - 1, WAVE);
            float xh = 0.0f;
            if (lane == h) xh = ms_serial(I, N, n, m, C, sh, beta, theta, u_r);
            xh = __shfl(xh, h, WAVE);
            const int h2 = hm ? __builtin_ctzll(hm) : WAVE;
            if (lane >= h && lane < h2) after = ms_eval(px, pc, f, xh);
          }
          sAfter[threadIdx.x] = valid ? after : 0.0f;
        }
        __syncthreads();
      }
    } else if (threadIdx.x == 0) {
      // 4c. a composition exceeded the capacity: the tile's chunk maps one after another
      float u = s_in;
      const int mend = min(M, m0 + tile);
      for (int mm = m0; mm < mend; ++mm) {
        const size_t oo = (size_t)mm * N + n;
        const float lo2 = sLo[mm - m0];
        const int cnt = CNT[oo];
        int gt = 0;
        for (int i = 0; i < cnt && i < K; ++i) gt += MX[((size_t)mm * K + i) * N + n] > lo2 ? 1 : 0;
        const int ne2 = min(cnt, gt + 1);
        if (OVFRAW[oo] != 0 && gt == cnt) {
          u = ms_serial(I, N, n, mm, C, u, beta, theta, u_r);
        } else {
          int k = 0;
          for (int i = 0; i < ne2; ++i) k += MX[((size_t)mm * K + i) * N + n] > u ? 1 : 0;
          u = k == ne2 ? __fadd_rn(__fmul_rn(MA[oo], u), MB[oo]) : MC[((size_t)mm * K + k) * N + n];
        }
        sAfter[mm - m0] = u;
      }
    }
    __syncthreads();
    // chunk starts: the exit of the chunk before (the tile's entry state for its first chunk)
    if (valid) starts[o] = threadIdx.x == 0 ? s_in : sAfter[threadIdx.x - 1];
    const int last = min(M - m0, tile) - 1;
    if (threadIdx.x == last) {
      sState = sAfter[last];
      sEnvIn = l_exit;  // the exit bound of the tile's last chunk
    }
  }
  // statistics of the truncation (as k_lif_carry): one atomic per wave
  ovf_acc = wave_sum_u64(ovf_acc);
  pcs_acc = wave_sum_u64(pcs_acc);
  pmax = wave_max_i(pmax);
  if (lane == 0) {
    if (ovf_acc) atomicAdd(&hdr->ovf_count, ovf_acc);
    if (pcs_acc) atomicAdd(&hdr->pieces_sum, pcs_acc);
    atomicMax(&hdr->pieces_max, (unsigned int)pmax);
  }
}
int lif_build_launch(const float* I, const float* u0, char* ws, const lsh_v3_layout& L, int64_t N,
                     int M, int C, int K, float beta, float theta, float u_r, hipStream_t st);
void lif_replay_repair_launch(const float* I, const float* u0, float* U, float* S, float* starts,
                              float* ends, int* list0, int* list1, WsHeader* hdr, int64_t N, int M,
                              int C, int64_t repair, float beta, float theta, float u_r,
                              hipStream_t st);
void v3_layout_fill(int64_t T, int64_t N, int C, int K, lsh_v3_layout* L);

static void launch_map_scan(const float* I, const float* u0, char* w, const lsh_v3_layout& L,
                            int64_t N, int M, int C, int K, float beta, float theta, float u_r,
                            hipStream_t st) {
  auto F = [&](size_t off) { return reinterpret_cast<float*>(w + off); };
  auto Iq = [&](size_t off) { return reinterpret_cast<int*>(w + off); };
  const int WG = M >= 64 * MS_WG ? MS_WG : (M + WAVE - 1) / WAVE;
  hipLaunchKernelGGL(k_map_scan, dim3((unsigned)(8 * ((N + 7) / 8))), dim3(WAVE * WG), 0, st, I, u0, F(L.EC),
                     F(L.EA), F(L.EB), F(L.MA), F(L.MB), Iq(L.CNT), Iq(L.OVFRAW), F(L.MX), F(L.MC),
                     F(L.LO), Iq(L.MN), Iq(L.OVF), F(L.STARTS), reinterpret_cast<WsHeader*>(w), N,
                     M, C, K, beta, theta, u_r);
}

static int assoc_check(int64_t T, int64_t N, int C, int K, float beta) {
  if (T < 0 || N < 0 || N > ((int64_t)1 << 31) - 8 || C < 1 || K < 1 || K > 32) return LSH_ERR_SHAPE;
  if (!(beta >= 0.0f)) return LSH_ERR_ARG;  // the envelope monoid needs a >= 0
  if (T % C != 0) return LSH_ERR_DIVISIBILITY;
  if (T / C > ((int64_t)1 << 31) - 1) return LSH_ERR_SHAPE;
  return LSH_OK;
}

}  // namespace lsh

using namespace lsh;

extern "C" size_t lsh_lif_scan_v3_assoc_workspace(int64_t T, int64_t N, int C, int K) {
  if (assoc_check(T, N, C, K, 0.0f) != LSH_OK) return 0;
  lsh_v3_layout L;
  v3_layout_fill(T, N, C, K, &L);
  return L.total;
}

extern "C" int lsh_lif_scan_v3_assoc_fwd(const float* I, const float* u0, float* U, float* S,
                                         int64_t T, int64_t N, float beta, float theta, float u_r,
                                         int C, int K, int64_t repair, void* ws, size_t ws_bytes,
                                         void* stream) {
  if (bad_ptr(I) || bad_ptr(u0) || bad_ptr(U) || bad_ptr(S) || bad_ptr(ws)) return LSH_ERR_ARG;
  if (repair < -1) return LSH_ERR_ARG;
  const int rc = assoc_check(T, N, C, K, beta);
  if (rc != LSH_OK) return rc;
  lsh_v3_layout L;
  v3_layout_fill(T, N, C, K, &L);
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
  int r = lif_build_launch(I, u0, w, L, N, M, C, K, beta, theta, u_r, st);
  if (r != LSH_OK) return r;
  launch_map_scan(I, u0, w, L, N, M, C, K, beta, theta, u_r, st);
  lif_replay_repair_launch(I, u0, U, S, reinterpret_cast<float*>(w + L.STARTS),
                           reinterpret_cast<float*>(w + L.ENDS), reinterpret_cast<int*>(w + L.LIST0),
                           reinterpret_cast<int*>(w + L.LIST1), h, N, M, C, repair, beta, theta, u_r,
                           st);
  LSH_CHECK_LAUNCH();
  return LSH_OK;
}
