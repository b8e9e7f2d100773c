// Affine-reset LIF kernels for MI355X (gfx950).  Reference: lifscan/triton_affine.py.
//
//   v = fl(fl(beta*u) + x);  s = v >= theta;  u' = s ? fl(fl(gamma*v) + delta) : v
//                                                     (triton_affine.py:19-23, 0 <= gamma <= 1)
// gamma = 0, delta = u_r is the hard reset; gamma = 1, delta = -theta the soft reset.
//
// Forward: serial / replay (k_aff_fwd) and the exact two-level scan (triton_affine.py:165-199):
// lower and upper reachable-state envelopes in one pass over the inputs (k_aff_env) and their
// sequential carries (k_aff_env_carry), capacity-K chunk maps of unsorted pieces
// [xl, xr) -> a*u + c (k_aff_build), the verified carry with serial fallback (k_aff_carry), the
// replay, and Jacobi repair on device (k_aff_repair).  The adjoint is the hard-reset adjoint
// with J_t = s_t ? gamma : 1 (lsh_aff_bwd in lif_kernels.hip).
//
// Workspace layout: header, envelope maps and bounds [M, N], pieces [M, N, K] as float4
// (xl, xr, a, c; the 32 lanes of one neuron store 512 contiguous bytes), counts, overflow
// flags, chunk starts / ends [M, N], repair work lists.
#include "lsh_abi.h"
#include "lsh_common.h"

namespace lsh {

// ---------------------------------------------------------------------------------------
// Serial / replay over segments of Ls steps from su (triton_affine.py:143-162).
template <int D>
__global__ __launch_bounds__(64) void k_aff_fwd(const float* __restrict__ I,
                                                const float* __restrict__ su, float* __restrict__ U,
                                                float* __restrict__ S, float* __restrict__ eu,
                                                int64_t N, int64_t Ls, int NB, float beta,
                                                float theta, float gamma, float delta) {
  const int64_t m = blockIdx.x / NB;
  const int nb = (int)(blockIdx.x - m * NB);
  const int64_t n = (int64_t)nb * WAVE + threadIdx.x;
  if (n >= N) return;
  float u = su[m * N + n];
  const size_t base = (size_t)m * (size_t)Ls * (size_t)N + (size_t)n;
  stream_rows<D>(I + base, (size_t)N, Ls, [&](int64_t j, float x) {
    bool s;
    u = aff_step(u, x, beta, theta, gamma, delta, s);
    const size_t o = base + (size_t)j * N;
    st_nt(U + o, u);
    st_nt(S + o, s ? 1.0f : 0.0f);
  });
  if (eu) eu[m * N + n] = u;
}

// ---------------------------------------------------------------------------------------
// Envelopes of the reachable states per chunk, both from one read of the inputs:
//  lower (triton_lif.py:699-719 with u_r = r(theta), as triton_affine.py:171-172):
//    l -> min(r, beta*l + x), composed as min(c, a*l + b);
//  upper (triton_affine.py:26-36): h -> max(theta, gamma*(beta*h + x) + delta), composed as
//    max(c, a*h + b) with a = (gamma*beta)^C.  From c = -inf, gamma = 0 gives 0*(-inf) = NaN,
//    which fmaxf drops (IEEE maxNum), leaving theta.
__global__ __launch_bounds__(64) void k_aff_env(const float* __restrict__ I,
                                                float* __restrict__ EC, float* __restrict__ EA,
                                                float* __restrict__ EB, float* __restrict__ HC,
                                                float* __restrict__ HA, float* __restrict__ HB,
                                                int64_t N, int NB, int C, float beta, float theta,
                                                float gamma, float delta, float r_theta) {
  const int64_t m = blockIdx.x / NB;
  const int nb = (int)(blockIdx.x - m * NB);
  const int64_t n = (int64_t)nb * WAVE + threadIdx.x;
  if (n >= N) return;
  const float gb = gamma * beta;
  float lc = INFINITY, la = 1.0f, lb = 0.0f;
  float hc = -INFINITY, ha = 1.0f, hb = 0.0f;
  stream_rows<16>(I + (size_t)m * C * N + n, (size_t)N, C, [&](int64_t, float x) {
    lc = fminf(r_theta, lif_v(lc, x, beta));
    la = beta * la;
    lb = lif_v(lb, x, beta);
    hc = fmaxf(theta, __fadd_rn(__fmul_rn(gamma, lif_v(hc, x, beta)), delta));
    ha = gb * ha;
    hb = __fadd_rn(__fmul_rn(gamma, lif_v(hb, x, beta)), delta);
  });
  const size_t o = (size_t)m * N + n;
  EC[o] = lc;
  EA[o] = la;
  EB[o] = lb;
  HC[o] = hc;
  HA[o] = ha;
  HB[o] = hb;
}

// Sequential envelope carries (triton_lif.py:723-733, triton_affine.py:39-48), margin 1e-5:
// LO[m] = l - 1e-5(|l| + 1), HI[m] = h + 1e-5(|h| + 1) with l, h the bounds at chunk m's start.
__global__ __launch_bounds__(64) void k_aff_env_carry(
    const float* __restrict__ u0, const float* __restrict__ EC, const float* __restrict__ EA,
    const float* __restrict__ EB, const float* __restrict__ HC, const float* __restrict__ HA,
    const float* __restrict__ HB, float* __restrict__ LO, float* __restrict__ HI, int64_t N, int M) {
  const int64_t n = (int64_t)blockIdx.x * WAVE + threadIdx.x;
  if (n >= N) return;
  const float margin = 1e-5f;
  float l = u0[n], h = l;
  for (int m = 0; m < M; ++m) {
    const size_t o = (size_t)m * N + n;
    LO[o] = l - margin * (fabsf(l) + 1.0f);
    HI[o] = h + margin * (fabsf(h) + 1.0f);
    l = fminf(EC[o], __fadd_rn(__fmul_rn(EA[o], l), EB[o]));
    h = fmaxf(HC[o], __fadd_rn(__fmul_rn(HA[o], h), HB[o]));
  }
}

// ---------------------------------------------------------------------------------------
// Chunk maps (triton_affine.py:51-111).  A workgroup owns 16 neurons of one chunk; 32 lanes
// serve one neuron (two per wave), lane i holding piece slot i.  Inputs are staged through LDS
// in tiles of 64 steps together with ct = (theta - x)/beta, computed once per (neuron, step).
// Per step every piece [xl, xr) with value a*u + c meets the threshold cut z = (ct - c)/a
// (u >= z spikes; a == 0: all or nothing); its left part [xl, min(xr, z)) and its spiking
// right part [z, xr) are kept when they meet [lo, hi].  When every live piece keeps exactly
// one part (the common case) the pieces stay in their slots; otherwise the list is compacted
// in order, left before right: an inclusive prefix sum of the part counts over the neuron's
// 32 lanes (DPP row shifts plus a row broadcast), then every part is written to its slot in
// this wave's LDS row and read back by the slot's lane.  A count above K sets the overflow
// flag and the parts beyond slot K are dropped, as the reference's compaction does.
constexpr int kAffNPW = 16;  // neurons per build workgroup
constexpr int kAffTS = 64;   // steps per staged tile

__global__ __launch_bounds__(WAVE * kAffNPW / 2) void k_aff_build(
    const float* __restrict__ I, const float* __restrict__ LO, const float* __restrict__ HI,
    float4* __restrict__ PC, int* __restrict__ NP, int* __restrict__ OVF, int64_t N, int NBLK,
    int C, int K, float beta, float theta, float gamma, float delta) {
  constexpr int NW = kAffNPW / 2;
  __shared__ float sX[kAffNPW][kAffTS], sCt[kAffNPW][kAffTS];
  __shared__ float4 sSlot[NW][WAVE];
  const int64_t m = blockIdx.x / NBLK;
  const int blk = (int)(blockIdx.x - m * NBLK);
  const int tid = threadIdx.x;
  const int wv = tid / WAVE;
  const int lane = tid % WAVE;
  const int half = lane >> 5;
  const int i = lane & 31;
  const int ln = wv * 2 + half;
  const int64_t n0 = (int64_t)blk * kAffNPW;
  const int64_t n = n0 + ln;
  const bool valid_n = n < N;
  const size_t o = (size_t)m * N + (valid_n ? n : N - 1);
  const float lo = LO[o], hi = HI[o];
  const float gb = gamma * beta;
  float pxl = i == 0 ? -INFINITY : INFINITY, pxr = INFINITY, pa = 1.0f, pc = 0.0f;
  int cnt = 1, ovf = 0;
  float4* slot = sSlot[wv] + (half << 5);
  const float* __restrict__ Im = I + (size_t)m * C * N;
  for (int j0 = 0; j0 < C; j0 += kAffTS) {
    const int ts = min(kAffTS, C - j0);
    for (int e = tid; e < kAffNPW * ts; e += NW * WAVE) {
      const int k = e / kAffNPW, nu = e - k * kAffNPW;
      const int64_t ne = n0 + nu < N ? n0 + nu : N - 1;
      const float x = Im[(size_t)(j0 + k) * N + ne];
      sX[nu][k] = x;
      sCt[nu][k] = (theta - x) / beta;
    }
    __syncthreads();
    for (int k = 0; k < ts; ++k) {
      const float x = sX[ln][k], ct = sCt[ln][k];
      const bool valid = i < cnt;
      const float num = ct - pc;
      const float z = pa == 0.0f ? (num > 0.0f ? INFINITY : -INFINITY) : num / pa;
      const bool full = z <= pxl;
      const bool split = (z > pxl) && (z < pxr) && valid;
      const float vns = lif_v(pc, x, beta);
      const float c_sp = __fadd_rn(__fmul_rn(gamma, vns), delta);
      const float a_sp = gb * pa;
      const float cl = full ? c_sp : vns;
      const float al = full ? a_sp : beta * pa;
      const float xrl = split ? z : pxr;
      const bool vl = valid && (xrl > lo) && (pxl <= hi);
      const bool vr = split && (pxr > lo) && (z <= hi);
      const int nl = vl ? 1 : 0;
      const int nout = nl + (vr ? 1 : 0);
      if (__ballot(valid && nout != 1) == 0ull) {
        // every live piece keeps one part in its slot
        if (valid) {
          if (vl) {
            pxr = xrl;
            pa = al;
            pc = cl;
          } else {
            pxl = z;
            pa = a_sp;
            pc = c_sp;
          }
        }
      } else {
        // inclusive prefix sum over the neuron's 32 slots: row shifts within 16-lane rows,
        // then the last lane of rows 0 / 2 added to rows 1 / 3
        int incl = nout;
        incl += __builtin_amdgcn_update_dpp(0, incl, 0x111, 0xF, 0xF, true);  // row_shr:1
        incl += __builtin_amdgcn_update_dpp(0, incl, 0x112, 0xF, 0xF, true);  // row_shr:2
        incl += __builtin_amdgcn_update_dpp(0, incl, 0x114, 0xF, 0xF, true);  // row_shr:4
        incl += __builtin_amdgcn_update_dpp(0, incl, 0x118, 0xF, 0xF, true);  // row_shr:8
        incl += __builtin_amdgcn_update_dpp(0, incl, 0x142, 0xA, 0xF, false);  // row_bcast:15
        const int p = incl - nout;
        const int ntot = __shfl(incl, 31, 32);
        if (ntot > K) ovf = 1;
        // same-wave LDS accesses complete in order: the scatter lands before the read-back
        if (vl && p < K) slot[p] = make_float4(pxl, xrl, al, cl);
        if (vr && p + nl < K) slot[p + nl] = make_float4(z, pxr, a_sp, c_sp);
        cnt = min(ntot, K);
        const float4 q = slot[i];
        const bool keep = i < cnt;
        pxl = keep ? q.x : INFINITY;
        pxr = keep ? q.y : INFINITY;
        pa = keep ? q.z : 1.0f;
        pc = keep ? q.w : 0.0f;
      }
    }
    __syncthreads();  // the tile's LDS rows are rewritten next
  }
  if (!valid_n) return;
  if (i < K) PC[o * K + i] = make_float4(pxl, pxr, pa, pc);
  if (i == 0) {
    NP[o] = cnt;
    OVF[o] = ovf;
  }
}

// Verified carry (triton_affine.py:114-140), two neurons per wave, lane i = piece slot i: the
// start u must lie in exactly one piece of a map that did not overflow, and the chunk's end
// state is that piece's a*u + c (plus 0.0: the reference sums the hit lanes, so a -0.0 reads
// as +0.0); otherwise the chunk runs serially.  The next chunk's map is loaded before the
// current one is evaluated.
__global__ __launch_bounds__(64) void k_aff_carry(
    const float* __restrict__ I, const float* __restrict__ u0, const float4* __restrict__ PC,
    const int* __restrict__ NP, const int* __restrict__ OVF, float* __restrict__ STARTS,
    WsHeader* hdr, int64_t N, int M, int C, int K, float beta, float theta, float gamma,
    float delta) {
  const int lane = threadIdx.x;
  const int half = lane >> 5;
  const int i = lane & 31;
  const int hb = half << 5;
  const int64_t n = (int64_t)blockIdx.x * 2 + half;
  const bool valid_n = n < N;
  const int64_t nn = valid_n ? n : N - 1;
  const unsigned long long hmask = 0xffffffffull << hb;
  // lanes i >= K read slot K - 1 (never a hit: i >= K >= count)
  const int ks = i < K ? i : K - 1;
  float u = u0[nn];
  unsigned long long ovf_acc = 0, pcs_acc = 0;
  int pmax = 0;
  float4 q = PC[(size_t)nn * K + ks];
  int cnt = NP[nn], ovf = OVF[nn];
  for (int m = 0; m < M; ++m) {
    const size_t o = (size_t)m * N + nn;
    float4 qn = q;
    int cntn = 0, ovfn = 0;
    if (m + 1 < M) {
      const size_t on = o + (size_t)N;
      qn = PC[on * K + ks];
      cntn = NP[on];
      ovfn = OVF[on];
    }
    if (valid_n && i == 0) STARTS[o] = u;
    const bool hit = i < cnt && q.x <= u && u < q.y;
    const unsigned long long hm = (__ballot(hit) & hmask) >> hb;
    const int nh = __builtin_popcountll(hm);
    const int hl = hm ? __builtin_ctzll(hm) : 0;
    const float val = __fadd_rn(__fmul_rn(q.z, u), q.w);
    float nu = __shfl(val, hl, 32) + 0.0f;  // all lanes shuffle
    if (ovf != 0 || nh != 1) {
      float w = u;
      stream_rows<16>(I + (size_t)m * C * N + nn, (size_t)N, C, [&](int64_t, float x) {
        bool s;
        w = aff_step(w, x, beta, theta, gamma, delta, s);
      });
      nu = w;
    }
    if (valid_n && i == 0) {
      ovf_acc += ovf ? 1ull : 0ull;
      pcs_acc += (unsigned long long)cnt;
      pmax = max(pmax, cnt);
    }
    u = nu;
    q = qn;
    cnt = cntn;
    ovf = ovfn;
  }
  ovf_acc = wave_sum_u64(ovf_acc);
  pcs_acc = wave_sum_u64(pcs_acc);
  pmax = wave_max_i(pmax);
  if (lane == 0) {
    atomicAdd(&hdr->ovf_count, ovf_acc);
    atomicAdd(&hdr->pieces_sum, pcs_acc);
    atomicMax(&hdr->pieces_max, (unsigned int)pmax);
  }
}

// Jacobi repair of the chunk starts on device (triton_affine.py:188-194): chunk m (> 0) whose
// start differs from chunk m-1's end is replayed from that end; a changed end queues chunk
// m+1.  One workgroup per 64 neurons with work lists in the workspace; the rounds counted are
// those the reference's loop counts (at most R).
__global__ __launch_bounds__(256) void k_aff_repair(
    const float* __restrict__ I, float* __restrict__ U, float* __restrict__ S,
    float* __restrict__ su, float* __restrict__ eu, int* __restrict__ list0,
    int* __restrict__ list1, WsHeader* hdr, int64_t N, int M, int C, int64_t R, float beta,
    float theta, float gamma, float delta) {
  __shared__ int s_nd, s_nc;
  const int nb = blockIdx.x;
  const int tid = threadIdx.x;
  const size_t cap = (size_t)M * WAVE;
  int* __restrict__ dl = list0 + (size_t)nb * cap;
  int* __restrict__ cl = list1 + (size_t)nb * cap;
  auto differs = [&](int m, int64_t n) {
    return eu[(size_t)(m - 1) * N + n] != su[(size_t)m * N + n];
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
    }
    __syncthreads();
    if (tid == 0) s_nc = 0;
    __syncthreads();
    for (int k = tid; k < nd; k += blockDim.x) {
      const int e = dl[k];
      const int m = e / WAVE;
      const int64_t n = (int64_t)nb * WAVE + (e % WAVE);
      float u = su[(size_t)m * N + n];
      const size_t base = (size_t)m * C * N + n;
      stream_rows<16>(I + base, (size_t)N, C, [&](int64_t j, float x) {
        bool s;
        u = aff_step(u, x, beta, theta, gamma, delta, s);
        U[base + (size_t)j * N] = u;
        S[base + (size_t)j * N] = s ? 1.0f : 0.0f;
      });
      const size_t oe = (size_t)m * N + n;
      if (u != eu[oe]) {
        eu[oe] = u;
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

// Reverse affine recurrence lam_t = a_t*lam_{t+1} + b_t, lam_T = 0, per column
// (triton_affine.py:202-211 reverse_affine_scan, there a Hillis-Steele scan over torch ops):
// one lane per column, rows consumed from the last in tiles of D loaded ahead.
template <int D>
__global__ __launch_bounds__(64) void k_rev_affine(const float* __restrict__ A,
                                                   const float* __restrict__ B,
                                                   float* __restrict__ L, int64_t T, int64_t N) {
  const int64_t n = (int64_t)blockIdx.x * WAVE + threadIdx.x;
  if (n >= N) return;
  float lam = 0.0f;
  const int64_t nt = T / D;
  auto row = [&](int64_t t) { return (size_t)t * (size_t)N + (size_t)n; };
  float a[D], b[D];
  if (nt > 0) {
#pragma unroll
    for (int k = 0; k < D; ++k) {
      a[k] = A[row(T - 1 - k)];
      b[k] = B[row(T - 1 - k)];
    }
  }
  for (int64_t g = 0; g < nt; ++g) {
    float an[D], bn[D];
    const bool more = g + 1 < nt;
    if (more) {
#pragma unroll
      for (int k = 0; k < D; ++k) {
        an[k] = A[row(T - 1 - (g + 1) * D - k)];
        bn[k] = B[row(T - 1 - (g + 1) * D - k)];
      }
    }
#pragma unroll
    for (int k = 0; k < D; ++k) {
      lam = __fadd_rn(__fmul_rn(a[k], lam), b[k]);
      L[row(T - 1 - g * D - k)] = lam;
    }
    if (more) {
#pragma unroll
      for (int k = 0; k < D; ++k) {
        a[k] = an[k];
        b[k] = bn[k];
      }
    }
  }
  for (int64_t t = T - nt * D - 1; t >= 0; --t) {
    lam = __fadd_rn(__fmul_rn(A[row(t)], lam), B[row(t)]);
    L[row(t)] = lam;
  }
}

static void aff_scan_layout(int64_t T, int64_t N, int C, int K, lsh_aff_layout* L) {
  const int64_t M = T / C;
  const size_t mn = (size_t)M * (size_t)N * 4;
  const size_t nb = (size_t)((N + WAVE - 1) / WAVE);
  Carver c;
  L->EC = c.take(mn);
  L->EA = c.take(mn);
  L->EB = c.take(mn);
  L->HC = c.take(mn);
  L->HA = c.take(mn);
  L->HB = c.take(mn);
  L->LO = c.take(mn);
  L->HI = c.take(mn);
  L->PIECES = c.take(mn * 4 * (size_t)K);
  L->NP = c.take(mn);
  L->OVF = c.take(mn);
  L->STARTS = c.take(mn);
  L->ENDS = c.take(mn);
  L->LIST0 = c.take(nb * (size_t)M * WAVE * 4);
  L->LIST1 = c.take(nb * (size_t)M * WAVE * 4);
  L->total = c.off;
}

static int aff_scan_check(int64_t T, int64_t N, int C, int K) {
  if (T < 0 || N < 0 || N > (int64_t)1 << 31) return LSH_ERR_SHAPE;
  if (C < 1 || K < 1 || K > 32) return LSH_ERR_SHAPE;
  if (T % C != 0) return LSH_ERR_DIVISIBILITY;
  const int64_t M = T / C;
  if (M * ((N + kAffNPW - 1) / kAffNPW) > ((int64_t)1 << 31) - 1) return LSH_ERR_SHAPE;
  return LSH_OK;
}

}  // namespace lsh

using namespace lsh;

extern "C" int lsh_aff_serial_fwd(const float* I, const float* u0, float* U, float* S, int64_t T,
                                  int64_t N, float beta, float theta, float gamma, float delta,
                                  void* stream) {
  if (bad_ptr(I) || bad_ptr(u0) || bad_ptr(U) || bad_ptr(S)) return LSH_ERR_ARG;
  if (!(gamma >= 0.0f && gamma <= 1.0f)) return LSH_ERR_ARG;
  if (T < 0 || N < 0 || N > (int64_t)1 << 31) return LSH_ERR_SHAPE;
  if (T == 0 || N == 0) return LSH_OK;
  aff_serial_fwd_pipe(I, u0, U, S, N, T, beta, theta, gamma, delta, (hipStream_t)stream);
  LSH_CHECK_LAUNCH();
  return LSH_OK;
}

extern "C" int lsh_aff_scan_layout(int64_t T, int64_t N, int C, int K, lsh_aff_layout* out) {
  if (bad_ptr(out)) return LSH_ERR_ARG;
  const int rc = aff_scan_check(T, N, C, K);
  if (rc != LSH_OK) return rc;
  aff_scan_layout(T, N, C, K, out);
  return LSH_OK;
}

extern "C" size_t lsh_aff_scan_workspace(int64_t T, int64_t N, int C, int K) {
  if (aff_scan_check(T, N, C, K) != LSH_OK) return 0;
  lsh_aff_layout L;
  aff_scan_layout(T, N, C, K, &L);
  return L.total;
}

extern "C" int lsh_aff_scan_fwd(const float* I, const float* u0, float* U, float* S, int64_t T,
                                int64_t N, float beta, float theta, float gamma, float delta,
                                float r_theta, int C, int K, int64_t repair, void* ws,
                                size_t ws_bytes, void* stream) {
  if (bad_ptr(I) || bad_ptr(u0) || bad_ptr(U) || bad_ptr(S) || bad_ptr(ws)) return LSH_ERR_ARG;
  if (repair < 0 || !(gamma >= 0.0f && gamma <= 1.0f)) return LSH_ERR_ARG;
  const int rc = aff_scan_check(T, N, C, K);
  if (rc != LSH_OK) return rc;
  lsh_aff_layout L;
  aff_scan_layout(T, N, C, K, &L);
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
  const int NBLK = (int)((N + kAffNPW - 1) / kAffNPW);
  auto F = [&](size_t off) { return reinterpret_cast<float*>(w + off); };
  auto Iq = [&](size_t off) { return reinterpret_cast<int*>(w + off); };
  float4* PC = reinterpret_cast<float4*>(w + L.PIECES);
  hipLaunchKernelGGL(k_aff_env, dim3((unsigned)((int64_t)M * NB)), dim3(WAVE), 0, st, I, F(L.EC),
                     F(L.EA), F(L.EB), F(L.HC), F(L.HA), F(L.HB), N, NB, C, beta, theta, gamma,
                     delta, r_theta);
  hipLaunchKernelGGL(k_aff_env_carry, dim3((unsigned)NB), dim3(WAVE), 0, st, u0, F(L.EC), F(L.EA),
                     F(L.EB), F(L.HC), F(L.HA), F(L.HB), F(L.LO), F(L.HI), N, M);
  hipLaunchKernelGGL(k_aff_build, dim3((unsigned)((int64_t)M * NBLK)), dim3(WAVE * kAffNPW / 2), 0,
                     st, I, F(L.LO), F(L.HI), PC, Iq(L.NP), Iq(L.OVF), N, NBLK, C, K, beta, theta,
                     gamma, delta);
  hipLaunchKernelGGL(k_aff_carry, dim3((unsigned)((N + 1) / 2)), dim3(WAVE), 0, st, I, u0, PC,
                     Iq(L.NP), Iq(L.OVF), F(L.STARTS), h, N, M, C, K, beta, theta, gamma, delta);
  hipLaunchKernelGGL((k_aff_fwd<16>), dim3((unsigned)((int64_t)M * NB)), dim3(WAVE), 0, st, I,
                     F(L.STARTS), U, S, F(L.ENDS), N, (int64_t)C, NB, beta, theta, gamma, delta);
  if (repair > 0 && M > 1) {
    const int64_t rounds = repair < (int64_t)M ? repair : (int64_t)M;
    hipLaunchKernelGGL(k_aff_repair, dim3((unsigned)NB), dim3(256), 0, st, I, U, S, F(L.STARTS),
                       F(L.ENDS), Iq(L.LIST0), Iq(L.LIST1), h, N, M, C, rounds, beta, theta, gamma,
                       delta);
  }
  LSH_CHECK_LAUNCH();
  return LSH_OK;
}

extern "C" int lsh_reverse_affine_scan(const float* A, const float* B, float* L, int64_t T,
                                       int64_t N, void* stream) {
  if (bad_ptr(A) || bad_ptr(B) || bad_ptr(L)) return LSH_ERR_ARG;
  if (T < 0 || N < 0 || N > (int64_t)1 << 31) return LSH_ERR_SHAPE;
  if (T == 0 || N == 0) return LSH_OK;
  hipLaunchKernelGGL((k_rev_affine<16>), dim3((unsigned)((N + WAVE - 1) / WAVE)), dim3(WAVE), 0,
                     (hipStream_t)stream, A, B, L, T, N);
  LSH_CHECK_LAUNCH();
  return LSH_OK;
}
