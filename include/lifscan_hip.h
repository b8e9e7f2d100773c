/*
 * lifscan_hip.h — C ABI of the MI355X (gfx950) exact hard-reset LIF / ALIF scan library
 * (liblifscan_hip.so).
 *
 * Conventions (every entry point):
 *   - All arrays are device pointers to fp32 (or int32 where stated), time-major [T, N]
 *     with element (t, n) at t*N + n, neurons contiguous.  Per-chunk arrays are [M, N]
 *     and per-chunk map slots [M, K, N] with M = T / C.
 *   - `stream` is a hipStream_t passed as void* (NULL = the default stream).  Kernels are
 *     launched asynchronously on it; no entry point synchronizes unless stated.
 *   - The library never allocates or frees device memory.  Scan entry points take a
 *     caller-provided workspace whose size is given by the matching *_workspace() query.
 *   - Return value: LSH_OK (0) or a negative LSH_ERR_* code; nothing is launched when an
 *     argument check fails.
 *   - Scalars beta, theta, u_r, alpha, rho, q, theta0 are fp32 (the reference passes
 *     Python floats, which its kernels use as fp32).
 *   - Step arithmetic: v = fl(fl(beta*u) + x), two IEEE round-to-nearest operations, no
 *     FMA contraction; spikes s = v >= theta; u' = s ? u_r : v.
 */
#ifndef LIFSCAN_HIP_H
#define LIFSCAN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LSH_ABI_VERSION 4

#define LSH_OK 0
#define LSH_ERR_ARG (-1)          /* null pointer or bad scalar argument */
#define LSH_ERR_SHAPE (-2)        /* T, N, C, K, G out of the supported range */
#define LSH_ERR_DIVISIBILITY (-3) /* T % C != 0 (or M % G != 0) */
#define LSH_ERR_WORKSPACE (-4)    /* workspace too small or misaligned */
#define LSH_ERR_HIP (-5)          /* HIP launch / runtime error */
#define LSH_ERR_SCRATCH (-6)      /* problem larger than the static scratch array (_noalloc) */

/* Library identity. */
int lsh_abi_version(void);
const char* lsh_arch(void);                /* "gfx950" */
const char* lsh_status_string(int status); /* static string for a status code */

/* The serial sweeps (lsh_lif_serial_fwd/_bwd, lsh_alif_serial_fwd*, lsh_alif_bwd mode 0,
 * lsh_aff_serial_fwd) run one workgroup per 64 neurons: producer waves load a tile of rows one
 * tile ahead, compute every per-step quantity that does not depend on the recurrence into an
 * LDS double buffer and store the outputs, while one consumer wave runs the recurrence itself,
 * with the serial step's operations in the reference's order. */

/* Serial hard-reset LIF forward.
 * Replaces triton_lif.py:460-466 (serial_forward_tiled), :246-251 (serial_forward) and
 * :1221-1225 (serial_forward_auto).  U, S: [T, N] outputs. */
int lsh_lif_serial_fwd(const float* I, const float* u0, float* U, float* S, int64_t T, int64_t N,
                       float beta, float theta, float u_r, void* stream);

/* Serial surrogate-gradient adjoint lam_t = gs_t*sg_t + J_t*(gu_t + beta*lam_{t+1}), lam_T = 0.
 * Replaces triton_lif.py:1130-1135 (serial_backward_tiled_pf), :254-259 (serial_backward),
 * :469-476 (serial_backward_tiled) and :1199-1203 (serial_backward_auto).
 * GU may be NULL (treated as all zeros: LIFTuned.backward, triton_lif.py:678).
 * detach != 0: J = 1 - s; detach == 0: J = 1 - s + (u_r - v)*sg (triton_lif.py:47-49). */
int lsh_lif_serial_bwd(const float* I, const float* u0, const float* U, const float* S,
                       const float* GS, const float* GU, float* Lam, int64_t T, int64_t N,
                       float beta, float theta, float u_r, float alpha, int detach, void* stream);

/* Two-level exact scan forward (envelope bound + capacity-K chunk maps, sequential carry
 * with overflow-to-serial fallback, replay, Jacobi repair on device).
 * Replaces triton_lif.py:782-817 (scan_forward_v3) and :1228-1232 (scan_forward_auto).
 * repair: maximum number of repair rounds (0 = none; the result is bit-identical to the
 * serial recurrence once the rounds converge, at most T/C rounds), or -1: repair to
 * convergence without counting rounds (the same U and S; where N and T/C are large, one
 * ordered pass per 64 neurons replays each chunk whose start differs from its predecessor's
 * exact exit, until it meets the stored trajectory; repair_iters is then not the reference's,
 * so request statistics with a finite budget).  Requires T % C == 0, 1 <= K <= 64, C >= 1. */
size_t lsh_lif_scan_v3_workspace(int64_t T, int64_t N, int C, int K);
int lsh_lif_scan_v3_fwd(const float* I, const float* u0, float* U, float* S, int64_t T, int64_t N,
                        float beta, float theta, float u_r, int C, int K, int64_t repair,
                        void* ws, size_t ws_bytes, void* stream);

/* The converged lsh_lif_scan_v3_fwd (repair to convergence, no statistics) in P pieces of T/P
 * steps: the chunk maps of every piece are built on a side stream (one non-blocking stream per
 * device at the default priority, created on first use and kept), while the caller's stream
 * carries, replays and repairs piece after piece, each from the last row of U of the one before
 * (u0 for the first).  U and S are the serial recurrence, as lsh_lif_scan_v3_fwd's converged
 * result; the memory-bound replays overlap the builds of later pieces.  The path of
 * scan_forward_v3 (triton_lif.py:782-817) for few neurons and long T.  Requires
 * T % (C*P) == 0, 1 <= P <= 64; workspace: P pieces of the v3 layout of (T/P, N, C, K), each
 * 256-byte aligned.  Ordering with the caller's stream is by events; concurrent calls from
 * several host threads on one device share the side stream (correct, serialised builds). */
size_t lsh_lif_scan_v3_pieces_workspace(int64_t T, int64_t N, int C, int K, int P);
int lsh_lif_scan_v3_pieces_fwd(const float* I, const float* u0, float* U, float* S, int64_t T,
                               int64_t N, float beta, float theta, float u_r, int C, int K, int P,
                               void* ws, size_t ws_bytes, void* stream);

/* The two-level map scan of lsh_lif_scan_v3_fwd with an associative carry: after the chunk-map
 * build, the chunk maps of each neuron are composed by a parallel prefix instead of being
 * evaluated one after another: one workgroup per neuron, one chunk per lane, an inclusive scan
 * inside each wave by DPP moves (row_shr 1/2/4/8, row_bcast 15/31) and the wave totals composed
 * in LDS, segmented at capacity-overflowed chunks, which run serially; the envelope bounds of
 * the chunk entries by the same scan over the min-affine envelope maps.  Then the replay and
 * `repair` Jacobi repair rounds (repair >= T/C: U and S are the serial recurrence; -1 as for
 * lsh_lif_scan_v3_fwd).  Replaces
 * the sequential carry of triton_lif.py:782-817 (scan_forward_v3: env_carry_kernel :723-733,
 * carry2_kernel :579-606) by the composition monoid of :864-892 (compose_group_kernel).
 * The starts before repair are predictions whose rounding differs from the sequential carry's,
 * so repair_iters is not the reference's; overflow_frac / mean_pieces / max_pieces are the
 * truncation's, as lsh_lif_scan_v3_fwd's.  Requires beta >= 0, T % C == 0, 1 <= K <= 32.
 * Workspace lsh_lif_scan_v3_assoc_workspace(T, N, C, K) bytes (the v3 layout). */
size_t lsh_lif_scan_v3_assoc_workspace(int64_t T, int64_t N, int C, int K);
int lsh_lif_scan_v3_assoc_fwd(const float* I, const float* u0, float* U, float* S, int64_t T,
                              int64_t N, float beta, float theta, float u_r, int C, int K,
                              int64_t repair, void* ws, size_t ws_bytes, void* stream);

/* The converged lsh_lif_scan_v3_fwd (repair to convergence, no statistics) by warm-started
 * chunks, for few neurons and long T: the entry state of chunk m >= 1 is predicted by W steps
 * of the recurrence over the W rows before the chunk, started from u_r (from u0 when those rows
 * reach row 0: then it is exact), every chunk is replayed from its prediction, and the device
 * repair of the two-level scan replays each chunk whose prediction differs from its
 * predecessor's replayed exit, stopping where the new trajectory meets the stored one, until
 * nothing changes.  U and S are the serial recurrence bit for bit.  The path of scan_forward_v3
 * (triton_lif.py:782-817, repair >= T/C) for few neurons and long T; the prediction is the
 * hard-reset analogue of the reference's ALIF warm predictor (triton_alif.py:75-92, :276-285).
 * Requires T % C == 0, C >= 1, W >= 0.  Workspace lsh_lif_scan_warm_workspace(T, N, C) bytes,
 * 256-byte aligned; its header's fused_fixups counts the predictions that missed. */
size_t lsh_lif_scan_warm_workspace(int64_t T, int64_t N, int C);
int lsh_lif_scan_warm_fwd(const float* I, const float* u0, float* U, float* S, int64_t T,
                          int64_t N, float beta, float theta, float u_r, int C, int W, void* ws,
                          size_t ws_bytes, void* stream);

/* Two-level scan pruned with one caller-given lower bound per neuron (lo[N], e.g. the loose
 * state_bounds of triton_lif.py:238-243) instead of the per-chunk envelope.  Replaces
 * triton_lif.py:262-295 (scan_forward), :479-509 (scan_forward_tiled) and :609-642
 * (scan_forward_v2).  Same workspace and `repair` as lsh_lif_scan_v3_fwd. */
int lsh_lif_scan_lo_fwd(const float* I, const float* u0, const float* lo, float* U, float* S,
                        int64_t T, int64_t N, float beta, float theta, float u_r, int C, int K,
                        int64_t repair, void* ws, size_t ws_bytes, void* stream);

/* Single-pass exact two-level scan forward: the result of lsh_lif_scan_v3_fwd with the repair
 * run to convergence (bit-identical to the serial recurrence), computed in one pass over I.
 * One workgroup per 64 neurons walks the chunks in rounds of 4 (one chunk per wave): chunk
 * maps of capacity K are built from registers into LDS, speculative chunk entries are read
 * off the maps, exact chunk exits are handed on through LDS and the chunk is stored from its
 * exact entry.  Replaces triton_lif.py:782-817 (scan_forward_v3 with repair >= T/C) and
 * :1228-1232.  C in {16, 32, 64, 128}, 1 <= K <= 16, T % C == 0.  Workspace:
 * lsh_lif_scan_exact_workspace() bytes (counters only). */
size_t lsh_lif_scan_exact_workspace(void);
int lsh_lif_scan_exact_fwd(const float* I, const float* u0, float* U, float* S, int64_t T,
                           int64_t N, float beta, float theta, float u_r, int C, int K, void* ws,
                           size_t ws_bytes, void* stream);

/* The same kernel without maps: each chunk waits for the exact exit of the previous one (a
 * serial recurrence tiled over chunks, in-house baseline).  Same constraints as above. */
int lsh_lif_chunked_serial_fwd(const float* I, const float* u0, float* U, float* S, int64_t T,
                               int64_t N, float beta, float theta, float u_r, int C, void* ws,
                               size_t ws_bytes, void* stream);

/* Diagnostics of the last scan run in `ws` (synchronizes `stream`).  Same definitions as
 * the reference's stats dict: triton_lif.py:812-816 (v3), :976-982 (v4),
 * triton_alif.py:351-357 (ALIF, alif = 1), triton_affine.py:195-198 (affine reset,
 * alif = 2). */
typedef struct lsh_scan_stats {
  int64_t repair_iters;
  double overflow_frac;
  double mean_pieces; /* mean(kept breakpoints) + 1 for LIF; mean(x-pieces) for ALIF;
                         mean(pieces) for the affine reset */
  int64_t max_pieces; /* the same maxima */
  double super_overflow_frac;
  double super_mean_pieces;
  int64_t super_max_pieces;
  double miss_frac;  /* ALIF only */
  double mean_lines; /* ALIF only */
  int64_t fused_fixups;  /* single-pass scans: chunk entries whose map prediction missed */
  int64_t fused_unknown; /* single-pass scans: chunk entries the maps could not predict */
  int64_t spin_timeouts; /* bounded waits that gave up; always 0 unless a kernel is broken */
} lsh_scan_stats;
int lsh_scan_stats_read(const void* ws, int64_t chunk_neurons, int64_t super_neurons,
                        int alif, lsh_scan_stats* out, void* stream);

/* Byte offsets of the arrays inside a v3 workspace (for tests and diagnostics). */
typedef struct lsh_v3_layout {
  size_t EC, EA, EB;   /* envelope chunk maps [M,N] */
  size_t MA, MB;       /* affine part of the chunk maps [M,N] */
  size_t CNT, OVFRAW;  /* breakpoints stored / capacity overflow before lower-bound pruning [M,N] int32 */
  size_t MX, MC;       /* breakpoints (descending) and constants [M,K,N] */
  size_t LO;           /* envelope lower bound of every chunk entry [M,N] */
  size_t MN, OVF;      /* breakpoints kept after pruning with LO, final overflow flag [M,N] int32 */
  size_t STARTS, ENDS; /* chunk entry / replayed exit states [M,N] */
  size_t LIST0, LIST1; /* repair work lists */
  size_t total;
} lsh_v3_layout;
int lsh_lif_scan_v3_layout(int64_t T, int64_t N, int C, int K, lsh_v3_layout* out);

/* Three-level exact scan for long sequences: capacity-K chunk maps composed in groups of G
 * into capacity-K2 super maps, carry over the super maps, carry inside every super map in
 * parallel, replay, Jacobi repair on device (`repair` as for lsh_lif_scan_v3_fwd, -1
 * included).  Replaces triton_lif.py:935-983
 * (scan_forward_v4), :829-899 (compose_group_kernel), :903-932 (carry_inner_kernel).
 * super_walk = 0: an overflowed super map runs its C*G steps serially (the reference's carry,
 * triton_lif.py:958-963); 1: it walks its G chunk maps as the inner carry does (an overflowed
 * chunk map runs its C steps serially); 2: it is evaluated as stored, a start that may be wrong
 * (only with repair = -1, else LSH_ERR_ARG).  Each way the repair gives the serial recurrence.
 * Requires T % C == 0, (T / C) % G == 0, 1 <= K <= K2, K <= 32, K2 <= 64. */
typedef struct lsh_v4_layout {
  lsh_v3_layout v3;     /* chunk-level arrays, as for lsh_lif_scan_v3_fwd */
  size_t SA, SB, SN, SOVF; /* super maps [M/G, N] */
  size_t SX, SC;        /* super breakpoints / constants [M/G, K2, N] */
  size_t SSTARTS;       /* super-chunk entry states [M/G, N] */
  size_t XT, CT;        /* chunk breakpoints / constants transposed [M, N, K], written with
                           super_walk = 1 for the one-wave-per-neuron super carry (N <= 2048;
                           empty, XT == CT, above) */
  size_t total;
} lsh_v4_layout;
size_t lsh_lif_scan_v4_workspace(int64_t T, int64_t N, int C, int G, int K, int K2);
int lsh_lif_scan_v4_layout(int64_t T, int64_t N, int C, int G, int K, int K2,
                           lsh_v4_layout* out);
int lsh_lif_scan_v4_fwd(const float* I, const float* u0, float* U, float* S, int64_t T, int64_t N,
                        float beta, float theta, float u_r, int C, int G, int K, int K2,
                        int super_walk, int64_t repair, void* ws, size_t ws_bytes, void* stream);

/* Affine-scan backward: chunk composition of lam_t = a_t*lam_{t+1} + b_t, reverse carry,
 * reverse replay.  Replaces triton_lif.py:512-526 (scan_backward_tiled), :298-312
 * (scan_backward) and :1235-1239 (scan_backward_auto).  GU may be NULL (zeros). */
size_t lsh_lif_scan_bwd_workspace(int64_t T, int64_t N, int C);
int lsh_lif_scan_bwd(const float* I, const float* u0, const float* U, const float* S,
                     const float* GS, const float* GU, float* Lam, int64_t T, int64_t N, float beta,
                     float theta, float u_r, float alpha, int detach, int C, void* ws,
                     size_t ws_bytes, void* stream);

/* Single-pass affine-scan backward: per-step coefficients kept in registers, chunk
 * aggregates composed through LDS, I/U/S/GS read once (20 B per neuron-step).  Same result
 * as lsh_lif_scan_bwd up to fp32 association.  Replaces triton_lif.py:512-526 and :1235-1239.
 * C (internal chunk) in {16, 32, 64}, T % C == 0.  GU may be NULL.  No workspace. */
int lsh_lif_scan_fused_bwd(const float* I, const float* u0, const float* U, const float* S,
                           const float* GS, const float* GU, float* Lam, int64_t T, int64_t N,
                           float beta, float theta, float u_r, float alpha, int detach, int C,
                           void* stream);

/* The autograd pair of LIFTuned / LIFAuto (triton_lif.py:654-683, :1003-1026) without the U
 * tensor, which those layers only keep for their backward: the forward writes S and the exact
 * entry state of every C-step chunk, STARTS[T/C][N] (STARTS[0] = u0), and the adjoint replays
 * each chunk's forward from its entry state in registers while it forms the coefficients, so
 * u_{t-1} and s_t are the forward's bits and Lam is the same as lsh_lif_scan_fused_bwd's with
 * the reset detached and no GU.  HBM traffic: forward 8 B, adjoint 12 B per neuron-step
 * (instead of 12 + 20).  C in {16, 32, 64}, the same C for both, T % C == 0; the forward is the
 * single-pass exact forward without maps.  Its ws is NULL (ws_bytes 0: no counters) or a
 * 256-byte aligned header of lsh_lif_scan_exact_workspace() bytes to which the kernel ADDS its
 * counters without clearing it first (no reset launch precedes the forward): clear it once
 * (any fill kernel) and read it with lsh_scan_stats_read whenever convenient; a non-zero
 * spin_timeouts means a chunk hand-off gave up and the S/STARTS of that call are not valid.
 * partials: NULL, or [ceil(N/64)] rows of 3 doubles as lsh_lif_param_bwd mode 2 (sum of
 * lam_t*u_{t-1}, gs_t*sg_t, s_t*lam_{t+1}). */
int lsh_lif_scan_exact_fwd_starts(const float* I, const float* u0, float* STARTS, float* S,
                                  int64_t T, int64_t N, float beta, float theta, float u_r, int C,
                                  void* ws, size_t ws_bytes, void* stream);
int lsh_lif_scan_fused_bwd_starts(const float* I, const float* STARTS, const float* GS, float* Lam,
                                  double* partials, int64_t T, int64_t N, float beta, float theta,
                                  float u_r, float alpha, int C, void* stream);

/* ---------------------------------------------------------------------------------------
 * ALIF: v = fl(fl(beta*u) + x); s = v >= fl(theta0 + w); u' = s ? u_r : v;
 *       w' = s ? fl(fl(rho*w) + q) : fl(rho*w)          (triton_alif.py:26-31)
 * U, W, S: [T, N] outputs. */

/* Serial ALIF forward.  Replaces triton_alif.py:263-273 (alif_serial_forward, plain and tiled). */
int lsh_alif_serial_fwd(const float* I, const float* u0, const float* w0, float* U, float* W,
                        float* S, int64_t T, int64_t N, float beta, float rho, float q,
                        float theta0, float u_r, void* stream);
/* The same forward with params = device pointer to [beta, rho, q, theta0] (fp32), for callers
 * whose parameters are device tensors (triton_alif.py:530 reads them with float(), a device-to-
 * host copy before every launch); U, W, S are bit-identical to lsh_alif_serial_fwd with those
 * values. */
int lsh_alif_serial_fwd_dparams(const float* I, const float* u0, const float* w0, float* U,
                                float* W, float* S, int64_t T, int64_t N, const float* params,
                                float u_r, void* stream);

/* Predicted chunk-entry adaptation WP[T/C, N]: chunk m simulates chunks max(m-Wn, 0)..m-1 from
 * (u_init, w_init), from (UI, WI)[max(m-Wn,0)] when both are given, or from (u0, w0) when the
 * warm-up reaches t = 0.  Replaces triton_alif.py:75-92, :276-285 (alif_warm_predict). */
int lsh_alif_warm_predict(const float* I, const float* u0, const float* w0, const float* UI,
                          const float* WI, float* WP, int64_t T, int64_t N, int C, int Wn,
                          float u_init, float w_init, float beta, float rho, float q,
                          float theta0, float u_r, void* stream);

/* Exact ALIF box scan: entry box [lu, hu) x [lw, hw] per chunk around the prediction Wpred
 * [T/C, N] (Wpred[0] is replaced by w0) with half-width dw, chunk maps of K1 first-spike lines
 * and K2 post-spike pieces, verified carry with serial fallback, replay, Jacobi repair on
 * device.  `block` neurons share the per-step decision to split pieces (the reference's
 * Triton BN; 1, 2, 4, 8 or 16).  rhoC = rho^C as fp32 (computed by the caller).  Replaces
 * triton_alif.py:301-358 (alif_scan_forward), :96-186 (build), :214-252 (carry).
 * K1 <= 32, K2 <= 32 and a power of two, T % C == 0.  repair: the maximum number of Jacobi
 * rounds (0 = none; T/C or more converges, stats' repair_iters counts them), or -1: repair to
 * convergence: the chunks whose carried starts are the serial states (those before MSTAR, the
 * first chunk whose start the carry took through a map) are replayed in parallel, and one
 * serial pass per 64 neurons runs from the least MSTAR on: the same U, W, S as converged
 * Jacobi rounds, the serial recurrence; the carry stops once every neuron of a wave is past its
 * MSTAR, so repair_iters is not counted (0) and the other statistics cover the chunks it walked
 * (request statistics with a finite repair budget, as the Python layer does). */
typedef struct lsh_alif_layout {
  size_t EC, EA, EB, LU, HU, LW, HW; /* envelope maps, box [M, N] */
  size_t MA, MB, NL, NP, OVF;        /* per-chunk scalars [M, N] (NL, NP, OVF int32) */
  size_t LS, LC, LX;                 /* first-spike lines [M, N, K1], slots < NL written */
  size_t POWN, PXL, PXR, PU, PA, POF; /* post-spike pieces [M, N, K2] (POWN int32), slots < NP
                                         written */
  size_t SU, SW, EU, EW, MISS;       /* chunk entry / exit states, carry misses [M, N] */
  size_t MSTAR;                      /* [N] int32: first chunk whose start came through a map */
  size_t LIST0, LIST1;               /* repair work lists */
  size_t total;
} lsh_alif_layout;
size_t lsh_alif_scan_workspace(int64_t T, int64_t N, int C, int K1, int K2);
int lsh_alif_scan_layout(int64_t T, int64_t N, int C, int K1, int K2, lsh_alif_layout* out);
int lsh_alif_scan_fwd(const float* I, const float* u0, const float* w0, const float* Wpred,
                      float dw, float* U, float* W, float* S, int64_t T, int64_t N, float beta,
                      float rho, float q, float theta0, float u_r, float rhoC, int C, int K1,
                      int K2, int block, int64_t repair, void* ws, size_t ws_bytes,
                      void* const* phase_events, void* stream);
/* phase_events: NULL or 5 hipEvent_t recorded on `stream` at the start and after the
 * envelope, the entry box + build, the carry and the first replay (the reference's `phases`,
 * triton_alif.py:305-341). */

/* Single-pass affine-scan adjoint for few neurons (replaces triton_lif.py:512-526 like
 * lsh_lif_scan_fused_bwd): workgroups own 256-step segments of 64 neurons and chain them with
 * a decoupled look-back, so every CU is busy even at N = 1024.  C in {16, 32} (steps per wave);
 * T % 256 == 0; workspace lsh_lif_scan_lookback_bwd_workspace(T, N) bytes, 256-byte aligned,
 * one call at a time.  A bounded wait that gave up is counted in the header's spin_timeouts
 * (lsh_scan_stats_read); it must stay 0. */
size_t lsh_lif_scan_lookback_bwd_workspace(int64_t T, int64_t N);
int lsh_lif_scan_lookback_bwd(const float* I, const float* u0, const float* U, const float* S,
                              const float* GS, const float* GU, float* Lam, int64_t T, int64_t N,
                              float beta, float theta, float u_r, float alpha, int detach, int C,
                              void* ws, size_t ws_bytes, void* stream);

/* lsh_lif_scan_lookback_bwd with no workspace argument, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference.  Its workspace is a static device array of
 * LSH_NOALLOC_SCRATCH_BYTES (64 MiB unless the library is built with another value) that every
 * device the library's code object is loaded on holds until the process ends, whether or not the
 * entry point is called; its address is looked up once per device (with that device current) on
 * the first call.
 * Returns LSH_ERR_SCRATCH, launching nothing, when lsh_lif_scan_lookback_bwd_workspace(T, N)
 * exceeds it (about T * N <= 1.4e9 neuron-steps: N = 1024, T = 2^20 fits).  Calls no allocating
 * routine.  Every call on one device shares its array (the call clears what must start at zero):
 * calls that overlap on one device, from several streams or threads, race.  Same outputs as
 * lsh_lif_scan_lookback_bwd, bit for bit. */
#ifndef LSH_NOALLOC_SCRATCH_BYTES
#define LSH_NOALLOC_SCRATCH_BYTES (64u << 20)
#endif
int lsh_lif_scan_lookback_bwd_noalloc(const float* I, const float* u0, const float* U,
                                      const float* S, const float* GS, const float* GU, float* Lam,
                                      int64_t T, int64_t N, float beta, float theta, float u_r,
                                      float alpha, int detach, int C, void* stream);

/* LIF adjoint with the neuron-parameter gradients of fit.py LIFParamFn.backward
 * (fit.py:30-48): Lam as lsh_lif_*_bwd with the reset detached and no GU, plus per block
 * partials[P][3] (fp64) = (sum lam_t*u_{t-1}, sum gs_t*sg_t, sum s_t*lam_{t+1}), whose column
 * sums give dbeta, -dtheta and dL/du_r / beta.  mode 0: serial; 1: chunked scan of chunk C
 * (workspace lsh_lif_scan_bwd_workspace(T, N, C)); 2: single pass, C in {16, 32, 64};
 * 3: look-back (T % 256 == 0, workspace lsh_lif_scan_lookback_bwd_workspace(T, N)).
 * P = lsh_lif_param_partials(T, N, mode, C). */
int64_t lsh_lif_param_partials(int64_t T, int64_t N, int mode, int C);
int lsh_lif_param_bwd(const float* I, const float* u0, const float* U, const float* S,
                      const float* GS, float* Lam, double* partials, int64_t T, int64_t N,
                      float beta, float theta, float u_r, float alpha, int mode, int C, void* ws,
                      size_t ws_bytes, void* stream);

/* ---- affine reset  u <- gamma*v + delta, 0 <= gamma <= 1 (triton_affine.py) -------------
 *   v = fl(fl(beta*u) + x);  s = v >= theta;  u' = s ? fl(fl(gamma*v) + delta) : v
 *                                                                  (triton_affine.py:19-23)
 * gamma outside [0, 1] (or NaN) is LSH_ERR_ARG. */

/* Serial forward.  Replaces triton_affine.py:143-162 (aff_run_kernel, aff_serial_forward). */
int lsh_aff_serial_fwd(const float* I, const float* u0, float* U, float* S, int64_t T,
                       int64_t N, float beta, float theta, float gamma, float delta, void* stream);

/* Exact two-level scan.  Replaces triton_affine.py:165-199 (aff_scan_forward) with its
 * kernels :26-48 (upper envelope), :51-111 (build), :114-140 (carry), :143-155 (replay) and
 * the repair loop :188-194 (run on device; `repair` bounds the rounds as there).
 * r_theta: the lower envelope's reset value gamma*theta + delta as the caller rounds it (the
 * reference computes it in double and passes it as fp32, :171).  C >= 1, T % C == 0,
 * 1 <= K <= 32.  Workspace lsh_aff_scan_workspace(T, N, C, K) bytes, 256-byte aligned; its
 * arrays (for tests and diagnostics) at the offsets of lsh_aff_scan_layout: */
typedef struct lsh_aff_layout {
  size_t EC, EA, EB, HC, HA, HB; /* lower / upper chunk envelope maps [M, N] */
  size_t LO, HI;                 /* envelope bounds at chunk starts [M, N] */
  size_t PIECES;                 /* [M, N, K] float4 (xl, xr, a, c) */
  size_t NP, OVF;                /* int32 [M, N]: pieces kept, overflow flag */
  size_t STARTS, ENDS;           /* chunk start / end states [M, N] */
  size_t LIST0, LIST1;           /* repair work lists */
  size_t total;
} lsh_aff_layout;
size_t lsh_aff_scan_workspace(int64_t T, int64_t N, int C, int K);
int lsh_aff_scan_layout(int64_t T, int64_t N, int C, int K, lsh_aff_layout* out);
int lsh_aff_scan_fwd(const float* I, const float* u0, float* U, float* S, int64_t T, int64_t N,
                     float beta, float theta, float gamma, float delta, float r_theta, int C,
                     int K, int64_t repair, void* ws, size_t ws_bytes, void* stream);

/* Adjoint of LIFAffineFn (triton_affine.py:229-242; the reference solves it with a torch
 * Hillis-Steele scan, :202-211): lam_t = gs_t*sg_t + beta*J_t*lam_{t+1}, J_t = s_t ? gamma : 1
 * (detached spike), Lam = lam = dL/dI, plus per block partials[P][3] (fp64) =
 * (sum lam_t*u_{t-1}, sum s_t*v_t*lam_{t+1}, sum s_t*lam_{t+1}), whose column sums give
 * dbeta, dgamma / beta and ddelta / beta.  mode, C, workspace and P as lsh_lif_param_bwd. */
int lsh_aff_bwd(const float* I, const float* u0, const float* U, const float* S, const float* GS,
                float* Lam, double* partials, int64_t T, int64_t N, float beta, float theta,
                float gamma, float alpha, int mode, int C, void* ws, size_t ws_bytes,
                void* stream);

/* ---- soft reset  u <- v - theta (triton_soft.py) ----------------------------------------
 * The forward is the affine reset with gamma = 1, delta = -theta (lsh_aff_serial_fwd,
 * lsh_aff_scan_fwd with r_theta = 0): fl(fl(1*v) - theta) = fl(v - theta), the reference's
 * rounding (triton_soft.py:106-110), and the soft scan's common-slope maps are the affine maps
 * with every slope equal.
 *
 * Soft-reset adjoint, reset detached: lam_t = b_t + beta*lam_{t+1}, b_t = gS_t*alpha*sg*(1-sg),
 * sg = sigmoid(alpha*(v_t - theta)) in fp32, the recurrence in float64, Lam stored as fp32.
 * Replaces triton_soft.py:214-221 (soft_adjoint_fft: the same float64 recurrence by FFT
 * convolution) and triton_lif.py:1052-1069, :1139-1210 (soft serial adjoints, fp32).
 * V != NULL: v_t = V[t] (soft_adjoint_fft's input); I, u0, U unused and partials must be NULL.
 * V == NULL: v_t = fl(fl(beta*u_{t-1}) + x_t) from I, u0 (t = 0) and U; partials NULL or
 * [lsh_soft_bwd_partials(T, N, C)] doubles, one per block: sum lam_t*u_{t-1} (dbeta,
 * fit.py:115, :149).  C: chunk length, T % C == 0 (C == T: one sweep per neuron, no
 * workspace; otherwise lsh_soft_bwd_workspace(T, N, C) bytes, 256-byte aligned). */
size_t lsh_soft_bwd_workspace(int64_t T, int64_t N, int C);
int64_t lsh_soft_bwd_partials(int64_t T, int64_t N, int C);
int lsh_soft_bwd(const float* I, const float* u0, const float* U, const float* V, const float* GS,
                 float* Lam, double* partials, int64_t T, int64_t N, double beta, float theta,
                 float alpha, int C, void* ws, size_t ws_bytes, void* stream);

/* L[t] = A[t]*L[t+1] + B[t] with L[T] = 0, per column of [T, N] arrays (two roundings per
 * step, rows from the last).  Replaces triton_affine.py:202-211 and fast.py:307-323
 * (reverse_affine_scan; there a Hillis-Steele scan, so the bits differ by reassociation). */
int lsh_reverse_affine_scan(const float* A, const float* B, float* L, int64_t T, int64_t N,
                            void* stream);

/* ALIF adjoint: LW[t] = dL/dw_t, LV[t] = dL/dv_t (= dL/dI_t) for dL/dS = GS.
 * mode 0: fused serial sweep (triton_alif.py:444-487); 1: chunked two-level affine scans of
 * chunk C (triton_alif.py:510-521, needs lsh_alif_bwd_workspace(T, N, C) bytes); 2: single
 * pass, internal chunk C in {16, 32} (no workspace); 3: single pass with look-back across
 * workgroups (T % 128 == 0, lsh_alif_bwd_lookback_workspace(T, N) bytes, C ignored).  Replaces
 * triton_alif.py:490-521 and the reductions of ALIFFn.backward (triton_alif.py:541-554):
 *   LW       may be NULL in modes 0, 2 and 3 (not written);
 *   DW0      NULL or [N]: dL/dw0 = lw_{-1} = rho*LW[0] - sg_0*(g_0 + q*LW[0]);
 *   partials NULL or [lsh_alif_bwd_partials(T, N, mode, C)][4] doubles, one row per workgroup:
 *            sum LV*u_{t-1}, sum LW*w_{t-1}, sum LW*S, sum sg*(g + q*LW) (fp64); their column
 *            sums are dbeta, drho, dq and -dtheta0. */
size_t lsh_alif_bwd_workspace(int64_t T, int64_t N, int C);
/* mode 3: the single pass for few neurons, segments of 128 steps chained across workgroups by
 * decoupled look-back (first lw, then lv); requires T % 128 == 0 and this many workspace bytes.
 * No counterpart in the reference (same recurrences as triton_alif.py:490-521). */
size_t lsh_alif_bwd_lookback_workspace(int64_t T, int64_t N);
int64_t lsh_alif_bwd_partials(int64_t T, int64_t N, int mode, int C);
int lsh_alif_bwd(const float* I, const float* U, const float* W, const float* S, const float* GS,
                 const float* u0, const float* w0, float* LV, float* LW, float* DW0,
                 double* partials, int64_t T, int64_t N, float beta, float rho, float q,
                 float theta0, float alpha, int mode, int C, void* ws, size_t ws_bytes,
                 void* stream);
/* lsh_alif_bwd with params = device pointer to [beta, rho, q, theta0] (fp32), the parameters of
 * ALIFFn.backward (triton_alif.py:543-554) when they stay on the device; outputs bit-identical. */
int lsh_alif_bwd_dparams(const float* I, const float* U, const float* W, const float* S,
                         const float* GS, const float* u0, const float* w0, float* LV, float* LW,
                         float* DW0, double* partials, int64_t T, int64_t N, const float* params,
                         float alpha, int mode, int C, void* ws, size_t ws_bytes, void* stream);
/* The ALIF adjoint of mode 2 (C in {16, 32}) or mode 3 (look-back; ws as for lsh_alif_bwd) above,
 * same outputs bit for bit, reading I and GS, and U, W only at the row before each chunk: u_{t-1},
 * w_{t-1} and s_t inside the chunk are recomputed with the forward step (reset value u_r).  Valid
 * when U, W (and the S they imply) are one serial trajectory from (u0, w0), as
 * lsh_alif_serial_fwd writes them; 8.5 bytes read per neuron-step at 16-step chunks instead of
 * 20.  params: NULL (use beta, rho, q, theta0) or a device pointer to [beta, rho, q, theta0].
 * Replaces the adjoint half of ALIFFn.backward (triton_alif.py:541-554) for its serial forward
 * (triton_alif.py:531-533). */
int lsh_alif_bwd_recompute(const float* I, const float* U, const float* W, const float* GS,
                           const float* u0, const float* w0, float* LV, float* LW, float* DW0,
                           double* partials, int64_t T, int64_t N, const float* params, float beta,
                           float rho, float q, float theta0, float u_r, float alpha, int mode,
                           int C, void* ws, size_t ws_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LIFSCAN_HIP_H */
