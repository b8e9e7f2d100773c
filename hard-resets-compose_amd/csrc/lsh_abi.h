// Internal glue shared by the HIP translation units: status codes, argument
// checks and the workspace header layout.  The public declarations live in
// include/lifscan_hip.h; this header re-includes it so the definitions are
// checked against the declarations by the compiler.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/lifscan_hip.h"

namespace lsh {

#define LSH_CHECK_LAUNCH()                          \
  do {                                              \
    hipError_t e_ = hipGetLastError();              \
    if (e_ != hipSuccess) return LSH_ERR_HIP;       \
  } while (0)

// Workspace header (first 256 bytes of every scan workspace).  Counters are
// cleared by a kernel at the start of each call, so a caller may capture the
// call in a HIP graph (no memset node).
struct WsHeader {
  unsigned long long ovf_count;        // chunk-neuron pairs whose map overflowed
  unsigned long long pieces_sum;       // sum over chunk-neuron pairs of breakpoints kept
  unsigned int pieces_max;             // max breakpoints kept
  unsigned int repair_iters;           // Jacobi repair rounds performed (max over neurons)
  unsigned long long super_ovf_count;  // three-level scan: super-chunk overflows
  unsigned long long super_pieces_sum;
  unsigned int super_pieces_max;
  unsigned int miss_count_lo;          // ALIF: box misses (low/high words of a u64)
  unsigned int miss_count_hi;
  unsigned int lines_max;
  unsigned long long lines_sum;        // ALIF: first-spike lines kept
  unsigned long long alif_pieces_sum;  // ALIF: post-spike x-pieces kept
  unsigned int alif_pieces_max;
  unsigned int pad0;
  unsigned long long fused_fixups;     // fused scan: speculative chunk entries that missed;
                                       // map scan: tiles with overflowed chunks (run in order)
  unsigned long long fused_unknown;    // fused scan: entries the maps could not predict;
                                       // map scan: tiles whose composition exceeded capacity
  unsigned int spin_timeouts;          // bounded waits that gave up (must stay 0)
  unsigned int epoch;                  // advanced once per call
  unsigned int ticket;                 // look-back scans: next tile in launch order
};
static_assert(sizeof(WsHeader) <= 256, "workspace header must fit in 256 bytes");
constexpr size_t kWsHeaderBytes = 256;

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Carves consecutive 256-byte aligned arrays out of a workspace.
struct Carver {
  size_t off = kWsHeaderBytes;
  size_t take(size_t bytes) {
    size_t o = off;
    off = align_up(off + bytes, 256);
    return o;
  }
};

__global__ void k_ws_header_reset(WsHeader* h);

inline bool bad_ptr(const void* p) { return p == nullptr; }

// Single-pass detached adjoint with parameter sums (lif_fused.hip); partials gets one row of
// 3 doubles per 64-neuron block.  ps 1: the hard reset's fit.py sums; ps 2: the affine
// reset's (u_r carries gamma).  Returns an LSH_* status.
int lif_param_bwd_fused(const float* I, const float* u0, const float* U, const float* S,
                        const float* GS, float* Lam, double* partials, int64_t T, int64_t N,
                        float beta, float theta, float u_r, float alpha, int C, int ps,
                        hipStream_t st);
// The same with the look-back adjoint (lif_lookback.hip); one partials row per (256-step
// segment, 64-neuron block); workspace as lsh_lif_scan_lookback_bwd.
int lif_param_bwd_lookback(const float* I, const float* u0, const float* U, const float* S,
                           const float* GS, float* Lam, double* partials, void* ws,
                           size_t ws_bytes, int64_t T, int64_t N, float beta, float theta,
                           float u_r, float alpha, int ps, hipStream_t st);

// Device repair rounds of the two-level scan (lif_kernels.hip, k_lif_repair) after a replay that
// wrote U, S and ends from starts: at most min(repair, M) rounds; list0/list1 hold
// ceil(N/64)*M*64 ints each.  repair = -1: to convergence without the round count (the ordered
// pass k_lif_repair_ordered where it is faster, else M rounds).
void lif_repair_launch(const float* I, float* U, float* S, float* starts, float* ends, int* list0,
                       int* list1, WsHeader* hdr, int64_t N, int M, int C, int64_t repair,
                       float beta, float theta, float u_r, hipStream_t st);

// Fills n ints with v on the stream (lif_lookback.hip; look-back flags).
void fill_i32_launch(int* p, int64_t n, int v, hipStream_t st);

// Wave-specialised serial sweeps (serial_pipe.hip): the serial entry points' kernels at every
// neuron count; the one-wave serial kernels remain for scan replays and the parameter sums.
void lif_serial_fwd_pipe(const float* I, const float* u0, float* U, float* S, int64_t N, int64_t T,
                         float beta, float theta, float u_r, hipStream_t st);
void aff_serial_fwd_pipe(const float* I, const float* u0, float* U, float* S, int64_t N, int64_t T,
                         float beta, float theta, float gamma, float delta, hipStream_t st);
void lif_serial_bwd_pipe(const float* I, const float* u0, const float* U, const float* S,
                         const float* GS, const float* GU, float* Lam, int64_t N, int64_t T,
                         float beta, float theta, float u_r, float alpha, bool detach,
                         hipStream_t st);

}  // namespace lsh
