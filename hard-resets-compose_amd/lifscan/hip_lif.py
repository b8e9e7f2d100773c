"""Hard-reset LIF on MI355X: serial kernels, exact two/three-level map scans, affine-scan
backward and the autograd layers, with the call signatures of the reference's
``lifscan/triton_lif.py`` so that callers (``shdnet``, ``fit``, experiments) drop in unchanged.

Every op runs hand-written HIP kernels of ``liblifscan_hip.so`` through its C ABI; there is
no CPU or PyTorch fallback.  Layout: I is [T, N] fp32 contiguous (N = batch * neurons),
element (t, n) at t*N + n.

Triton tile keywords of the reference (BN, nw, BNc, nwc, BNr, D, nwr, BNg, nwg, num_warps,
STAGES, CSTAGES) are accepted for signature compatibility and ignored: the HIP kernels pick
their own tiles (one lane per neuron, register-prefetched time tiles).

Numerics: every path uses the same fp32 step v = fl(fl(beta*u) + x) (no FMA), so the
serial kernel, the scan's replay and its fallbacks agree bit for bit, and after repair the
scan equals the serial recurrence exactly.
"""
import math
import os

import torch

from . import _native as _n

BN_DEFAULT = 128

# auto dispatch thresholds (serial vs scan per pass), measured on MI355X (beta = 0.95, N from
# 256 to 65536, T from 1024 to 65536): the scan forward of lif_auto (scan_forward_auto, no
# repair) beats the serial kernel only with <= 1024 neurons and T >= 16384 (e.g. N = 1024,
# T = 65536: 1.03 vs 1.87 ms; N = 4096, T = 65536: 2.45 vs 2.06 ms).  The scan adjoint, one
# layer's fwd + bwd through autograd (beta 0.9, x ~ N(0.15, 0.4^2)), serial fwd + serial bwd
# against serial fwd + scan bwd: below 16384 neurons the serial adjoint wins up to T = 1024
# (N = 1024, T = 1024: 0.108 vs 0.126 ms; N = 8192: 0.117 vs 0.127) and they tie at T = 2048
# (N = 1024: 0.128 vs 0.125; N = 8192: 0.156 vs 0.154), after which the scan wins (N = 1024,
# T = 4096: 0.226 vs 0.131); from 16384 neurons the scan (the single pass) wins from T = 256
# (N = 16384, T = 1024: 0.128 vs 0.110; N = 32768, T = 512: 0.129 vs 0.108).
AUTO_FWD_MAX_N = 1024
AUTO_FWD_MIN_T = 16384
AUTO_BWD_MAX_N = 1 << 31
AUTO_BWD_MIN_T = 2048
AUTO_BWD_WIDE_N = 16384     # from this many neurons the scan adjoint from AUTO_BWD_WIDE_MIN_T
AUTO_BWD_WIDE_MIN_T = 256


# ----------------------------------------------------------------------------- helpers
def _f32(x):
    """Scalar parameter as a Python float (the kernels take fp32)."""
    if torch.is_tensor(x):
        return float(x.detach().item())
    return float(x)


def _f32s(*xs):
    """Several scalar parameters as Python floats with at most one device-to-host transfer
    (each .item() on a GPU tensor is a synchronizing copy)."""
    dev = [i for i, x in enumerate(xs) if torch.is_tensor(x) and x.device.type != "cpu"]
    out = [float(x.detach().item()) if torch.is_tensor(x) and i not in dev else
           (None if i in dev else float(x)) for i, x in enumerate(xs)]
    if len(dev) == 1:
        out[dev[0]] = float(xs[dev[0]].detach().item())
    elif dev:
        vals = torch.stack([xs[i].detach().reshape(()).to(torch.float64) for i in dev]).cpu().tolist()
        for i, v in zip(dev, vals):
            out[i] = float(v)
    return tuple(out)


def _input(I):
    if not torch.is_tensor(I) or I.dim() != 2:
        raise ValueError("I must be a 2-D [T, N] tensor")
    if I.device.type != "cuda":
        raise ValueError("I must be a GPU (HIP) tensor")
    if I.dtype != torch.float32:
        raise ValueError("I must be float32")
    return I.contiguous()


def _vec(v, N, like, name="u0"):
    if not torch.is_tensor(v):
        v = torch.full((N,), float(v), device=like.device, dtype=torch.float32)
    elif (v.dim() == 1 and v.shape[0] == N and v.dtype == torch.float32 and v.device == like.device
          and v.is_contiguous()):
        return v  # already the [N] fp32 vector the kernels read (only its pointer is passed)
    v = v.detach()
    if v.numel() != N:
        raise ValueError(f"{name} must have N={N} elements")
    if v.device != like.device:
        raise ValueError(f"{name} must be on {like.device}")
    return v.reshape(N).to(torch.float32).contiguous()


def _same(t, like, name):
    if t is None:
        return None
    if t.shape != like.shape or t.device != like.device or t.dtype != torch.float32:
        raise ValueError(f"{name} must be float32 {tuple(like.shape)} on {like.device}")
    return t.contiguous()


def _fill_stats(stats, st, v4=False):
    if stats is None:
        return
    stats["repair_iters"] = int(st.repair_iters)
    stats["overflow_frac"] = float(st.overflow_frac)
    stats["mean_pieces"] = float(st.mean_pieces)
    if v4:
        stats["super_overflow_frac"] = float(st.super_overflow_frac)
        stats["super_mean_pieces"] = float(st.super_mean_pieces)
        stats["super_max_pieces"] = int(st.super_max_pieces)
    else:
        stats["max_pieces"] = int(st.max_pieces)


# ----------------------------------------------------------------------------- serial
def serial_forward(I, beta, theta, u_r, u0, BN=BN_DEFAULT):
    """Serial forward (triton_lif.py:246-251) -> (U, S), both [T, N] fp32."""
    I = _input(I)
    T, N = I.shape
    u0 = _vec(u0, N, I)
    U = torch.empty_like(I)
    S = torch.empty_like(I)
    with _n.on_device(I):
        _n.check(_n.lib().lsh_lif_serial_fwd(_n.ptr(I), _n.ptr(u0), _n.ptr(U), _n.ptr(S), T, N,
                                             _f32(beta), _f32(theta), _f32(u_r), _n.stream_of(I)),
                 "lsh_lif_serial_fwd")
    return U, S


def serial_forward_tiled(I, beta, theta, u_r, u0, BN=32, D=4, num_warps=1):
    """Time-tiled serial forward (triton_lif.py:460-466); same kernel as serial_forward."""
    return serial_forward(I, beta, theta, u_r, u0)


def serial_forward_auto(I, beta, theta, u_r, u0):
    """Tuned serial forward (triton_lif.py:1221-1225)."""
    return serial_forward(I, beta, theta, u_r, u0)


def serial_backward(I, u0, U, S, GS, GU, beta, theta, u_r, alpha=4.0, detach=True, BN=BN_DEFAULT):
    """Serial adjoint (triton_lif.py:254-259) -> Lam [T, N] (= dL/dI).  GU may be None (zeros)."""
    I = _input(I)
    T, N = I.shape
    u0 = _vec(u0, N, I)
    U, S, GS = _same(U, I, "U"), _same(S, I, "S"), _same(GS, I, "GS")
    GU = _same(GU, I, "GU")
    Lam = torch.empty_like(I)
    with _n.on_device(I):
        _n.check(_n.lib().lsh_lif_serial_bwd(
            _n.ptr(I), _n.ptr(u0), _n.ptr(U), _n.ptr(S), _n.ptr(GS), _n.ptr(GU), _n.ptr(Lam), T, N,
            _f32(beta), _f32(theta), _f32(u_r), _f32(alpha), int(bool(detach)), _n.stream_of(I)),
            "lsh_lif_serial_bwd")
    return Lam


def serial_backward_tiled(I, u0, U, S, GS, GU, beta, theta, u_r, alpha=4.0, detach=True,
                          BN=32, D=4, num_warps=1):
    """triton_lif.py:469-476; same kernel as serial_backward."""
    return serial_backward(I, u0, U, S, GS, GU, beta, theta, u_r, alpha, detach)


def serial_backward_tiled_pf(I, u0, U, S, GS, GU, beta, theta, u_r, alpha=4.0, detach=True,
                             BN=32, D=4, num_warps=1):
    """Prefetching serial adjoint (triton_lif.py:1130-1135); same kernel as serial_backward."""
    return serial_backward(I, u0, U, S, GS, GU, beta, theta, u_r, alpha, detach)


def serial_backward_auto(I, u0, U, S, GS, GU, beta, theta, u_r, alpha=4.0, detach=True):
    """Tuned serial adjoint (triton_lif.py:1199-1203)."""
    return serial_backward(I, u0, U, S, GS, GU, beta, theta, u_r, alpha, detach)


def serial_bwd_cfg(N):
    """(BN, D, num_warps) table of the reference (triton_lif.py:1184-1189), kept for callers
    that read it; the HIP kernels choose their own tiles."""
    if N <= 8: return 16, 16, 1
    if N <= 64: return 16, 2, 2
    if N <= 16384: return 64, 16, 1
    return 128, 2, 1


def serial_fwd_cfg(N):
    """(BN, D, num_warps) table of the reference (triton_lif.py:1213-1218); see serial_bwd_cfg."""
    if N <= 8: return 16, 32, 1
    if N <= 64: return 16, 4, 1
    if N <= 512: return 128, 16, 1
    return 64, 32, 1


# ----------------------------------------------------------------------------- scan forward
def state_bounds(I, beta, theta, u_r, u0):
    """Loose per-neuron bounds [lo, hi] of every state (triton_lif.py:238-243)."""
    Imin = I.min(0).values.clamp(max=0)
    base = torch.minimum(u0, torch.full_like(u0, u_r)).clamp(max=0)
    lo = base + (Imin / (1 - beta) if beta < 1 else I.clamp(max=0).sum(0))
    hi = torch.maximum(u0, torch.full_like(u0, max(theta, u_r)))
    return lo.contiguous(), hi.contiguous()


class _ScanRun:
    """Holds the workspace of one scan call (maps, starts, ends) for stats and tests."""

    pieces = 1  # lsh_lif_scan_v3_pieces_fwd: the arrays are the first piece's (T = its steps)
    warm = False

    def __init__(self, ws, T, N, C, K):
        self.ws, self.T, self.N, self.C, self.K = ws, T, N, C, K

    def layout(self):
        L = _n.V3Layout()
        _n.check(_n.lib().lsh_lif_scan_v3_layout(self.T, self.N, self.C, self.K,
                                                 _n.ctypes.byref(L)), "lsh_lif_scan_v3_layout")
        return L

    def view(self, name, dtype=torch.float32):
        """[M, N] or [M, K, N] view of one workspace array (MX/MC are [M, K, N])."""
        L = self.layout()
        M = self.T // self.C
        off = getattr(L, name)
        shape = (M, self.K, self.N) if name in ("MX", "MC") else (M, self.N)
        nbytes = 4 * math.prod(shape)
        return self.ws[off:off + nbytes].view(dtype).view(*shape)


_LAST_RUN = None


def last_scan_run():
    """Workspace of the most recent two-level scan on this process (diagnostics/tests)."""
    return _LAST_RUN


def _repair_arg(repair, M, stats):
    """The C entry's repair argument: -1 (to convergence without the round count, the ordered
    pass where it is faster) for a converged repair whose round count nobody reads, else the
    Jacobi round budget."""
    repair = int(repair)
    if repair < 0:
        raise ValueError("repair must be >= 0")
    return -1 if (stats is None and repair >= M and M > 1) else repair


def _scan2(I, beta, theta, u_r, u0, C, K, repair, stats, lo=None):
    global _LAST_RUN
    I = _input(I)
    T, N = I.shape
    u0 = _vec(u0, N, I)
    C, K = int(C), int(K)
    if C < 1 or T % C:
        raise ValueError(f"T={T} must be divisible by the chunk length C={C}")
    if not 1 <= K <= 64:
        raise ValueError("map capacity K must be in [1, 64]")
    repair = _repair_arg(repair, T // C, stats)
    L = _n.lib()
    nbytes = L.lsh_lif_scan_v3_workspace(T, N, C, K)
    if nbytes == 0:
        raise ValueError(f"unsupported scan shape T={T} N={N} C={C} K={K}")
    ws = _n.workspace(nbytes, I.device)
    U = torch.empty_like(I)
    S = torch.empty_like(I)
    with _n.on_device(I):
        st = _n.stream_of(I)
        if lo is None:
            rc = L.lsh_lif_scan_v3_fwd(_n.ptr(I), _n.ptr(u0), _n.ptr(U), _n.ptr(S), T, N,
                                       _f32(beta), _f32(theta), _f32(u_r), C, K, repair,
                                       _n.ptr(ws), nbytes, st)
        else:
            lo = _vec(lo, N, I, "lo")
            rc = L.lsh_lif_scan_lo_fwd(_n.ptr(I), _n.ptr(u0), _n.ptr(lo), _n.ptr(U), _n.ptr(S), T,
                                       N, _f32(beta), _f32(theta), _f32(u_r), C, K, repair,
                                       _n.ptr(ws), nbytes, st)
        _n.check(rc, "two-level scan forward")
    _LAST_RUN = _ScanRun(ws, T, N, C, K)
    if stats is not None:
        _fill_stats(stats, _n.read_stats(ws, (T // C) * N))
    return U, S


def scan_forward_v3(I, beta, theta, u_r, u0, C=64, K=16, BN=32, nw=1, BNc=16, nwc=1, BNr=32, D=8,
                    nwr=1, repair=0, stats=None):
    """Two-level exact scan with per-chunk envelope bounds (triton_lif.py:782-817) -> (U, S).

    Stricter than the reference: T % C != 0 raises ValueError (the reference leaves the tail
    uninitialised).  stats receives repair_iters, overflow_frac, mean_pieces, max_pieces with
    the reference's definitions (mean/max of kept breakpoints + 1).  With the repair budget at
    least T/C (converged) and no stats requested, the result is the serial recurrence and the
    fastest exact path computes it: for up to 8192 neurons and long T the warm-started chunks
    (warm_plan), else the single-pass kernel, or for few neurons and long T the same two-level
    scan with long chunks (long_sequence_C)."""
    I = _input(I)
    out = _converged_fast(I, beta, theta, u_r, u0, C, min(int(K), 16), repair, stats)
    if out is not None:
        return out
    return _scan2(I, beta, theta, u_r, u0, C, K, repair, stats)


def _converged_fast(I, beta, theta, u_r, u0, C, K, repair, stats):
    """(U, S) by the fastest exact path when the call asks for the converged result (repair
    budget >= T/C) and no statistics: the warm-started chunks (warm_plan), else for few neurons
    and long T the two-level scan with long chunks, else the single pass; None when the call
    needs the maps' own pipeline (a finite repair budget, statistics, or K > 16)."""
    T, N = I.shape
    if not (int(C) >= 1 and T % int(C) == 0):
        return None
    if stats is None and int(repair) >= T // int(C) and T > 0 and N > 0:
        plan = warm_plan(T, N, beta)
        if plan is not None:
            return _scan_warm_run(I, beta, theta, u_r, u0, *plan)
    if _fused_fwd_ok(T, C, K, repair, stats):
        long_c = long_sequence_C(T, N)
        if long_c:  # few neurons, long T: the multi-kernel scan with long chunks is faster
            C2, P = long_sequence_plan(T, N)
            if P > 1:
                return _scan2_pieces(I, beta, theta, u_r, u0, C2, LONG_K, P)
            return _scan2(I, beta, theta, u_r, u0, long_c, LONG_K, T // long_c, None)
        return scan_forward_exact(I, beta, theta, u_r, u0, K=K)
    return None


# Converged exact forward for few neurons and long sequences: the single-pass kernel's hand-off
# chain (T dependent steps per 64-neuron block) dominates there, while the two-level scan with
# long chunks and capacity 32 keeps the whole chip busy in its build and replay.  Measured on
# MI355X: N = 1024, T = 2^20: 24.2 ms single pass vs 8.0 ms (C = 4096); N = 256, T = 2^18:
# 5.6 vs 1.6 ms (C = 1024); N = 1024, T = 65536: 1.42 vs 1.17 ms (C = 1024); from 4096 neurons
# the single pass wins (N = 4096, T = 65536: 1.65 vs 2.24 ms).
LONG_MAX_N = 1024
LONG_MIN_T = 65536
LONG_K = 32


def long_sequence_C(T, N):
    """Chunk of the long-sequence exact forward, or 0 when the single pass is used: the longest
    of 4096, 2048, 1024 dividing T that leaves >= 1024 chunk x 64-neuron blocks."""
    if N > LONG_MAX_N or T < LONG_MIN_T:
        return 0
    nb = (N + 63) // 64
    for c in (4096, 2048, 1024):
        if T % c == 0 and (T // c) * nb >= 1024:
            return c
    return 0


# The long-chunk path in pieces of consecutive chunks (lsh_lif_scan_v3_pieces_fwd): the
# builds of later pieces run on a side stream while earlier pieces carry and replay.  Each
# piece costs at least one chunk's serial replay, so it pays only on large work: measured on
# MI355X, N = 1024, T = 2^20: unsplit (C 4096) 8.15 ms, C 4096 in 2 pieces 7.33, C 2048 in 4
# pieces 7.13, C 1024 in 8 pieces 8.43; at 2^27-2^28 neuron-steps (N = 256, T = 2^18; N = 512,
# T = 2^19; N = 1024, T = 2^18) every split was slower than or within 4 % of the unsplit scan.
LONG_PIECES = 4
LONG_PIECES_MIN_WORK = 2 ** 30  # neuron-steps


def long_sequence_plan(T, N):
    """(C, P) of the converged long-chunk forward: the chunk and pieces, (long_sequence_C, 1)
    below LONG_PIECES_MIN_WORK neuron-steps, else half that chunk in LONG_PIECES pieces; C is 0
    when the single pass is used."""
    C = long_sequence_C(T, N)
    if C and T * N >= LONG_PIECES_MIN_WORK and T % (C // 2 * LONG_PIECES) == 0:
        return C // 2, LONG_PIECES
    return C, 1


def _scan2_pieces(I, beta, theta, u_r, u0, C, K, P):
    """The converged two-level scan in P pieces -> (U, S), the serial recurrence."""
    global _LAST_RUN
    I = _input(I)
    T, N = I.shape
    u0 = _vec(u0, N, I)
    C, K, P = int(C), int(K), int(P)
    if C < 1 or P < 1 or T % (C * P):
        raise ValueError(f"T={T} must be divisible by C*P={C * P}")
    L = _n.lib()
    nbytes = L.lsh_lif_scan_v3_pieces_workspace(T, N, C, K, P)
    if nbytes == 0:
        raise ValueError(f"unsupported scan shape T={T} N={N} C={C} K={K} P={P}")
    ws = _n.workspace(nbytes, I.device)
    U = torch.empty_like(I)
    S = torch.empty_like(I)
    with _n.on_device(I):
        _n.check(L.lsh_lif_scan_v3_pieces_fwd(
            _n.ptr(I), _n.ptr(u0), _n.ptr(U), _n.ptr(S), T, N, _f32(beta), _f32(theta), _f32(u_r),
            C, K, P, _n.ptr(ws), nbytes, _n.stream_of(I)), "lsh_lif_scan_v3_pieces_fwd")
    _LAST_RUN = _ScanRun(ws, T // P, N, C, K)  # the first piece's arrays
    _LAST_RUN.pieces = P
    return U, S


# Warm-started converged forward (lsh_lif_scan_warm_fwd): the warm-up must run long enough for
# the true trajectory and the one from u_r to spike together; the time to forget a start grows
# like 1/(1 - beta), so W = 24/(1 - |beta|) steps rounded up to 256 (256 to 8192).  Above
# WARM_FEW_MAX_N neurons, chunks of at least 3W keep the re-read of the warm-up rows <= 1/3 of a
# pass; the longest chunk (a power of two dividing T) that still gives >= WARM_WAVES (chunk,
# 64-neuron block) waves, else the shortest, with >= 4 chunks.  Up to WARM_FEW_MAX_N neurons the
# chunk gives the waves the pass needs instead (below).  Measured on MI355X with the 3W rule
# (converged scan_forward_v3 before -> warm):
# N = 1024, T = 2^20: 7.2 -> 3.1 ms (beta .99), 6.8 -> 2.7 ms (.9); N = 256, T = 2^18: 1.7 ->
# 0.57 / 1.4 -> 0.19; N = 64, T = 2^20: 3.5 -> 0.56 / 3.3 -> 0.23; N = 1024, T = 65536: 1.14 ->
# 0.54 / 0.92 -> 0.16; N = 4096, T = 65536: 1.62 -> 0.93 / 1.62 -> 0.69; N = 8192, T = 65536:
# 1.89 -> 1.71 / 1.89 -> 1.41.  With only 2 chunks (N = 4096 or 1024, T = 16384, beta .99) the
# single pass stays faster, and from 16384 neurons it is as fast or faster.
WARM_MAX_N = 8192
WARM_MIN_CHUNKS = 4
WARM_WAVES = 1024
WARM_K = 24.0
# Up to WARM_FEW_MAX_N neurons the chip has waves to spare, so the chunks are made short enough
# for about WARM_TARGET_WAVES waves (WARM_TARGET_WAVES_LARGE from WARM_LARGE_WORK neuron-steps,
# where the pass is bandwidth-bound) instead of 3W long: a wave's time is its W + C dependent
# steps.  Measured on MI355X (beta 0.99, W 2560, x ~ N(0.012, 0.08^2) / N(0.15, 0.4^2); this
# rule's chunk against the 3W rule's, or the single pass where that had none): N 128, T 16384
# 0.15 / 0.10 ms against 0.37 / 0.39 (single pass); N 128, T 65536 0.28 / 0.13 against 0.40 /
# 0.39; N 1024, T 65536 0.34 / 0.21 against 0.47 / 0.40; N 256, T 2^18 0.40 / 0.23 against 0.46
# / 0.40; N 4096, T 16384 0.32 / 0.20 against 0.41 / 0.42; N 4096, T 65536 and cfg4 (N 1024,
# T 2^20) keep their chunk (8192, 16384).  From 8192 neurons the single pass is as fast.
WARM_FEW_MAX_N = 4096
WARM_MIN_C = 256
WARM_TARGET_WAVES = 512
WARM_TARGET_WAVES_LARGE = 1024
WARM_LARGE_WORK = 2 ** 29


def warm_plan(T, N, beta):
    """(C, W) of the warm-started converged forward for [T, N] inputs and decay beta, or None
    when the single pass or the long-chunk scan is used."""
    if N > WARM_MAX_N or N < 1 or T < 1:
        return None
    b = abs(_f32(beta))
    W = 8192 if b >= 1.0 else int(min(8192, max(256, 256 * math.ceil(WARM_K / (1.0 - b) / 256.0))))
    nb = (N + 63) // 64
    if N <= WARM_FEW_MAX_N:
        # warm-ups that reach back to row 0 for most chunks make the pass a serial sweep
        if T < WARM_MIN_CHUNKS * W:
            return None
        target = WARM_TARGET_WAVES_LARGE if T * N >= WARM_LARGE_WORK else WARM_TARGET_WAVES
        best = None
        c = 1 << 16
        while c >= WARM_MIN_C:
            if T % c == 0 and T // c >= WARM_MIN_CHUNKS:
                miss = abs(math.log2((T // c) * nb / target))
                if best is None or miss < best[0]:  # ties keep the longer chunk
                    best = (miss, c)
            c //= 2
        return (best[1], W) if best else None
    best = None
    c = 1 << 16
    while c >= 3 * W:
        if T % c == 0 and T // c >= WARM_MIN_CHUNKS:
            best = c
            if (T // c) * nb >= WARM_WAVES:
                break
        c //= 2
    return (best, W) if best else None


def _scan_warm_run(I, beta, theta, u_r, u0, C, W):
    global _LAST_RUN
    U, S = scan_forward_warm(I, beta, theta, u_r, u0, C=C, W=W)
    _LAST_RUN = _WarmRun(C, W)
    return U, S


class _WarmRun:
    """The most recent converged forward took the warm-started chunks (chunk C, warm-up W)."""

    pieces = 1
    warm = True

    def __init__(self, C, W):
        self.C, self.W = C, W


def scan_forward_warm(I, beta, theta, u_r, u0, C=2048, W=None, stats=None):
    """Converged exact forward by warm-started chunks (lsh_lif_scan_warm_fwd) -> (U, S), the
    serial recurrence: chunk m's entry is predicted by W steps of the recurrence from u_r over
    the rows before it (W defaults to C), every chunk is replayed from its prediction, and the
    device repair replays the chunks whose prediction missed.  stats receives repair_iters
    (rounds) and missed_frac (the fraction of chunk entries m >= 1 whose prediction differed
    from the exit of chunk m-1 replayed from its own prediction, before the repair)."""
    I = _input(I)
    T, N = I.shape
    u0 = _vec(u0, N, I)
    C = int(C)
    W = C if W is None else int(W)
    if C < 1 or T % C or W < 0:
        raise ValueError(f"the warm-started forward needs C >= 1 dividing T={T} and W >= 0")
    if T == 0 or N == 0:  # nothing to compute (an empty tensor has no device address)
        if stats is not None:
            stats["repair_iters"], stats["missed_frac"] = 0, 0.0
        return torch.empty_like(I), torch.empty_like(I)
    L = _n.lib()
    nbytes = L.lsh_lif_scan_warm_workspace(T, N, C)
    if nbytes == 0:
        raise ValueError(f"unsupported scan shape T={T} N={N} C={C}")
    ws = _n.workspace(nbytes, I.device)
    U = torch.empty_like(I)
    S = torch.empty_like(I)
    with _n.on_device(I):
        _n.check(L.lsh_lif_scan_warm_fwd(
            _n.ptr(I), _n.ptr(u0), _n.ptr(U), _n.ptr(S), T, N, _f32(beta), _f32(theta), _f32(u_r),
            C, W, _n.ptr(ws), nbytes, _n.stream_of(I)), "lsh_lif_scan_warm_fwd")
    if stats is not None:
        st = _n.read_stats(ws, max((T // C - 1) * N, 1))
        stats["repair_iters"] = int(st.repair_iters)
        stats["missed_frac"] = float(st.fused_fixups) / max((T // C - 1) * N, 1)
    return U, S


def scan_forward_assoc(I, beta, theta, u_r, u0, C=2048, K=32, repair=None, stats=None):
    """The two-level map scan with the associative carry (lsh_lif_scan_v3_assoc_fwd) -> (U, S):
    the single-read chunk-map build, then the chunk maps of each neuron composed by a parallel
    prefix (DPP inside each wave, the wave totals in LDS; overflowed chunks run serially), the
    replay, and repair rounds (default: to convergence, T/C rounds: the serial recurrence bit
    for bit).  With repair = 0 the chunk starts are the scan's own predictions.  stats:
    repair_iters, overflow_frac, mean_pieces, max_pieces (the truncation's, as scan_forward_v3).
    beta >= 0 (the envelope maps compose only then), 1 <= K <= 32, T % C == 0."""
    global _LAST_RUN
    I = _input(I)
    T, N = I.shape
    u0 = _vec(u0, N, I)
    C, K = int(C), int(K)
    if C < 1 or T % C or not 1 <= K <= 32 or _f32(beta) < 0:
        raise ValueError(f"the associative map scan needs C >= 1 dividing T={T}, 1 <= K <= 32, "
                         f"beta >= 0")
    R = _repair_arg(T // C if repair is None else repair, T // C, stats)
    if T == 0 or N == 0:
        if stats is not None:
            stats.update(repair_iters=0, overflow_frac=0.0, mean_pieces=1.0, max_pieces=1)
        return torch.empty_like(I), torch.empty_like(I)
    L = _n.lib()
    nbytes = L.lsh_lif_scan_v3_assoc_workspace(T, N, C, K)
    if nbytes == 0:
        raise ValueError(f"unsupported scan shape T={T} N={N} C={C} K={K}")
    ws = _n.workspace(nbytes, I.device)
    U = torch.empty_like(I)
    S = torch.empty_like(I)
    with _n.on_device(I):
        _n.check(L.lsh_lif_scan_v3_assoc_fwd(
            _n.ptr(I), _n.ptr(u0), _n.ptr(U), _n.ptr(S), T, N, _f32(beta), _f32(theta), _f32(u_r),
            C, K, R, _n.ptr(ws), nbytes, _n.stream_of(I)), "lsh_lif_scan_v3_assoc_fwd")
    _LAST_RUN = _ScanRun(ws, T, N, C, K)
    if stats is not None:
        _fill_stats(stats, _n.read_stats(ws, (T // C) * N))
    return U, S


def scan_forward_mapscan(I, beta, theta, u_r, u0, C=64, K=16, repair=0, stats=None):
    """The two-level map scan of scan_forward_v3 itself (envelope + capacity-K chunk maps, carry
    with overflow fallback, replay, device repair) -> (U, S), also where scan_forward_v3 would
    compute its converged result by a faster exact path.  For measuring the map scan."""
    return _scan2(I, beta, theta, u_r, u0, C, K, repair, stats)


def scan_forward(I, beta, theta, u_r, u0, C=64, K=16, BN=BN_DEFAULT, repair=0, stats=None):
    """Two-level scan pruned with the loose global state_bounds (triton_lif.py:262-295)."""
    I = _input(I)
    u0v = _vec(u0, I.shape[1], I)
    lo, _ = state_bounds(I, _f32(beta), _f32(theta), _f32(u_r), u0v)
    st = {} if stats is not None else None
    U, S = _scan2(I, beta, theta, u_r, u0v, C, K, repair, st, lo=lo)
    if stats is not None:
        stats["repair_iters"] = st["repair_iters"]
        stats["overflow_frac"] = st["overflow_frac"]
        stats["max_pieces"] = st["max_pieces"]
    return U, S


def scan_forward_tiled(I, beta, theta, u_r, u0, C=64, K=16, BN=128, BNr=32, D=4, nw=4, nwr=1,
                       repair=0, stats=None):
    """triton_lif.py:479-509: same maps as scan_forward, tiled replay."""
    st = {} if stats is not None else None
    U, S = scan_forward(I, beta, theta, u_r, u0, C=C, K=K, repair=repair, stats=st)
    if stats is not None:
        stats["repair_iters"] = st["repair_iters"]
        stats["overflow_frac"] = st["overflow_frac"]
    return U, S


def scan_forward_v2(I, beta, theta, u_r, u0, C=64, K=16, BN=128, nw=4, STAGES=3, CSTAGES=1,
                    BNr=32, D=4, nwr=1, repair=0, stats=None, Imin=None):
    """triton_lif.py:609-642: pruned with lo = min(u0, u_r, 0) + min(Imin, 0) * 1/(1-beta)
    (or * T when beta == 1), computed in fp32 as the reference's build2 kernel does."""
    I = _input(I)
    T, N = I.shape
    u0v = _vec(u0, N, I)
    b = _f32(beta)
    if Imin is None:
        Imin = I.amin(0)
    inv = 1.0 / (1.0 - b) if b < 1 else float(T)
    imin = torch.minimum(Imin.float(), torch.zeros_like(u0v))
    base = torch.minimum(torch.minimum(u0v, torch.full_like(u0v, _f32(u_r))), torch.zeros_like(u0v))
    lo = (base + imin * torch.tensor(inv, dtype=torch.float32, device=I.device)).contiguous()
    st = {} if stats is not None else None
    U, S = _scan2(I, beta, theta, u_r, u0v, C, K, repair, st, lo=lo)
    if stats is not None:
        stats["repair_iters"] = st["repair_iters"]
        stats["overflow_frac"] = st["overflow_frac"]
    return U, S


class _ScanRunV4(_ScanRun):
    """Workspace of one three-level scan call: chunk arrays as in v3, plus super maps."""

    def __init__(self, ws, T, N, C, G, K, K2):
        super().__init__(ws, T, N, C, K)
        self.G, self.K2 = G, K2

    def layout(self):
        L = _n.V4Layout()
        _n.check(_n.lib().lsh_lif_scan_v4_layout(self.T, self.N, self.C, self.G, self.K, self.K2,
                                                 _n.ctypes.byref(L)), "lsh_lif_scan_v4_layout")
        return L

    def view(self, name, dtype=torch.float32):
        L = self.layout()
        M = self.T // self.C
        M2 = M // self.G
        if name in ("SA", "SB", "SN", "SOVF", "SX", "SC", "SSTARTS"):
            off = getattr(L, name)
            shape = (M2, self.K2, self.N) if name in ("SX", "SC") else (M2, self.N)
        else:
            off = getattr(L.v3, name)
            shape = (M, self.K, self.N) if name in ("MX", "MC") else (M, self.N)
        nbytes = 4 * math.prod(shape)
        return self.ws[off:off + nbytes].view(dtype).view(*shape)


def scan_forward_v4(I, beta, theta, u_r, u0, C=64, G=16, K=16, K2=32, BN=32, nw=1, BNg=16, nwg=1,
                    BNc=16, nwc=1, BNr=32, D=8, nwr=1, repair=0, stats=None, super_fallback="auto"):
    """Three-level exact scan (triton_lif.py:935-983) -> (U, S).  T must be divisible by C*G
    (ValueError, the reference asserts).  stats receives repair_iters, overflow_frac,
    super_overflow_frac, mean_pieces, super_mean_pieces, super_max_pieces (:976-982).
    super_fallback: how the super-map carry passes an overflowed super map: "chunks" walks its
    G chunk maps (as the inner carry does; an overflowed chunk map runs its C steps serially),
    "serial" runs its C*G steps serially (the reference's carry, triton_lif.py:958-963), "none"
    evaluates it as stored (a start the repair replaces where it is wrong: only with the repair
    budget at least T/C and no stats), "auto" is "none" there for groups of 16 chunks or more
    (AUTO_V4_AS_STORED_MIN_G) and "chunks" otherwise.  With the
    repair budget at least T/C and no stats requested, the result is the serial recurrence and
    the fastest exact path computes it, as in scan_forward_v3 (scan_forward_v4_maps runs the
    three-level pipeline itself)."""
    I = _input(I)
    T = I.shape[0]
    if int(C) >= 1 and int(G) >= 1 and T % int(C) == 0 and (T // int(C)) % int(G) == 0:
        out = _converged_fast(I, beta, theta, u_r, u0, C, min(int(K), 16), repair, stats)
        if out is not None:
            return out
    return scan_forward_v4_maps(I, beta, theta, u_r, u0, C=C, G=G, K=K, K2=K2, repair=repair,
                                stats=stats, super_fallback=super_fallback)


# Converged calls pass an overflowed super map as stored ("none") from groups of this many
# chunks: the walk over a group's chunk maps grows with G, the repair of the starts the stored
# map gets wrong does not.  Measured on MI355X, scan_forward_v4_maps with repair to
# convergence, K 16, K2 32, beta 0.99, "none" against "chunks" (ms): G 16 (C 64): cfg4 15.6 /
# 18.5; N 128 / 1024, T 2^18, x ~ N(0.15, 0.4^2) 1.12 / 1.17, 2.94 / 3.07; N 4096 / 16384 at
# N*T = 2^28, x ~ N(0.012, 0.08^2) 8.35 / 9.73, 4.31 / 4.66; N 128 / 1024, T 65536 1.02 / 0.92,
# 2.12 / 2.05.  G 8 (C 128): 0.77 / 0.77, 2.51 / 2.53; 8.01 / 7.53, 3.90 / 3.72; 1.35 / 0.91,
# 2.59 / 1.74.
AUTO_V4_AS_STORED_MIN_G = 16


def scan_forward_v4_maps(I, beta, theta, u_r, u0, C=64, G=16, K=16, K2=32, repair=0, stats=None,
                         super_fallback="auto"):
    """The three-level pipeline of scan_forward_v4 itself (envelope, chunk maps, group
    composition, super-map carry, inner carry, replay, device repair) -> (U, S), also where
    scan_forward_v4 would compute its converged result by a faster exact path.  For measuring
    the three-level scan."""
    global _LAST_RUN
    if super_fallback not in ("auto", "chunks", "serial", "none"):
        raise ValueError('super_fallback must be "auto", "chunks", "serial" or "none"')
    I = _input(I)
    T, N = I.shape
    u0 = _vec(u0, N, I)
    C, G, K, K2 = int(C), int(G), int(K), int(K2)
    if C < 1 or G < 1 or T % C or (T // C) % G:
        raise ValueError(f"T={T} must be divisible by C*G={C * G}")
    if not (1 <= K <= 32 and K <= K2 <= 64):
        raise ValueError("three-level scan needs 1 <= K <= 32 and K <= K2 <= 64")
    rep = _repair_arg(repair, T // C, stats)
    if super_fallback == "auto":
        super_fallback = "none" if rep == -1 and G >= AUTO_V4_AS_STORED_MIN_G else "chunks"
    if super_fallback == "none" and rep != -1:
        raise ValueError('super_fallback="none" needs repair >= T/C and no stats (the repair '
                         'replaces the starts it gets wrong)')
    L = _n.lib()
    nbytes = L.lsh_lif_scan_v4_workspace(T, N, C, G, K, K2)
    if nbytes == 0:
        raise ValueError(f"unsupported three-level scan shape T={T} N={N} C={C} G={G}")
    ws = _n.workspace(nbytes, I.device)
    U = torch.empty_like(I)
    S = torch.empty_like(I)
    with _n.on_device(I):
        _n.check(L.lsh_lif_scan_v4_fwd(_n.ptr(I), _n.ptr(u0), _n.ptr(U), _n.ptr(S), T, N,
                                       _f32(beta), _f32(theta), _f32(u_r), C, G, K, K2,
                                       {"serial": 0, "chunks": 1, "none": 2}[super_fallback],
                                       rep, _n.ptr(ws), nbytes,
                                       _n.stream_of(I)),
                 "lsh_lif_scan_v4_fwd")
    _LAST_RUN = _ScanRunV4(ws, T, N, C, G, K, K2)
    if stats is not None:
        _fill_stats(stats, _n.read_stats(ws, (T // C) * N, (T // C // G) * N), v4=True)
    return U, S


# ----------------------------------------------------------------------------- single-pass exact scan
# Internal chunk lengths of the single-pass kernels (their results do not depend on them:
# the forward is bit-identical to the serial recurrence, the backward equals the two-level
# affine scan up to fp32 association).
FUSED_FWD_C = 32
FUSED_BWD_C = 32
FUSED_CHUNKS = (16, 32, 64, 128)
# Map speculation shortens the in-workgroup hand-off chain but puts the map build on every
# round's critical path; measured on MI355X it never beat the plain chain (at large N the
# chain is hidden by other workgroups, at small N the build costs more than it saves), so
# maps="auto" leaves it off.  maps=True still selects it.
FUSED_MAPS_MAX_N = 0

_LAST_FUSED = None


def last_fused_counters():
    """Counters of the most recent single-pass forward: fused_fixups (chunk entries whose
    map prediction missed), fused_unknown (entries the maps could not predict) and
    spin_timeouts (must be 0).  Synchronizes."""
    if _LAST_FUSED is None:
        return None
    st = _n.read_stats(_LAST_FUSED, 1)
    return {"fused_fixups": int(st.fused_fixups), "fused_unknown": int(st.fused_unknown),
            "spin_timeouts": int(st.spin_timeouts)}


def scan_forward_exact(I, beta, theta, u_r, u0, C=None, K=8, maps="auto"):
    """Single-pass exact two-level scan -> (U, S), bit-identical to the serial recurrence
    (= scan_forward_v3 with the repair run to convergence), reading I once.  C is the
    kernel's internal chunk length (16/32/64/128, default FUSED_FWD_C), K the map capacity
    (<= 16).  maps=False hands chunk exits on without map predictions (chunked serial);
    "auto" builds maps when N <= FUSED_MAPS_MAX_N."""
    global _LAST_FUSED
    I = _input(I)
    T, N = I.shape
    u0 = _vec(u0, N, I)
    C = int(C or FUSED_FWD_C)
    if C not in FUSED_CHUNKS or T % C:
        raise ValueError(f"single-pass scan needs C in {FUSED_CHUNKS} dividing T={T}")
    if not 1 <= int(K) <= 16:
        raise ValueError("single-pass scan supports map capacity K in [1, 16]")
    if maps == "auto":
        maps = N <= FUSED_MAPS_MAX_N
    L = _n.lib()
    nbytes = L.lsh_lif_scan_exact_workspace()
    ws = _n.workspace(nbytes, I.device)
    U = torch.empty_like(I)
    S = torch.empty_like(I)
    with _n.on_device(I):
        st = _n.stream_of(I)
        if maps:
            rc = L.lsh_lif_scan_exact_fwd(_n.ptr(I), _n.ptr(u0), _n.ptr(U), _n.ptr(S), T, N,
                                          _f32(beta), _f32(theta), _f32(u_r), C, int(K),
                                          _n.ptr(ws), nbytes, st)
        else:
            rc = L.lsh_lif_chunked_serial_fwd(_n.ptr(I), _n.ptr(u0), _n.ptr(U), _n.ptr(S), T, N,
                                              _f32(beta), _f32(theta), _f32(u_r), C, _n.ptr(ws),
                                              nbytes, st)
        _n.check(rc, "single-pass scan forward")
    _LAST_FUSED = ws
    return U, S


def _fused_fwd_ok(T, C, K, repair, stats):
    """The single-pass kernel gives the converged result; finite repair budgets and the
    reference's stats (which describe the chunk-C maps) use the multi-kernel path."""
    return stats is None and int(repair) >= T // int(C) and int(K) <= 16 and T % FUSED_FWD_C == 0


def scan_backward_fused(I, u0, U, S, GS, GU, beta, theta, u_r, alpha=4.0, detach=True, C=None):
    """Single-pass affine-scan adjoint -> Lam (I, U, S, GS read once)."""
    I = _input(I)
    T, N = I.shape
    u0 = _vec(u0, N, I)
    U, S, GS = _same(U, I, "U"), _same(S, I, "S"), _same(GS, I, "GS")
    GU = _same(GU, I, "GU")
    C = int(C or FUSED_BWD_C)
    if C not in (16, 32, 64) or T % C:
        raise ValueError(f"single-pass backward needs C in (16, 32, 64) dividing T={T}")
    Lam = torch.empty_like(I)
    with _n.on_device(I):
        _n.check(_n.lib().lsh_lif_scan_fused_bwd(
            _n.ptr(I), _n.ptr(u0), _n.ptr(U), _n.ptr(S), _n.ptr(GS), _n.ptr(GU), _n.ptr(Lam), T, N,
            _f32(beta), _f32(theta), _f32(u_r), _f32(alpha), int(bool(detach)), C, _n.stream_of(I)),
            "lsh_lif_scan_fused_bwd")
    return Lam


# ----------------------------------------------------------------------------- recomputing pair
# LIFTuned keeps U only for its backward.  When both passes run the single-pass kernels, the
# forward writes S and the exact entry state of every FUSED_FWD_C-step chunk instead of U, and
# the adjoint replays each chunk's forward from that state in registers: the same Lam (the
# forward's own u_{t-1} and s_t bits), 20 instead of 32 bytes of HBM traffic per neuron-step.
RECOMPUTE_BWD = True


# The starts-only forward adds the count of chunk hand-offs whose bounded wait gave up to a
# per-device counter header that is cleared once and never by the calls themselves (no reset
# launch per call).  It must stay 0: starts_forward_timeouts() reads it (synchronizing), and
# with CHECK_WAITS (environment LIFSCAN_CHECK_WAITS=1) every call reads it and raises.
CHECK_WAITS = os.environ.get("LIFSCAN_CHECK_WAITS", "0") not in ("", "0")
_WAIT_HEADERS = {}


def _wait_header(device):
    h = _WAIT_HEADERS.get(device)
    if h is None:
        h = torch.zeros(max(int(_n.lib().lsh_lif_scan_exact_workspace()), 256), dtype=torch.uint8,
                        device=device)
        _WAIT_HEADERS[device] = h
    return h


def starts_forward_timeouts(device=None):
    """Hand-offs of the starts-only forward on `device` (default: the current one) that gave
    up since the process started (must be 0).  Synchronizes."""
    device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    h = _WAIT_HEADERS.get(device)
    return 0 if h is None else int(_n.read_stats(h, 1).spin_timeouts)


def scan_forward_exact_starts(I, beta, theta, u_r, u0, C=None):
    """Single-pass exact forward -> (S, STARTS [T//C, N]): S as scan_forward_exact, and the
    state before every C-step chunk (STARTS[0] = u0) in place of U."""
    I = _input(I)
    T, N = I.shape
    u0 = _vec(u0, N, I)
    C = int(C or FUSED_FWD_C)
    if C not in (16, 32, 64) or T % C:
        raise ValueError(f"the starts-only forward needs C in (16, 32, 64) dividing T={T}")
    S = torch.empty_like(I)
    ST = torch.empty(T // C, N, device=I.device, dtype=torch.float32)
    hdr = _wait_header(I.device)
    with _n.on_device(I):
        _n.check(_n.lib().lsh_lif_scan_exact_fwd_starts(
            _n.ptr(I), _n.ptr(u0), _n.ptr(ST), _n.ptr(S), T, N, _f32(beta), _f32(theta), _f32(u_r), C,
            _n.ptr(hdr), hdr.numel(), _n.stream_of(I)), "lsh_lif_scan_exact_fwd_starts")
    if CHECK_WAITS and int(_n.read_stats(hdr, 1).spin_timeouts) != 0:
        raise RuntimeError("lsh_lif_scan_exact_fwd_starts: a chunk hand-off wait gave up; "
                           "S and the chunk entry states are not valid")
    return S, ST


def scan_backward_fused_starts(I, STARTS, GS, beta, theta, u_r, alpha=4.0, want_sums=False):
    """Single-pass adjoint from the chunk entry states (detached reset, no GU) -> (Lam, sums):
    sums (fp64 [3]: sum lam*u_{t-1}, sum gS*sg, sum s*lam_{t+1}) when want_sums, else None."""
    I = _input(I)
    T, N = I.shape
    GS = _same(GS, I, "GS")
    M = STARTS.shape[0]
    if M == 0 or T % M or STARTS.shape != (M, N):
        raise ValueError(f"STARTS must be [T//C, {N}]")
    C = T // M
    STARTS = STARTS.contiguous()
    Lam = torch.empty_like(I)
    parts = None
    if want_sums:
        parts = torch.zeros((N + 63) // 64, 3, device=I.device, dtype=torch.float64)
    with _n.on_device(I):
        _n.check(_n.lib().lsh_lif_scan_fused_bwd_starts(
            _n.ptr(I), _n.ptr(STARTS), _n.ptr(GS), _n.ptr(Lam), _n.ptr(parts), T, N,
            _f32(beta), _f32(theta), _f32(u_r), _f32(alpha), C, _n.stream_of(I)),
            "lsh_lif_scan_fused_bwd_starts")
    return Lam, (parts.sum(0) if want_sums else None)


def _recompute_ok(T, N, K, repair):
    """True when scan_forward_auto and scan_backward_auto would both take the single-pass
    kernels (converged forward without maps, fused adjoint): then the recomputing pair gives
    the same S and Lam.  False (never an error) for lengths the chunk policy rejects."""
    if not RECOMPUTE_BWD or FUSED_FWD_C != FUSED_BWD_C or T == 0 or N == 0:
        return False
    if T % FUSED_FWD_C:
        return False
    C = _chunk_or_none(T, 16)
    if C is None or not _fused_fwd_ok(T, C, K, repair, None):
        return False
    if long_sequence_C(T, N) or N <= FUSED_MAPS_MAX_N:
        return False
    return N >= FUSED_BWD_MIN_N and T % FUSED_BWD_C == 0


# ----------------------------------------------------------------------------- scan backward
# The single-pass adjoint owns 64 neurons per workgroup: with fewer than this many neurons the
# chip is not filled, and the look-back adjoint (workgroups over 256-step segments chained by
# a decoupled look-back) wins: N = 1024, T = 2^20: 3.63 ms vs 36.4 ms single pass and 8.13 ms
# three-kernel chunk scan; N = 8192, T = 8192: 0.27 vs 0.38 / 0.47 ms.  From 16384 neurons
# the single pass is as fast or faster (N = 16384, T = 1024: 0.068 vs 0.077 ms).
FUSED_BWD_MIN_N = 16384
CHUNKED_BWD_MIN_BLOCKS = 2048  # chunk x 64-neuron blocks that keep every CU busy


def chunked_bwd_C(T, N, C=64):
    """Chunk of the three-kernel adjoint: the longest of 512..8 dividing T that still gives
    CHUNKED_BWD_MIN_BLOCKS blocks (fewer, longer chunks cut the carry and aggregate traffic),
    else the given C."""
    nb = (N + 63) // 64
    for c in (512, 256, 128, 64, 32, 16, 8):
        if T % c == 0 and (T // c) * nb >= CHUNKED_BWD_MIN_BLOCKS:
            return c
    return int(C)


LOOKBACK_SEG = 256  # steps per workgroup segment of the look-back adjoint
_LAST_LOOKBACK = None


def scan_backward_lookback(I, u0, U, S, GS, GU, beta, theta, u_r, alpha=4.0, detach=True, C=16):
    """Single-pass affine-scan adjoint with a decoupled look-back across workgroups -> Lam
    (for few neurons; T % 256 == 0; C in {16, 32} steps per wave)."""
    global _LAST_LOOKBACK
    I = _input(I)
    T, N = I.shape
    u0 = _vec(u0, N, I)
    U, S, GS = _same(U, I, "U"), _same(S, I, "S"), _same(GS, I, "GS")
    GU = _same(GU, I, "GU")
    L = _n.lib()
    nbytes = L.lsh_lif_scan_lookback_bwd_workspace(T, N)
    if nbytes == 0:
        raise ValueError(f"look-back adjoint needs T % {LOOKBACK_SEG} == 0 (T={T})")
    ws = _n.workspace(nbytes, I.device)
    Lam = torch.empty_like(I)
    with _n.on_device(I):
        _n.check(L.lsh_lif_scan_lookback_bwd(
            _n.ptr(I), _n.ptr(u0), _n.ptr(U), _n.ptr(S), _n.ptr(GS), _n.ptr(GU), _n.ptr(Lam), T, N,
            _f32(beta), _f32(theta), _f32(u_r), _f32(alpha), int(bool(detach)), int(C), _n.ptr(ws),
            nbytes, _n.stream_of(I)), "lsh_lif_scan_lookback_bwd")
    _LAST_LOOKBACK = ws
    return Lam


def last_lookback_timeouts():
    """Bounded waits of the most recent look-back adjoint that gave up (must be 0)."""
    if _LAST_LOOKBACK is None:
        return None
    return int(_n.read_stats(_LAST_LOOKBACK, 1).spin_timeouts)


def scan_backward_tiled(I, u0, U, S, GS, GU, beta, theta, u_r, alpha=4.0, detach=True, C=64,
                        BNr=32, D=4, nwr=1):
    """Affine-scan adjoint (triton_lif.py:512-526) -> Lam.  GU may be None (zeros).
    Runs the single-pass kernel when there are enough neurons to fill the chip and T is a
    multiple of its internal chunk, else the three-kernel chunk scan (chunk from
    chunked_bwd_C; the given C when none fits)."""
    I = _input(I)
    T, N = I.shape
    if N >= FUSED_BWD_MIN_N and T % FUSED_BWD_C == 0:
        return scan_backward_fused(I, u0, U, S, GS, GU, beta, theta, u_r, alpha, detach)
    if LOOKBACK_BWD and T % LOOKBACK_SEG == 0:
        return scan_backward_lookback(I, u0, U, S, GS, GU, beta, theta, u_r, alpha, detach)
    return scan_backward_chunked(I, u0, U, S, GS, GU, beta, theta, u_r, alpha, detach,
                                 chunked_bwd_C(T, N, C))


LOOKBACK_BWD = True


def scan_backward_chunked(I, u0, U, S, GS, GU, beta, theta, u_r, alpha=4.0, detach=True, C=64):
    """Three-kernel affine scan: chunk aggregates, reverse carry, reverse replay."""
    I = _input(I)
    T, N = I.shape
    u0 = _vec(u0, N, I)
    U, S, GS = _same(U, I, "U"), _same(S, I, "S"), _same(GS, I, "GS")
    GU = _same(GU, I, "GU")
    C = int(C)
    if C < 1 or T % C:
        raise ValueError(f"T={T} must be divisible by the chunk length C={C}")
    L = _n.lib()
    nbytes = L.lsh_lif_scan_bwd_workspace(T, N, C)
    ws = _n.workspace(nbytes, I.device)
    Lam = torch.empty_like(I)
    with _n.on_device(I):
        _n.check(L.lsh_lif_scan_bwd(_n.ptr(I), _n.ptr(u0), _n.ptr(U), _n.ptr(S), _n.ptr(GS),
                                    _n.ptr(GU), _n.ptr(Lam), T, N, _f32(beta), _f32(theta),
                                    _f32(u_r), _f32(alpha), int(bool(detach)), C, _n.ptr(ws),
                                    nbytes, _n.stream_of(I)), "lsh_lif_scan_bwd")
    return Lam


def scan_backward(I, u0, U, S, GS, GU, beta, theta, u_r, alpha=4.0, detach=True, C=64,
                  BN=BN_DEFAULT):
    """triton_lif.py:298-312; same kernels as scan_backward_tiled."""
    return scan_backward_tiled(I, u0, U, S, GS, GU, beta, theta, u_r, alpha, detach, C=C)


# ----------------------------------------------------------------------------- auto policies
def _pick_C(T, D=8):
    """Chunk length policy of the reference (triton_lif.py:647-651)."""
    for C in (256, 128, 64, 32, 16, 8):
        if T % C == 0 and C % D == 0 and C * C <= 4 * T:
            return C
    raise ValueError(f"T={T} needs a chunk length divisible by {D}")


def _chunk_or_none(T, D):
    """_pick_C(T, D), or None where that policy raises."""
    try:
        return _pick_C(T, D=D)
    except ValueError:
        return None


def scan_forward_auto(I, beta, theta, u_r, u0, K=16, repair=0):
    """Two-level exact forward with the reference's default chunking (triton_lif.py:1228-1232)."""
    T = I.shape[0]
    C = _pick_C(T, D=16)
    return scan_forward_v3(I, beta, theta, u_r, u0, C=C, K=K, repair=repair)


def scan_backward_auto(I, u0, U, S, GS, GU, beta, theta, u_r, alpha=4.0):
    """Affine-scan backward with the reference's default chunking (triton_lif.py:1235-1239)."""
    T = I.shape[0]
    C = min(128, _pick_C(T, D=2))
    return scan_backward_tiled(I, u0, U, S, GS, GU, beta, theta, u_r, alpha, C=C)


def auto_modes(N, T):
    """Serial or scan per pass from (N, T) (triton_lif.py:997-1000).  A pass whose chunk policy
    has no chunk for T (scan_forward_auto: _pick_C(T, D=16); scan_backward_auto: D=2) stays
    serial, so lif_auto runs for every T (e.g. T = 1000 or 1002), as the reference's does at
    its thresholds."""
    fwd = "scan" if (N <= AUTO_FWD_MAX_N and T >= AUTO_FWD_MIN_T) else "serial"
    bwd = "scan" if (N <= AUTO_BWD_MAX_N and (T >= AUTO_BWD_MIN_T or (
        N >= AUTO_BWD_WIDE_N and T >= AUTO_BWD_WIDE_MIN_T))) else "serial"
    if fwd == "scan" and _chunk_or_none(T, 16) is None:
        fwd = "serial"
    if bwd == "scan" and _chunk_or_none(T, 2) is None:
        bwd = "serial"
    return fwd, bwd


# ----------------------------------------------------------------------------- autograd layers
def _beta_grad(Lam, U, u0, need):
    """dL/dbeta = sum_t lam_t * u_{t-1} (fit.py:44)."""
    if not need:
        return None
    uprev = torch.cat([u0[None], U[:-1]], 0)
    return (Lam * uprev).sum(dtype=torch.float64).float().reshape(())


class LIFFunction(torch.autograd.Function):
    """Hard-reset LIF, mode in {"serial", "scan"} (triton_lif.py:315-339); returns S."""

    @staticmethod
    def forward(ctx, I, u0, beta, theta, u_r, alpha, mode, C, K, repair):
        I = I.contiguous()
        b = _f32(beta)
        if mode == "serial":
            U, S = serial_forward(I, b, theta, u_r, u0)
        else:
            U, S = scan_forward(I, b, theta, u_r, u0, C=C, K=K, repair=repair)
        ctx.save_for_backward(I, u0, U, S)
        ctx.cfg = (b, theta, u_r, alpha, mode, C)
        return S

    @staticmethod
    def backward(ctx, gS):
        I, u0, U, S = ctx.saved_tensors
        b, theta, u_r, alpha, mode, C = ctx.cfg
        gS = gS.contiguous()
        if mode == "serial":
            Lam = serial_backward(I, u0, U, S, gS, None, b, theta, u_r, alpha)
        else:
            Lam = scan_backward(I, u0, U, S, gS, None, b, theta, u_r, alpha, C=C)
        du0 = b * Lam[0] if ctx.needs_input_grad[1] else None
        return (Lam, du0, _beta_grad(Lam, U, u0, ctx.needs_input_grad[2]),
                None, None, None, None, None, None, None)


def lif(I, u0, beta=0.9, theta=1.0, u_r=0.0, alpha=4.0, mode="scan", C=64, K=16, repair=0):
    return LIFFunction.apply(I, u0, beta, theta, u_r, alpha, mode, C, K, repair)


class LIFTuned(torch.autograd.Function):
    """Hard-reset LIF (detached reset, sigmoid surrogate), mode in {"serial", "scan"}
    (triton_lif.py:654-683).  Returns S; gradients for I and u0 as the reference, plus
    dL/dbeta when beta is passed as a 0-d tensor that requires grad (the reference returns
    None for beta).  The backward reads no GU array (it is identically zero here)."""

    @staticmethod
    def forward(ctx, I, u0, beta, theta, u_r, alpha, mode, K, repair):
        I = I.contiguous()
        b = _f32(beta)
        ctx.cfg = (b, theta, u_r, alpha, mode)
        T, N = I.shape
        if mode != "serial" and _recompute_ok(T, N, K, repair):
            # U is kept only for the backward: store the chunk entry states instead
            S, ST = scan_forward_exact_starts(I, b, theta, u_r, u0)
            ctx.save_for_backward(I, u0, ST)
            ctx.recompute = True
            return S
        if mode == "serial":
            U, S = serial_forward_auto(I, b, theta, u_r, u0)
        else:
            U, S = scan_forward_auto(I, b, theta, u_r, u0, K=K, repair=repair)
        ctx.save_for_backward(I, u0, U, S)
        ctx.recompute = False
        return S

    @staticmethod
    def backward(ctx, gS):
        b, theta, u_r, alpha, mode = ctx.cfg
        gS = gS.contiguous()
        if ctx.recompute:
            I, u0, ST = ctx.saved_tensors
            need_b = ctx.needs_input_grad[2]
            Lam, sums = scan_backward_fused_starts(I, ST, gS, b, theta, u_r, alpha, need_b)
            db = sums[0].float().reshape(()) if need_b else None
            du0 = b * Lam[0] if ctx.needs_input_grad[1] else None
            return (Lam, du0, db, None, None, None, None, None, None)
        I, u0, U, S = ctx.saved_tensors
        if mode == "serial":
            Lam = serial_backward_auto(I, u0, U, S, gS, None, b, theta, u_r, alpha)
        else:
            Lam = scan_backward_auto(I, u0, U, S, gS, None, b, theta, u_r, alpha)
        du0 = b * Lam[0] if ctx.needs_input_grad[1] else None
        return (Lam, du0, _beta_grad(Lam, U, u0, ctx.needs_input_grad[2]),
                None, None, None, None, None, None)


_RC_OK = {}


def _rc_path(I, u0, beta, mode, K, repair):
    """u0 as the [N] vector of the C++ recomputing pair (lifscan/_ops.cpp) when lif_tuned can take
    it: the recomputing pair applies, beta needs no gradient, u0 is already the layer's [N] fp32
    vector (or needs none) and the module is built; else None."""
    if mode == "serial" or CHECK_WAITS or not torch.is_tensor(I) or I.dim() != 2:
        return None
    if not I.is_cuda or I.dtype != torch.float32:
        return None
    if torch.is_tensor(beta) and beta.requires_grad:
        return None
    T, N = I.shape
    key = (T, N, int(K), int(repair))
    ok = _RC_OK.get(key)
    if ok is None:
        ok = _RC_OK[key] = _recompute_ok(T, N, K, repair)
    if not ok:
        return None
    if (torch.is_tensor(u0) and u0.dim() == 1 and u0.shape[0] == N and u0.dtype == torch.float32
            and u0.device == I.device and u0.is_contiguous()):
        u0v = u0
    elif torch.is_tensor(u0) and u0.requires_grad:
        return None
    else:
        u0v = _vec(u0, N, I)
    return u0v if _n.ops() is not None else None


def lif_tuned(I, u0, beta=0.9, theta=1.0, u_r=0.0, alpha=4.0, mode="scan", K=16, repair=0):
    u0v = _rc_path(I, u0, beta, mode, K, repair)
    if u0v is not None:  # the same kernels and bits as LIFTuned's recomputing pair, from C++
        return _n.ops().lif_tuned_rc(I, u0v, _f32(beta), float(theta), float(u_r), float(alpha),
                                     _wait_header(I.device), FUSED_FWD_C)
    return LIFTuned.apply(I, u0, beta, theta, u_r, alpha, mode, K, repair)


class LIFAuto(torch.autograd.Function):
    """Serial or scan chosen per pass (triton_lif.py:1003-1026)."""

    @staticmethod
    def forward(ctx, I, u0, beta, theta, u_r, alpha, K, repair, fwd_mode, bwd_mode):
        I = I.contiguous()
        b = _f32(beta)
        ctx.cfg = (b, theta, u_r, alpha, bwd_mode)
        T, N = I.shape
        # the serial forward's bits are the single-pass exact forward's; with the fused adjoint
        # behind it the recomputing pair applies (U is kept only for the backward)
        if (fwd_mode == "serial" and bwd_mode == "scan"
                and _recompute_ok(T, N, K, max(int(repair), T))):
            S, ST = scan_forward_exact_starts(I, b, theta, u_r, u0)
            ctx.save_for_backward(I, u0, ST)
            ctx.recompute = True
            return S
        if fwd_mode == "scan":
            U, S = scan_forward_auto(I, b, theta, u_r, u0, K=K, repair=repair)
        else:
            U, S = serial_forward_auto(I, b, theta, u_r, u0)
        ctx.save_for_backward(I, u0, U, S)
        ctx.recompute = False
        return S

    @staticmethod
    def backward(ctx, gS):
        b, theta, u_r, alpha, bwd_mode = ctx.cfg
        gS = gS.contiguous()
        if ctx.recompute:
            I, u0, ST = ctx.saved_tensors
            need_b = ctx.needs_input_grad[2]
            Lam, sums = scan_backward_fused_starts(I, ST, gS, b, theta, u_r, alpha, need_b)
            db = sums[0].float().reshape(()) if need_b else None
            du0 = b * Lam[0] if ctx.needs_input_grad[1] else None
            return (Lam, du0, db, None, None, None, None, None, None, None)
        I, u0, U, S = ctx.saved_tensors
        if bwd_mode == "scan":
            Lam = scan_backward_auto(I, u0, U, S, gS, None, b, theta, u_r, alpha)
        else:
            Lam = serial_backward_auto(I, u0, U, S, gS, None, b, theta, u_r, alpha)
        du0 = b * Lam[0] if ctx.needs_input_grad[1] else None
        return (Lam, du0, _beta_grad(Lam, U, u0, ctx.needs_input_grad[2]),
                None, None, None, None, None, None, None)


def lif_auto(I, u0, beta=0.9, theta=1.0, u_r=0.0, alpha=4.0, K=16, repair=0):
    fwd, bwd = auto_modes(I.shape[1], I.shape[0])
    if fwd == bwd:  # one mode for both passes: lif_tuned's path (the same kernels and bits)
        return lif_tuned(I, u0, beta, theta, u_r, alpha, mode=fwd, K=K, repair=repair)
    return LIFAuto.apply(I, u0, beta, theta, u_r, alpha, K, repair, fwd, bwd)


def surrogate_grad(x, alpha):
    """Derivative of sigmoid(alpha*x) (fast.py:48-51); used by fit.lif_param."""
    sg = torch.sigmoid(alpha * x)
    return alpha * sg * (1 - sg)



# Soft-reset serial functions the reference keeps in triton_lif.py (:1034-1083, :1139-1210);
# implemented in hip_soft, imported at call time (hip_soft uses this module's helpers).
def soft_serial_forward(I, beta, theta, u0, BN=32):
    from . import hip_soft
    return hip_soft.soft_serial_forward(I, beta, theta, u0)


def soft_serial_backward(I, u0, U, GS, beta, theta, alpha=4.0, BN=32):
    from . import hip_soft
    return hip_soft.soft_serial_backward(I, u0, U, GS, beta, theta, alpha)


def soft_serial_backward_pf(I, u0, U, GS, beta, theta, alpha=4.0, BN=32, D=4, num_warps=1):
    from . import hip_soft
    return hip_soft.soft_serial_backward(I, u0, U, GS, beta, theta, alpha)


def soft_serial_backward_auto(I, u0, U, GS, beta, theta, alpha=4.0):
    from . import hip_soft
    return hip_soft.soft_serial_backward(I, u0, U, GS, beta, theta, alpha)


def soft_bwd_cfg(N):
    """(BN, D, num_warps) table of the reference (triton_lif.py:1192-1197); kept for callers."""
    if N <= 8: return 16, 8, 1
    if N <= 64: return 16, 4, 1
    if N <= 16384: return 64, 16, 1
    return 128, 4, 1
