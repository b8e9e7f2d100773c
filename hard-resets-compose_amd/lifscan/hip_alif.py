"""Adaptive-threshold LIF (ALIF) on MI355X with the call signatures of the reference's
``lifscan/triton_alif.py``:

    v = beta*u + I_t;  s = [v >= theta0 + w];  u <- u_r if s else v;  w <- rho*w + q*s

Serial kernels, the warm-up predictor of chunk-entry adaptation, the exact box scan
(first-spike lines + post-spike pieces, verified carry, serial fallback, replay and repair) and
the adjoint as two affine recurrences, all in hand-written HIP kernels of liblifscan_hip.so.
Triton tile keywords (BN for the serial kernels, nw, BNc, BNr, D) are accepted and ignored,
except that alif_scan_forward's BN is the number of neurons that share the per-step piece
split decision, as in the reference's Triton block.
"""
import math

import torch

from . import _native as _n
from .hip_lif import _f32, _f32s, _input, _vec, _same

# single-pass backward (one workgroup per 64 neurons) pays off only with many neuron blocks
ALIF_FUSED_BWD_MIN_N = 8192
ALIF_FUSED_BWD_C = 16
# below that, the single pass with look-back across workgroups when T is a multiple of its segment
ALIF_LOOKBACK_SEG = 128
ALIF_LOOKBACK = True
# ALIFFn's single-pass adjoint after the serial forward recomputes u, w, s inside each chunk from
# the stored row before it (lsh_alif_bwd_recompute) instead of reading U, W, S: same bits
ALIF_RECOMPUTE_BWD = True


def alif_fwd_cfg(N):
    """(BN, D, num_warps) table of the reference (triton_alif.py:255-260); kept for callers."""
    if N <= 8: return 16, 16, 1
    if N <= 64: return 16, 4, 1
    if N <= 4096: return 32, 32, 1
    return 128, 8, 1


def alif_serial_forward(I, beta, rho, q, theta0, u_r, u0, w0, BN=32, D=0, num_warps=1):
    """Serial ALIF (triton_alif.py:263-273) -> (U, W, S); plain and tiled are one kernel."""
    I = _input(I)
    T, N = I.shape
    u0 = _vec(u0, N, I)
    w0 = _vec(w0, N, I, "w0")
    U, W, S = torch.empty_like(I), torch.empty_like(I), torch.empty_like(I)
    with _n.on_device(I):
        _n.check(_n.lib().lsh_alif_serial_fwd(
            _n.ptr(I), _n.ptr(u0), _n.ptr(w0), _n.ptr(U), _n.ptr(W), _n.ptr(S), T, N, _f32(beta),
            _f32(rho), _f32(q), _f32(theta0), _f32(u_r), _n.stream_of(I)), "lsh_alif_serial_fwd")
    return U, W, S


def _dev_params(I, beta, rho, q, theta0):
    """[beta, rho, q, theta0] as one fp32 vector on I's device when any of them is a device tensor
    (device ops only: nothing is read back to the host), else None.  Each value is rounded to
    fp32 as the kernels' float arguments round it."""
    ps = (beta, rho, q, theta0)
    if not any(torch.is_tensor(p) and p.device.type != "cpu" for p in ps):
        return None
    return torch.stack([p.detach().reshape(()).to(device=I.device, dtype=torch.float32)
                        if torch.is_tensor(p) else
                        torch.full((), float(p), device=I.device, dtype=torch.float32) for p in ps])


def _alif_serial_forward_dp(I, dp, u_r, u0, w0):
    """Serial ALIF with the parameters read by the kernel from dp = [beta, rho, q, theta0]."""
    I = _input(I)
    T, N = I.shape
    u0 = _vec(u0, N, I)
    w0 = _vec(w0, N, I, "w0")
    U, W, S = torch.empty_like(I), torch.empty_like(I), torch.empty_like(I)
    with _n.on_device(I):
        _n.check(_n.lib().lsh_alif_serial_fwd_dparams(
            _n.ptr(I), _n.ptr(u0), _n.ptr(w0), _n.ptr(U), _n.ptr(W), _n.ptr(S), T, N, _n.ptr(dp),
            _f32(u_r), _n.stream_of(I)), "lsh_alif_serial_fwd_dparams")
    return U, W, S


def alif_warm_predict(I, beta, rho, q, theta0, u_r, u0, w0, C, Wn=4, u_init=0.0, w_init=0.0, BN=32,
                      UI=None, WI=None):
    """Predicted entry adaptation of every chunk (triton_alif.py:276-285) -> WP [T//C, N]."""
    I = _input(I)
    T, N = I.shape
    u0 = _vec(u0, N, I)
    w0 = _vec(w0, N, I, "w0")
    M = T // int(C)
    if (UI is None) != (WI is None):
        raise ValueError("UI and WI must be given together")
    if UI is not None:
        UI = UI.contiguous().float()
        WI = WI.contiguous().float()
        if UI.shape != (M, N) or WI.shape != (M, N):
            raise ValueError(f"UI, WI must be [{M}, {N}]")
    WP = torch.empty(M, N, device=I.device, dtype=torch.float32)
    with _n.on_device(I):
        _n.check(_n.lib().lsh_alif_warm_predict(
            _n.ptr(I), _n.ptr(u0), _n.ptr(w0), _n.ptr(UI), _n.ptr(WI), _n.ptr(WP), T, N, int(C),
            int(Wn), float(u_init), float(w_init), _f32(beta), _f32(rho), _f32(q), _f32(theta0),
            _f32(u_r), _n.stream_of(I)), "lsh_alif_warm_predict")
    return WP


def alif_prev_wpred(Wprev, w0, C):
    """Chunk-entry adaptation taken from the previous fitting iterate's W [T, N]
    (experiments/e28_allen_alif.py:36): row 0 is w0, row m the adaptation after step m*C - 1.
    A strided device copy of M rows; nothing goes through the host."""
    Wprev = _input(Wprev)
    T, N = Wprev.shape
    C = int(C)
    if T % C:
        raise ValueError(f"T={T} is not a multiple of C={C}")
    w0 = _vec(w0, N, Wprev, "w0")
    return torch.cat([w0[None], Wprev[C - 1:-1:C]], 0).contiguous()


class _ALIFRun:
    """Workspace of one box-scan call (maps, box, chunk states) for stats and tests."""

    def __init__(self, ws, T, N, C, K1, K2):
        self.ws, self.T, self.N, self.C, self.K1, self.K2 = ws, T, N, C, K1, K2

    def layout(self):
        L = _n.ALIFLayout()
        _n.check(_n.lib().lsh_alif_scan_layout(self.T, self.N, self.C, self.K1, self.K2,
                                               _n.ctypes.byref(L)), "lsh_alif_scan_layout")
        return L

    def view(self, name, dtype=torch.float32):
        """[M, N] arrays; MSTAR as [N]; LS/LC/LX as [M, K1, N] and piece arrays as [M, K2, N]
        (the reference's layout; the workspace stores them slot-contiguous, [M, N, K])."""
        L = self.layout()
        M = self.T // self.C
        off = getattr(L, name)
        if name == "MSTAR":
            return self.ws[off:off + 4 * self.N].view(dtype)
        if name in ("LS", "LC", "LX"):
            K = self.K1
        elif name in ("POWN", "PXL", "PXR", "PU", "PA", "POF"):
            K = self.K2
        else:
            return self.ws[off:off + 4 * M * self.N].view(dtype).view(M, self.N)
        return self.ws[off:off + 4 * M * self.N * K].view(dtype).view(M, self.N, K).permute(0, 2, 1)


_LAST_ALIF = None


def last_alif_run():
    return _LAST_ALIF


def _rho_pow_c(rho, C):
    """rho^C in fp32 exactly as the reference computes it (triton_alif.py:332)."""
    return float(torch.tensor(_f32(rho), dtype=torch.float32) ** C)


def _repair_arg(repair, M, stats):
    """The C entry's repair argument: -1 (ordered chain to convergence) for a converged repair
    whose round count nobody reads, else the Jacobi round budget."""
    repair = int(repair)
    if repair < 0:
        raise ValueError("repair must be >= 0")
    return -1 if (stats is None and repair >= M and M > 1) else repair


def alif_scan_forward(I, beta, rho, q, theta0, u_r, u0, w0, Wpred, dw, C=128, K1=16, K2=32, BN=16,
                      nw=1, BNc=1, BNr=32, D=4, repair=0, stats=None, phases=None):
    """Exact ALIF scan with a predicted adaptation box (triton_alif.py:301-358) -> (U, W, S).
    Wpred: [T//C, N] predicted entry adaptation (row 0 is replaced by w0); dw: box half-width.
    stats: repair_iters, miss_frac, overflow_frac, mean_lines, mean_pieces, max_pieces.
    phases: per-phase GPU times in ms (envelope, build, carry, replay).
    With the repair budget at least T//C (converged) and neither stats nor phases requested, the
    result is the serial recurrence and the serial forward computes it: the box scan's
    converged call ends in a serial pass from the first chunk whose start came through a map,
    which is all but the first few chunks (cfg5: 2.04 ms against 0.16 ms for the same bits).
    alif_scan_forward_maps runs the box-scan pipeline itself.  The arguments are checked as the
    pipeline checks them either way."""
    I = _input(I)
    T, N = I.shape
    M = _alif_scan_check(I, Wpred, C, K1, K2, D)
    if stats is None and phases is None and int(repair) >= M and M > 1:
        return alif_serial_forward(I, beta, rho, q, theta0, u_r, u0, w0)
    return alif_scan_forward_maps(I, beta, rho, q, theta0, u_r, u0, w0, Wpred, dw, C=C, K1=K1, K2=K2,
                                  BN=BN, nw=nw, BNc=BNc, BNr=BNr, D=D, repair=repair, stats=stats,
                                  phases=phases)


def _alif_scan_check(I, Wpred, C, K1, K2, D):
    """The box scan's argument checks (ValueError); returns the chunk count T // C."""
    T, N = I.shape
    C, K1, K2 = int(C), int(K1), int(K2)
    if C < 1 or T % C or C % int(D):
        raise ValueError(f"T={T} must be divisible by C={C} and C by D={D}")
    M = T // C
    if tuple(Wpred.shape) != (M, N):
        raise ValueError(f"Wpred must be [{M}, {N}]")
    if _n.lib().lsh_alif_scan_workspace(T, N, C, K1, K2) == 0:
        raise ValueError("ALIF scan needs K1 <= 32 and K2 <= 32 a power of two")
    return M


def alif_scan_forward_maps(I, beta, rho, q, theta0, u_r, u0, w0, Wpred, dw, C=128, K1=16, K2=32,
                           BN=16, nw=1, BNc=1, BNr=32, D=4, repair=0, stats=None, phases=None):
    """The box-scan pipeline of alif_scan_forward itself (envelope, box, chunk maps, verified
    carry, replay, device repair) -> (U, W, S), also where alif_scan_forward would compute its
    converged result by the serial forward.  With repair >= T//C (converged) and no stats, the
    repair is one ordered pass over each neuron's chunks (the replay below the first chunk whose
    start came through a map, then one serial pass from there): the same result, the serial
    recurrence, without the round count that stats would report.  For measuring the box scan."""
    global _LAST_ALIF
    I = _input(I)
    T, N = I.shape
    u0 = _vec(u0, N, I)
    w0 = _vec(w0, N, I, "w0")
    C, K1, K2, BN = int(C), int(K1), int(K2), int(BN)
    M = _alif_scan_check(I, Wpred, C, K1, K2, D)
    Wp = Wpred.detach().float().contiguous()
    L = _n.lib()
    nbytes = L.lsh_alif_scan_workspace(T, N, C, K1, K2)
    ws = _n.workspace(nbytes, I.device)
    U, W, S = torch.empty_like(I), torch.empty_like(I), torch.empty_like(I)
    evs, ev_arr = None, None
    if phases is not None:
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(5)]
        for e in evs:
            e.record()  # creates the underlying HIP event
        ev_arr = (_n.c_p * 5)(*[e.cuda_event for e in evs])
    with _n.on_device(I):
        _n.check(L.lsh_alif_scan_fwd(
            _n.ptr(I), _n.ptr(u0), _n.ptr(w0), _n.ptr(Wp), _f32(dw), _n.ptr(U), _n.ptr(W), _n.ptr(S),
            T, N, _f32(beta), _f32(rho), _f32(q), _f32(theta0), _f32(u_r), _rho_pow_c(rho, C), C, K1,
            K2, BN, _repair_arg(repair, M, stats), _n.ptr(ws), nbytes, ev_arr, _n.stream_of(I)),
            "lsh_alif_scan_fwd")
    _LAST_ALIF = _ALIFRun(ws, T, N, C, K1, K2)
    if phases is not None:
        torch.cuda.synchronize(I.device)
        for k, name in enumerate(("envelope", "build", "carry", "replay")):
            phases[name] = evs[k].elapsed_time(evs[k + 1])
    if stats is not None:
        st = _n.read_stats(ws, M * N, alif=True)
        stats["repair_iters"] = int(st.repair_iters)
        stats["miss_frac"] = float(st.miss_frac)
        stats["overflow_frac"] = float(st.overflow_frac)
        stats["mean_lines"] = float(st.mean_lines)
        stats["mean_pieces"] = float(st.mean_pieces)
        stats["max_pieces"] = int(st.max_pieces)
    return U, W, S


def alif_chunked_C(T, C=64):
    """Chunk of the chunked (four-pass) adjoint: the power of two in 16..512 dividing T nearest
    to sqrt(T/4), which balances the passes' per-chunk sweeps against the sequential carry over
    T/C chunks (swept on MI355X at N = 64..8192: best 32 at T = 4096, 128 at T = 65536, 256-512
    at T = 262144); the given C when none divides T."""
    cands = [c for c in (16, 32, 64, 128, 256, 512) if T % c == 0]
    if not cands:
        return int(C)
    target = math.sqrt(max(T, 1) / 4.0)
    return min(cands, key=lambda c: abs(math.log2(c / target)))


def _bwd_mode(mode, T, N, C):
    """Kernel mode code and chunk for an alif_backward mode name.  "scan": the single pass from
    ALIF_FUSED_BWD_MIN_N neurons; below that the look-back single pass when T is a multiple of
    ALIF_LOOKBACK_SEG, else the chunked passes at alif_chunked_C.  (The workgroup-per-64-neurons
    single pass is slow there: N = 1024, T = 65536: 2.99 ms against 1.44 ms chunked.)"""
    C = int(C)
    if mode == "scan":
        if N >= ALIF_FUSED_BWD_MIN_N and T % ALIF_FUSED_BWD_C == 0:
            mode, C = "fused", ALIF_FUSED_BWD_C
        elif ALIF_LOOKBACK and T % ALIF_LOOKBACK_SEG == 0:
            mode = "lookback"
        else:
            mode, C = "chunked", alif_chunked_C(T, C)
    if mode == "lookback":
        if T % ALIF_LOOKBACK_SEG:
            raise ValueError(f"T={T} must be divisible by {ALIF_LOOKBACK_SEG} for the look-back pass")
        return 3, 16
    if mode in ("serial_pf", "serial_tuned", "serial"):
        return 0, C
    if mode == "fused":  # single pass, C in {16, 32}
        return 2, C
    if mode == "chunked":
        if T % C:
            raise ValueError(f"T={T} must be divisible by C={C}")
        return 1, C
    raise ValueError(f"unknown mode {mode!r}")


def _alif_bwd_call(I, U, W, S, GS, beta, rho, q, theta0, u0, w0, alpha, mode, C, want_lw, want_params,
                   dp=None, recompute_ur=None):
    """One lsh_alif_bwd call -> (LV, LW or None, DW0 [N], param sums [4] fp64 or None); with dp
    (device [beta, rho, q, theta0]) the kernels read the parameters from it (lsh_alif_bwd_dparams)
    and beta, rho, q, theta0 are ignored.  recompute_ur (the reset value u_r) selects, when the
    mode resolves to a single pass (fused or look-back), lsh_alif_bwd_recompute: S is not read
    and U, W only at chunk boundaries, for U, W, S of one serial trajectory."""
    I = _input(I)
    T, N = I.shape
    u0 = _vec(u0, N, I)
    w0 = _vec(w0, N, I, "w0")
    U, W, GS = (_same(a, I, nm) for a, nm in ((U, "U"), (W, "W"), (GS, "GS")))
    code, C = _bwd_mode(mode, T, N, C)
    rc = recompute_ur is not None and code in (2, 3)
    if not rc:
        S = _same(S, I, "S")
    L = _n.lib()
    LV = torch.empty_like(I)
    LW = torch.empty_like(I) if (want_lw or code == 1) else None
    DW0 = torch.empty(N, device=I.device, dtype=torch.float32)
    parts = None
    if want_params:
        P = L.lsh_alif_bwd_partials(T, N, code, C)
        if P < 0:
            raise ValueError("bad backward shape")
        parts = torch.empty(max(P, 1), 4, device=I.device, dtype=torch.float64)
        if T == 0 or N == 0:
            parts.zero_()
    ws, nbytes = None, 0
    if code == 1:
        nbytes = L.lsh_alif_bwd_workspace(T, N, C)
        ws = _n.workspace(nbytes, I.device)
    elif code == 3:
        nbytes = L.lsh_alif_bwd_lookback_workspace(T, N)
        ws = _n.workspace(nbytes, I.device)
    with _n.on_device(I):
        if rc:
            p = (0.0,) * 4 if dp is not None else (beta, rho, q, theta0)
            _n.check(L.lsh_alif_bwd_recompute(
                _n.ptr(I), _n.ptr(U), _n.ptr(W), _n.ptr(GS), _n.ptr(u0), _n.ptr(w0), _n.ptr(LV),
                _n.ptr(LW), _n.ptr(DW0), _n.ptr(parts), T, N, _n.ptr(dp), *(_f32(v) for v in p),
                _f32(recompute_ur), _f32(alpha), code, C, _n.ptr(ws), nbytes, _n.stream_of(I)),
                "lsh_alif_bwd_recompute")
        elif dp is not None:
            _n.check(L.lsh_alif_bwd_dparams(
                _n.ptr(I), _n.ptr(U), _n.ptr(W), _n.ptr(S), _n.ptr(GS), _n.ptr(u0), _n.ptr(w0),
                _n.ptr(LV), _n.ptr(LW), _n.ptr(DW0), _n.ptr(parts), T, N, _n.ptr(dp), _f32(alpha), code,
                C, _n.ptr(ws), nbytes, _n.stream_of(I)), "lsh_alif_bwd_dparams")
        else:
            _n.check(L.lsh_alif_bwd(
                _n.ptr(I), _n.ptr(U), _n.ptr(W), _n.ptr(S), _n.ptr(GS), _n.ptr(u0), _n.ptr(w0),
                _n.ptr(LV), _n.ptr(LW), _n.ptr(DW0), _n.ptr(parts), T, N, _f32(beta), _f32(rho),
                _f32(q), _f32(theta0), _f32(alpha), code, C, _n.ptr(ws), nbytes, _n.stream_of(I)),
                "lsh_alif_bwd")
    global _LAST_BWD_WS
    _LAST_BWD_WS = ws
    sums = parts.sum(0) if parts is not None else None
    return LV, (LW if want_lw else None), DW0, sums


_LAST_BWD_WS = None


def last_bwd_spin_timeouts():
    """Bounded waits that gave up in the last look-back adjoint (0 when its result is valid)."""
    if _LAST_BWD_WS is None:
        return 0
    return int(_n.read_stats(_LAST_BWD_WS, 1).spin_timeouts)


def alif_backward(I, U, W, S, GS, beta, rho, q, theta0, u0, w0, alpha=4.0, mode="scan", C=64,
                  BN=32, D=4, nw=1):
    """(LV, LW) with LV[t] = dL/dv_t (= dL/dI_t), LW[t] = dL/dw_t for dL/dS = GS
    (triton_alif.py:490-521).  mode: serial_pf / serial_tuned / serial (fused serial sweep),
    chunked (two-level affine scans over chunks of C), fused (single pass, C in {16, 32}),
    lookback (single pass with look-back across workgroups, T % 128 == 0) or scan (fused when N
    is large, else lookback or chunked; _bwd_mode)."""
    LV, LW, _, _ = _alif_bwd_call(I, U, W, S, GS, beta, rho, q, theta0, u0, w0, alpha, mode, C,
                                  want_lw=True, want_params=False)
    return LV, LW


class ALIFFn(torch.autograd.Function):
    """S = ALIF(I; u0, w0, beta, rho, q, theta0) with u_r fixed (triton_alif.py:524-554).
    Forward: serial, or the box scan with prediction Wpred (K1 = K2 = 32, block 4, no repair,
    as the reference); backward: serial or scan.  Gradients for I, u0, w0, beta, rho, q, theta0:
    the adjoint kernels also return dL/dw0 and the four parameter sums (fp64), so LW is never
    written to memory.  Parameters may be floats or 0-d tensors; with the serial forward, device
    tensors stay on the device (the kernels read them there, no host synchronization), while the
    box scan reads them on the host as the reference does (triton_alif.py:530)."""

    @staticmethod
    def forward(ctx, I, u0, w0, beta, rho, q, theta0, u_r, alpha, fwd, bwd, Wpred, dw, C, Cb):
        ctx.set_materialize_grads(False)  # U and W usually get no gradient: no zero fills
        dp = _dev_params(I, beta, rho, q, theta0) if fwd == "serial" else None
        ctx.dp = dp
        if dp is not None:
            b = r = qq = th = None
            U, W, S = _alif_serial_forward_dp(I, dp, u_r, u0, w0)
        elif fwd == "serial":
            b, r, qq, th = _f32s(beta, rho, q, theta0)
            U, W, S = alif_serial_forward(I, b, r, qq, th, u_r, u0, w0)
        else:
            b, r, qq, th = _f32s(beta, rho, q, theta0)
            U, W, S = alif_scan_forward(I, b, r, qq, th, u_r, u0, w0, Wpred, dw, C=C, K1=32, K2=32,
                                        BN=4, BNc=1, D=4)
        ctx.save_for_backward(I, u0, w0, U, W, S)
        ctx.c = (b, r, qq, th, u_r, alpha, bwd, Cb)
        ctx.serial = fwd == "serial"
        ctx.mark_non_differentiable(U, W)
        return S, U, W

    @staticmethod
    def backward(ctx, gS, gU, gW):
        if gS is None:  # S took no part in the loss
            return (None,) * 15
        I, u0, w0, U, W, S = ctx.saved_tensors
        b, r, qq, th, u_r, alpha, bwd, Cb = ctx.c
        need = ctx.needs_input_grad
        want_params = any(need[3:7])
        dp = ctx.dp
        LV, _, DW0, sums = _alif_bwd_call(I, U, W, S, gS.contiguous(), b, r, qq, th, u0, w0, alpha,
                                          "serial_tuned" if bwd == "serial" else bwd, Cb,
                                          want_lw=False, want_params=want_params, dp=dp,
                                          recompute_ur=u_r if ctx.serial and ALIF_RECOMPUTE_BWD else None)
        db = dr = dq = dth = None
        if sums is not None:  # a gradient only for the parameters given as tensors
            sums = sums.float()
            db, dr, dq = (sums[k] if need[3 + k] else None for k in range(3))
            dth = -sums[3] if need[6] else None
        du0 = (dp[0] if dp is not None else b) * LV[0] if need[1] else None
        return (LV, du0, DW0.reshape(w0.shape) if w0.dim() else DW0, db, dr, dq, dth,
                None, None, None, None, None, None, None, None)


def alif(I, u0, w0, beta, rho, q, theta0=1.0, u_r=0.0, alpha=4.0, fwd="serial", bwd="scan",
         Wpred=None, dw=None, C=128, Cb=64):
    """Differentiable ALIF layer -> (S, U, W) (triton_alif.py:557-560).  Parameters may be
    0-d tensors (requires_grad) or floats; floats are passed to the kernels as they are (the
    reference wraps them in device tensors and reads them back, the same fp32 values)."""
    return ALIFFn.apply(I, u0, w0, beta, rho, q, theta0, u_r, alpha, fwd, bwd, Wpred, dw, C, Cb)
