"""LIF with an affine reset u <- gamma*v + delta (0 <= gamma <= 1) on MI355X, with the call
signatures of the reference's ``lifscan/triton_affine.py``:

    v = beta*u + I_t;  s = [v >= theta];  u <- gamma*v + delta if s else v

gamma = 0, delta = u_r is the hard reset, gamma = 1, delta = -theta the soft reset.  Serial
forward, the exact two-level scan (envelopes, chunk maps of unsorted pieces, verified carry,
replay, device repair) and the adjoint with the gradients for I, u0, beta, gamma and delta, all
in hand-written HIP kernels of liblifscan_hip.so.  Triton tile keywords (BN, BNc, BNr) are
accepted and ignored.
"""
import torch

from . import _native as _n
from . import hip_lif as L
from .hip_lif import _f32, _f32s, _input, _vec, _same


def _gamma(g):
    g = float(g)
    if not 0.0 <= g <= 1.0:
        raise ValueError(f"gamma={g} must lie in [0, 1]")
    return g


def aff_serial_forward(I, beta, theta, gamma, delta, u0, BN=32):
    """Serial affine-reset LIF (triton_affine.py:158-162) -> (U, S)."""
    I = _input(I)
    T, N = I.shape
    u0 = _vec(u0, N, I)
    U, S = torch.empty_like(I), torch.empty_like(I)
    if I.numel() == 0:
        _gamma(_f32(gamma))
        return U, S
    with _n.on_device(I):
        _n.check(_n.lib().lsh_aff_serial_fwd(
            _n.ptr(I), _n.ptr(u0), _n.ptr(U), _n.ptr(S), T, N, _f32(beta), _f32(theta),
            _gamma(_f32(gamma)), _f32(delta), _n.stream_of(I)), "lsh_aff_serial_fwd")
    return U, S


class _AffRun:
    """Workspace of one scan call (envelopes, maps, chunk states) for stats and tests."""

    def __init__(self, ws, T, N, C, K):
        self.ws, self.T, self.N, self.C, self.K = ws, T, N, C, K

    def view(self, name, dtype=torch.float32):
        """[M, N] arrays; PIECES as [M, N, K, 4] (xl, xr, a, c)."""
        lay = _n.AffLayout()
        _n.check(_n.lib().lsh_aff_scan_layout(self.T, self.N, self.C, self.K, _n.ctypes.byref(lay)),
                 "lsh_aff_scan_layout")
        M = self.T // self.C
        off = getattr(lay, name)
        if name == "PIECES":
            return self.ws[off:off + 16 * M * self.N * self.K].view(torch.float32).view(
                M, self.N, self.K, 4)
        return self.ws[off:off + 4 * M * self.N].view(dtype).view(M, self.N)


_LAST_AFF = None


def last_aff_run():
    return _LAST_AFF


def aff_scan_forward(I, beta, theta, gamma, delta, u0, C=128, K=32, BN=16, BNc=16, BNr=32, repair=0,
                     stats=None):
    """Exact affine-reset scan (triton_affine.py:165-199) -> (U, S).  With repair the result is
    bit-identical to aff_serial_forward.  stats: repair_iters, overflow_frac, mean_pieces."""
    global _LAST_AFF
    I = _input(I)
    T, N = I.shape
    u0 = _vec(u0, N, I)
    C, K = int(C), int(K)
    b, th, g, d = _f32s(beta, theta, gamma, delta)
    g = _gamma(g)
    if C < 1 or T % C:
        raise ValueError(f"T={T} must be divisible by C={C}")
    lib = _n.lib()
    if I.numel() == 0:  # nothing to run; the statistics of an empty map set are those of torch
        if not 1 <= K <= 32:
            raise ValueError(f"affine scan needs 1 <= K <= 32 (K={K})")
        if stats is not None:
            stats.update(repair_iters=0, overflow_frac=float("nan"), mean_pieces=float("nan"))
        return torch.empty_like(I), torch.empty_like(I)
    nbytes = lib.lsh_aff_scan_workspace(T, N, C, K)
    if nbytes == 0:
        raise ValueError(f"affine scan needs 1 <= K <= 32 (K={K})")
    ws = _n.workspace(nbytes, I.device)
    U, S = torch.empty_like(I), torch.empty_like(I)
    r_theta = g * th + d  # in double from the Python floats, as the reference (:171)
    with _n.on_device(I):
        _n.check(lib.lsh_aff_scan_fwd(
            _n.ptr(I), _n.ptr(u0), _n.ptr(U), _n.ptr(S), T, N, b, th, g, d, r_theta, C, K,
            int(repair), _n.ptr(ws), nbytes, _n.stream_of(I)), "lsh_aff_scan_fwd")
    _LAST_AFF = _AffRun(ws, T, N, C, K)
    if stats is not None:
        st = _n.read_stats(ws, (T // C) * N, alif=2)
        stats["repair_iters"] = int(st.repair_iters)
        stats["overflow_frac"] = float(st.overflow_frac)
        stats["mean_pieces"] = float(st.mean_pieces)
    return U, S


def reverse_affine_scan(a, b):
    """lam_t = a_t*lam_{t+1} + b_t, lam_T = 0 over dim 0 (triton_affine.py:202-211)."""
    a = _input(a)
    b = _same(b, a, "b")
    T, N = a.shape
    out = torch.empty_like(a)
    with _n.on_device(a):
        _n.check(_n.lib().lsh_reverse_affine_scan(_n.ptr(a), _n.ptr(b), _n.ptr(out), T, N,
                                                  _n.stream_of(a)), "lsh_reverse_affine_scan")
    return out


def _aff_backward(I, u0, U, S, GS, beta, theta, gamma, alpha, mode="auto", C=None):
    """lsh_aff_bwd -> (Lam, sums [3] fp64: sum lam*u_{t-1}, sum s*v*lam_{t+1}, sum s*lam_{t+1}).
    mode "auto" picks the adjoint by shape as the LIF scan adjoint does; "serial", "chunked",
    "fused" and "lookback" force one."""
    I = _input(I)
    T, N = I.shape
    u0 = _vec(u0, N, I)
    U, S, GS = (_same(a, I, nm) for a, nm in ((U, "U"), (S, "S"), (GS, "GS")))
    if mode == "auto":
        if N >= L.FUSED_BWD_MIN_N and T % L.FUSED_BWD_C == 0:
            mode = "fused"
        elif L.LOOKBACK_BWD and T % L.LOOKBACK_SEG == 0:
            mode = "lookback"
        elif T >= L.AUTO_BWD_MIN_T:
            mode = "chunked"
        else:
            mode = "serial"
    if mode == "fused":
        code, C = 2, int(C or L.FUSED_BWD_C)
    elif mode == "lookback":
        code, C = 3, 16
    elif mode == "chunked":
        code, C = 1, int(C or L.chunked_bwd_C(T, N, min(128, L._pick_C(T, D=2))))
    elif mode == "serial":
        code, C = 0, 1
    else:
        raise ValueError(f"unknown mode {mode!r}")
    lib = _n.lib()
    P = lib.lsh_lif_param_partials(T, N, code, C)
    if P < 0:
        raise ValueError(f"T={T} must be divisible by C={C}")
    parts = torch.zeros(max(P, 1), 3, device=I.device, dtype=torch.float64)
    Lam = torch.empty_like(I)
    ws, nbytes = None, 0
    if code == 1:
        nbytes = lib.lsh_lif_scan_bwd_workspace(T, N, C)
        ws = _n.workspace(nbytes, I.device)
    elif code == 3:
        nbytes = lib.lsh_lif_scan_lookback_bwd_workspace(T, N)
        ws = _n.workspace(nbytes, I.device)
    with _n.on_device(I):
        _n.check(lib.lsh_aff_bwd(
            _n.ptr(I), _n.ptr(u0), _n.ptr(U), _n.ptr(S), _n.ptr(GS), _n.ptr(Lam), _n.ptr(parts), T, N,
            _f32(beta), _f32(theta), _gamma(_f32(gamma)), _f32(alpha), code, C, _n.ptr(ws), nbytes,
            _n.stream_of(I)), "lsh_aff_bwd")
    return Lam, parts.sum(0)


class LIFAffineFn(torch.autograd.Function):
    """Affine-reset LIF; gradients w.r.t. I, u0, beta, gamma, delta with the spike detached in
    the reset and the sigmoid surrogate (triton_affine.py:214-242).  The three parameter sums
    are accumulated in fp64 inside the adjoint kernel."""

    @staticmethod
    def forward(ctx, I, u0, beta, gamma, delta, theta, alpha, mode, C, K):
        b, g, dl, th = _f32s(beta, gamma, delta, theta)
        I = I.contiguous()
        if mode == "scan":
            U, S = aff_scan_forward(I, b, th, g, dl, u0, C=C, K=K)
        else:
            U, S = aff_serial_forward(I, b, th, g, dl, u0)
        ctx.save_for_backward(I, u0, U, S)
        ctx.cfg = (b, g, dl, th, float(alpha))
        return S

    @staticmethod
    def backward(ctx, gS):
        I, u0, U, S = ctx.saved_tensors
        b, g, dl, th, alpha = ctx.cfg
        lam, sums = _aff_backward(I, u0, U, S, gS.contiguous(), b, th, g, alpha)
        need = ctx.needs_input_grad
        grads = (sums[0], b * sums[1], b * sums[2])
        db, dg, dd = (grads[k].float().reshape(()) if need[2 + k] else None for k in range(3))
        return (lam, b * lam[0] if need[1] else None, db, dg, dd, None, None, None, None, None)


def lif_affine(I, u0, beta, gamma, delta, theta=1.0, alpha=4.0, mode="scan", C=128, K=32):
    """triton_affine.py:245-246: spikes S [T, N]; mode "scan" (the two-level scan with the
    reference's default repair = 0: chunk starts from the verified maps, serial fallback on a
    miss) or "serial"."""
    return LIFAffineFn.apply(I, u0, beta, gamma, delta, theta, alpha, mode, C, K)
