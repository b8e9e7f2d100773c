"""Differentiable hard-reset LIF with gradients w.r.t. the neuron parameters (beta, theta,
u_r), the interface of the reference's ``lifscan/fit.py`` (LIFParamFn, lif_param):

    dL/dbeta  = sum_t lambda_t u_{t-1}
    dL/dtheta = -sum_t gS_t sigma'(v_t - theta)           (detached reset)
    dL/du_r   = sum_t s_t beta lambda_{t+1}

with lambda_t = dL/dv_t from the adjoint.  The three sums are accumulated in fp64 inside the
adjoint kernel (lsh_lif_param_bwd), one row per block, so no [T, N] temporaries are formed.

The soft-reset layers (LIFSoftFn / lif_soft, LIFSoftScanFn / lif_soft_scan, fit.py:93-153) give
gradients for I, u0 and beta; their adjoint is lsh_soft_bwd (float64 recurrence, dbeta summed in
the kernel).  The reference's CPU prototype backend (LIFParamFnCPU) is not part of this package.
"""
import torch

from . import _native as _n
from . import hip_lif as L
from .hip_lif import _f32, _f32s, _input, _vec, _same


def _param_backward(I, u0, U, S, GS, beta, theta, u_r, alpha, mode):
    """lsh_lif_param_bwd -> (Lam, sums [3] fp64)."""
    I = _input(I)
    T, N = I.shape
    u0 = _vec(u0, N, I)
    U, S, GS = (_same(a, I, nm) for a, nm in ((U, "U"), (S, "S"), (GS, "GS")))
    lib = _n.lib()
    if mode == "scan":
        if N >= L.FUSED_BWD_MIN_N and T % L.FUSED_BWD_C == 0:
            code, C = 2, L.FUSED_BWD_C
        elif L.LOOKBACK_BWD and T % L.LOOKBACK_SEG == 0:
            code, C = 3, 16
        else:
            code, C = 1, L.chunked_bwd_C(T, N, min(128, L._pick_C(T, D=2)))
    else:
        code, C = 0, 1
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
        _n.check(lib.lsh_lif_param_bwd(
            _n.ptr(I), _n.ptr(u0), _n.ptr(U), _n.ptr(S), _n.ptr(GS), _n.ptr(Lam), _n.ptr(parts), T, N,
            _f32(beta), _f32(theta), _f32(u_r), _f32(alpha), code, C, _n.ptr(ws), nbytes,
            _n.stream_of(I)), "lsh_lif_param_bwd")
    return Lam, parts.sum(0)


class LIFParamFn(torch.autograd.Function):
    """S = LIF(I; u0, beta, theta, u_r) with gradients for I, u0 and the three parameters
    (fit.py:15-48).  fwd_mode / bwd_mode: "serial" or "scan"."""

    @staticmethod
    def forward(ctx, I, u0, beta, theta, u_r, alpha, fwd_mode, bwd_mode, K):
        b, th, ur = _f32s(beta, theta, u_r)
        I = I.contiguous()
        ctx.cfg = (b, th, ur, float(alpha), bwd_mode)
        T, N = I.shape
        # the serial forward's bits are the single-pass exact forward's: with the single-pass
        # adjoint behind it, keep the chunk entry states instead of U (same S and gradients)
        if fwd_mode == "serial" and bwd_mode == "scan" and L._recompute_ok(T, N, K, T):
            S, ST = L.scan_forward_exact_starts(I, b, th, ur, u0)
            ctx.save_for_backward(I, u0, ST)
            ctx.recompute = True
            return S
        if fwd_mode == "scan":
            U, S = L.scan_forward_auto(I, b, th, ur, u0, K=K)
        else:
            U, S = L.serial_forward_auto(I, b, th, ur, u0)
        ctx.save_for_backward(I, u0, U, S)
        ctx.recompute = False
        return S

    @staticmethod
    def backward(ctx, gS):
        b, th, ur, alpha, bwd_mode = ctx.cfg
        if ctx.recompute:
            I, u0, ST = ctx.saved_tensors
            lam, sums = L.scan_backward_fused_starts(I, ST, gS.contiguous(), b, th, ur, alpha, True)
        else:
            I, u0, U, S = ctx.saved_tensors
            lam, sums = _param_backward(I, u0, U, S, gS.contiguous(), b, th, ur, alpha, bwd_mode)
        sums = sums.float()
        need = ctx.needs_input_grad  # a gradient only for the parameters given as tensors
        du0 = b * lam[0] if ctx.needs_input_grad[1] else None
        return (lam, du0, sums[0] if need[2] else None, -sums[1] if need[3] else None,
                b * sums[2] if need[4] else None, None, None, None, None)


def lif_param(I, u0, beta, theta, u_r, alpha=4.0, mode="auto", K=16):
    """fit.py:51-57: mode "auto" picks serial / scan per pass from (N, T).  Parameters may be
    0-d tensors or floats; floats go to the kernels as they are (the reference wraps them in
    device tensors and reads them back: the same fp32 values, one synchronizing copy more)."""
    T, N = I.shape
    if mode == "auto":
        fwd, bwd = L.auto_modes(N, T)
    else:
        fwd = bwd = mode
    return LIFParamFn.apply(I, u0, beta, theta, u_r, alpha, fwd, bwd, K)


class LIFSoftFn(torch.autograd.Function):
    """Soft (subtractive) reset LIF, serial forward; gradients for I, u0, beta (fit.py:93-114)."""

    @staticmethod
    def forward(ctx, I, u0, beta, theta, alpha):
        from . import hip_soft as TS
        b, th = _f32s(beta, theta)
        I = I.contiguous()
        U, S = TS.soft_serial_forward(I, b, th, u0)
        ctx.save_for_backward(I, u0, U)
        ctx.cfg = (b, th, float(alpha))
        return S

    @staticmethod
    def backward(ctx, gS):
        from . import hip_soft as TS
        I, u0, U = ctx.saved_tensors
        b, th, alpha = ctx.cfg
        need_b = ctx.needs_input_grad[2]
        lam, db = TS._soft_backward(I, u0, U, gS.contiguous(), b, th, alpha, need_b)
        du0 = b * lam[0] if ctx.needs_input_grad[1] else None
        return lam, du0, (db.float().reshape(()) if need_b else None), None, None


def lif_soft(I, u0, beta, theta=1.0, alpha=4.0):
    """fit.py:117-118."""
    return LIFSoftFn.apply(I, u0, beta, theta, alpha)


class LIFSoftScanFn(torch.autograd.Function):
    """Soft-reset LIF with the exact soft scan forward (mode "scan", the reference's default
    repair = 0) or the serial forward; the adjoint is the float64 recurrence in both modes (the
    reference: FFT convolution for "scan", the fp32 serial sweep otherwise); gradients for I,
    u0, beta (fit.py:121-149)."""

    @staticmethod
    def forward(ctx, I, u0, beta, theta, alpha, mode, C, K):
        from . import hip_soft as TS
        b, th = _f32s(beta, theta)
        I = I.contiguous()
        if mode == "scan":
            U, S = TS.soft_scan_forward(I, b, th, u0, C=C, K=K)
        else:
            U, S = TS.soft_serial_forward(I, b, th, u0)
        ctx.save_for_backward(I, u0, U)
        ctx.cfg = (b, th, float(alpha))
        return S

    @staticmethod
    def backward(ctx, gS):
        from . import hip_soft as TS
        I, u0, U = ctx.saved_tensors
        b, th, alpha = ctx.cfg
        need_b = ctx.needs_input_grad[2]
        lam, db = TS._soft_backward(I, u0, U, gS.contiguous(), b, th, alpha, need_b)
        du0 = b * lam[0] if ctx.needs_input_grad[1] else None
        return (lam, du0, (db.float().reshape(()) if need_b else None), None, None, None, None,
                None)


def lif_soft_scan(I, u0, beta, theta=1.0, alpha=4.0, mode="scan", C=128, K=32):
    """fit.py:152-153."""
    return LIFSoftScanFn.apply(I, u0, beta, theta, alpha, mode, C, K)
