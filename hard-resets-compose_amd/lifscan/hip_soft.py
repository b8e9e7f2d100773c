"""Soft-reset LIF (u <- v - theta) on MI355X with the call signatures of the reference's
``lifscan/triton_soft.py`` and the soft serial functions of ``lifscan/triton_lif.py``:

    v = beta*u + I_t;  s = [v >= theta];  u <- v - theta if s else v

The forward runs the affine-reset kernels with gamma = 1, delta = -theta: fl(fl(1*v) - theta)
is the reference's single rounding fl(v - theta), and the soft scan's common-slope maps are the
affine maps whose slopes all equal beta^j (the CPU pins in tests/test_oracle_soft.py show the two
restatements agree bit for bit).  The adjoint with the reset detached is the constant-
coefficient recurrence lam_t = b_t + beta*lam_{t+1}; the reference solves it by a float64 FFT
convolution (soft_adjoint_fft), here a HIP kernel solves the same recurrence directly in float64
(lsh_soft_bwd).  Triton tile keywords are accepted and ignored.
"""
import math

import torch

from . import _native as _n
from . import hip_affine as _AF
from .hip_lif import _f32, _f32s, _input, _vec, _same, soft_bwd_cfg  # noqa: F401


def soft_serial_forward(I, beta, theta, u0, BN=32):
    """Serial soft-reset LIF (triton_soft.py:168-172, triton_lif.py:1072-1076) -> (U, S)."""
    b, th = _f32s(beta, theta)
    return _AF.aff_serial_forward(I, b, th, 1.0, -th, u0)


def soft_serial_forward_tiled(I, beta, theta, u0, BN=32, D=8, num_warps=1):
    """triton_soft.py:250-254: bit-identical to soft_serial_forward (one kernel here)."""
    return soft_serial_forward(I, beta, theta, u0)


def soft_scan_forward(I, beta, theta, u0, C=32, K=16, BN=16, nw=1, BNc=16, BNr=32, repair=0,
                      stats=None):
    """Exact soft-reset scan (triton_soft.py:175-211) -> (U, S); with repair bit-identical to
    the serial forward.  stats: repair_iters, overflow_frac, mean_pieces, max_pieces."""
    b, th = _f32s(beta, theta)
    st = {} if stats is not None else None
    U, S = _AF.aff_scan_forward(I, b, th, 1.0, -th, u0, C=C, K=K, repair=repair, stats=st)
    if stats is not None:
        stats.update(st)
        run = _AF.last_aff_run()
        if I.numel() and run is not None:
            st2 = _n.read_stats(run.ws, (run.T // run.C) * run.N, alif=2)
            stats["max_pieces"] = int(st2.max_pieces)
        else:
            stats["max_pieces"] = 0
    return U, S


def _soft_C(T, N, target_blocks=2048, min_C=32):
    """Chunk length of the soft adjoint: one sweep per neuron when the 64-neuron blocks alone
    fill the chip; otherwise the smallest divisor of T of at least T*NB/target_blocks steps (about
    target_blocks (chunk, block) pairs) and at least max(min_C, sqrt(T)) steps, so that the
    sequential carry over chunks stays short."""
    NB = (N + 63) // 64
    if T == 0 or NB >= target_blocks:
        return max(T, 1)
    want = max(min_C, math.isqrt(T), T * NB // target_blocks)
    for C in range(min(want, T), T + 1):
        if T % C == 0:
            return C
    return T


def _soft_call(I, u0, U, V, GS, beta, theta, alpha, want_dbeta):
    like = V if V is not None else I
    like = _input(like)
    T, N = like.shape
    GS = _same(GS, like, "GS")
    Lam = torch.empty_like(like)
    if like.numel() == 0:
        return Lam, torch.zeros((), dtype=torch.float64, device=like.device)
    C = _soft_C(T, N)
    lib = _n.lib()
    nbytes = lib.lsh_soft_bwd_workspace(T, N, C)
    ws = _n.workspace(nbytes, like.device)
    parts = None
    if want_dbeta:
        parts = torch.zeros(max(lib.lsh_soft_bwd_partials(T, N, C), 1), dtype=torch.float64,
                            device=like.device)
    with _n.on_device(like):
        _n.check(lib.lsh_soft_bwd(
            _n.ptr(I), _n.ptr(u0), _n.ptr(U), _n.ptr(V), _n.ptr(GS), _n.ptr(Lam), _n.ptr(parts), T, N,
            float(beta), _f32(theta), _f32(alpha), C, _n.ptr(ws), nbytes, _n.stream_of(like)),
            "lsh_soft_bwd")
    return Lam, (parts.sum() if want_dbeta else None)


def soft_adjoint_fft(V, gS, beta, theta, alpha=4.0):
    """lam_t = b_t + beta*lam_{t+1}, b_t = gS_t*sigma'(V_t - theta) (detached soft reset;
    triton_soft.py:214-221): the float64 value of the reference's FFT convolution, by a direct
    float64 recurrence on the device, returned in V's dtype (fp32)."""
    V = _input(V)
    return _soft_call(None, None, None, V, gS, beta, theta, alpha, False)[0]


def _soft_backward(I, u0, U, GS, beta, theta, alpha, want_dbeta=True):
    """Adjoint from I, u0, U (v recomputed as the forward computes it) -> (Lam, dbeta fp64)."""
    I = _input(I)
    T, N = I.shape
    u0 = _vec(u0, N, I)
    U = _same(U, I, "U")
    return _soft_call(I, u0, U, None, GS, beta, theta, alpha, want_dbeta)


def soft_serial_backward(I, u0, U, GS, beta, theta, alpha=4.0, BN=32):
    """Soft-reset adjoint (triton_lif.py:1052-1069, :1079-1083) -> Lam."""
    return _soft_backward(I, u0, U, GS, beta, theta, alpha, False)[0]


def soft_serial_backward_pf(I, u0, U, GS, beta, theta, alpha=4.0, BN=32, D=4, num_warps=1):
    """triton_lif.py:1139-1180 (prefetching variant of the same sweep)."""
    return soft_serial_backward(I, u0, U, GS, beta, theta, alpha)


def soft_serial_backward_auto(I, u0, U, GS, beta, theta, alpha=4.0):
    """triton_lif.py:1206-1210."""
    return soft_serial_backward(I, u0, U, GS, beta, theta, alpha)
