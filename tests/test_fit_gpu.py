"""GPU: lif_param (fit.py LIFParamFn) gradients for I, u0, beta, theta, u_r against the fp64
assembly of the oracle (oracle/lif_oracle.py param_grads, pinned against fp64 autograd), in the
reference's own configuration (tests/test_fit_grad.py: T=4096, N=64, I = 0.5 x + 0.08, bar 1e-3)
and on ragged shapes that take the chunked scan.  Tensor gradients at 1e-4."""
import numpy as np
import pytest
import torch

from oracle import lif_oracle as O
from tests._inputs import gpu, host, normal, uniform

pytestmark = pytest.mark.gpu


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("mode", ["serial", "scan"])
@pytest.mark.parametrize("T,N", [(4096, 64), (1008, 100), (2048, 9000)])
def test_lif_param_gradients(dev, mode, T, N):
    from lifscan.fit import lif_param
    beta, theta, u_r = 0.93, 1.0, -0.1
    x = normal(T, N, 0.0, 1.0, 41)
    W = normal(T, N, 0.0, 1.0, 42)
    I = (np.float32(0.5) * x + np.float32(0.08)).astype(np.float32)
    u0 = np.zeros(N, np.float32)
    print(f"lif_param {mode} T={T} N={N}", flush=True)
    Ig = gpu(I, dev).requires_grad_(True)
    ug = gpu(u0, dev).requires_grad_(True)
    ps = [torch.tensor(v, device=dev, requires_grad=True) for v in (beta, theta, u_r)]
    S = lif_param(Ig, ug, *ps, mode=mode)
    (gpu(W, dev) * S).sum().backward()
    if mode == "scan":  # the scan forward runs without repair (fit.py:21): spikes from it
        Uo, So = O.scan_forward_v3(I, beta, theta, u_r, u0, C=O.pick_C(T, 16), K=16, repair=0)
    else:
        Uo, So = O.serial_forward(I, beta, theta, u_r, u0)
    assert np.array_equal(host(S), So)
    Lam = O.serial_backward(I, u0, Uo, So, W, None, beta, theta, u_r, 4.0, True, dtype=np.float64)
    want = O.param_grads(I, u0, Uo, So, W, Lam, beta, theta, u_r, 4.0)
    assert rel(host(Ig.grad), want[0]) < 1e-4
    assert rel(host(ug.grad), want[1]) < 1e-4
    for k, p in enumerate(ps):
        assert rel(p.grad.item(), want[2 + k]) < 1e-4, k


@pytest.mark.parametrize("mode,C", [(0, 1), (1, 16), (1, 64), (2, 16), (2, 32), (2, 64), (3, 16)])
def test_lif_param_partials(dev, mode, C):
    """lsh_lif_param_bwd directly: Lam and the three column sums of the per-block rows."""
    from lifscan import _native as nat
    T, N = 1024, 200
    beta, theta, u_r = 0.9, 1.0, 0.0
    I = normal(T, N, 0.12, 0.25, 43)
    GS = normal(T, N, 0.0, 1.0, 44)
    u0 = np.zeros(N, np.float32)
    U, S = O.serial_forward(I, beta, theta, u_r, u0)
    lib = nat.lib()
    P = lib.lsh_lif_param_partials(T, N, mode, C)
    nb = (N + 63) // 64
    assert P == {1: (T // C) * nb, 3: (T // 256) * nb}.get(mode, nb)
    parts = torch.full((P, 3), float("nan"), device=dev, dtype=torch.float64)
    Lam = torch.empty(T, N, device=dev)
    ws, nb = None, 0
    if mode == 1:
        nb = lib.lsh_lif_scan_bwd_workspace(T, N, C)
        ws = nat.workspace(nb, dev)
    elif mode == 3:
        nb = lib.lsh_lif_scan_lookback_bwd_workspace(T, N)
        ws = nat.workspace(nb, dev)
    args = [gpu(a, dev) for a in (I, u0, U, S, GS)]
    print(f"lif_param_bwd mode={mode} C={C}", flush=True)
    nat.check(lib.lsh_lif_param_bwd(*[nat.ptr(a) for a in args], nat.ptr(Lam), nat.ptr(parts), T, N, beta,
                                    theta, u_r, 4.0, mode, C, nat.ptr(ws), nb, nat.stream_of(Lam)), "param")
    sums = host(parts.sum(0))
    Lo = O.serial_backward(I, u0, U, S, GS, None, beta, theta, u_r, 4.0, True, dtype=np.float64)
    want = O.param_grads(I, u0, U, S, GS, Lo, beta, theta, u_r, 4.0)
    assert rel(host(Lam), Lo) < 1e-4
    assert rel(sums[0], want[2]) < 1e-4
    assert rel(-sums[1], want[3]) < 1e-4
    assert rel(beta * sums[2], want[4]) < 1e-4


def test_lif_param_auto_recomputing_path(dev):
    """mode="auto" at N = 16384: serial forward and scan adjoint, which lif_param runs as the
    recomputing pair; S, dI, du0 equal the stored path's, the parameter gradients agree to
    fp64 summation order, and both match the fp64 assembly."""
    from lifscan import hip_lif as L
    from lifscan.fit import lif_param
    T, N = 1024, 16384
    beta, theta, u_r = 0.93, 1.0, -0.1
    I = (np.float32(0.5) * normal(T, N, 0.0, 1.0, 51) + np.float32(0.08)).astype(np.float32)
    W = normal(T, N, 0.0, 1.0, 52)
    res = []
    for rc in (True, False):
        L.RECOMPUTE_BWD = rc
        try:
            Ig = gpu(I, dev).requires_grad_(True)
            ug = torch.zeros(N, device=dev, requires_grad=True)
            ps = [torch.tensor(v, device=dev, requires_grad=True) for v in (beta, theta, u_r)]
            S = lif_param(Ig, ug, *ps, mode="auto")
            (gpu(W, dev) * S).sum().backward()
            res.append((S.detach(), Ig.grad, ug.grad, [p.grad.item() for p in ps]))
        finally:
            L.RECOMPUTE_BWD = True
    (S1, g1, u1, p1), (S2, g2, u2, p2) = res
    assert torch.equal(S1, S2) and torch.equal(g1, g2) and torch.equal(u1, u2)
    for a, b in zip(p1, p2):
        assert abs(a - b) <= 1e-6 * abs(b)
    u0 = np.zeros(N, np.float32)
    Uo, So = O.serial_forward(I, beta, theta, u_r, u0)
    assert np.array_equal(host(S1), So)
    Lam = O.serial_backward(I, u0, Uo, So, W, None, beta, theta, u_r, 4.0, True, dtype=np.float64)
    want = O.param_grads(I, u0, Uo, So, W, Lam, beta, theta, u_r, 4.0)
    assert rel(host(g1), want[0]) < 1e-4
    for k in range(3):
        assert rel(p1[k], want[2 + k]) < 1e-4, k


@pytest.mark.parametrize("mode", ["serial", "scan"])
def test_lif_param_float_and_tensor_params_agree(dev, mode):
    """lif_param with float parameters, with 0-d tensors and with a mix: the same S bit for bit and
    the same input gradients bit for bit; parameter gradients
    only for the tensors, equal to the all-tensor call's."""
    from lifscan.fit import lif_param
    T, N = 512, 96
    I = gpu(normal(T, N, 0.12, 0.3, 81), dev)
    G = gpu(normal(T, N, 0.0, 1.0, 82), dev)
    u0 = gpu(uniform(N, 0.0, 0.5, 83), dev)
    print(f"lif_param float/tensor {mode}", flush=True)

    def run(ps):
        Ig, ug = I.clone().requires_grad_(True), u0.clone().requires_grad_(True)
        S = lif_param(Ig, ug, *ps, mode=mode)
        (S * G).sum().backward()
        return S, Ig.grad, ug.grad

    r1 = run([0.9, 1.0, 0.1])
    pt = [torch.tensor(v, device=dev, requires_grad=True) for v in (0.9, 1.0, 0.1)]
    r2 = run(pt)
    pm = [torch.tensor(0.9, device=dev, requires_grad=True), 1.0, 0.1]
    r3 = run(pm)
    assert torch.equal(r1[0], r2[0]) and torch.equal(r1[0], r3[0])
    # in scan mode at this size the adjoint is the look-back pass (deterministic: the same bits)
    for a, b, c in zip(r1[1:], r2[1:], r3[1:]):
        assert torch.equal(a, b) and torch.equal(a, c)
    assert torch.equal(pm[0].grad, pt[0].grad) and all(p.grad is not None for p in pt)
