"""GPU parity of the soft-reset path (triton_soft.py, the soft functions of triton_lif.py and
fit.py) against the CPU oracle (oracle/soft_oracle.py), through the C ABI.

Bars: U, S bit-exact for the serial forward, the scan without repair (and its statistics) and
the repaired scan on the reference's own grid (tests/test_soft_scan.py); the adjoint within 1e-6
of the float64 recurrence (the reference's FFT convolution restated in the oracle, itself pinned
to the direct recurrence); lif_soft / lif_soft_scan gradients for I, u0, beta within 1e-5 of the
fp64 assembly (tests/test_soft_gpu.py, tests/test_soft_scan_grad.py shapes).
"""
import numpy as np
import pytest
import torch

from oracle import soft_oracle as SO
from tests._inputs import gpu, host, normal, uniform

pytestmark = pytest.mark.gpu


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.fixture(scope="module")
def TS():
    from lifscan import triton_soft
    return triton_soft


def _inputs(mu, sd, T, N, seed):
    g = torch.Generator().manual_seed(seed)
    I = (mu + sd * torch.randn(T, N, generator=g)).numpy()
    u0 = (0.3 * torch.randn(N, generator=g)).numpy()
    return I, u0


@pytest.mark.parametrize("beta,theta", [(0.9, 1.0), (0.97, 0.8), (1.0, 1.0)])
def test_soft_serial_bitexact(TS, dev, beta, theta):
    I, u0 = _inputs(0.15, 0.4, 1500, 77, 1)
    Ur, Sr = SO.serial_forward(I, beta, theta, u0)
    for fn in (TS.soft_serial_forward, TS.soft_serial_forward_tiled):
        U, S = fn(gpu(I, dev), beta, theta, gpu(u0, dev))
        assert np.array_equal(host(U), Ur) and np.array_equal(host(S), Sr)
    from lifscan import triton_lif as L
    U, S = L.soft_serial_forward(gpu(I, dev), beta, theta, gpu(u0, dev))
    assert np.array_equal(host(U), Ur)


@pytest.mark.parametrize("beta,mu,sd", [(0.9, 0.15, 0.4), (0.99, -0.1, 0.6), (0.95, 0.4, 0.3)])
@pytest.mark.parametrize("C,K", [(16, 16), (32, 32), (32, 4)])
def test_soft_scan_matches_oracle(TS, dev, beta, mu, sd, C, K):
    """repair = 0: outputs and statistics equal the literal restatement of triton_soft.py."""
    T, N = 1024, 70
    I, u0 = _inputs(mu, sd, T, N, 2)
    sto, st = {}, {}
    Uo, So = SO.scan_forward(I, beta, 1.0, u0, C=C, K=K, stats=sto)
    U, S = TS.soft_scan_forward(gpu(I, dev), beta, 1.0, gpu(u0, dev), C=C, K=K, stats=st)
    assert np.array_equal(host(U), Uo) and np.array_equal(host(S), So)
    assert st["repair_iters"] == sto["repair_iters"] == 0
    assert st["overflow_frac"] == pytest.approx(sto["overflow_frac"], abs=1e-12)
    assert st["mean_pieces"] == pytest.approx(sto["mean_pieces"], abs=1e-9)
    assert st["max_pieces"] == sto["max_pieces"]


@pytest.mark.parametrize("beta", [0.9, 0.95, 0.97, 0.99])
@pytest.mark.parametrize("mu,sd", [(0.15, 0.4), (-0.1, 0.6), (0.4, 0.3)])
def test_soft_scan_with_repair_equals_serial(TS, dev, beta, mu, sd):
    """tests/test_soft_scan.py: T = 8192, N = 333, (C, K) in {(16, 16), (32, 32)}."""
    T, N = 8192, 333
    I, u0 = _inputs(mu, sd, T, N, 0)
    print(f"soft repair beta={beta} mu={mu}", flush=True)
    Ig, ug = gpu(I, dev), gpu(u0, dev)
    Ur, Sr = TS.soft_serial_forward(Ig, beta, 1.0, ug)
    for C, K in ((16, 16), (32, 32)):
        st = {}
        U, S = TS.soft_scan_forward(Ig, beta, 1.0, ug, C=C, K=K, repair=10 ** 6, stats=st)
        assert torch.equal(U, Ur) and torch.equal(S, Sr), (C, K)
        assert st["max_pieces"] <= K


@pytest.mark.parametrize("T,N", [(700, 9), (4096, 8), (64, 70000), (1009, 5)])
def test_soft_adjoint_fft(TS, dev, T, N):
    V = normal(T, N, 0.8, 0.4, 4)
    gS = normal(T, N, 0.0, 1.0, 5)
    ref = SO.adjoint_fft(V, gS, 0.95, 1.0)
    direct = SO.adjoint_direct64(V, gS, 0.95, 1.0)
    lam = host(TS.soft_adjoint_fft(gpu(V, dev), gpu(gS, dev), 0.95, 1.0))
    assert rel(lam, direct) < 1e-6
    assert rel(lam, ref) < 1e-6


@pytest.mark.parametrize("T,N", [(1024, 130), (2048, 3)])
def test_soft_backward_from_states(TS, dev, T, N):
    I, u0 = _inputs(0.2, 0.4, T, N, 6)
    gS = normal(T, N, 0.0, 1.0, 7)
    U, S = SO.serial_forward(I, 0.93, 1.0, u0)
    up = np.concatenate([u0[None], U[:-1]], 0)
    V = (np.float32(0.93) * up + I).astype(np.float32)
    ref = SO.adjoint_direct64(V, gS, 0.93, 1.0)
    lam, db = TS._soft_backward(gpu(I, dev), gpu(u0, dev), gpu(U, dev), gpu(gS, dev), 0.93, 1.0, 4.0)
    assert rel(host(lam), ref) < 1e-6
    db_ref = float((ref.astype(np.float32).astype(np.float64) * up).sum())
    assert abs(db.item() - db_ref) <= 1e-6 * (abs(db_ref) + 1.0)
    from lifscan import triton_lif as L
    lam2 = L.soft_serial_backward_auto(gpu(I, dev), gpu(u0, dev), gpu(U, dev), gpu(gS, dev), 0.93, 1.0)
    assert torch.equal(lam2, lam)


@pytest.mark.parametrize("layer,T,N,gain,bias,beta", [
    ("lif_soft", 2048, 32, 0.5, 0.1, 0.93),
    ("scan", 16384, 8, 0.3, 0.06, 0.95),
    ("serial", 16384, 8, 0.3, 0.06, 0.95),
    ("scan", 1024, 300, 0.4, 0.08, 0.9)])
def test_soft_layer_gradients(TS, dev, layer, T, N, gain, bias, beta):
    """The reference's soft-layer checks: lif_soft (tests/test_soft_gpu.py) and lif_soft_scan in
    both modes (tests/test_soft_scan_grad.py), gradients of sum(W*S) for I (through the gain),
    u0 and beta against the fp64 recurrence on the same forward."""
    from lifscan.fit import lif_soft, lif_soft_scan
    x = normal(T, N, 0.0, 1.0, 11)
    W = normal(T, N, 0.0, 1.0, 12)
    print(f"soft layer {layer} T={T} N={N}", flush=True)
    b = torch.tensor(beta, device=dev, requires_grad=True)
    g = torch.tensor(gain, device=dev, requires_grad=True)
    u0 = torch.zeros(N, device=dev, requires_grad=True)
    I = g * gpu(x, dev) + bias
    if layer == "lif_soft":
        S = lif_soft(I, u0, b)
    else:
        S = lif_soft_scan(I, u0, b, mode=layer)
    (gpu(W, dev) * S).sum().backward()
    I32 = host(I)
    z = np.zeros(N, np.float32)
    if layer == "scan":
        U, So = SO.scan_forward(I32, beta, 1.0, z, C=128, K=32)
    else:
        U, So = SO.serial_forward(I32, beta, 1.0, z)
    assert np.array_equal(host(S), So)
    up = np.concatenate([z[None], U[:-1]], 0)
    V = (np.float32(beta) * up + I32).astype(np.float32)
    lam = SO.adjoint_direct64(V, W, float(np.float32(beta)), 1.0)
    dgain = float((lam * x.astype(np.float64)).sum())
    dbeta = float((lam * up).sum())
    assert abs(g.grad.item() - dgain) <= 1e-5 * abs(dgain) + 1e-6
    assert abs(b.grad.item() - dbeta) <= 1e-5 * abs(dbeta) + 1e-6
    assert rel(host(u0.grad), float(np.float32(beta)) * lam[0]) < 1e-5
