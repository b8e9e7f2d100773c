"""GPU parity of the affine-reset kernels against the CPU oracle (oracle/affine_oracle.py),
through the C ABI.

Bars: U, S bit-exact for the serial forward and the repaired scan (the reference's own grid,
tests/test_affine.py:7-18); every intermediate of the scan without repair (envelopes, pieces,
counts, overflow flags, chunk starts) and its outputs bit-exact against the oracle; stats
equal; the adjoint within 1e-4 relative of the fp64 adjoint in every mode, parameter sums
within 1e-4; lif_affine's gradients (I, u0, beta, gamma, delta) within 1e-4 of the fp64
assembly (the reference's bar is 1e-3, tests/test_affine.py:35).
"""
import numpy as np
import pytest
import torch

from oracle import affine_oracle as A
from tests._inputs import gpu, host, normal, uniform

pytestmark = pytest.mark.gpu

GRID = [(0.0, 0.0), (0.0, -0.2), (0.3, -0.1), (0.7, -0.5), (1.0, -1.0), (0.5, 0.2)]


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.fixture(scope="module")
def AF():
    from lifscan import triton_affine
    return triton_affine


def _ref_inputs(T, N, seed=0):
    g = torch.Generator().manual_seed(seed)
    I = (0.15 + 0.4 * torch.randn(T, N, generator=g)).numpy()
    u0 = (0.2 * torch.randn(N, generator=g)).numpy()
    return I, u0


@pytest.mark.parametrize("gamma,delta", GRID)
@pytest.mark.parametrize("T,N", [(1024, 200), (37, 65), (1, 1)])
def test_serial_bitexact(AF, dev, gamma, delta, T, N):
    I, u0 = _ref_inputs(T, N, 1)
    Ur, Sr = A.serial_forward(I, 0.93, 1.0, gamma, delta, u0)
    U, S = AF.aff_serial_forward(gpu(I, dev), 0.93, 1.0, gamma, delta, gpu(u0, dev))
    assert np.array_equal(host(U), Ur) and np.array_equal(host(S), Sr)


@pytest.mark.parametrize("gamma,delta", [(0.3, -0.1), (1.0, -1.0), (0.0, -0.2), (0.7, -0.5)])
@pytest.mark.parametrize("K", [32, 8, 3])
def test_scan_intermediates_match_oracle(AF, dev, gamma, delta, K):
    """repair = 0: envelopes, pieces, counts, overflow flags, chunk starts, outputs and stats
    equal the oracle's bit for bit (K = 8, 3 force overflows and the compaction's drops)."""
    T, N, C, beta = 1024, 70, 128, 0.95
    I, u0 = _ref_inputs(T, N, 2)
    print(f"affine scan gamma={gamma} delta={delta} K={K}", flush=True)
    keep, sto = {}, {}
    Uo, So = A.scan_forward(I, beta, 1.0, gamma, delta, u0, C=C, K=K, stats=sto, keep=keep)
    st = {}
    U, S = AF.aff_scan_forward(gpu(I, dev), beta, 1.0, gamma, delta, gpu(u0, dev), C=C, K=K,
                               stats=st)
    run = AF.last_aff_run()
    assert np.array_equal(host(run.view("LO")), keep["Lo"])
    assert np.array_equal(host(run.view("HI")), keep["Hi"])
    np_ = host(run.view("NP", torch.int32))
    assert np.array_equal(np_, keep["n"])
    assert np.array_equal(host(run.view("OVF", torch.int32)), keep["ovf"])
    P = host(run.view("PIECES"))
    for f, name in enumerate(("xl", "xr", "a", "c")):
        assert np.array_equal(P[..., f], keep[name]), name
    assert np.array_equal(host(run.view("STARTS")), keep["starts"])
    assert np.array_equal(host(U), Uo) and np.array_equal(host(S), So)
    assert st["overflow_frac"] == pytest.approx(sto["overflow_frac"], abs=1e-12)
    assert st["mean_pieces"] == pytest.approx(sto["mean_pieces"], abs=1e-9)
    assert st["repair_iters"] == sto["repair_iters"] == 0
    if K == 3:
        assert sto["overflow_frac"] > 0


@pytest.mark.parametrize("gamma,delta", GRID)
@pytest.mark.parametrize("beta", [0.9, 0.97])
def test_scan_with_repair_equals_serial(AF, dev, gamma, delta, beta):
    """The reference's own check (tests/test_affine.py:7-18): T = 8192, N = 200, C = 128,
    K = 32; with repair the scan is bit-identical to the serial recurrence."""
    T, N = 8192, 200
    g = torch.Generator().manual_seed(0)
    I = (0.15 + 0.4 * torch.randn(T, N, generator=g)).numpy()
    u0 = (0.2 * torch.randn(N, generator=g)).numpy()
    print(f"affine repair gamma={gamma} delta={delta} beta={beta}", flush=True)
    Ig, ug = gpu(I, dev), gpu(u0, dev)
    Ur, Sr = AF.aff_serial_forward(Ig, beta, 1.0, gamma, delta, ug)
    st = {}
    U, S = AF.aff_scan_forward(Ig, beta, 1.0, gamma, delta, ug, C=128, K=32, repair=10 ** 6,
                               stats=st)
    assert torch.equal(U, Ur) and torch.equal(S, Sr)
    assert 0.0 <= st["overflow_frac"] <= 1.0 and st["mean_pieces"] >= 1.0


@pytest.mark.parametrize("R", [1, 2, 10 ** 6])
def test_repair_rounds_match_oracle(AF, dev, R):
    T, N, C = 2048, 40, 128
    I, u0 = _ref_inputs(T, N, 3)
    sto, st = {}, {}
    Uo, So = A.scan_forward(I, 0.97, 1.0, 0.4, -0.3, u0, C=C, K=8, repair=R, stats=sto)
    U, S = AF.aff_scan_forward(gpu(I, dev), 0.97, 1.0, 0.4, -0.3, gpu(u0, dev), C=C, K=8, repair=R,
                               stats=st)
    assert np.array_equal(host(U), Uo) and np.array_equal(host(S), So)
    assert st["repair_iters"] == sto["repair_iters"]


def test_rejects_bad_arguments(AF, dev):
    I = torch.zeros(256, 8, device=dev)
    u0 = torch.zeros(8, device=dev)
    with pytest.raises(ValueError):
        AF.aff_scan_forward(I, 0.9, 1.0, 1.5, 0.0, u0)
    with pytest.raises(ValueError):
        AF.aff_serial_forward(I, 0.9, 1.0, -0.5, 0.0, u0)
    with pytest.raises(ValueError):
        AF.aff_scan_forward(I, 0.9, 1.0, 0.5, 0.0, u0, C=100)
    with pytest.raises(ValueError):
        AF.aff_scan_forward(I, 0.9, 1.0, 0.5, 0.0, u0, K=64)


@pytest.mark.parametrize("T,N", [(256, 8), (0, 5), (64, 0)])
def test_empty_and_tiny_shapes(AF, dev, T, N):
    I, u0 = _ref_inputs(T, N, 4)
    Ur, Sr = A.serial_forward(I, 0.9, 1.0, 0.5, -0.2, u0)
    U, S = AF.aff_scan_forward(gpu(I, dev), 0.9, 1.0, 0.5, -0.2, gpu(u0, dev), C=64, K=16,
                               repair=10 ** 6)
    assert U.shape == (T, N)
    assert np.array_equal(host(U), Ur) and np.array_equal(host(S), Sr)


@pytest.mark.parametrize("mode,C", [("serial", None), ("chunked", 64), ("chunked", 16),
                                    ("fused", 16), ("fused", 32), ("lookback", None)])
@pytest.mark.parametrize("gamma,delta", [(0.4, -0.3), (1.0, -1.0), (0.0, 0.1)])
def test_adjoint_modes_match_fp64(AF, dev, mode, C, gamma, delta):
    T, N, beta = 1024, 130, 0.95
    I = normal(T, N, 0.2, 0.4, 31)
    u0 = uniform(N, -0.2, 0.6, 32)
    GS = normal(T, N, 0.0, 1.0, 33)
    U, S = A.serial_forward(I, beta, 1.0, gamma, delta, u0)
    lam, du0, db, dg, dd = A.backward(I, u0, U, S, GS, beta, gamma, delta, dtype=np.float64)
    print(f"affine adjoint {mode} C={C} gamma={gamma}", flush=True)
    Lam, sums = AF._aff_backward(gpu(I, dev), gpu(u0, dev), gpu(U, dev), gpu(S, dev), gpu(GS, dev),
                                 beta, 1.0, gamma, 4.0, mode=mode, C=C)
    sums = host(sums)
    b = float(np.float32(beta))
    assert rel(host(Lam), lam) < 1e-4
    for mine, ref in ((sums[0], db), (b * sums[1], dg), (b * sums[2], dd)):
        assert abs(mine - ref) <= 1e-4 * (abs(ref) + 1e-3 * np.abs(lam).sum() / T)


def test_reverse_affine_scan(AF, dev):
    T, N = 777, 90
    a = uniform(T * N, 0.0, 1.0, 51).reshape(T, N)
    b = normal(T, N, 0.0, 1.0, 52)
    ref = np.zeros((T, N))
    nxt = np.zeros(N)
    for t in range(T - 1, -1, -1):
        nxt = a[t].astype(np.float64) * nxt + b[t]
        ref[t] = nxt
    out = host(AF.reverse_affine_scan(gpu(a, dev), gpu(b, dev)))
    assert rel(out, ref) < 1e-5
    # the serial fp32 recurrence exactly (two roundings per step)
    nxt = np.zeros(N, np.float32)
    for t in range(T - 1, -1, -1):
        nxt = a[t] * nxt + b[t]
        assert np.array_equal(out[t], nxt)


@pytest.mark.parametrize("mode", ["serial", "scan"])
@pytest.mark.parametrize("T,N", [(4096, 8), (1024, 96), (256, 17000)])
def test_lif_affine_gradients(AF, dev, mode, T, N):
    """The reference's gradient check (tests/test_affine.py:19-35): I = gain*x + 0.08 with
    tensors beta, gamma, delta, gain; gradients of sum(W*S) against the fp64 assembly of the
    oracle's adjoint on the same spikes."""
    x = normal(T, N, 0.0, 1.0, 61)
    W = normal(T, N, 0.0, 1.0, 62)
    print(f"lif_affine {mode} T={T} N={N}", flush=True)
    ps = [torch.tensor(v, device=dev, requires_grad=True) for v in (0.95, 0.4, -0.3, 0.3)]
    xg = gpu(x, dev)
    u0 = torch.zeros(N, device=dev, requires_grad=True)
    I = ps[3] * xg + 0.08
    S = AF.lif_affine(I, u0, ps[0], ps[1], ps[2], mode=mode)
    (gpu(W, dev) * S).sum().backward()
    # reference: the oracle forward (the scan without repair when mode == "scan") and adjoint
    I32 = host(I)
    if mode == "scan":
        U, So = A.scan_forward(I32, 0.95, 1.0, 0.4, -0.3, np.zeros(N, np.float32), C=128, K=32)
    else:
        U, So = A.serial_forward(I32, 0.95, 1.0, 0.4, -0.3, np.zeros(N, np.float32))
    assert np.array_equal(host(S), So)
    lam, du0, db, dg, dd = A.backward(I32, np.zeros(N, np.float32), U, So, W, 0.95, 0.4, -0.3,
                                      dtype=np.float64)
    dgain = float((lam * x.astype(np.float64)).sum())
    got = [p.grad.item() for p in ps]
    for g_, r_ in zip(got, (db, dg, dd, dgain)):
        assert abs(g_ - r_) <= 1e-4 * abs(r_) + 1e-6, (got, (db, dg, dd, dgain))
    assert rel(host(u0.grad), du0) < 1e-4


@pytest.mark.parametrize("T,N", [(1, 1), (63, 64), (65, 7), (1000, 130), (4113, 1029)])
@pytest.mark.parametrize("gamma,delta", [(0.3, -0.1), (1.0, -1.0), (0.0, 0.0)])
def test_aff_serial_pipe(dev, T, N, gamma, delta):
    """The producer/consumer serial forward of the affine reset (and so of the soft reset) gives
    the oracle's U, S bit for bit."""
    from lifscan import hip_affine
    I = normal(T, N, 0.15, 0.5, 91)
    u0 = uniform(N, -0.2, 0.9, 92)
    Ur, Sr = A.serial_forward(I, 0.93, 1.0, gamma, delta, u0)
    print(f"aff serial pipe T={T} N={N} gamma={gamma}", flush=True)
    U2, S2 = hip_affine.aff_serial_forward(gpu(I, dev), 0.93, 1.0, gamma, delta, gpu(u0, dev))
    assert np.array_equal(host(U2), Ur) and np.array_equal(host(S2), Sr)
