"""GPU parity of the single-pass fused kernels (lsh_lif_scan_exact_fwd,
lsh_lif_chunked_serial_fwd, lsh_lif_scan_fused_bwd) against the CPU oracle.

Forward: U and S bit-exact to the serial recurrence for every internal chunk length, map
capacity and regime, including partial rounds (fewer chunks than waves per workgroup) and
ragged neuron counts.  Backward: within 1e-5 relative of the fp32 oracle affine scan and
1e-4 relative of the fp64 adjoint.
"""
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


@pytest.fixture(scope="module")
def L():
    from lifscan import hip_lif
    return hip_lif


REGIMES = [(b, mu, sd) for b in (0.5, 0.9, 0.99, 1.0) for (mu, sd) in ((0.15, 0.4), (-0.1, 0.6), (0.4, 0.2))]


@pytest.mark.parametrize("beta,mu,sd", REGIMES)
def test_exact_forward_regimes(L, dev, beta, mu, sd):
    T, N = 1024, 777
    I = normal(T, N, mu, sd, 3)
    u0 = uniform(N, -0.3, 0.3, 4)
    Us, Ss = O.serial_forward(I, beta, 1.0, -0.1, u0)
    Ig, u0g = gpu(I, dev), gpu(u0, dev)
    for C, K in ((16, 4), (32, 8), (64, 16), (128, 8)):
        print(f"exact fwd beta={beta} mu={mu} C={C} K={K}", flush=True)
        U, S = L.scan_forward_exact(Ig, beta, 1.0, -0.1, u0g, C=C, K=K)
        assert np.array_equal(host(U), Us) and np.array_equal(host(S), Ss)
        assert L.last_fused_counters()["spin_timeouts"] == 0


@pytest.mark.parametrize("T,N,C", [(16, 1, 16), (48, 65, 16), (160, 130, 32), (320, 64, 64),
                                   (640, 200, 128), (4096, 3, 32)])
def test_exact_forward_partial_rounds_and_ragged(L, dev, T, N, C):
    I = normal(T, N, 0.12, 0.25, 5)
    u0 = uniform(N, 0.0, 0.9, 6)
    Us, Ss = O.serial_forward(I, 0.9, 1.0, 0.0, u0)
    for K in (1, 16):
        for maps in (True, False):
            print(f"exact fwd T={T} N={N} C={C} K={K} maps={maps}", flush=True)
            U, S = L.scan_forward_exact(gpu(I, dev), 0.9, 1.0, 0.0, gpu(u0, dev), C=C, K=K, maps=maps)
            assert np.array_equal(host(U), Us) and np.array_equal(host(S), Ss)
            assert L.last_fused_counters()["spin_timeouts"] == 0


def test_exact_forward_dyadic_ties(L, dev):
    """beta = 1/2 on a 1/64 grid: exact ties v == theta (e2_float.py:30-41)."""
    rng = np.random.default_rng(7)
    T, N = 512, 256
    I = (rng.integers(-40, 80, (T, N)) / 64.0).astype(np.float32)
    u0 = (rng.integers(-64, 64, N) / 64.0).astype(np.float32)
    Us, Ss = O.serial_forward(I, 0.5, 1.0, 0.0, u0)
    U, S = L.scan_forward_exact(gpu(I, dev), 0.5, 1.0, 0.0, gpu(u0, dev), C=32, K=8)
    assert np.array_equal(host(U), Us) and np.array_equal(host(S), Ss)


def test_v3_dispatches_to_single_pass_when_converged(L, dev):
    T, N = 2048, 300
    I = normal(T, N, 0.012, 0.08, 8)
    u0 = np.zeros(N, np.float32)
    Us, Ss = O.serial_forward(I, 0.99, 1.0, 0.0, u0)
    U, S = L.scan_forward_v3(gpu(I, dev), 0.99, 1.0, 0.0, gpu(u0, dev), C=128, K=8, repair=10 ** 6)
    assert np.array_equal(host(U), Us) and np.array_equal(host(S), Ss)
    c = L.last_fused_counters()
    assert c["spin_timeouts"] == 0


@pytest.mark.parametrize("C", [16, 32, 64])
@pytest.mark.parametrize("detach,with_gu", [(True, False), (False, True)])
def test_fused_backward(L, dev, C, detach, with_gu):
    T, N = 1024, 333
    I = normal(T, N, 0.15, 0.4, 9)
    u0 = uniform(N, -0.2, 0.2, 10)
    GS = normal(T, N, 0.0, 1.0, 11)
    GU = normal(T, N, 0.0, 1.0, 12) if with_gu else None
    U, S = O.serial_forward(I, 0.9, 1.0, -0.1, u0)
    print(f"fused bwd C={C} detach={detach} gu={with_gu}", flush=True)
    Lam = L.scan_backward_fused(gpu(I, dev), gpu(u0, dev), gpu(U, dev), gpu(S, dev), gpu(GS, dev),
                                gpu(GU, dev) if with_gu else None, 0.9, 1.0, -0.1, 4.0, detach, C=C)
    ref32 = O.scan_backward(I, u0, U, S, GS, GU, 0.9, 1.0, -0.1, 4.0, detach, C=C)
    ref64 = O.serial_backward(I, u0, U, S, GS, GU, 0.9, 1.0, -0.1, 4.0, detach, dtype=np.float64)
    assert rel(host(Lam), ref32) < 1e-5
    assert rel(host(Lam), ref64) < 1e-4


@pytest.mark.parametrize("T,N", [(16, 1), (48, 65), (4096, 3)])
def test_fused_backward_partial_rounds(L, dev, T, N):
    I = normal(T, N, 0.15, 0.4, 13)
    u0 = np.zeros(N, np.float32)
    GS = normal(T, N, 0.0, 1.0, 14)
    U, S = O.serial_forward(I, 0.9, 1.0, 0.0, u0)
    Lam = L.scan_backward_fused(gpu(I, dev), gpu(u0, dev), gpu(U, dev), gpu(S, dev), gpu(GS, dev),
                                None, 0.9, 1.0, 0.0, 4.0, C=16)
    ref64 = O.serial_backward(I, u0, U, S, GS, None, 0.9, 1.0, 0.0, 4.0, dtype=np.float64)
    assert rel(host(Lam), ref64) < 1e-4


def test_fused_cfg2_full_size(L, dev):
    """cfg2 (65,536 x 4,096, beta = 0.9 and 0.99): single-pass forward == serial kernel bit for
    bit; single-pass backward within 1e-5 of the three-kernel affine scan."""
    T, N = 4096, 65536
    for beta, mu, sd in ((0.9, 0.12, 0.25), (0.99, 0.012, 0.08)):
        print(f"cfg2 fused beta={beta}", flush=True)
        g = torch.Generator().manual_seed(0)
        I = (mu + sd * torch.randn(T, N, generator=g)).to(dev)
        g1 = torch.Generator().manual_seed(1)
        GS = torch.randn(T, N, generator=g1).to(dev)
        u0 = torch.zeros(N, device=dev)
        Us, Ss = L.serial_forward(I, beta, 1.0, 0.0, u0)
        for C in (32, 128):
            U, S = L.scan_forward_exact(I, beta, 1.0, 0.0, u0, C=C, K=8)
            assert torch.equal(U, Us) and torch.equal(S, Ss)
            print(f"  C={C} counters={L.last_fused_counters()}", flush=True)
        L1 = L.scan_backward_fused(I, u0, Us, Ss, GS, None, beta, 1.0, 0.0, 4.0)
        L2 = L.scan_backward_chunked(I, u0, Us, Ss, GS, None, beta, 1.0, 0.0, 4.0, C=128)
        assert ((L1 - L2).norm() / L2.norm()).item() < 1e-5
        del I, GS, Us, Ss, U, S, L1, L2
        torch.cuda.empty_cache()


@pytest.mark.parametrize("T,N,detach,with_gu,C", [(4096, 1000, True, False, 16), (2048, 64, True, True, 32),
                                                  (8192, 130, False, True, 16), (256, 7, True, False, 32),
                                                  (65536, 256, True, False, 16)])
def test_lookback_backward(dev, T, N, detach, with_gu, C):
    """Decoupled look-back adjoint vs the fp32 serial oracle (1e-5) and fp64 (1e-4); the same
    bits on a second run (fixed association order); every bounded wait ended on its flag (no
    give-ups).  (256, 7): one segment; (65536, 256): 256 segments, 16 anchor runs."""
    from lifscan import hip_lif as L
    beta = 0.95
    I = normal(T, N, 0.06, 0.2, 31)
    u0 = uniform(N, -0.2, 0.5, 32)
    GS = normal(T, N, 0.0, 1.0, 33)
    GU = normal(T, N, 0.0, 1.0, 34) if with_gu else None
    U, S = O.serial_forward(I, beta, 1.0, -0.1, u0)
    print(f"lookback bwd T={T} N={N} detach={detach} gu={with_gu} C={C}", flush=True)
    args = [gpu(a, dev) for a in (I, u0, U, S, GS)] + [gpu(GU, dev) if with_gu else None]
    Lam = L.scan_backward_lookback(*args, beta, 1.0, -0.1, 4.0, detach, C=C)
    assert L.last_lookback_timeouts() == 0
    assert torch.equal(L.scan_backward_lookback(*args, beta, 1.0, -0.1, 4.0, detach, C=C), Lam)
    Lo = O.serial_backward(I, u0, U, S, GS, GU, beta, 1.0, -0.1, 4.0, detach)
    L6 = O.serial_backward(I, u0, U, S, GS, GU, beta, 1.0, -0.1, 4.0, detach, dtype=np.float64)
    assert rel(host(Lam), Lo) < 1e-5 and rel(host(Lam), L6) < 1e-4


@pytest.mark.parametrize("C", [16, 32, 64])
@pytest.mark.parametrize("T,N", [(1024, 777), (64, 65), (2048, 130)])
def test_starts_forward_and_recomputing_adjoint(L, dev, C, T, N):
    """The recomputing pair: S and the chunk entry states equal the serial recurrence's bits,
    and the adjoint rebuilt from those states equals the single-pass adjoint that reads U and
    S (same chunking, same arithmetic), with and without the parameter sums."""
    if T % C:
        pytest.skip("T % C")
    beta, u_r = 0.9, -0.1
    I = normal(T, N, 0.15, 0.4, 21)
    u0 = uniform(N, -0.3, 0.3, 22)
    GS = normal(T, N, 0.0, 1.0, 23)
    Us, Ss = O.serial_forward(I, beta, 1.0, u_r, u0)
    Ig, u0g, Gg = gpu(I, dev), gpu(u0, dev), gpu(GS, dev)
    print(f"recompute pair C={C} T={T} N={N}", flush=True)
    S, ST = L.scan_forward_exact_starts(Ig, beta, 1.0, u_r, u0g, C=C)
    assert np.array_equal(host(S), Ss)
    ref_st = np.concatenate([u0[None], Us[C - 1:-1:C]], 0)
    assert np.array_equal(host(ST), ref_st)
    Lam_ref = L.scan_backward_fused(Ig, u0g, gpu(Us, dev), gpu(Ss, dev), Gg, None, beta, 1.0, u_r,
                                    4.0, C=C)
    Lam, sums = L.scan_backward_fused_starts(Ig, ST, Gg, beta, 1.0, u_r, 4.0)
    assert sums is None and torch.equal(Lam, Lam_ref)
    Lam2, sums2 = L.scan_backward_fused_starts(Ig, ST, Gg, beta, 1.0, u_r, 4.0, want_sums=True)
    # with the sums the kernel is the parameter variant (fewer waves per workgroup, so another
    # association than Lam_ref): it equals lsh_lif_param_bwd's single pass bit for bit
    from lifscan import _native as nat
    lib = nat.lib()
    Lam3 = torch.empty_like(Ig)
    parts = torch.zeros(lib.lsh_lif_param_partials(T, N, 2, C), 3, device=dev, dtype=torch.float64)
    Ug, Sg = gpu(Us, dev), gpu(Ss, dev)  # held: the call takes raw pointers
    nat.check(lib.lsh_lif_param_bwd(nat.ptr(Ig), nat.ptr(u0g), nat.ptr(Ug), nat.ptr(Sg), nat.ptr(Gg),
                                    nat.ptr(Lam3), nat.ptr(parts), T, N, beta, 1.0, u_r, 4.0, 2, C,
                                    None, 0, nat.stream_of(Ig)), "lsh_lif_param_bwd")
    assert torch.equal(Lam2, Lam3) and torch.equal(sums2, parts.sum(0))
    assert rel(host(Lam2), host(Lam_ref)) < 1e-6
    # the sums against the fp64 assembly of fit.py:44-47 on the serial trajectory and this Lam
    _, _, dbeta, dtheta, du_r = O.param_grads(I, u0, Us, Ss, GS, host(Lam2).astype(np.float64),
                                              beta, 1.0, u_r)
    s2 = host(sums2)
    bf = float(beta)  # param_grads scales by beta in fp64
    assert abs(s2[0] - dbeta) <= 1e-9 * (abs(dbeta) + 1.0)
    assert abs(-s2[1] - dtheta) <= 1e-5 * (abs(dtheta) + 1.0)
    # s_t*lam_{t+1} takes lam_{t+1} at a chunk's last step from the composed chain, one fp32
    # rounding away from the stored value
    assert abs(bf * s2[2] - du_r) <= 1e-6 * (abs(du_r) + 1.0)


@pytest.mark.parametrize("T,N", [(1024, 16384), (256, 17000)])
def test_lif_tuned_recomputing_path_equals_stored_path(L, dev, T, N):
    """lif_tuned in scan mode takes the recomputing pair at these shapes; S and every gradient
    equal those of the path that stores U (switch off)."""
    assert L._recompute_ok(T, N, 8, 10 ** 6)
    I = gpu(normal(T, N, 0.15, 0.4, 31), dev)
    GS = gpu(normal(T, N, 0.0, 1.0, 32), dev)
    u0 = gpu(uniform(N, -0.3, 0.3, 33), dev)
    out = []
    for rc in (True, False):
        L.RECOMPUTE_BWD = rc
        try:
            Ig = I.clone().requires_grad_(True)
            ug = u0.clone().requires_grad_(True)
            b = torch.tensor(0.9, device=dev, requires_grad=True)
            S = L.lif_tuned(Ig, ug, b, 1.0, 0.0, 4.0, mode="scan", K=8, repair=10 ** 6)
            S.backward(GS)
            out.append((S.detach(), Ig.grad, ug.grad, b.grad.item()))
        finally:
            L.RECOMPUTE_BWD = True
    (S1, g1, u1, b1), (S2, g2, u2, b2) = out
    assert torch.equal(S1, S2) and torch.equal(g1, g2) and torch.equal(u1, u2)
    assert abs(b1 - b2) <= 1e-6 * abs(b2)


def test_lif_auto_recomputing_path_equals_stored_path(L, dev):
    """lif_auto at N = 16384 runs the serial forward and the scan adjoint; the recomputing pair
    gives the same S and gradients."""
    T, N = 1024, 16384
    assert L.auto_modes(N, T) == ("serial", "scan")
    I = gpu(normal(T, N, 0.15, 0.4, 41), dev)
    GS = gpu(normal(T, N, 0.0, 1.0, 42), dev)
    out = []
    for rc in (True, False):
        L.RECOMPUTE_BWD = rc
        try:
            Ig = I.clone().requires_grad_(True)
            u0 = torch.zeros(N, device=dev, requires_grad=True)
            S = L.lif_auto(Ig, u0, 0.95, 1.0, 0.0, 4.0)
            S.backward(GS)
            out.append((S.detach(), Ig.grad, u0.grad))
        finally:
            L.RECOMPUTE_BWD = True
    (S1, g1, u1), (S2, g2, u2) = out
    assert torch.equal(S1, S2) and torch.equal(g1, g2) and torch.equal(u1, u2)
