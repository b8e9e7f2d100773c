"""GPU parity at the full sizes of BASELINE.json's configurations (cfg2, cfg4, cfg5; cfg3 is in
test_shdnet_gpu.py, cfg1 is the CPU path of test_fast_port.py), through the public layers.

The serial kernels these are compared with are pinned to the oracle bit for bit in
test_lif_gpu.py / test_alif_gpu.py; here every config is also checked against the oracle
itself where it finishes in seconds (a column subset for cfg4's 2^20 steps, all of cfg5).
Bars: spikes and potentials bit-exact; gradients 1e-5 of the fp32 oracle and 1e-4 of fp64;
ALIF's four parameter gradients 1e-4 of their fp64 assembly (the north star's bar; the fp32
arithmetic floor at cfg5 is about 2e-6).
"""
import numpy as np
import pytest
import torch

from oracle import alif_oracle as A
from oracle import lif_oracle as O
from tests._inputs import host

pytestmark = pytest.mark.gpu


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _normal(T, N, mu, sd, seed, dev):
    g = torch.Generator().manual_seed(seed)
    return (mu + sd * torch.randn(T, N, generator=g)).to(dev)


@pytest.mark.parametrize("beta,mu,sd", [(0.9, 0.12, 0.25), (0.99, 0.012, 0.08)])
def test_cfg2_headline_pair_full_size(dev, beta, mu, sd):
    """The timed step of bench.py at cfg2 (65,536 x 4,096): lif_tuned(mode="scan", K=8, repair on)
    runs the starts-only forward and the recomputing adjoint.  S equals the serial forward; dI and
    du0 equal the stored-U single pass (same chunk and wave count) bit for bit; dbeta its fp64
    sum to 1e-6; 512 columns of S and dI equal the oracle's (dI to 1e-5 / 1e-4 of fp64)."""
    from lifscan import hip_lif as L
    T, N = 4096, 65536
    assert L._recompute_ok(T, N, 8, 10 ** 6)
    print(f"cfg2 headline pair beta={beta}", flush=True)
    I = _normal(T, N, mu, sd, 0, dev)
    gS = _normal(T, N, 0.0, 1.0, 1, dev)
    u0 = torch.zeros(N, device=dev, requires_grad=True)
    b = torch.tensor(beta, device=dev, requires_grad=True)
    Ig = I.clone().requires_grad_(True)
    S = L.lif_tuned(Ig, u0, b, 1.0, 0.0, 4.0, mode="scan", K=8, repair=10 ** 6)
    S.backward(gS)
    assert L.starts_forward_timeouts(dev) == 0
    Us, Ss = L.serial_forward(I, beta, 1.0, 0.0, u0.detach())
    assert torch.equal(S.detach(), Ss)
    U2, S2 = L.scan_forward_exact(I, beta, 1.0, 0.0, u0.detach())
    assert torch.equal(U2, Us) and torch.equal(S2, Ss)
    Lam = L.scan_backward_fused(I, u0.detach(), U2, S2, gS, None, beta, 1.0, 0.0, 4.0)
    assert torch.equal(Ig.grad, Lam)
    assert torch.equal(u0.grad, torch.tensor(beta, device=dev) * Lam[0])
    uprev = torch.cat([u0.detach()[None], Us[:-1]], 0)
    db = float((Lam.double() * uprev.double()).sum())
    assert abs(b.grad.item() - db) <= 1e-6 * abs(db)
    cols = np.arange(0, N, N // 512)
    Ic, gc = host(I[:, cols]), host(gS[:, cols])
    z = np.zeros(len(cols), np.float32)
    Uo, So = O.serial_forward(Ic, beta, 1.0, 0.0, z)
    assert np.array_equal(host(S.detach()[:, cols]), So) and np.array_equal(host(Us[:, cols]), Uo)
    L32 = O.serial_backward(Ic, z, Uo, So, gc, None, beta, 1.0, 0.0, 4.0)
    L64 = O.serial_backward(Ic, z, Uo, So, gc, None, beta, 1.0, 0.0, 4.0, dtype=np.float64)
    assert rel(host(Lam[:, cols]), L32) < 1e-5 and rel(host(Lam[:, cols]), L64) < 1e-4
    del I, gS, Ig, S, Us, Ss, U2, S2, Lam, uprev
    torch.cuda.empty_cache()


def _cfg4_inputs(dev):
    T, N = 2 ** 20, 1024
    I = _normal(T, N, 0.012, 0.08, 0, dev)
    u0 = torch.rand(N, generator=torch.Generator().manual_seed(2)).to(dev)
    return T, N, I, u0


def test_cfg4_scan_v4_equals_serial(dev):
    """cfg4 (N = 1024, T = 2^20, beta = 0.99, x ~ N(0.012, 0.08^2), u0 ~ U[0, 1)): the three-level
    scan_forward_v4 with repair at the reference default (C 64, G 16, K 16, K2 32; most super maps
    overflow, passed by walking their chunk maps or by their serial steps) and at C 2048, G 4,
    K 32, K2 64 returns the serial forward bit for bit, with statistics (the Jacobi rounds) and
    without (the segmented ordered repair; there also with the super maps passed as stored, the
    converged default); 64 columns of the serial forward equal the oracle's."""
    from lifscan import hip_lif as L
    T, N, I, u0 = _cfg4_inputs(dev)
    Us, Ss = L.serial_forward(I, 0.99, 1.0, 0.0, u0)
    for C, G, K, K2, fb in ((64, 16, 16, 32, "chunks"), (64, 16, 16, 32, "serial"), (2048, 4, 32, 64, "chunks")):
        print(f"cfg4 v4 C={C} G={G} K={K} K2={K2} fallback={fb}", flush=True)
        st = {}
        U, S = L.scan_forward_v4(I, 0.99, 1.0, 0.0, u0, C=C, G=G, K=K, K2=K2, repair=10 ** 6, stats=st,
                                 super_fallback=fb)
        assert torch.equal(U, Us) and torch.equal(S, Ss), st
        print(f"  stats {st}", flush=True)
        # without statistics: the pipeline's converged repair (the segmented ordered walk here)
        U, S = L.scan_forward_v4_maps(I, 0.99, 1.0, 0.0, u0, C=C, G=G, K=K, K2=K2, repair=10 ** 6,
                                      super_fallback=fb)
        assert torch.equal(U, Us) and torch.equal(S, Ss)
        if fb == "chunks":  # the default of converged calls: overflowed super maps as stored
            U, S = L.scan_forward_v4_maps(I, 0.99, 1.0, 0.0, u0, C=C, G=G, K=K, K2=K2,
                                          repair=10 ** 6, super_fallback="none")
            assert torch.equal(U, Us) and torch.equal(S, Ss)
        del U, S
        torch.cuda.empty_cache()
    U, S = L.scan_forward_v4(I, 0.99, 1.0, 0.0, u0, C=64, G=16, K=16, K2=32, repair=10 ** 6)
    assert torch.equal(U, Us) and torch.equal(S, Ss)  # the converged dispatch
    del U, S
    cols = np.arange(0, N, N // 64)
    Uo, So = O.serial_forward(host(I[:, cols]), 0.99, 1.0, 0.0, host(u0[cols]))
    assert np.array_equal(host(Us[:, cols]), Uo) and np.array_equal(host(Ss[:, cols]), So)
    del I, Us, Ss
    torch.cuda.empty_cache()


def test_cfg4_lookback_adjoint(dev):
    """cfg4's adjoint (scan_backward_tiled takes the look-back pass at N = 1024): the same bits on
    three runs; against the serial adjoint kernel at full size (1e-5) and, on 64 columns, against
    the fp32 oracle (1e-5) and the fp64 one (1e-4); no bounded wait gave up."""
    from lifscan import hip_lif as L
    T, N, I, u0 = _cfg4_inputs(dev)
    gS = _normal(T, N, 0.0, 1.0, 1, dev)
    U, S = L.serial_forward(I, 0.99, 1.0, 0.0, u0)
    print("cfg4 look-back adjoint", flush=True)
    Lam = L.scan_backward_tiled(I, u0, U, S, gS, None, 0.99, 1.0, 0.0, 4.0)
    assert L.last_lookback_timeouts() == 0
    for _ in range(2):  # deterministic: the same bits on every run
        assert torch.equal(L.scan_backward_tiled(I, u0, U, S, gS, None, 0.99, 1.0, 0.0, 4.0), Lam)
    Lser = L.serial_backward(I, u0, U, S, gS, None, 0.99, 1.0, 0.0, 4.0)
    assert float((Lam - Lser).norm() / Lser.norm()) < 1e-5
    cols = np.arange(0, N, N // 64)
    Ic, Uc, Sc, gc = (host(a[:, cols]) for a in (I, U, S, gS))
    uc = host(u0[cols])
    L32 = O.serial_backward(Ic, uc, Uc, Sc, gc, None, 0.99, 1.0, 0.0, 4.0)
    L64 = O.serial_backward_long(Ic, uc, Uc, Sc, gc, 0.99, 1.0, 0.0, 4.0)
    got = host(Lam[:, cols])
    assert rel(got, L32) < 1e-5 and rel(got, L64) < 1e-4
    del I, gS, U, S, Lam, Lser
    torch.cuda.empty_cache()


CFG5 = dict(T=4096, N=16384, beta=0.95, rho=0.995, q=0.2, C=128)


def _cfg5_inputs(dev):
    c = CFG5
    I = _normal(c["T"], c["N"], 0.15, 0.3, 0, dev)
    return I, torch.zeros(c["N"], device=dev)


def test_cfg5_alif_layer_gradients(dev):
    """cfg5 (ALIF, N = 16,384, T = 4,096, beta .95, rho .995, q .2, x ~ N(0.15, 0.3^2), u0 = w0 = 0):
    alif() with the serial forward and the scan adjoint (its default), parameters as 0-d tensors;
    U, W, S equal the oracle, gradients for I, u0, w0 against the fp64 adjoint (1e-4) and for
    beta, rho, q, theta0 against ALIFFn's fp64 assembly (1e-4)."""
    from lifscan import triton_alif as AL
    c = CFG5
    I, z = _cfg5_inputs(dev)
    G = _normal(c["T"], c["N"], 0.0, 1.0, 1, dev)
    xg = I.clone().requires_grad_(True)
    ug = z.clone().requires_grad_(True)
    wg = z.clone().requires_grad_(True)
    ps = [torch.tensor(v, device=dev, requires_grad=True) for v in (c["beta"], c["rho"], c["q"], 1.0)]
    print("cfg5 alif layer", flush=True)
    S, U, W = AL.alif(xg, ug, wg, *ps, fwd="serial", bwd="scan")
    (S * G).sum().backward()
    x, Gh, zh = host(I), host(G), np.zeros(c["N"], np.float32)
    Uo, Wo, So = A.serial_forward(x, c["beta"], c["rho"], c["q"], 1.0, 0.0, zh, zh)
    assert np.array_equal(host(U), Uo) and np.array_equal(host(W), Wo)
    assert np.array_equal(host(S.detach()), So)
    LV6, LW6 = A.backward(x, Uo, Wo, So, Gh, c["beta"], c["rho"], c["q"], 1.0, zh, zh, 4.0,
                          dtype=np.float64)
    want = A.param_grads(x, Uo, Wo, So, Gh, LV6, LW6, c["beta"], c["rho"], c["q"], 1.0, zh, zh, 4.0)
    got = (xg.grad, ug.grad, wg.grad, *(p.grad for p in ps))
    errs = [rel(host(a), b) for a, b in zip(got, want)]
    print("  cfg5 gradient rel errs dI, du0, dw0, dbeta, drho, dq, dtheta0: "
          + ", ".join(f"{e:.2e}" for e in errs), flush=True)
    for k, e in enumerate(errs):
        assert e < 1e-4, k
    del I, G, xg, S, U, W
    torch.cuda.empty_cache()


def test_cfg5_box_scan_with_repair_equals_serial(dev):
    """cfg5's box scan (C = 128, K1 = K2 = 32, block 4) with repair equals the serial forward bit
    for bit for both chunk-entry predictions of the reference's protocol (the warm-up predictor
    with Wn = 4, and the previous iterate emulated by a 1.005x input,
    experiments/e25d_alif_fwd.py:44-50) at dw = 0.1q and 0.3q, with the Jacobi rounds (stats
    requested) and with the ordered chain pass (no stats)."""
    from lifscan import triton_alif as AL
    c = CFG5
    I, z = _cfg5_inputs(dev)
    b, r, q, C = c["beta"], c["rho"], c["q"], c["C"]
    U, W, S = AL.alif_serial_forward(I, b, r, q, 1.0, 0.0, z, z)
    _, Wprev, _ = AL.alif_serial_forward((1.005 * I).contiguous(), b, r, q, 1.0, 0.0, z, z)
    preds = {"warm4": AL.alif_warm_predict(I, b, r, q, 1.0, 0.0, z, z, C, Wn=4),
             "prev": AL.alif_prev_wpred(Wprev, z, C)}
    del Wprev
    for name, WP in preds.items():
        for dwq in (0.1, 0.3):
            print(f"cfg5 box scan pred={name} dw={dwq}q", flush=True)
            st = {}
            U2, W2, S2 = AL.alif_scan_forward(I, b, r, q, 1.0, 0.0, z, z, WP, dwq * q, C=C, K1=32, K2=32,
                                              BN=4, repair=10 ** 6, stats=st)
            assert torch.equal(U2, U) and torch.equal(W2, W) and torch.equal(S2, S), (name, dwq, st)
            print(f"  stats {st}", flush=True)
            U2, W2, S2 = AL.alif_scan_forward_maps(I, b, r, q, 1.0, 0.0, z, z, WP, dwq * q, C=C, K1=32,
                                                   K2=32, BN=4, repair=10 ** 6)  # no stats: the ordered chain
            assert torch.equal(U2, U) and torch.equal(W2, W) and torch.equal(S2, S), (name, dwq, "chain")
            U2, W2, S2 = AL.alif_scan_forward(I, b, r, q, 1.0, 0.0, z, z, WP, dwq * q, C=C, K1=32, K2=32,
                                              BN=4, repair=10 ** 6)  # the converged dispatch
            assert torch.equal(U2, U) and torch.equal(W2, W) and torch.equal(S2, S), (name, dwq, "dispatch")
            del U2, W2, S2
    del I, U, W, S
    torch.cuda.empty_cache()
