"""Pins of the ALIF oracle (oracle/alif_oracle.py).

* the serial step equals an exact rational recurrence with fp32 round-to-nearest-even emulated
  per operation (triton_alif.py:26-31: theta0 + w rounded first, rho*w + q two roundings);
* the box scan with repair equals the serial recurrence for oracle, previous-iterate, warm-up
  and deliberately bad boxes, for two block sizes of the split decision (the reference's own
  contract, tests/test_alif.py:10-39);
* states the carry predicts without falling back land on the serial end state (u exactly,
  w to rounding), and exactly, u and w bit for bit, on dyadic inputs with beta = rho = 1/2,
  where every operation of the build and the carry is exact (first-spike lines, post-spike
  pieces and the no-spike map pinned, not only to rounding);
* the warm predictor equals its definition; the adjoint equals fp64 autograd through the
  recurrence (tests/test_alif_grad.py:8-36 restated).
"""
import math
from fractions import Fraction as Fr

import numpy as np
import pytest
import torch

from oracle import alif_oracle as A
from tests._inputs import normal, uniform
from tests.test_oracle_lif import round_f32

NEURONS = [("lsnn", 0.95, 0.995, 0.9), ("glif2", 0.99, 0.96, 0.2), ("appD-a", 0.9, 0.95, 0.5)]


def _inputs(beta, mfree, T, N, seed):
    g = torch.Generator().manual_seed(seed)
    sig = 0.5
    return ((1 - beta) * mfree + sig * math.sqrt(1 - beta * beta) * torch.randn(T, N, generator=g)).float().numpy()


@pytest.mark.parametrize("name,beta,rho,q", NEURONS)
def test_alif_step_is_two_rounding(name, beta, rho, q):
    T, N = 80, 4
    I = _inputs(beta, 2.0, T, N, 1)
    u0 = uniform(N, -0.2, 0.5, 2)
    w0 = uniform(N, 0.0, 0.3, 3)
    U, W, S = A.serial_forward(I, beta, rho, q, 1.0, 0.0, u0, w0)
    b, r, qq, th = (Fr(float(np.float32(v))) for v in (beta, rho, q, 1.0))
    for n in range(N):
        u, w = Fr(float(u0[n])), Fr(float(w0[n]))
        for t in range(T):
            v = round_f32(round_f32(b * u) + Fr(float(I[t, n])))
            s = v >= round_f32(th + w)
            rw = round_f32(r * w)
            u, w = (Fr(0), round_f32(rw + qq)) if s else (v, rw)
            assert Fr(float(U[t, n])) == u and Fr(float(W[t, n])) == w and S[t, n] == s


@pytest.mark.parametrize("name,beta,rho,q", NEURONS)
@pytest.mark.parametrize("mfree", [0.5, 2.0])
def test_box_scan_with_repair_equals_serial(name, beta, rho, q, mfree):
    T, N, C = 2048, 16, 128
    I = _inputs(beta, mfree, T, N, 4)
    u0 = np.zeros(N, np.float32)
    w0 = uniform(N, 0.0, 0.1, 5)
    Ur, Wr, Sr = A.serial_forward(I, beta, rho, q, 1.0, 0.0, u0, w0)
    Wentry = np.concatenate([w0[None], Wr[C - 1:-1:C]], 0)
    _, Wprev, _ = A.serial_forward((1.005 * I).astype(np.float32), beta, rho, q, 1.0, 0.0, u0, w0)
    preds = {"oracle": Wentry, "prev": np.concatenate([w0[None], Wprev[C - 1:-1:C]], 0),
             "warm4": A.warm_predict(I, beta, rho, q, 1.0, 0.0, u0, w0, C, Wn=4),
             "bad": Wentry + 5 * q}
    for tag, Wp in preds.items():
        for block in (1, 4):
            st = {}
            U, W, S = A.scan_forward(I, beta, rho, q, 1.0, 0.0, u0, w0, Wp, 0.1 * q, C=C, K1=16, K2=32,
                                     block=block, repair=10 ** 6, stats=st)
            assert np.array_equal(U, Ur) and np.array_equal(W, Wr) and np.array_equal(S, Sr), (tag, block)
            if tag == "bad":
                assert st["miss_frac"] > 0.9
            if tag == "oracle" and mfree == 2.0:
                assert st["miss_frac"] < 0.5


def test_carry_predictions_land_on_the_serial_state():
    beta, rho, q = 0.95, 0.995, 0.9
    T, N, C = 4096, 32, 128
    I = _inputs(beta, 2.0, T, N, 6)
    u0 = np.zeros(N, np.float32)
    w0 = np.zeros(N, np.float32)
    Ur, Wr, Sr = A.serial_forward(I, beta, rho, q, 1.0, 0.0, u0, w0)
    Wentry = np.concatenate([w0[None], Wr[C - 1:-1:C]], 0)
    keep = {}
    A.scan_forward(I, beta, rho, q, 1.0, 0.0, u0, w0, Wentry, 0.1 * q, C=C, K1=16, K2=32, keep=keep)
    SU, SW, MISS = keep["SU"], keep["SW"], keep["MISS"]
    checked = exact = 0
    for m in range(T // C - 1):
        ok = MISS[m] == 0
        su, sw = A.serial_segment(I[m * C:(m + 1) * C], beta, rho, q, 1.0, 0.0, SU[m], SW[m])
        # a fired first-spike line puts the state on a post-spike piece: u is the serial
        # tail from u_r (same step arithmetic); a chunk without a spike uses A*u + B
        assert np.allclose(SU[m + 1][ok], su[ok], rtol=1e-5, atol=1e-6)
        assert np.allclose(SW[m + 1][ok], sw[ok], rtol=1e-5, atol=1e-6)
        exact += int((ok & (SU[m + 1] == su)).sum())
        checked += int(ok.sum())
    assert checked > 100 and exact > 0.8 * checked


def test_carry_is_exact_on_dyadic_inputs():
    """beta = rho = 1/2 and q, theta0, u_r, the entries, the box and the inputs on dyadic grids:
    every operation of the build and of the carry is then exact in fp32 (products by powers of
    two, short dyadic sums; 16-step chunks keep every state within 24 bits), so a chunk the carry
    takes through its map (no miss) lands exactly on the serial chunk end, u and w bit for bit.
    This pins the first-spike lines (which line fires first), the post-spike pieces (their u,
    their w affine in x = lx*w + q, the piece that holds x) and the no-spike map exactly, where
    test_carry_predictions_land_on_the_serial_state pins w to rounding only."""
    beta, rho, q, theta0, u_r = 0.5, 0.5, 0.25, 1.0, -0.25
    C, N = 16, 512
    rng = np.random.default_rng(21)
    # half the columns driven hard (they spike), half kept below threshold (the no-spike map)
    hi_cols = rng.integers(-32, 96, (2 * C, N // 2))
    lo_cols = rng.integers(-32, 16, (2 * C, N - N // 2))
    I = (np.concatenate([hi_cols, lo_cols], 1) / 64.0).astype(np.float32)
    u0 = (rng.integers(-48, 64, N) / 64.0).astype(np.float32)
    w0 = (rng.integers(0, 33, N) / 64.0).astype(np.float32)
    Lu = np.full((2, N), -1.0, np.float32)
    Hu = np.full((2, N), 3.0, np.float32)
    Lw = np.zeros((2, N), np.float32)
    Hw = np.full((2, N), 0.5, np.float32)
    su, sw = A.serial_segment(I[:C], beta, rho, q, theta0, u_r, u0, w0)
    for block in (1, 4):
        mp = A.build_maps(I, Lu, Hu, Lw, Hw, beta, rho, q, theta0, u_r, C, 32, 32, block)
        SU, SW, MISS = A.carry(I, u0, w0, Lu, Hu, Lw, Hw, mp, beta, rho, q, theta0, u_r, C)
        took = MISS[0] == 0
        assert took.sum() > N // 2, (block, int(took.sum()))
        assert np.array_equal(SU[1][took], su[took]), block
        assert np.array_equal(SW[1][took], sw[took]), block
        # the lines and pieces were exercised: chunks that spiked and chunks that did not
        spiked = np.array([A.serial_forward(I[:C, [n]], beta, rho, q, theta0, u_r, u0[[n]], w0[[n]])[2].any()
                           for n in range(N)])
        assert (took & spiked).sum() > 100 and (took & ~spiked).sum() > 5, block


def test_warm_predict_definition():
    beta, rho, q = 0.99, 0.96, 0.2
    T, N, C = 1024, 8, 64
    I = _inputs(beta, 2.0, T, N, 7)
    u0 = uniform(N, 0.0, 0.5, 8)
    w0 = uniform(N, 0.0, 0.2, 9)
    WP = A.warm_predict(I, beta, rho, q, 1.0, 0.0, u0, w0, C, Wn=3, u_init=0.1, w_init=0.05)
    _, Wr, _ = A.serial_forward(I, beta, rho, q, 1.0, 0.0, u0, w0)
    assert np.array_equal(WP[0], w0)
    for m in (1, 2, 3):  # warm-up reaches t = 0: exact
        assert np.array_equal(WP[m], Wr[m * C - 1])
    m = 10
    _, w = A.serial_segment(I[(m - 3) * C:m * C], beta, rho, q, 1.0, 0.0, np.full(N, 0.1, np.float32),
                            np.full(N, 0.05, np.float32))
    assert np.array_equal(WP[m], w)


@pytest.mark.parametrize("beta,rho,q", [(0.95, 0.995, 0.9), (0.99, 0.96, 0.2)])
def test_alif_adjoint_matches_fp64_autograd(beta, rho, q):
    """Gradients w.r.t. I, u0, w0, beta, rho, q, theta0 from the oracle's adjoint and
    ALIFFn's assembly (triton_alif.py:541-554) equal fp64 autograd through the recurrence run
    on the fp32 trajectory (reset mask and state values from the fp32 run)."""
    T, N = 512, 6
    x = normal(T, N, 0.06, 0.15, 10)
    G = normal(T, N, 0.0, 1.0, 11)
    u0 = uniform(N, -0.1, 0.3, 12)
    w0 = uniform(N, 0.0, 0.2, 13)
    U, W, S = A.serial_forward(x, beta, rho, q, 1.0, 0.0, u0, w0)
    LV, LW = A.backward(x, U, W, S, G, beta, rho, q, 1.0, u0, w0, 4.0, dtype=np.float64)
    got = A.param_grads(x, U, W, S, G, LV, LW, beta, rho, q, 1.0, u0, w0, 4.0)
    ps = [torch.tensor(v, dtype=torch.float64, requires_grad=True) for v in (beta, rho, q, 1.0)]
    xd = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    ud = torch.tensor(u0, dtype=torch.float64, requires_grad=True)
    wd = torch.tensor(w0, dtype=torch.float64, requires_grad=True)
    U64, W64, S64 = (torch.tensor(a, dtype=torch.float64) for a in (U, W, S))
    u, w, loss = ud, wd, 0
    for t in range(T):
        if t > 0:
            u = u + (U64[t - 1] - u).detach()
            w = w + (W64[t - 1] - w).detach()
        v = ps[0] * u + xd[t]
        sg = torch.sigmoid(4.0 * (v - ps[3] - w))
        s = S64[t] + (sg - sg.detach())
        u = (1 - S64[t]) * v
        w = ps[1] * w + ps[2] * s
        loss = loss + (torch.tensor(G[t], dtype=torch.float64) * s).sum()
    gx, gu, gw, gb, gr, gq, gt = torch.autograd.grad(loss, (xd, ud, wd, *ps))
    assert np.allclose(got[0], gx.numpy(), rtol=1e-9, atol=1e-12)
    assert np.allclose(got[1], gu.numpy(), rtol=1e-9, atol=1e-12)
    assert np.allclose(got[2], gw.numpy(), rtol=1e-9, atol=1e-12)
    for a, b in zip(got[3:], (gb, gr, gq, gt)):
        assert a == pytest.approx(b.item(), rel=1e-9)
