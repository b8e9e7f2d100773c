"""Pins of the affine-reset oracle (oracle/affine_oracle.py) that do not retype its formulas:
the per-operation fp32 rounding of the step in exact rationals, the hard-reset special case,
envelope validity on the serial trajectory, chunk maps that reproduce the serial chunk for every
start on exact (dyadic) inputs and stay within the piece bound of Theorem 7(b), repair == serial
on the reference's own test grid (tests/test_affine.py:7-18, smaller T), and the adjoint with
its parameter gradients against fp64 autograd of the serial recurrence (tests/test_affine.py:
19-35).
"""
from fractions import Fraction as Fr

import numpy as np
import pytest
import torch

from oracle import affine_oracle as A
from oracle import lif_oracle as O
from tests._inputs import normal, uniform
from tests.test_oracle_lif import round_f32

GRID = [(0.0, 0.0), (0.0, -0.2), (0.3, -0.1), (0.7, -0.5), (1.0, -1.0), (0.5, 0.2)]


def _f(v):
    return Fr(float(np.float32(v)))


@pytest.mark.parametrize("gamma,delta", GRID)
def test_step_is_two_rounding_with_affine_reset(gamma, delta):
    T, N = 50, 5
    I = normal(T, N, 0.15, 0.4, 3)
    u0 = uniform(N, -0.3, 0.9, 4)
    U, S = A.serial_forward(I, 0.93, 1.0, gamma, delta, u0)
    b, th, g, d = _f(0.93), _f(1.0), _f(gamma), _f(delta)
    for n in range(N):
        u = Fr(float(u0[n]))
        for t in range(T):
            v = round_f32(round_f32(b * u) + Fr(float(I[t, n])))
            s = v >= th
            u = round_f32(round_f32(g * v) + d) if s else v
            assert Fr(float(U[t, n])) == u, (n, t)
            assert S[t, n] == (1.0 if s else 0.0)


def test_gamma_zero_is_the_hard_reset():
    I = normal(300, 40, 0.15, 0.4, 5)
    u0 = uniform(40, -0.5, 0.9, 6)
    U, S = A.serial_forward(I, 0.9, 1.0, 0.0, -0.2, u0)
    Uh, Sh = O.serial_forward(I, 0.9, 1.0, -0.2, u0)
    assert np.array_equal(U, Uh) and np.array_equal(S, Sh)


@pytest.mark.parametrize("gamma,delta", GRID)
@pytest.mark.parametrize("beta", [0.9, 0.97])
def test_envelopes_bound_the_serial_chunk_starts(gamma, delta, beta):
    T, N, C = 2048, 32, 64
    I = normal(T, N, 0.15, 0.4, 7)
    u0 = uniform(N, -0.4, 0.9, 8)
    U, _ = A.serial_forward(I, beta, 1.0, gamma, delta, u0)
    starts = np.concatenate([u0[None], U[C - 1:-1:C]], 0)
    Lo, Hi = A.envelopes(I, beta, 1.0, gamma, delta, u0, C)
    assert (Lo <= starts).all() and (starts <= Hi).all()
    # the bounds are not vacuous: no wider than the free swing of the inputs
    assert np.isfinite(Lo).all() and np.isfinite(Hi).all()
    assert float((Hi - Lo).max()) < 20.0


def _dyadic(rng, T, N):
    return (rng.integers(-24, 80, (T, N)) / 64.0).astype(np.float32)


@pytest.mark.parametrize("gamma,delta", [(0.5, -0.25), (0.0, 0.125), (1.0, -1.0), (0.25, 0.0)])
def test_chunk_maps_equal_serial_chunk_on_exact_inputs(gamma, delta):
    """beta = 1/2, gamma in {0, 1/4, 1/2, 1} and inputs on a 1/64 grid: every fp32 operation of
    the build and of the serial step is exact, so for every start in [lo, hi] exactly one piece
    holds it and a*u + c is the serial chunk result bit for bit, ties v == theta included."""
    rng = np.random.default_rng(11)
    T, N, C, K = 64, 24, 8, 64
    I = _dyadic(rng, T, N)
    M = T // C
    Lo = np.full((M, N), -2.0, np.float32)
    Hi = np.full((M, N), 2.0, np.float32)
    xl, xr, a, c, n, ovf = A.build_maps(I, Lo, Hi, 0.5, 1.0, gamma, delta, C, K)
    assert not ovf.any()
    us = (np.arange(-128, 129) / 64.0).astype(np.float32)
    ties = 0
    for m in range(M):
        for u in us:
            uu = np.full(N, u, np.float32)
            val, found = A.eval_map(xl[m], xr[m], a[m], c[m], n[m], uu)
            ser = A.serial_segment(I[m * C:(m + 1) * C], 0.5, 1.0, gamma, delta, uu)
            assert found.all(), (m, u)
            assert np.array_equal(val, ser), (m, u)
        # starts exactly on the breakpoints: the spiking side holds them
        for k in range(K):
            on = k < n[m]
            if not on.any():
                continue
            uu = np.where(on & np.isfinite(xl[m, :, k]), xl[m, :, k], 0.0).astype(np.float32)
            val, found = A.eval_map(xl[m], xr[m], a[m], c[m], n[m], uu)
            ser = A.serial_segment(I[m * C:(m + 1) * C], 0.5, 1.0, gamma, delta, uu)
            assert found.all() and np.array_equal(val, ser)
            ties += int((on & np.isfinite(xl[m, :, k])).sum())
    assert ties > 0


@pytest.mark.parametrize("gamma,delta", [(0.5, -0.25), (1.0, -1.0), (0.3, -0.1)])
def test_unpruned_piece_count_within_theorem_bound(gamma, delta):
    """Theorem 7(b) (triton_affine.py:2-4): an order-preserving non-expanding reset gives at
    most 1 + L(L+1)/2 pieces over L steps; with no pruning the build must not exceed it."""
    T, N, C, K = 80, 40, 10, 64
    I = normal(T, N, 0.3, 0.5, 12)
    M = T // C
    big = np.float32(1e30)
    xl, xr, a, c, n, ovf = A.build_maps(I, np.full((M, N), -big), np.full((M, N), big), 0.9, 1.0,
                                        gamma, delta, C, K)
    assert not ovf.any()
    assert int(n.max()) <= 1 + C * (C + 1) // 2
    assert int(n.max()) > 1
    # pieces are disjoint and cover the line (sorted by xl they tile it)
    for m in range(M):
        for j in range(N):
            k = n[m, j]
            order = np.argsort(xl[m, j, :k])
            L_, R_ = xl[m, j, :k][order], xr[m, j, :k][order]
            assert L_[0] == -np.inf and R_[-1] == np.inf
            assert np.array_equal(L_[1:], R_[:-1])


def test_map_agrees_with_serial_away_from_breakpoints():
    """General inputs: the map is the real-number composition, so away from its breakpoints it
    gives the serial spike pattern and a value within a few ulps of the serial chunk."""
    T, N, C, K = 512, 64, 64, 32
    I = normal(T, N, 0.15, 0.4, 13)
    u0 = uniform(N, -0.3, 0.9, 14)
    Lo, Hi = A.envelopes(I, 0.95, 1.0, 0.4, -0.3, u0, C)
    xl, xr, a, c, n, ovf = A.build_maps(I, Lo, Hi, 0.95, 1.0, 0.4, -0.3, C, K)
    rng = np.random.default_rng(15)
    close, total = 0, 0
    for m in range(T // C):
        for _ in range(8):
            uu = (Lo[m] + (Hi[m] - Lo[m]) * rng.random(N)).astype(np.float32)
            val, found = A.eval_map(xl[m], xr[m], a[m], c[m], n[m], uu)
            ser = A.serial_segment(I[m * C:(m + 1) * C], 0.95, 1.0, 0.4, -0.3, uu)
            ok = found & (ovf[m] == 0)
            close += int((ok & (np.abs(val - ser) <= 1e-5 * (1 + np.abs(ser)))).sum())
            total += int(ok.sum())
    assert total > 0.9 * 8 * N * (T // C)
    assert close >= 0.995 * total


@pytest.mark.parametrize("gamma,delta", GRID)
@pytest.mark.parametrize("beta", [0.9, 0.97])
def test_scan_with_repair_equals_serial(gamma, delta, beta):
    """tests/test_affine.py:7-18 at T = 1024, N = 24: with repair the scan is bit-identical to
    the serial recurrence."""
    T, N = 1024, 24
    g = torch.Generator().manual_seed(0)
    I = (0.15 + 0.4 * torch.randn(T, N, generator=g)).numpy()
    u0 = (0.2 * torch.randn(N, generator=g)).numpy()
    Ur, Sr = A.serial_forward(I, beta, 1.0, gamma, delta, u0)
    st = {}
    U, S = A.scan_forward(I, beta, 1.0, gamma, delta, u0, C=128, K=32, repair=10 ** 6, stats=st)
    assert np.array_equal(U, Ur) and np.array_equal(S, Sr)
    assert st["mean_pieces"] >= 1.0 and 0.0 <= st["overflow_frac"] <= 1.0


def _autograd(I, u0, S32, U32, GS, beta, gamma, delta, alpha):
    """fp64 autograd of the serial recurrence with the fp32 spike pattern as the detached reset
    mask and the sigmoid surrogate as ds/dv; states pinned to the fp32 trajectory by a detached
    correction (derivatives are those of the recurrence)."""
    Id = torch.tensor(I, dtype=torch.float64, requires_grad=True)
    u0d = torch.tensor(u0, dtype=torch.float64, requires_grad=True)
    b, g, d = (torch.tensor(float(np.float32(v)), dtype=torch.float64, requires_grad=True)
               for v in (beta, gamma, delta))
    Sd = torch.tensor(S32, dtype=torch.float64)
    Ud = torch.tensor(U32, dtype=torch.float64)
    u = u0d
    loss = 0
    for t in range(I.shape[0]):
        if t > 0:
            u = u + (Ud[t - 1] - u).detach()
        v = b * u + Id[t]
        sg = torch.sigmoid(alpha * (v - 1.0))
        s = Sd[t] + (sg - sg.detach())
        u = (1 - Sd[t]) * v + Sd[t] * (g * v + d)
        loss = loss + (torch.tensor(GS[t], dtype=torch.float64) * s).sum()
    return [z.detach().numpy() for z in torch.autograd.grad(loss, (Id, u0d, b, g, d))]


@pytest.mark.parametrize("gamma,delta", [(0.4, -0.3), (0.0, 0.0), (1.0, -1.0)])
def test_adjoint_and_parameter_gradients_match_fp64_autograd(gamma, delta):
    T, N = 300, 12
    I = normal(T, N, 0.2, 0.4, 21)
    u0 = uniform(N, -0.2, 0.6, 22)
    GS = normal(T, N, 0.0, 1.0, 23)
    U, S = A.serial_forward(I, 0.95, 1.0, gamma, delta, u0)
    lam, du0, db, dg, dd = A.backward(I, u0, U, S, GS, 0.95, gamma, delta, dtype=np.float64)
    gI, g0, gb, gg, gd = _autograd(I, u0, S, U, GS, 0.95, gamma, delta, 4.0)
    assert np.linalg.norm(lam - gI) / np.linalg.norm(gI) < 1e-10
    assert np.allclose(du0, g0, rtol=1e-10, atol=1e-12)
    for mine, ref in ((db, gb), (dg, gg), (dd, gd)):
        assert abs(mine - float(ref)) <= 1e-9 * (abs(float(ref)) + 1e-6)
    # the fp32 recurrence stays within the kernels' tolerance of fp64
    lam32 = A.backward(I, u0, U, S, GS, 0.95, gamma, delta)[0]
    assert np.linalg.norm(lam32 - gI) / np.linalg.norm(gI) < 1e-5
