"""Pins of the CPU oracle (oracle/lif_oracle.py) against what the mathematics fixes.

The reference commits no golden vectors for this path, so the oracle is pinned by
  * exact rational arithmetic with fp32 round-to-nearest-even emulated per operation
    (an independent statement of the two-rounding step v = fl(fl(beta*u) + x));
  * dyadic inputs on which every fp32 operation is exact, compared with the exact
    recurrence (exact.py:31-43 serial_hard) and the Theorem-1 closed form of the chunk map
    (paper/main.tex:132-140, exact.py:154-179) including the lo/hi pruning rule;
  * brute force: map evaluation vs serial simulation; envelope <= trajectory (lemma,
    paper/main.tex:266-272); Jacobi repair rounds against their definition;
  * fp64 autograd through the serial recurrence for the adjoint (fast.py:54-66).
"""
import math
from fractions import Fraction as Fr

import numpy as np
import pytest
import torch

from oracle import lif_oracle as O
from tests._inputs import normal, uniform

F32_MAX = (2 - Fr(1, 2 ** 23)) * Fr(2) ** 127


def round_f32(q):
    """Nearest binary32 value of the rational q (ties to even), as a Fraction (own code)."""
    if q == 0:
        return Fr(0)
    sign = -1 if q < 0 else 1
    a = abs(Fr(q))
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fr(2) ** e > a:
        e -= 1
    while Fr(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)
    ulp = Fr(2) ** (e - 23)
    k = a / ulp
    n = k.numerator // k.denominator
    r = k - n
    if r > Fr(1, 2) or (r == Fr(1, 2) and n % 2 == 1):
        n += 1
    val = n * ulp
    if val > F32_MAX:
        return sign * Fr(10) ** 400  # stands for inf; never reached by the tests
    return sign * val


def test_round_f32_matches_numpy_conversion():
    rng = np.random.default_rng(0)
    for v in rng.standard_normal(200) * 10.0 ** rng.integers(-40, 30, 200):
        assert Fr(float(np.float32(v))) == round_f32(Fr(float(v)))
    assert round_f32(Fr(1, 3)) == Fr(float(np.float32(1 / 3)))
    # subnormal
    assert round_f32(Fr(3, 2 ** 149)) == Fr(3, 2 ** 149)


@pytest.mark.parametrize("beta,u_r,mu,sd,seed", [
    (0.9, 0.0, 0.12, 0.25, 0), (0.99, 0.0, 0.012, 0.08, 1), (0.5, -0.1, 0.4, 0.3, 2),
    (1.0, -0.2, 0.05, 0.3, 3), (0.95, 0.0, 0.15, 0.4, 4)])
def test_serial_forward_is_two_rounding_step(beta, u_r, mu, sd, seed):
    T, N = 60, 6
    I = normal(T, N, mu, sd, seed)
    u0 = uniform(N, -0.5, 1.0, seed + 100)
    U, S = O.serial_forward(I, beta, 1.0, u_r, u0)
    b, th, ur = (Fr(float(np.float32(v))) for v in (beta, 1.0, u_r))
    for n in range(N):
        u = Fr(float(u0[n]))
        for t in range(T):
            v = round_f32(round_f32(b * u) + Fr(float(I[t, n])))
            s = v >= th
            u = ur if s else v
            assert Fr(float(U[t, n])) == u, (n, t)
            assert S[t, n] == (1.0 if s else 0.0)


def _serial_exact(I, beta, theta, u_r, u0):
    """Exact rational serial recurrence (restates exact.py:31-43)."""
    u, us, ss = u0, [], []
    for x in I:
        v = beta * u + x
        if v >= theta:
            u, s = u_r, 1
        else:
            u, s = v, 0
        us.append(u)
        ss.append(s)
    return us, ss


def _dyadic_case(rng, T, lo=-16, hi=24, den=16):
    return [Fr(int(k), den) for k in rng.integers(lo, hi, T)]


def test_serial_dyadic_is_exact_with_ties():
    """beta = 1/2 and inputs on a 1/64 grid: every fp32 operation is exact, so the oracle
    equals the exact recurrence, including exact ties v == theta (e2_float.py:30-41)."""
    rng = np.random.default_rng(7)
    T, N = 20, 50
    ties = 0
    for n in range(N):
        xs = [Fr(int(k), 64) for k in rng.integers(-40, 80, T)]
        u0 = Fr(int(rng.integers(-64, 64)), 64)
        us, ss = _serial_exact(xs, Fr(1, 2), Fr(1), Fr(0), u0)
        I = np.array([[float(x)] for x in xs], dtype=np.float32)
        U, S = O.serial_forward(I, 0.5, 1.0, 0.0, np.array([float(u0)], np.float32))
        assert [Fr(float(v)) for v in U[:, 0]] == us
        assert [int(v) for v in S[:, 0]] == ss
        u = u0
        for x in xs:
            v = u / 2 + x
            ties += v == 1
            u = 0 if v >= 1 else v
    assert ties > 0


def _closed_form(I, beta, theta, u_r):
    """Theorem 1 (paper/main.tex:132-140; exact.py:154-179): breakpoints are the strict
    prefix minima a_k = (theta - b_k)/beta^k of the zero-start free trajectory b_k, listed
    in the order they appear (descending); constants are the serial tail from u_r."""
    b, recs, cur, a = Fr(0), [], None, []
    bk = []
    for k, x in enumerate(I, start=1):
        b = beta * b + x
        bk.append(b)
        a.append((theta - b) / beta ** k)
    for k in range(1, len(I) + 1):
        if cur is None or a[k - 1] < cur:
            recs.append(k)
            cur = a[k - 1]
    xs, cs = [], []
    for k in recs:
        xs.append(a[k - 1])
        tail, _ = _serial_exact(I[k:], beta, theta, u_r, u_r)
        cs.append(tail[-1] if tail else u_r)
    return beta ** len(I), bk[-1], xs, cs


@pytest.mark.parametrize("u_r", [Fr(0), Fr(-1, 4)])
def test_build_maps_equal_closed_form_on_exact_inputs(u_r):
    rng = np.random.default_rng(11)
    C, N = 8, 64
    cols = [_dyadic_case(rng, C) for _ in range(N)]
    I = np.array([[float(c[t]) for c in cols] for t in range(C)], dtype=np.float32)
    A, B, xd, cd, n, ovf = O.build_maps(I, 0.5, 1.0, float(u_r), np.full(N, -np.inf, np.float32),
                                        np.full(N, np.inf, np.float32), C, C)
    for j in range(N):
        Ae, Be, xs, cs = _closed_form(cols[j], Fr(1, 2), Fr(1), u_r)
        assert Fr(float(A[0, j])) == Ae and Fr(float(B[0, j])) == Be
        assert n[0, j] == len(xs) and ovf[0, j] == 0
        assert [Fr(float(v)) for v in xd[0, :n[0, j], j]] == xs
        assert [Fr(float(v)) for v in cd[0, :n[0, j], j]] == cs


def test_build_maps_pruning_rule_on_exact_inputs():
    """Pruned map = records <= hi, cut after the first record <= lo; overflow iff more
    than K such records are needed (triton_lif.py:760-764)."""
    rng = np.random.default_rng(12)
    C, N = 8, 200
    cols = [_dyadic_case(rng, C, -24, 30) for _ in range(N)]
    I = np.array([[float(c[t]) for c in cols] for t in range(C)], dtype=np.float32)
    lo = np.array([float(Fr(int(k), 8)) for k in rng.integers(-30, 4, N)], np.float32)
    hi = np.array([float(Fr(int(k), 8)) for k in rng.integers(0, 30, N)], np.float32)
    for K in (1, 2, 3, 8):
        A, B, xd, cd, n, ovf = O.build_maps(I, 0.5, 1.0, 0.0, lo, hi, C, K)
        for j in range(N):
            _, _, xs, cs = _closed_form(cols[j], Fr(1, 2), Fr(1), Fr(0))
            keep = []
            for z, c in zip(xs, cs):
                if z > Fr(float(hi[j])):
                    continue
                keep.append((z, c))
                if z <= Fr(float(lo[j])):
                    break
            want = keep[:K]
            assert n[0, j] == len(want)
            assert ovf[0, j] == (1 if len(keep) > K else 0)
            assert [Fr(float(v)) for v in xd[0, :n[0, j], j]] == [z for z, _ in want]
            assert [Fr(float(v)) for v in cd[0, :n[0, j], j]] == [c for _, c in want]


def test_map_evaluation_matches_serial_segment():
    """Brute force on float inputs: a state in a constant piece maps to exactly the serial
    end state (same step arithmetic); affine pieces agree to rounding."""
    T, N, C, K = 256, 512, 64, 16
    I = normal(T, N, 0.12, 0.25, 5)
    u0 = np.zeros(N, np.float32)
    keep = {}
    O.scan_forward_v3(I, 0.9, 1.0, 0.0, u0, C=C, K=K, keep=keep)
    rng = np.random.default_rng(3)
    checked_const = 0
    for m in range(T // C):
        u = (keep["Lo"][m] + rng.random(N).astype(np.float32) * (1.0 - keep["Lo"][m])).astype(np.float32)
        got = O.eval_map(keep["A"][m], keep["B"][m], keep["xd"][m], keep["cd"][m], keep["n"][m], u)
        ref = O.serial_segment(I[m * C:(m + 1) * C], 0.9, 1.0, 0.0, u)
        nv = keep["n"][m]
        k = ((keep["xd"][m] > u[None]) & (np.arange(K)[:, None] < nv[None])).sum(0)
        ok = keep["ovf"][m] == 0
        xdv = np.where(np.arange(K)[:, None] < nv[None], keep["xd"][m], np.inf)
        near = (np.abs(xdv - u[None]) <= 1e-5 * (np.abs(u[None]) + 1)).any(0)
        const = ok & (k < nv) & ~near
        assert np.array_equal(got[const], ref[const])
        aff = ok & (k == nv) & ~near
        assert np.allclose(got[aff], ref[aff], rtol=1e-5, atol=1e-6)
        checked_const += int(const.sum())
    assert checked_const > 100


@pytest.mark.parametrize("beta,mu,sd", [(0.9, 0.12, 0.25), (0.99, 0.012, 0.08), (0.5, -0.1, 0.6),
                                        (1.0, 0.05, 0.3)])
def test_envelope_is_below_the_trajectory(beta, mu, sd):
    T, N, C = 1024, 256, 64
    I = normal(T, N, mu, sd, 8)
    u0 = uniform(N, -0.3, 0.9, 9)
    U, _ = O.serial_forward(I, beta, 1.0, 0.0, u0)
    EC, EA, EB = O.envelope_chunks(I, beta, 0.0, C)
    Lo = O.envelope_carry(u0, EC, EA, EB)
    starts = np.concatenate([u0[None], U[C - 1:-1:C]], 0)
    assert (Lo <= starts).all()


@pytest.mark.parametrize("beta,mu,sd", [(0.9, 0.12, 0.25), (0.99, 0.012, 0.08), (0.5, -0.1, 0.6),
                                        (1.0, 0.05, 0.3)])
def test_envelope_bound_equals_stepwise_brute_force(beta, mu, sd):
    """Lo at every chunk start against the stepwise envelope l_t = min(u_r, beta*l_{t-1} + x_t),
    l_0 = u0, run in fp64 over all T steps, minus the margin 1e-5(|l| + 1): two-sided, to 3e-6
    (|l| + 1) (the fp32 chunk sums of 64 steps round to ~1e-6 at beta = 1), so a wrong margin, a
    dropped min or a wrong composition fails (a bound that is merely below the trajectory would
    pass test_envelope_is_below_the_trajectory)."""
    T, N, C, u_r = 1024, 256, 64, -0.1
    I = normal(T, N, mu, sd, 10)
    u0 = uniform(N, -0.3, 0.9, 11)
    EC, EA, EB = O.envelope_chunks(I, beta, u_r, C)
    Lo = O.envelope_carry(u0, EC, EA, EB)
    l = u0.astype(np.float64)
    b = np.float64(np.float32(beta))
    want = np.empty((T // C, N))
    for t in range(T):
        if t % C == 0:
            want[t // C] = l - 1e-5 * (np.abs(l) + 1.0)
        l = np.minimum(np.float64(np.float32(u_r)), b * l + I[t].astype(np.float64))
    assert np.all(np.abs(Lo - want) <= 3e-6 * (np.abs(want) + 1.0))


def test_envelope_chunk_map_is_the_closed_form_composition():
    """On dyadic inputs (beta = 1/2, x on a 1/64 grid, 8-step chunks: every fp32 operation is
    exact) the chunk map l -> min(c, a*l + b) equals the 8-step min-affine recurrence from
    every entry l exactly, with a = beta^8 (the composition lemma of paper/main.tex:266-272)."""
    C, N = 8, 64
    g = np.random.default_rng(3)
    I = (g.integers(-32, 48, size=(4 * C, N)) / 64.0).astype(np.float32)
    EC, EA, EB = O.envelope_chunks(I, 0.5, 0.0, C)
    assert np.all(EA == np.float32(0.5 ** C))
    for l0 in (np.float32(-3.0), np.float32(-0.25), np.float32(0.0), np.float32(0.75)):
        for m in range(I.shape[0] // C):
            l = np.full(N, l0, np.float32)
            for t in range(m * C, (m + 1) * C):
                l = np.minimum(np.float32(0.0), np.float32(0.5) * l + I[t])
            got = np.minimum(EC[m], EA[m] * l0 + EB[m])
            assert np.array_equal(got, l), (l0, m)


def test_long_sequence_fp64_adjoint_equals_the_serial_one():
    T, N = 4096, 32
    I = normal(T, N, 0.012, 0.08, 51)
    u0 = uniform(N, 0.0, 1.0, 52)
    GS = normal(T, N, 0.0, 1.0, 53)
    U, S = O.serial_forward(I, 0.99, 1.0, 0.0, u0)
    ref = O.serial_backward(I, u0, U, S, GS, None, 0.99, 1.0, 0.0, 4.0, dtype=np.float64)
    got = O.serial_backward_long(I, u0, U, S, GS, 0.99, 1.0, 0.0, 4.0, block=256)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 1e-12


REGIMES = [(b, mu, sd) for b in (0.5, 0.9, 0.99, 1.0) for (mu, sd) in ((0.15, 0.4), (-0.1, 0.6), (0.4, 0.2))]


@pytest.mark.parametrize("beta,mu,sd", REGIMES)
def test_scan_with_repair_equals_serial(beta, mu, sd):
    """The reference's own contract (fast.py:13-15, paper/main.tex:318-319)."""
    T, N = 1024, 96
    I = normal(T, N, mu, sd, 1)
    u0 = uniform(N, -0.3, 0.3, 2)
    Us, Ss = O.serial_forward(I, beta, 1.0, -0.1, u0)
    for K in (2, 4, 16):
        st = {}
        U, S = O.scan_forward_v3(I, beta, 1.0, -0.1, u0, C=64, K=K, repair=10 ** 6, stats=st)
        assert np.array_equal(U, Us) and np.array_equal(S, Ss)
        assert st["repair_iters"] <= T // 64


def _jacobi_by_definition(I, beta, theta, u_r, u0, starts0, C, R):
    """Starts after R rounds, by definition: S^R_m = serial from S^0_{m-R} across chunks
    m-R .. m-1 (exact start from u0 when m < R)."""
    T, N = I.shape
    M = T // C
    Us, _ = O.serial_forward(I, beta, theta, u_r, u0)
    exact = np.concatenate([u0[None], Us[C - 1:-1:C]], 0)
    out = np.empty_like(starts0)
    for m in range(M):
        if m < R:
            out[m] = exact[m]
        else:
            out[m] = O.serial_segment(I[(m - R) * C:m * C], beta, theta, u_r, starts0[m - R]) if R else starts0[m]
    return out


def test_finite_repair_rounds_follow_their_definition():
    T, N, C = 2048, 128, 64
    I = normal(T, N, 0.012, 0.08, 21)
    u0 = np.zeros(N, np.float32)
    keep = {}
    O.scan_forward_v3(I, 0.99, 1.0, 0.0, u0, C=C, K=4, repair=0, keep=keep)
    s0 = keep["starts"]
    st = {}
    O.scan_forward_v3(I, 0.99, 1.0, 0.0, u0, C=C, K=4, repair=10 ** 6, stats=st)
    rounds = st["repair_iters"]
    assert rounds >= 2
    for R in range(0, rounds + 2):
        want = _jacobi_by_definition(I, 0.99, 1.0, 0.0, u0, s0, C, R)
        U, S, _ = O.replay(I, want, 0.99, 1.0, 0.0, C)
        kp = {}
        U2, S2 = O.scan_forward_v3(I, 0.99, 1.0, 0.0, u0, C=C, K=4, repair=R, keep=kp)
        assert np.array_equal(kp["starts"], want), R
        assert np.array_equal(U2, U) and np.array_equal(S2, S)
    # the round count is the first R whose starts are exact
    Us, _ = O.serial_forward(I, 0.99, 1.0, 0.0, u0)
    exact = np.concatenate([u0[None], Us[C - 1:-1:C]], 0)
    first = next(R for R in range(0, T // C + 1)
                 if np.array_equal(_jacobi_by_definition(I, 0.99, 1.0, 0.0, u0, s0, C, R), exact))
    assert first == rounds


def _autograd_adjoint(I, u0, S32, GS, beta, theta, u_r, alpha, detach):
    """fp64 autograd through the serial recurrence with the fp32 run's spike pattern as the
    (detached) reset mask and the sigmoid surrogate as d s/d v (fast.py:33-66).  The state
    values are pinned to the fp32 trajectory (a detached correction term), so the surrogate
    is evaluated where the kernels evaluate it; derivatives are those of the recurrence."""
    Id = torch.tensor(I, dtype=torch.float64, requires_grad=True)
    u0d = torch.tensor(u0, dtype=torch.float64, requires_grad=True)
    Sd = torch.tensor(S32, dtype=torch.float64)
    U32, _ = O.serial_forward(I, beta, theta, u_r, u0)
    U32 = torch.tensor(U32, dtype=torch.float64)
    u = u0d
    loss = 0
    for t in range(I.shape[0]):
        if t > 0:
            u = u + (U32[t - 1] - u).detach()
        v = beta * u + Id[t]
        sg = torch.sigmoid(alpha * (v - theta))
        s = Sd[t] + (sg - sg.detach())  # value = fp32 spike, derivative = surrogate
        sr = Sd[t] if detach else s
        u = v * (1 - sr) + u_r * sr
        loss = loss + (torch.tensor(GS[t], dtype=torch.float64) * s).sum()
    gI, g0 = torch.autograd.grad(loss, (Id, u0d))
    return gI.numpy(), g0.numpy()


@pytest.mark.parametrize("detach", [True, False])
def test_adjoint_matches_fp64_autograd(detach):
    T, N = 256, 16
    I = normal(T, N, 0.15, 0.4, 31)
    u0 = uniform(N, -0.2, 0.5, 32)
    GS = normal(T, N, 0.0, 1.0, 33)
    U, S = O.serial_forward(I, 0.9, 1.0, -0.1, u0)
    Lam = O.serial_backward(I, u0, U, S, GS, None, 0.9, 1.0, -0.1, 4.0, detach, dtype=np.float64)
    gI, g0 = _autograd_adjoint(I, u0, S, GS, 0.9, 1.0, -0.1, 4.0, detach)
    assert np.linalg.norm(Lam - gI) / np.linalg.norm(gI) < 1e-10
    assert np.allclose(0.9 * Lam[0], g0, rtol=1e-10, atol=1e-12)


def test_scan_backward_matches_serial_adjoint():
    T, N = 1024, 64
    I = normal(T, N, 0.15, 0.4, 41)
    u0 = np.zeros(N, np.float32)
    GS = normal(T, N, 0.0, 1.0, 42)
    GU = normal(T, N, 0.0, 1.0, 43)
    U, S = O.serial_forward(I, 0.9, 1.0, 0.0, u0)
    for detach, gu in ((True, None), (False, GU)):
        ref = O.serial_backward(I, u0, U, S, GS, gu, 0.9, 1.0, 0.0, 4.0, detach, dtype=np.float64)
        L32 = O.serial_backward(I, u0, U, S, GS, gu, 0.9, 1.0, 0.0, 4.0, detach)
        Lsc = O.scan_backward(I, u0, U, S, GS, gu, 0.9, 1.0, 0.0, 4.0, detach, C=64)
        assert np.linalg.norm(L32 - ref) / np.linalg.norm(ref) < 1e-5
        assert np.linalg.norm(Lsc - ref) / np.linalg.norm(ref) < 1e-5


def test_pick_C_policy():
    assert O.pick_C(4096, 16) == 128 and O.pick_C(1024, 16) == 64 and O.pick_C(2 ** 20, 16) == 256
    with pytest.raises(ValueError):
        O.pick_C(100, 16)


def test_group_composition_equals_map_of_concatenation():
    """Maps are closed under composition (paper/main.tex:132-140; exact.py:108-131): on exact
    inputs, composing G chunk maps (unpruned) gives the Theorem-1 map of the G*C-step segment."""
    rng = np.random.default_rng(21)
    C, G, N = 4, 4, 48
    cols = [_dyadic_case(rng, C * G, -12, 20) for _ in range(N)]
    I = np.array([[float(c[t]) for c in cols] for t in range(C * G)], dtype=np.float32)
    M = G
    lo = np.full((M, N), -np.inf, np.float32)
    hi = np.full(N, np.inf, np.float32)
    A, B, xd, cd, n, ovf = O.build_maps(I, 0.5, 1.0, 0.0, lo, hi, C, C)
    SA, SB, SX, SC, SN, SOVF = O.compose_groups(A, B, xd, cd, n, ovf, lo, np.zeros(N, np.float32) - 1e30,
                                                1e30, 0.0, G, C * G)
    for j in range(N):
        Ae, Be, xs, cs = _closed_form(cols[j], Fr(1, 2), Fr(1), Fr(0))
        assert Fr(float(SA[0, j])) == Ae and Fr(float(SB[0, j])) == Be
        assert SN[0, j] == len(xs) and SOVF[0, j] == 0
        assert [Fr(float(v)) for v in SX[0, :SN[0, j], j]] == xs
        assert [Fr(float(v)) for v in SC[0, :SN[0, j], j]] == cs


@pytest.mark.parametrize("beta,mu,sd", [(0.9, 0.15, 0.4), (0.99, 0.012, 0.08), (0.5, -0.1, 0.6), (1.0, 0.4, 0.2)])
def test_scan_v4_with_repair_equals_serial(beta, mu, sd):
    T, N = 2048, 64
    I = normal(T, N, mu, sd, 22)
    u0 = uniform(N, -0.3, 0.3, 23)
    Us, Ss = O.serial_forward(I, beta, 1.0, -0.1, u0)
    for K, K2 in ((16, 32), (8, 16), (2, 4)):
        st = {}
        U, S = O.scan_forward_v4(I, beta, 1.0, -0.1, u0, C=64, G=8, K=K, K2=K2, repair=10 ** 6, stats=st)
        assert np.array_equal(U, Us) and np.array_equal(S, Ss)
        assert set(st) == {"repair_iters", "overflow_frac", "super_overflow_frac", "mean_pieces",
                           "super_mean_pieces", "super_max_pieces"}


def test_scan_v4_super_starts_match_serial_where_maps_are_exact():
    """Super-chunk starts read off the composed maps equal the serial states at super
    boundaries except where a map's affine piece or overflow makes them approximate."""
    T, N, C, G = 4096, 128, 64, 8
    I = normal(T, N, 0.15, 0.4, 24)
    u0 = np.zeros(N, np.float32)
    keep = {}
    O.scan_forward_v4(I, 0.9, 1.0, 0.0, u0, C=C, G=G, K=16, K2=32, keep=keep)
    Us, _ = O.serial_forward(I, 0.9, 1.0, 0.0, u0)
    exact = np.concatenate([u0[None], Us[C * G - 1:-1:C * G]], 0)
    frac = (keep["sstarts"] == exact).mean()
    assert frac > 0.99


@pytest.mark.parametrize("fallback", ["chunks", "serial"])
def test_carry_super_fallbacks_exact_on_dyadic_inputs(fallback):
    """beta = 1/2 and inputs on a 1/4 grid, with spikes often enough that every fp32 state is
    exact (checked against the rational recurrence first): every map evaluation is then exact,
    so the super starts equal the serial states at every super boundary, for both ways of
    passing an overflowed super map (capacity 1 for chunk and super maps: 74% of the super maps
    and 26% of the chunk maps overflow, so the walk evaluates chunk maps and runs chunks
    serially)."""
    rng = np.random.default_rng(31)
    C, G, M2, N = 4, 4, 16, 64
    T = C * G * M2
    cols = [_dyadic_case(rng, T, -4, 9, den=4) for _ in range(N)]
    I = np.array([[float(c[t]) for c in cols] for t in range(T)], dtype=np.float32)
    u0 = np.zeros(N, np.float32)
    Us, _ = O.serial_forward(I, 0.5, 1.0, 0.0, u0)
    for j in range(N):  # precondition: the fp32 recurrence is the exact one
        us, _ = _serial_exact(cols[j], Fr(1, 2), Fr(1), Fr(0), Fr(0))
        assert [Fr(float(v)) for v in Us[:, j]] == us
    keep = {}
    O.scan_forward_v4(I, 0.5, 1.0, 0.0, u0, C=C, G=G, K=1, K2=1, keep=keep, super_fallback=fallback)
    assert keep["SOVF"].mean() > 0.5 and keep["ovf"].mean() > 0.1
    exact = np.concatenate([u0[None], Us[C * G - 1:-1:C * G]], 0)
    assert np.array_equal(keep["sstarts"], exact)


def test_carry_super_chunks_continues_the_inner_carry():
    """With the "chunks" fallback the start of the super map after an overflowed one is the
    state the inner carry reaches at the end of the overflowed one (its last chunk start
    carried through its last chunk map, or that chunk's serial steps where it overflowed); with
    "serial" it is the serial state instead."""
    T, N, C, G = 4096, 96, 64, 8
    I = normal(T, N, 0.012, 0.08, 33)
    u0 = uniform(N, 0.0, 1.0, 34)
    for fallback in ("chunks", "serial"):
        keep = {}
        O.scan_forward_v4(I, 0.99, 1.0, 0.0, u0, C=C, G=G, K=8, K2=8, keep=keep, super_fallback=fallback)
        assert keep["SOVF"].mean() > 0.2
        starts, ss = keep["starts"], keep["sstarts"]
        M2 = ss.shape[0]
        for s_ in range(M2 - 1):
            m = s_ * G + G - 1
            end = O.eval_map(keep["A"][m], keep["B"][m], keep["xd"][m], keep["cd"][m], keep["n"][m], starts[m])
            ser = O.serial_segment(I[m * C:(m + 1) * C], 0.99, 1.0, 0.0, starts[m])
            end = np.where(keep["ovf"][m] > 0, ser, end)
            full = O.serial_segment(I[s_ * C * G:(s_ + 1) * C * G], 0.99, 1.0, 0.0, ss[s_])
            bad = keep["SOVF"][s_] > 0
            want = end if fallback == "chunks" else full
            assert np.array_equal(ss[s_ + 1][bad], want[bad]), (fallback, s_)


def test_carry_super_as_stored_then_repair_is_serial():
    """Fallback "none" passes an overflowed super map as stored: its next start is the stored
    map's value (a start that may be wrong), and with repair to convergence the scan is the
    serial recurrence all the same."""
    T, N, C, G = 4096, 96, 64, 8
    I = normal(T, N, 0.012, 0.08, 35)
    u0 = uniform(N, 0.0, 1.0, 36)
    keep = {}
    U, S = O.scan_forward_v4(I, 0.99, 1.0, 0.0, u0, C=C, G=G, K=4, K2=8, repair=T // C, keep=keep,
                             super_fallback="none")
    assert keep["SOVF"].mean() > 0.2
    ss = keep["sstarts"]
    for s_ in range(ss.shape[0] - 1):
        want = O.eval_map(keep["SA"][s_], keep["SB"][s_], keep["SX"][s_], keep["SC"][s_],
                          keep["SN"][s_], ss[s_])
        assert np.array_equal(ss[s_ + 1], want), s_
    Us, Ss = O.serial_forward(I, 0.99, 1.0, 0.0, u0)
    assert np.array_equal(U, Us) and np.array_equal(S, Ss)
