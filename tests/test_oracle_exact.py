"""Pins of the exact map algebra (oracle/exact_maps.py, restating exact.py) with the reference's
own seeded exact tests restated: tests/test_exact.py (random.seed(0), 3000 trials: tree scan ==
serial, left-fold map == Theorem-1 closed form, map evaluation == serial at sample states and at
every breakpoint, pieces <= T+1) and tests/test_timevarying.py (random.seed(11), 2000 trials with
time-varying leak, threshold and reset).  The same seeds and call order give the reference's
inputs; its expected outcome is "bad 0".  Then the float oracle's chunk maps are tied to the
exact algebra on dyadic inputs."""
import random
from fractions import Fraction as Fr

import numpy as np

from oracle import exact_maps as E
from oracle import lif_oracle as O


def test_reference_exact_trials():
    random.seed(0)
    for trial in range(3000):
        T = random.randint(1, 40)
        beta = Fr(random.randint(1, 10), 10)
        theta = Fr(1)
        u_r = Fr(random.choice([0, 0, 0, -3, 2, 7]), 10)
        I = [Fr(random.randint(-15, 15), 10) for _ in range(T)]
        u0 = Fr(random.randint(-30, 12), 10)
        us, ss = E.serial_hard(I, beta, theta, u_r, u0)
        u2, s2 = E.tree_scan_states(I, beta, theta, u_r, u0)
        M = E.segment_map(I, beta, theta, u_r, merge=False)
        A, B, x, c = E.closed_form_segment(I, beta, theta, u_r)
        assert us == u2 and ss == s2, trial
        assert M(u0) == us[-1] and (M.A, M.B, M.x, M.c) == (A, B, x, c) and M.pieces <= T + 1, trial
        Mm = E.segment_map(I, beta, theta, u_r, merge=True)
        for uu in [Fr(random.randint(-50, 20), 10) for _ in range(5)] + x:
            want = E.serial_hard(I, beta, theta, u_r, uu)[0][-1]
            assert M(uu) == want and Mm(uu) == want, trial


def test_reference_timevarying_trials():
    def serial(I, al, th, rr, u0):
        u, us = u0, []
        for x, a, t, r in zip(I, al, th, rr):
            v = a * u + x
            u = r if v >= t else v
            us.append(u)
        return us

    random.seed(11)
    for trial in range(2000):
        L = random.randint(1, 30)
        I = [Fr(random.randint(-15, 20), 10) for _ in range(L)]
        al = [Fr(random.randint(1, 15), 10) for _ in range(L)]
        th = [Fr(random.randint(5, 20), 10) for _ in range(L)]
        rr = [Fr(random.randint(-5, 5), 10) for _ in range(L)]
        steps = [E.HardMap(a, x, [(t - x) / a], [r], 1) for x, a, t, r in zip(I, al, th, rr)]
        M = steps[0]
        for s in steps[1:]:
            M = M.then(s)
        assert M.pieces <= L + 1
        for u0 in [Fr(random.randint(-60, 30), 10) for _ in range(6)] + list(M.x):
            assert M(u0) == serial(I, al, th, rr, u0)[-1], trial
        u0 = Fr(random.randint(-20, 10), 10)
        P = steps[0]
        ser = serial(I, al, th, rr, u0)
        assert P(u0) == ser[0]
        for k in range(1, L):
            P = P.then(steps[k])
            assert P(u0) == ser[k], trial


def test_float_chunk_maps_equal_exact_algebra_on_dyadic_inputs():
    """beta = 1/2 and inputs on a 1/64 grid make every fp32 operation of the float build exact:
    the float oracle's unpruned chunk map (capacity C, lo = -inf, hi = +inf) is then the exact
    left fold's map, breakpoint for breakpoint (descending order in the float layout)."""
    rng = np.random.default_rng(5)
    C, N = 12, 40
    I = (rng.integers(-40, 96, size=(C, N)) / 64.0).astype(np.float32)
    lo = np.full(N, -np.inf, np.float32)
    hi = np.full(N, np.inf, np.float32)
    A, B, xd, cd, n, ovf = O.build_maps(I, 0.5, 1.0, 0.0, lo, hi, C, C)
    for j in range(N):
        M = E.segment_map([Fr(float(v)) for v in I[:, j]], Fr(1, 2), Fr(1), Fr(0), merge=False)
        assert Fr(float(A[0, j])) == M.A and Fr(float(B[0, j])) == M.B
        k = int(n[0, j])
        assert k == len(M.x) and not ovf[0, j]
        assert [Fr(float(v)) for v in xd[0, :k, j]] == M.x[::-1]
        assert [Fr(float(v)) for v in cd[0, :k, j]] == M.c[::-1]
