"""Exact (rational) hard-reset map algebra, restating the reference's lifscan/exact.py.

TEST INFRASTRUCTURE ONLY: imported by tests/ as the ground truth for map semantics; the HIP
product never imports it.

A hard-reset segment map over L steps (exact.py:64-78):

    M(u) = A*u + B          for u < x[0]
           c[i]             for x[i] <= u < x[i+1]      (x increasing, x[len] = +inf)

One step is (beta, I_t, [(theta - I_t)/beta], [u_r]) (exact.py:83-85).  Composition `then`
(exact.py:110-131): g's breakpoints pulled back through the affine part while they stay
below the first breakpoint of the earlier map, then the earlier map's constants pushed
through g; adjacent equal constants merged (exact.py:134-145).  Values are
fractions.Fraction, so every operation is exact.
"""
from dataclasses import dataclass, field
from fractions import Fraction
from typing import List


def serial_hard(I, beta, theta, u_r, u0):
    """Plain serial recurrence (exact.py:31-43) -> (states, spikes)."""
    u, us, ss = u0, [], []
    for x in I:
        v = beta * u + x
        fire = v >= theta
        u = u_r if fire else v
        us.append(u)
        ss.append(1 if fire else 0)
    return us, ss


@dataclass
class HardMap:
    A: object
    B: object
    x: List = field(default_factory=list)
    c: List = field(default_factory=list)
    L: int = 1

    @staticmethod
    def step(I_t, beta, theta, u_r):
        return HardMap(beta, I_t, [(theta - I_t) / beta], [u_r], 1)

    def __call__(self, u):
        """Evaluate (exact.py:92-104): affine below x[0], else the constant of the last
        breakpoint <= u."""
        k = -1
        for i, xi in enumerate(self.x):
            if xi <= u:
                k = i
            else:
                break
        return self.A * u + self.B if k < 0 else self.c[k]

    @property
    def pieces(self):
        return 1 + len(self.x)

    def then(self, g, merge=True):
        """g o self (apply self first)."""
        A, B = self.A, self.B
        xs, cs = [], []
        first = self.x[0] if self.x else None
        for yj, cj in zip(g.x, g.c):
            z = (yj - B) / A
            if first is not None and z >= first:
                break
            xs.append(z)
            cs.append(cj)
        for xi, ci in zip(self.x, self.c):
            xs.append(xi)
            cs.append(g(ci))
        if merge:
            xs, cs = merge_equal(xs, cs)
        return HardMap(g.A * A, g.A * B + g.B, xs, cs, self.L + g.L)


def merge_equal(x, c):
    """Drop a breakpoint whose constant equals the previous piece's (exact.py:134-145)."""
    if not x:
        return list(x), list(c)
    nx, nc = [x[0]], [c[0]]
    for xi, ci in zip(x[1:], c[1:]):
        if ci != nc[-1]:
            nx.append(xi)
            nc.append(ci)
    return nx, nc


def segment_map(I, beta, theta, u_r, merge=True):
    """Left fold of the step maps (exact.py:148-152)."""
    M = HardMap.step(I[0], beta, theta, u_r)
    for x in I[1:]:
        M = M.then(HardMap.step(x, beta, theta, u_r), merge=merge)
    return M


def closed_form_segment(I, beta, theta, u_r):
    """Theorem 1 (exact.py:155-179): breakpoints are the strict prefix minima of
    a_k = (theta - b_k)/beta^k (b_k = sum_j beta^(k-j) I_j), in increasing order; the constant
    of record k is the serial state at the end from u_r after step k.  Unmerged."""
    b, a, bk = Fraction(0), [], []
    for k, x in enumerate(I, start=1):
        b = beta * b + x
        bk.append(b)
        a.append((theta - b) / beta ** k)
    records, best = [], None
    for k in range(1, len(I) + 1):
        if best is None or a[k - 1] < best:
            records.append(k)
            best = a[k - 1]
    xs, cs = [], []
    for k in reversed(records):
        xs.append(a[k - 1])
        tail, _ = serial_hard(I[k:], beta, theta, u_r, u_r)
        cs.append(tail[-1] if tail else u_r)
    return beta ** len(I), bk[-1], xs, cs


def tree_scan_states(I, beta, theta, u_r, u0, merge=True):
    """Balanced-tree scan (exact.py:186-227): segment maps composed bottom-up, scalar states
    pushed top-down; returns (states, spikes) of every step."""
    T = len(I)
    leaves = [HardMap.step(x, beta, theta, u_r) for x in I]

    def up(lo, hi):
        if hi - lo == 1:
            return (leaves[lo], None, None, lo)
        mid = (lo + hi) // 2
        left, right = up(lo, mid), up(mid, hi)
        return (left[0].then(right[0], merge=merge), left, right, lo)

    start = [None] * T

    def down(node, u_in):
        M, left, right, lo = node
        if left is None:
            start[lo] = u_in
            return
        down(left, u_in)
        down(right, left[0](u_in))

    down(up(0, T), u0)
    us, ss = [], []
    for t in range(T):
        v = beta * start[t] + I[t]
        fire = v >= theta
        us.append(u_r if fire else v)
        ss.append(1 if fire else 0)
    return us, ss
