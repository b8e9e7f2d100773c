"""CPU pins of the associative-carry oracle (oracle/map_scan.py), the checker of k_map_scan.

  * the wave scan's association order: with a non-commutative monoid (list concatenation) every
    lane gets exactly the lanes 0..l in order, so a wrong DPP source (row, broadcast lane) fails;
  * compose() is the reference's monoid: equal, slot for slot, to the sequential group
    composition of lif_oracle.compose_groups (pinned to exact maps in test_oracle_lif.py) for
    G = 2, on random fp32 maps;
  * on inputs where fp32 arithmetic is exact (beta = 1, theta = 1, inputs on a 1/4 grid: every
    state, breakpoint and affine part is a small multiple of 1/4) the tree-scan chunk starts
    equal the serial recurrence's states exactly, through several waves and tiles, overflowed
    chunks (K small) and ties v == theta.
"""
import numpy as np
import pytest

from oracle import lif_oracle as O
from oracle import map_scan as MS

f32 = np.float32


def test_wave_scan_order_is_lane_order():
    vals = [[l] for l in range(64)]
    out = MS.wave_scan(vals, lambda a, b: a + b)
    for l in range(64):
        assert out[l] == list(range(l + 1))
    # inactive lanes keep their own value
    act = [l < 3 for l in range(64)]
    out = MS.wave_scan(vals, lambda a, b: a + b, active=act)
    assert out[:3] == [[0], [0, 1], [0, 1, 2]] and out[5] == [5]


def _chunk_arrays(I, beta, theta, u_r, u0, C, K):
    T, N = I.shape
    hi = np.maximum(np.asarray(u0, f32), max(f32(theta), f32(u_r)))
    EC, EA, EB = O.envelope_chunks(I, beta, u_r, C)
    A, B, xd, cd, cnt, ovf = O.build_maps(I, beta, theta, u_r, -np.inf, hi, C, K)
    return EC, EA, EB, A, B, cnt, ovf, xd, cd


@pytest.mark.parametrize("seed", [0, 1])
def test_compose_equals_sequential_group_composition(seed):
    rng = np.random.default_rng(seed)
    T, N, C, K, beta = 64 * 16, 24, 64, 16, 0.95
    I = (0.1 + 0.35 * rng.standard_normal((T, N))).astype(f32)
    u0 = rng.uniform(-0.5, 0.9, N).astype(f32)
    EC, EA, EB, A, B, cnt, ovf, xd, cd = _chunk_arrays(I, beta, 1.0, 0.0, u0, C, K)
    Lo = O.envelope_carry(u0, EC, EA, EB)
    # truncate at Lo as the scans do
    M = T // C
    n = np.zeros((M, N), np.int32)
    ov = np.zeros((M, N), np.int32)
    for m in range(M):
        gt = ((xd[m] > Lo[m][None]) & (np.arange(K)[:, None] < cnt[m][None])).sum(0)
        n[m] = np.minimum(cnt[m], gt + 1)
        ov[m] = (ovf[m] > 0) & (gt == cnt[m])
    SA, SB, SX, SC, SN, SOVF = O.compose_groups(A, B, xd, cd, n, ov, Lo, u0, 1.0, 0.0, 2, MS.KS)
    hi = np.maximum(u0, f32(1.0))
    checked = 0
    for s in range(M // 2):
        for j in range(N):
            m0 = 2 * s
            if ov[m0, j] or ov[m0 + 1, j]:
                continue
            H = MS.Elem(A[m0, j], B[m0, j], Lo[m0, j],
                        [(xd[m0, i, j], cd[m0, i, j]) for i in range(n[m0, j])], 0)
            g = MS.Elem(A[m0 + 1, j], B[m0 + 1, j], Lo[m0 + 1, j],
                        [(xd[m0 + 1, i, j], cd[m0 + 1, i, j]) for i in range(n[m0 + 1, j])], 0)
            R = MS.compose(H, g, hi[j])
            assert R.A == SA[s, j] and R.B == SB[s, j] and len(R.slots) == SN[s, j]
            for i, (x, c) in enumerate(R.slots):
                assert x == SX[s, i, j] and c == SC[s, i, j]
            checked += 1
    assert checked > 100


@pytest.mark.parametrize("K,WG,KS", [(16, 2, 32), (4, 1, 32), (2, 4, 32), (8, 2, 3)])
def test_tree_scan_starts_are_exact_on_exact_arithmetic(monkeypatch, K, WG, KS):
    """KS = 3 forces compositions past the capacity, so the sequential fallback runs too."""
    monkeypatch.setattr(MS, "KS", KS)
    rng = np.random.default_rng(5)
    C, M, N = 8, 300, 6
    T = C * M
    I = (rng.integers(-3, 5, (T, N)) / 4.0).astype(f32)
    u0 = (rng.integers(-8, 4, N) / 4.0).astype(f32)
    beta, theta, u_r = 1.0, 1.0, 0.0
    arrs = _chunk_arrays(I, beta, theta, u_r, u0, C, K)
    LO, MN, OVF, ST = MS.map_scan_carry(*arrs, I, u0, beta, theta, u_r, C, WG)
    U, S = O.serial_forward(I, beta, theta, u_r, u0)
    true = np.concatenate([u0[None], U[C - 1::C][:-1]], 0)
    assert np.array_equal(ST, true)
    assert (S == 1).sum() > 100
    if K <= 4:
        assert OVF.sum() > 0  # the overflow path (serial heads) was taken
    # the envelope bounds lie below the states they bound
    assert (LO <= true).all()
