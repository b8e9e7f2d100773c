"""GPU parity of the warm-started converged forward (lsh_lif_scan_warm_fwd, hip_lif.scan_forward_warm)
and of the repair's early stop that it relies on.

Oracle: the serial fp32 recurrence (oracle/lif_oracle.serial_forward).  U and S must equal it bit
for bit whatever the predictions were: W = 0 (every chunk entry predicted as u_r, most of them
wrong), short warm-ups and full ones.  The number of predictions that missed is pinned against
the oracle's own count (the prediction of chunk m is by definition the serial recurrence over the
W rows before it from u_r, or from u0 when those rows reach row 0).
"""
import numpy as np
import pytest
import torch

from oracle import lif_oracle as O
from tests._inputs import host

pytestmark = pytest.mark.gpu


def _normal(T, N, mu, sd, seed):
    g = np.random.default_rng(seed)
    return (mu + sd * g.standard_normal((T, N))).astype(np.float32)


def _oracle_misses(I, beta, u0, C, W):
    """Chunk entries (m >= 1) whose warm-up prediction differs from the exit of chunk m-1 replayed
    from its own prediction (what the repair finds before its first round)."""
    T, N = I.shape
    pred = []
    for m in range(T // C):
        t0 = m * C
        w = min(W, t0)
        start = u0 if w == t0 else np.zeros(N, np.float32)
        pred.append(O.serial_forward(I[t0 - w:t0], beta, 1.0, 0.0, start)[0][-1] if w else start)
    miss = 0
    for m in range(1, T // C):
        end = O.serial_forward(I[(m - 1) * C:m * C], beta, 1.0, 0.0, pred[m - 1])[0][-1]
        miss += int((pred[m] != end).sum())
    return miss


@pytest.mark.parametrize("beta,mu,sd", [(0.9, 0.12, 0.25), (0.99, 0.012, 0.08)])
@pytest.mark.parametrize("C,W", [(64, 0), (64, 16), (256, 256), (128, 1024)])
def test_warm_forward_equals_serial(dev, beta, mu, sd, C, W):
    from lifscan import hip_lif as L
    T, N = 4096, 320
    I = _normal(T, N, mu, sd, 3)
    u0 = np.random.default_rng(4).random(N).astype(np.float32)
    print(f"warm forward beta={beta} C={C} W={W}", flush=True)
    st = {}
    U, S = L.scan_forward_warm(torch.from_numpy(I).to(dev), beta, 1.0, 0.0,
                               torch.from_numpy(u0).to(dev), C=C, W=W, stats=st)
    Uo, So = O.serial_forward(I, beta, 1.0, 0.0, u0)
    assert np.array_equal(host(U), Uo) and np.array_equal(host(S), So)
    miss = _oracle_misses(I, beta, u0, C, W)
    assert st["missed_frac"] * (T // C - 1) * N == pytest.approx(miss, abs=0.5)
    assert 0 <= st["repair_iters"] <= T // C


def test_warm_forward_ragged_and_empty(dev):
    """N not a multiple of 64, a single chunk, and empty inputs."""
    from lifscan import hip_lif as L
    for T, N, C in ((512, 65, 128), (256, 3, 256), (0, 5, 64), (128, 0, 64)):
        I = _normal(T, N, 0.012, 0.08, 5)
        u0 = np.full(N, 0.5, np.float32)
        U, S = L.scan_forward_warm(torch.from_numpy(I).to(dev), 0.99, 1.0, 0.0,
                                   torch.from_numpy(u0).to(dev), C=C, W=32)
        Uo, So = O.serial_forward(I, 0.99, 1.0, 0.0, u0)
        assert U.shape == (T, N)
        assert np.array_equal(host(U), Uo) and np.array_equal(host(S), So)


def test_warm_forward_rejects_bad_shapes(dev):
    from lifscan import hip_lif as L
    I = torch.zeros(100, 8, device=dev)
    with pytest.raises(ValueError):
        L.scan_forward_warm(I, 0.9, 1.0, 0.0, torch.zeros(8, device=dev), C=64)
    with pytest.raises(ValueError):
        L.scan_forward_warm(I, 0.9, 1.0, 0.0, torch.zeros(8, device=dev), C=50, W=-1)
