"""GPU paths on the reference's near-threshold stress regime (experiments/e2b_stress.py:9-27):
T 4096, N 512, beta in {0.9, 0.99}, eps in {1e-5, 1e-6, 1e-7}; 30% of the steps put the fp64
serial pre-reset potential within +-eps of theta, so the fp32 breakpoints z = num/den of the
chunk maps, and the comparisons v >= theta, are decided at near-ties.  The inputs are pinned
to the reference's record in test_stress_cpu.py.

Bars: the map scan at repair 0 equals the oracle's scan_forward_v3 bit for bit (U, S and the
stats), at the reference's K 64 and at configs[1]'s K 8; its spike flips against the serial
recurrence are printed beside the reference's (0 for fast.py at K 64).  Every exact path with
repair (map scan, associative carry, warm-started chunks, single-pass, three-level, lif_tuned)
equals the serial recurrence bit for bit, and lif_tuned's input gradient is within 1e-5 of the
fp32 oracle and 1e-4 of the fp64 adjoint.
"""
import json
import os

import numpy as np
import pytest
import torch

from oracle import lif_oracle as O
from tests._inputs import gpu, host, near_threshold

pytestmark = pytest.mark.gpu

T, N = 4096, 512
GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "e2b_stress.json")))["rows"]
_CACHE = {}


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _case(beta, eps):
    key = (beta, eps)
    if key not in _CACHE:
        _, I32 = near_threshold(T, N, beta, eps)
        U, S = O.serial_forward(I32, beta, 1.0, 0.0, np.zeros(N, np.float32))
        _CACHE.clear()  # one case at a time keeps host memory flat
        _CACHE[key] = (I32, U, S)
    return _CACHE[key]


@pytest.fixture(scope="module")
def L():
    from lifscan import hip_lif
    return hip_lif


@pytest.mark.parametrize("K", [64, 8])
@pytest.mark.parametrize("row", GOLDEN, ids=lambda r: f"b{r['beta']}-e{r['eps']}")
def test_stress_map_scan_repair0_matches_oracle(L, dev, row, K):
    beta, eps = row["beta"], row["eps"]
    I32, Us, Ss = _case(beta, eps)
    u0 = np.zeros(N, np.float32)
    print(f"stress map scan beta={beta} eps={eps} K={K}", flush=True)
    st, sto = {}, {}
    U, S = L.scan_forward_mapscan(gpu(I32, dev), beta, 1.0, 0.0, gpu(u0, dev), C=64, K=K,
                                  repair=0, stats=st)
    Uo, So = O.scan_forward_v3(I32, beta, 1.0, 0.0, u0, C=64, K=K, stats=sto)
    assert np.array_equal(host(U), Uo) and np.array_equal(host(S), So)
    for k in sto:
        assert st[k] == pytest.approx(sto[k], rel=1e-12), k
    flips = float((host(S) != Ss).mean())
    print(f"  flips vs serial {flips} (reference fast.py K 64: {row['flip_scan32_vs_ser32']}); "
          f"stats {st}", flush=True)


@pytest.mark.parametrize("row", GOLDEN, ids=lambda r: f"b{r['beta']}-e{r['eps']}")
def test_stress_exact_paths_equal_serial(L, dev, row):
    beta, eps = row["beta"], row["eps"]
    I32, Us, Ss = _case(beta, eps)
    Ig = gpu(I32, dev)
    z = torch.zeros(N, device=dev)
    R = 10 ** 6
    paths = {
        "serial": lambda: L.serial_forward(Ig, beta, 1.0, 0.0, z),
        "v3 converged": lambda: L.scan_forward_v3(Ig, beta, 1.0, 0.0, z, C=64, K=8, repair=R),
        "map scan K8 repair": lambda: L.scan_forward_mapscan(Ig, beta, 1.0, 0.0, z, C=64, K=8, repair=R),
        "map scan K64 repair": lambda: L.scan_forward_mapscan(Ig, beta, 1.0, 0.0, z, C=64, K=64, repair=R),
        "associative carry": lambda: L.scan_forward_assoc(Ig, beta, 1.0, 0.0, z, C=64, K=32),
        "warm-started": lambda: L.scan_forward_warm(Ig, beta, 1.0, 0.0, z, C=256),
        "single pass": lambda: L.scan_forward_exact(Ig, beta, 1.0, 0.0, z),
        "single pass maps": lambda: L.scan_forward_exact(Ig, beta, 1.0, 0.0, z, C=32, K=8, maps=True),
        "three-level": lambda: L.scan_forward_v4_maps(Ig, beta, 1.0, 0.0, z, C=64, G=16, K=16, K2=32, repair=R,
                                                      super_fallback="chunks"),
        "three-level as stored": lambda: L.scan_forward_v4_maps(Ig, beta, 1.0, 0.0, z, C=64, G=16, K=16,
                                                                K2=32, repair=R),
        "three-level serial fallback": lambda: L.scan_forward_v4_maps(
            Ig, beta, 1.0, 0.0, z, C=64, G=16, K=16, K2=32, repair=R, super_fallback="serial"),
    }
    for name, fn in paths.items():
        print(f"stress beta={beta} eps={eps}: {name}", flush=True)
        U, S = fn()
        assert np.array_equal(host(S), Ss), name
        assert np.array_equal(host(U), Us), name
    counters = L.last_fused_counters()
    assert counters["spin_timeouts"] == 0


@pytest.mark.parametrize("beta,eps", [(0.9, 1e-7), (0.99, 1e-7)])
def test_stress_lif_tuned_gradients(L, dev, beta, eps):
    """lif_tuned (configs[1]'s K 8, repair on) at the tightest eps: spikes equal the serial
    recurrence, dI within 1e-5 of the fp32 oracle and 1e-4 of the fp64 adjoint."""
    I32, Us, Ss = _case(beta, eps)
    G = np.random.default_rng(7).standard_normal((T, N)).astype(np.float32)
    Ig = gpu(I32, dev).requires_grad_(True)
    print(f"stress lif_tuned beta={beta} eps={eps}", flush=True)
    S = L.lif_tuned(Ig, torch.zeros(N, device=dev), beta, 1.0, 0.0, 4.0, mode="scan", K=8, repair=10 ** 6)
    (S * gpu(G, dev)).sum().backward()
    assert np.array_equal(host(S), Ss)
    u0 = np.zeros(N, np.float32)
    ref32 = O.serial_backward(I32, u0, Us, Ss, G, None, beta, 1.0, 0.0, 4.0)
    ref64 = O.serial_backward(I32, u0, Us, Ss, G, None, beta, 1.0, 0.0, 4.0, dtype=np.float64)
    e32, e64 = rel(host(Ig.grad), ref32), rel(host(Ig.grad), ref64)
    print(f"  dI rel err: {e32:.2e} vs fp32 oracle, {e64:.2e} vs fp64", flush=True)
    assert e32 < 1e-5 and e64 < 1e-4
