"""GPU parity of the carries' exact fallbacks in converged calls (repair to convergence, no
statistics): a lane carry (one lane per neuron: k_lif_carry, k_lif_carry_staged, v4's
k_lif_carry_inner) whose wave meets an overflowed chunk replays that chunk for all its lanes,
writes U, S and the chunk's end itself and flags the (chunk, 64-neuron block) for the replay to
skip.  The shapes put many neurons on the lane carries (more than 2048, or few chunks above
1024), a ragged last block (N not a multiple of 64, its tail lanes writing nothing), chunk lengths
that are and are not multiples of the fallback's 32-row tiles, and small capacities, so that most
waves fall back somewhere.  U and S must equal the serial recurrence bit for bit, and the same
call with statistics (which keeps the plain fallbacks) must give the same bits.
"""
import numpy as np
import pytest

from oracle import lif_oracle as O
from tests._inputs import gpu, host, normal, uniform

pytestmark = pytest.mark.gpu


# (N, C, M, K): the staged carry (M >= 4 stages of its chunks), the plain lane carry (few chunks),
# C = 100 (three 32-row tiles and 4 more rows) and C = 64 (two tiles)
@pytest.mark.parametrize("N,C,M,K", [(2113, 100, 150, 4), (4100, 64, 40, 8), (4100, 32, 96, 1),
                                     (1090, 64, 60, 2)])
def test_converged_map_scan_exact_fallbacks(dev, N, C, M, K):
    from lifscan import hip_lif as L
    T, beta = C * M, 0.99
    I = normal(T, N, 0.012, 0.08, 71)
    u0 = uniform(N, 0.0, 1.0, 72)
    Ig, u0g = gpu(I, dev), gpu(u0, dev)
    print(f"converged map scan exact fallbacks N={N} C={C} M={M} K={K}", flush=True)
    Us, Ss = O.serial_forward(I, beta, 1.0, 0.0, u0)
    U, S = L.scan_forward_mapscan(Ig, beta, 1.0, 0.0, u0g, C=C, K=K, repair=10 ** 6)
    assert np.array_equal(host(U), Us) and np.array_equal(host(S), Ss)
    st = {}
    U2, S2 = L.scan_forward_mapscan(Ig, beta, 1.0, 0.0, u0g, C=C, K=K, repair=10 ** 6, stats=st)
    assert np.array_equal(host(U2), Us) and np.array_equal(host(S2), Ss)
    print(f"  overflow_frac {st['overflow_frac']:.4f}, repair_iters {st['repair_iters']}", flush=True)
    assert st["overflow_frac"] > 0.005  # the fallbacks ran


@pytest.mark.parametrize("N,C,G,K,K2", [(2113, 64, 8, 4, 8), (4100, 32, 4, 2, 4)])
def test_converged_v4_inner_carry_exact_fallbacks(dev, N, C, G, K, K2):
    """v4 above the one-wave-per-neuron bound: the lane super carry and the lane inner carry,
    whose overflowing chunks replay for the whole wave in converged calls."""
    from lifscan import hip_lif as L
    M2, beta = 12, 0.99
    T = C * G * M2
    I = normal(T, N, 0.012, 0.08, 73)
    u0 = uniform(N, 0.0, 1.0, 74)
    Ig, u0g = gpu(I, dev), gpu(u0, dev)
    print(f"converged v4 exact fallbacks N={N} C={C} G={G} K={K} K2={K2}", flush=True)
    Us, Ss = O.serial_forward(I, beta, 1.0, 0.0, u0)
    for fb in ("chunks", "serial", "none"):
        U, S = L.scan_forward_v4_maps(Ig, beta, 1.0, 0.0, u0g, C=C, G=G, K=K, K2=K2,
                                      repair=10 ** 6, super_fallback=fb)
        assert np.array_equal(host(U), Us) and np.array_equal(host(S), Ss), fb
    st = {}
    U2, S2 = L.scan_forward_v4_maps(Ig, beta, 1.0, 0.0, u0g, C=C, G=G, K=K, K2=K2, repair=10 ** 6,
                                    stats=st)
    assert np.array_equal(host(U2), Us) and np.array_equal(host(S2), Ss)
    print(f"  overflow_frac {st['overflow_frac']:.4f}, super {st.get('super_overflow_frac')}",
          flush=True)
    assert st["overflow_frac"] > 0.005
