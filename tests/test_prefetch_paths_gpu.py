"""GPU parity of the walks that read their data ahead of use, at shapes that exercise the ends of
their read-ahead (odd counts, partial tiles), and of the warm-start plan for few neurons.

  * v4's super-map carry (maps one ahead in a ring of two): an odd number of super maps; every
    intermediate equals the oracle's bit for bit and repair gives the serial recurrence;
  * the ALIF envelope carry (chunk maps in tiles of 16): 40 chunks, two tiles and a partial one;
    the entry bounds LU and every later intermediate equal the oracle's;
  * the converged scan_forward_v3 with few neurons takes warm-started chunks shorter than 3W
    (the chunk length that gives the pass its waves) and returns the serial recurrence.
"""
import numpy as np
import pytest
import torch

from oracle import lif_oracle as O
from tests._inputs import gpu, host, normal, uniform
from tests.test_alif_gpu import _check_box_scan, _inputs, _preds

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("K,K2", [(16, 32), (4, 8)])
def test_v4_odd_super_map_count(dev, K, K2):
    from lifscan import hip_lif as L
    T, N, C, G, beta = 1344, 130, 64, 3, 0.99  # 21 chunks, 7 super maps
    I = normal(T, N, 0.012, 0.08, 51)
    u0 = uniform(N, 0.0, 1.0, 52)
    Ig, u0g = gpu(I, dev), gpu(u0, dev)
    print(f"v4 odd super maps K={K} K2={K2}", flush=True)
    st, sto, keep = {}, {}, {}
    U, S = L.scan_forward_v4(Ig, beta, 1.0, 0.0, u0g, C=C, G=G, K=K, K2=K2, stats=st)
    run = L.last_scan_run()
    Uo, So = O.scan_forward_v4(I, beta, 1.0, 0.0, u0, C=C, G=G, K=K, K2=K2, stats=sto, keep=keep)
    assert np.array_equal(host(run.view("SSTARTS")), keep["sstarts"])
    assert np.array_equal(host(run.view("STARTS")), keep["starts"])
    assert np.array_equal(host(U), Uo) and np.array_equal(host(S), So)
    Us, Ss = O.serial_forward(I, beta, 1.0, 0.0, u0)
    U, S = L.scan_forward_v4_maps(Ig, beta, 1.0, 0.0, u0g, C=C, G=G, K=K, K2=K2, repair=10 ** 6)
    assert np.array_equal(host(U), Us) and np.array_equal(host(S), Ss)


def test_alif_envelope_tiles(dev):
    from lifscan import triton_alif as AL
    beta, rho, q = 0.95, 0.995, 0.9
    T, N, C, K1, K2 = 1280, 20, 32, 16, 32  # 40 chunks: envelope tiles of 16, 16 and 8
    I = _inputs(beta, 2.0, T, N, 53)
    u0 = np.zeros(N, np.float32)
    w0 = uniform(N, 0.0, 0.1, 54)
    _, preds = _preds(I, beta, rho, q, u0, w0, C)
    for tag in ("oracle", "bad"):
        print(f"alif envelope tiles pred={tag}", flush=True)
        _check_box_scan(AL, dev, I, u0, w0, preds[tag], 0.1 * q, beta, rho, q, C, K1, K2, 4, tag)


@pytest.mark.parametrize("beta", [0.99, 0.9])
def test_converged_v3_few_neurons_short_warm_chunks(dev, beta):
    from lifscan import hip_lif as L
    T, N = 16384, 130
    C, W = L.warm_plan(T, N, beta)
    assert C < 3 * W or beta == 0.9  # the few-neuron rule, not the 3W one, at beta 0.99
    I = normal(T, N, 0.012, 0.08, 55)
    u0 = uniform(N, 0.0, 1.0, 56)
    print(f"converged v3, few neurons, beta={beta}: warm C={C} W={W}", flush=True)
    U, S = L.scan_forward_v3(gpu(I, dev), beta, 1.0, 0.0, gpu(u0, dev), C=64, K=16, repair=10 ** 6)
    run = L.last_scan_run()
    assert run.warm and (run.C, run.W) == (C, W)
    Us, Ss = O.serial_forward(I, beta, 1.0, 0.0, u0)
    assert np.array_equal(host(U), Us) and np.array_equal(host(S), Ss)


@pytest.mark.parametrize("N,K", [(70, 1), (70, 4), (70, 16), (70, 32), (2113, 1), (2113, 4), (2113, 8),
                                 (2113, 16), (2113, 32)])
def test_v3_carry_windows_and_fallback(dev, N, K):
    """The carry at few neurons (one wave per neuron, chunks in windows of 64) and just above
    them (one lane per neuron, maps staged through LDS): M = 150 chunks (two windows and a
    partial one), C = 100 (the overflow fallback reads 64 rows, then 36), overflowed chunks at
    small K.  LO, starts, kept counts, overflow flags, U, S and the stats equal the oracle's
    bit for bit."""
    from lifscan import hip_lif as L
    C, M, beta = 100, 150, 0.99
    T = C * M
    I = normal(T, N, 0.012, 0.08, 57)
    u0 = uniform(N, 0.0, 1.0, 58)
    print(f"v3 carry windows N={N} K={K}", flush=True)
    st, sto, keep = {}, {}, {}
    U, S = L.scan_forward_v3(gpu(I, dev), beta, 1.0, 0.0, gpu(u0, dev), C=C, K=K, stats=st)
    run = L.last_scan_run()
    Uo, So = O.scan_forward_v3(I, beta, 1.0, 0.0, u0, C=C, K=K, stats=sto, keep=keep)
    assert np.array_equal(host(run.view("LO")), keep["Lo"])
    assert np.array_equal(host(run.view("STARTS")), keep["starts"])
    assert np.array_equal(host(run.view("MN", torch.int32)), keep["n"])
    assert np.array_equal(host(run.view("OVF", torch.int32)), keep["ovf"])
    assert np.array_equal(host(U), Uo) and np.array_equal(host(S), So)
    assert st["overflow_frac"] == pytest.approx(sto["overflow_frac"], abs=0)
    assert st["mean_pieces"] == pytest.approx(sto["mean_pieces"], rel=1e-12)
    assert st["max_pieces"] == sto["max_pieces"]
    if K <= 4:
        assert sto["overflow_frac"] > 0.01


@pytest.mark.parametrize("C,K", [(512, 32), (256, 32), (512, 16)])
def test_v3_wave_carry_full_rows_and_overflow(dev, C, K):
    """The one-wave-per-neuron carry on long chunks whose maps fill their row: x ~ N(0.012, 0.02^2)
    at beta 0.99 keeps 28 pieces a chunk on average at K 32 and overflows 28% of the chunks, so
    full 32-lane rows (33 pieces), the min(k, row width - 1) clamp and the overflow fallback over
    C rows all run.  LO, starts, kept counts, overflow flags, U, S and the stats equal the
    oracle's bit for bit."""
    from lifscan import hip_lif as L
    N, beta = 70, 0.99
    T = 8192
    I = normal(T, N, 0.012, 0.02, 61)
    u0 = uniform(N, 0.0, 1.0, 62)
    print(f"v3 wave carry full rows C={C} K={K}", flush=True)
    st, sto, keep = {}, {}, {}
    U, S = L.scan_forward_v3(gpu(I, dev), beta, 1.0, 0.0, gpu(u0, dev), C=C, K=K, stats=st)
    run = L.last_scan_run()
    Uo, So = O.scan_forward_v3(I, beta, 1.0, 0.0, u0, C=C, K=K, stats=sto, keep=keep)
    assert np.array_equal(host(run.view("LO")), keep["Lo"])
    assert np.array_equal(host(run.view("STARTS")), keep["starts"])
    assert np.array_equal(host(run.view("MN", torch.int32)), keep["n"])
    assert np.array_equal(host(run.view("OVF", torch.int32)), keep["ovf"])
    assert np.array_equal(host(U), Uo) and np.array_equal(host(S), So)
    assert st["overflow_frac"] == pytest.approx(sto["overflow_frac"], abs=0)
    assert st["mean_pieces"] == pytest.approx(sto["mean_pieces"], rel=1e-12)
    assert st["max_pieces"] == sto["max_pieces"] == K + 1
    assert sto["overflow_frac"] > 0.05
    print(f"  stats {st}", flush=True)


@pytest.mark.parametrize("fallback", ["chunks", "serial"])
@pytest.mark.parametrize("N,K,K2", [(70, 4, 8), (70, 16, 32), (70, 32, 32), (2113, 4, 8), (2113, 16, 16)])
def test_v4_walks_windows_and_fallback(dev, N, K, K2, fallback):
    """v4's envelope walk and super-map carry at few neurons (one wave per neuron, maps in
    windows of 64) and just above them (one lane per neuron): 150 super maps of G = 5 chunks of
    C = 20 steps, overflowed super maps at small K2, passed by their serial steps (the fallback
    reads 64 rows, then 36) or by walking their chunk maps (rows of 16 or 32 lanes on the wave
    path, overflowed chunk maps among them at K 4).  LO, super starts, chunk starts, U, S and
    the stats equal the oracle's bit for bit."""
    from lifscan import hip_lif as L
    C, G, M2, beta = 20, 5, 150, 0.99
    T = C * G * M2
    I = normal(T, N, 0.012, 0.08, 59)
    u0 = uniform(N, 0.0, 1.0, 60)
    print(f"v4 walks windows N={N} K={K} K2={K2} fallback={fallback}", flush=True)
    st, sto, keep = {}, {}, {}
    U, S = L.scan_forward_v4(gpu(I, dev), beta, 1.0, 0.0, gpu(u0, dev), C=C, G=G, K=K, K2=K2, stats=st,
                             super_fallback=fallback)
    run = L.last_scan_run()
    Uo, So = O.scan_forward_v4(I, beta, 1.0, 0.0, u0, C=C, G=G, K=K, K2=K2, stats=sto, keep=keep,
                               super_fallback=fallback)
    assert np.array_equal(host(run.view("LO")), keep["Lo"])
    assert np.array_equal(host(run.view("SSTARTS")), keep["sstarts"])
    assert np.array_equal(host(run.view("STARTS")), keep["starts"])
    assert np.array_equal(host(U), Uo) and np.array_equal(host(S), So)
    for k in sto:
        assert st[k] == pytest.approx(sto[k], rel=1e-12), k
    if K2 <= 16:
        assert keep["SOVF"].mean() > 0.01
    if K == 4:
        assert keep["ovf"].mean() > 0.01
    print(f"  super overflow {keep['SOVF'].mean():.3f}, chunk overflow {keep['ovf'].mean():.3f}", flush=True)


@pytest.mark.parametrize("N", [1, 5, 2048])
def test_wave_walks_neuron_order_edges(dev, N):
    """The one-wave-per-neuron walks place neurons in eight contiguous ranges (one per XCD);
    fewer neurons than ranges (1, 5) and the largest count they take (2048) give the oracle's
    v3 and v4 intermediates and outputs bit for bit."""
    from lifscan import hip_lif as L
    C, G, M2, beta = 16, 4, 35, 0.99
    T = C * G * M2
    I = normal(T, N, 0.012, 0.08, 61)
    u0 = uniform(N, 0.0, 1.0, 62)
    Ig, u0g = gpu(I, dev), gpu(u0, dev)
    print(f"wave walks neuron order N={N}", flush=True)
    st, sto, keep = {}, {}, {}
    U, S = L.scan_forward_v3(Ig, beta, 1.0, 0.0, u0g, C=C, K=8, stats=st)
    run = L.last_scan_run()
    Uo, So = O.scan_forward_v3(I, beta, 1.0, 0.0, u0, C=C, K=8, stats=sto, keep=keep)
    assert np.array_equal(host(run.view("LO")), keep["Lo"])
    assert np.array_equal(host(run.view("STARTS")), keep["starts"])
    assert np.array_equal(host(run.view("MN", torch.int32)), keep["n"])
    assert np.array_equal(host(U), Uo) and np.array_equal(host(S), So)
    assert st["max_pieces"] == sto["max_pieces"]
    st, sto, keep = {}, {}, {}
    U, S = L.scan_forward_v4(Ig, beta, 1.0, 0.0, u0g, C=C, G=G, K=8, K2=16, stats=st)
    run = L.last_scan_run()
    Uo, So = O.scan_forward_v4(I, beta, 1.0, 0.0, u0, C=C, G=G, K=8, K2=16, stats=sto, keep=keep)
    assert np.array_equal(host(run.view("SSTARTS")), keep["sstarts"])
    assert np.array_equal(host(run.view("SN", torch.int32)), keep["SN"])
    assert np.array_equal(host(run.view("STARTS")), keep["starts"])
    assert np.array_equal(host(U), Uo) and np.array_equal(host(S), So)
    for k in sto:
        assert st[k] == pytest.approx(sto[k], rel=1e-12), k
