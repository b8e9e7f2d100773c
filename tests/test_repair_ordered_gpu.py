"""GPU parity of the repair run to convergence without its round count (repair = -1 at the C
ABI: k_lif_repair_ordered where the launcher picks it, with fewer neurons and at least 1024
chunks the segmented ordered walk k_lif_repair_seg, else Jacobi rounds to convergence).

Bar: U and S equal the serial recurrence (oracle/lif_oracle.serial_forward) bit for bit, for
the two-level scan, the scan with a caller-given bound, the associative carry and the
three-level scan, on inputs whose carried starts miss often (beta = 0.99, x ~ N(0.012, 0.08^2):
the BASELINE cfg2 beta = 0.99 distribution, 28 % of the chunk maps overflow at K = 8, C = 32),
with N not a multiple of 64; and the same U, S as the Jacobi rounds with statistics.
"""
import numpy as np
import pytest
import torch

from oracle import lif_oracle as O
from tests._inputs import gpu, host, normal, uniform

pytestmark = pytest.mark.gpu

# (T, N, C): the first two take the ordered pass (N >= 4096 and T/C >= 64), the last the
# Jacobi rounds (few neurons, 128 chunks)
SHAPES = [(4096, 4160, 32), (4096, 4100, 64), (8192, 130, 64)]


def _case(T, N, seed):
    I = normal(T, N, 0.012, 0.08, seed)
    u0 = uniform(N, 0.0, 1.0, seed + 1)
    return I, u0, O.serial_forward(I, 0.99, 1.0, 0.0, u0)


@pytest.mark.parametrize("T,N,C", SHAPES)
def test_converged_map_scan_equals_serial(dev, T, N, C):
    from lifscan import hip_lif as L
    I, u0, (Us, Ss) = _case(T, N, 41)
    Ig, u0g = gpu(I, dev), gpu(u0, dev)
    print(f"ordered repair v3 T={T} N={N} C={C}", flush=True)
    U, S = L.scan_forward_mapscan(Ig, 0.99, 1.0, 0.0, u0g, C=C, K=8, repair=10 ** 6)
    assert np.array_equal(host(U), Us) and np.array_equal(host(S), Ss)
    st = {}
    Uj, Sj = L.scan_forward_mapscan(Ig, 0.99, 1.0, 0.0, u0g, C=C, K=8, repair=10 ** 6, stats=st)
    assert torch.equal(U, Uj) and torch.equal(S, Sj)
    assert st["repair_iters"] > 1  # the starts did miss: the repair had work to do
    print(f"ordered repair lo-bound T={T} N={N} C={C}", flush=True)
    U, S = L.scan_forward(Ig, 0.99, 1.0, 0.0, u0g, C=C, K=8, repair=10 ** 6)
    assert np.array_equal(host(U), Us) and np.array_equal(host(S), Ss)


@pytest.mark.parametrize("T,N,C", SHAPES[:1] + SHAPES[2:])
def test_converged_assoc_and_v4_equal_serial(dev, T, N, C):
    from lifscan import hip_lif as L
    I, u0, (Us, Ss) = _case(T, N, 43)
    Ig, u0g = gpu(I, dev), gpu(u0, dev)
    print(f"ordered repair assoc T={T} N={N} C={C}", flush=True)
    U, S = L.scan_forward_assoc(Ig, 0.99, 1.0, 0.0, u0g, C=C, K=8)
    assert np.array_equal(host(U), Us) and np.array_equal(host(S), Ss)
    print(f"ordered repair v4 T={T} N={N} C={C}", flush=True)
    U, S = L.scan_forward_v4_maps(Ig, 0.99, 1.0, 0.0, u0g, C=C, G=4, K=8, K2=16, repair=10 ** 6)
    assert np.array_equal(host(U), Us) and np.array_equal(host(S), Ss)


def test_c_abi_repair_minus_one_and_range(dev):
    """The C entry itself: repair = -1 gives the serial recurrence, also with one chunk (nothing
    to repair); repair = -2 is an argument error."""
    from lifscan import _native as _n
    lib = _n.lib()
    for T, N, C in ((4096, 4160, 32), (64, 70, 64)):
        I, u0, (Us, Ss) = _case(T, N, 45)
        Ig, u0g = gpu(I, dev), gpu(u0, dev)
        nb = lib.lsh_lif_scan_v3_workspace(T, N, C, 8)
        ws = _n.workspace(nb, Ig.device)
        U, S = torch.empty_like(Ig), torch.empty_like(Ig)
        print(f"C ABI repair=-1 T={T} N={N} C={C}", flush=True)
        rc = lib.lsh_lif_scan_v3_fwd(_n.ptr(Ig), _n.ptr(u0g), _n.ptr(U), _n.ptr(S), T, N, 0.99, 1.0,
                                     0.0, C, 8, -1, _n.ptr(ws), nb, _n.stream_of(Ig))
        assert rc == 0
        assert np.array_equal(host(U), Us) and np.array_equal(host(S), Ss)
        rc = lib.lsh_lif_scan_v3_fwd(_n.ptr(Ig), _n.ptr(u0g), _n.ptr(U), _n.ptr(S), T, N, 0.99, 1.0,
                                     0.0, C, 8, -2, _n.ptr(ws), nb, _n.stream_of(Ig))
        assert rc == _n.LSH_ERR_ARG


def test_python_rejects_negative_repair(dev):
    from lifscan import hip_lif as L
    I = torch.zeros(128, 64, device=dev)
    z = torch.zeros(64, device=dev)
    for fn in (lambda: L.scan_forward_mapscan(I, 0.9, 1.0, 0.0, z, C=32, K=8, repair=-1),
               lambda: L.scan_forward_v4(I, 0.9, 1.0, 0.0, z, C=16, G=2, K=8, K2=16, repair=-1),
               lambda: L.scan_forward_assoc(I, 0.9, 1.0, 0.0, z, C=32, K=8, repair=-1)):
        with pytest.raises(ValueError):
            fn()


@pytest.mark.parametrize("T,N,beta,mu,sd", [(16384, 5, 0.999, 2e-4, 0.01), (16384, 70, 0.999, 2e-4, 0.01),
                                             (16384, 200, 0.999, 2e-4, 0.01), (65536, 5, 0.9999, 1e-4, 1e-3)])
def test_segmented_repair_long_dirty_runs(dev, T, N, beta, mu, sd):
    """The segmented ordered walk when the carried starts are wrong for hundreds of chunks in a
    row: beta near 1 and inputs far below threshold leave the neurons subthreshold for most of
    the sequence, so the chunk maps' affine pieces give starts that differ from the stepwise
    states in their last bits across whole runs of segment boundaries (C = 16: 1023 chunks in
    15 segments of 69; the Jacobi rounds need about 500).  The last case (4095 chunks in 63
    segments of 65, 7 spikes in all: runs of about 2600 chunks) needs more than the 32 rounds
    the launcher runs, so the gated ordered walk over all chunks finishes it.  U and S equal the
    serial recurrence and the Jacobi rounds' result (with statistics)."""
    from lifscan import hip_lif as L
    C = 16
    I = normal(T, N, mu, sd, 47)
    u0 = uniform(N, 0.0, 0.5, 48)
    Us, Ss = O.serial_forward(I, beta, 1.0, 0.0, u0)
    Ig, u0g = gpu(I, dev), gpu(u0, dev)
    print(f"segmented repair T={T} N={N} beta={beta}", flush=True)
    U, S = L.scan_forward_mapscan(Ig, beta, 1.0, 0.0, u0g, C=C, K=8, repair=10 ** 6)
    assert np.array_equal(host(U), Us) and np.array_equal(host(S), Ss)
    st = {}
    Uj, Sj = L.scan_forward_mapscan(Ig, beta, 1.0, 0.0, u0g, C=C, K=8, repair=10 ** 6, stats=st)
    assert torch.equal(U, Uj) and torch.equal(S, Sj)
    print(f"  Jacobi rounds {st['repair_iters']}", flush=True)
    assert st["repair_iters"] > 69  # dirty runs longer than a segment
