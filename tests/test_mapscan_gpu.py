"""GPU parity of the associative carry (k_map_scan, lsh_lif_scan_v3_assoc_fwd,
hip_lif.scan_forward_assoc).

  * intermediates: with repair = 0 the kernel's LO, MN, OVF and chunk STARTS equal, bit for bit,
    the oracle's restatement (oracle/map_scan.py, same association order) applied to the
    kernel's own chunk-map build (whose arrays test_lif_gpu.py pins against the oracle's build);
  * result: with the repair run to convergence U and S equal the serial recurrence
    (oracle/lif_oracle.serial_forward) bit for bit, also with many overflowed chunks;
  * the truncation statistics equal the sequential carry's (scan_forward_v3 with stats).
"""
import numpy as np
import pytest
import torch

from oracle import lif_oracle as O
from oracle import map_scan as MS
from tests._inputs import gpu, host, normal, uniform

pytestmark = pytest.mark.gpu


def _wg(M):
    return 4 if M >= 256 else (M + 63) // 64


CASES = [  # T, N, C, K, beta, mu, sd
    (2400, 5, 8, 8, 0.9, 0.12, 0.25),     # 300 chunks: two tiles of 4 waves
    (2560, 3, 64, 32, 0.99, 0.012, 0.08),  # 40 chunks: one partial wave
    (4096, 4, 16, 2, 0.99, 0.012, 0.08),   # 256 chunks, K = 2: many overflowed chunks
    (8192, 2, 16, 16, 0.95, 0.15, 0.3),    # 512 chunks: two full tiles
]


@pytest.mark.parametrize("T,N,C,K,beta,mu,sd", CASES)
def test_assoc_carry_intermediates_equal_oracle(dev, T, N, C, K, beta, mu, sd):
    from lifscan import hip_lif as L
    I = normal(T, N, mu, sd, 31)
    u0 = uniform(N, 0.0, 0.9, 32)
    print(f"assoc carry T={T} N={N} C={C} K={K} beta={beta}", flush=True)
    L.scan_forward_assoc(gpu(I, dev), beta, 1.0, 0.0, gpu(u0, dev), C=C, K=K, repair=0)
    run = L.last_scan_run()
    v = lambda name, dt=torch.float32: host(run.view(name, dt))
    arrs = (v("EC"), v("EA"), v("EB"), v("MA"), v("MB"), v("CNT", torch.int32),
            v("OVFRAW", torch.int32), v("MX"), v("MC"))
    LO, MN, OVF, ST = MS.map_scan_carry(*arrs, I, u0, beta, 1.0, 0.0, C, _wg(T // C))
    assert np.array_equal(v("LO"), LO)
    assert np.array_equal(v("MN", torch.int32), MN)
    assert np.array_equal(v("OVF", torch.int32), OVF)
    assert np.array_equal(v("STARTS"), ST)


@pytest.mark.parametrize("T,N,C,K,beta,mu,sd", CASES + [(65536, 70, 256, 32, 0.99, 0.012, 0.08)])
def test_assoc_map_scan_converged_equals_serial(dev, T, N, C, K, beta, mu, sd):
    from lifscan import hip_lif as L
    I = normal(T, N, mu, sd, 33)
    u0 = uniform(N, 0.0, 0.9, 34)
    print(f"assoc map scan T={T} N={N} C={C} K={K}", flush=True)
    st, sto = {}, {}
    U, S = L.scan_forward_assoc(gpu(I, dev), beta, 1.0, 0.0, gpu(u0, dev), C=C, K=K, stats=st)
    Uo, So = O.serial_forward(I, beta, 1.0, 0.0, u0)
    assert np.array_equal(host(U), Uo) and np.array_equal(host(S), So)
    # the truncation statistics are the sequential carry's (same build, same rule); the
    # envelope bounds differ only in rounding, which moves no breakpoint across them here
    L.scan_forward_v3(gpu(I, dev), beta, 1.0, 0.0, gpu(u0, dev), C=C, K=K, repair=10 ** 6,
                      stats=sto)
    assert st["max_pieces"] == sto["max_pieces"]
    assert st["overflow_frac"] == pytest.approx(sto["overflow_frac"], rel=1e-3, abs=1e-6)


def test_assoc_rejects_negative_beta_and_bad_shapes(dev):
    from lifscan import hip_lif as L
    I = torch.zeros(128, 4, device=dev)
    z = torch.zeros(4, device=dev)
    with pytest.raises(ValueError):
        L.scan_forward_assoc(I, -0.5, 1.0, 0.0, z, C=64, K=8)
    with pytest.raises(ValueError):
        L.scan_forward_assoc(I, 0.9, 1.0, 0.0, z, C=48, K=8)
    with pytest.raises(ValueError):
        L.scan_forward_assoc(I, 0.9, 1.0, 0.0, z, C=64, K=33)


def test_assoc_carry_at_cfg4(dev):
    """cfg4 (N = 1024, T = 2^20, beta = 0.99, x ~ N(0.012, 0.08^2), u0 ~ U[0, 1)) with C = 2048,
    K = 32 (512 chunks a neuron, two tiles): the carry's intermediates on 4 columns equal the
    oracle's, and the converged scan equals the serial forward bit for bit."""
    from lifscan import hip_lif as L
    T, N, beta, C, K = 2 ** 20, 1024, 0.99, 2048, 32
    g = torch.Generator().manual_seed(0)
    I = (0.012 + 0.08 * torch.randn(T, N, generator=g)).to(dev)
    u0 = torch.rand(N, generator=torch.Generator().manual_seed(2)).to(dev)
    print("assoc carry at cfg4 (repair 0)", flush=True)
    L.scan_forward_assoc(I, beta, 1.0, 0.0, u0, C=C, K=K, repair=0)
    run = L.last_scan_run()
    cols = [0, 333, 700, 1023]
    v = lambda name, dt=torch.float32: host(run.view(name, dt))[..., cols]
    arrs = (v("EC"), v("EA"), v("EB"), v("MA"), v("MB"), v("CNT", torch.int32),
            v("OVFRAW", torch.int32), v("MX"), v("MC"))
    LO, MN, OVF, ST = MS.map_scan_carry(*arrs, host(I[:, cols]), host(u0[cols]), beta, 1.0, 0.0,
                                        C, _wg(T // C))
    assert np.array_equal(v("LO"), LO) and np.array_equal(v("MN", torch.int32), MN)
    assert np.array_equal(v("OVF", torch.int32), OVF) and np.array_equal(v("STARTS"), ST)
    print("assoc map scan at cfg4 (converged)", flush=True)
    U, S = L.scan_forward_assoc(I, beta, 1.0, 0.0, u0, C=C, K=K)
    Us, Ss = L.serial_forward(I, beta, 1.0, 0.0, u0)
    assert torch.equal(U, Us) and torch.equal(S, Ss)
    del I, U, S, Us, Ss
    torch.cuda.empty_cache()
