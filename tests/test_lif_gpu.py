"""GPU parity of the HIP LIF kernels against the CPU oracle (through the C ABI).

Bars: spikes and membrane potentials bit-exact (integer/byte-level equality of fp32 arrays)
for every forward path; the adjoint within 1e-5 relative of the fp32 oracle (the reference's
own scan-vs-serial bar, tests/test_triton.py:47) and 1e-4 relative of the fp64 adjoint
(north-star gradient bar).
"""
import numpy as np
import pytest
import torch

from oracle import lif_oracle as O
from tests._inputs import gpu, host, normal, uniform

pytestmark = pytest.mark.gpu

REL_FP32 = 1e-5
REL_FP64 = 1e-4


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.fixture(scope="module")
def L():
    from lifscan import triton_lif
    return triton_lif


@pytest.mark.parametrize("T,N,beta,u_r,mu,sd", [
    (1024, 4096, 0.9, 0.0, 0.12, 0.25),   # cfg1 shape
    (777, 333, 0.99, -0.1, 0.012, 0.08),  # ragged: N % 64 != 0, T % tile != 0
    (3, 65, 0.5, -0.2, 0.4, 0.3),
    (1, 1, 0.9, 0.0, 1.5, 0.1),
    (2048, 200, 1.0, -0.1, 0.05, 0.3),
])
def test_serial_forward_bitexact(L, dev, T, N, beta, u_r, mu, sd):
    I = normal(T, N, mu, sd, 1)
    u0 = uniform(N, -0.3, 0.9, 2)
    print(f"serial fwd T={T} N={N} beta={beta}", flush=True)
    U, S = L.serial_forward(gpu(I, dev), beta, 1.0, u_r, gpu(u0, dev))
    Uo, So = O.serial_forward(I, beta, 1.0, u_r, u0)
    assert np.array_equal(host(U), Uo)
    assert np.array_equal(host(S), So)


@pytest.mark.parametrize("detach,with_gu", [(True, False), (True, True), (False, True)])
def test_serial_backward(L, dev, detach, with_gu):
    T, N = 1000, 300
    I = normal(T, N, 0.15, 0.4, 3)
    u0 = uniform(N, -0.2, 0.5, 4)
    GS = normal(T, N, 0.0, 1.0, 5)
    GU = normal(T, N, 0.0, 1.0, 6) if with_gu else None
    U, S = O.serial_forward(I, 0.9, 1.0, -0.1, u0)
    print(f"serial bwd detach={detach} gu={with_gu}", flush=True)
    Lam = L.serial_backward(gpu(I, dev), gpu(u0, dev), gpu(U, dev), gpu(S, dev), gpu(GS, dev),
                            gpu(GU, dev) if with_gu else None, 0.9, 1.0, -0.1, 4.0, detach)
    ref32 = O.serial_backward(I, u0, U, S, GS, GU, 0.9, 1.0, -0.1, 4.0, detach)
    ref64 = O.serial_backward(I, u0, U, S, GS, GU, 0.9, 1.0, -0.1, 4.0, detach, dtype=np.float64)
    assert rel(host(Lam), ref32) < REL_FP32
    assert rel(host(Lam), ref64) < REL_FP64


REGIMES = [(b, mu, sd) for b in (0.5, 0.9, 0.99, 1.0) for (mu, sd) in ((0.15, 0.4), (-0.1, 0.6), (0.4, 0.2))]


@pytest.mark.parametrize("beta,mu,sd", REGIMES)
def test_scan_v3_matches_oracle(L, dev, beta, mu, sd):
    """repair=0: U, S, chunk starts, kept maps and stats equal the oracle's v3 bit for bit;
    repair on: U, S equal the serial recurrence (test_v3.py's N=777, not a multiple of 64)."""
    T, N, C = 1024, 777, 64
    I = normal(T, N, mu, sd, 7)
    u0 = uniform(N, -0.3, 0.3, 8)
    Ig, u0g = gpu(I, dev), gpu(u0, dev)
    Us, Ss = O.serial_forward(I, beta, 1.0, -0.1, u0)
    for K in (4, 16):
        print(f"v3 beta={beta} mu={mu} K={K}", flush=True)
        st, sto, keep = {}, {}, {}
        U, S = L.scan_forward_v3(Ig, beta, 1.0, -0.1, u0g, C=C, K=K, stats=st)
        run = L.last_scan_run()
        Uo, So = O.scan_forward_v3(I, beta, 1.0, -0.1, u0, C=C, K=K, stats=sto, keep=keep)
        assert np.array_equal(host(U), Uo) and np.array_equal(host(S), So)
        assert np.array_equal(host(run.view("LO")), keep["Lo"])
        assert np.array_equal(host(run.view("STARTS")), keep["starts"])
        n = host(run.view("MN", torch.int32))
        assert np.array_equal(n, keep["n"])
        assert np.array_equal(host(run.view("OVF", torch.int32)), keep["ovf"])
        assert np.array_equal(host(run.view("MA")), keep["A"])
        assert np.array_equal(host(run.view("MB")), keep["B"])
        valid = np.arange(K)[None, :, None] < n[:, None, :]
        assert np.array_equal(host(run.view("MX"))[valid], keep["xd"][valid])
        assert np.array_equal(host(run.view("MC"))[valid], keep["cd"][valid])
        assert st["overflow_frac"] == pytest.approx(sto["overflow_frac"], abs=0)
        assert st["mean_pieces"] == pytest.approx(sto["mean_pieces"], rel=1e-12)
        assert st["max_pieces"] == sto["max_pieces"]
        st2 = {}
        U2, S2 = L.scan_forward_v3(Ig, beta, 1.0, -0.1, u0g, C=C, K=K, repair=10 ** 6, stats=st2)
        assert np.array_equal(host(U2), Us) and np.array_equal(host(S2), Ss)
        sto2 = {}
        O.scan_forward_v3(I, beta, 1.0, -0.1, u0, C=C, K=K, repair=10 ** 6, stats=sto2)
        assert st2["repair_iters"] == sto2["repair_iters"]


@pytest.mark.parametrize("C,beta,mu,sd", [(512, 0.99, 0.012, 0.08), (2048, 0.99, 0.012, 0.08),
                                          (1024, 0.9, 0.15, 0.4), (256, 0.5, 0.15, 0.4)])
def test_scan_v3_long_chunks_32_slots_match_oracle(L, dev, C, beta, mu, sd):
    """Long chunks with 32 slots (cfg4's chunk lengths, up to 33 pieces a map at beta 0.99):
    U, S, starts, the kept breakpoints and constants, overflow flags and stats equal the oracle's
    bit for bit at repair = 0 (N = 130, a ragged second wave)."""
    T, N, K = 4096, 130, 32
    I = normal(T, N, mu, sd, 41)
    u0 = uniform(N, 0.0, 1.0, 42)
    print(f"v3 long chunks C={C} beta={beta} K=32", flush=True)
    st, sto, keep = {}, {}, {}
    U, S = L.scan_forward_v3(gpu(I, dev), beta, 1.0, 0.0, gpu(u0, dev), C=C, K=K, stats=st)
    run = L.last_scan_run()
    Uo, So = O.scan_forward_v3(I, beta, 1.0, 0.0, u0, C=C, K=K, stats=sto, keep=keep)
    assert np.array_equal(host(U), Uo) and np.array_equal(host(S), So)
    assert np.array_equal(host(run.view("LO")), keep["Lo"])
    assert np.array_equal(host(run.view("STARTS")), keep["starts"])
    n = host(run.view("MN", torch.int32))
    assert np.array_equal(n, keep["n"])
    assert np.array_equal(host(run.view("OVF", torch.int32)), keep["ovf"])
    assert np.array_equal(host(run.view("MA")), keep["A"])
    assert np.array_equal(host(run.view("MB")), keep["B"])
    valid = np.arange(K)[None, :, None] < n[:, None, :]
    assert np.array_equal(host(run.view("MX"))[valid], keep["xd"][valid])
    assert np.array_equal(host(run.view("MC"))[valid], keep["cd"][valid])
    assert st["mean_pieces"] == pytest.approx(sto["mean_pieces"], rel=1e-12)
    assert st["max_pieces"] == sto["max_pieces"]
    print(f"  max pieces {sto['max_pieces']}, mean {sto['mean_pieces']:.2f}", flush=True)


@pytest.mark.parametrize("K", [4, 8, 16, 32])
def test_scan_v3_long_sequence_wave_carry(L, dev, K):
    """Many chunks per neuron (M = 1024) with few neurons (N = 130: the carry takes one wave per
    neuron, a chunk map on a row of 16 or 32 lanes); LO, starts, kept pieces, overflow flags and
    outputs equal the oracle's bit for bit, including overflowed chunks (K = 4 at beta = 0.99).
    The staged carry (maps through LDS, above 2048 neurons) is pinned by
    test_v3_carry_windows_and_fallback at N = 2113, K 1 to 32."""
    T, N, C, beta = 16384, 130, 16, 0.99
    I = normal(T, N, 0.012, 0.08, 21)
    u0 = uniform(N, 0.0, 1.0, 22)
    print(f"v3 long-sequence wave carry K={K}", flush=True)
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
    assert st["max_pieces"] == sto["max_pieces"]
    if K == 4:
        assert sto["overflow_frac"] > 0.01


def test_converged_v3_long_sequence_path(L, dev):
    """Few neurons, long T, converged repair: the two-level scan with long chunks (C = 1024,
    K = 32) returns the serial recurrence bit for bit; scan_forward_v3 itself takes the
    warm-started chunks there (warm_plan) and returns the same bits."""
    from lifscan import hip_lif as H
    T, N, beta = 65536, 1000, 0.99
    assert L.long_sequence_C(T, N) == 1024
    I = normal(T, N, 0.012, 0.08, 23)
    u0 = uniform(N, 0.0, 1.0, 24)
    print("v3 long-sequence path", flush=True)
    Ig, u0g = gpu(I, dev), gpu(u0, dev)
    U, S = H._scan2(Ig, beta, 1.0, 0.0, u0g, 1024, H.LONG_K, T // 1024, None)
    Us, Ss = O.serial_forward(I, beta, 1.0, 0.0, u0)
    assert np.array_equal(host(U), Us) and np.array_equal(host(S), Ss)
    U, S = L.scan_forward_v3(Ig, beta, 1.0, 0.0, u0g, C=256, K=16, repair=10 ** 6)
    assert H.last_scan_run().warm and (H.last_scan_run().C, H.last_scan_run().W) == H.warm_plan(T, N, beta)
    assert np.array_equal(host(U), Us) and np.array_equal(host(S), Ss)


def test_converged_v3_pieces_path_cfg4(L, dev):
    """At cfg4's size (N = 1024, T = 2^20, beta = 0.99) the long-chunk scan in pieces (C = 2048,
    4 pieces) and the converged scan_forward_v3 (warm-started chunks, C = 16384) return the
    serial forward bit for bit (the serial forward is pinned to the oracle by
    test_serial_forward_bitexact)."""
    from lifscan import hip_lif as H
    T, N, beta = 2 ** 20, 1024, 0.99
    assert H.long_sequence_plan(T, N) == (2048, 4)
    assert H.warm_plan(T, N, beta)[0] == 16384
    g = torch.Generator(device=dev).manual_seed(41)
    I = torch.randn(T, N, device=dev, generator=g).mul_(0.08).add_(0.012)
    u0 = torch.rand(N, device=dev, generator=g)
    print("v3 pieces at cfg4", flush=True)
    Us, Ss = H.serial_forward(I, beta, 1.0, 0.0, u0)
    U, S = H._scan2_pieces(I, beta, 1.0, 0.0, u0, 2048, H.LONG_K, 4)
    assert H.last_scan_run().pieces == 4 and H.last_scan_run().C == 2048
    assert torch.equal(U, Us) and torch.equal(S, Ss)
    del U, S
    print("v3 converged (warm) at cfg4", flush=True)
    U, S = L.scan_forward_v3(I, beta, 1.0, 0.0, u0, C=256, K=16, repair=10 ** 6)
    assert H.last_scan_run().warm and H.last_scan_run().C == 16384
    assert torch.equal(U, Us) and torch.equal(S, Ss)
    del I, U, S, Us, Ss
    torch.cuda.empty_cache()


def test_scan_v3_pieces_on_a_user_stream(L, dev):
    """The pieces forward on a non-default stream, right after that stream produced I: the side
    stream's builds wait for the caller's stream (event fork), and the caller's stream waits for
    every build, so the result is the serial recurrence."""
    from lifscan import hip_lif as H
    T, N, C, P, beta = 16384, 1024, 256, 4, 0.99
    g = torch.Generator(device=dev).manual_seed(43)
    u0 = torch.rand(N, device=dev, generator=g)
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    print("v3 pieces on a user stream", flush=True)
    with torch.cuda.stream(s):
        I = torch.randn(T, N, device=dev, generator=g).mul_(0.08).add_(0.012)
        U, S = H._scan2_pieces(I, beta, 1.0, 0.0, u0, C, 32, P)
    s.synchronize()
    Us, Ss = H.serial_forward(I, beta, 1.0, 0.0, u0)
    assert torch.equal(U, Us) and torch.equal(S, Ss)


@pytest.mark.parametrize("K", [4, 32])
@pytest.mark.parametrize("P", [1, 2, 3, 4, 8])
def test_scan_v3_pieces_equals_serial(L, dev, P, K):
    """The converged two-level scan in P pieces (maps built on a side stream, each piece
    carried and repaired from the previous piece's last row of U) is the serial recurrence bit
    for bit, with overflowing maps (K = 4 at beta = 0.99) and a reset value below zero."""
    T, N, C, beta, u_r = 24576, 300, 256, 0.99, -0.1
    I = normal(T, N, 0.012, 0.08, 31)
    u0 = uniform(N, 0.0, 1.0, 32)
    from lifscan import hip_lif as H
    print(f"v3 pieces P={P} K={K}", flush=True)
    U, S = H._scan2_pieces(gpu(I, dev), beta, 1.0, u_r, gpu(u0, dev), C, K, P)
    Us, Ss = O.serial_forward(I, beta, 1.0, u_r, u0)
    assert np.array_equal(host(U), Us) and np.array_equal(host(S), Ss)
    with pytest.raises(ValueError):
        H._scan2_pieces(gpu(I, dev), beta, 1.0, u_r, gpu(u0, dev), C, K, 7)  # 96 chunks


@pytest.mark.parametrize("R", [1, 2, 3])
def test_scan_v3_finite_repair_rounds(L, dev, R):
    T, N, C = 2048, 300, 64
    I = normal(T, N, 0.012, 0.08, 9)
    u0 = np.zeros(N, np.float32)
    print(f"v3 finite repair R={R}", flush=True)
    st, sto = {}, {}
    U, S = L.scan_forward_v3(gpu(I, dev), 0.99, 1.0, 0.0, gpu(u0, dev), C=C, K=4, repair=R, stats=st)
    Uo, So = O.scan_forward_v3(I, 0.99, 1.0, 0.0, u0, C=C, K=4, repair=R, stats=sto)
    assert np.array_equal(host(U), Uo) and np.array_equal(host(S), So)
    assert st["repair_iters"] == sto["repair_iters"]


def test_scan_v1_global_bounds(L, dev):
    """scan_forward prunes with the loose global state_bounds (triton_lif.py:262-295)."""
    T, N = 1024, 500
    I = normal(T, N, 0.15, 0.4, 10)
    u0 = uniform(N, -0.3, 0.3, 11)
    Ig, u0g = gpu(I, dev), gpu(u0, dev)
    lo_g, _ = L.state_bounds(Ig, 0.9, 1.0, -0.1, u0g)
    lo = host(lo_g)
    print("v1 scan", flush=True)
    for K in (4, 16, 64):
        st, sto = {}, {}
        U, S = L.scan_forward(Ig, 0.9, 1.0, -0.1, u0g, C=64, K=K, stats=st)
        Uo, So = O.scan_forward_v3(I, 0.9, 1.0, -0.1, u0, C=64, K=K, lo=lo, stats=sto)
        assert np.array_equal(host(U), Uo) and np.array_equal(host(S), So)
        assert st["overflow_frac"] == pytest.approx(sto["overflow_frac"], abs=0)
        assert st["max_pieces"] == sto["max_pieces"]


@pytest.mark.parametrize("C,K", [(8, 1), (16, 2), (128, 64), (1024, 8)])
def test_scan_v3_edge_shapes(L, dev, C, K):
    T, N = 1024, 65
    I = normal(T, N, 0.12, 0.25, 12)
    u0 = np.zeros(N, np.float32)
    print(f"v3 edge C={C} K={K}", flush=True)
    U, S = L.scan_forward_v3(gpu(I, dev), 0.9, 1.0, 0.0, gpu(u0, dev), C=C, K=K, repair=10 ** 6)
    Us, Ss = O.serial_forward(I, 0.9, 1.0, 0.0, u0)
    assert np.array_equal(host(U), Us) and np.array_equal(host(S), Ss)


def test_scan_v3_rejects_bad_shapes(L, dev):
    I = torch.zeros(100, 8, device=dev)
    u0 = torch.zeros(8, device=dev)
    with pytest.raises(ValueError):
        L.scan_forward_v3(I, 0.9, 1.0, 0.0, u0, C=64)
    with pytest.raises(ValueError):
        L.scan_forward_v3(I, 0.9, 1.0, 0.0, u0, C=10, K=65)


@pytest.mark.parametrize("C", [32, 64, 128])
def test_scan_backward(L, dev, C):
    T, N = 1024, 333
    I = normal(T, N, 0.15, 0.4, 13)
    u0 = uniform(N, -0.2, 0.2, 14)
    GS = normal(T, N, 0.0, 1.0, 15)
    U, S = O.serial_forward(I, 0.9, 1.0, 0.0, u0)
    print(f"scan bwd C={C}", flush=True)
    Lam = L.scan_backward_tiled(gpu(I, dev), gpu(u0, dev), gpu(U, dev), gpu(S, dev), gpu(GS, dev),
                                None, 0.9, 1.0, 0.0, 4.0, C=C)
    ref32 = O.scan_backward(I, u0, U, S, GS, None, 0.9, 1.0, 0.0, 4.0, True, C=C)
    ref64 = O.serial_backward(I, u0, U, S, GS, None, 0.9, 1.0, 0.0, 4.0, dtype=np.float64)
    assert rel(host(Lam), ref32) < REL_FP32
    assert rel(host(Lam), ref64) < REL_FP64
    GU = normal(T, N, 0.0, 1.0, 16)
    Lam2 = L.scan_backward_tiled(gpu(I, dev), gpu(u0, dev), gpu(U, dev), gpu(S, dev), gpu(GS, dev),
                                 gpu(GU, dev), 0.9, 1.0, 0.0, 4.0, detach=False, C=C)
    ref = O.serial_backward(I, u0, U, S, GS, GU, 0.9, 1.0, 0.0, 4.0, False, dtype=np.float64)
    assert rel(host(Lam2), ref) < REL_FP64


@pytest.mark.parametrize("mode", ["serial", "scan"])
def test_lif_tuned_gradients(L, dev, mode):
    """Gradients w.r.t. I, u0 and beta within 1e-4 relative of the fp64 adjoint."""
    T, N = 1024, 256
    I = normal(T, N, 0.15, 0.4, 17)
    u0 = uniform(N, -0.2, 0.2, 18)
    W = normal(T, N, 0.0, 1.0, 19)
    Ig = gpu(I, dev).requires_grad_(True)
    u0g = gpu(u0, dev).requires_grad_(True)
    beta = torch.tensor(0.95, device=dev, requires_grad=True)
    print(f"lif_tuned mode={mode}", flush=True)
    S = L.lif_tuned(Ig, u0g, beta, 1.0, 0.0, 4.0, mode=mode, K=16, repair=10 ** 6)
    (gpu(W, dev) * S).sum().backward()
    Uo, So = O.serial_forward(I, 0.95, 1.0, 0.0, u0)
    assert np.array_equal(host(S), So)
    Lam = O.serial_backward(I, u0, Uo, So, W, None, 0.95, 1.0, 0.0, 4.0, dtype=np.float64)
    assert rel(host(Ig.grad), Lam) < REL_FP64
    assert rel(host(u0g.grad), np.float64(np.float32(0.95)) * Lam[0]) < REL_FP64
    uprev = np.concatenate([u0[None], Uo[:-1]], 0).astype(np.float64)
    dbeta = float((Lam * uprev).sum())
    assert abs(beta.grad.item() - dbeta) <= REL_FP64 * abs(dbeta)


def test_lif_auto_matches_serial(L, dev):
    T, N = 1024, 128
    I = normal(T, N, 0.15, 0.4, 20)
    Ig = gpu(I, dev)
    u0 = torch.zeros(N, device=dev)
    S = L.lif_auto(Ig, u0, 0.9, 1.0, 0.0, 4.0)
    _, So = O.serial_forward(I, 0.9, 1.0, 0.0, np.zeros(N, np.float32))
    assert np.array_equal(host(S), So)


@pytest.mark.parametrize("T", [1000, 1032])
def test_lif_auto_and_lif_param_lengths_without_a_chunk(L, dev, T):
    """T with no chunk divisible by 16 (the scan forward's policy): lif_auto and
    lif_param(mode="auto") run (serial forward, chunked scan adjoint at C = 8: from 16384 neurons
    auto takes the scan adjoint from T = 256), spikes equal the serial recurrence and the
    gradients the fp64 adjoint."""
    from lifscan.fit import lif_param
    N = 16384
    assert L.auto_modes(N, T) == ("serial", "scan")
    I = normal(T, N, 0.12, 0.25, 40)
    W = normal(T, N, 0.0, 1.0, 41)
    u0 = np.zeros(N, np.float32)
    Uo, So = O.serial_forward(I, 0.9, 1.0, 0.0, u0)
    Lam = O.serial_backward(I, u0, Uo, So, W, None, 0.9, 1.0, 0.0, 4.0, dtype=np.float64)
    print(f"lif_auto / lif_param T={T}", flush=True)
    for fn in ("auto", "param"):
        Ig = gpu(I, dev).requires_grad_(True)
        if fn == "auto":
            S = L.lif_auto(Ig, torch.zeros(N, device=dev), 0.9, 1.0, 0.0, 4.0)
        else:
            S = lif_param(Ig, torch.zeros(N, device=dev), 0.9, 1.0, 0.0, 4.0, mode="auto")
        (gpu(W, dev) * S).sum().backward()
        assert np.array_equal(host(S), So), fn
        assert rel(host(Ig.grad), Lam) < REL_FP64, fn


def test_cfg2_scan_equals_serial_full_size(L, dev):
    """BASELINE cfg2 at full size (65,536 x 4,096, beta in {0.9, 0.99}, K=8, repair on):
    spikes and potentials of the scan equal the serial kernel's everywhere, and 512 columns
    equal the oracle (the serial kernel itself is pinned to the oracle above)."""
    T, N = 4096, 65536
    for beta, mu, sd in ((0.9, 0.12, 0.25), (0.99, 0.012, 0.08)):
        print(f"cfg2 beta={beta}", flush=True)
        g = torch.Generator().manual_seed(0)
        I = (mu + sd * torch.randn(T, N, generator=g)).to(dev)
        u0 = torch.zeros(N, device=dev)
        Us, Ss = L.serial_forward(I, beta, 1.0, 0.0, u0)
        for C in (32, 64, 128):
            st = {}
            U, S = L.scan_forward_v3(I, beta, 1.0, 0.0, u0, C=C, K=8, repair=10 ** 6, stats=st)
            assert torch.equal(U, Us) and torch.equal(S, Ss)
            print(f"  C={C} stats={st}", flush=True)
            # without statistics the map scan repairs by the ordered pass
            U, S = L.scan_forward_mapscan(I, beta, 1.0, 0.0, u0, C=C, K=8, repair=10 ** 6)
            assert torch.equal(U, Us) and torch.equal(S, Ss)
        cols = np.arange(0, N, N // 512)
        Uo, So = O.serial_forward(host(I[:, cols]), beta, 1.0, 0.0, np.zeros(len(cols), np.float32))
        assert np.array_equal(host(Us[:, cols]), Uo) and np.array_equal(host(Ss[:, cols]), So)
        del I, Us, Ss, U, S
        torch.cuda.empty_cache()


@pytest.mark.parametrize("fallback", ["chunks", "serial"])
@pytest.mark.parametrize("beta,mu,sd", [(0.5, 0.15, 0.4), (0.9, 0.15, 0.4), (0.99, 0.012, 0.08),
                                        (1.0, -0.1, 0.6), (0.9, 0.4, 0.2)])
def test_scan_v4_matches_oracle(L, dev, beta, mu, sd, fallback):
    """Three-level scan (experiments/test_v4.py shapes: N=777): chunk and super maps, starts,
    U, S and stats equal the oracle bit for bit at repair=0, with either pass of an overflowed
    super map; repair on gives the serial recurrence (the three-level pipeline itself,
    scan_forward_v4_maps, and scan_forward_v4's converged dispatch)."""
    T, N, C, G = 2048, 777, 64, 8
    I = normal(T, N, mu, sd, 25)
    u0 = uniform(N, -0.3, 0.3, 26)
    Ig, u0g = gpu(I, dev), gpu(u0, dev)
    Us, Ss = O.serial_forward(I, beta, 1.0, -0.1, u0)
    # K2 = 64: the one-wave super carry with a whole wave per super map
    for K, K2 in ((16, 32), (8, 16), (4, 4), (32, 64)):
        print(f"v4 beta={beta} mu={mu} K={K} K2={K2} fallback={fallback}", flush=True)
        st, sto, keep = {}, {}, {}
        U, S = L.scan_forward_v4(Ig, beta, 1.0, -0.1, u0g, C=C, G=G, K=K, K2=K2, stats=st,
                                 super_fallback=fallback)
        run = L.last_scan_run()
        Uo, So = O.scan_forward_v4(I, beta, 1.0, -0.1, u0, C=C, G=G, K=K, K2=K2, stats=sto, keep=keep,
                                   super_fallback=fallback)
        assert np.array_equal(host(run.view("LO")), keep["Lo"])
        assert np.array_equal(host(run.view("MN", torch.int32)), keep["n"])
        assert np.array_equal(host(run.view("OVF", torch.int32)), keep["ovf"])
        SN = host(run.view("SN", torch.int32))
        assert np.array_equal(SN, keep["SN"])
        assert np.array_equal(host(run.view("SOVF", torch.int32)), keep["SOVF"])
        assert np.array_equal(host(run.view("SA")), keep["SA"])
        assert np.array_equal(host(run.view("SB")), keep["SB"])
        valid = np.arange(K2)[None, :, None] < SN[:, None, :]
        assert np.array_equal(host(run.view("SX"))[valid], keep["SX"][valid])
        assert np.array_equal(host(run.view("SC"))[valid], keep["SC"][valid])
        assert np.array_equal(host(run.view("SSTARTS")), keep["sstarts"])
        assert np.array_equal(host(run.view("STARTS")), keep["starts"])
        assert np.array_equal(host(U), Uo) and np.array_equal(host(S), So)
        for k in sto:
            assert st[k] == pytest.approx(sto[k], rel=1e-12), k
        U2, S2 = L.scan_forward_v4_maps(Ig, beta, 1.0, -0.1, u0g, C=C, G=G, K=K, K2=K2, repair=10 ** 6,
                                        super_fallback=fallback)
        assert np.array_equal(host(U2), Us) and np.array_equal(host(S2), Ss)
        # overflowed super maps passed as stored (converged calls only), the repair fixes the starts
        U2, S2 = L.scan_forward_v4_maps(Ig, beta, 1.0, -0.1, u0g, C=C, G=G, K=K, K2=K2, repair=10 ** 6,
                                        super_fallback="none")
        assert np.array_equal(host(U2), Us) and np.array_equal(host(S2), Ss)
        with pytest.raises(ValueError):
            L.scan_forward_v4_maps(Ig, beta, 1.0, -0.1, u0g, C=C, G=G, K=K, K2=K2, repair=1,
                                   super_fallback="none")
        U2, S2 = L.scan_forward_v4(Ig, beta, 1.0, -0.1, u0g, C=C, G=G, K=K, K2=K2, repair=10 ** 6)
        assert np.array_equal(host(U2), Us) and np.array_equal(host(S2), Ss)


@pytest.mark.parametrize("beta,mu,sd", [(0.9, 0.15, 0.4), (0.99, 0.012, 0.08), (0.5, -0.1, 0.6)])
def test_scan_v4_lane_compose_matches_oracle(L, dev, beta, mu, sd):
    """The group composition with one lane per neuron (k_lif_compose; the test above has too few
    neurons and super maps for it and takes the one-wave-per-neuron composition): N = 4160 with
    four super maps gives 260 waves.  Super maps, starts, U and S equal the oracle bit for bit at
    repair = 0, for K2 above, at and below twice K."""
    T, N, C, G = 2048, 4160, 64, 8
    I = normal(T, N, mu, sd, 27)
    u0 = uniform(N, -0.3, 0.3, 28)
    Ig, u0g = gpu(I, dev), gpu(u0, dev)
    for K, K2 in ((16, 32), (8, 16), (8, 8)):
        print(f"v4 lane compose beta={beta} mu={mu} K={K} K2={K2}", flush=True)
        st, sto, keep = {}, {}, {}
        U, S = L.scan_forward_v4(Ig, beta, 1.0, -0.1, u0g, C=C, G=G, K=K, K2=K2, stats=st,
                                 super_fallback="chunks")
        run = L.last_scan_run()
        Uo, So = O.scan_forward_v4(I, beta, 1.0, -0.1, u0, C=C, G=G, K=K, K2=K2, stats=sto, keep=keep,
                                   super_fallback="chunks")
        SN = host(run.view("SN", torch.int32))
        assert np.array_equal(SN, keep["SN"])
        assert np.array_equal(host(run.view("SOVF", torch.int32)), keep["SOVF"])
        assert np.array_equal(host(run.view("SA")), keep["SA"])
        assert np.array_equal(host(run.view("SB")), keep["SB"])
        valid = np.arange(K2)[None, :, None] < SN[:, None, :]
        assert np.array_equal(host(run.view("SX"))[valid], keep["SX"][valid])
        assert np.array_equal(host(run.view("SC"))[valid], keep["SC"][valid])
        assert np.array_equal(host(run.view("SSTARTS")), keep["sstarts"])
        assert np.array_equal(host(run.view("STARTS")), keep["starts"])
        assert np.array_equal(host(U), Uo) and np.array_equal(host(S), So)
        print(f"  super pieces mean {sto['super_mean_pieces'] if 'super_mean_pieces' in sto else '-'}, "
              f"super overflow {st.get('super_overflow_frac')}", flush=True)


def test_scan_v4_rejects_bad_shapes(L, dev):
    I = torch.zeros(64 * 5, 8, device=dev)
    u0 = torch.zeros(8, device=dev)
    with pytest.raises(ValueError):
        L.scan_forward_v4(I, 0.9, 1.0, 0.0, u0, C=64, G=2)
    with pytest.raises(ValueError):
        L.scan_forward_v4(I, 0.9, 1.0, 0.0, u0, C=64, G=5, K=16, K2=8)


@pytest.mark.parametrize("T,N", [(1, 1), (63, 64), (64, 100), (65, 7), (1000, 130), (4113, 1029)])
@pytest.mark.parametrize("detach,with_gu", [(True, False), (True, True), (False, True)])
def test_serial_backward_pipe(L, dev, T, N, detach, with_gu):
    """The producer/consumer serial adjoint (full and partial tiles, ragged neuron blocks,
    detached or not, with and without GU) against the fp32 oracle; detached without GU it gives
    the one-wave kernel's Lam (lif_param's serial adjoint) bit for bit."""
    from lifscan.fit import _param_backward
    I = normal(T, N, 0.1, 0.5, 61)
    u0 = uniform(N, -0.2, 0.6, 62)
    GS = normal(T, N, 0.0, 1.0, 63)
    GU = normal(T, N, 0.0, 0.3, 64) if with_gu else None
    U, S = O.serial_forward(I, 0.93, 1.0, 0.1, u0)
    args = [gpu(a, dev) for a in (I, u0, U, S, GS)] + [gpu(GU, dev) if with_gu else None]
    print(f"serial bwd pipe T={T} N={N} detach={detach} gu={with_gu}", flush=True)
    got = L.serial_backward(*args, 0.93, 1.0, 0.1, 4.0, detach)
    ref = O.serial_backward(I, u0, U, S, GS, GU, 0.93, 1.0, 0.1, 4.0, detach)
    assert rel(host(got), ref) < REL_FP32
    if detach and not with_gu:
        one_wave, _ = _param_backward(*args[:5], 0.93, 1.0, 0.1, 4.0, "serial")
        assert torch.equal(got, one_wave)


@pytest.mark.parametrize("T,N", [(1, 1), (63, 64), (64, 100), (65, 7), (1000, 130), (4113, 1029)])
def test_serial_forward_pipe_equals_one_wave(L, dev, T, N):
    """The producer/consumer serial forward gives the oracle's U, S bit for bit, and the one-wave
    replay kernel's (the two-level scan with one chunk of T steps and no repair replays from u0)."""
    I = normal(T, N, 0.15, 0.5, 65)
    u0 = uniform(N, -0.2, 0.9, 66)
    Ur, Sr = O.serial_forward(I, 0.93, 1.0, 0.1, u0)
    print(f"serial fwd pipe T={T} N={N}", flush=True)
    U, S = L.serial_forward(gpu(I, dev), 0.93, 1.0, 0.1, gpu(u0, dev))
    U1, S1 = L.scan_forward_v3(gpu(I, dev), 0.93, 1.0, 0.1, gpu(u0, dev), C=T, K=1, repair=0)
    assert np.array_equal(host(U), Ur) and np.array_equal(host(S), Sr)
    assert torch.equal(U, U1) and torch.equal(S, S1)
