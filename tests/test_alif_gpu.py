"""GPU parity of the HIP ALIF kernels against the CPU oracle (oracle/alif_oracle.py), through
the C ABI.

Bars: U, W, S bit-exact for serial, replay and the repaired box scan; every intermediate of the
box scan (entry box, chunk maps, carried chunk states, miss flags) bit-exact at the same block
size of the split decision; the adjoint within 1e-5 relative of the fp32 oracle and 1e-4 of the
fp64 adjoint; the four parameter gradients (dbeta, drho, dq, dtheta0) within 1e-4 of the fp64
assembly, or within 4x the error that the same fp64 assembly makes from the fp32 oracle's adjoint
where that floor is above 2.5e-5 (param_bars).
"""
import math

import numpy as np
import pytest
import torch

from oracle import alif_oracle as A
from tests._inputs import gpu, host, normal, uniform

pytestmark = pytest.mark.gpu

NEURONS = [("lsnn", 0.95, 0.995, 0.9), ("glif2", 0.99, 0.96, 0.2), ("appD-a", 0.9, 0.95, 0.5)]


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def param_bars(x, U, W, S, G, beta, rho, q, u0, w0, want, theta0=1.0):
    """Bars for the four parameter gradients (dbeta, drho, dq, dtheta0) against their fp64 assembly
    `want[3:7]`: 1e-4 relative (the north star's gradient bar), raised to 4x the fp32 floor where
    that is higher.  The floor is the error of the same fp64 assembly applied to the fp32 oracle's
    adjoint: dtheta0 = -sum sg (gS + q LW) cancels to about 1e-3 of its terms at some shapes
    (5e-4 of fp64 at T 1024, N 96), which no fp32 adjoint can beat.  Prints both."""
    LV, LW = A.backward(x, U, W, S, G, beta, rho, q, theta0, u0, w0, 4.0)
    f32 = A.param_grads(x, U, W, S, G, LV.astype(np.float64), LW.astype(np.float64), beta, rho, q,
                        theta0, u0, w0, 4.0)
    floors = [rel(f32[k], want[k]) for k in range(3, 7)]
    return [max(1e-4, 4 * f) for f in floors], floors


def check_params(got, want, bars, floors, label=""):
    """got: (dbeta, drho, dq, dtheta0) as arrays or scalars; want[3:7] their fp64 assembly."""
    errs = [rel(g, want[3 + k]) for k, g in enumerate(got)]
    print(f"  {label} parameter grads rel err " + ", ".join(
        f"{n}={e:.2e} (fp32 floor {f:.2e})" for n, e, f in zip(("dbeta", "drho", "dq", "dtheta0"), errs, floors)),
        flush=True)
    for k, (e, b) in enumerate(zip(errs, bars)):
        assert e < b, (k, e, b)


def _inputs(beta, mfree, T, N, seed):
    g = torch.Generator().manual_seed(seed)
    sig = 0.5
    return ((1 - beta) * mfree + sig * math.sqrt(1 - beta * beta)
            * torch.randn(T, N, generator=g)).float().numpy()


@pytest.fixture(scope="module")
def AL():
    from lifscan import triton_alif
    return triton_alif


@pytest.mark.parametrize("name,beta,rho,q", NEURONS)
@pytest.mark.parametrize("T,N", [(1024, 300), (37, 65), (1, 1)])
def test_alif_serial_bitexact(AL, dev, name, beta, rho, q, T, N):
    I = _inputs(beta, 2.0, T, N, 1)
    u0 = uniform(N, -0.2, 0.8, 2)
    w0 = uniform(N, 0.0, 0.3, 3)
    print(f"alif serial {name} T={T} N={N}", flush=True)
    U, W, S = AL.alif_serial_forward(gpu(I, dev), beta, rho, q, 1.0, 0.0, gpu(u0, dev), gpu(w0, dev))
    Uo, Wo, So = A.serial_forward(I, beta, rho, q, 1.0, 0.0, u0, w0)
    assert np.array_equal(host(U), Uo) and np.array_equal(host(W), Wo) and np.array_equal(host(S), So)


@pytest.mark.parametrize("with_init", [False, True])
def test_alif_warm_predict(AL, dev, with_init):
    beta, rho, q = 0.99, 0.96, 0.2
    T, N, C = 2048, 130, 64
    I = _inputs(beta, 2.0, T, N, 4)
    u0 = uniform(N, 0.0, 0.5, 5)
    w0 = uniform(N, 0.0, 0.2, 6)
    kw, kwo = {}, {}
    if with_init:
        UI = normal(T // C, N, 0.3, 0.1, 7)
        WI = uniform(T // C * N, 0.0, 0.3, 8).reshape(T // C, N)
        kw = dict(UI=gpu(UI, dev), WI=gpu(WI, dev))
        kwo = dict(UI=UI, WI=WI)
    print(f"alif warm init={with_init}", flush=True)
    WP = AL.alif_warm_predict(gpu(I, dev), beta, rho, q, 1.0, 0.0, gpu(u0, dev), gpu(w0, dev), C, Wn=3,
                              u_init=0.1, w_init=0.05, **kw)
    WPo = A.warm_predict(I, beta, rho, q, 1.0, 0.0, u0, w0, C, Wn=3, u_init=0.1, w_init=0.05, **kwo)
    assert np.array_equal(host(WP), WPo)


def _preds(I, beta, rho, q, u0, w0, C):
    Ur, Wr, Sr = A.serial_forward(I, beta, rho, q, 1.0, 0.0, u0, w0)
    Wentry = np.concatenate([w0[None], Wr[C - 1:-1:C]], 0)
    _, Wprev, _ = A.serial_forward((1.005 * I).astype(np.float32), beta, rho, q, 1.0, 0.0, u0, w0)
    return (Ur, Wr, Sr), {
        "oracle": Wentry,
        "prev": np.concatenate([w0[None], Wprev[C - 1:-1:C]], 0),
        "warm4": A.warm_predict(I, beta, rho, q, 1.0, 0.0, u0, w0, C, Wn=4),
        "bad": (Wentry + 5 * q).astype(np.float32)}


def test_alif_prev_wpred(AL, dev):
    """The previous-iterate prediction (experiments/e28_allen_alif.py:36): row 0 = w0, row m =
    W[m*C - 1]; non-multiple T is rejected."""
    T, N, C = 1024, 70, 128
    W = uniform(T * N, -1.0, 1.0, 21).reshape(T, N)
    w0 = uniform(N, 0.0, 0.1, 22)
    P = host(AL.alif_prev_wpred(gpu(W, dev), gpu(w0, dev), C))
    assert P.shape == (T // C, N)
    assert np.array_equal(P[0], w0)
    for m in range(1, T // C):
        assert np.array_equal(P[m], W[m * C - 1])
    with pytest.raises(ValueError):
        AL.alif_prev_wpred(gpu(W[:1000], dev), gpu(w0, dev), C)


def _check_box_scan(AL, dev, I, u0, w0, Wp, dw, beta, rho, q, C, K1, K2, block, tag):
    """repair = 0: every intermediate of the box scan and the replayed outputs equal the
    oracle's (same block of the split decision), in pipeline order."""
    T, N = I.shape
    st, sto, keep = {}, {}, {}
    U, W, S = AL.alif_scan_forward(gpu(I, dev), beta, rho, q, 1.0, 0.0, gpu(u0, dev), gpu(w0, dev),
                                   gpu(Wp, dev), dw, C=C, K1=K1, K2=K2, BN=block, repair=0, stats=st)
    run = AL.last_alif_run()
    Uo, Wo, So = A.scan_forward(I, beta, rho, q, 1.0, 0.0, u0, w0, Wp, dw, C=C, K1=K1, K2=K2,
                                block=block, repair=0, stats=sto, keep=keep)
    # in pipeline order, so a failure names the first stage that differs
    for g, o in (("LU", "Lu"), ("HU", "Hu"), ("LW", "Lw"), ("HW", "Hw"), ("MA", "A"), ("MB", "B")):
        assert np.array_equal(host(run.view(g)), keep[o]), (tag, g)
    for g, o in (("NL", "nl"), ("NP", "npc"), ("OVF", "ovf")):
        assert np.array_equal(host(run.view(g, torch.int32)), keep[o]), (tag, g)
    nl, npc = keep["nl"], keep["npc"]
    lmask = np.arange(K1)[None, :, None] < nl[:, None]
    pmask = np.arange(K2)[None, :, None] < npc[:, None]
    for g, o in (("LS", "ls"), ("LC", "lc"), ("LX", "lx")):
        assert np.array_equal(host(run.view(g))[lmask], keep[o][lmask]), (tag, g)
    for g, o in (("PXL", "pxl"), ("PXR", "pxr"), ("PU", "pu"), ("PA", "pa"), ("POF", "pof")):
        assert np.array_equal(host(run.view(g))[pmask], keep[o][pmask]), (tag, g)
    assert np.array_equal(host(run.view("POWN", torch.int32))[pmask], keep["pown"][pmask])
    for g in ("SU", "SW"):
        assert np.array_equal(host(run.view(g)), keep[g]), (tag, g)
    assert np.array_equal(host(run.view("MISS", torch.int32)), keep["MISS"]), tag
    # the first chunk whose start the carry took through a map: chunk m's start is the
    # serial state while every chunk before it was replayed serially (a miss)
    miss = keep["MISS"]
    used_map = np.nonzero(miss == 0)
    mstar = np.full(N, T // C, np.int32)
    for m_, n_ in zip(*used_map):
        mstar[n_] = min(mstar[n_], m_ + 1)
    assert np.array_equal(host(run.view("MSTAR", torch.int32)), mstar), tag
    assert np.array_equal(host(U), Uo) and np.array_equal(host(W), Wo) and np.array_equal(host(S), So)
    for k in ("miss_frac", "overflow_frac", "mean_lines", "mean_pieces"):
        assert st[k] == pytest.approx(sto[k], abs=1e-12), (tag, k)
    assert st["max_pieces"] == sto["max_pieces"] and st["repair_iters"] == 0


@pytest.mark.parametrize("name,beta,rho,q", NEURONS)
@pytest.mark.parametrize("block", [1, 2, 4, 8, 16])
def test_alif_box_scan_matches_oracle(AL, dev, name, beta, rho, q, block):
    """repair = 0: every intermediate of the box scan and the replayed outputs equal the
    oracle's (same block of the split decision); N = 72, so the carry runs one neuron a wave."""
    T, N, C, K1, K2 = 2048, 72, 128, 16, 32
    I = _inputs(beta, 2.0, T, N, 9)
    u0 = np.zeros(N, np.float32)
    w0 = uniform(N, 0.0, 0.1, 10)
    _, preds = _preds(I, beta, rho, q, u0, w0, C)
    for tag in ("oracle", "warm4", "bad"):
        print(f"alif box {name} block={block} pred={tag}", flush=True)
        _check_box_scan(AL, dev, I, u0, w0, preds[tag], 0.1 * q, beta, rho, q, C, K1, K2, block, tag)


def test_alif_box_scan_matches_oracle_four_neurons_a_wave(AL, dev):
    """The same intermediates above the carry's one-neuron-a-wave range (N = 1030 > 1024: four
    neurons a wave, the last workgroup partial), for a good and a bad prediction."""
    beta, rho, q = 0.95, 0.995, 0.9
    T, N, C, K1, K2 = 512, 1030, 128, 16, 32
    I = _inputs(beta, 2.0, T, N, 9)
    u0 = np.zeros(N, np.float32)
    w0 = uniform(N, 0.0, 0.1, 10)
    _, preds = _preds(I, beta, rho, q, u0, w0, C)
    for tag in ("oracle", "bad"):
        print(f"alif box N={N} pred={tag}", flush=True)
        _check_box_scan(AL, dev, I, u0, w0, preds[tag], 0.1 * q, beta, rho, q, C, K1, K2, 4, tag)


@pytest.mark.parametrize("M", [1, 2, 3])
def test_alif_box_scan_converged_few_chunks(AL, dev, M):
    """Repair to convergence with one to three chunks: M = 1 runs the replay only (no serial
    pass), M = 2, 3 the replay below MSTAR and the serial pass from the least MSTAR; the result
    is the serial recurrence for a good and a bad prediction."""
    beta, rho, q = 0.95, 0.995, 0.9
    C, N = 128, 100
    T = M * C
    I = _inputs(beta, 2.0, T, N, 17)
    u0 = np.zeros(N, np.float32)
    w0 = uniform(N, 0.0, 0.1, 18)
    (Ur, Wr, Sr), preds = _preds(I, beta, rho, q, u0, w0, C)
    for tag in ("oracle", "bad"):
        print(f"alif converged M={M} pred={tag}", flush=True)
        U, W, S = AL.alif_scan_forward_maps(gpu(I, dev), beta, rho, q, 1.0, 0.0, gpu(u0, dev),
                                            gpu(w0, dev), gpu(preds[tag], dev), 0.1 * q, C=C, K1=32,
                                            K2=32, BN=4, repair=10 ** 6)
        assert np.array_equal(host(U), Ur) and np.array_equal(host(W), Wr), tag
        assert np.array_equal(host(S), Sr), tag


def test_alif_box_scan_chunk_not_multiple_of_16(AL, dev):
    """C = 40: the carry's fallback streams its inputs row by row (the register path needs C a
    multiple of 16) and the converged pass starts inside a 64-row tile; intermediates equal the
    oracle's, the converged scan the serial recurrence."""
    beta, rho, q = 0.95, 0.995, 0.9
    T, N, C = 2000, 70, 40
    I = _inputs(beta, 2.0, T, N, 15)
    u0 = np.zeros(N, np.float32)
    w0 = uniform(N, 0.0, 0.1, 16)
    (Ur, Wr, Sr), preds = _preds(I, beta, rho, q, u0, w0, C)
    for tag in ("oracle", "warm4"):
        Wp = preds[tag]
        print(f"alif box C=40 pred={tag}", flush=True)
        st, sto, keep = {}, {}, {}
        U, W, S = AL.alif_scan_forward(gpu(I, dev), beta, rho, q, 1.0, 0.0, gpu(u0, dev), gpu(w0, dev),
                                       gpu(Wp, dev), 0.1 * q, C=C, K1=16, K2=32, BN=4, repair=0, stats=st)
        run = AL.last_alif_run()
        Uo, Wo, So = A.scan_forward(I, beta, rho, q, 1.0, 0.0, u0, w0, Wp, 0.1 * q, C=C, K1=16, K2=32,
                                    block=4, repair=0, stats=sto, keep=keep)
        for g in ("SU", "SW"):
            assert np.array_equal(host(run.view(g)), keep[g]), (tag, g)
        assert np.array_equal(host(run.view("MISS", torch.int32)), keep["MISS"]), tag
        assert np.array_equal(host(U), Uo) and np.array_equal(host(W), Wo) and np.array_equal(host(S), So)
        U, W, S = AL.alif_scan_forward_maps(gpu(I, dev), beta, rho, q, 1.0, 0.0, gpu(u0, dev),
                                            gpu(w0, dev), gpu(Wp, dev), 0.1 * q, C=C, K1=16, K2=32, BN=4,
                                            repair=10 ** 6)
        assert np.array_equal(host(U), Ur) and np.array_equal(host(W), Wr), tag
        assert np.array_equal(host(S), Sr), tag


@pytest.mark.parametrize("name,beta,rho,q", NEURONS)
@pytest.mark.parametrize("mfree", [0.5, 2.0])
def test_alif_box_scan_with_repair_equals_serial(AL, dev, name, beta, rho, q, mfree):
    """The reference's contract (tests/test_alif.py:10-39): with repair the box scan equals the
    serial recurrence for any prediction, good or bad; with the Jacobi rounds (stats requested)
    and with the ordered chain pass (no stats)."""
    T, N, C = 4096, 200, 128
    I = _inputs(beta, mfree, T, N, 11)
    u0 = np.zeros(N, np.float32)
    w0 = uniform(N, 0.0, 0.1, 12)
    (Ur, Wr, Sr), preds = _preds(I, beta, rho, q, u0, w0, C)
    Ig, ug, wg = gpu(I, dev), gpu(u0, dev), gpu(w0, dev)
    for tag, Wp in preds.items():
        for block in (1, 4):
            print(f"alif repair {name} mfree={mfree} pred={tag} block={block}", flush=True)
            st, sto = {}, {}
            U, W, S = AL.alif_scan_forward(Ig, beta, rho, q, 1.0, 0.0, ug, wg, gpu(Wp, dev), 0.1 * q,
                                           C=C, K1=16, K2=32, BN=block, repair=10 ** 6, stats=st)
            assert np.array_equal(host(U), Ur) and np.array_equal(host(W), Wr), (tag, block)
            assert np.array_equal(host(S), Sr), (tag, block)
            # without stats the pipeline's converged repair is the ordered chain pass: the same
            # result; alif_scan_forward itself then takes the serial forward
            U, W, S = AL.alif_scan_forward_maps(Ig, beta, rho, q, 1.0, 0.0, ug, wg, gpu(Wp, dev),
                                                0.1 * q, C=C, K1=16, K2=32, BN=block, repair=10 ** 6)
            assert np.array_equal(host(U), Ur) and np.array_equal(host(W), Wr), (tag, block, "chain")
            assert np.array_equal(host(S), Sr), (tag, block, "chain")
            U, W, S = AL.alif_scan_forward(Ig, beta, rho, q, 1.0, 0.0, ug, wg, gpu(Wp, dev), 0.1 * q,
                                           C=C, K1=16, K2=32, BN=block, repair=10 ** 6)
            assert np.array_equal(host(U), Ur) and np.array_equal(host(W), Wr), (tag, block, "dispatch")
            assert np.array_equal(host(S), Sr), (tag, block, "dispatch")
            if T * N <= 4096 * 200 and block == 4 and tag in ("oracle", "bad"):
                A.scan_forward(I, beta, rho, q, 1.0, 0.0, u0, w0, Wp, 0.1 * q, C=C, K1=16, K2=32,
                               block=block, repair=10 ** 6, stats=sto)
                assert st["repair_iters"] == sto["repair_iters"]
                assert st["miss_frac"] == pytest.approx(sto["miss_frac"], abs=1e-12)


def test_alif_converged_dispatch(AL, dev):
    """alif_scan_forward with the repair budget at least T/C and neither stats nor phases computes
    the serial recurrence by the serial forward (the same bits as the box-scan pipeline's
    converged call), keeps the pipeline's argument checks, and runs the pipeline when phases or
    stats are asked for or the budget is finite."""
    beta, rho, q = 0.95, 0.995, 0.9
    T, N, C = 1024, 70, 128
    I = _inputs(beta, 2.0, T, N, 19)
    u0 = np.zeros(N, np.float32)
    w0 = uniform(N, 0.0, 0.1, 20)
    (Ur, Wr, Sr), preds = _preds(I, beta, rho, q, u0, w0, C)
    Ig, ug, wg, Wp = gpu(I, dev), gpu(u0, dev), gpu(w0, dev), gpu(preds["warm4"], dev)
    print("alif converged dispatch", flush=True)
    AL.alif_scan_forward(Ig, beta, rho, q, 1.0, 0.0, ug, wg, Wp, 0.1 * q, C=C, repair=0)
    before = AL.last_alif_run()
    U, W, S = AL.alif_scan_forward(Ig, beta, rho, q, 1.0, 0.0, ug, wg, Wp, 0.1 * q, C=C, repair=10 ** 6)
    assert AL.last_alif_run() is before  # no box-scan pipeline ran
    assert np.array_equal(host(U), Ur) and np.array_equal(host(W), Wr) and np.array_equal(host(S), Sr)
    ph = {}
    U, W, S = AL.alif_scan_forward(Ig, beta, rho, q, 1.0, 0.0, ug, wg, Wp, 0.1 * q, C=C, repair=10 ** 6,
                                   phases=ph)
    assert AL.last_alif_run() is not before and set(ph) == {"envelope", "build", "carry", "replay"}
    assert np.array_equal(host(U), Ur) and np.array_equal(host(W), Wr) and np.array_equal(host(S), Sr)
    with pytest.raises(ValueError):
        AL.alif_scan_forward(Ig, beta, rho, q, 1.0, 0.0, ug, wg, Wp, 0.1 * q, C=100, repair=10 ** 6)
    with pytest.raises(ValueError):
        AL.alif_scan_forward(Ig, beta, rho, q, 1.0, 0.0, ug, wg, Wp[1:], 0.1 * q, C=C, repair=10 ** 6)
    with pytest.raises(ValueError):
        AL.alif_scan_forward(Ig, beta, rho, q, 1.0, 0.0, ug, wg, Wp, 0.1 * q, C=C, K2=24, repair=10 ** 6)


@pytest.mark.parametrize("R", [1, 2, 5])
def test_alif_finite_repair_rounds(AL, dev, R):
    beta, rho, q = 0.95, 0.995, 0.9
    T, N, C = 2048, 64, 64
    I = _inputs(beta, 2.0, T, N, 13)
    u0 = np.zeros(N, np.float32)
    w0 = np.zeros(N, np.float32)
    _, preds = _preds(I, beta, rho, q, u0, w0, C)
    Wp = preds["bad"]
    print(f"alif finite repair R={R}", flush=True)
    st, sto = {}, {}
    U, W, S = AL.alif_scan_forward(gpu(I, dev), beta, rho, q, 1.0, 0.0, gpu(u0, dev), gpu(w0, dev),
                                   gpu(Wp, dev), 0.1 * q, C=C, K1=16, K2=32, BN=1, repair=R, stats=st)
    Uo, Wo, So = A.scan_forward(I, beta, rho, q, 1.0, 0.0, u0, w0, Wp, 0.1 * q, C=C, K1=16, K2=32,
                                block=1, repair=R, stats=sto)
    assert np.array_equal(host(U), Uo) and np.array_equal(host(W), Wo) and np.array_equal(host(S), So)
    assert st["repair_iters"] == sto["repair_iters"]


def test_alif_scan_phases_and_shapes(AL, dev):
    beta, rho, q = 0.95, 0.995, 0.9
    T, N, C = 1024, 64, 128
    I = gpu(_inputs(beta, 2.0, T, N, 14), dev)
    z = torch.zeros(N, device=dev)
    Wp = torch.zeros(T // C, N, device=dev)
    ph = {}
    AL.alif_scan_forward(I, beta, rho, q, 1.0, 0.0, z, z, Wp, 0.1, C=C, phases=ph)
    assert set(ph) == {"envelope", "build", "carry", "replay"} and all(v >= 0 for v in ph.values())
    with pytest.raises(ValueError):
        AL.alif_scan_forward(I, beta, rho, q, 1.0, 0.0, z, z, Wp, 0.1, C=100)
    with pytest.raises(ValueError):
        AL.alif_scan_forward(I, beta, rho, q, 1.0, 0.0, z, z, Wp, 0.1, C=C, K2=24)
    with pytest.raises(ValueError):
        AL.alif_scan_forward(I, beta, rho, q, 1.0, 0.0, z, z, Wp[1:], 0.1, C=C)


@pytest.mark.parametrize("beta,rho,q", [(0.95, 0.995, 0.9), (0.99, 0.96, 0.2)])
@pytest.mark.parametrize("mode,C", [("serial", 64), ("chunked", 64), ("chunked", 16), ("fused", 16),
                                    ("fused", 32), ("lookback", 16)])
def test_alif_backward_modes(AL, dev, beta, rho, q, mode, C):
    T, N = 1024, 130
    x = _inputs(beta, 2.0, T, N, 15)
    G = normal(T, N, 0.0, 1.0, 16)
    u0 = uniform(N, -0.1, 0.3, 17)
    w0 = uniform(N, 0.0, 0.2, 18)
    U, W, S = A.serial_forward(x, beta, rho, q, 1.0, 0.0, u0, w0)
    print(f"alif bwd {mode} C={C} beta={beta}", flush=True)
    LV, LW = AL.alif_backward(gpu(x, dev), gpu(U, dev), gpu(W, dev), gpu(S, dev), gpu(G, dev), beta, rho, q,
                              1.0, gpu(u0, dev), gpu(w0, dev), alpha=4.0, mode=mode, C=C)
    LVo, LWo = A.backward(x, U, W, S, G, beta, rho, q, 1.0, u0, w0, 4.0)
    LV6, LW6 = A.backward(x, U, W, S, G, beta, rho, q, 1.0, u0, w0, 4.0, dtype=np.float64)
    assert rel(host(LV), LVo) < 1e-5 and rel(host(LW), LWo) < 1e-5
    assert rel(host(LV), LV6) < 1e-4 and rel(host(LW), LW6) < 1e-4


def test_alif_backward_rejects(AL, dev):
    T, N = 100, 8
    z = torch.zeros(T, N, device=dev)
    v = torch.zeros(N, device=dev)
    with pytest.raises(ValueError):
        AL.alif_backward(z, z, z, z, z, 0.9, 0.95, 0.5, 1.0, v, v, mode="chunked", C=64)
    with pytest.raises(ValueError):
        AL.alif_backward(z, z, z, z, z, 0.9, 0.95, 0.5, 1.0, v, v, mode="fused", C=16)
    with pytest.raises(ValueError):
        AL.alif_backward(z, z, z, z, z, 0.9, 0.95, 0.5, 1.0, v, v, mode="nope")


@pytest.mark.parametrize("fwd,bwd", [("serial", "serial"), ("serial", "scan"), ("scan", "scan")])
@pytest.mark.parametrize("beta,rho,q,T,N", [(0.95, 0.995, 0.9, 1024, 96), (0.99, 0.96, 0.2, 4096, 8)])
def test_alif_layer_gradients(AL, dev, fwd, bwd, beta, rho, q, T, N):
    """alif() gradients for I, u0, w0 and the four parameters against the fp64 adjoint and
    ALIFFn's assembly (triton_alif.py:541-554); the second case is the reference's own
    (tests/test_alif_grad.py:8-36, bar 1e-3 there; param_bars here)."""
    C = 128
    x = _inputs(beta, 2.0, T, N, 19)
    G = normal(T, N, 0.0, 1.0, 20)
    u0 = uniform(N, -0.1, 0.3, 21) if N > 8 else np.zeros(N, np.float32)
    w0 = uniform(N, 0.0, 0.2, 22) if N > 8 else np.zeros(N, np.float32)
    U, W, S = A.serial_forward(x, beta, rho, q, 1.0, 0.0, u0, w0)
    Wentry = np.concatenate([w0[None], W[C - 1:-1:C]], 0)
    if fwd == "scan":  # the layer's scan runs without repair (triton_alif.py:535)
        U, W, S = A.scan_forward(x, beta, rho, q, 1.0, 0.0, u0, w0, Wentry, 0.1 * q, C=C, K1=32, K2=32,
                                 block=4, repair=0)
    xg = gpu(x, dev).requires_grad_(True)
    ug = gpu(u0, dev).requires_grad_(True)
    wg = gpu(w0, dev).requires_grad_(True)
    ps = [torch.tensor(v, device=dev, requires_grad=True) for v in (beta, rho, q, 1.0)]
    print(f"alif layer fwd={fwd} bwd={bwd}", flush=True)
    Sg, Ug, Wg = AL.alif(xg, ug, wg, *ps, fwd=fwd, bwd=bwd, Wpred=gpu(Wentry, dev), dw=0.1 * q, C=C, Cb=64)
    assert np.array_equal(host(Sg), S) and np.array_equal(host(Ug), U) and np.array_equal(host(Wg), W)
    (Sg * gpu(G, dev)).sum().backward()
    LV6, LW6 = A.backward(x, U, W, S, G, beta, rho, q, 1.0, u0, w0, 4.0, dtype=np.float64)
    want = A.param_grads(x, U, W, S, G, LV6, LW6, beta, rho, q, 1.0, u0, w0, 4.0)
    got = (xg.grad, ug.grad, wg.grad, *(p.grad for p in ps))
    for k, (a, b) in enumerate(zip(got[:3], want[:3])):
        assert rel(host(a), b) < 1e-4, k
    bars, floors = param_bars(x, U, W, S, G, beta, rho, q, u0, w0, want)
    check_params([host(p) for p in got[3:]], want, bars, floors, f"layer {fwd}/{bwd}")


@pytest.mark.parametrize("mode,C", [("serial", 64), ("chunked", 64), ("fused", 16), ("fused", 32),
                                    ("lookback", 16)])
@pytest.mark.parametrize("T,N", [(1024, 130), (77 * 16, 33)])
def test_alif_backward_param_sums_and_dw0(AL, dev, mode, C, T, N):
    """The adjoint kernels' own reductions (dL/dw0 and the four parameter sums, one fp64 row per
    block) against the fp64 assembly of ALIFFn.backward (triton_alif.py:541-554); LV the same
    with and without LW written."""
    from lifscan import hip_alif
    beta, rho, q = 0.95, 0.995, 0.9
    if mode == "lookback" and T % 128:  # its segments are 128 steps: refused, not mis-computed
        z = torch.zeros(T, N, device=dev)
        v = torch.zeros(N, device=dev)
        with pytest.raises(ValueError):
            hip_alif._alif_bwd_call(z, z, z, z, z, beta, rho, q, 1.0, v, v, 4.0, mode, C,
                                    want_lw=False, want_params=True)
        return
    if mode != "serial" and T % C:
        C = 16
    x = _inputs(beta, 2.0, T, N, 23)
    G = normal(T, N, 0.0, 1.0, 24)
    u0 = uniform(N, -0.1, 0.3, 25)
    w0 = uniform(N, 0.0, 0.2, 26)
    U, W, S = A.serial_forward(x, beta, rho, q, 1.0, 0.0, u0, w0)
    args = [gpu(a, dev) for a in (x, U, W, S, G)]
    print(f"alif bwd sums {mode} C={C} T={T} N={N}", flush=True)
    LV, LW, DW0, sums = hip_alif._alif_bwd_call(*args, beta, rho, q, 1.0, gpu(u0, dev), gpu(w0, dev), 4.0,
                                                mode, C, want_lw=False, want_params=True)
    LV2, LW2 = AL.alif_backward(*args, beta, rho, q, 1.0, gpu(u0, dev), gpu(w0, dev), mode=mode, C=C)
    # the variant without LW may group chunks into rounds differently (another rounding order)
    assert LW is None and rel(host(LV), host(LV2)) < 1e-6
    LV6, LW6 = A.backward(x, U, W, S, G, beta, rho, q, 1.0, u0, w0, 4.0, dtype=np.float64)
    want = A.param_grads(x, U, W, S, G, LV6, LW6, beta, rho, q, 1.0, u0, w0, 4.0)
    assert rel(host(DW0), want[2]) < 1e-4
    got = host(sums)
    bars, floors = param_bars(x, U, W, S, G, beta, rho, q, u0, w0, want)
    check_params([got[0], got[1], got[2], -got[3]], want, bars, floors, f"sums T={T} N={N}")


@pytest.mark.parametrize("mode,C", [("serial", 64), ("chunked", 64), ("fused", 16), ("fused", 32)])
def test_alif_device_params_entries_bitexact(AL, dev, mode, C):
    """lsh_alif_serial_fwd_dparams and lsh_alif_bwd_dparams (parameters read from a device
    vector) give the bits of the entries that take them as floats: U, W, S, LV, LW, dL/dw0 and
    the parameter partial sums."""
    from lifscan import hip_alif
    beta, rho, q, th = 0.95, 0.995, 0.9, 1.0
    T, N = 1024, 130
    x = _inputs(beta, 2.0, T, N, 31)
    G = normal(T, N, 0.0, 1.0, 32)
    u0 = gpu(uniform(N, -0.1, 0.3, 33), dev)
    w0 = gpu(uniform(N, 0.0, 0.2, 34), dev)
    xg = gpu(x, dev)
    print(f"alif dparams {mode} C={C}", flush=True)
    dp = hip_alif._dev_params(xg, torch.tensor(beta, device=dev), rho, q, th)
    U, W, S = AL.alif_serial_forward(xg, beta, rho, q, th, 0.0, u0, w0)
    U2, W2, S2 = hip_alif._alif_serial_forward_dp(xg, dp, 0.0, u0, w0)
    assert torch.equal(U, U2) and torch.equal(W, W2) and torch.equal(S, S2)
    args = (xg, U, W, S, gpu(G, dev), beta, rho, q, th, u0, w0, 4.0, mode, C)
    ref = hip_alif._alif_bwd_call(*args, want_lw=True, want_params=True)
    got = hip_alif._alif_bwd_call(*args[:5], None, None, None, None, *args[9:], want_lw=True,
                                  want_params=True, dp=dp)
    for a, b in zip(ref, got):
        assert torch.equal(a, b)


@pytest.mark.parametrize("fwd", ["serial", "scan"])
def test_alif_float_and_tensor_params_agree(AL, dev, fwd):
    """alif() with float parameters (kernel arguments), with device tensors (read on the device
    by the serial forward and the adjoint) and with a mix: identical S, U, W and input
    gradients; parameter gradients only for the tensors, equal to the all-tensor call's."""
    beta, rho, q, T, N, C = 0.95, 0.995, 0.9, 1024, 96, 128
    x = _inputs(beta, 2.0, T, N, 35)
    G = gpu(normal(T, N, 0.0, 1.0, 36), dev)
    u0 = uniform(N, -0.1, 0.3, 37)
    w0 = uniform(N, 0.0, 0.2, 38)
    _, W, _ = A.serial_forward(x, beta, rho, q, 1.0, 0.0, u0, w0)
    Wp = gpu(np.concatenate([w0[None], W[C - 1:-1:C]], 0), dev)
    print(f"alif float/tensor params fwd={fwd}", flush=True)

    def run(ps):
        xg = gpu(x, dev).requires_grad_(True)
        ug = gpu(u0, dev).requires_grad_(True)
        wg = gpu(w0, dev).requires_grad_(True)
        out = AL.alif(xg, ug, wg, *ps, fwd=fwd, bwd="scan", Wpred=Wp, dw=0.1 * q, C=C)
        (out[0] * G).sum().backward()
        return out, (xg.grad, ug.grad, wg.grad)

    o1, g1 = run([beta, rho, q, 1.0])
    pt = [torch.tensor(v, device=dev, requires_grad=True) for v in (beta, rho, q, 1.0)]
    o2, g2 = run(pt)
    pm = [torch.tensor(beta, device=dev, requires_grad=True), rho,
          torch.tensor(q, device=dev, requires_grad=True), 1.0]
    o3, g3 = run(pm)
    for a, b, c in zip(o1, o2, o3):
        assert torch.equal(a, b) and torch.equal(a, c)
    # below 8192 neurons the adjoint is the look-back pass (deterministic: the same bits)
    for a, b, c in zip(g1, g2, g3):
        assert torch.equal(a, b) and torch.equal(a, c)
    assert torch.equal(pm[0].grad, pt[0].grad) and torch.equal(pm[2].grad, pt[2].grad)
    assert all(p.grad is not None for p in pt)


@pytest.mark.parametrize("C", [16, 32])
@pytest.mark.parametrize("T,N,u_r", [(1024, 130, 0.0), (512, 33, -0.2), (32, 70, 0.1)])
def test_alif_recompute_bwd_bitexact(AL, dev, C, T, N, u_r):
    """lsh_alif_bwd_recompute (S not read, U and W only before each chunk) equals the single pass
    that reads the stored states, bit for bit, for float and device parameters; and both match
    the fp64 adjoint."""
    from lifscan import hip_alif
    beta, rho, q, th = 0.95, 0.995, 0.9, 1.0
    x = _inputs(beta, 2.0, T, N, 41)
    G = normal(T, N, 0.0, 1.0, 42)
    u0 = uniform(N, -0.1, 0.3, 43)
    w0 = uniform(N, 0.0, 0.2, 44)
    U, W, S = A.serial_forward(x, beta, rho, q, th, u_r, u0, w0)
    args = [gpu(a, dev) for a in (x, U, W, S, G)]
    ug, wg = gpu(u0, dev), gpu(w0, dev)
    print(f"alif recompute bwd C={C} T={T} N={N} u_r={u_r}", flush=True)
    ref = hip_alif._alif_bwd_call(*args, beta, rho, q, th, ug, wg, 4.0, "fused", C, want_lw=True,
                                  want_params=True)
    got = hip_alif._alif_bwd_call(*args, beta, rho, q, th, ug, wg, 4.0, "fused", C, want_lw=True,
                                  want_params=True, recompute_ur=u_r)
    dp = hip_alif._dev_params(args[0], torch.tensor(beta, device=dev), rho, q, th)
    got2 = hip_alif._alif_bwd_call(*args[:3], None, args[4], None, None, None, None, ug, wg, 4.0, "fused",
                                   C, want_lw=True, want_params=True, dp=dp, recompute_ur=u_r)
    for a, b, c in zip(ref, got, got2):
        assert torch.equal(a, b) and torch.equal(a, c)
    LV6, LW6 = A.backward(x, U, W, S, G, beta, rho, q, th, u0, w0, 4.0, dtype=np.float64)
    assert rel(host(got[0]), LV6) < 1e-4 and rel(host(got[1]), LW6) < 1e-4


def test_alif_layer_recompute_equals_stored(AL, dev, monkeypatch):
    """alif(fwd="serial", bwd="scan") at N >= 8192 takes the recomputing single pass: the
    gradients for I, u0, w0 and the four parameters equal those of the stored-state pass."""
    from lifscan import hip_alif
    beta, rho, q, T, N = 0.95, 0.995, 0.2, 256, 8256
    x = gpu(_inputs(beta, 2.0, T, N, 45), dev)
    G = gpu(normal(T, N, 0.0, 1.0, 46), dev)
    u0 = gpu(uniform(N, -0.1, 0.3, 47), dev)
    w0 = gpu(uniform(N, 0.0, 0.2, 48), dev)
    print("alif layer recompute vs stored", flush=True)

    def run(flag):
        monkeypatch.setattr(hip_alif, "ALIF_RECOMPUTE_BWD", flag)
        xg, ug, wg = (a.clone().requires_grad_(True) for a in (x, u0, w0))
        ps = [torch.tensor(v, device=dev, requires_grad=True) for v in (beta, rho, q, 1.0)]
        S, _, _ = AL.alif(xg, ug, wg, *ps, u_r=-0.1, fwd="serial", bwd="scan")
        (S * G).sum().backward()
        return [xg.grad, ug.grad, wg.grad] + [p.grad for p in ps]

    for a, b in zip(run(True), run(False)):
        assert torch.equal(a, b)


@pytest.mark.parametrize("T,N", [(1, 1), (63, 64), (64, 100), (65, 7), (1000, 130), (4113, 1029)])
def test_alif_serial_bwd_pipe(AL, dev, T, N):
    """The producer/consumer serial adjoint (mode 0; full and partial tiles, ragged neuron blocks):
    LV, LW and dL/dw0 within 1e-5 of the fp32 oracle and 1e-4 of the fp64 adjoint, the parameter
    sums within param_bars of their fp64 assembly; alif_backward(mode="serial") gives the same
    bits."""
    from lifscan import hip_alif
    beta, rho, q = 0.95, 0.995, 0.9
    x = _inputs(beta, 2.0, T, N, 51)
    G = normal(T, N, 0.0, 1.0, 52)
    u0 = uniform(N, -0.1, 0.3, 53)
    w0 = uniform(N, 0.0, 0.2, 54)
    U, W, S = A.serial_forward(x, beta, rho, q, 1.0, 0.0, u0, w0)
    args = [gpu(a, dev) for a in (x, U, W, S, G)]
    ug, wg = gpu(u0, dev), gpu(w0, dev)
    print(f"alif serial bwd pipe T={T} N={N}", flush=True)
    LV, LW, DW0, sums = hip_alif._alif_bwd_call(*args, beta, rho, q, 1.0, ug, wg, 4.0, "serial", 64,
                                                want_lw=True, want_params=True)
    LV2, LW2 = AL.alif_backward(*args, beta, rho, q, 1.0, ug, wg, mode="serial")
    assert torch.equal(LV, LV2) and torch.equal(LW, LW2)
    LVo, LWo = A.backward(x, U, W, S, G, beta, rho, q, 1.0, u0, w0, 4.0)
    LV6, LW6 = A.backward(x, U, W, S, G, beta, rho, q, 1.0, u0, w0, 4.0, dtype=np.float64)
    assert rel(host(LV), LVo) < 1e-5 and rel(host(LW), LWo) < 1e-5
    assert rel(host(LV), LV6) < 1e-4 and rel(host(LW), LW6) < 1e-4
    want = A.param_grads(x, U, W, S, G, LV6, LW6, beta, rho, q, 1.0, u0, w0, 4.0)
    assert rel(host(DW0), want[2]) < 1e-4
    got = host(sums)
    bars, floors = param_bars(x, U, W, S, G, beta, rho, q, u0, w0, want)
    check_params([got[0], got[1], got[2], -got[3]], want, bars, floors, f"sums T={T} N={N}")


@pytest.mark.parametrize("T,N", [(1, 1), (63, 64), (64, 100), (65, 7), (1000, 130), (4113, 1029)])
def test_alif_serial_fwd_pipe(AL, dev, T, N):
    """The producer/consumer serial forward gives U, W, S of the oracle bit for bit, with float
    and with device parameters."""
    from lifscan import hip_alif
    beta, rho, q = 0.95, 0.995, 0.9
    x = _inputs(beta, 2.0, T, N, 55)
    u0 = uniform(N, -0.1, 0.3, 56)
    w0 = uniform(N, 0.0, 0.2, 57)
    Ur, Wr, Sr = A.serial_forward(x, beta, rho, q, 1.0, 0.0, u0, w0)
    xg, ug, wg = gpu(x, dev), gpu(u0, dev), gpu(w0, dev)
    print(f"alif serial fwd pipe T={T} N={N}", flush=True)
    got = AL.alif_serial_forward(xg, beta, rho, q, 1.0, 0.0, ug, wg)
    dp = hip_alif._dev_params(xg, torch.tensor(beta, device=dev), rho, q, 1.0)
    got2 = hip_alif._alif_serial_forward_dp(xg, dp, 0.0, ug, wg)
    for b, c, o in zip(got, got2, (Ur, Wr, Sr)):
        assert torch.equal(b, c) and np.array_equal(host(b), o)


@pytest.mark.parametrize("T,N", [(128, 1), (1280, 64), (4096, 70), (16384, 130)])
def test_alif_lookback_bwd(AL, dev, T, N):
    """The look-back single pass (mode 3): LV and LW against the fp32 oracle and the fp64
    adjoint, dL/dw0 and the four sums against the fp64 assembly, with float and device
    parameters (the same bits: the look-back's association order is fixed), and no bounded wait
    given up."""
    from lifscan import hip_alif
    beta, rho, q = 0.95, 0.995, 0.9
    x = _inputs(beta, 2.0, T, N, 95)
    G = normal(T, N, 0.0, 1.0, 96)
    u0 = uniform(N, -0.1, 0.3, 97)
    w0 = uniform(N, 0.0, 0.2, 98)
    U, W, S = A.serial_forward(x, beta, rho, q, 1.0, 0.0, u0, w0)
    args = [gpu(a, dev) for a in (x, U, W, S, G)]
    ug, wg = gpu(u0, dev), gpu(w0, dev)
    print(f"alif lookback T={T} N={N}", flush=True)
    LV, LW, DW0, sums = hip_alif._alif_bwd_call(*args, beta, rho, q, 1.0, ug, wg, 4.0, "lookback", 16,
                                                want_lw=True, want_params=True)
    assert hip_alif.last_bwd_spin_timeouts() == 0
    dp = hip_alif._dev_params(args[0], torch.tensor(beta, device=dev), rho, q, 1.0)
    got = hip_alif._alif_bwd_call(*args, None, None, None, None, ug, wg, 4.0, "lookback", 16,
                                  want_lw=True, want_params=True, dp=dp)
    for a, b in zip((LV, LW, DW0, sums), got):  # deterministic look-back: the same bits
        assert torch.equal(a, b)
    LVo, LWo = A.backward(x, U, W, S, G, beta, rho, q, 1.0, u0, w0, 4.0)
    LV6, LW6 = A.backward(x, U, W, S, G, beta, rho, q, 1.0, u0, w0, 4.0, dtype=np.float64)
    assert rel(host(LV), LVo) < 1e-5 and rel(host(LW), LWo) < 1e-5
    assert rel(host(LV), LV6) < 1e-4 and rel(host(LW), LW6) < 1e-4
    want = A.param_grads(x, U, W, S, G, LV6, LW6, beta, rho, q, 1.0, u0, w0, 4.0)
    assert rel(host(DW0), want[2]) < 1e-4
    got_s = host(sums)
    bars, floors = param_bars(x, U, W, S, G, beta, rho, q, u0, w0, want)
    check_params([got_s[0], got_s[1], got_s[2], -got_s[3]], want, bars, floors, f"lookback T={T} N={N}")


@pytest.mark.parametrize("T,N,u_r", [(1280, 130, 0.0), (512, 33, -0.2)])
def test_alif_lookback_recompute(AL, dev, T, N, u_r):
    """The look-back pass recomputing the chunk states (lsh_alif_bwd_recompute, mode 3) agrees with
    the look-back pass reading them, for float and device parameters, bit for bit (the recomputed
    chunk states are the stored bits, and the look-back's association order is fixed)."""
    from lifscan import hip_alif
    beta, rho, q, th = 0.95, 0.995, 0.9, 1.0
    x = _inputs(beta, 2.0, T, N, 101)
    G = normal(T, N, 0.0, 1.0, 102)
    u0 = uniform(N, -0.1, 0.3, 103)
    w0 = uniform(N, 0.0, 0.2, 104)
    U, W, S = A.serial_forward(x, beta, rho, q, th, u_r, u0, w0)
    args = [gpu(a, dev) for a in (x, U, W, S, G)]
    ug, wg = gpu(u0, dev), gpu(w0, dev)
    print(f"alif lookback recompute T={T} N={N}", flush=True)
    ref = hip_alif._alif_bwd_call(*args, beta, rho, q, th, ug, wg, 4.0, "lookback", 16, want_lw=True,
                                  want_params=True)
    got = hip_alif._alif_bwd_call(*args, beta, rho, q, th, ug, wg, 4.0, "lookback", 16, want_lw=True,
                                  want_params=True, recompute_ur=u_r)
    dp = hip_alif._dev_params(args[0], torch.tensor(beta, device=dev), rho, q, th)
    got2 = hip_alif._alif_bwd_call(*args[:3], None, args[4], None, None, None, None, ug, wg, 4.0,
                                   "lookback", 16, want_lw=True, want_params=True, dp=dp,
                                   recompute_ur=u_r)
    assert hip_alif.last_bwd_spin_timeouts() == 0
    for a, b, c in zip(ref, got, got2):
        assert torch.equal(a, b) and torch.equal(a, c)


def test_alif_layer_small_n_recompute_equals_stored(AL, dev, monkeypatch):
    """alif(fwd="serial", bwd="scan") below 8192 neurons takes the recomputing look-back pass: the
    gradients of the look-back pass that reads the stored states, bit for bit."""
    from lifscan import hip_alif
    beta, rho, q, T, N = 0.95, 0.995, 0.2, 1024, 200
    x = gpu(_inputs(beta, 2.0, T, N, 105), dev)
    G = gpu(normal(T, N, 0.0, 1.0, 106), dev)
    u0 = gpu(uniform(N, -0.1, 0.3, 107), dev)
    w0 = gpu(uniform(N, 0.0, 0.2, 108), dev)
    print("alif layer small-N recompute vs stored", flush=True)

    def run(flag):
        monkeypatch.setattr(hip_alif, "ALIF_RECOMPUTE_BWD", flag)
        xg, ug, wg = (a.clone().requires_grad_(True) for a in (x, u0, w0))
        ps = [torch.tensor(v, device=dev, requires_grad=True) for v in (beta, rho, q, 1.0)]
        S, _, _ = AL.alif(xg, ug, wg, *ps, u_r=-0.1, fwd="serial", bwd="scan")
        (S * G).sum().backward()
        return [xg.grad, ug.grad, wg.grad] + [p.grad for p in ps]

    for a, b in zip(run(True), run(False)):
        assert torch.equal(a, b)
