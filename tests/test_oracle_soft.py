"""Pins of the soft-reset oracle (oracle/soft_oracle.py).

The GPU path runs the soft reset as the affine reset with gamma = 1, delta = -theta.  These tests
show, on the CPU, that the literal restatement of triton_soft.py (common slope, offsets only)
and the affine oracle give the same bits for the step, both envelopes, every piece, the counts,
the overflow flags and the carried chunk starts; that the repaired scan equals the serial
recurrence on the reference's own grid (tests/test_soft_scan.py, smaller T and N); and that the
FFT adjoint equals the direct float64 recurrence, which equals fp64 autograd of the serial
recurrence with the detached reset (tests/test_soft_gpu.py, tests/test_soft_scan_grad.py).
"""
import numpy as np
import pytest
import torch

from oracle import affine_oracle as A
from oracle import soft_oracle as SO
from tests._inputs import normal, uniform

CASES = [(0.9, 0.15, 0.4), (0.95, -0.1, 0.6), (0.97, 0.4, 0.3), (0.99, 0.15, 0.4)]


def _inputs(mu, sd, T, N, seed):
    g = torch.Generator().manual_seed(seed)
    I = (mu + sd * torch.randn(T, N, generator=g)).numpy()
    u0 = (0.3 * torch.randn(N, generator=g)).numpy()
    return I, u0


@pytest.mark.parametrize("beta,mu,sd", CASES)
def test_soft_step_is_affine_with_gamma_one(beta, mu, sd):
    I, u0 = _inputs(mu, sd, 400, 50, 1)
    Us, Ss = SO.serial_forward(I, beta, 1.0, u0)
    Ua, Sa = A.serial_forward(I, beta, 1.0, 1.0, -1.0, u0)
    assert np.array_equal(Us, Ua) and np.array_equal(Ss, Sa)


@pytest.mark.parametrize("beta,mu,sd", CASES)
@pytest.mark.parametrize("C,K", [(16, 16), (32, 32), (32, 4)])
def test_soft_maps_equal_affine_maps(beta, mu, sd, C, K):
    T, N = 512, 40
    I, u0 = _inputs(mu, sd, T, N, 2)
    Lo_s, Hi_s = SO.envelopes(I, beta, 1.0, u0, C)
    Lo_a, Hi_a = A.envelopes(I, beta, 1.0, 1.0, -1.0, u0, C)
    assert np.array_equal(Lo_s, Lo_a) and np.array_equal(Hi_s, Hi_a)
    As, xl, xr, c, n, ovf = SO.build_maps(I, Lo_s, Hi_s, beta, 1.0, C, K)
    xl2, xr2, a2, c2, n2, ovf2 = A.build_maps(I, Lo_a, Hi_a, beta, 1.0, 1.0, -1.0, C, K)
    assert np.array_equal(n, n2) and np.array_equal(ovf, ovf2)
    assert np.array_equal(xl, xl2) and np.array_equal(xr, xr2) and np.array_equal(c, c2)
    live = np.arange(K)[None, None, :] < n[..., None]
    assert np.array_equal(np.broadcast_to(As[..., None], a2.shape)[live], a2[live])
    st_s = SO.carry(I, u0, As, xl, xr, c, n, ovf, beta, 1.0, C)
    st_a = A.carry(I, u0, xl2, xr2, a2, c2, n2, ovf2, beta, 1.0, 1.0, -1.0, C)
    assert np.array_equal(st_s, st_a)


@pytest.mark.parametrize("beta,mu,sd", CASES)
@pytest.mark.parametrize("C,K", [(16, 16), (32, 32)])
def test_soft_scan_with_repair_equals_serial(beta, mu, sd, C, K):
    I, u0 = _inputs(mu, sd, 1024, 32, 3)
    Ur, Sr = SO.serial_forward(I, beta, 1.0, u0)
    st = {}
    U, S = SO.scan_forward(I, beta, 1.0, u0, C=C, K=K, repair=10 ** 6, stats=st)
    assert np.array_equal(U, Ur) and np.array_equal(S, Sr)
    assert st["max_pieces"] <= K and st["mean_pieces"] >= 1.0


def test_fft_adjoint_is_the_float64_recurrence():
    T, N = 700, 9
    V = normal(T, N, 0.8, 0.4, 4)
    gS = normal(T, N, 0.0, 1.0, 5)
    fft = SO.adjoint_fft(V, gS, 0.95, 1.0)
    direct = SO.adjoint_direct64(V, gS, 0.95, 1.0)
    assert np.abs(fft - direct).max() <= 1e-6 * np.abs(direct).max()
    assert np.array_equal(fft, direct.astype(np.float32)) or \
        np.abs(fft - direct.astype(np.float32)).max() <= 2 ** -22 * np.abs(direct).max()


def test_direct_adjoint_matches_fp64_autograd():
    """fp64 autograd of the soft recurrence u = v - s (s detached, surrogate ds/dv), states
    pinned to the fp32 trajectory: dI = lam, du0 = beta*lam_0, dbeta = sum lam_t u_{t-1}."""
    T, N, beta = 300, 7, 0.93
    I = normal(T, N, 0.1, 0.5, 6)
    u0 = uniform(N, -0.2, 0.5, 7)
    gS = normal(T, N, 0.0, 1.0, 8)
    U, S = SO.serial_forward(I, beta, 1.0, u0)
    up = np.concatenate([u0[None], U[:-1]], 0)
    V = (np.float32(beta) * up + I).astype(np.float32)
    lam = SO.adjoint_direct64(V, gS, float(np.float32(beta)), 1.0)
    Id = torch.tensor(I, dtype=torch.float64, requires_grad=True)
    u0d = torch.tensor(u0, dtype=torch.float64, requires_grad=True)
    bd = torch.tensor(float(np.float32(beta)), dtype=torch.float64, requires_grad=True)
    Ud = torch.tensor(U, dtype=torch.float64)
    Sd = torch.tensor(S, dtype=torch.float64)
    u, loss = u0d, 0
    for t in range(T):
        if t > 0:
            u = u + (Ud[t - 1] - u).detach()
        v = bd * u + Id[t]
        sg = torch.sigmoid(4.0 * (v - 1.0))
        s = Sd[t] + (sg - sg.detach())
        u = v - Sd[t]
        loss = loss + (torch.tensor(gS[t], dtype=torch.float64) * s).sum()
    gI, g0, gb = torch.autograd.grad(loss, (Id, u0d, bd))
    assert np.linalg.norm(lam - gI.numpy()) / np.linalg.norm(gI.numpy()) < 1e-6
    assert np.allclose(float(np.float32(beta)) * lam[0], g0.numpy(), rtol=1e-6, atol=1e-9)
    assert abs((lam * up).sum() - gb.item()) <= 1e-6 * abs(gb.item())
