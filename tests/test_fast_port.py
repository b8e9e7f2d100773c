"""Pins of oracle/fast_port.py (the PyTorch-CPU restatement of fast.py timed as bench.py's
cpu_baseline), restating the reference's tests/test_fast.py checks at smaller sizes:
  * the two-level scan (unpruned and pruned capacity K) with repair is bit-identical to the
    serial recurrence, fp32 and fp64, over beta in {0.5, 0.9, 0.99, 1.0} and two resets;
  * the serial recurrence equals the numpy fp32 oracle (two roundings);
  * the Hillis-Steele reverse affine scan equals the serial adjoint (fp64, 1e-10), and the
    serial adjoint equals the fp64 oracle adjoint;
  * state_bounds brackets the trajectory."""
import numpy as np
import pytest
import torch

from oracle import fast_port as F
from oracle import lif_oracle as O


def gen(T, N, dt, seed, mu=0.15, sd=0.4):
    g = torch.Generator().manual_seed(seed)
    return (mu + sd * torch.randn(T, N, generator=g)).to(dt)


@pytest.mark.parametrize("dt", [torch.float64, torch.float32])
@pytest.mark.parametrize("beta", [0.5, 0.9, 0.99, 1.0])
@pytest.mark.parametrize("u_r", [0.0, -0.2])
def test_scan_with_repair_is_bit_identical(dt, beta, u_r):
    I = gen(512, 32, dt, 0)
    u0 = torch.zeros(32, dtype=dt)
    us, ss, vs = F.serial_forward_nograd(I, beta, 1.0, u_r, u0)
    for C, K in ((8, None), (64, None), (64, 2), (64, 16)):
        st = {}
        u, s, v = F.scan_forward(I, beta, 1.0, u_r, u0, C=C, K=K, repair=10 ** 6, stats=st)
        assert torch.equal(u, us) and torch.equal(s, ss), (C, K)
        assert st["repair_iters"] <= 512 // C


def test_serial_matches_numpy_oracle():
    I = gen(300, 50, torch.float32, 1, 0.1, 0.3)
    u0 = (0.3 * torch.randn(50, generator=torch.Generator().manual_seed(2))).float()
    us, ss, _ = F.serial_forward_nograd(I, 0.9, 1.0, -0.1, u0)
    Uo, So = O.serial_forward(I.numpy(), 0.9, 1.0, -0.1, u0.numpy())
    assert np.array_equal(us.numpy(), Uo) and np.array_equal(ss.numpy(), So)


@pytest.mark.parametrize("detach", [True, False])
def test_adjoints(detach):
    T, N, beta = 256, 12, 0.9
    I = gen(T, N, torch.float64, 3)
    u0 = torch.zeros(N, dtype=torch.float64)
    us, ss, vs = F.serial_forward_nograd(I, beta, 1.0, 0.0, u0)
    gs = torch.randn(T, N, generator=torch.Generator().manual_seed(4), dtype=torch.float64)
    lam = F.serial_backward(vs, ss, gs, torch.zeros_like(gs), beta, 1.0, 0.0, 4.0, detach)
    Uprev = torch.cat([u0[None], us[:-1]], 0)
    Lo = O.serial_backward(I.numpy(), u0.numpy(), us.numpy(), ss.numpy(), gs.numpy(), None, beta, 1.0, 0.0,
                           4.0, detach, dtype=np.float64)
    assert np.allclose(lam.numpy(), Lo, rtol=1e-10, atol=1e-13)
    if detach:
        lam2 = F.scan_backward(vs, ss, gs, beta, 1.0)
        assert float((lam2 - lam).norm() / lam.norm()) < 1e-10
    assert torch.equal(Uprev[0], u0)


def test_state_bounds_bracket_the_trajectory():
    for beta, mu, sd in ((0.9, 0.15, 0.4), (0.99, -0.1, 0.6), (1.0, 0.0, 0.3)):
        I = gen(400, 20, torch.float64, 5, mu, sd)
        u0 = (0.3 * torch.randn(20, generator=torch.Generator().manual_seed(6))).double()
        us, _, _ = F.serial_forward_nograd(I, beta, 1.0, -0.1, u0)
        lo, hi = F.state_bounds(I, beta, 1.0, -0.1, u0)
        assert bool((us >= lo).all()) and bool((us <= hi).all())


@pytest.mark.parametrize("detach", [True, False])
def test_scan_lif_gradients_equal_serial_autograd(detach):
    """ScanLIF (two-level scan + Hillis-Steele adjoint) against autograd through the serial loop
    (serial_lif, SpikeFn), fp64, with upstream gradients on both outputs u and s and both reset
    variants (the reference's tests/test_fast.py bar, 1e-10)."""
    T, N, beta = 256, 24, 0.9
    I = gen(T, N, torch.float64, 7)
    u0 = (0.2 * torch.randn(N, generator=torch.Generator().manual_seed(8))).double()
    gu = torch.randn(T, N, generator=torch.Generator().manual_seed(9), dtype=torch.float64)
    gs = torch.randn(T, N, generator=torch.Generator().manual_seed(10), dtype=torch.float64)
    grads = []
    for fn in (F.serial_lif, F.scan_lif):
        Ig = I.clone().requires_grad_(True)
        ug = u0.clone().requires_grad_(True)
        kw = dict(detach_reset=detach)
        if fn is F.scan_lif:
            kw.update(C=32, repair=10 ** 6)
        u, s = fn(Ig, beta, 1.0, -0.1, ug, 4.0, **kw)
        ((u * gu).sum() + (s * gs).sum()).backward()
        grads.append((u.detach(), s.detach(), Ig.grad, ug.grad))
    (u1, s1, gI1, g01), (u2, s2, gI2, g02) = grads
    assert torch.equal(u1, u2) and torch.equal(s1, s2)
    assert float((gI2 - gI1).norm() / gI1.norm()) < 1e-10
    assert float((g02 - g01).norm() / g01.norm()) < 1e-10


def test_cfg1_cpu_path():
    """BASELINE cfg1: fast.py's two-level scan at N = 4096 (16 x 256), T = 1024, beta = 0.9,
    x ~ N(0.12, 0.25^2), u0 = 0, fp32.  Forward spikes and membrane equal the serial fp32
    recurrence bit for bit (repair on); the adjoint equals the serial autograd gradient
    (serial_lif) to 1e-5 and the fp64 adjoint of the oracle to 1e-4."""
    T, N, beta = 1024, 4096, 0.9
    I = gen(T, N, torch.float32, 11, 0.12, 0.25)
    u0 = torch.zeros(N)
    gs = torch.randn(T, N, generator=torch.Generator().manual_seed(12))
    us, ss, _ = F.serial_forward_nograd(I, beta, 1.0, 0.0, u0)
    Ig = I.clone().requires_grad_(True)
    u, s = F.scan_lif(Ig, beta, 1.0, 0.0, u0, 4.0, C=64, repair=10 ** 6)
    assert torch.equal(u.detach(), us) and torch.equal(s.detach(), ss)
    (s * gs).sum().backward()
    Ir = I.clone().requires_grad_(True)
    _, sr = F.serial_lif(Ir, beta, 1.0, 0.0, u0, 4.0)
    (sr * gs).sum().backward()
    assert float((Ig.grad - Ir.grad).norm() / Ir.grad.norm()) < 1e-5
    Lam = O.serial_backward(I.numpy(), u0.numpy(), us.numpy(), ss.numpy(), gs.numpy(), None, beta,
                            1.0, 0.0, 4.0, dtype=np.float64)
    assert np.linalg.norm(Ig.grad.numpy() - Lam) / np.linalg.norm(Lam) < 1e-4
