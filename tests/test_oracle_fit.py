"""Pin of the neuron-parameter gradient assembly (oracle lif_oracle.param_grads, restating
fit.py:36-48) against fp64 autograd through the serial recurrence with the detached reset
(fast.py:54-66 serial_lif; the reference's own check is tests/test_fit_grad_cpu.py, bar 1e-9).
The trajectory (reset mask, states) comes from the fp32 run and is held fixed, so the
comparison isolates the gradient formulas."""
import numpy as np
import pytest
import torch

from oracle import lif_oracle as O
from tests._inputs import normal


@pytest.mark.parametrize("beta,theta,u_r", [(0.93, 1.0, -0.1), (0.9, 0.8, 0.2)])
def test_param_grads_match_fp64_autograd(beta, theta, u_r):
    T, N = 600, 8
    x = normal(T, N, 0.0, 1.0, 31)
    I = (0.5 * x + 0.08).astype(np.float32)
    W = normal(T, N, 0.0, 1.0, 32)
    u0 = np.zeros(N, np.float32)
    U, S = O.serial_forward(I, beta, theta, u_r, u0)
    Lam = O.serial_backward(I, u0, U, S, W, None, beta, theta, u_r, 4.0, True, dtype=np.float64)
    got = O.param_grads(I, u0, U, S, W, Lam, beta, theta, u_r, 4.0)
    ps = [torch.tensor(v, dtype=torch.float64, requires_grad=True) for v in (beta, theta, u_r)]
    Id = torch.tensor(I, dtype=torch.float64, requires_grad=True)
    U64, S64 = torch.tensor(U, dtype=torch.float64), torch.tensor(S, dtype=torch.float64)
    u, loss = torch.zeros(N, dtype=torch.float64), 0
    for t in range(T):
        if t > 0:
            u = u + (U64[t - 1] - u).detach()  # fp32 trajectory, gradient paths kept
        v = ps[0] * u + Id[t]
        sig = torch.sigmoid(4.0 * (v - ps[1]))
        s = S64[t] + (sig - sig.detach())  # Heaviside forward, surrogate backward
        u = v * (1 - S64[t]) + ps[2] * S64[t]  # detached reset
        loss = loss + (torch.tensor(W[t], dtype=torch.float64) * s).sum()
    gI, gb, gt, gr = torch.autograd.grad(loss, (Id, *ps))
    assert np.allclose(got[0], gI.numpy(), rtol=1e-9, atol=1e-12)
    for a, b in zip(got[2:], (gb, gt, gr)):
        assert a == pytest.approx(b.item(), rel=1e-9)
