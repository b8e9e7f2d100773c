"""Seeded inputs shared by the tests (CPU torch.Generator, so CPU and GPU see the same data)."""
import numpy as np
import torch


def normal(T, N, mu, sd, seed):
    g = torch.Generator().manual_seed(seed)
    return (mu + sd * torch.randn(T, N, generator=g)).to(torch.float32).numpy()


def uniform(N, lo, hi, seed):
    g = torch.Generator().manual_seed(seed)
    return (lo + (hi - lo) * torch.rand(N, generator=g)).to(torch.float32).numpy()


def gpu(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def host(t):
    return t.detach().cpu().numpy()


def near_threshold(T, N, beta, eps, seed=0, theta=1.0):
    """The reference's near-threshold stress inputs (experiments/e2b_stress.py:12-19), fp64 on
    the CPU generator: I ~ 0.15 + 0.4 N(0, 1); at a random 30% of (t, n) the input is chosen so
    that the fp64 serial pre-reset potential lands uniformly within +-eps of theta.  Returns
    (I64 [T, N] float64 tensor, I32 numpy float32 = I64 rounded once)."""
    g = torch.Generator().manual_seed(seed)
    I = 0.15 + 0.4 * torch.randn(T, N, dtype=torch.float64, generator=g)
    hit = torch.rand(T, N, generator=g) < 0.3
    u = torch.zeros(N, dtype=torch.float64)
    for t in range(T):
        tgt = theta + eps * (2 * torch.rand(N, dtype=torch.float64, generator=g) - 1)
        I[t] = torch.where(hit[t], tgt - beta * u, I[t])
        v = beta * u + I[t]
        u = torch.where(v >= theta, torch.zeros_like(v), v)
    return I, I.float().numpy()
