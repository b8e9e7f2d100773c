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
