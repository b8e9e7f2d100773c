"""GPU: the C++ autograd function of lif_tuned's recomputing pair (lifscan/_ops.cpp) returns the
same bits as the Python autograd function over the same kernels (LIFTuned): S, dL/dI, dL/du0, at
cfg3's per-layer shape (N = 64 x 256, T = 1024) and a small one, through lif_tuned, and is the
path lif_tuned takes there."""
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T,N", [(1024, 16384), (256, 20000)])
def test_cpp_recomputing_pair_equals_python_layer(dev, T, N):
    from lifscan import _native as n
    from lifscan import hip_lif as L
    assert n.ops() is not None, "lifscan_ops.so is not built"
    g = torch.Generator().manual_seed(5)
    I = (0.12 + 0.25 * torch.randn(T, N, generator=g)).to(dev)
    gS = torch.randn(T, N, generator=g).to(dev)
    u0 = (0.3 * torch.rand(N, generator=g)).to(dev)
    print(f"c++ lif_tuned T={T} N={N}", flush=True)
    assert L._rc_path(I, u0, 0.95, "scan", 16, 10 ** 6) is not None
    outs = []
    for use_cpp in (True, False):
        Ig = I.clone().requires_grad_(True)
        ug = u0.clone().requires_grad_(True)
        if use_cpp:
            S = L.lif_tuned(Ig, ug, 0.95, 1.0, 0.0, 4.0, mode="scan", K=16, repair=10 ** 6)
        else:
            S = L.LIFTuned.apply(Ig, ug, 0.95, 1.0, 0.0, 4.0, "scan", 16, 10 ** 6)
        S.backward(gS)
        outs.append((S.detach(), Ig.grad, ug.grad))
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    assert L.starts_forward_timeouts(dev) == 0
