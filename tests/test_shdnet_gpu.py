"""GPU: the SHD network (shdnet.py:30-66) on the HIP layers.  Scan (exact, repair on) and serial
modes give identical spikes and logits; parameter gradients agree (1e-5); each LIF layer's
spikes equal the oracle's serial recurrence on that layer's input current, and its input
gradient the oracle's adjoint of the upstream spike gradient (1e-4 of fp64)."""
import numpy as np
import pytest
import torch

from oracle import lif_oracle as O
from tests._inputs import host

pytestmark = pytest.mark.gpu


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _raster(T, B, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.rand(T, B, 700, generator=g) < 0.015).float()


@pytest.mark.parametrize("T,B", [(256, 8), (1024, 64)])  # (1024, 64): BASELINE cfg3
def test_net_scan_equals_serial_and_oracle(dev, T, B):
    """experiments/e7c_timing.py's step (cross-entropy on the logits, backward) in scan and
    serial mode, on a Bernoulli(0.015) raster."""
    from lifscan.shdnet import Net
    x = _raster(T, B, 3).to(dev)
    y = torch.randint(0, 20, (B,), generator=torch.Generator().manual_seed(5)).to(dev)
    nets, out = {}, {}
    for mode in ("scan", "serial"):
        torch.manual_seed(4)
        net = Net(mode).to(dev)
        logits, (s1, s2) = net(x)
        s1.retain_grad()
        s2.retain_grad()
        loss = torch.nn.functional.cross_entropy(logits, y)
        loss.backward()
        nets[mode] = net
        out[mode] = (logits.detach(), s1, s2)
        print(f"shdnet T={T} B={B} {mode} loss {loss.item():.6f}", flush=True)
    assert torch.equal(out["scan"][0], out["serial"][0])
    assert torch.equal(out["scan"][1], out["serial"][1]) and torch.equal(out["scan"][2], out["serial"][2])
    for (n1, p1), (n2, p2) in zip(nets["scan"].named_parameters(), nets["serial"].named_parameters()):
        assert rel(host(p1.grad), host(p2.grad)) < 1e-5, n1
    # layer 1 against the oracle: current = fc(x), spikes and dL/dI
    net = nets["scan"]
    with torch.no_grad():  # the layer's own current computation (one GEMM over T*B rows)
        I1 = torch.nn.functional.linear(x.reshape(T * B, -1), net.l1.fc.weight,
                                        net.l1.fc.bias).reshape(T, -1).contiguous()
    I1h = host(I1)
    N1 = I1h.shape[1]
    u0 = np.zeros(N1, np.float32)
    U1, S1 = O.serial_forward(I1h, 0.95, 1.0, 0.0, u0)
    assert np.array_equal(host(out["scan"][1]).reshape(T, -1), S1)
    g1 = host(out["scan"][1].grad).reshape(T, -1)
    Lam = O.serial_backward(I1h, u0, U1, S1, g1, None, 0.95, 1.0, 0.0, 4.0, True, dtype=np.float64)
    Ig = I1.detach().requires_grad_(True)
    from lifscan import hip_lif as L
    S = L.lif_tuned(Ig, torch.zeros(N1, device=dev), beta=0.95, mode="scan", K=16, repair=10 ** 6)
    S.backward(out["scan"][1].grad.reshape(T, -1))
    assert rel(host(Ig.grad), Lam) < 1e-4


def test_net_auto_mode_runs(dev):
    from lifscan.shdnet import Net
    T, B = 128, 4
    x = _raster(T, B, 6).to(dev)
    torch.manual_seed(4)
    net = Net("auto").to(dev)
    logits, _ = net(x)
    logits.sum().backward()
    assert logits.shape == (B, 20) and torch.isfinite(net.l1.fc.weight.grad).all()
