"""The two-level map scan captured in a HIP graph (through torch.cuda.CUDAGraph) and replayed:
its launches take torch's current stream, clear the workspace header with a kernel (no memset
node) and read nothing back when no statistics are asked for, so a captured call can be
replayed.  Every replay, with eager calls and synchronizations between them, gives the eager
result bit for bit: with few neurons (one-wave-per-neuron carry) and with many (staged carry).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("N", [128, 4096])
def test_map_scan_graph_replays(dev, N):
    from lifscan import hip_lif as L
    T, C, K, beta = 16384, 128, 16, 0.99
    g = torch.Generator().manual_seed(63)
    I = (0.15 + 0.4 * torch.randn(T, N, generator=g)).to(dev)
    u0 = torch.zeros(N, device=dev)
    print(f"map scan graph replays N={N}", flush=True)
    U0, S0 = L.scan_forward_mapscan(I, beta, 1.0, 0.0, u0, C=C, K=K, repair=0)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        L.scan_forward_mapscan(I, beta, 1.0, 0.0, u0, C=C, K=K, repair=0)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        U, S = L.scan_forward_mapscan(I, beta, 1.0, 0.0, u0, C=C, K=K, repair=0)
    for _ in range(3):
        U.fill_(-1.0)
        S.fill_(-1.0)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(U, U0) and torch.equal(S, S0)
        U1, S1 = L.scan_forward_mapscan(I, beta, 1.0, 0.0, u0, C=C, K=K, repair=0)
        torch.cuda.synchronize()
        assert torch.equal(U1, U0) and torch.equal(S1, S0)
