"""GPU: the look-back adjoint's entry point that allocates nothing
(lsh_lif_scan_lookback_bwd_noalloc, its workspace a static device array) against the entry point
that takes a caller-allocated workspace (lsh_lif_scan_lookback_bwd), through the C ABI: the same
Lam bit for bit on two calls in a row, the second with a smaller input (the array keeps the first
call's contents), and the fp32 oracle to 1e-5; sizes beyond the array are rejected before any
launch."""
import numpy as np
import pytest
import torch

from oracle import lif_oracle as O
from tests._inputs import gpu, host, normal, uniform

pytestmark = pytest.mark.gpu


def _call(name, args, T, N, beta, detach, C, ws=None):
    from lifscan import _native as nat
    lib = nat.lib()
    I, u0, U, S, GS, GU = args
    Lam = torch.empty_like(I)
    p = [nat.ptr(t) for t in (I, u0, U, S, GS, GU, Lam)]
    st = nat.stream_of(I)
    if name == "noalloc":
        rc = lib.lsh_lif_scan_lookback_bwd_noalloc(*p, T, N, beta, 1.0, -0.1, 4.0, int(detach), C, st)
    else:
        nbytes = lib.lsh_lif_scan_lookback_bwd_workspace(T, N)
        ws = nat.workspace(nbytes, I.device)
        rc = lib.lsh_lif_scan_lookback_bwd(*p, T, N, beta, 1.0, -0.1, 4.0, int(detach), C, nat.ptr(ws),
                                           nbytes, st)
    nat.check(rc, name)
    torch.cuda.synchronize()
    return Lam


def _case(T, N, seed, with_gu, dev):
    I = normal(T, N, 0.06, 0.2, seed)
    u0 = uniform(N, -0.2, 0.5, seed + 1)
    GS = normal(T, N, 0.0, 1.0, seed + 2)
    GU = normal(T, N, 0.0, 1.0, seed + 3) if with_gu else None
    U, S = O.serial_forward(I, 0.95, 1.0, -0.1, u0)
    host_args = (I, u0, U, S, GS, GU)
    return host_args, [gpu(a, dev) if a is not None else None for a in host_args]


@pytest.mark.parametrize("detach,with_gu,C", [(True, False, 16), (False, True, 32)])
def test_noalloc_lookback_equals_workspace_entry(dev, detach, with_gu, C):
    for T, N, seed in ((16384, 1000, 71), (4096, 130, 81)):  # second call smaller
        print(f"noalloc lookback T={T} N={N} detach={detach} gu={with_gu} C={C}", flush=True)
        h, args = _case(T, N, seed, with_gu, dev)
        got = _call("noalloc", args, T, N, 0.95, detach, C)
        ref = _call("workspace", args, T, N, 0.95, detach, C)
        assert torch.equal(got, ref), (T, N)
        Lo = O.serial_backward(*h[:5], h[5], 0.95, 1.0, -0.1, 4.0, detach)
        err = np.linalg.norm(host(got).astype(np.float64) - Lo) / np.linalg.norm(Lo)
        assert err < 1e-5, (T, N, err)


def test_noalloc_rejects_sizes_beyond_the_array(dev):
    """T * N above what LSH_NOALLOC_SCRATCH_BYTES holds: ValueError (LSH_ERR_SCRATCH) from the
    host-side check, before anything is launched (the small buffers passed are never read)."""
    from lifscan import _native as nat
    lib = nat.lib()
    T, N = 1 << 22, 1 << 16
    assert lib.lsh_lif_scan_lookback_bwd_workspace(T, N) > (64 << 20)
    x = torch.zeros(256, device=dev)
    p = [nat.ptr(x)] * 7
    rc = lib.lsh_lif_scan_lookback_bwd_noalloc(*p[:5], None, p[6], T, N, 0.95, 1.0, 0.0, 4.0, 1, 16,
                                               nat.stream_of(x))
    assert rc == nat.LSH_ERR_SCRATCH
    with pytest.raises(ValueError):
        nat.check(rc, "lsh_lif_scan_lookback_bwd_noalloc")
    torch.cuda.synchronize()


def test_noalloc_near_the_limit(dev):
    """A problem that needs 48 MiB of the 64 MiB array (N = 1024, T = 2^20, cfg4's shape), then a
    small one: both equal the workspace entry point bit for bit."""
    from lifscan import hip_lif as L
    for T, N in ((1 << 20, 1024), (2048, 70)):
        print(f"noalloc lookback near limit T={T} N={N}", flush=True)
        g = torch.Generator(device=dev).manual_seed(T + N)
        I = torch.randn(T, N, device=dev, generator=g).mul_(0.08).add_(0.012)
        GS = torch.randn(T, N, device=dev, generator=g)
        u0 = torch.rand(N, device=dev, generator=g)
        U, S = L.serial_forward(I, 0.99, 1.0, -0.1, u0)
        args = [I, u0, U, S, GS, None]
        got = _call("noalloc", args, T, N, 0.99, True, 16)
        ref = _call("workspace", args, T, N, 0.99, True, 16)
        assert torch.equal(got, ref), (T, N)
        del I, GS, U, S, got, ref, args
        torch.cuda.empty_cache()


def test_noalloc_lookback_graph_replays(dev):
    """The entry point that allocates nothing, captured in a HIP graph (torch.cuda.CUDAGraph) and
    replayed three times with eager calls and synchronizations between the replays: every replay
    gives the workspace entry point's Lam bit for bit.  The capture holds only kernel nodes: the
    flags and the header of the static array are cleared by a kernel at every call, and the
    array's address was taken by an eager call before the capture."""
    from lifscan import _native as nat
    lib = nat.lib()
    T, N, C, beta = 8192, 300, 16, 0.95
    h, args = _case(T, N, 91, False, dev)
    ref = _call("workspace", args, T, N, beta, True, C)
    I, u0, U, S, GS, GU = args
    Lam = torch.empty_like(I)
    p = [nat.ptr(t) for t in (I, u0, U, S, GS, GU, Lam)]
    print(f"noalloc lookback graph capture T={T} N={N}", flush=True)

    def launch():
        nat.check(lib.lsh_lif_scan_lookback_bwd_noalloc(*p, T, N, beta, 1.0, -0.1, 4.0, 1, C,
                                                        nat.stream_of(I)), "noalloc")

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        launch()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert torch.equal(Lam, ref)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch()
    for r in range(3):
        Lam.fill_(-1.0)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(Lam, ref), r
        eager = _call("noalloc", args, T, N, beta, True, C)
        assert torch.equal(eager, ref), r
