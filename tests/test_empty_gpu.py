"""GPU: empty inputs (T = 0 or N = 0) through the public LIF, ALIF and fitting entry points.
Each call either returns results of the right (empty) shapes, gradients included, or raises
ValueError (the reference's chunk policy rejects T = 0, triton_lif.py:647-651); no kernel is
launched on an empty grid (every C entry returns before its launches when T or N is 0)."""
import pytest
import torch

pytestmark = pytest.mark.gpu

SHAPES = [(0, 64), (256, 0)]


def _check(fn, *shapes):
    """fn() -> tensor or tuple of tensors with the given shapes, or ValueError."""
    try:
        out = fn()
    except ValueError:
        return
    out = out if isinstance(out, tuple) else (out,)
    for t, shp in zip(out, shapes):
        assert tuple(t.shape) == tuple(shp)


@pytest.mark.parametrize("T,N", SHAPES)
def test_lif_entry_points_on_empty_inputs(dev, T, N):
    from lifscan import triton_lif as TL
    I = torch.zeros(T, N, device=dev)
    u0 = torch.zeros(N, device=dev)
    print(f"empty LIF T={T} N={N}", flush=True)
    _check(lambda: TL.serial_forward_tiled(I, 0.9, 1.0, 0.0, u0), (T, N), (T, N))
    for repair in (0, 10 ** 6):
        _check(lambda: TL.scan_forward_v3(I, 0.9, 1.0, 0.0, u0, C=64, K=8, repair=repair), (T, N), (T, N))
    _check(lambda: TL.scan_forward_v4(I, 0.9, 1.0, 0.0, u0, C=64, G=4, K=8, K2=16, repair=10 ** 6),
           (T, N), (T, N))
    for mode in ("serial", "scan"):
        Ig = I.clone().requires_grad_(True)

        def step():
            S = TL.lif_tuned(Ig, u0, beta=0.9, mode=mode, K=8, repair=10 ** 6)
            S.sum().backward()
            return S, Ig.grad
        _check(step, (T, N), (T, N))


@pytest.mark.parametrize("T,N", SHAPES)
def test_alif_and_fit_entry_points_on_empty_inputs(dev, T, N):
    from lifscan import triton_alif as A
    from lifscan import fit
    I = torch.zeros(T, N, device=dev)
    z = torch.zeros(N, device=dev)
    print(f"empty ALIF / lif_param T={T} N={N}", flush=True)
    for fwd in ("serial", "scan"):
        Ig = I.clone().requires_grad_(True)
        ps = [torch.tensor(v, device=dev, requires_grad=True) for v in (0.95, 0.995, 0.2, 1.0)]

        def step():
            Wp = torch.zeros(T // 128, N, device=dev) if fwd == "scan" else None
            S, U, W = A.alif(Ig, z, z, *ps, fwd=fwd, bwd="scan", Wpred=Wp, dw=0.02, C=128)
            S.sum().backward()
            return S, U, W, Ig.grad
        _check(step, (T, N), (T, N), (T, N), (T, N))
    _check(lambda: A.alif_backward(I, I, I, I, I, 0.95, 0.995, 0.2, 1.0, z, z), (T, N), (T, N))
    Ig = I.clone().requires_grad_(True)
    b = torch.tensor(0.9, device=dev, requires_grad=True)

    def fit_step():
        S = fit.lif_param(Ig, z, b, 1.0, 0.0)
        S.sum().backward()
        return S, Ig.grad
    _check(fit_step, (T, N), (T, N))
