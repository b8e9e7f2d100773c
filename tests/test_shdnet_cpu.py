"""CPU: shdnet's host helpers (dense raster from event lists) and module construction."""
import torch


def test_batch_dense_places_events():
    from lifscan.shdnet import batch_dense
    ev = [torch.tensor([[0, 3], [5, 699], [5, 3]]), torch.tensor([[9, 0]])]
    x = batch_dense(ev, [1, 0], 10, dev="cpu")
    assert x.shape == (10, 2, 700)
    assert x.sum() == 4
    assert x[9, 0, 0] == 1 and x[0, 1, 3] == 1 and x[5, 1, 699] == 1 and x[5, 1, 3] == 1


def test_net_init_matches_reference_shapes():
    from lifscan.shdnet import Net
    torch.manual_seed(0)
    net = Net("scan")
    assert net.l1.fc.weight.shape == (256, 700) and net.l2.fc.weight.shape == (256, 256)
    assert net.out.weight.shape == (20, 256)
    assert net.l1.fc.weight.abs().max() <= 1.5 / 700 ** 0.5
    assert net.l1.repair == 10 ** 6 and net.l1.K == 16
