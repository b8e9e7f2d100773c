"""CPU: the SHD network's construction (parameter names, shapes and init bounds of the reference's
shdnet.py:30-66), mode handling and the readout (no GPU needed)."""
import pytest
import torch


def test_net_parameters_match_reference_names_and_init():
    from lifscan.shdnet import Net
    torch.manual_seed(0)
    net = Net("scan")
    names = {k: tuple(v.shape) for k, v in net.state_dict().items()}
    assert names == {"l1.fc.weight": (256, 700), "l1.fc.bias": (256,),
                     "l2.fc.weight": (256, 256), "l2.fc.bias": (256,),
                     "out.weight": (20, 256), "out.bias": (20,)}
    assert net.l1.fc.weight.abs().max() <= 1.5 / 700 ** 0.5
    assert net.l2.fc.weight.abs().max() <= 1.5 / 256 ** 0.5
    assert net.l1.fc.weight.abs().max() > 0.9 * 1.5 / 700 ** 0.5   # spread over the whole range
    assert net.l1.repair == 10 ** 6 and net.l1.K == 16 and net.l1.beta == 0.95
    net.set_mode("serial")
    assert net.l1.mode == net.l2.mode == "serial"


def test_seeded_construction_draws_the_same_weights():
    """nn.Linear's own init first, then the U(+-1.5/sqrt(din)) weight draw: a seeded build is
    reproducible and independent of the mode."""
    from lifscan.shdnet import Net
    torch.manual_seed(4)
    a = Net("scan").state_dict()
    torch.manual_seed(4)
    b = Net("serial").state_dict()
    assert all(torch.equal(a[k], b[k]) for k in a)


def test_readout_is_the_time_average_of_the_linear_readout():
    """out(mean_t s) equals mean_t out(s) (out is affine), the reference's readout."""
    from lifscan.shdnet import Net, READOUT_GAIN
    torch.manual_seed(1)
    net = Net("scan", H=32, n_out=5)
    s2 = (torch.rand(50, 3, 32) < 0.2).float()
    ref = net.out(s2).mean(0) * 10
    got = READOUT_GAIN * net.out(s2.mean(0))
    assert torch.allclose(got, ref, rtol=1e-5, atol=1e-6)


def test_unknown_mode_is_rejected():
    from lifscan.shdnet import spike_train
    with pytest.raises(ValueError):
        spike_train(torch.zeros(4, 3), 0.9, "sj", 16, 0)
