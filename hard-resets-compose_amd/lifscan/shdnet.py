"""The spiking classifier the reference trains on SHD (its ``lifscan/shdnet.py``): two hard-reset
LIF layers of H neurons fed by linear maps, and a linear readout of the second layer's spikes.

What a caller of the reference can rely on, kept here (shdnet.py:30-66):
  * ``Net(mode, beta=0.95, H=256, n_out=20)`` with children ``l1``, ``l2`` (``LIFLayer``) and
    ``out`` (``nn.Linear``), so parameter names and state dicts are the reference's;
  * ``LIFLayer(din, dout, beta, mode, K=16, repair=10**6)`` with attributes ``fc``, ``beta``,
    ``mode``, ``K``, ``repair`` (experiments set ``repair`` on a built net);
  * the LIF weight init U(-1.5/sqrt(din), +1.5/sqrt(din)) drawn after nn.Linear's own init, so
    a seeded construction draws the same numbers; the readout's default nn.Linear init;
  * ``forward(x)`` with x time-major [T, B, din] -> (logits [B, n_out], (s1, s2)), logits = 10 x
    the time average of the readout; ``set_mode(mode)``.
Modes: "serial" and "scan" run ``lif_tuned`` (repair as given), "auto" runs ``lif_auto`` without
repair.  The reference's SpikingJelly mode and its SHD/SSC h5 loader are not part of this
package (the benchmark input is a synthetic raster built by the caller).

The readout is applied to the time-averaged spikes, out(mean_t s2), rather than averaging the
readout of every step: the same function (out is affine), one [B, H] x [H, n_out] product
instead of a [T*B, H] one, and no [T, B, n_out] intermediate.
"""
import torch
import torch.nn as nn
import torch.nn.functional as F

from . import hip_lif as L

THETA = 1.0       # firing threshold of every LIF neuron of the network
RESET = 0.0       # hard-reset value
SURROGATE = 4.0   # slope alpha of the sigmoid surrogate gradient
READOUT_GAIN = 10.0
_LAYER_MODES = ("serial", "scan", "auto")


def spike_train(I, beta, mode, K, repair):
    """Spikes [T, N] of LIF neurons that start at rest, driven by the currents I [T, N]."""
    if mode not in _LAYER_MODES:
        raise ValueError(f"mode {mode!r}: one of {_LAYER_MODES}")
    rest = I.new_zeros(I.shape[1])
    if mode == "auto":
        return L.lif_auto(I, rest, beta, THETA, RESET, SURROGATE, K=K, repair=0)
    return L.lif_tuned(I, rest, beta, THETA, RESET, SURROGATE, mode=mode, K=K, repair=repair)


class LIFLayer(nn.Module):
    """x [T, B, din] -> spikes [T, B, dout]: currents fc(x) for all B*dout neurons, one exact
    LIF scan over time (B and dout flattened into the neuron axis)."""

    def __init__(self, din, dout, beta, mode, K=16, repair=10 ** 6):
        super().__init__()
        self.fc = nn.Linear(din, dout)
        bound = 1.5 / din ** 0.5
        with torch.no_grad():
            self.fc.weight.uniform_(-bound, bound)
        self.beta, self.mode, self.K, self.repair = beta, mode, K, repair

    def forward(self, x):
        steps, batch, din = x.shape
        currents = F.linear(x.reshape(steps * batch, din), self.fc.weight, self.fc.bias)
        s = spike_train(currents.view(steps, -1), self.beta, self.mode, self.K, self.repair)
        return s.view(steps, batch, -1)


class Net(nn.Module):
    """din=700 -> H -> H spiking layers, linear readout of the time-averaged second-layer
    spikes (x READOUT_GAIN)."""

    def __init__(self, mode, beta=0.95, H=256, n_out=20):
        super().__init__()
        self.l1 = LIFLayer(700, H, beta, mode)
        self.l2 = LIFLayer(H, H, beta, mode)
        self.out = nn.Linear(H, n_out)

    def set_mode(self, mode):
        for layer in (self.l1, self.l2):
            layer.mode = mode

    def forward(self, x):
        s1 = self.l1(x)
        s2 = self.l2(s1)
        return READOUT_GAIN * self.out(s2.mean(0)), (s1, s2)
