"""Feed-forward hard-reset LIF network of the reference's ``lifscan/shdnet.py`` (LIFLayer, Net)
on the HIP kernels: Linear(din -> H) -> lif_tuned / lif_auto per layer, two layers, linear
readout averaged over time (x10).  Input is time-major [T, B, 700].

SHD/SSC loading needs h5py, imported only by `load` (it is not installed in every environment);
`batch_dense` builds the dense raster on the device from (time bin, unit) event lists.  The
spikingjelly baseline mode of the reference is not provided.
"""
import os

import numpy as np
import torch
import torch.nn as nn

from . import hip_lif as L

DATA = os.environ.get("SHD_DATA", "data/shd")  # directory with {shd,ssc}_{train,test}.h5


def load(split, T, dataset="shd"):
    """(events, labels) of one split (shdnet.py:12-19): events[i] = int64 [n, 2] (time bin in
    [0, T), unit) from a 1 s window."""
    try:
        import h5py
    except ImportError as e:  # pragma: no cover - depends on the environment
        raise ImportError("shdnet.load needs h5py to read the SHD/SSC files") from e
    with h5py.File(f"{DATA}/{dataset}_{split}.h5", "r") as f:
        y = torch.tensor(f["labels"][:].astype(np.int64))
        ev = []
        for tt, uu in zip(f["spikes"]["times"][:], f["spikes"]["units"][:]):
            b = np.minimum((tt * T).astype(np.int64), T - 1)
            ev.append(torch.tensor(np.stack([b, uu.astype(np.int64)], 1)))
    return ev, y


def batch_dense(ev, idx, T, dev="cuda"):
    """Dense 0/1 raster [T, len(idx), 700] of the chosen samples (shdnet.py:22-27)."""
    x = torch.zeros(T, len(idx), 700, device=dev)
    for j, i in enumerate(idx):
        e = ev[i].to(dev, non_blocking=True)
        x[e[:, 0], j, e[:, 1]] = 1.0
    return x


class LIFLayer(nn.Module):
    """Linear(din -> dout) with weights U(+-1.5/sqrt(din)), then the LIF layer over time
    (shdnet.py:30-50).  mode: serial / scan (lif_tuned, repair as given) or auto (lif_auto,
    no repair)."""

    def __init__(self, din, dout, beta, mode, K=16, repair=10 ** 6):
        super().__init__()
        self.fc = nn.Linear(din, dout)
        nn.init.uniform_(self.fc.weight, -1.5 / din ** 0.5, 1.5 / din ** 0.5)
        self.beta, self.mode, self.K, self.repair = beta, mode, K, repair

    def forward(self, x):
        Tn, B, _ = x.shape
        I = self.fc(x).reshape(Tn, -1).contiguous()
        u0 = torch.zeros(I.shape[1], device=I.device)
        if self.mode == "auto":
            s = L.lif_auto(I, u0, beta=self.beta, theta=1.0, u_r=0.0, alpha=4.0, K=self.K, repair=0)
        elif self.mode in ("serial", "scan"):
            s = L.lif_tuned(I, u0, beta=self.beta, theta=1.0, u_r=0.0, alpha=4.0, mode=self.mode,
                            K=self.K, repair=self.repair)
        else:
            raise ValueError(f"mode {self.mode!r}: only serial, scan and auto are provided")
        return s.reshape(Tn, B, -1)


class Net(nn.Module):
    """700 -> H -> H LIF layers and a linear readout; logits = mean over time x 10
    (shdnet.py:53-66)."""

    def __init__(self, mode, beta=0.95, H=256, n_out=20):
        super().__init__()
        self.l1 = LIFLayer(700, H, beta, mode)
        self.l2 = LIFLayer(H, H, beta, mode)
        self.out = nn.Linear(H, n_out)

    def set_mode(self, mode):
        self.l1.mode = self.l2.mode = mode

    def forward(self, x):
        s1 = self.l1(x)
        s2 = self.l2(s1)
        return self.out(s2).mean(0) * 10, (s1, s2)
