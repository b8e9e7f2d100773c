"""The reference's near-threshold stress regime (experiments/e2b_stress.py:9-27) on the CPU.

The reference records, per (beta, eps), the spike flips of the fp32 serial recurrence against
the fp64 one and of fast.py's pruned scan (C 64, K 64) against the fp32 serial recurrence
(results/e2b_stress.json, kept as tests/golden/e2b_stress.json).  Reproducing the first
number exactly pins the input construction (tests._inputs.near_threshold) and the fp32 and
fp64 serial arithmetic; the second pins oracle/fast_port.scan_forward on these inputs.  The
GPU paths are held to the same inputs in test_stress_gpu.py.
"""
import json
import os

import numpy as np
import pytest
import torch

from oracle import fast_port as F
from oracle import lif_oracle as O
from tests._inputs import near_threshold

T, N = 4096, 512
GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "e2b_stress.json")))["rows"]


@pytest.mark.parametrize("row", GOLDEN, ids=lambda r: f"b{r['beta']}-e{r['eps']}")
def test_stress_inputs_and_fast_port_match_reference_record(row):
    beta, eps = row["beta"], row["eps"]
    I64, I32 = near_threshold(T, N, beta, eps)
    u0 = np.zeros(N, np.float32)
    U32, S32 = O.serial_forward(I32, beta, 1.0, 0.0, u0)
    _, s64, _ = F.serial_forward_nograd(I64, beta, 1.0, 0.0, torch.zeros(N, dtype=torch.float64))
    flips64 = float((S32 != s64.numpy().astype(np.float32)).mean())
    print(f"beta={beta} eps={eps}: ser32 vs ser64 flips {flips64} (reference {row['flip_ser32_vs_ser64']})")
    assert flips64 == row["flip_ser32_vs_ser64"]
    # the fast.py port's serial recurrence is the oracle's, bit for bit
    u_t, s_t, _ = F.serial_forward_nograd(torch.from_numpy(I32), beta, 1.0, 0.0, torch.zeros(N))
    assert np.array_equal(u_t.numpy(), U32) and np.array_equal(s_t.numpy(), S32)
    I = torch.from_numpy(I32)
    st = {}
    _, sc, _ = F.scan_forward(I, beta, 1.0, 0.0, torch.zeros(N), C=64, K=64, stats=st)
    diff = sc.numpy() != S32
    assert float(diff.mean()) == row["flip_scan32_vs_ser32"]
    assert float(diff.any(0).mean()) == row["neurons_diverged"]
    st2 = {}
    u2, s2, _ = F.scan_forward(I, beta, 1.0, 0.0, torch.zeros(N), C=64, K=64, repair=10 ** 6, stats=st2)
    assert st2["repair_iters"] == row["repair_iters"]
    assert np.array_equal(s2.numpy(), S32) == row["bitexact_after_repair"]
    assert np.array_equal(u2.numpy(), U32)
