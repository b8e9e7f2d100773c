#!/usr/bin/env python3
"""Benchmark of the exact hard-reset LIF scan on one MI355X (BASELINE.json metric).

Workload ("cfg2"): 65,536 neurons x T = 4,096, fp32, beta = 0.9,
x ~ N(0.12, 0.25^2) (seeded CPU generator, copied to HBM before timing), u0 = 0, theta = 1,
u_r = 0, upstream gradient gS ~ N(0, 1).  One step = lif_tuned(mode="scan", K=8, repair on)
forward + backward (autograd), i.e. the two-level exact scan (chunk C = 128 from the
reference's _pick_C) and the affine-scan adjoint; spikes are bit-identical to the serial
recurrence.  value = neuron-steps/s of that fwd+bwd step.

Printed JSON (one line on stdout) also carries: the forward-only throughput, the in-house
tuned HIP serial baseline (fwd, fwd+bwd), the beta = 0.99 variant, scan stats, the roofline
of the dominant kernel and the CPU baseline (PyTorch-CPU port of the reference's fast.py,
timed on a bounded sample on this host).
"""
import argparse
import json
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(REPO, "hard-resets-compose_amd"), REPO):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0  # MI355X published HBM3E bandwidth
B_FWD, B_BWD = 12, 20  # algorithmic bytes per neuron-step (read I; write U, S | read I, U, S, gS; write dI)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def ev_time(fn, reps, warm=1):
    """Median ms of fn() over reps, HIP events on torch's current stream (the stream every
    library call launches on)."""
    import torch
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        torch.cuda.synchronize()
        ts.append(a.elapsed_time(b))
    return statistics.median(ts)


def cpu_baseline(I_cpu, beta, n_cols):
    """PyTorch-CPU port of fast.py: two-level pruned scan forward (C=64, K=8, repair on) and
    the Hillis-Steele affine-scan backward, plus the serial pair, on the first n_cols neurons
    of the same workload."""
    import torch
    from oracle import fast_port as F
    torch.set_num_threads(os.cpu_count() or 1)
    T = I_cpu.shape[0]
    I = I_cpu[:, :n_cols].contiguous()
    g = torch.Generator().manual_seed(1)
    gs = torch.randn(T, n_cols, generator=g)
    u0 = torch.zeros(n_cols)

    def scan_fb():
        u, s, v = F.scan_forward(I, beta, 1.0, 0.0, u0, C=64, K=8, repair=10 ** 6)
        F.scan_backward(v, s, gs, beta, 1.0)

    def serial_fb():
        u, s, v = F.serial_forward_nograd(I, beta, 1.0, 0.0, u0)
        F.serial_backward(v, s, gs, torch.zeros_like(gs), beta, 1.0, 0.0)

    out = {}
    for name, fn in (("scan", scan_fb), ("serial", serial_fb)):
        fn()  # warm-up
        ts = []
        for _ in range(3):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        out[name] = statistics.median(ts)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-cols", type=int, default=8192)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the exact LIF scan shards along neurons with no "
              "communication, so N GPUs give N x the one-GPU value; run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import torch
    from lifscan import triton_lif as L

    dev = torch.device("cuda:0")
    T, N, beta = 4096, 65536, 0.9
    g = torch.Generator().manual_seed(0)
    I_cpu = (0.12 + 0.25 * torch.randn(T, N, generator=g)).float()
    g1 = torch.Generator().manual_seed(1)
    gS = torch.randn(T, N, generator=g1).float().to(dev)
    I = I_cpu.to(dev)
    u0 = torch.zeros(N, device=dev)
    K = 8

    def step():
        Ig = I.detach().requires_grad_(True)
        S = L.lif_tuned(Ig, u0, beta, 1.0, 0.0, 4.0, mode="scan", K=K, repair=10 ** 6)
        S.backward(gS)
        return Ig.grad

    log(f"warmup {args.warmup}")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log(f"timing {args.steps} steps")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t0) * 1000.0 / args.steps
    value = N * T / (ms_step / 1000.0)
    log(f"fwd+bwd {ms_step:.3f} ms/step  {value / 1e9:.1f} G neuron-steps/s")

    # component timings (HIP events, median)
    C = L._pick_C(T, D=16)
    Cb = min(128, L._pick_C(T, D=2))
    st = {}
    L.scan_forward_v3(I, beta, 1.0, 0.0, u0, C=C, K=K, repair=10 ** 6, stats=st)
    U, S = L.scan_forward_v3(I, beta, 1.0, 0.0, u0, C=C, K=K, repair=10 ** 6)
    t_fwd = ev_time(lambda: L.scan_forward_v3(I, beta, 1.0, 0.0, u0, C=C, K=K, repair=10 ** 6), 10)
    t_bwd = ev_time(lambda: L.scan_backward_tiled(I, u0, U, S, gS, None, beta, 1.0, 0.0, 4.0, C=Cb), 10)
    t_sf = ev_time(lambda: L.serial_forward(I, beta, 1.0, 0.0, u0), 10)
    t_sb = ev_time(lambda: L.serial_backward(I, u0, U, S, gS, None, beta, 1.0, 0.0, 4.0), 10)
    log(f"scan fwd {t_fwd:.3f} ms, scan bwd {t_bwd:.3f} ms, serial fwd {t_sf:.3f}, serial bwd {t_sb:.3f}")
    del U, S

    # beta = 0.99 variant of cfg2
    g2 = torch.Generator().manual_seed(0)
    I99 = (0.012 + 0.08 * torch.randn(T, N, generator=g2)).float().to(dev)
    st99 = {}
    L.scan_forward_v3(I99, 0.99, 1.0, 0.0, u0, C=C, K=K, repair=10 ** 6, stats=st99)
    U99, S99 = L.scan_forward_v3(I99, 0.99, 1.0, 0.0, u0, C=C, K=K, repair=10 ** 6)
    t_fwd99 = ev_time(lambda: L.scan_forward_v3(I99, 0.99, 1.0, 0.0, u0, C=C, K=K, repair=10 ** 6), 10)
    t_bwd99 = ev_time(lambda: L.scan_backward_tiled(I99, u0, U99, S99, gS, None, 0.99, 1.0, 0.0, 4.0, C=Cb), 10)
    del U99, S99, I99

    # dominant cost: the larger of the two passes, priced on its algorithmic bytes
    if t_bwd >= t_fwd:
        dom, dom_ms, dom_b = "scan backward (lsh_lif_scan_bwd)", t_bwd, B_BWD
    else:
        dom, dom_ms, dom_b = "scan forward (lsh_lif_scan_v3_fwd)", t_fwd, B_FWD
    achieved = dom_b * N * T / (dom_ms / 1000.0) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                "kernel": dom, "bytes_per_neuron_step": dom_b}

    cpu = None
    if not args.no_cpu:
        log(f"cpu baseline on {args.cpu_cols} neurons x T={T}")
        r = cpu_baseline(I_cpu, beta, args.cpu_cols)
        ns = args.cpu_cols * T
        cpu = {"value": round(ns / r["scan"], 1), "unit": "neuron-steps/s", "cores": torch.get_num_threads(),
               "kind": "port",
               "sample": f"fast.py two-level pruned scan (C=64,K=8,repair on) + affine-scan bwd, "
                         f"{args.cpu_cols} of {N} neurons x T={T}, median of 3",
               "serial_value": round(ns / r["serial"], 1), "os_cpu_count": os.cpu_count()}

    out = {
        "metric": "neuron-steps/s fwd and fwd+bwd (LIF, 65536xT4096 fp32); % of HBM roofline",
        "value": round(value, 1),
        "unit": "neuron-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded CPU generator, x~N(0.12,0.25^2), gS~N(0,1))",
        "config": {"workload": "cfg2: lif_tuned scan fwd+bwd, N=65536 (256x256), T=4096, beta=0.9, "
                               "theta=1, u_r=0, u0=0, C=128, K=8, repair on",
                   "N": N, "T": T, "beta": beta, "C": C, "K": K},
        "fwd_value": round(N * T / (t_fwd / 1000.0), 1),
        "pct_roofline_fwd_bwd": round(100 * (B_FWD + B_BWD) * N * T / (ms_step / 1000.0) / 1e9 / HBM_PEAK_GBS, 2),
        "pct_roofline_fwd": round(100 * B_FWD * N * T / (t_fwd / 1000.0) / 1e9 / HBM_PEAK_GBS, 2),
        "ms": {"scan_fwd": round(t_fwd, 4), "scan_bwd": round(t_bwd, 4), "serial_fwd": round(t_sf, 4),
               "serial_bwd": round(t_sb, 4), "scan_fwd_beta0.99": round(t_fwd99, 4),
               "scan_bwd_beta0.99": round(t_bwd99, 4)},
        "serial_hip_value": round(N * T / ((t_sf + t_sb) / 1000.0), 1),
        "stats": {"beta0.9": st, "beta0.99": st99},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
