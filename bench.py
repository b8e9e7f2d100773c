#!/usr/bin/env python3
"""Benchmark of the exact hard-reset LIF scan on one MI355X (BASELINE.json metric).

Workload ("cfg2"): 65,536 neurons x T = 4,096, fp32, beta = 0.9,
x ~ N(0.12, 0.25^2) (seeded CPU generator, copied to HBM before timing), u0 = 0, theta = 1,
u_r = 0, upstream gradient gS ~ N(0, 1).  One step = lif_tuned(mode="scan", K=8, repair on)
forward + backward through autograd.  What runs: the exact single-pass forward with 32-step
chunks handed on from wave to wave (no chunk maps: K is unused) and the single-pass affine-scan
adjoint.  lif_tuned keeps U only for its backward, so its forward stores S and the exact state
at every 32-step chunk entry, and the adjoint replays each chunk's forward from that state in
registers (same S, same gradients): 20 bytes of HBM traffic per neuron-step instead of 32.
value = neuron-steps/s of that fwd+bwd step, whose S and dI are checked once (outside the timed
region) against the serial forward and the stored-U adjoint; the passes that store U are timed
beside it ("stored_U_path").

The JSON line also carries the forward-only rate, the in-house HIP serial baseline, the map
scan of configs[1] as stated (C = 32/64/128, K = 8, repair on, beta = 0.9 and 0.99:
"cfg2_mapscan"), the roofline of the dominant kernel (HIP events on the stream it runs on) and
the CPU baseline (PyTorch-CPU port of the reference's fast.py on a bounded sample, timed on
this host).

The other BASELINE configurations (cfg3 network step, cfg4 long sequence, cfg5 ALIF) are
measured after the headline and reported under "other_configs" (--headline-only skips them).

  python bench.py [--steps K] [--warmup W] [--no-cpu] [--headline-only]
  python bench.py --only cfg4        # one other configuration (profiling runs; also
                                     # cfg2_mapscan, cfg3, cfg5, affine)
  python bench.py --dominant-only    # short run for rocprofv3 --pmc passes (copy + kernel)
  python bench.py --counters-workload  # the non-HBM-bound kernels once each (counter passes)
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
# algorithmic bytes per neuron-step of the passes that store U (scan_forward_v3 returns it):
# read I; write U, S | read I, U_{t-1}, S, gS; write dI
B_FWD, B_BWD = 12, 20
# lif_tuned keeps U only for its backward; its recomputing pair stores the chunk entry states
# instead: read I; write S | read I, gS; write dI (the states are 1/32 of a row per step)
B_FWD_RC, B_BWD_RC = 8, 12
T_CFG, N_CFG = 4096, 65536


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def ev_time(fn, reps, warm=1, warm_s=0.0):
    """Median ms of fn() over reps with HIP events on torch's current stream, the stream
    every library call launches on.  warm_s: also keep calling fn untimed for that many
    seconds first (the GPU's clocks ramp up over a fraction of a second after idle)."""
    import torch
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    t_end = time.perf_counter() + warm_s
    while time.perf_counter() < t_end:
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


def bb_time(fn, reps, groups=5, warm=2, warm_s=0.0):
    """Throughput ms per call: fn() called reps times back to back between two HIP events
    (as the headline's step loop runs), the median over groups.  Unlike ev_time, the host's
    work before each launch overlaps the previous call's kernels."""
    import torch
    for _ in range(warm):
        fn()
    t_end = time.perf_counter() + warm_s
    while time.perf_counter() < t_end:
        fn()
    ts = []
    for _ in range(groups):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        torch.cuda.synchronize()
        ts.append(a.elapsed_time(b) / reps)
    return statistics.median(ts)


_SCRUB = []


def scrub():
    """Read and write 1 GiB (four times MI355X's 256 MB Infinity Cache), so that the next call
    finds none of its operands in that cache: its reads come from HBM."""
    import torch
    if not _SCRUB:
        _SCRUB.append(torch.zeros(256 * 2 ** 20, device="cuda"))
    _SCRUB[0].add_(1.0)


def ev_time_cold(fn, reps, warm=1):
    """Median ms of fn() over reps with HIP events, each call after scrub() (outside the events):
    the cache-cold time, as a call on operands last touched long ago would see."""
    import torch
    for _ in range(warm):
        fn()
    ts = []
    for _ in range(reps):
        scrub()
        torch.cuda.synchronize()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        torch.cuda.synchronize()
        ts.append(a.elapsed_time(b))
    return statistics.median(ts)


def hbm_ceilings(torch, dev):
    """This box's own HBM ceilings on 1 GiB arrays (cache-cold, HIP events, median of 5): a copy
    (read 1 GiB, write 1 GiB) and a fill (write 1 GiB), in GB/s.  No kernel of this build is
    credited above them."""
    x = torch.empty(256 * 2 ** 20, device=dev)
    y = torch.empty_like(x)
    nb = 4 * x.numel()
    t_copy = ev_time_cold(lambda: y.copy_(x), 5)
    t_fill = ev_time_cold(lambda: y.fill_(1.0), 5)
    del x, y
    torch.cuda.empty_cache()
    return {"copy_GBps": round(2 * nb / (t_copy / 1000.0) / 1e9, 1),
            "fill_GBps": round(nb / (t_fill / 1000.0) / 1e9, 1), "bytes": nb}


def bench_auto_grid(torch, dev, reps=15):
    """The reference's lif_auto grid (experiments/e11_auto.py:16-41; results/e11_auto.json): one
    LIF layer's forward + backward through autograd with library defaults at N in {128, 1024,
    8192, 32768, 131072} x T in {1024, 4096, 16384, 65536}, N*T <= 2^28, x ~ N(0.15, 0.4^2),
    beta 0.9, u0 = 0, G ~ N(0, 1): lif_tuned(mode="serial"), lif_tuned(mode="scan", repair=0)
    and lif_auto.  Each time is ms per call of calls run back to back between two HIP events (as
    a training loop runs them; at the smallest cells a call is ~10 us of GPU work and one call
    between two synchronizations measures the host's latency instead), groups of the three modes
    interleaved so that clock drift favours none, median of 7 groups.  Per cell: the three times,
    auto's modes, whether the spikes of all three are equal and auto's gradient against serial's;
    auto_vs_best = auto's time over the faster of the two modes."""
    from lifscan import hip_lif as L
    rows = []
    for N in (128, 1024, 8192, 32768, 131072):
        for T in (1024, 4096, 16384, 65536):
            if N * T > 2 ** 28:
                continue
            g = torch.Generator().manual_seed(0)
            I0 = (0.15 + 0.4 * torch.randn(T, N, generator=g)).to(dev)
            G = torch.randn(T, N, generator=torch.Generator().manual_seed(1)).to(dev)
            u0 = torch.zeros(N, device=dev)
            fns = {"serial": lambda I: L.lif_tuned(I, u0, beta=0.9, mode="serial"),
                   "scan": lambda I: L.lif_tuned(I, u0, beta=0.9, mode="scan", repair=0),
                   "auto": lambda I: L.lif_auto(I, u0, beta=0.9)}
            res = {}
            steps = {}
            for name, f in fns.items():
                I = I0.clone().requires_grad_(True)

                def step(f=f, I=I):
                    I.grad = None
                    f(I).backward(G)
                for _ in range(3):
                    step()
                steps[name] = step
                I.grad = None
                s = f(I)
                s.backward(G)
                res[name] = [None, s.detach(), I.grad.clone()]
            times = {name: [] for name in fns}
            calls = 20 if N * T <= 2 ** 24 else 5
            for _ in range(7):
                for name, step in steps.items():
                    torch.cuda.synchronize()
                    a = torch.cuda.Event(enable_timing=True)
                    b = torch.cuda.Event(enable_timing=True)
                    a.record()
                    for _ in range(calls):
                        step()
                    b.record()
                    torch.cuda.synchronize()
                    times[name].append(a.elapsed_time(b) / calls)
            for name in fns:
                res[name][0] = statistics.median(times[name])
            del steps
            gs = res["serial"][2]
            best = min(res["serial"][0], res["scan"][0])
            rows.append({"N": N, "T": T, "modes": list(L.auto_modes(N, T)),
                         **{k: round(res[k][0], 4) for k in fns},
                         "spikes_equal": all(torch.equal(res[k][1], res["serial"][1]) for k in ("scan", "auto")),
                         "grad_rel_auto": float((res["auto"][2] - gs).norm() / gs.norm()),
                         "auto_vs_best": round(res["auto"][0] / best, 3),
                         "x_auto_vs_serial": round(res["serial"][0] / res["auto"][0], 3)})
            del I0, G, res, gs
            torch.cuda.empty_cache()
    worst = max(r["auto_vs_best"] for r in rows)
    return {"cells": rows, "worst_auto_vs_best": worst,
            "cells_within_5pct": sum(r["auto_vs_best"] <= 1.05 for r in rows), "n_cells": len(rows),
            "all_spikes_equal": all(r["spikes_equal"] for r in rows),
            "max_grad_rel_auto": max(r["grad_rel_auto"] for r in rows)}


def profiled_traffic():
    """HBM bytes per launch of the dominant kernel from the committed counter summary
    (two rocprofv3 --pmc passes, FETCH_SIZE and WRITE_SIZE, scaled on a copy kernel)."""
    path = os.path.join(REPO, "profiles", "k_lif_bwd_fused_rc_cfg2_traffic.txt")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def inputs(beta, dev):
    import torch
    mu, sd = (0.12, 0.25) if beta == 0.9 else (0.012, 0.08)
    g = torch.Generator().manual_seed(0)
    I_cpu = (mu + sd * torch.randn(T_CFG, N_CFG, generator=g)).float()
    g1 = torch.Generator().manual_seed(1)
    gS = torch.randn(T_CFG, N_CFG, generator=g1).float().to(dev)
    return I_cpu, I_cpu.to(dev), gS


def cpu_model():
    """The host CPU's model name (lscpu's "Model name", else /proc/cpuinfo's "model name")."""
    import subprocess
    try:
        txt = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in txt.splitlines():
            if line.strip().startswith("Model name"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_baseline(I_cpu, beta, n_cols):
    """PyTorch-CPU port of fast.py: two-level pruned scan forward (C=64, K=8, repair on) and
    the Hillis-Steele affine-scan backward, plus the serial pair, on the first n_cols neurons
    of the same workload; median of 3 after one warm-up."""
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
        fn()
        ts = []
        for _ in range(3):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        out[name] = statistics.median(ts)
    return out


def check_step(L, step, I, gS, u0, beta):
    """One timed-step call checked outside the timed region: its S equals the serial forward's
    and its dI the stored-U single-pass adjoint's (same chunk and wave count), bit for bit; no
    chunk hand-off of the starts-only forward gave up.  Raises on a mismatch: a wrong step gets
    no throughput line."""
    import torch
    S, dI = step()
    Us, Ss = L.serial_forward(I, beta, 1.0, 0.0, u0)
    Lam = L.scan_backward_fused(I, u0, Us, Ss, gS, None, beta, 1.0, 0.0, 4.0)
    out = {"S_equals_serial_forward": bool(torch.equal(S, Ss)),
           "dI_equals_stored_U_adjoint": bool(torch.equal(dI, Lam)),
           "spin_timeouts": L.starts_forward_timeouts(I.device)}
    if not (out["S_equals_serial_forward"] and out["dI_equals_stored_U_adjoint"]
            and out["spin_timeouts"] == 0):
        raise RuntimeError(f"the timed step's result is wrong: {out}")
    return out


def bench_cfg2_mapscan(torch, L, dev, u0, reps):
    """BASELINE configs[1] as stated: the two-level map-scan forward (scan_forward_v3's own
    pipeline: envelope + capacity-K chunk maps, carry with overflow fallback, replay, device
    repair to convergence) at C in {32, 64, 128}, K = 8, for beta = 0.9 and 0.99, against the
    serial forward; % of the 12 B/neuron-step roofline, overflow fraction and repair rounds.
    The timed calls request no statistics, so their repair is the ordered pass (one walk over
    each neuron's chunks) where the launcher picks it; repair_iters is the Jacobi round count
    of a separate call with statistics (the reference's definition).  Also the single pass
    with map speculation (C = 16, K = 8), and reference_inputs: the reference's published cfg2
    cells (results/logs/node5/e6d_0.9.log:15, e6d_0.99.log:15: x ~ N(0.15, 0.4^2), u0 = 0,
    scan_forward_v3 at its best cell C = 256, K = 8, timed there without repair) on the same
    inputs, without and with repair, and its few-neuron, long-sequence cells (N = 128 / 1024,
    T = 16384 / 65536) against this build's exact forward and scan adjoint."""
    T, N = T_CFG, N_CFG
    out = {}
    for beta in (0.9, 0.99):
        _, I, _ = inputs(beta, dev)
        Us, Ss = L.serial_forward(I, beta, 1.0, 0.0, u0)
        r = {"serial_fwd_ms": round(ev_time(lambda: L.serial_forward(I, beta, 1.0, 0.0, u0), reps), 4)}
        for C in (32, 64, 128):
            st = {}
            U, S = L.scan_forward_mapscan(I, beta, 1.0, 0.0, u0, C=C, K=8, repair=10 ** 6, stats=st)
            ok = bool(torch.equal(U, Us) and torch.equal(S, Ss))
            del U, S
            t = ev_time(lambda: L.scan_forward_mapscan(I, beta, 1.0, 0.0, u0, C=C, K=8, repair=10 ** 6),
                        reps)
            r[f"C{C}_K8"] = {"ms": round(t, 4),
                             "pct_roofline_12B": round(100 * B_FWD * N * T / (t / 1000.0) / 1e9 / HBM_PEAK_GBS, 2),
                             "equals_serial": ok, "overflow_frac": round(st["overflow_frac"], 6),
                             "repair_iters": st["repair_iters"], "mean_pieces": round(st["mean_pieces"], 4),
                             "max_pieces": st["max_pieces"]}
        t = ev_time(lambda: L.scan_forward_exact(I, beta, 1.0, 0.0, u0, C=16, K=8, maps=True), reps)
        U, S = L.scan_forward_exact(I, beta, 1.0, 0.0, u0, C=16, K=8, maps=True)
        r["single_pass_maps_C16_K8"] = {"ms": round(t, 4), "equals_serial": bool(torch.equal(U, Us) and torch.equal(S, Ss)),
                                        **L.last_fused_counters()}
        out[f"beta{beta}"] = r
        del I, Us, Ss, U, S
        torch.cuda.empty_cache()
    # results/e6d_full_beta0.9.json / _beta0.99.json, the N = 65536, T = 4096 rows: the best
    # scan cell's time, overflow fraction and mean pieces (its inputs are drawn on the device, so
    # these are the same distribution, not the same values), and the tuned serial forward
    published = {0.9: {"scan_fwd_ms": 4.156, "serial_fwd_ms": 2.226, "overflow_frac": 0.000177,
                       "mean_pieces": 4.0647, "spike_flips": 0},
                 0.99: {"scan_fwd_ms": 4.560, "serial_fwd_ms": 2.238, "overflow_frac": 0.027790,
                        "mean_pieces": 5.2204, "spike_flips": 0}}
    ref = {}
    for beta in (0.9, 0.99):
        g = torch.Generator().manual_seed(0)
        I = (0.15 + 0.4 * torch.randn(T, N, generator=g)).to(dev)
        Us, Ss = L.serial_forward(I, beta, 1.0, 0.0, u0)
        st = {}
        U, S = L.scan_forward_mapscan(I, beta, 1.0, 0.0, u0, C=256, K=8, repair=0, stats=st)
        flips = int((S != Ss).sum().item())
        t0 = ev_time(lambda: L.scan_forward_mapscan(I, beta, 1.0, 0.0, u0, C=256, K=8, repair=0), reps)
        U, S = L.scan_forward_mapscan(I, beta, 1.0, 0.0, u0, C=256, K=8, repair=10 ** 6)
        ok = bool(torch.equal(U, Us) and torch.equal(S, Ss))
        t1 = ev_time(lambda: L.scan_forward_mapscan(I, beta, 1.0, 0.0, u0, C=256, K=8, repair=10 ** 6), reps)
        ts = ev_time(lambda: L.serial_forward(I, beta, 1.0, 0.0, u0), reps)
        pub = published[beta]
        ref[f"beta{beta}"] = {
            "scan_no_repair_ms": round(t0, 4), "scan_no_repair_spike_flips": flips,
            "overflow_frac": round(st["overflow_frac"], 6), "mean_pieces": round(st["mean_pieces"], 4),
            "scan_repair_ms": round(t1, 4),
            "scan_repair_equals_serial": ok, "serial_fwd_ms": round(ts, 4),
            "reference_rtx5090_ms": pub,
            "speedup_vs_reference": {"scan_fwd": round(pub["scan_fwd_ms"] / t0, 3),
                                     "serial_fwd": round(pub["serial_fwd_ms"] / ts, 3)}}
        del I, Us, Ss, U, S
        torch.cuda.empty_cache()
    out["reference_inputs"] = ref
    # the reference's few-neuron, long-sequence cells (the same e6d logs, rows N = 128 / 1024,
    # T = 16384 / 65536): its tuned serial sweeps and its best scan cell (forward without repair,
    # the chunked affine-scan adjoint) against this build's serial sweeps, its converged exact
    # forward (scan_forward_v3 with repair to convergence: the serial recurrence) and
    # scan_backward_auto, on the reference's inputs
    pub = {(0.9, 128, 16384): (0.341, 1.310, 0.137, 0.072), (0.9, 128, 65536): (1.495, 7.765, 0.265, 0.314),
           (0.9, 1024, 16384): (0.411, 1.980, 0.334, 0.487), (0.9, 1024, 65536): (1.600, 7.793, 1.326, 1.957),
           (0.99, 128, 16384): (0.342, 1.318, 0.149, 0.073), (0.99, 128, 65536): (1.499, 7.758, 0.287, 0.313),
           (0.99, 1024, 16384): (0.412, 1.969, 0.403, 0.489), (0.99, 1024, 65536): (1.604, 7.808, 1.601, 1.965)}
    few = {}
    for (beta, Nf, Tf), (rsf, rsb, rcf, rcb) in pub.items():
        g = torch.Generator().manual_seed(0)
        I = (0.15 + 0.4 * torch.randn(Tf, Nf, generator=g)).to(dev)
        GS = torch.randn(Tf, Nf, generator=torch.Generator().manual_seed(1)).to(dev)
        z = torch.zeros(Nf, device=dev)
        U, S = L.serial_forward(I, beta, 1.0, 0.0, z)
        U2, S2 = L.scan_forward_v3(I, beta, 1.0, 0.0, z, C=64, K=16, repair=10 ** 6)
        ok = bool(torch.equal(U2, U) and torch.equal(S2, S))
        mine = (ev_time(lambda: L.serial_forward(I, beta, 1.0, 0.0, z), reps),
                ev_time(lambda: L.serial_backward(I, z, U, S, GS, None, beta, 1.0, 0.0), reps),
                ev_time(lambda: L.scan_forward_v3(I, beta, 1.0, 0.0, z, C=64, K=16, repair=10 ** 6), reps),
                ev_time(lambda: L.scan_backward_auto(I, z, U, S, GS, None, beta, 1.0, 0.0), reps))
        keys = ("serial_fwd_ms", "serial_bwd_ms", "scan_fwd_ms", "scan_bwd_ms")
        # the map scan itself without repair, as the reference's scan cell (best of C 128 / 256, K 16)
        ms = min((ev_time(lambda: L.scan_forward_mapscan(I, beta, 1.0, 0.0, z, C=C, K=16, repair=0), reps), C)
                 for C in (128, 256))
        _, S3 = L.scan_forward_mapscan(I, beta, 1.0, 0.0, z, C=ms[1], K=16, repair=0)
        few[f"beta{beta}_N{Nf}_T{Tf}"] = {
            **{k: round(v, 4) for k, v in zip(keys, mine)}, "scan_fwd_equals_serial": ok,
            "map_scan_no_repair_ms": round(ms[0], 4), "map_scan_C": ms[1],
            "map_scan_spike_flips": int((S3 != S).sum().item()),
            "reference_rtx5090_ms": dict(zip(keys, (rsf, rsb, rcf, rcb))),
            "speedup_vs_reference": {**{k: round(r / v, 3) for k, v, r in zip(keys, mine, (rsf, rsb, rcf, rcb))},
                                     "map_scan_no_repair": round(rcf / ms[0], 3)}}
        del I, GS, U, S, U2, S2, S3
    out["reference_inputs"]["few_neurons"] = few
    torch.cuda.empty_cache()
    return out


def bench_cfg3(torch, dev, reps):
    """cfg3: the 700-256-256-20 network, batch 64, T=1024, Bernoulli(0.015)
    raster, beta=0.95, cross-entropy on random labels; one step = zero_grad + forward + loss +
    backward (the reference's e7c_timing.py step).  Also the two LIF layers alone (fwd+bwd on
    their [1024, 16384] currents, HIP events)."""
    import torch.nn as nn
    from lifscan.shdnet import Net
    from lifscan import hip_lif as L
    T, B = 1024, 64
    g = torch.Generator().manual_seed(3)
    x = (torch.rand(B, T, 700, generator=g) < 0.015).float().transpose(0, 1).contiguous().to(dev)
    y = torch.randint(0, 20, (B,), generator=torch.Generator().manual_seed(5)).to(dev)
    out = {}
    torch.manual_seed(4)
    net = Net("scan").to(dev)
    with torch.no_grad():
        I1 = net.l1.fc(x).reshape(T, -1).contiguous()
        s1 = L.lif_tuned(I1, torch.zeros(I1.shape[1], device=dev), beta=0.95, mode="scan", K=16,
                         repair=10 ** 6).reshape(T, B, -1)
        I2 = net.l2.fc(s1).reshape(T, -1).contiguous()
    g2 = torch.randn(T, I1.shape[1], generator=torch.Generator().manual_seed(6)).to(dev)

    def layers():
        for I in (I1, I2):
            Ig = I.detach().requires_grad_(True)
            S = L.lif_tuned(Ig, torch.zeros(I.shape[1], device=dev), beta=0.95, mode="scan", K=16,
                            repair=10 ** 6)
            S.backward(g2)
    # small kernels (~65 us per layer): timed back to back (the host's per-call work overlaps
    # the previous call's kernels, as in a training loop), and per call (one call between two
    # synchronizations, the host's launch latency included)
    out["lif_layers_fwd_bwd_ms"] = bb_time(layers, max(reps, 10), warm=2, warm_s=0.5)
    out["lif_layers_fwd_bwd_per_call_ms"] = ev_time(layers, max(reps, 10), warm=2)
    # cache-cold: each layer's arrays are 64 MiB, within the 256 MB Infinity Cache when called
    # back to back; after a 1 GiB scrub the operands come from HBM
    out["lif_layers_fwd_bwd_cold_ms"] = ev_time_cold(layers, max(reps, 10), warm=2)
    # lif_tuned runs its recomputing pair from the C++ autograd function (lifscan/_ops.cpp);
    # the same kernels through the Python autograd function, for the host cost it removes
    out["lif_tuned_host_path"] = "c++" if L._rc_path(I1, torch.zeros(I1.shape[1], device=dev), 0.95,
                                                     "scan", 16, 10 ** 6) is not None else "python"

    def layers_py():
        for I in (I1, I2):
            Ig = I.detach().requires_grad_(True)
            S = L.LIFTuned.apply(Ig, torch.zeros(I.shape[1], device=dev), 0.95, 1.0, 0.0, 4.0, "scan",
                                 16, 10 ** 6)
            S.backward(g2)
    out["lif_layers_fwd_bwd_python_autograd_ms"] = bb_time(layers_py, max(reps, 10), warm=2, warm_s=0.5)
    out["lif_layers_fwd_bwd_python_autograd_per_call_ms"] = ev_time(layers_py, max(reps, 10), warm=2)
    for mode in ("scan", "serial", "auto"):
        torch.manual_seed(4)
        netm = Net(mode).to(dev)

        def step():
            netm.zero_grad()
            logits, _ = netm(x)
            nn.functional.cross_entropy(logits, y).backward()
        out[f"step_ms_{mode}"] = ev_time(step, reps, warm=3)
    nsteps = 2 * T * I1.shape[1]
    nbytes = (B_FWD_RC + B_BWD_RC) if L._recompute_ok(T, I1.shape[1], 16, 10 ** 6) else (B_FWD + B_BWD)
    out["lif_layers_bytes_per_neuron_step"] = nbytes
    out["lif_layers_pct_roofline"] = round(
        100 * nbytes * nsteps / (out["lif_layers_fwd_bwd_ms"] / 1000.0) / 1e9 / HBM_PEAK_GBS, 2)
    out["lif_layers_pct_roofline_cold"] = round(
        100 * nbytes * nsteps / (out["lif_layers_fwd_bwd_cold_ms"] / 1000.0) / 1e9 / HBM_PEAK_GBS, 2)
    out["config"] = "700-256-256-20, B=64, T=1024, beta=0.95, lif_tuned(scan, K=16, repair on)"
    return {k: (round(v, 4) if isinstance(v, float) else v) for k, v in out.items()}


def bench_cfg4(torch, dev, reps):
    """cfg4: N=1024, T=2^20, beta=0.99, x~N(0.012,0.08^2), u0~U[0,1).
    Forward: the three-level pipeline (scan_forward_v4_maps, repair on; an overflowed super map
    passed as stored, and at the reference default also by walking its chunk maps and by the
    reference's serial fallback) on a small grid of (C, G, K, K2) with overflow statistics, as the
    reference's e9d grid does (the reference default first), and scan_forward_v4's converged
    dispatch; the
    converged two-level scan_forward_v3 (which takes the warm-started chunks here), the warm
    forward at other chunk / warm-up lengths and the long-chunk map scan in pieces it replaced;
    the single-pass exact forward; the serial forward.  Backward: the affine-scan adjoint and the
    serial one.
    fwd+bwd = the fastest exact forward + the scan adjoint.  reference_cells: the reference's
    published e9d cells (N = 128 / 1024, T = 2^18, its inputs) against this build's passes."""
    from lifscan import hip_lif as L
    T, N, beta = 2 ** 20, 1024, 0.99
    I = (0.012 + 0.08 * torch.randn(T, N, generator=torch.Generator().manual_seed(0))).to(dev)
    u0 = torch.rand(N, generator=torch.Generator().manual_seed(2)).to(dev)
    gS = torch.randn(T, N, generator=torch.Generator().manual_seed(1)).to(dev)
    out = {}
    U, S = L.serial_forward(I, beta, 1.0, 0.0, u0)
    exact = lambda A, B: bool(torch.equal(A, U) and torch.equal(B, S))
    v4 = {}
    # the timed call is converged without statistics; "auto" there passes an overflowed super map
    # as stored (the repair corrects its start), the other rules are timed at the reference default
    for C, G, K, K2, fb in ((64, 16, 16, 32, "auto"), (64, 16, 16, 32, "chunks"), (64, 16, 16, 32, "serial"),
                            (1024, 4, 32, 64, "auto"), (2048, 4, 32, 64, "auto")):
        st = {}
        U4, S4 = L.scan_forward_v4_maps(I, beta, 1.0, 0.0, u0, C=C, G=G, K=K, K2=K2, repair=10 ** 6, stats=st,
                                        super_fallback="serial" if fb == "serial" else "chunks")
        ok = exact(U4, S4)
        del U4, S4
        U4, S4 = L.scan_forward_v4_maps(I, beta, 1.0, 0.0, u0, C=C, G=G, K=K, K2=K2, repair=10 ** 6,
                                        super_fallback=fb)
        ok = ok and exact(U4, S4)
        del U4, S4
        ms = ev_time(lambda: L.scan_forward_v4_maps(I, beta, 1.0, 0.0, u0, C=C, G=G, K=K, K2=K2,
                                                    repair=10 ** 6, super_fallback=fb), 2, warm=1)
        key = f"C{C}_G{G}_K{K}_K2{K2}" + {"auto": "", "chunks": "_chunk_walk", "serial": "_serial_fallback"}[fb]
        v4[key] = {"ms": round(ms, 4), "equals_serial": ok,
                   **{k: (round(v, 6) if isinstance(v, float) else v) for k, v in st.items()}}
    out["v4"] = v4
    # scan_forward_v4 itself at the reference default: converged without statistics it takes the
    # fastest exact path, as scan_forward_v3 does
    U4, S4 = L.scan_forward_v4(I, beta, 1.0, 0.0, u0, C=64, G=16, K=16, K2=32, repair=10 ** 6)
    out["v4_converged_dispatch_equals_serial"] = exact(U4, S4)
    del U4, S4
    out["v4_converged_dispatch_ms"] = ev_time(lambda: L.scan_forward_v4(I, beta, 1.0, 0.0, u0, C=64, G=16, K=16,
                                                                        K2=32, repair=10 ** 6), reps)
    U3, S3 = L.scan_forward_v3(I, beta, 1.0, 0.0, u0, C=256, K=16, repair=10 ** 6)
    out["v3_converged_equals_serial"] = exact(U3, S3)
    run = L.last_scan_run()
    out["v3_converged_path"] = ("warm-started chunks" if getattr(run, "warm", False) else
                                f"long-chunk map scan in {run.pieces} piece(s)")
    out["v3_converged_chunk"] = run.C
    if getattr(run, "warm", False):
        out["v3_converged_warmup"] = run.W
    else:
        out["v3_converged_pieces"] = run.pieces
    del U3, S3
    out["fwd_v3_converged_ms"] = ev_time(lambda: L.scan_forward_v3(I, beta, 1.0, 0.0, u0, C=256, K=16,
                                                                   repair=10 ** 6), reps)
    warm = {}
    for C, W in ((16384, 2560), (16384, 4096), (8192, 2048), (4096, 2048)):
        st = {}
        Uw, Sw = L.scan_forward_warm(I, beta, 1.0, 0.0, u0, C=C, W=W, stats=st)
        ok = exact(Uw, Sw)
        del Uw, Sw
        ms = ev_time(lambda: L.scan_forward_warm(I, beta, 1.0, 0.0, u0, C=C, W=W), reps)
        warm[f"C{C}_W{W}"] = {"ms": round(ms, 4), "equals_serial": ok,
                              "missed_frac": round(st["missed_frac"], 6),
                              "repair_iters": st["repair_iters"]}
    out["warm"] = warm
    # the two-level map scan at long chunks with its two carries: the associative one (chunk
    # maps composed by a parallel prefix, DPP in the wave and LDS across waves) and the
    # sequential one (one map after another per neuron), both run to convergence
    maps = {}
    for carry, fn in (("assoc", L.scan_forward_assoc), ("sequential", L.scan_forward_mapscan)):
        for C, K in ((2048, 32), (4096, 32)):
            st = {}
            kw = {} if carry == "assoc" else {"repair": 10 ** 6}
            Um, Sm = fn(I, beta, 1.0, 0.0, u0, C=C, K=K, stats=st, **kw)
            ok = exact(Um, Sm)
            del Um, Sm
            ms = ev_time(lambda: fn(I, beta, 1.0, 0.0, u0, C=C, K=K, **kw), 3)
            maps[f"{carry}_C{C}_K{K}"] = {"ms": round(ms, 4), "equals_serial": ok,
                                          **{k: (round(v, 6) if isinstance(v, float) else v)
                                             for k, v in st.items()}}
    out["mapscan_converged"] = maps
    C2, P = L.long_sequence_plan(T, N)
    U2, S2 = L._scan2_pieces(I, beta, 1.0, 0.0, u0, C2, L.LONG_K, P)
    out["longchunk_pieces_equals_serial"] = exact(U2, S2)
    del U2, S2
    out["fwd_longchunk_pieces_ms"] = ev_time(
        lambda: L._scan2_pieces(I, beta, 1.0, 0.0, u0, C2, L.LONG_K, P), reps)
    U2, S2 = L.scan_forward_exact(I, beta, 1.0, 0.0, u0, K=8, maps=False)
    out["single_pass_equals_serial"] = exact(U2, S2)
    del U2, S2
    out["fwd_single_pass_ms"] = ev_time(lambda: L.scan_forward_exact(I, beta, 1.0, 0.0, u0, K=8, maps=False), 3)
    out["fwd_serial_ms"] = ev_time(lambda: L.serial_forward(I, beta, 1.0, 0.0, u0), 3)
    out["bwd_scan_ms"] = ev_time(lambda: L.scan_backward_tiled(I, u0, U, S, gS, None, beta, 1.0, 0.0, 4.0), reps)
    out["bwd_serial_ms"] = ev_time(lambda: L.serial_backward(I, u0, U, S, gS, None, beta, 1.0, 0.0, 4.0), 2)
    ns = T * N
    t_fwd = min(out["fwd_v3_converged_ms"], out["fwd_single_pass_ms"], min(r["ms"] for r in v4.values()),
                min(r["ms"] for r in warm.values() if r["equals_serial"]))
    t_fb = t_fwd + out["bwd_scan_ms"]
    out["fwd_bwd_ms"] = t_fb
    out["fwd_bwd_value"] = round(ns / (t_fb / 1000.0), 1)
    out["pct_roofline_fwd_bwd"] = round(100 * (B_FWD + B_BWD) * ns / (t_fb / 1000.0) / 1e9 / HBM_PEAK_GBS, 2)
    out["config"] = "N=1024, T=1048576, beta=0.99, x~N(0.012,0.08^2), u0~U[0,1)"
    del I, U, S, gS
    torch.cuda.empty_cache()
    # the reference's nearest published cells (results/logs/node5/e9d_0.99.log: N = 128 / 1024,
    # T = 2^18, x ~ N(0.15, 0.4^2), u0 = 0): its tuned serial sweeps, its best v3 and v4 cells
    # (no repair; v4 at C 128, G 8, K 16) and its scan adjoint, against this build's serial sweeps,
    # converged exact forward, v4 at the same cell without repair and scan_backward_auto
    e9d = {}
    for Nr, pub in ((128, (6.021, 1.280, 1.565, 30.981, 1.255)), (1024, (6.459, 6.297, 8.279, 31.040, 8.071))):
        Tr = 2 ** 18
        g = torch.Generator().manual_seed(0)
        Ir = (0.15 + 0.4 * torch.randn(Tr, Nr, generator=g)).to(dev)
        GSr = torch.randn(Tr, Nr, generator=torch.Generator().manual_seed(1)).to(dev)
        z = torch.zeros(Nr, device=dev)
        Ur, Sr = L.serial_forward(Ir, beta, 1.0, 0.0, z)
        U2, S2 = L.scan_forward_v3(Ir, beta, 1.0, 0.0, z, C=256, K=16, repair=10 ** 6)
        ok = bool(torch.equal(U2, Ur) and torch.equal(S2, Sr))
        del U2, S2
        mine = (ev_time(lambda: L.serial_forward(Ir, beta, 1.0, 0.0, z), 3),
                ev_time(lambda: L.scan_forward_v3(Ir, beta, 1.0, 0.0, z, C=256, K=16, repair=10 ** 6), 3),
                ev_time(lambda: L.scan_forward_v4(Ir, beta, 1.0, 0.0, z, C=128, G=8, K=16, K2=32, repair=0), 3),
                ev_time(lambda: L.serial_backward(Ir, z, Ur, Sr, GSr, None, beta, 1.0, 0.0), 3),
                ev_time(lambda: L.scan_backward_auto(Ir, z, Ur, Sr, GSr, None, beta, 1.0, 0.0), 3))
        keys = ("serial_fwd_ms", "v3_fwd_ms", "v4_fwd_ms", "serial_bwd_ms", "scan_bwd_ms")
        e9d[f"N{Nr}_T{Tr}"] = {**{k: round(v, 4) for k, v in zip(keys, mine)}, "v3_equals_serial": ok,
                               "reference_rtx5090_ms": dict(zip(keys, pub)),
                               "speedup_vs_reference": {k: round(r / v, 3) for k, v, r in zip(keys, mine, pub)}}
        del Ir, GSr, Ur, Sr
        torch.cuda.empty_cache()
    out["reference_cells"] = e9d
    return {k: (round(v, 4) if isinstance(v, float) else v) for k, v in out.items()}


def bench_cfg5(torch, dev, reps):
    """cfg5: ALIF, N=16384, T=4096, beta=0.95, rho=0.995, q=0.2,
    theta0=1, u_r=0, x~N(0.15,0.3^2), u0=w0=0.  alif() fwd+bwd with the parameter gradients:
    serial forward + scan adjoint, and the box scan (Wpred from alif_warm_predict(Wn=4), its
    cost included, dw=0.1q, C=128, K1=K2=32) + scan adjoint; plus the exact box-scan pipeline
    with repair (alif_scan_forward_maps) for both predictions (warm-up, previous iterate) and dw
    in {0.1q, 0.3q} (statistics), alif_scan_forward's converged dispatch (the serial forward),
    and the serial forward."""
    from lifscan import triton_alif as A
    T, N, beta, rho, q, C = 4096, 16384, 0.95, 0.995, 0.2, 128
    I = (0.15 + 0.3 * torch.randn(T, N, generator=torch.Generator().manual_seed(0))).to(dev)
    gS = torch.randn(T, N, generator=torch.Generator().manual_seed(1)).to(dev)
    z = torch.zeros(N, device=dev)
    ps = [torch.tensor(v, device=dev, requires_grad=True) for v in (beta, rho, q, 1.0)]
    Ig = I.clone().requires_grad_(True)
    out = {}
    for fwd in ("serial", "scan"):
        def step():
            Ig.grad = None
            for p in ps:
                p.grad = None
            Wp = A.alif_warm_predict(I, beta, rho, q, 1.0, 0.0, z, z, C, Wn=4) if fwd == "scan" else None
            S, _, _ = A.alif(Ig, z, z, *ps, fwd=fwd, bwd="scan", Wpred=Wp, dw=0.1 * q, C=C)
            S.backward(gS)
        # back to back as the headline's step loop; per call: one step between two synchronizations
        out[f"alif_fwd_{fwd}_bwd_scan_ms"] = bb_time(step, reps, warm=2)
        out[f"alif_fwd_{fwd}_bwd_scan_per_call_ms"] = ev_time(step, reps, warm=1)
        # cache-cold: cfg5's arrays are 256 MiB each, so back-to-back calls find part of their
        # operands in the 256 MB Infinity Cache; after a 1 GiB scrub they read HBM
        out[f"alif_fwd_{fwd}_bwd_scan_cold_ms"] = ev_time_cold(step, reps)
    out["serial_fwd_ms"] = ev_time(lambda: A.alif_serial_forward(I, beta, rho, q, 1.0, 0.0, z, z), reps)
    out["serial_fwd_cold_ms"] = ev_time_cold(lambda: A.alif_serial_forward(I, beta, rho, q, 1.0, 0.0, z, z),
                                             reps)
    U, W, S = A.alif_serial_forward(I, beta, rho, q, 1.0, 0.0, z, z)
    # Two predictions of the chunk-entry adaptation (experiments/e25d_alif_fwd.py:44-50): the
    # warm-up predictor, and the previous fitting iterate emulated by a 1.005x input.
    _, Wprev, _ = A.alif_serial_forward((1.005 * I).contiguous(), beta, rho, q, 1.0, 0.0, z, z)
    preds = {"warm4": A.alif_warm_predict(I, beta, rho, q, 1.0, 0.0, z, z, C, Wn=4),
             "prev": A.alif_prev_wpred(Wprev, z, C)}
    box = {}
    for pname, WP in preds.items():
        for dwq in (0.1, 0.3):
            st, ph = {}, {}
            U2, W2, S2 = A.alif_scan_forward(I, beta, rho, q, 1.0, 0.0, z, z, WP, dwq * q, C=C, K1=32, K2=32,
                                             BN=4, repair=10 ** 6, stats=st, phases=ph)
            eq = bool(torch.equal(U2, U) and torch.equal(W2, W) and torch.equal(S2, S))
            # the box-scan pipeline itself, converged without statistics (alif_scan_forward would
            # take the serial forward for such a call: timed once below)
            box_fn = lambda: A.alif_scan_forward_maps(I, beta, rho, q, 1.0, 0.0, z, z, WP, dwq * q, C=C,
                                                      K1=32, K2=32, BN=4, repair=10 ** 6)
            U2, W2, S2 = box_fn()
            eq = eq and bool(torch.equal(U2, U) and torch.equal(W2, W) and torch.equal(S2, S))
            ms = ev_time(box_fn, 3)
            box[f"{pname}_dw{dwq}q"] = {
                "ms": round(ms, 4), "ms_cold": round(ev_time_cold(box_fn, 3), 4), "equals_serial": eq,
                "stats": st, "phases_ms": {k: round(v, 4) for k, v in ph.items()}}
            del U2, W2, S2
    out["box_scan_repair"] = box
    # alif_scan_forward converged without statistics: the serial forward (the same bits)
    WP = preds["warm4"]
    disp = lambda: A.alif_scan_forward(I, beta, rho, q, 1.0, 0.0, z, z, WP, 0.1 * q, C=C, K1=32, K2=32, BN=4,
                                       repair=10 ** 6)
    U2, W2, S2 = disp()
    out["box_scan_converged_dispatch"] = {
        "ms": round(ev_time(disp, reps), 4),
        "equals_serial": bool(torch.equal(U2, U) and torch.equal(W2, W) and torch.equal(S2, S))}
    del U2, W2, S2
    del Wprev, preds
    out["bwd_scan_ms"] = ev_time(lambda: A.alif_backward(I, U, W, S, gS, beta, rho, q, 1.0, z, z), reps)
    # the layer's adjoint (dI, dw0 and the parameter sums, LW not written): reading the stored
    # states, and recomputing them inside each chunk from the row before it
    from lifscan import hip_alif as H
    for name, rc in (("stored", None), ("recompute", 0.0)):
        out[f"bwd_layer_{name}_ms"] = ev_time(lambda: H._alif_bwd_call(
            I, U, W, S, gS, beta, rho, q, 1.0, z, z, 4.0, "scan", 64, want_lw=False, want_params=True,
            recompute_ur=rc), reps)
    ns = T * N
    t = out["alif_fwd_serial_bwd_scan_ms"]
    out["fwd_bwd_value"] = round(ns / (t / 1000.0), 1)
    # ALIF algorithmic bytes: fwd read I, write U, W, S (16); bwd read I, U, W, S, gS, write dI
    # (24), or with the recomputing adjoint read I, gS and U, W once per 16-step chunk, write dI
    # (12.5)
    bps = 16 + (12.5 if H.ALIF_RECOMPUTE_BWD else 24)
    out["bytes_per_neuron_step"] = bps
    out["pct_roofline_fwd_bwd"] = round(100 * bps * ns / (t / 1000.0) / 1e9 / HBM_PEAK_GBS, 2)
    tc = out["alif_fwd_serial_bwd_scan_cold_ms"]
    out["fwd_bwd_value_cold"] = round(ns / (tc / 1000.0), 1)
    out["pct_roofline_fwd_bwd_cold"] = round(100 * bps * ns / (tc / 1000.0) / 1e9 / HBM_PEAK_GBS, 2)
    out["serial_fwd_cold_GBps"] = round(16 * ns / (out["serial_fwd_cold_ms"] / 1000.0) / 1e9, 1)
    out["config"] = "ALIF N=16384, T=4096, beta=0.95, rho=0.995, q=0.2, x~N(0.15,0.3^2)"
    del I, gS, U, W, S, Ig
    torch.cuda.empty_cache()
    out["reference_shape"] = bench_alif_reference_shape(torch, dev)
    return {k: (round(v, 4) if isinstance(v, float) else v) for k, v in out.items()}


def bench_alif_reference_shape(torch, dev):
    """The shape the reference publishes for ALIF (lsnn beta=0.95,
    rho=0.995, q=0.9, free mean 1.0, N=1024, T=65536; inputs as experiments/e25d_alif_fwd.py:37,
    u0=w0=0): serial forward; box scan with the previous-iterate prediction (1.005x input, C=256,
    dw=0.1q, K1=K2=32; without repair as the reference times it, and with repair, exact); serial
    and scan adjoints.  RTX 5090 figures (results/e25d_alif_fwd.json, e25e_alif_fb.json): 2.94 /
    9.42 ms forward, 8.82 / 3.90 ms adjoint.  few_neurons: the same at N = 16 and 128, where the
    box scan beats the serial forward (0.677 / 1.385 ms there against 2.14 / 2.78 serial)."""
    import math
    from lifscan import triton_alif as A
    beta, rho, q, m, N, T, C = 0.95, 0.995, 0.9, 1.0, 1024, 65536, 256
    g = torch.Generator().manual_seed(0)
    I = ((1 - beta) * m + 0.5 * math.sqrt(1 - beta * beta) * torch.randn(T, N, generator=g)).to(dev)
    gS = torch.randn(T, N, generator=torch.Generator().manual_seed(1)).to(dev)
    z = torch.zeros(N, device=dev)
    out = {"fwd_serial_ms": ev_time(lambda: A.alif_serial_forward(I, beta, rho, q, 1.0, 0.0, z, z), 5)}
    U, W, S = A.alif_serial_forward(I, beta, rho, q, 1.0, 0.0, z, z)
    _, Wprev, _ = A.alif_serial_forward((1.005 * I).contiguous(), beta, rho, q, 1.0, 0.0, z, z)
    WP = A.alif_prev_wpred(Wprev, z, C)
    del Wprev
    for name, rep in (("no_repair", 0), ("repair", 10 ** 6)):
        st = {}
        U2, W2, S2 = A.alif_scan_forward(I, beta, rho, q, 1.0, 0.0, z, z, WP, 0.1 * q, C=C, K1=32, K2=32,
                                         BN=4, repair=rep, stats=st)
        # the box-scan pipeline itself (converged, alif_scan_forward would take the serial forward)
        out[f"fwd_box_scan_{name}_ms"] = ev_time(lambda: A.alif_scan_forward_maps(
            I, beta, rho, q, 1.0, 0.0, z, z, WP, 0.1 * q, C=C, K1=32, K2=32, BN=4, repair=rep), 3)
        out[f"fwd_box_scan_{name}_spike_flips"] = int((S2 != S).sum().item())
        out[f"fwd_box_scan_{name}_miss_frac"] = round(float(st["miss_frac"]), 6)
        del U2, W2, S2
    for mode in ("serial", "scan"):
        out[f"bwd_{mode}_ms"] = ev_time(lambda: A.alif_backward(I, U, W, S, gS, beta, rho, q, 1.0, z, z,
                                                                mode=mode), 3)
    ref = {"fwd_serial_ms": 2.94, "fwd_box_scan_no_repair_ms": 9.42, "bwd_serial_ms": 8.82,
           "bwd_scan_ms": 3.90}
    out["reference_rtx5090_ms"] = ref
    out["speedup_vs_reference"] = {k: round(v / out[k], 3) for k, v in ref.items()}
    del I, gS, U, W, S, WP
    # the box scan's own regime, few neurons (results/e25d_alif_fwd.json, lsnn m = 1.0, T = 65536,
    # the previous-iterate prediction; the reference's best cell of its grid): the best of
    # C in {256, 512} x dw in {0.1q, 0.3q}, without repair as timed there, against its times
    small = {}
    for Ns, ref_serial, ref_box in ((16, 2.143, 0.677), (128, 2.783, 1.385)):
        g = torch.Generator().manual_seed(0)
        I = ((1 - beta) * m + 0.5 * math.sqrt(1 - beta * beta) * torch.randn(T, Ns, generator=g)).to(dev)
        z = torch.zeros(Ns, device=dev)
        _, _, S = A.alif_serial_forward(I, beta, rho, q, 1.0, 0.0, z, z)
        ts = ev_time(lambda: A.alif_serial_forward(I, beta, rho, q, 1.0, 0.0, z, z), 5)
        _, Wprev, _ = A.alif_serial_forward((1.005 * I).contiguous(), beta, rho, q, 1.0, 0.0, z, z)
        best = None
        for Cs in (256, 512):
            WPs = A.alif_prev_wpred(Wprev, z, Cs)
            for dwq in (0.1, 0.3):
                t = ev_time(lambda: A.alif_scan_forward(I, beta, rho, q, 1.0, 0.0, z, z, WPs, dwq * q, C=Cs,
                                                        K1=32, K2=32, BN=4, repair=0), 5)
                if best is None or t < best[0]:
                    best = (t, Cs, dwq, WPs)
        t, Cs, dwq, WPs = best
        _, _, S2 = A.alif_scan_forward(I, beta, rho, q, 1.0, 0.0, z, z, WPs, dwq * q, C=Cs, K1=32, K2=32, BN=4,
                                       repair=0)
        small[f"N{Ns}"] = {"fwd_serial_ms": round(ts, 4), "fwd_box_scan_no_repair_ms": round(t, 4), "C": Cs,
                           "dw_over_q": dwq, "spike_flips": int((S2 != S).sum().item()),
                           "reference_rtx5090_ms": {"fwd_serial_ms": ref_serial, "fwd_box_scan_no_repair_ms": ref_box},
                           "speedup_vs_reference": {"fwd_serial_ms": round(ref_serial / ts, 3),
                                                    "fwd_box_scan_no_repair_ms": round(ref_box / t, 3)}}
        del I, S, S2, Wprev, WPs
    out["few_neurons"] = small
    out["config"] = "ALIF lsnn N=1024, T=65536, free mean 1.0 (experiments/e25d_alif_fwd.py inputs)"
    torch.cuda.empty_cache()
    return {k: (round(v, 4) if isinstance(v, float) else v) for k, v in out.items()}


def bench_affine(torch, dev, reps):
    """Affine reset u <- gamma*v + delta (triton_affine.py; no published number).
    (a) the reference's own test shape (tests/test_affine.py:7-18): T=8192, N=200, beta=0.9,
        x~N(0.15,0.4^2), u0~N(0,0.2^2), C=128, K=32: serial forward vs the scan with repair
        (bit-identical) for gamma, delta = (0.3, -0.1) and (1, -1);
    (b) the cfg2 shape (65536 x T=4096, beta=0.9, x~N(0.12,0.25^2), u0=0) with gamma=0.5,
        delta=-0.25: lif_affine fwd (serial) + bwd with the five gradients through autograd, and
        the adjoint alone against its 20 B/neuron-step roofline;
    (c) the soft reset on the reference's soft test shapes."""
    from lifscan import triton_affine as AF
    out = {}
    T, N = 8192, 200
    g = torch.Generator().manual_seed(0)
    I = (0.15 + 0.4 * torch.randn(T, N, generator=g)).to(dev)
    u0 = (0.2 * torch.randn(N, generator=g)).to(dev)
    for gamma, delta in ((0.3, -0.1), (1.0, -1.0)):
        tag = f"small_g{gamma}_d{delta}"
        Ur, Sr = AF.aff_serial_forward(I, 0.9, 1.0, gamma, delta, u0)
        st = {}
        U, S = AF.aff_scan_forward(I, 0.9, 1.0, gamma, delta, u0, C=128, K=32, repair=10 ** 6, stats=st)
        out[tag] = {
            "serial_fwd_ms": round(ev_time(lambda: AF.aff_serial_forward(I, 0.9, 1.0, gamma, delta, u0), reps), 4),
            "scan_repair_ms": round(ev_time(lambda: AF.aff_scan_forward(
                I, 0.9, 1.0, gamma, delta, u0, C=128, K=32, repair=10 ** 6), reps), 4),
            "scan_equals_serial": bool(torch.equal(U, Ur) and torch.equal(S, Sr)),
            "stats": st}
    del I, u0, U, S, Ur, Sr
    T, N = T_CFG, N_CFG
    I = (0.12 + 0.25 * torch.randn(T, N, generator=torch.Generator().manual_seed(0))).to(dev)
    gS = torch.randn(T, N, generator=torch.Generator().manual_seed(1)).to(dev)
    z = torch.zeros(N, device=dev)
    ps = [torch.tensor(v, device=dev, requires_grad=True) for v in (0.9, 0.5, -0.25)]
    Ig = I.clone().requires_grad_(True)

    def step():
        Ig.grad = None
        for p in ps:
            p.grad = None
        S = AF.lif_affine(Ig, z, *ps, mode="serial")
        S.backward(gS)
    t = ev_time(step, reps, warm=2)
    U, S = AF.aff_serial_forward(I, 0.9, 1.0, 0.5, -0.25, z)
    tb = ev_time(lambda: AF._aff_backward(I, z, U, S, gS, 0.9, 1.0, 0.5, 4.0), reps)
    ns = T * N
    out["cfg2_shape"] = {
        "lif_affine_fwd_bwd_ms": round(t, 4),
        "fwd_bwd_value": round(ns / (t / 1000.0), 1),
        "pct_roofline_fwd_bwd": round(100 * (B_FWD + B_BWD) * ns / (t / 1000.0) / 1e9 / HBM_PEAK_GBS, 2),
        "serial_fwd_ms": round(ev_time(lambda: AF.aff_serial_forward(I, 0.9, 1.0, 0.5, -0.25, z), reps), 4),
        "bwd_with_param_sums_ms": round(tb, 4),
        "pct_roofline_bwd": round(100 * B_BWD * ns / (tb / 1000.0) / 1e9 / HBM_PEAK_GBS, 2),
        "config": "65536 x 4096, beta=0.9, gamma=0.5, delta=-0.25, x~N(0.12,0.25^2)"}
    del I, gS, U, S, Ig
    torch.cuda.empty_cache()
    # soft reset (triton_soft.py) on the reference's test shapes: the scan with repair vs serial
    # (tests/test_soft_scan.py: T=8192, N=333, x~N(0.15,0.4^2), C=K=32), and the soft layer's
    # float64 adjoint on the long narrow fitting shape (tests/test_soft_scan_grad.py: T=16384, N=8)
    from lifscan import triton_soft as TS
    from lifscan.hip_soft import _soft_backward
    T, N = 8192, 333
    g = torch.Generator().manual_seed(0)
    I = (0.15 + 0.4 * torch.randn(T, N, generator=g)).to(dev)
    u0 = (0.3 * torch.randn(N, generator=g)).to(dev)
    Ur, Sr = TS.soft_serial_forward(I, 0.95, 1.0, u0)
    st = {}
    U, S = TS.soft_scan_forward(I, 0.95, 1.0, u0, C=32, K=32, repair=10 ** 6, stats=st)
    out["soft_small"] = {
        "serial_fwd_ms": round(ev_time(lambda: TS.soft_serial_forward(I, 0.95, 1.0, u0), reps), 4),
        "scan_repair_ms": round(ev_time(lambda: TS.soft_scan_forward(I, 0.95, 1.0, u0, C=32, K=32,
                                                                     repair=10 ** 6), reps), 4),
        "scan_equals_serial": bool(torch.equal(U, Ur) and torch.equal(S, Sr)), "stats": st}
    T, N = 16384, 8
    I = (0.06 + 0.3 * torch.randn(T, N, generator=g)).to(dev)
    gS = torch.randn(T, N, generator=g).to(dev)
    z = torch.zeros(N, device=dev)
    U, S = TS.soft_serial_forward(I, 0.95, 1.0, z)
    out["soft_adjoint_T16384_N8_ms"] = round(ev_time(lambda: _soft_backward(I, z, U, gS, 0.95, 1.0, 4.0), reps), 4)
    del I, gS, U, S, Ur, Sr
    return out


def dominant_only(L, torch, dev):
    """Short program for counter passes: a 256 MiB copy (FETCH/WRITE calibration), then the
    dominant kernel (single-pass backward, cfg2) three times."""
    x = torch.empty(64 * 2 ** 20, device=dev)
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    I_cpu, I, gS = inputs(0.9, dev)
    u0 = torch.zeros(N_CFG, device=dev)
    S, ST = L.scan_forward_exact_starts(I, 0.9, 1.0, 0.0, u0)
    torch.cuda.synchronize()
    for _ in range(3):
        L.scan_backward_fused_starts(I, ST, gS, 0.9, 1.0, 0.0, 4.0)
    torch.cuda.synchronize()
    print(json.dumps({"dominant_only": True, "copy_bytes_each_way": 4 * x.numel(),
                      "kernel": "k_lif_bwd_fused<32, 4, true, false, 0, true>", "launches": 3}))


def counters_workload(torch, dev):
    """Short program for counter passes (rocprofv3 --pmc) over the kernels that are not HBM-bound
    by design, each launched once or twice at its configuration: a 256 MiB copy (FETCH/WRITE
    calibration); cfg5's box scan with repair, converged (k_alif_build<4>, k_alif_carry, the
    replay k_alif_fwd<16> below MSTAR and the serial pass k_alif_fwd_pipe from it) and with the
    statistics (k_alif_repair); cfg2's map scan at C = 128, K = 8
    (k_lif_build<8,8>, k_lif_carry<8>); at cfg4: the converged forward (k_lif_fwd_warm,
    k_lif_repair_wide), the long-chunk map scan in pieces (k_lif_build<32,8>,
    k_lif_carry_wave<32>) and with the associative carry (k_map_scan), v4 at C 2048 / G 4 /
    K 32 / K2 64 and at the reference default (k_lif_compose, k_map_carry; with 1024 neurons the
    one-wave-per-neuron walks k_lif_env_lo_wave, k_map_carry_wave) and the look-back adjoint
    (k_lif_bwd_lookback<16,16,...>); with few neurons (N = 128, T = 65536): the map scan at C 256,
    K 16 (k_lif_carry_wave) and v4 at C 128, G 8 (k_lif_compose_wave)."""
    from lifscan import hip_lif as L
    from lifscan import triton_alif as A
    x = torch.empty(64 * 2 ** 20, device=dev)
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    del x, y
    torch.cuda.synchronize()
    log("counters: cfg5 box scan")
    T, N, b, r, q, C = 4096, 16384, 0.95, 0.995, 0.2, 128
    I = (0.15 + 0.3 * torch.randn(T, N, generator=torch.Generator().manual_seed(0))).to(dev)
    z = torch.zeros(N, device=dev)
    WP = A.alif_warm_predict(I, b, r, q, 1.0, 0.0, z, z, C, Wn=4)
    A.alif_scan_forward_maps(I, b, r, q, 1.0, 0.0, z, z, WP, 0.1 * q, C=C, K1=32, K2=32, BN=4, repair=10 ** 6)
    A.alif_scan_forward_maps(I, b, r, q, 1.0, 0.0, z, z, WP, 0.1 * q, C=C, K1=32, K2=32, BN=4, repair=10 ** 6,
                             stats={})
    torch.cuda.synchronize()
    del I, WP
    log("counters: cfg2 map scan")
    _, I, _ = inputs(0.9, dev)
    u0 = torch.zeros(N_CFG, device=dev)
    L.scan_forward_mapscan(I, 0.9, 1.0, 0.0, u0, C=128, K=8, repair=10 ** 6)
    torch.cuda.synchronize()
    del I
    torch.cuda.empty_cache()
    log("counters: cfg4")
    T, N = 2 ** 20, 1024
    I = (0.012 + 0.08 * torch.randn(T, N, generator=torch.Generator().manual_seed(0))).to(dev)
    u0 = torch.rand(N, generator=torch.Generator().manual_seed(2)).to(dev)
    U, S = L.scan_forward_v3(I, 0.99, 1.0, 0.0, u0, C=256, K=16, repair=10 ** 6)  # warm-started
    C2, P = L.long_sequence_plan(T, N)
    L._scan2_pieces(I, 0.99, 1.0, 0.0, u0, C2, L.LONG_K, P)
    L.scan_forward_assoc(I, 0.99, 1.0, 0.0, u0, C=2048, K=32)
    for C, G, K, K2 in ((2048, 4, 32, 64), (64, 16, 16, 32)):
        L.scan_forward_v4_maps(I, 0.99, 1.0, 0.0, u0, C=C, G=G, K=K, K2=K2, repair=10 ** 6)
        torch.cuda.synchronize()
    gS = torch.randn(T, N, generator=torch.Generator().manual_seed(1)).to(dev)
    L.scan_backward_tiled(I, u0, U, S, gS, None, 0.99, 1.0, 0.0, 4.0)
    torch.cuda.synchronize()
    del I, U, S, gS
    torch.cuda.empty_cache()
    log("counters: few neurons")
    T, N = 65536, 128
    I = (0.15 + 0.4 * torch.randn(T, N, generator=torch.Generator().manual_seed(0))).to(dev)
    u0 = torch.zeros(N, device=dev)
    L.scan_forward_mapscan(I, 0.99, 1.0, 0.0, u0, C=256, K=16, repair=0)
    L.scan_forward_v4(I, 0.99, 1.0, 0.0, u0, C=128, G=8, K=16, K2=32, repair=0)
    torch.cuda.synchronize()
    print(json.dumps({"counters_workload": True}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-cols", type=int, default=8192)
    ap.add_argument("--dominant-only", action="store_true")
    ap.add_argument("--counters-workload", action="store_true",
                    help="run each non-HBM-bound kernel once at its configuration (counter passes)")
    ap.add_argument("--headline-only", action="store_true",
                    help="skip the cfg3 / cfg4 / cfg5 / affine-reset measurements")
    ap.add_argument("--only", choices=("cfg2_mapscan", "cfg3", "cfg4", "cfg5", "affine", "auto_grid",
                                       "ceilings"),
                    help="measure one of the other configurations only (for profiling runs); "
                         "prints its JSON, not the headline line")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the exact LIF scan shards along neurons with no "
              "communication, so N GPUs give N x the one-GPU value; run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import torch
    from lifscan import hip_lif as L
    from lifscan import triton_lif as TL

    dev = torch.device("cuda:0")
    if args.dominant_only:
        dominant_only(L, torch, dev)
        return
    if args.counters_workload:
        counters_workload(torch, dev)
        return
    if args.only:
        fn = {"cfg2_mapscan": lambda torch, dev, reps: bench_cfg2_mapscan(
                  torch, L, dev, torch.zeros(N_CFG, device=dev), reps),
              "cfg3": bench_cfg3, "cfg4": bench_cfg4, "cfg5": bench_cfg5,
              "affine": bench_affine, "auto_grid": lambda torch, dev, reps: bench_auto_grid(torch, dev),
              "ceilings": lambda torch, dev, reps: hbm_ceilings(torch, dev)}[args.only]
        print(json.dumps({args.only: fn(torch, dev, 5)}))
        return
    T, N, beta, K = T_CFG, N_CFG, 0.9, 8
    I_cpu, I, gS = inputs(beta, dev)
    u0 = torch.zeros(N, device=dev)

    def step():
        Ig = I.detach().requires_grad_(True)
        S = TL.lif_tuned(Ig, u0, beta, 1.0, 0.0, 4.0, mode="scan", K=K, repair=10 ** 6)
        S.backward(gS)
        return S, Ig.grad

    log(f"warmup {args.warmup}")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    check = check_step(L, step, I, gS, u0, beta)
    log(f"timed step checked: {json.dumps(check)}")
    log(f"timing {args.steps} steps")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t0) * 1000.0 / args.steps
    value = N * T / (ms_step / 1000.0)
    log(f"fwd+bwd {ms_step:.3f} ms/step  {value / 1e9:.1f} G neuron-steps/s")

    # components (HIP events, median of 10)
    reps = 10
    ms = {}
    U, S = L.serial_forward(I, beta, 1.0, 0.0, u0)
    ms["exact_fwd_stored_U"] = ev_time(lambda: L.scan_forward_exact(I, beta, 1.0, 0.0, u0, maps=False), reps)
    ms["scan_fwd_maps_forced_C16"] = ev_time(
        lambda: L.scan_forward_exact(I, beta, 1.0, 0.0, u0, C=16, K=K, maps=True), reps)
    L.scan_forward_exact(I, beta, 1.0, 0.0, u0, C=16, K=K, maps=True)
    maps_ctr = L.last_fused_counters()
    ms["adjoint_stored_U"] = ev_time(lambda: L.scan_backward_fused(I, u0, U, S, gS, None, beta, 1.0, 0.0, 4.0), reps)
    ms["serial_fwd"] = ev_time(lambda: L.serial_forward(I, beta, 1.0, 0.0, u0), reps)
    ms["serial_bwd"] = ev_time(lambda: L.serial_backward(I, u0, U, S, gS, None, beta, 1.0, 0.0, 4.0), reps)
    del U, S
    # the recomputing pair lif_tuned runs here: S + chunk entry states, adjoint from them
    S_rc, ST = L.scan_forward_exact_starts(I, beta, 1.0, 0.0, u0)
    ms["rc_fwd"] = ev_time(lambda: L.scan_forward_exact_starts(I, beta, 1.0, 0.0, u0), reps)
    # dominant kernel: the recomputing adjoint is one launch of k_lif_bwd_fused<..., RC> per call
    t_dom = ev_time(lambda: L.scan_backward_fused_starts(I, ST, gS, beta, 1.0, 0.0, 4.0), 20)
    ms["rc_bwd"] = t_dom
    log("ms " + json.dumps({k: round(v, 4) for k, v in ms.items()}) + f" dominant {t_dom:.4f}")
    del S_rc, ST
    mapscan = bench_cfg2_mapscan(torch, L, dev, u0, reps=5)
    log("cfg2 map scan " + json.dumps(mapscan))

    achieved = B_BWD_RC * N * T / (t_dom / 1000.0) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": profiled_traffic(),
                "traffic_source": "profiles/k_lif_bwd_fused_rc_cfg2_traffic.txt (rocprofv3 --pmc "
                                  "FETCH_SIZE, WRITE_SIZE; bytes per launch)",
                "kernel": "k_lif_bwd_fused<32, 4, true, false, 0, true> (single-pass adjoint "
                          "recomputing each chunk from its entry state)",
                "algorithmic_bytes_per_launch": B_BWD_RC * N * T, "avg_launch_ms": round(t_dom, 4)}

    others = None
    if not args.headline_only:
        del I
        torch.cuda.empty_cache()
        others = {}
        for name, fn in (("cfg3", bench_cfg3), ("cfg5", bench_cfg5), ("cfg4", bench_cfg4),
                         ("affine", bench_affine),
                         ("auto_grid", lambda torch, dev, reps: bench_auto_grid(torch, dev))):
            log(f"{name}")
            others[name] = fn(torch, dev, 5)
            log(f"{name} " + json.dumps(others[name]))
    ceilings = hbm_ceilings(torch, dev)
    log("hbm ceilings " + json.dumps(ceilings))

    cpu = None
    if not args.no_cpu:
        log(f"cpu baseline on {args.cpu_cols} neurons x T={T}")
        r = cpu_baseline(I_cpu, beta, args.cpu_cols)
        nsteps = args.cpu_cols * T
        cpu = {"value": round(nsteps / r["scan"], 1), "unit": "neuron-steps/s",
               "cores": torch.get_num_threads(), "kind": "port",
               "sample": f"fast.py two-level pruned scan fwd (C=64,K=8,repair on) + Hillis-Steele "
                         f"affine-scan bwd on {args.cpu_cols} of {N} neurons x T={T}, median of 3",
               "serial_fwd_bwd_value": round(nsteps / r["serial"], 1),
               "os_cpu_count": os.cpu_count(), "cpu_model": cpu_model()}

    pct = lambda b, t: round(100 * b * N * T / (t / 1000.0) / 1e9 / HBM_PEAK_GBS, 2)
    stored_u = {"fwd_bwd_ms": round(ms["exact_fwd_stored_U"] + ms["adjoint_stored_U"], 4),
                "pct_roofline_fwd_bwd": pct(B_FWD + B_BWD, ms["exact_fwd_stored_U"] + ms["adjoint_stored_U"]),
                "pct_roofline_fwd": pct(B_FWD, ms["exact_fwd_stored_U"]),
                "pct_roofline_bwd": pct(B_BWD, ms["adjoint_stored_U"]),
                "bytes_per_neuron_step": B_FWD + B_BWD}
    summary = compact_summary(value, ms_step, pct(B_FWD_RC + B_BWD_RC, ms_step), stored_u, mapscan,
                              others, ceilings)
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
        "data": "synthetic (seeded CPU generator: x~N(0.12,0.25^2), gS~N(0,1))",
        "config": {"workload": "cfg2: lif_tuned(I, u0, beta, mode='scan', K=8, repair=1e6) forward + "
                               "backward through autograd at N=65536 (256x256), T=4096, beta=0.9, "
                               "theta=1, u_r=0, u0=0.  Kernels that run: forward "
                               "k_lif_fwd_fused<1,32,4,SPEC=false,SO=true> (exact single pass: 32-step "
                               "chunks handed on wave to wave, no chunk maps, K unused; writes S and "
                               "the chunk entry states), adjoint k_lif_bwd_fused<32,4,...,RC=true> "
                               "(single-pass affine-scan adjoint replaying each chunk from its entry "
                               "state).  The map scan (C=32..128, K=8) is measured in cfg2_mapscan.",
                   "N": N, "T": T, "beta": beta, "internal_chunk": L.FUSED_FWD_C, "maps": False},
        "bytes_per_neuron_step": B_FWD_RC + B_BWD_RC,
        "roofline_basis": "20 B per neuron-step, the bytes the recomputing pair moves (fwd: read I, "
                          "write S and 1/32 row of entry states; bwd: read I, gS, write dI).  The "
                          "32 B basis of the stored path counts U written and re-read, which "
                          "lif_tuned never exposes: "
                          "on that basis this step would be above the HBM peak; the stored-U passes "
                          "are reported on it in stored_U_path",
        "pct_roofline_fwd_bwd": pct(B_FWD_RC + B_BWD_RC, ms_step),
        "fwd_value": round(N * T / (ms["rc_fwd"] / 1000.0), 1),
        "pct_roofline_fwd": pct(B_FWD_RC, ms["rc_fwd"]),
        "pct_roofline_bwd": pct(B_BWD_RC, ms["rc_bwd"]),
        "timed_step_check": check,
        "summary": summary,
        "stored_U_path": stored_u,
        "hbm_ceilings": ceilings,
        "ms": {k: round(v, 4) for k, v in ms.items()},
        "serial_hip_fwd_bwd_value": round(N * T / ((ms["serial_fwd"] + ms["serial_bwd"]) / 1000.0), 1),
        "maps_forced_counters": maps_ctr,
        "cfg2_mapscan": mapscan,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "other_configs": others,
    }
    print(json.dumps(out))
    sys.stdout.flush()
    log("summary " + json.dumps(summary, separators=(",", ":")))


def compact_summary(value, ms_step, pct_step, stored_u, mapscan, others, ceilings):
    """The figures a reader of the run's tail needs, in one short object: the headline, the
    stored-U pair on the 32 B basis, the six configs[1] map-scan cells (ms, % of the 12 B
    roofline, overflow fraction, equal to serial), cfg3 / cfg4 / cfg5's headline figures (cfg3 and
    cfg5 back to back and cache-cold), the auto grid and the HBM ceilings."""
    sm = {"headline": {"value": round(value, 1), "ms": round(ms_step, 4), "pct_20B": pct_step},
          "stored_U": {"ms": stored_u["fwd_bwd_ms"], "pct_32B": stored_u["pct_roofline_fwd_bwd"]},
          "cfg2_mapscan": {f"b{b}_C{C}": [c["ms"], c["pct_roofline_12B"], c["overflow_frac"],
                                          c["equals_serial"]]
                           for b in (0.9, 0.99) for C in (32, 64, 128)
                           for c in (mapscan[f"beta{b}"][f"C{C}_K8"],)},
          "ceilings_GBps": [ceilings["copy_GBps"], ceilings["fill_GBps"]]}
    if others:
        c3, c4, c5, ag = others["cfg3"], others["cfg4"], others["cfg5"], others["auto_grid"]
        v4 = c4["v4"]
        sm["cfg3"] = {"layers_ms": c3["lif_layers_fwd_bwd_ms"], "layers_cold_ms": c3["lif_layers_fwd_bwd_cold_ms"],
                      "pct_cold": c3["lif_layers_pct_roofline_cold"], "step_ms_scan": c3["step_ms_scan"]}
        sm["cfg4"] = {"fwd_bwd_ms": c4["fwd_bwd_ms"], "pct": c4["pct_roofline_fwd_bwd"],
                      "v4_ms": {k: [r["ms"], r["equals_serial"]] for k, r in v4.items()},
                      "assoc_vs_seq_ms": {k: r["ms"] for k, r in c4["mapscan_converged"].items()}}
        box = c5["box_scan_repair"]
        sm["cfg5"] = {"fwd_bwd_ms": c5["alif_fwd_serial_bwd_scan_ms"],
                      "fwd_bwd_cold_ms": c5["alif_fwd_serial_bwd_scan_cold_ms"],
                      "pct_cold": c5["pct_roofline_fwd_bwd_cold"],
                      "serial_fwd_cold_GBps": c5["serial_fwd_cold_GBps"],
                      "box_scan_ms": {k: [r["ms"], r["ms_cold"], r["equals_serial"]] for k, r in box.items()},
                      "box_converged_dispatch_ms": c5["box_scan_converged_dispatch"]["ms"],
                      "ref_shape_box_repair_ms": c5["reference_shape"]["fwd_box_scan_repair_ms"],
                      "ref_shape_serial_ms": c5["reference_shape"]["fwd_serial_ms"],
                      "N16_box_ms": c5["reference_shape"]["few_neurons"]["N16"]["fwd_box_scan_no_repair_ms"]}
        sm["auto_grid"] = {"worst_auto_vs_best": ag["worst_auto_vs_best"],
                           "within_5pct": f'{ag["cells_within_5pct"]}/{ag["n_cells"]}',
                           "spikes_equal": ag["all_spikes_equal"]}
    return sm


if __name__ == "__main__":
    main()
