"""Benchmark of the torchwarp alignment hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--config cfg2] [--all] [--no-cpu] [--eager]
    python bench.py --copy-probe      # HBM counter calibration: 5 copies of 256 MiB

A "step" is one forward + loss + backward of the configured alignment loss on
synthetic inputs already resident in HBM (inputs are
drawn from a CPU ``torch.Generator().manual_seed(0)`` in config order, then
moved to the GPU). The headline workload is configs[1]: uDTW fp32 fwd+bwd,
B=256, N=M=140, D=1 -- metric "DP cells/s" (N*M*B per step / step time).

The step goes through the public API. It is captured once as a HIP graph and
the timed steps are graph replays, so the figure is the GPU's, not the host's:
an eager step costs 0.1-0.2 ms of Python and autograd-engine work on the host,
as much as the kernels. The eager step is timed beside it
(``config.eager_ms_per_step``); ``--eager`` makes it the headline.

One JSON line is printed with ``roofline`` for the dominant kernel (algorithmic
bytes per launch / its mean duration, timed with HIP events on the stream the
kernel runs on) and ``cpu_baseline`` (the CPU oracle, the clean-room
restatement of the reference's vectorised PyTorch backend, timed on this
host on a bounded sample). The metric has two halves; the second, JEANIE
with two viewpoint axes (K = 25, configs[4]), is measured in the same run and
reported in the same line as ``config.jeanie_k25`` with its own roofline and
CPU baseline. ``--all`` adds one line per config to stderr.
"""

import argparse
import json
import os
import sys
import time

import torch

HBM_PEAK_GBS = 8000.0
METRIC = ("DP cells/sec & pairs/sec fwd+bwd (uDTW B=256 N=M=140; JEANIE K=25), "
          "% HBM roofline")
SETTLE_S = 0.25    # minimum untimed warm-up per config (seconds)
LAST_TIMES = {}   # label -> mean ms of every kernel timed by the last _hip_call_times
EAGER_MS = {}     # config -> ms per eagerly run step (run_config with mode "eager"/"both")
CONFIGS = ("cfg1", "cfg2", "cfg3", "cfg4", "cfg5a", "cfg5b", "cost", "cost_band", "cfg3_band")
# The cost-path workloads beside the BASELINE configs: uDTW on precomputed
# matrices, B = 64, N = M = 1024, gamma = 1, without a band ("cost") and with
# a Sakoe-Chiba band of 102 ("cost_band", the banded sweep; its cells are the
# band's cells). "cfg3_band": cfg3's features with the same band (the banded
# feature path; its cells are the band's cells).
BAND = 102


# ------------------------------------------------------------------ inputs

def _walk(g, B, L):
    x = torch.cumsum(0.1 * torch.randn(B, L, 1, generator=g), 1)
    return (x - x.mean(1, keepdim=True)) / x.std(1, keepdim=True)


def make_inputs(name, device="cpu", dtype=torch.float32):
    """Synthetic inputs of one BASELINE config (seed 0, drawn in config order)."""
    g = torch.Generator().manual_seed(0)
    if name == "cfg1":
        t = (torch.randn(32, 64, 1, generator=g), torch.randn(32, 64, 1, generator=g))
    elif name == "cfg2":
        X, Y = _walk(g, 256, 140), _walk(g, 256, 140)
        sx, sy = 0.5 + torch.rand(256, 140, 1, generator=g), 0.5 + torch.rand(256, 140, 1, generator=g)
        t = (X, Y, sx, sy)
    elif name in ("cfg3", "cfg3_band"):
        X, Y = torch.randn(64, 1024, 16, generator=g), torch.randn(64, 1024, 16, generator=g)
        sx, sy = 0.5 + torch.rand(64, 1024, 1, generator=g), 0.5 + torch.rand(64, 1024, 1, generator=g)
        t = (X, Y, sx, sy)
    elif name == "cfg4":
        q = torch.nn.functional.normalize(torch.randn(400, 9, 8, 256, generator=g), dim=-1)
        s = torch.nn.functional.normalize(torch.randn(400, 8, 256, generator=g), dim=-1)
        t = (q, s)
    elif name in ("cfg5a", "cfg5b"):
        t = (4.0 * torch.rand(1024, 25, 16, 16, generator=g),)
    elif name in ("cost", "cost_band"):
        t = (torch.rand(64, 1024, 1024, generator=g), 0.1 * torch.rand(64, 1024, 1024, generator=g))
    else:
        raise ValueError(name)
    return tuple(x.to(device=device, dtype=dtype) for x in t)


# Work units and algorithmic HBM bytes per fwd+bwd (fp32), BASELINE.md table:
# inputs read once per pass, outputs written once, carried tensors (R, P)
# written once and read once.
def work(name):
    return {
        "cfg1": dict(cells=32 * 64 * 64, pairs=32),
        "cfg2": dict(cells=256 * 140 * 140, pairs=256),
        "cfg3": dict(cells=64 * 1024 * 1024, pairs=64),
        "cfg4": dict(cells=400 * 9 * 8 * 8, pairs=400),
        "cfg5a": dict(cells=1024 * 25 * 16 * 16, pairs=1024),
        "cfg5b": dict(cells=1024 * 16 * 16, pairs=1024),
        "cost": dict(cells=64 * 1024 * 1024, pairs=64),
        "cost_band": dict(cells=64 * (1024 * (2 * BAND + 1) - BAND * (BAND + 1)), pairs=64),
        "cfg3_band": dict(cells=64 * (1024 * (2 * BAND + 1) - BAND * (BAND + 1)), pairs=64),
    }[name]


def step_fn(name, inputs):
    """One forward + loss + backward through the public API."""
    import torchwarp_amd as tw
    import torchwarp_amd.functional as TF

    if name == "cfg1":
        m = tw.SoftDTW(gamma=1.0)
        X, Y = inputs

        def f():
            x = X.detach().requires_grad_(True)
            m(x, Y).mean().backward()
        return f
    if name in ("cfg2", "cfg3", "cfg3_band"):
        gamma = 1.0 if name == "cfg2" else 0.1
        m = tw.UDTW(gamma=gamma, beta=1.0, bandwidth=BAND if name == "cfg3_band" else None)
        X, Y, sx, sy = inputs

        def f():
            xs = [t.detach().requires_grad_(True) for t in (X, Y, sx, sy)]
            d, p = m(*xs)
            (d + p).mean().backward()
        return f
    if name in ("cost", "cost_band"):
        C, Q = inputs
        band = BAND if name == "cost_band" else None

        def f():
            c, q = C.detach().requires_grad_(True), Q.detach().requires_grad_(True)
            d, p = TF.udtw_from_cost(c, q, gamma=1.0, bandwidth=band)
            (d + p).mean().backward()
        return f
    if name == "cfg4":
        q, s = inputs

        def f():
            qq, ss = q.detach().requires_grad_(True), s.detach().requires_grad_(True)
            TF.jeanie(qq, ss, gamma=0.1, max_shift=1).mean().backward()
        return f
    (c,) = inputs
    if name == "cfg5a":
        def f():
            cc = c.detach().view(1024, 5, 5, 16, 16).requires_grad_(True)
            TF.jeanie_from_cost(cc, gamma=0.1, max_shift=1).mean().backward()
        return f

    def f():
        cc = c.detach().requires_grad_(True)
        TF.fvm_from_cost(cc, gamma=0.1).mean().backward()
    return f


# ------------------------------------------------------------- kernel timing

def _hip_call_times(name, inputs, iters):
    """Mean durations (ms) of the forward and backward DP launches of one config,
    called through the C ABI and bracketed by HIP events on the same stream.
    Returns (label, mean_ms, algorithmic_bytes_per_launch) for the dominant one."""
    from torchwarp_amd import _hip
    dev = inputs[0].device
    stream = torch.cuda.current_stream(dev)
    f32 = torch.float32
    calls = []
    if name in ("cfg1", "cfg2", "cfg3", "cfg3_band"):
        # standard deviations, squared inside the kernels (as the public API calls them)
        if name == "cfg1":
            X, Y = inputs
            vx = torch.ones(X.shape[:2], device=dev)
            vy = torch.ones(Y.shape[:2], device=dev)
            beta, gamma = 0.0, 1.0
        else:
            X, Y, sx, sy = inputs
            vx, vy = sx.squeeze(-1), sy.squeeze(-1)
            beta, gamma = 1.0, (1.0 if name == "cfg2" else 0.1)
        B, N, D = X.shape
        M = Y.shape[1]
        pen = beta != 0
        band = float(BAND) if name == "cfg3_band" else 0.0
        R = X.new_empty(B, _hip.carry_cols(N, M, gamma, X.dtype))
        P = X.new_empty(B, N * M) if pen else None
        o1, o2 = X.new_empty(B), X.new_empty(B)
        nws = _hip.udtw_workspace_elems(B, N, M, D, X.dtype)
        ws = X.new_empty(nws) if nws else None
        wsb = 0 if ws is None else nws * 4
        g = torch.full((B,), 1.0 / B, device=dev)
        dX, dY, dvx, dvy = [torch.empty_like(t) for t in (X, Y, vx, vy)]
        io = 4 * (X.numel() + Y.numel() + vx.numel() + vy.numel())
        # R and P at 4 B/cell each (fp32); where the kernels keep R in double
        # precision (long sequences, small gamma) its extra 4 B/cell count as
        # overhead, not as algorithmic bytes
        # (with a band: of the band's cells)
        carried = 4 * work(name)["cells"] * (2 if pen else 1)
        # the banded path's backward reads the forward's band planes, as the
        # public API passes them (fwd_ws)
        fwd_ws = X.new_empty(nws) if band > 0 else None
        bwd_ws = ws if fwd_ws is None else X.new_empty(nws)
        calls.append(("udtw_fwd", lambda: _hip.call(
            "tw_udtw_feat_fwd", f32, X, Y, vx, vy, B, N, M, D, gamma, beta, 1e-8, band, 1, R, P,
            o1, o2, ws if fwd_ws is None else fwd_ws, wsb), io + carried))
        calls.append(("udtw_bwd", lambda: _hip.call(
            "tw_udtw_feat_bwd", f32, X, Y, vx, vy, R, P, g, g if pen else None, B, N, M, D, gamma,
            beta, 1e-8, band, 1, 1, dX, dY, dvx, dvy, fwd_ws, bwd_ws, wsb), 2 * io + carried))
    elif name in ("cost", "cost_band"):
        C, Q = inputs
        B, N, M = C.shape
        band = float(BAND) if name == "cost_band" else 0.0
        R = C.new_empty(B, _hip.carry_cols(N, M, 1.0, C.dtype))
        P = C.new_empty(B, N * M)
        o1, o2 = C.new_empty(B), C.new_empty(B)
        nws = _hip.udtw_cost_workspace_elems(B, N, M, C.dtype, band)
        ws = C.new_empty(nws) if nws else None
        wsb = 0 if ws is None else nws * 4
        g = torch.full((B,), 1.0 / B, device=dev)
        dC, dQ = torch.empty_like(C), torch.empty_like(Q)
        # the cells the sweep visits: C, Q read and R, P written (forward),
        # R, P read (backward) at 4 B each; the gradients are written in full
        # (zero outside the band)
        cells = work(name)["cells"]
        calls.append(("udtw_fwd", lambda: _hip.call(
            "tw_udtw_cost_fwd", f32, C, Q, B, N, M, 1.0, band, R, P, o1, o2), 16 * cells))
        calls.append(("udtw_bwd", lambda: _hip.call(
            "tw_udtw_cost_bwd", f32, C, Q, R, P, g, g, B, N, M, 1.0, band, 1, dC, dQ, ws, wsb),
            8 * cells + 8 * B * N * M))
    elif name == "cfg5a":
        (c,) = inputs
        B = c.shape[0]
        R, out = torch.empty_like(c), c.new_empty(B)
        dC = torch.empty_like(c)
        g = torch.full((B,), 1.0 / B, device=dev)
        nb = 4 * c.numel()
        calls.append(("jeanie_fwd", lambda: _hip.call(
            "tw_jeanie_cost_fwd", f32, c, B, 5, 5, 16, 16, 0, 1, 1, 0.1, R, out), 2 * nb))
        calls.append(("jeanie_bwd", lambda: _hip.call(
            "tw_jeanie_cost_bwd", f32, c, R, g, None, B, 5, 5, 16, 16, 0, 1, 1, 0.1, dC), 3 * nb))
    else:
        return None
    best = None
    LAST_TIMES.clear()
    for label, fn, nbytes in calls:
        fn()
        torch.cuda.synchronize(dev)
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record(stream)
        for _ in range(iters):
            fn()
        ev1.record(stream)
        torch.cuda.synchronize(dev)
        ms = ev0.elapsed_time(ev1) / iters
        LAST_TIMES[label] = ms
        if best is None or ms > best[1]:
            best = (label, ms, nbytes)
    return best


def _roofline(name, inputs, iters):
    """Roofline record of a config's dominant DP kernel, or None."""
    kt = _hip_call_times(name, inputs, iters)
    if kt is None:
        return None
    label, kms, nbytes = kt
    gbs = nbytes / (kms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 5), "traffic": _traffic(label, name),
            "kernel": label, "kernel_ms": round(kms, 5), "algorithmic_bytes": nbytes}


def _traffic(label, name):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, if any."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        with open(path) as fh:
            return json.load(fh).get("{}/{}".format(label, name))
    except (OSError, ValueError):
        return None


# --------------------------------------------------------------- CPU oracle

def cpu_baseline(name, budget_s=10.0):
    """The CPU oracle (restatement of the reference's vectorised PyTorch
    backend) timed on this host, fp32, on the full config batch repeated
    until ~budget_s of work; returns cells/s."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import jeanie as OJ, udtw as OU
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    inp = make_inputs(name)
    w = work(name)

    def once():
        if name == "cfg3_band":
            # a bounded sample: 2 of the 64 pairs (cells scaled below)
            X, Y, sx, sy = (t[:2].clone().requires_grad_(True) for t in inp)
            d, p = OU.udtw(X, Y, sx, sy, gamma=0.1, beta=1.0, bandwidth=BAND)
            (d + p).sum().backward()
        elif name in ("cfg1", "cfg2", "cfg3"):
            if name == "cfg1":
                X, Y = inp
                vx = torch.ones(X.shape[:2])
                vy = torch.ones(Y.shape[:2])
                beta, gamma = 0.0, 1.0
            else:
                X, Y, sx, sy = inp
                vx, vy = sx.squeeze(-1) ** 2, sy.squeeze(-1) ** 2
                beta, gamma = 1.0, (1.0 if name == "cfg2" else 0.1)
            B = X.shape[0]
            r, p, R, P = OU.features_forward(X, Y, vx, vy, gamma, beta, 1e-8)
            g = torch.full((B,), 1.0 / B)
            OU.features_backward(X, Y, vx, vy, R, P, g, g, gamma, beta, 1e-8)
        elif name == "cfg5a":
            c = inp[0].view(1024, 5, 5, 16, 16)
            out, R = OJ.forward(c, 1, 1, 0.1)
            OJ.backward(c, R, torch.full((1024,), 1 / 1024), 1, 1, 0.1)
        elif name == "cfg5b":
            OJ.fvm_backward(inp[0], torch.full((1024,), 1 / 1024), 0.1)
        elif name in ("cost", "cost_band"):
            # a bounded sample: 2 of the 64 pairs (cells scaled below)
            C, Q = (t[:2].clone().requires_grad_(True) for t in inp)
            d, p = OU.udtw_from_cost(C, Q, gamma=1.0,
                                     bandwidth=BAND if name == "cost_band" else None)
            (d + p).sum().backward()
        else:
            q, s = inp
            c = OJ.euclidean_cost(q.requires_grad_(True), s.requires_grad_(True))
            OJ.jeanie_from_cost(c, gamma=0.1, max_shift=1).mean().backward()

    once()
    n, t0 = 0, time.perf_counter()
    while True:
        once()
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 50:
            break
    share = 2 / 64 if name in ("cost", "cost_band", "cfg3_band") else 1.0   # pairs run
    return {"value": w["cells"] * share * n / el, "unit": "cells/s", "cores": cores,
            "kind": "port", "cpu_model": _cpu_model(),
            "pairs_per_s": w["pairs"] * share * n / el,
            "sample": "{}: {} fwd+bwd x{} in {:.1f} s, fp32, oracle/ on {} threads"
                      .format(name, "full batch" if share == 1.0 else "2 pairs", n, el, cores)}


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


# -------------------------------------------------------------------- main

def graphed(f, dev):
    """The step ``f`` captured once as a HIP graph (torch.cuda.graph); returns
    its replay. A replay launches every kernel of the eager step -- forward,
    loss, backward -- on the same device-resident inputs, with the host's
    per-step Python and autograd-engine work taken out of the loop. The
    library allocates nothing, synchronises nothing and records no memset,
    so the step captures as is (tests/test_gpu_graph.py checks replays
    against eager steps)."""
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        for _ in range(3):
            f()
    torch.cuda.current_stream(dev).wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        f()
    torch.cuda.synchronize(dev)
    return g.replay


def _time_steps(f, dev, steps, warmup):
    """ms per step of ``f`` over exactly ``steps`` steps, bracketed by
    synchronisations, after ``warmup`` untimed steps (continued until at least
    SETTLE_S seconds have passed, so the GPU's clocks have left their idle
    state before the timed steps)."""
    t_w = time.perf_counter()
    n = 0
    while n < warmup or time.perf_counter() - t_w < SETTLE_S:
        f()
        n += 1
        if n % 8 == 0:
            torch.cuda.synchronize(dev)
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    for _ in range(steps):
        f()
    torch.cuda.synchronize(dev)
    return (time.perf_counter() - t0) * 1e3 / steps


def run_config(name, steps, warmup, mode="graph"):
    """Time one config: ``mode`` "graph" replays the captured step, "eager"
    runs it through Python and the autograd engine every time, "both" times
    both (the graph figure is returned, the eager one in ``EAGER_MS``)."""
    dev = torch.device("cuda", 0)
    inputs = make_inputs(name, dev)
    f = step_fn(name, inputs)
    if mode in ("eager", "both"):
        EAGER_MS[name] = _time_steps(f, dev, steps, warmup)
    ms = EAGER_MS[name] if mode == "eager" else _time_steps(graphed(f, dev), dev, steps, warmup)
    w = work(name)
    return inputs, ms, w["cells"] / (ms * 1e-3), w["pairs"] / (ms * 1e-3)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="cfg2", choices=CONFIGS)
    ap.add_argument("--all", action="store_true", help="also time every config (stderr)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--eager", action="store_true",
                    help="time eager steps only (default: graph replays, eager timed beside)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run 5 device copies of 256 MiB (calibrates FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()
    if args.copy_probe:
        src = torch.ones(64 << 20, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes_read": src.numel() * 4,
                          "copy_probe_bytes_written": dst.numel() * 4, "launches": 5}))
        return
    if args.gpus != 1:
        print("bench.py: this build measures one GPU; pairs are independent, so N GPUs would "
              "each run this same per-GPU workload on B/N pairs (no collective inside the op). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    name = args.config
    mode = "eager" if args.eager else "both"
    inputs, ms, cells_s, pairs_s = run_config(name, args.steps, args.warmup, mode)
    roof = _roofline(name, inputs, max(args.steps, 10))
    # The metric's second half: JEANIE with two viewpoint axes, K = 25
    # (configs[4], the 5 x 5 cost fwd+bwd), measured the same way.
    second = None
    if name != "cfg5a":
        j_in, j_ms, j_cells, j_pairs = run_config("cfg5a", args.steps, args.warmup, mode)
        second = {"workload": "cfg5a", "metric": "JEANIE K=25 fwd+bwd, cells/s",
                  "value": round(j_cells, 1), "unit": "cells/s", "ms_per_step": round(j_ms, 5),
                  "pairs_per_s": round(j_pairs, 1), "cells": work("cfg5a")["cells"],
                  "pairs": work("cfg5a")["pairs"],
                  "eager_ms_per_step": round(EAGER_MS["cfg5a"], 5),
                  "roofline": _roofline("cfg5a", j_in, max(args.steps, 10)),
                  "cpu_baseline": None if args.no_cpu else cpu_baseline("cfg5a", 8.0)}
    line = {
        "metric": METRIC,
        "value": round(cells_s, 1),
        "unit": "cells/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": name, "pairs_per_s": round(pairs_s, 1), "cells": work(name)["cells"],
                   "pairs": work(name)["pairs"],
                   "timing": ("eager steps" if args.eager else
                              "HIP-graph replays of the public-API step (forward, loss, backward)"),
                   "eager_ms_per_step": round(EAGER_MS[name], 5),
                   "jeanie_k25": second},
        "roofline": roof,
        "cpu_baseline": None if args.no_cpu else cpu_baseline(name),
    }
    print(json.dumps(line), flush=True)
    if args.all:
        for other in CONFIGS:
            inp, oms, oc, op = run_config(other, max(10, args.steps), 2, mode)
            kt = _hip_call_times(other, inp, 10)
            rec = {"config": other, "ms_per_step": round(oms, 4), "cells_per_s": round(oc, 1),
                   "pairs_per_s": round(op, 1), "eager_ms_per_step": round(EAGER_MS[other], 4)}
            if kt is not None:
                rec.update(kernel=kt[0], kernel_ms=round(kt[1], 5),
                           hbm_frac=round(kt[2] / (kt[1] * 1e-3) / 1e9 / HBM_PEAK_GBS, 5))
            print(json.dumps(rec), file=sys.stderr, flush=True)


if __name__ == "__main__":
    main()
