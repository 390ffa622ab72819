"""
Wide-forward throughput of the MI355X build on one GPU.

Workload (the configuration the headline metric is quoted on): WideGRU over N=32
nn.GRU(64 -> 128, batch_first) models, x [32, 4, 32, 64] ~ N(0, 1) fp32, h0 = 0.  One
step = one wide forward (input-projection GEMM + persistent recurrence) over that batch,
inputs resident in HBM.  Prints ONE JSON line.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--mode graph|eager] [--no-cpu]

* value: samples/s = N*B*K / wall time of K steps (torch.cuda.synchronize on both sides).
  --mode graph (default) replays the forward as one captured HIP graph per step; eager
  calls the module from Python each step (both are reported).
* roofline: the recurrence kernel (dominant) -- algorithmic flops per launch
  2*N*B*T*3H*H over its average duration, timed with HIP events on the launch stream;
  peak = MI355X dense fp32 MFMA 157.3 TFLOP/s.
* cpu_baseline: the oracle (op-for-op CPU restatement of the reference wide path, torch CPU
  ops) on the host cores, over a bounded number of full forwards.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "pytorch-parallel-compiler_amd"))
sys.path.insert(0, ROOT)

METRIC = "wide fwd samples/sec (N×B) at 1 MI355X; % of MFMA / HBM roofline"
PEAK_FP32_MFMA = 157.3e12  # FLOP/s, MI355X dense fp32 matrix
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "rnn_recurrence_gru_n32.traffic.json")


def _cpu_baseline(work, seconds: float):
    import torch
    from oracle import wide_ref

    threads = min(16, os.cpu_count() or 1)
    torch.set_num_threads(threads)
    mods = work.models
    p = [torch.stack([getattr(m, k).detach().float() for m in mods])
         for k in ("weight_ih_l0", "weight_hh_l0", "bias_ih_l0", "bias_hh_l0")]
    x = work.inputs["x"]
    with torch.inference_mode():
        for _ in range(2):
            wide_ref.gru(x, *p)
        iters, t0 = 0, time.perf_counter()
        while True:
            wide_ref.gru(x, *p)
            iters += 1
            el = time.perf_counter() - t0
            if (el >= seconds and iters >= 3) or iters >= 100000:
                break
    return {"value": work.n * work.batch * iters / el, "unit": "samples/s", "cores": threads, "kind": "port",
            "sample": f"{iters} full forwards of the same workload (oracle GRU restatement, torch CPU, "
                      f"fp32, {threads} threads), {el:.1f} s"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--mode", choices=("graph", "eager"), default="graph")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested)", file=sys.stderr)
        return 2

    import torch
    import wide_compiler as wc
    from wide_compiler import _hip, workloads

    dev = torch.device("cuda", 0)
    work = workloads.gru_n32()
    n, b = work.n, work.batch
    x_cpu = work.inputs["x"]
    _, _, t, i = x_cpu.shape
    h = work.models[0].hidden_size
    wide = wc.WideGRU.from_modules(work.models).to(dev).eval()
    x = x_cpu.to(dev)

    # ---- parity of the measured path against the oracle (float64) ----
    from oracle import wide_ref
    with torch.inference_mode():
        out, _ = wide(x)
    p64 = [getattr(wide, k).detach().cpu().double() for k in ("weight_ih", "weight_hh", "bias_ih", "bias_hh")]
    ref, _ = wide_ref.gru(x_cpu.double(), *p64)
    parity = ((out.cpu().double() - ref).abs().max() / ref.abs().max()).item()

    def step():
        return wide(x)

    def timed(fn, k, w):
        with torch.inference_mode():
            for _ in range(w):
                fn()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(k):
                fn()
            torch.cuda.synchronize()
            return time.perf_counter() - t0

    eager_s = timed(step, args.steps, args.warmup)
    graph_s = None
    if args.mode == "graph":
        with torch.inference_mode():
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                for _ in range(3):
                    step()
            torch.cuda.current_stream().wait_stream(s)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                static_out = step()
        graph_s = timed(graph.replay, args.steps, args.warmup)
        with torch.inference_mode():
            torch.cuda.synchronize()
            g_err = ((static_out[0].cpu().double() - ref).abs().max() / ref.abs().max()).item()
        parity = max(parity, g_err)
    wall = graph_s if graph_s is not None else eager_s

    # ---- per-kernel durations with HIP events on the launch stream ----
    with torch.inference_mode():
        o = torch.empty((n, b, t, h), device=dev)
        hn = torch.empty((n, b, h), device=dev)
        a, ws = _hip.rnn_args(cell=_hip.CELL_GRU, x=x, w_ih=wide.weight_ih, w_hh=wide.weight_hh,
                              b_ih=wide.bias_ih, b_hh=wide.bias_hh, h0=None, c0=None, out=o, h_n=hn, c_n=None)
        kt = {}
        for phase in ("input_projection", "recurrence"):
            for _ in range(args.warmup):
                _hip.rnn_phase(a, phase, x)
            st = torch.cuda.current_stream()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(st)
            for _ in range(args.steps):
                _hip.rnn_phase(a, phase, x)
            e1.record(st)
            e1.synchronize()
            kt[phase] = e0.elapsed_time(e1) / args.steps * 1e-3  # seconds per launch
    flops_rec = 2.0 * n * b * t * 3 * h * h
    flops_proj = 2.0 * n * b * t * 3 * h * i
    achieved = flops_rec / kt["recurrence"]
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get("bytes_per_launch")

    cpu = None if args.no_cpu else _cpu_baseline(work, args.cpu_seconds)

    line = {
        "metric": METRIC,
        "value": n * b * args.steps / wall,
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall / args.steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded torch.nn default init, x ~ N(0,1))",
        "config": {"workload": work.name, "n_models": n, "batch": b, "seq_len": t, "input_size": i,
                   "hidden": h, "mode": args.mode},
        "roofline": {"bound": "mfma", "achieved": achieved / 1e12, "peak": PEAK_FP32_MFMA / 1e12,
                     "unit": "TFLOP/s", "frac": achieved / PEAK_FP32_MFMA, "traffic": traffic,
                     "kernel": "rnn_seq_kernel (recurrence)", "flops_per_launch": flops_rec,
                     "us_per_launch": kt["recurrence"] * 1e6},
        "kernels_us": {"input_projection_gemm": kt["input_projection"] * 1e6,
                       "recurrence": kt["recurrence"] * 1e6,
                       "input_projection_tflops": flops_proj / kt["input_projection"] / 1e12},
        "eager_samples_per_s": n * b * args.steps / eager_s,
        "graph_samples_per_s": None if graph_s is None else n * b * args.steps / graph_s,
        "parity_rel_err_vs_oracle": parity,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
