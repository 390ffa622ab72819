"""
Wide-forward throughput of the MI355X build on one GPU.  Prints ONE JSON line.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--config NAME] [--mode best|graph|eager]
                  [--no-cpu] [--cpu-seconds S] [--no-extra]

Default workload (the largest single-GPU configuration): N=64 sequence models, each
Embedding(8192, 256) - LayerNorm(256) - LSTM(256 -> 512) - Linear(512 -> 8192), bf16 weights,
ids [64, 16, 128] uniform in [0, 8192).  --config selects another configuration as the headline
(mlp, gru, resblock, attention, groupnorm); the others are reported under "configs".

* step  = one wide forward over one batch, inputs already resident in HBM.
* value = samples/s = N*B*K / wall time of K steps, bracketed by torch.cuda.synchronize().
  Two ways to run a step are timed: graph replays the forward as one captured HIP graph per
  step; eager calls the module from Python (kernel launches queue asynchronously).  --mode
  best (default) reports the faster of the two as value; both rates are in the line.
* roofline = the kernel with the largest share of the step's GPU time: algorithmic flops (or
  bytes) per launch divided by its average duration, timed with HIP events around a graph of
  back-to-back launches on the stream they run on; "kernels" lists every kernel of the step
  with its own fraction.  Peaks are MI355X datasheet values (dense MFMA fp32 157.3 TFLOP/s,
  bf16 2516.6 TFLOP/s; HBM 8 TB/s).  "traffic" is the counter-measured HBM bytes per launch
  of that kernel (profiles/traffic_<config>.json) when one was recorded for it.
* configs = the other configurations (value, ms per step, dominant kernel and its fraction),
  plus "pack": the boundary pack and transpose kernels in GB/s.  Each is timed like the headline
  but with at least 50 ms of untimed warm-up steps and at least 30 ms of timed steps (more than
  K / W when its steps are short: the shader clock takes ~25 ms of work to ramp up after the
  idle set-up); the step counts used are in its entry.
* cache regimes: per-step GPU times (HIP events around each step, in the mode used) over K
  steps, median reported hot (steps back to back) and cold (a 512 MiB buffer rewritten before
  every step, so the 256 MB Infinity Cache and the L2s hold none of the step's data).
* cpu_baseline = the oracle (op-for-op CPU restatement of the reference wide path, torch CPU
  ops) on the host cores over a bounded sample, scaled to samples/s.  Threads = the CPUs this
  process may use (affinity, capped by the cgroup CPU quota); the CPU model, core counts,
  thread count and BLAS / oneDNN build are recorded beside it.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from typing import Callable, Dict, Optional

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "pytorch-parallel-compiler_amd"))
sys.path.insert(0, ROOT)

METRIC = "wide fwd samples/sec (N×B) at 1 MI355X; % of MFMA / HBM roofline"
PEAK = {"fp32_mfma": 157.3e12, "bf16_mfma": 2516.6e12, "hbm": 8.0e12}


def _rel(a, b) -> float:
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return ((a - b).abs().max() / b.abs().max()).item()


def _event_time(fn: Callable[[], None], k: int, w: int) -> float:
    """Average seconds per call of fn (kernel launches on torch's current stream): k calls are
    captured back to back into one HIP graph, so host dispatch does not enter the figure, and
    each replay is bracketed by HIP events recorded on the stream the graph runs on.  The
    graph is replayed until about 40 ms of GPU work have run (the clock climbs for ~25 ms
    after the GPU idles, e.g. during the capture), then 7 more times; the figure is the
    median of those 7."""
    import torch
    for _ in range(max(w, 1)):
        fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(k):
            fn()
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def replay() -> float:
        e0.record(st)
        graph.replay()
        e1.record(st)
        e1.synchronize()
        return e0.elapsed_time(e1) * 1e-3

    warm = 0.0
    for _ in range(200):                # warm replays
        warm += replay()
        if warm >= 0.04:
            break
    return _median([replay() for _ in range(7)]) / k


def _step_times(fn: Callable[[], None], k: int, flush=None) -> list:
    """GPU seconds of each of k calls of fn (HIP events on torch's current stream around each
    call); with flush, the buffer is rewritten before every call, outside the timed window."""
    import torch
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(k)]
    st = torch.cuda.current_stream()
    for i in range(k):
        if flush is not None:
            flush.fill_(i & 0x7f)
        ev[i][0].record(st)
        fn()
        ev[i][1].record(st)
    torch.cuda.synchronize()
    return [a.elapsed_time(b) * 1e-3 for a, b in ev]


def _median(v: list) -> float:
    v = sorted(v)
    return v[len(v) // 2] if len(v) % 2 else 0.5 * (v[len(v) // 2 - 1] + v[len(v) // 2])


def _cpu_loop(fn: Callable[[], None], seconds: float, min_iters: int = 2):
    fn()  # warm-up
    iters, t0 = 0, time.perf_counter()
    while True:
        fn()
        iters += 1
        el = time.perf_counter() - t0
        if (el >= seconds and iters >= min_iters) or iters >= 100000:
            return iters, el


def _kernel(name: str, bound: str, sec: float, launches: int = 1, flops: float = 0.0,
            byts: float = 0.0, peak: Optional[float] = None) -> Dict:
    """One kernel of a step: algorithmic work per launch over its measured average duration."""
    if bound == "hbm":
        peak = PEAK["hbm"] if peak is None else peak
        achieved, unit, scale, work = byts / sec, "GB/s", 1e9, {"bytes_per_launch": byts}
    else:
        achieved, unit, scale, work = flops / sec, "TFLOP/s", 1e12, {"flops_per_launch": flops}
    return {"kernel": name, "bound": "hbm" if bound == "hbm" else "mfma", "us_per_launch": sec * 1e6,
            "launches_per_step": launches, "achieved": achieved / scale, "peak": peak / scale, "unit": unit,
            "frac": achieved / peak, **work}


# ---------------------------------------------------------------------------------------
# configurations: each returns the step, a parity check against the oracle, the step's
# kernels (measured), and a bounded CPU sample of the oracle
# ---------------------------------------------------------------------------------------

def cfg_seq(dev, steps, warmup) -> Dict:
    import torch
    from wide_compiler import _hip, workloads
    from oracle import wide_ref

    work = workloads.seq_n64()
    n, b = work.n, work.batch
    ids_cpu = work.inputs["ids"]
    _, _, t = ids_cpu.shape
    wide = workloads.WideSeqModel([m.to(dev) for m in work.models]).eval()
    ids = ids_cpu.to(dev)
    hdim, v, d = wide.lstm.hidden_size, wide.fc.out_features, wide.lstm.input_size
    logits = torch.empty((n, b, t, v), device=dev, dtype=torch.bfloat16)

    def step():
        return wide(ids, logits)

    def parity():
        with torch.inference_mode():
            y = step()
        errs = []
        for k in (0, n - 1):
            p = {kk: (vv.double() if torch.is_tensor(vv) else vv)
                 for kk, vv in workloads.seq_params([work.models[k]]).items()}
            errs.append(_rel(y[k:k + 1], wide_ref.seq_model(ids_cpu[k:k + 1], p)))
        return max(errs)

    def kernels():
        with torch.inference_mode():
            x = wide.emb.forward_layernorm(ids, wide.ln, per_model=True)
            hs, _ = wide.lstm(x)
            lstm = wide.lstm
            a, ws = _hip.rnn_args(cell=_hip.CELL_LSTM, x=x, w_ih=lstm.weight_ih, w_hh=lstm.weight_hh,
                                  b_ih=lstm.bias_ih, b_hh=lstm.bias_hh, h0=None, c0=None, out=hs,
                                  h_n=None, c_n=None, status=_hip.rnn_status_word(x.device))
            t_emb = _event_time(lambda: wide.emb.forward_layernorm(ids, wide.ln, per_model=True), 20, 2)
            t_proj = _event_time(lambda: _hip.rnn_phase(a, "input_projection", x), 10, 2)
            t_rec = _event_time(lambda: _hip.rnn_phase(a, "recurrence", x), 10, 2)
            t_fc = _event_time(lambda: wide.fc.forward_into(hs, logits), 10, 2)
        _hip.rnn_sync_check(block=True)      # every timed recurrence ran to its end
        rows = n * b * t
        g = 4 * hdim
        return [
            _kernel("layernorm_vec_kernel<gather> (per-model embedding gather + LayerNorm, 256-wide rows, bf16, "
                    "fp32 statistics)", "hbm", t_emb, byts=rows * (8 + 2 * d * 2) + 2 * n * d * 2),
            _kernel("LSTM input projection (part_prep_kernel + gemm_xl8_kernel, 256 -> 2048, bf16 out)",
                    "mfma", t_proj, flops=2.0 * rows * g * d, peak=PEAK["bf16_mfma"]),
            _kernel("part_kernel<512, bf16, LSTM> (LSTM recurrence, 128 steps, W_hh on-chip, 4 CUs per model)", "mfma",
                    t_rec, flops=2.0 * rows * g * hdim, peak=PEAK["bf16_mfma"]),
            _kernel("gemm_xl8_kernel (vocab projection 512 -> 8192 + bias, bf16)", "mfma", t_fc,
                    flops=2.0 * rows * v * hdim, peak=PEAK["bf16_mfma"]),
        ]

    n_cpu = 1
    p_cpu = {kk: (vv.float() if torch.is_tensor(vv) and vv.is_floating_point() else vv)
             for kk, vv in workloads.seq_params(work.models[:n_cpu]).items()}
    p_cpu = {kk: (vv.to(torch.bfloat16) if torch.is_tensor(vv) and vv.is_floating_point() else vv)
             for kk, vv in p_cpu.items()}
    ids_sub = ids_cpu[:n_cpu, :4].contiguous()

    def cpu_run():
        wide_ref.seq_model(ids_sub, p_cpu)

    return {"name": work.name, "n": n, "batch": b, "dtype": "bf16", "step": step, "parity": parity,
            "kernels": kernels, "cpu": cpu_run, "cpu_samples": n_cpu * 4,
            "cpu_sample": f"{n_cpu} of the {n} models, 4 of the {b} sequences (no cross-model or cross-sequence "
                          f"terms), bf16",
            "extra": {"seq_len": t, "vocab": v, "embed": d, "hidden": hdim}}


def cfg_gru(dev, steps, warmup) -> Dict:
    import torch
    import wide_compiler as wc
    from wide_compiler import _hip, workloads
    from oracle import wide_ref

    work = workloads.gru_n32()
    n, b = work.n, work.batch
    x_cpu = work.inputs["x"]
    _, _, t, i = x_cpu.shape
    h = work.models[0].hidden_size
    wide = wc.WideGRU.from_modules(work.models).to(dev).eval()
    x = x_cpu.to(dev)

    def parity():
        with torch.inference_mode():
            out, _ = wide(x)
        p = [getattr(wide, k).detach().cpu().double() for k in ("weight_ih", "weight_hh", "bias_ih", "bias_hh")]
        ref, _ = wide_ref.gru(x_cpu.double(), *p)
        return _rel(out, ref)

    def kernels():
        o = torch.empty((n, b, t, h), device=dev)
        hn = torch.empty((n, b, h), device=dev)
        a, ws = _hip.rnn_args(cell=_hip.CELL_GRU, x=x, w_ih=wide.weight_ih, w_hh=wide.weight_hh, b_ih=wide.bias_ih,
                              b_hh=wide.bias_hh, h0=None, c0=None, out=o, h_n=hn, c_n=None)
        t_proj = _event_time(lambda: _hip.rnn_phase(a, "input_projection", x), steps, warmup)
        t_rec = _event_time(lambda: _hip.rnn_phase(a, "recurrence", x), steps, warmup)
        return [_kernel("gemm_kernel (GRU input projection 64 -> 384, fp32)", "mfma", t_proj,
                        flops=2.0 * n * b * t * 3 * h * i, peak=PEAK["fp32_mfma"]),
                _kernel("rnn_seq_kernel (GRU recurrence, fp32)", "mfma", t_rec,
                        flops=2.0 * n * b * t * 3 * h * h, peak=PEAK["fp32_mfma"])]

    mods = work.models
    p32 = [torch.stack([getattr(m, k).detach().float() for m in mods])
           for k in ("weight_ih_l0", "weight_hh_l0", "bias_ih_l0", "bias_hh_l0")]

    def cpu_run():
        wide_ref.gru(x_cpu, *p32)

    return {"name": work.name, "n": n, "batch": b, "dtype": "fp32", "step": lambda: wide(x), "parity": parity,
            "kernels": kernels, "cpu": cpu_run, "cpu_samples": n * b, "cpu_sample": "full workload",
            "extra": {"seq_len": t, "input_size": i, "hidden": h}}


def cfg_mlp(dev, steps, warmup) -> Dict:
    import torch
    import wide_compiler as wc
    from wide_compiler import workloads
    from oracle import wide_ref

    work = workloads.mlp_n100()
    n, b = work.n, work.batch
    xs = work.inputs["per_model"]
    packed_cpu = wide_ref.pack_inputs(xs)
    models = [m.to(dev) for m in work.models]
    wide = wc.compile(models, xs[0].to(dev)).eval()
    packed = packed_cpu.to(dev)
    st = lambda k: torch.stack([getattr(getattr(m, k.split('.')[0]), k.split('.')[1]).detach().cpu().float()  # noqa
                                for m in models])
    w1, b1, w2, b2 = st("fc1.weight"), st("fc1.bias"), st("fc2.weight"), st("fc2.bias")

    def parity():
        with torch.inference_mode():
            y = wide(packed)
        return _rel(y, wide_ref.mlp_wide(packed_cpu.double(), n, w1.double(), b1.double(), w2.double(),
                                         b2.double()))

    def kernels():
        xn = packed.view(b, n, 64).movedim(1, 0)
        fused = getattr(wide, "_mlp2", {}).get("fc2")
        if fused is not None:
            sec = _event_time(lambda: fused(xn), steps, warmup)
            byts = 4.0 * (n * 128 * 64 + n * 128 + n * 64 * 128 + n * 64 + n * b * 64 + n * b * 64)
            return [_kernel("mlp2_kernel (fc1 + bias + ReLU + fc2 + bias, fp32)", "hbm", sec, byts=byts)]
        fc1 = wide.stages["fc1"]
        sec = _event_time(lambda: fc1(xn), steps, warmup)
        byts = 4.0 * (n * 128 * 64 + n * 128 + n * b * 64 + n * b * 128)
        return [_kernel("gemm_kernel (fc1 + bias + ReLU, fp32)", "hbm", sec, byts=byts)]

    def cpu_run():
        wide_ref.mlp_wide(packed_cpu, n, w1, b1, w2, b2)

    def compiled():
        """The same forward through compile(..., compile_model=True, compile_mode="reduce-overhead"):
        torch.compile around the traced model, whose forward is one operator
        (wide_compiler::module_call) that the cudagraph trees capture."""
        cm = wc.compile(models, xs[0].to(dev), compile_model=True, compile_mode="reduce-overhead").eval()
        with torch.inference_mode():
            y = cm(packed).clone()
        err = _rel(y, wide_ref.mlp_wide(packed_cpu.double(), n, w1.double(), b1.double(), w2.double(),
                                        b2.double()))
        sec = _timed(lambda: cm(packed), steps, max(warmup, 3))
        return {"mode": "compile_model=True, reduce-overhead", "ms_per_step": sec / steps * 1e3,
                "value": n * b * steps / sec, "unit": "samples/s", "parity_rel_err_vs_oracle": err}

    return {"name": work.name, "n": n, "batch": b, "dtype": "fp32", "step": lambda: wide(packed),
            "compiled": compiled,
            "parity": parity, "kernels": kernels, "cpu": cpu_run, "cpu_samples": n * b,
            "cpu_sample": "full workload", "extra": {"layers": "Linear(64,128)-ReLU-Linear(128,64)"}}


def cfg_resblock(dev, steps, warmup) -> Dict:
    import torch
    import wide_compiler as wc
    from wide_compiler import workloads
    from oracle import wide_ref

    work = workloads.resblock_n100()
    n, b, c, hw = work.n, work.batch, 64, 32
    x_cpu = work.inputs["packed"]
    models = [m.to(dev) for m in work.models]
    wide = wc.compile(models, x_cpu[:, :c].to(dev)).eval()
    x = x_cpu.to(dev)

    def parity():
        with torch.inference_mode():
            y = wide(x).cpu()
        errs = []
        for k in (0, n // 2, n - 1):
            pk = workloads.resblock_params([models[k]], torch.float64)
            errs.append(_rel(y[:, k * c:(k + 1) * c],
                             wide_ref.resblock_wide(x_cpu[:, k * c:(k + 1) * c].double(), 1, pk)))
        return max(errs)

    def kernels():
        conv1 = wide.stages["conv1"]
        xn = x.view(b, n, c, hw, hw).movedim(1, 0)
        sec = _event_time(lambda: conv1(xn), steps, warmup)
        flops = 2.0 * n * b * hw * hw * c * c * 9
        return [_kernel("conv_res_kernel (resident-weight conv3x3 + BN + ReLU, bf16)", "mfma", sec, launches=2,
                        flops=flops, peak=PEAK["bf16_mfma"])]

    n_cpu = 4
    pk_cpu = workloads.resblock_params([m for m in models[:n_cpu]], torch.bfloat16)
    x_sub = x_cpu[:, :n_cpu * c].contiguous()

    def cpu_run():
        wide_ref.resblock_wide(x_sub, n_cpu, pk_cpu)

    return {"name": work.name, "n": n, "batch": b, "dtype": "bf16", "step": lambda: wide(x), "parity": parity,
            "kernels": kernels, "cpu": cpu_run, "cpu_samples": n_cpu * b,
            "cpu_sample": f"{n_cpu} of the {n} models (the wide path has no cross-model terms), bf16",
            "extra": {"channels": c, "hw": hw}}


def cfg_attention(dev, steps, warmup) -> Dict:
    import torch
    import wide_compiler as wc
    from wide_compiler import _hip, workloads
    from oracle import wide_ref

    work = workloads.attention_n16()
    n, b = work.n, work.batch
    x_cpu = work.inputs["x"]
    _, _, s, d = x_cpu.shape
    hh = work.models[0].num_heads
    dh = d // hh
    wide = wc.WideAttention.from_modules([m.to(dev) for m in work.models]).eval()
    x = x_cpu.to(dev)
    prm = lambda w, k: getattr(w, k).detach().cpu()  # noqa: E731

    def parity():
        with torch.inference_mode():
            y = wide(x).cpu()
        errs = []
        for k in (0, n - 1):
            c = lambda t: t[k:k + 1].double()  # noqa: E731
            xs = c(x_cpu)
            ref = wide_ref.attention(xs, xs, xs, *(c(prm(wide, a)) for a in
                                     ("q_weight", "kv_weight", "out_weight", "q_bias", "kv_bias", "out_bias")), hh)
            errs.append(_rel(y[k:k + 1], ref))
        return max(errs)

    def kernels():
        o = torch.empty((n, b, s, d), device=dev, dtype=x.dtype)
        fused = lambda: _hip.self_attention(x=x, q_weight=wide.q_weight, kv_weight=wide.kv_weight,  # noqa: E731
                                            q_bias=wide.q_bias, kv_bias=wide.kv_bias, o=o, heads=hh,
                                            scale=dh ** -0.5, causal=False)
        t_attn = _event_time(fused, steps, warmup)
        t_out = _event_time(lambda: wide._project(o, wide.out_weight, d * d, wide.out_bias, d, d), steps, warmup)
        rows = n * b * s
        return [_kernel("attn_qkv_kernel (Q/K/V projections 256 -> 3 x 256 + softmax(QK^T)V, bf16, head_dim 32, "
                        "K/V resident in LDS)", "mfma", t_attn,
                        flops=2.0 * rows * 3 * d * d + 4.0 * n * b * hh * s * s * dh, peak=PEAK["bf16_mfma"]),
                _kernel("gemm_xl8_kernel (output projection 256 -> 256, bf16)", "mfma", t_out,
                        flops=2.0 * rows * d * d, peak=PEAK["bf16_mfma"])]

    n_cpu = 1
    xs_cpu = x_cpu[:n_cpu].contiguous()
    pc = [prm(wide, a)[:n_cpu].contiguous() for a in
          ("q_weight", "kv_weight", "out_weight", "q_bias", "kv_bias", "out_bias")]

    def cpu_run():
        wide_ref.attention(xs_cpu, xs_cpu, xs_cpu, *pc, hh)

    return {"name": work.name, "n": n, "batch": b, "dtype": "bf16", "step": lambda: wide(x), "parity": parity,
            "kernels": kernels, "cpu": cpu_run, "cpu_samples": n_cpu * b,
            "cpu_sample": f"{n_cpu} of the {n} models (the wide path has no cross-model terms), bf16",
            "extra": {"seq_len": s, "embed": d, "heads": hh}}


def cfg_groupnorm(dev, steps, warmup) -> Dict:
    """WideGroupNorm over N=32 nn.GroupNorm(8, 64) (the reference benchmark's groups = min(8, C),
    wide_groupnorm.py:281), x [32, 8, 64, 32, 32] ~ N(0, 1) fp32."""
    import torch
    import torch.nn as nn
    import wide_compiler as wc
    from oracle import wide_ref

    n, b, c, groups, hw = 32, 8, 64, 8, 32
    torch.manual_seed(1234)
    mods = [nn.GroupNorm(groups, c) for _ in range(n)]
    with torch.no_grad():
        for m in mods:
            m.weight.normal_(1, 0.1)
            m.bias.normal_(0, 0.1)
    wide = wc.WideGroupNorm.from_modules(mods).to(dev)
    g = torch.Generator().manual_seed(4321)
    x_cpu = torch.randn(n, b, c, hw, hw, generator=g)
    x = x_cpu.to(dev)
    w_cpu, b_cpu = wide.norm.weight.detach().cpu(), wide.norm.bias.detach().cpu()

    def parity():
        with torch.inference_mode():
            y = wide(x)
        return _rel(y, wide_ref.group_norm(x_cpu.double(), w_cpu.double(), b_cpu.double(), groups, 1e-5))

    def kernels():
        sec = _event_time(lambda: wide(x), steps, warmup)
        return [_kernel("groupnorm_kernel (8192-element rows, fp32)", "hbm", sec,
                        byts=2.0 * x.numel() * 4 + 2 * n * c * 4)]

    n_cpu = 8

    def cpu_run():
        wide_ref.group_norm(x_cpu[:n_cpu], w_cpu[:n_cpu * c], b_cpu[:n_cpu * c], groups, 1e-5)

    return {"name": f"WideGroupNorm N={n} B={b} C={c} G={groups} {hw}x{hw} fp32", "n": n, "batch": b,
            "dtype": "fp32", "step": lambda: wide(x), "parity": parity, "kernels": kernels, "cpu": cpu_run,
            "cpu_samples": n_cpu * b, "cpu_sample": f"{n_cpu} of the {n} models (no cross-model terms)",
            "extra": {"channels": c, "groups": groups, "spatial": [hw, hw]}}


CONFIGS = {"seq": cfg_seq, "gru": cfg_gru, "mlp": cfg_mlp, "resblock": cfg_resblock, "attention": cfg_attention,
           "groupnorm": cfg_groupnorm}
EXTRA = ("mlp", "gru", "resblock", "attention")


# ---------------------------------------------------------------------------------------
# measurement
# ---------------------------------------------------------------------------------------

def _timed(step, k: int, w: int) -> float:
    import torch
    with torch.inference_mode():
        for _ in range(w):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(k):
            step()
        torch.cuda.synchronize()
        return time.perf_counter() - t0


def _first(out):
    return out[0] if isinstance(out, tuple) else out


def _graph_of(step):
    """The step captured as one HIP graph (after warm-up on a side stream), and whether a
    replay's output equals an eager forward's bit for bit.  The replay's output is copied
    before the eager forward runs, since a step may write into a persistent buffer."""
    import torch
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
        graph.replay()
        replayed = _first(static_out).clone()
        eager = _first(step())
        torch.cuda.synchronize()
        same = torch.equal(replayed, eager)
    return graph, same


def _run_config(cfg: Dict, steps: int, warmup: int, mode: str, min_warm_s: float = 0.0,
                min_timed_s: float = 0.0) -> Dict:
    """value / mode / parity / kernels of one configuration.  With min_warm_s / min_timed_s the
    warm-up and timed step counts are raised (never lowered) to cover that much time, from a
    step time estimated over 3 steps."""
    import torch
    from wide_compiler import _hip
    n, b = cfg["n"], cfg["batch"]
    step = cfg["step"]
    # rnn_sync_check(block=True) raises if a bounded wait of the partitioned LSTM gave up in
    # any launch or graph replay since the last check (the status word collects them all)
    parity = cfg["parity"]()
    _hip.rnn_sync_check(block=True)
    if min_warm_s > 0 or min_timed_s > 0:
        est = _timed(step, 3, 1) / 3
        warmup = max(warmup, int(min_warm_s / est) + 1)
        steps = max(steps, int(min_timed_s / est) + 1)
    eager_s = _timed(step, steps, warmup)
    _hip.rnn_sync_check(block=True)
    graph_s, graph = None, None
    if mode in ("graph", "best"):
        graph, same = _graph_of(step)
        if not same:
            raise RuntimeError("graph replay differs from the eager forward")
        graph_s = _timed(graph.replay, steps, warmup)
        _hip.rnn_sync_check(block=True)
    if mode == "eager" or graph_s is None:
        wall, used = eager_s, "eager"
    elif mode == "graph":
        wall, used = graph_s, "graph"
    else:
        wall, used = (graph_s, "graph") if graph_s <= eager_s else (eager_s, "eager")
    with torch.inference_mode():
        kernels = cfg["kernels"]()
    dom = max(kernels, key=lambda k: k["us_per_launch"] * k["launches_per_step"])
    return {"wall": wall, "mode": used, "eager_s": eager_s, "graph_s": graph_s, "graph": graph,
            "parity": parity, "kernels": kernels, "dominant": dom, "steps": steps, "warmup": warmup,
            "samples_per_s": n * b * steps / wall, "ms_per_step": wall / steps * 1e3,
            "eager_ms_per_step": eager_s / steps * 1e3,
            "graph_ms_per_step": None if graph_s is None else graph_s / steps * 1e3}


def _pack_leg(dev) -> Dict:
    """The boundary byte-movement kernels at the ResBlock configuration's size (100 tensors of
    [8, 64, 32, 32] bf16, 104.9 MB): wc_pack_rows (pack from N separate tensors) and wc_swap01
    (channel-packed -> N-first transpose).  Bytes = 2 * numel * sizeof (read + write)."""
    import torch
    from wide_compiler import _hip
    n, b, c, hw = 100, 8, 64, 32
    srcs = [torch.randn(b, c, hw, hw, device=dev).to(torch.bfloat16) for _ in range(n)]
    packed = torch.empty(b, n * c, hw, hw, device=dev, dtype=torch.bfloat16)
    row = c * hw * hw * 2
    nfirst = torch.empty(n, b, c, hw, hw, device=dev, dtype=torch.bfloat16)
    t_pack = _event_time(lambda: _hip.pack_rows(srcs, packed, b, row, [row] * n), 10, 2)
    t_swap = _event_time(lambda: _hip.swap01(packed, b, n, n * row, row, row, nfirst), 10, 2)
    byts = 2.0 * n * b * c * hw * hw * 2
    return {"pack_rows": _kernel("seg_copy_kernel<PackMap> (wc_pack_rows, 100 x [8,64,32,32] bf16)", "hbm",
                                 t_pack, byts=byts),
            "boundary_transpose": _kernel("seg_copy_kernel (wc_swap01, [8,6400,32,32] -> [100,8,64,32,32] bf16)",
                                          "hbm", t_swap, byts=byts)}


def _cpu_info() -> Dict:
    import torch
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, period = f.read().split()
            if q != "max":
                quota = int(q) / int(period)
    except (OSError, ValueError):
        pass
    threads = affinity if quota is None else max(1, min(affinity, int(quota)))
    cfg = torch.__config__.show()
    blas = [ln.strip() for ln in cfg.split("\n") if "MKL" in ln or "LAPACK" in ln]
    build = [ln for ln in cfg.split(",") if "BLAS_INFO" in ln or "USE_MKLDNN" in ln]
    return {"cpu_model": model, "os_cpu_count": os.cpu_count(), "affinity_cpus": affinity,
            "cgroup_cpu_quota": quota, "threads": threads, "torch": torch.__version__,
            "blas": "; ".join(blas + [b.strip() for b in build])}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", choices=sorted(CONFIGS), default="seq")
    ap.add_argument("--mode", choices=("best", "graph", "eager"), default="best")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the other configurations and the pack leg")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 5 device-to-device copies of MIB MiB (the reference kernel whose "
                         "FETCH_SIZE / WRITE_SIZE counters calibrate the HBM traffic figures) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested)", file=sys.stderr)
        return 2

    import torch
    from wide_compiler import _hip

    dev = torch.device("cuda", 0)
    if args.copy_calibration:
        nbytes = args.copy_calibration << 20
        src = torch.ones(nbytes // 4, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": nbytes, "copies": 5}))
        return 0

    cfg = CONFIGS[args.config](dev, args.steps, args.warmup)
    n, b = cfg["n"], cfg["batch"]
    r = _run_config(cfg, args.steps, args.warmup, args.mode)
    print(f"bench: {args.config} {r['samples_per_s']:.4g} samples/s ({r['mode']}), parity {r['parity']:.3e}",
          file=sys.stderr, flush=True)

    # hot / cold cache regimes: per-step GPU times in the mode used
    run_step = r["graph"].replay if r["mode"] == "graph" else cfg["step"]
    with torch.inference_mode():
        hot = _step_times(run_step, args.steps)
        flush = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
        cold = _step_times(run_step, args.steps, flush)
        del flush
    _hip.rnn_sync_check(block=True)
    hot_med, cold_med = _median(hot), _median(cold)

    dom = dict(r["dominant"])
    step_gpu_us = sum(k["us_per_launch"] * k["launches_per_step"] for k in r["kernels"])
    roofline = {"bound": dom["bound"], "achieved": dom["achieved"], "peak": dom["peak"], "unit": dom["unit"],
                "frac": dom["frac"], "traffic": None, "kernel": dom["kernel"], "us_per_launch": dom["us_per_launch"],
                "share_of_step_kernel_time": dom["us_per_launch"] * dom["launches_per_step"] / step_gpu_us}
    for key in ("flops_per_launch", "bytes_per_launch"):
        if key in dom:
            roofline[key] = dom[key]
    traffic_file = os.path.join(ROOT, "profiles", f"traffic_{args.config}.json")
    if os.path.exists(traffic_file):
        with open(traffic_file) as f:
            tr = json.load(f)
        if tr.get("kernel") == dom["kernel"]:
            roofline["traffic"] = tr.get("bytes_per_launch")
    roofline["kernels"] = r["kernels"]

    line = {
        "metric": METRIC,
        "value": r["samples_per_s"],
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": r["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg["dtype"],
        "data": "synthetic (seeded torch.nn default init, inputs ~ N(0,1) / uniform ids)",
        "config": {"workload": cfg["name"], "n_models": n, "batch": b, "mode": r["mode"], **cfg["extra"]},
        "roofline": roofline,
        "eager_samples_per_s": n * b * args.steps / r["eager_s"],
        "graph_samples_per_s": None if r["graph_s"] is None else n * b * args.steps / r["graph_s"],
        "cache_regimes": {"mode": r["mode"], "steps": args.steps, "flush_bytes": 512 << 20,
                          "hot_median_ms": hot_med * 1e3, "hot_samples_per_s": n * b / hot_med,
                          "cold_median_ms": cold_med * 1e3, "cold_samples_per_s": n * b / cold_med},
        "parity_rel_err_vs_oracle": r["parity"],
    }
    del r["graph"]

    if not args.no_extra:
        extra: Dict[str, Dict] = {}
        for name in EXTRA:
            if name == args.config:
                continue
            c = CONFIGS[name](dev, args.steps, args.warmup)
            rc = _run_config(c, args.steps, args.warmup, args.mode, min_warm_s=0.05, min_timed_s=0.03)
            d = rc["dominant"]
            extra[name] = {"workload": c["name"], "value": rc["samples_per_s"], "unit": "samples/s",
                           "ms_per_step": rc["ms_per_step"], "mode": rc["mode"], "dtype": c["dtype"],
                           "steps": rc["steps"], "warmup": rc["warmup"],
                           "eager_ms_per_step": rc["eager_ms_per_step"],
                           "graph_ms_per_step": rc["graph_ms_per_step"],
                           "parity_rel_err_vs_oracle": rc["parity"],
                           "roofline": {"kernel": d["kernel"], "bound": d["bound"], "achieved": d["achieved"],
                                        "peak": d["peak"], "unit": d["unit"], "frac": d["frac"],
                                        "us_per_launch": d["us_per_launch"]},
                           "kernels": rc["kernels"]}
            if "compiled" in c:
                extra[name]["torch_compile"] = c["compiled"]()
            print(f"bench: {name} {rc['samples_per_s']:.4g} samples/s ({rc['mode']}), {d['kernel'].split()[0]} "
                  f"{d['frac']:.3f}", file=sys.stderr, flush=True)
            del c, rc
            torch.cuda.empty_cache()
        with torch.inference_mode():
            extra["pack"] = _pack_leg(dev)
        line["configs"] = extra

    cpu = None
    if not args.no_cpu:
        info = _cpu_info()
        torch.set_num_threads(info["threads"])
        with torch.inference_mode():
            iters, el = _cpu_loop(cfg["cpu"], args.cpu_seconds)
        cpu = {"value": cfg["cpu_samples"] * iters / el, "unit": "samples/s", "cores": info["threads"],
               "kind": "port",
               "sample": f"{iters} forwards of the oracle ({cfg['cpu_sample']}; torch CPU ops, "
                         f"{torch.get_num_threads()} threads) in {el:.1f} s",
               **info, "torch_threads": torch.get_num_threads()}
    line["cpu_baseline"] = cpu
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
