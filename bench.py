"""Benchmark of the MoE expert-FFN layer forward on one MI355X.

    python bench.py [--steps K] [--warmup W] [--workload NAME] [--no-cpu]

A step is one whole MoE layer forward (router -> top-k -> capacity plan ->
grouped SwiGLU experts -> weighted combine) over one batch of synthetic input
already resident in HBM.  Prints ONE JSON line: throughput of the headline
workload (bf16 prefill, T=8192, d=2048, 64 experts, d_ff=1024, top-2,
capacity factor 1.25) with a roofline entry for the expert-FFN stage, the
CPU baseline (the reference's forward restated with torch CPU ops, whole
workload, on the host cores), per-workload numbers for the other workloads
(each with its own CPU baseline), the same layer timed through the TopKMoE
module, and the batch-1 decode step
(qw_moe_decode_step: the routed experts of one token, fp32 routing, no
capacity) at three of the workloads' layer shapes, eager and replayed from a
HIP graph.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP32_PEAK_TFLOPS = 157.3


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 100 untimed steps bring the GPU to its steady clocks first (with 10, the timed
    # wall clock still includes the ramp); 200 timed headline steps take ~60 ms
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--workload", default=None)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only-headline", action="store_true")
    ap.add_argument("--decode-steps-only", action="store_true",
                    help="only time the batch-1 decode steps (one JSON line with their figures)")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="only run a plain device copy of this many MiB (calibrates HBM byte counters)")
    ap.add_argument("--stream-probe", action="store_true",
                    help="only measure the HBM rates the chip sustains for a plain read (a 2 GiB sum) and a "
                         "plain copy (1 GiB to 1 GiB): the practical ceiling next to the 8 TB/s peak")
    return ap.parse_args()


def event_time(fn, iters, stream):
    """Average ms per call of fn() measured with HIP events on `stream`."""
    import torch

    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(iters):
        fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / iters


def event_samples(fn, iters, stream, flush=None):
    """Per-call ms of fn() from HIP event pairs on `stream`; flush() runs between calls, outside the pairs."""
    import torch

    pairs = []
    for _ in range(iters):
        if flush is not None:
            flush()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        fn()
        b.record(stream)
        pairs.append((a, b))
    torch.cuda.synchronize()
    t = np.array([a.elapsed_time(b) for a, b in pairs])
    return dict(median=float(np.median(t)), p10=float(np.percentile(t, 10)), p90=float(np.percentile(t, 90)))


def stage_times(calls, iters, stream):
    """Average ms of each stage as it runs inside the layer: the stages called
    in layer order, iters times, each bracketed by its own HIP event pair on
    `stream` (the caches then hold what a layer call leaves in them, which
    repeated calls of one stage alone do not reproduce)."""
    import torch

    names = list(calls)
    pairs = []
    for _ in range(iters):
        row = []
        for n in names:
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            calls[n]()
            b.record(stream)
            row.append((a, b))
        pairs.append(row)
    torch.cuda.synchronize()
    return {n: sum(r[j][0].elapsed_time(r[j][1]) for r in pairs) / iters for j, n in enumerate(names)}


def stage_calls(run):
    """The forward split into its entry points, with the same buffers as qw_moe_forward."""
    import torch
    from quantaweave_amd import _hip, _lib

    lay, w = run.layer, run.layer.w
    lib = _lib.load()
    T, E, K, D, F = w.tokens, w.experts, w.top_k, w.d_model, w.d_ff
    R = T * K
    P = _hip.ptr
    logits = run.workspace_view("logits")
    slot_token = run.workspace_view("slot_token")
    slot_weight = run.workspace_view("slot_weight")
    route_slot = run.workspace_view("route_slot")
    kept_offsets = run.workspace_view("kept_offsets")
    y = run.workspace_view("y")
    plan_bytes = lib.qw_moe_plan_workspace_bytes(T, K, E)
    plan_ws = _hip.workspace(plan_bytes, lay.x.device)
    max_rows = min(R, run.capacity * E)
    exp_bytes = lib.qw_moe_experts_workspace_bytes(max_rows, E, D, F, run.act)
    exp_ws = _hip.workspace(exp_bytes, lay.x.device)
    route_bytes = lib.qw_moe_route_workspace_bytes(T, D, E)
    route_ws = _hip.workspace(route_bytes, lay.x.device)
    s = run.stream

    def route():
        _lib.check(lib.qw_moe_route(P(lay.x), run.act, D, P(lay.router), run.act, T, D, E, K, 1.0, P(lay.bias),
                                    P(logits), P(run.probs), P(run.top_idx), P(run.top_w), P(route_ws), route_bytes,
                                    s), "route")

    def plan():
        _lib.check(lib.qw_moe_plan(P(run.top_idx), P(run.top_w), T, K, E, run.capacity, P(run.counts),
                                   P(run.kept_counts), P(kept_offsets), P(slot_token), P(slot_weight), P(route_slot),
                                   P(run.dropped_token), P(run.dropped_expert), P(run.totals), P(plan_ws),
                                   plan_bytes, s), "plan")

    def experts():
        _lib.check(lib.qw_moe_experts(P(lay.x), run.act, P(slot_token), P(kept_offsets), E, D, F, max_rows,
                                      min(run.capacity, R), *lay.weight_args(), None, P(y), P(exp_ws),
                                      exp_bytes, s), "experts")

    def combine():
        _lib.check(lib.qw_moe_combine_weighted(P(y), run.act, P(route_slot), P(run.top_idx), P(run.top_w), T, K, D,
                                               P(run.out), run.act, s), "combine")

    return dict(route=route, plan=plan, experts=experts, combine=combine)


def measure(name, steps, warmup):
    import torch
    from quantaweave_amd import workloads as W

    w = W.WORKLOADS[name]
    layer = W.build_layer(w).add_tiles()  # bf16 experts in QW_BF16T tiles, as the TopKMoE module keeps them
    run = W.LayerRunner(layer)
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        run()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1000 / steps
    ev_ms = event_time(run, steps, stream)
    torch.cuda.synchronize()
    # routing outcome of this workload (fixed seed): touched experts and kept rows
    counts = run.kept_counts.cpu().numpy()
    kept = int(run.totals[0].item())
    dropped = int(run.totals[1].item())
    touched = int((counts > 0).sum())
    calls = stage_calls(run)
    for k_, fn in calls.items():
        fn()
    torch.cuda.synchronize()
    stages = stage_times(calls, max(5, steps // 2), stream)
    # the expert stage again with the 256 MB last-level cache (MALL) flushed before every call: reading
    # 512 MiB between calls evicts the weights (and leaves no dirty lines), so each call streams them from HBM
    scratch = torch.ones(64 << 20, dtype=torch.int64, device=layer.x.device)
    cold = event_samples(calls["experts"], max(20, steps), stream, flush=lambda: scratch.max())
    del scratch
    flops = 6.0 * kept * w.d_model * w.d_ff
    act_bytes = 4 if w.act == "f32" else 2
    weight_bytes = touched * layer.expert_bytes()
    # algorithmic bytes of the expert stage: touched experts' weights once, each kept row read once
    # (gathered x) and written once (y), plus the d_ff-wide hidden row written and read back
    stage_bytes = weight_bytes + kept * (2 * w.d_model + 2 * w.d_ff) * act_bytes
    layer_bytes = weight_bytes + 2 * w.tokens * w.d_model * act_bytes + w.experts * w.d_model * act_bytes
    return dict(
        workload=w, wall_ms=wall_ms, event_ms=ev_ms, kept=kept, dropped=dropped, touched=touched, stages=stages,
        experts_cold=cold,
        flops=flops, stage_bytes=stage_bytes, layer_bytes=layer_bytes, weight_bytes=weight_bytes,
        tokens_per_s=w.tokens / (wall_ms / 1000.0),
    )


DECODE_SHAPES = ["int4-decode-T16-d4096-E64-f1408-k2", "int8-decode-T64-d2048-E64-f1024-k2",
                 "bf16-prefill-T8192-d2048-E64-f1024-k2"]


def measure_decode(name, steps, warmup):
    """One-token decode step on the layer of workload `name`: per-step ms of eager
    calls and of HIP-graph replays (warm, and with the last-level cache flushed)."""
    import torch
    from quantaweave_amd import workloads as W

    w = W.WORKLOADS[name]
    layer = W.build_layer(W.scaled(w, tokens=1)).add_tiles()
    run = W.DecodeRunner(layer, tokens=1)
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    eager = event_samples(run, max(20, steps), stream)
    eager_pace = event_time(run, max(50, steps), stream)  # back-to-back calls, as replay_ms below
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        for _ in range(3):
            run()
    stream.wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    replay_ms = event_time(graph.replay, max(50, steps), stream)
    scratch = torch.ones(64 << 20, dtype=torch.int64, device="cuda")
    cold = event_samples(graph.replay, max(20, steps), stream, flush=lambda: scratch.max())
    del scratch
    touched = int(torch.unique(run.top_idx).numel())
    # algorithmic bytes: the routed experts' stored weights once, x, residual and out (fp32), the fp32 router
    nbytes = touched * layer.expert_bytes() + 3 * w.d_model * 4 + w.experts * w.d_model * 4
    return dict(
        shape=f"T1-d{w.d_model}-E{w.experts}-f{w.d_ff}-k{w.top_k}-{w.weights}", experts_read=touched,
        algorithmic_bytes=nbytes, eager_ms={k: round(v, 4) for k, v in eager.items()},
        eager_pace_ms=round(eager_pace, 4), graph_replay_ms=round(replay_ms, 4),
        graph_replay_cold_ms={k: round(v, 4) for k, v in cold.items()},
        tokens_per_s_graph=round(1000.0 / replay_ms, 1),
        hbm_frac_cold=round(nbytes / (cold["median"] / 1000) / 1e9 / HBM_PEAK_GBS, 4),
    )


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(name, budget_s=8.0):
    """The reference's layer forward (loop executor, dequantise-then-matmul for
    int8/int4 experts) restated with torch CPU operators (oracle.torch_ref), on
    the whole workload, timed on the host cores: one warm-up, then the median
    of up to five runs within `budget_s`."""
    import torch
    from oracle import torch_ref
    from quantaweave_amd import workloads as W

    w = W.WORKLOADS[name]
    layer = W.build_layer(w)
    cpu = lambda t: None if t is None else t.cpu()  # noqa: E731
    x, router = layer.x.cpu(), layer.router.cpu()
    experts = torch_ref.Experts(w.weights, cpu(layer.gate), cpu(layer.up), cpu(layer.down), cpu(layer.gate_s),
                                cpu(layer.up_s), cpu(layer.down_s))
    bias = cpu(layer.bias)
    del layer
    torch.cuda.empty_cache()
    cap = w.capacity()
    # the host's cores (BASELINE's plan: torch.set_num_threads(os.cpu_count())), but
    # never more threads than this process may run on (a cpuset or affinity mask)
    host_cores = os.cpu_count() or 1
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else host_cores
    threads = min(host_cores, usable)
    prev_threads = torch.get_num_threads()
    torch.set_num_threads(threads)
    with torch.no_grad():
        t0 = time.perf_counter()
        torch_ref.moe_forward(x, router, experts, w.top_k, cap, expert_bias=bias)  # warm-up
        times = []
        t_end = t0 + budget_s
        while len(times) < 5 and (not times or time.perf_counter() < t_end):
            t1 = time.perf_counter()
            torch_ref.moe_forward(x, router, experts, w.top_k, cap, expert_bias=bias)
            times.append(time.perf_counter() - t1)
    torch.set_num_threads(prev_threads)
    med = float(np.median(times))
    return dict(value=round(w.tokens / med, 1), unit="tokens/s", cores=threads, kind="port",
                sample=f"the whole workload ({w.tokens} tokens, {w.experts} experts, capacity {cap}) through the "
                       f"reference's loop-executor forward restated with torch CPU ops (oracle/torch_ref.py), "
                       f"{w.act} activations, {w.weights} experts; median of {len(times)} runs after one warm-up; "
                       f"{threads} torch threads (host: {host_cores} logical CPUs, {usable} usable by this "
                       f"process) on {cpu_model()}")


def committed_traffic(name):
    """HBM bytes per call of the expert stage from the committed counter summary
    (profiles/moe_layer_all_workloads_hbm_bytes.md, its json block), or None."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "moe_layer_all_workloads_hbm_bytes.md")
    try:
        text = open(path).read()
        block = text.split("```json", 1)[1].split("```", 1)[0]
        return json.loads(block)["expert_stage_bytes"].get(name)
    except (OSError, IndexError, KeyError, ValueError):
        return None


def measure_module(name, steps, warmup):
    """The drop-in surface: TopKMoE.forward (no grad) on the workload's layer,
    wall ms per call, with the module's own per-call work (workspace,
    balance loss, Python)."""
    import torch
    from quantaweave_amd import workloads as W

    w = W.WORKLOADS[name]
    layer = W.build_layer(w)
    moe = W.module_from_layer(layer)
    hidden = layer.x.reshape(w.batch, w.seq, w.d_model)
    with torch.no_grad():
        for _ in range(warmup):
            moe(hidden)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            moe(hidden)
        torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1000 / steps


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); runs over several GPUs are not implemented",
              file=sys.stderr)
        sys.exit(2)
    import torch
    from quantaweave_amd import workloads as W

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm device", file=sys.stderr)
        sys.exit(1)
    if args.copy_probe_mib:
        n = args.copy_probe_mib * (1 << 20)
        src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": n, "launches": 3}), flush=True)
        return
    if args.stream_probe:
        n = 1 << 31
        src = torch.ones(n // 4, dtype=torch.float32, device="cuda")
        dst = torch.empty(n // 8, dtype=torch.float32, device="cuda")
        stream = torch.cuda.current_stream()
        read_ms = min(event_time(lambda: src.sum(), 5, stream) for _ in range(3))
        copy_ms = min(event_time(lambda: dst.copy_(src[: n // 8]), 5, stream) for _ in range(3))
        print(json.dumps({"read_gbs": round(n / (read_ms / 1000) / 1e9, 1),
                          "copy_gbs": round(n / (copy_ms / 1000) / 1e9, 1),
                          "read_bytes": n, "copy_bytes_read_plus_written": n}), flush=True)
        return
    if args.decode_steps_only:
        decode = {}
        for name in DECODE_SHAPES:
            r = measure_decode(name, args.steps, args.warmup)
            decode[r.pop("shape")] = r
        print(json.dumps({"decode_step": decode}), flush=True)
        return
    head = args.workload or W.HEADLINE
    results = {}
    if not args.only_headline:
        for name in W.WORKLOADS:
            if name != head:
                results[name] = measure(name, args.steps, args.warmup)
    # the headline last, on a GPU already at its steady clocks
    results[head] = measure(head, args.steps, args.warmup)
    module_ms = measure_module(head, args.steps, args.warmup)
    h = results[head]
    w = h["workload"]
    t_exp = h["stages"]["experts"]
    mfma = w.act == "bf16" and w.tokens * w.top_k // w.experts >= 64
    if mfma:
        achieved = h["flops"] / (t_exp / 1000) / 1e12
        roof = dict(bound="mfma", achieved=round(achieved, 2), peak=BF16_PEAK_TFLOPS, unit="TFLOP/s",
                    frac=round(achieved / BF16_PEAK_TFLOPS, 4), traffic=committed_traffic(head))
    else:
        achieved = h["stage_bytes"] / (t_exp / 1000) / 1e9
        roof = dict(bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                    frac=round(achieved / HBM_PEAK_GBS, 4), traffic=committed_traffic(head))
    roof["kernel"] = "qw_moe_experts (grouped SwiGLU: gate/up+SiLU*mul, down+weight)"
    roof["algorithmic"] = dict(flops=h["flops"], bytes=h["stage_bytes"], launch_ms=round(t_exp, 4))
    per = {}
    for name, r in results.items():
        ww = r["workload"]
        te = r["stages"]["experts"]
        tc = r["experts_cold"]["median"]
        per[name] = dict(
            tokens_per_s=round(r["tokens_per_s"], 1), ms_per_step=round(r["wall_ms"], 4),
            event_ms=round(r["event_ms"], 4), stages_ms={k: round(v, 4) for k, v in r["stages"].items()},
            kept_routes=r["kept"], dropped_routes=r["dropped"], experts_touched=r["touched"],
            expert_stage_tflops=round(r["flops"] / (te / 1000) / 1e12, 2),
            expert_stage_gbs=round(r["stage_bytes"] / (te / 1000) / 1e9, 1),
            hbm_frac=round(r["stage_bytes"] / (te / 1000) / 1e9 / HBM_PEAK_GBS, 4),
            mfma_frac=round(r["flops"] / (te / 1000) / 1e12 / BF16_PEAK_TFLOPS, 4) if ww.act in ("bf16", "f16") else None,
            experts_cold_ms={k: round(v, 4) for k, v in r["experts_cold"].items()},
            hbm_frac_cold=round(r["stage_bytes"] / (tc / 1000) / 1e9 / HBM_PEAK_GBS, 4),
        )
    per[head]["module_ms_per_step"] = round(module_ms, 4)
    per[head]["module_tokens_per_s"] = round(w.tokens / (module_ms / 1000.0), 1)
    decode = {}
    if not args.only_headline:
        for name in DECODE_SHAPES:
            r = measure_decode(name, args.steps, args.warmup)
            decode[r.pop("shape")] = r
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(head)
        per[head]["cpu_tokens_per_s"] = cpu["value"]
        if not args.only_headline:
            for name in results:
                if name != head:
                    per[name]["cpu_tokens_per_s"] = cpu_baseline(name)["value"]
    line = {
        "metric": "MoE FFN tokens/s + % roofline (HBM GB/s decode, MFMA util prefill)",
        "value": round(h["tokens_per_s"], 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(h["wall_ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": w.act,
        "data": "synthetic (N(0,1) activations, N(0,0.02) weights, fixed seed)",
        "config": {"workload": head, "tokens": w.tokens, "d_model": w.d_model, "experts": w.experts, "d_ff": w.d_ff,
                   "top_k": w.top_k, "capacity_factor": w.capacity_factor, "weights": w.weights, "seed": w.seed},
        "roofline": roof,
        "cpu_baseline": cpu,
        # the same layer through the drop-in module (TopKMoE.forward, no grad): the
        # value above plus the balance loss the reference computes on every call
        # (src/quantweave_moe_model.py:152-154), the int64 counts and the Python call
        "module": {"ms_per_step": round(module_ms, 4), "tokens_per_s": round(w.tokens / (module_ms / 1000.0), 1),
                   "includes": "route, plan, experts, combine, balance loss, Python"},
        "workloads": per,
        "decode_step": decode,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
