#!/usr/bin/env python3
"""Q4_RDNA group-64 GEMV benchmark on one MI355X (gfx950).

Workload: one decode step's weight streaming for the Qwen3-8B 36-layer stack,
252 distinct packed tensors (q 4096x4096, k/v 1024x4096, o 4096x4096,
gate/up 12288x4096, down 4096x12288 per layer, 3,689,938,944 packed bytes),
swept in layer order at batch 1 with a fresh N(0,1) activation per tensor.
Weights are N(0, 0.02) fp32 generated on the GPU and packed by the GPU packer
(bit-identical to the reference's native packer); everything is resident in
HBM before timing.

A step is one sweep of the stack by the multi-tensor plan kernel (one
launch).  Printed: one JSON line with the step throughput over algorithmic
bytes (17*M*K/32 + 4*K + 4*M per tensor), the per-launch roofline figures
measured with HIP events on the launch stream, and the CPU oracle's
sequential GEMV timed on a bounded sample of the same stack.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "rdna-gfx1201-v0.1_amd"))
sys.path.insert(0, ROOT)

METRIC = "Q4g64 GEMV HBM GB/s (% of 8 TB/s peak) + µs per Qwen3-8B 252-tensor stack"
PEAK_GBS = 8000.0


def algorithmic_bytes(rows: int, cols: int, n: int = 1) -> int:
    return 17 * rows * cols // 32 + 4 * cols * n + 4 * rows * n


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def build_stack(layers: int, seed: int):
    """Generate and pack the stack on the GPU; returns tensors and buffers."""
    import torch
    from q4rdna import api
    from q4rdna.sidecar import layout, qwen3_8b_stack

    names = qwen3_8b_stack(layers)
    data_offset, entries, end = layout(names)
    dev = torch.device("cuda", 0)
    data = torch.empty(end - data_offset, dtype=torch.uint8, device=dev)
    gen = torch.Generator(device=dev)
    tensors = []
    t0 = time.time()
    for i, (name, rows, cols, off, size) in enumerate(entries):
        gen.manual_seed(seed + i)
        w = torch.randn(rows, cols, generator=gen, device=dev, dtype=torch.float32).mul_(0.02)
        view = data[off - data_offset: off - data_offset + size]
        api.pack(w, out=view)
        del w
        gen.manual_seed(seed + 0x8000 + i)
        x = torch.randn(cols, generator=gen, device=dev, dtype=torch.float32)
        y = torch.empty(rows, dtype=torch.float32, device=dev)
        tensors.append(dict(name=name, rows=rows, cols=cols, w=api.QWeight.from_tiles(view, rows, cols), x=x, y=y))
    torch.cuda.synchronize()
    log(f"[bench] generated and packed {len(tensors)} tensors ({end - data_offset} bytes) in {time.time() - t0:.1f}s")
    return tensors, data


def time_plan(plan, steps: int, warmup: int):
    """Per-launch durations (ms) from HIP events on the launch stream."""
    import torch
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        plan.launch(stream.cuda_stream)
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        starts[i].record(stream)
        plan.launch(stream.cuda_stream)
        ends[i].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    return per, wall


def time_per_tensor(tensors, steps: int, warmup: int):
    """One launch per tensor (the reference's dispatch pattern), stack time."""
    import torch
    from q4rdna import api
    stream = torch.cuda.current_stream()
    def sweep():
        for t in tensors:
            api.mul_mat(t["w"], t["x"], t["y"], stream=stream.cuda_stream)
    for _ in range(warmup):
        sweep()
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(steps):
        sweep()
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / steps


def check_parity(tensors, picks):
    """Stack outputs vs the fp64 oracle for a few tensors (full size)."""
    import numpy as np
    import oracle as O
    worst = 0.0
    for i in picks:
        t = tensors[i]
        tiles = t["w"].tiles.cpu().numpy()
        x = t["x"].cpu().numpy()
        y64, a64 = O.gemv_f64(tiles, t["rows"], t["cols"], x)
        err = O.gemv_errors(t["y"].cpu().numpy(), y64, a64)
        worst = max(worst, err["gate"])
    return worst


def cpu_baseline(tensors, budget_s: float):
    """The oracle's sequential fp32 GEMV (the reference bench's CPU loop,
    source/q4rdna_gemv_bench.hip:189-211) on host cores, one thread, over the
    stack's tensors in order until about budget_s of CPU work."""
    import oracle as O
    done_bytes, elapsed, n = 0, 0.0, 0
    for t in tensors:
        tiles = t["w"].tiles.cpu().numpy()
        x = t["x"].cpu().numpy()
        t0 = time.perf_counter()
        O.gemv_seq_f32(tiles, t["rows"], t["cols"], x)
        elapsed += time.perf_counter() - t0
        done_bytes += algorithmic_bytes(t["rows"], t["cols"])
        n += 1
        if elapsed >= budget_s:
            break
    return dict(value=round(done_bytes / elapsed / 1e9, 4), unit="GB/s", cores=1, kind="port",
                sample=f"first {n} of {len(tensors)} stack tensors in layer order, {done_bytes} algorithmic bytes, "
                       f"{elapsed:.2f}s single-thread (oracle/q4oracle.c, gcc -O2, x86-64 baseline)",
                us_per_stack_extrapolated=round(elapsed / done_bytes * sum(
                    algorithmic_bytes(t["rows"], t["cols"]) for t in tensors) * 1e6, 1))


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--seed", type=int, default=0x51EE0000)
    ap.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of CPU baseline work")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-per-tensor", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported (this path does not shard)",
              file=sys.stderr)
        return 2

    import torch
    from q4rdna import api

    tensors, _data = build_stack(args.layers, args.seed)
    stack_bytes = sum(algorithmic_bytes(t["rows"], t["cols"]) for t in tensors)
    plan = api.Plan([(t["w"], t["x"], t["y"]) for t in tensors])
    log(f"[bench] plan: {len(tensors)} GEMVs, {plan.workgroups} workgroups")

    torch.cuda.synchronize()
    per_launch, wall = time_plan(plan, args.steps, args.warmup)
    ms_per_step = wall * 1000.0 / args.steps
    avg_launch_ms = sum(per_launch) / len(per_launch)
    log(f"[bench] plan: {avg_launch_ms * 1000:.1f} us per launch (events), {ms_per_step * 1000:.1f} us per step (wall)")
    parity = check_parity(tensors, [0, 1, 4, 6, len(tensors) - 1])
    log(f"[bench] parity vs fp64 oracle on 5 tensors: gate {parity:.2e}")

    per_tensor_us = None
    if not args.no_per_tensor:
        per_tensor_us = time_per_tensor(tensors, max(3, args.steps // 10), 2) * 1000.0
        log(f"[bench] per-tensor launches: {per_tensor_us:.1f} us per stack")

    value = stack_bytes / (ms_per_step / 1000.0) / 1e9
    achieved = stack_bytes / (avg_launch_ms / 1000.0) / 1e9
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"qwen3-8b {args.layers}-layer stack, {len(tensors)} Q4_RDNA group-64 tensors, "
                               "batch 1, fresh x per tensor, one multi-tensor launch per step",
                   "tensors": len(tensors), "algorithmic_bytes_per_step": stack_bytes, "batch": 1},
        "us_per_stack": round(avg_launch_ms * 1000.0, 2),
        "pct_of_peak": round(100.0 * achieved / PEAK_GBS, 2),
        "per_tensor_launches_us_per_stack": None if per_tensor_us is None else round(per_tensor_us, 2),
        "parity_gate_max": parity,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_GBS, 4), "traffic": None},
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(tensors, args.cpu_budget)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
