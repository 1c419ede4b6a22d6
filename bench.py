"""Benchmark of the DiT attention hot path (qk_prep + attend) on one MI355X.

One step = fused qk_prep on a (B, L, 9216) bf16 QKV activation followed by bounded
attention on its output, at the Klein 4B 1024^2 shape by default (512 text + 64x64
image tokens = 4608, 24 heads x 128).  Inputs are resident in HBM before timing.

Each kernel is bracketed by HIP events on the stream it is launched on (torch's
current stream); `value` is attend's TFLOP/s over its own launches, and the line also
reports qk_prep's GB/s and both roofline fractions.  To keep the QKV input from being
served by the 256 MB Infinity Cache between steps, steps rotate over buffer sets
whose total exceeds it.  A CPU baseline (the torch-CPU restatement of the reference's
plain-XLA path, the oracle) is timed on the host cores.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload klein_1024]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

HBM_PEAK_GBS = 8000.0           # MI355X HBM3E, GB/s
BF16_DENSE_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, TFLOP/s
METRIC = "attend TFLOP/s + qk_prep GB/s at 1024² Klein shape; % of MI355X roofline"
INFINITY_CACHE_BYTES = 256 * 2 ** 20


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="klein_1024")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-reps", type=int, default=3)
    return ap.parse_args()


def cpu_baseline(w, qkv, qs, ks, ids, reps: int) -> dict:
    """Time the oracle's torch-CPU plain path on the full step (all heads), p50 of `reps`."""
    import torch

    from oracle import cpu_baseline as cb
    from oracle import path as P

    pe = torch.from_numpy(P.embed_nd(ids)[0, 0])
    threads = torch.get_num_threads()
    cb.plain_attention(qkv, qs, ks, pe, w.num_heads, heads=[0])   # warm-up
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        cb.plain_attention(qkv, qs, ks, pe, w.num_heads)
        times.append(time.perf_counter() - t0)
    times.sort()
    p50 = times[len(times) // 2]
    return {"value": round(w.attend_flops() / p50 / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
            "kind": "port", "ms": round(p50 * 1e3, 1),
            "sample": f"full {w.name} step (qk norm+RoPE+sdpa, all {w.num_heads} heads, f32 torch CPU), "
                      f"p50 of {reps} after 1 warm-up"}


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); multi-GPU sharding of this "
              "path is a design note, not a measured configuration", file=sys.stderr)
        return 2

    import torch

    from flicker_amd import kernels, rope, workloads

    w = workloads.WORKLOADS[args.workload]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    qkv_cpu = workloads.make_qkv(w)
    qs_cpu, ks_cpu = workloads.make_scales(w)
    ids = workloads.make_ids(w)
    qs, ks = qs_cpu.to(dev), ks_cpu.to(dev)
    freqs = rope.rope_lanes(ids, workloads.q_gain(w), device=dev)

    act_bytes = qkv_cpu.numel() * 2
    set_bytes = 2 * act_bytes + act_bytes // 3
    n_sets = max(2, -(-2 * INFINITY_CACHE_BYTES // set_bytes))
    sets = []
    for i in range(n_sets):
        qkv = qkv_cpu.to(dev)
        out = tuple(torch.empty((w.batch, w.num_heads, w.length, w.head_dim), dtype=torch.bfloat16, device=dev)
                    for _ in range(3))
        o = torch.empty_like(out[0])
        sets.append((qkv, out, o))

    def step(i, ev=None):
        qkv, out, o = sets[i % n_sets]
        if ev is not None:
            ev[0].record()
        kernels.qk_prep(qkv, qs, ks, freqs, w.num_heads, out=out)
        if ev is not None:
            ev[1].record()
        kernels.attend(*out, out=o)
        if ev is not None:
            ev[2].record()

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i, events[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0

    qk_ms = sum(e[0].elapsed_time(e[1]) for e in events) / args.steps
    at_ms = sum(e[1].elapsed_time(e[2]) for e in events) / args.steps
    qk_gbs = w.qk_prep_bytes() / (qk_ms * 1e-3) / 1e9
    at_tflops = w.attend_flops() / (at_ms * 1e-3) / 1e12

    result = {
        "metric": METRIC,
        "value": round(at_tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 QKV, 1+N(0,0.05) bf16 norm scales, Klein RoPE ids)",
        "config": {"workload": f"{w.name}: one Klein 4B DiT attention op, B={w.batch}, "
                               f"{w.num_txt} text + {w.height}x{w.width} image tokens",
                   "batch": w.batch, "seq_len": w.length, "heads": w.num_heads, "head_dim": w.head_dim,
                   "buffer_sets": n_sets},
        "roofline": {"bound": "mfma", "achieved": round(at_tflops, 2), "peak": BF16_DENSE_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(at_tflops / BF16_DENSE_PEAK_TFLOPS, 4),
                     "traffic": None, "kernel": "attend_kernel",
                     "flops_per_launch": w.attend_flops(), "avg_launch_us": round(at_ms * 1e3, 2)},
        "qk_prep": {"roofline": {"bound": "hbm", "achieved": round(qk_gbs, 1), "peak": HBM_PEAK_GBS,
                                 "unit": "GB/s", "frac": round(qk_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                                 "kernel": "qk_prep_kernel", "bytes_per_launch": w.qk_prep_bytes(),
                                 "avg_launch_us": round(qk_ms * 1e3, 2)}},
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(w, qkv_cpu, qs_cpu, ks_cpu, ids, args.cpu_reps)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
