"""Benchmark of the DiT attention hot path (qk_prep + attend) on one MI355X.

One step = fused qk_prep on a (B, L, 9216) bf16 QKV activation followed by bounded
attention on its output, at the Klein 4B 1024^2 shape by default (512 text + 64x64
image tokens = 4608, 24 heads x 128).  Inputs are resident in HBM before timing.

The timed region is `--steps` steps (qk_prep then attend) between two HIP events on the
launch stream (torch's current stream) -> ms_per_step.  Before it run `--warmup` untimed
steps and then untimed steps for `--clock-warmup-s` seconds (reported as clock_warmup_s):
the GPU takes about a second of load to reach its working clock, which a few warm-up steps
do not give.  Each kernel is then timed alone the same way, `--kernel-launches`
back-to-back launches over the same rotating buffers after `--leg-warmup-s` seconds of
untimed ones (the clock falls while the host sets a leg up), which gives its average launch
duration: `value` is attend's TFLOP/s from that, and the line also reports
qk_prep's GB/s and both roofline fractions.  To keep the QKV input from being
served by the 256 MB Infinity Cache between steps, steps rotate over buffer sets
whose total exceeds it.  A CPU baseline (the torch-CPU restatement of the reference's
plain-XLA path, the oracle) is timed on the host cores.  `head_share` times attend on one
GPU's share of an 8-way head-parallel run (3 of the 24 heads, the full sequence), the grid
that the key-split path exists for.  `vendor` times the same operations through ROCm's own
libraries (torch's flash SDPA, hipBLASLt's int8 and bf16 GEMMs) for comparison.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload klein_1024]

Counter runs (rocprofv3 --pmc) use --only to launch one kernel kind, and
--ingest-pmc turns a FETCH_SIZE run and a WRITE_SIZE run of
`--only calibrate` into the per-launch HBM traffic summary
profiles/hbm_traffic_<workload>.json that the default run reports as roofline.traffic.
--ingest-mfma turns one run with the MFMA counters (MFMA_COUNTERS) into
profiles/mfma_util_<workload>.json: per dispatch of attend and of the int8 GEMM, the
fraction of cycles the matrix pipe is busy and the shader clock the kernel ran at, which the
default run reports as roofline.mfma_busy / roofline.sclk_ghz.
"""

from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import sys
import time

HBM_PEAK_GBS = 8000.0           # MI355X HBM3E, GB/s
BF16_DENSE_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, TFLOP/s
INT8_DENSE_PEAK_TOPS = 5000.0    # MI355X dense int8 MFMA, TOP/s
METRIC = "attend TFLOP/s + qk_prep GB/s at 1024² Klein shape; % of MI355X roofline"
INFINITY_CACHE_BYTES = 256 * 2 ** 20
ROOT = os.path.dirname(os.path.abspath(__file__))
COPY_BYTES = 64 * 2 ** 20       # calibration copy: 64 MiB read + 64 MiB written per launch
# One rocprofv3 --pmc pass (7 SQ counters + 1 GRBM counter, within one pass's limits).
MFMA_COUNTERS = ("SQ_VALU_MFMA_BUSY_CYCLES", "SQ_BUSY_CYCLES", "SQ_INSTS_MFMA", "SQ_INSTS_VALU_MFMA_MOPS_BF16",
                 "SQ_INSTS_VALU_MFMA_MOPS_I8", "SQ_VALU_MFMA_COEXEC_CYCLES", "SQ_INSTS_VALU", "GRBM_GUI_ACTIVE")


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=300,
                    help="untimed steps before the timed region")
    ap.add_argument("--clock-warmup-s", type=float, default=2.0,
                    help="further untimed steps, for this many seconds, before the timed region: the "
                         "GPU needs ~1 s of load to settle at its working clock whatever --warmup is; "
                         "reported as clock_warmup_s (0 = off)")
    ap.add_argument("--leg-warmup-s", type=float, default=0.5,
                    help="back-to-back untimed calls, for this many seconds, before each per-kernel leg")
    ap.add_argument("--kernel-launches", type=int, default=200,
                    help="back-to-back launches of each kernel alone behind its average launch duration")
    ap.add_argument("--workload", default="klein_1024")
    ap.add_argument("--eager-kernel-timing", action="store_true",
                    help="time each kernel leg as eager back-to-back launches instead of a replayed HIP graph")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-w8a8", action="store_true", help="skip the int8 W8A8 QKV projection leg")
    ap.add_argument("--no-vendor", action="store_true",
                    help="skip the comparison legs through ROCm's libraries (torch SDPA flash, hipBLASLt GEMMs)")
    ap.add_argument("--projection", default="qkv_1024")
    ap.add_argument("--workloads", default="klein_512,klein_1536x640,klein_2048,klein_1024_b4",
                    help="the other Klein configurations timed after the headline one (qk_prep and attend "
                         "legs, same method), reported under 'workloads'; empty = none")
    ap.add_argument("--cpu-reps", type=int, default=9,
                    help="timed CPU-baseline steps (after 3 warm-up steps); the p50 is reported")
    ap.add_argument("--only", choices=["step", "calibrate"], default="step",
                    help="calibrate: the step plus a plain device copy of known size, for counter runs")
    ap.add_argument("--ingest-pmc", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="rocprofv3 --pmc output dirs of FETCH_SIZE / WRITE_SIZE runs of --only calibrate")
    ap.add_argument("--ingest-mfma", metavar="DIR",
                    help="rocprofv3 --pmc output dir of a default run with the MFMA_COUNTERS")
    ap.add_argument("--ingest-trace", metavar="DIR",
                    help="rocprofv3 --kernel-trace --output-format csv output dir: print its per-leg and "
                         "all-dispatch tables (markdown)")
    return ap.parse_args()


def traffic_file(workload: str) -> str:
    return os.path.join(ROOT, "profiles", f"hbm_traffic_{workload}.json")


def _is_attend(kernel_name: str) -> bool:
    """Any of attend's one-pass kernels (256- or 192-query tiles, rounds, balanced, key split),
    not the split path's merge."""
    return "attend_" in kernel_name and "_kernel" in kernel_name and "merge" not in kernel_name


def _counter_means(directory: str, counter: str) -> dict:
    files = glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no counter_collection.csv under {directory}")
    sums: dict = {}
    for f in files:
        for row in csv.DictReader(open(f)):
            if row["Counter_Name"] != counter:
                continue
            name = row["Kernel_Name"]
            key = ("attend" if _is_attend(name) else "qk_prep" if "qk_prep_kernel" in name
                   else "w8a8_gemm" if "w8a8_gemm_kernel<false, false" in name
                   else "copy" if ("copyBuffer" in name or "copy" in name.lower()) else None)
            if key:
                sums.setdefault(key, []).append(float(row["Counter_Value"]))
    if "copy" in sums:  # keep the calibration copies, not the small host-to-device copies
        big = max(sums["copy"])
        sums["copy"] = [v for v in sums["copy"] if v >= 0.5 * big]
    return {k: sum(v) / len(v) for k, v in sums.items()}


def mfma_file(workload: str) -> str:
    return os.path.join(ROOT, "profiles", f"mfma_util_{workload}.json")


def ingest_mfma(directory: str, workload: str, last: int = 20) -> dict:
    """MFMA busy fraction and shader clock of attend and the plain int8 GEMM, from one counter
    run.  Every SQ counter is summed over the GPU: SQ_VALU_MFMA_BUSY_CYCLES over the SIMDs
    (32 per 32x32 MFMA), SQ_BUSY_CYCLES over the shader engines, so per-SIMD busy cycles /
    per-engine busy cycles = the matrix pipe's busy fraction, and per-engine busy cycles /
    the dispatch's duration = the clock.  Means over the last `last` dispatches (warm clock)."""
    files = glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True)
    agents = glob.glob(os.path.join(directory, "**", "*agent_info.csv"), recursive=True)
    if not files or not agents:
        raise SystemExit(f"no counter_collection.csv / agent_info.csv under {directory}")
    gpu = next(a for a in csv.DictReader(open(agents[0])) if a.get("Simd_Count", "0") not in ("0", ""))
    simds = int(gpu["Simd_Count"])
    engines = int(gpu["Cu_Count"]) // int(gpu["Cu_Per_Engine"])
    rows: dict = {}
    for f in files:
        for row in csv.DictReader(open(f)):
            name = row["Kernel_Name"]
            key = ("attend" if _is_attend(name) else
                   "w8a8_gemm" if "w8a8_gemm_kernel<false, false" in name else None)
            if key:
                d = rows.setdefault(key, {}).setdefault(int(row["Dispatch_Id"]), {})
                d[row["Counter_Name"]] = float(row["Counter_Value"])
                d["ns"] = int(row["End_Timestamp"]) - int(row["Start_Timestamp"])
    out = {"workload": workload, "simds": simds, "shader_engines": engines, "dispatches_averaged": last,
           "kernels": {}}
    for key, disp in rows.items():
        sel = [disp[i] for i in sorted(disp)[-last:]]
        mean = {c: sum(d.get(c, 0.0) for d in sel) / len(sel) for c in MFMA_COUNTERS + ("ns",)}
        busy_simd = mean["SQ_VALU_MFMA_BUSY_CYCLES"] / simds
        cycles = mean["SQ_BUSY_CYCLES"] / engines
        out["kernels"][key] = {
            "duration_us": mean["ns"] / 1e3, "mfma_busy_cycles_per_simd": busy_simd,
            "busy_cycles_per_engine": cycles, "mfma_busy": busy_simd / cycles,
            "sclk_ghz": cycles / mean["ns"], "mfma_insts": mean["SQ_INSTS_MFMA"],
            "coexec_cycles_per_simd": mean["SQ_VALU_MFMA_COEXEC_CYCLES"] / simds,
            "valu_insts": mean["SQ_INSTS_VALU"],
            "bf16_gflop_counted": mean["SQ_INSTS_VALU_MFMA_MOPS_BF16"] * 512 / 1e9,
            "i8_gop_counted": mean["SQ_INSTS_VALU_MFMA_MOPS_I8"] * 512 / 1e9,
            "counters": mean}
    return out


def ingest_pmc(fetch_dir: str, write_dir: str, workload: str) -> dict:
    """Per-launch HBM bytes of each kernel: counter KiB per dispatch scaled by what the same
    counter reads for the calibration copy (COPY_BYTES read, COPY_BYTES written)."""
    fetch = _counter_means(fetch_dir, "FETCH_SIZE")
    write = _counter_means(write_dir, "WRITE_SIZE")
    f_scale = COPY_BYTES / (fetch["copy"] * 1024)
    w_scale = COPY_BYTES / (write["copy"] * 1024)
    out = {"workload": workload, "fetch_scale": f_scale, "write_scale": w_scale,
           "copy_fetch_kib": fetch["copy"], "copy_write_kib": write["copy"], "kernels": {}}
    for k in ("qk_prep", "attend", "w8a8_gemm"):
        if k not in fetch or k not in write:
            continue
        rb, wb = fetch[k] * 1024 * f_scale, write[k] * 1024 * w_scale
        out["kernels"][k] = {"fetch_kib": fetch[k], "write_kib": write[k], "read_bytes": rb,
                             "write_bytes": wb, "traffic_bytes": rb + wb}
    return out


CPU_WARMUPS = 3   # the reference's method: 3 warm-up calls, then the p50 (tools/bench.py:21,25-33)


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), or the platform's processor string."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def cpu_baseline(w, qkv, qs, ks, ids, reps: int) -> dict:
    """Time the oracle's torch-CPU plain path on the full step (all heads): CPU_WARMUPS warm-up
    steps, then the p50 of `reps` steps.  `cores` is the number of threads torch computes
    with (the host's CPU share: OMP_NUM_THREADS where the launcher sets it), `host_cpus` the
    CPUs this process may run on."""
    import torch

    from oracle import cpu_baseline as cb
    from oracle import path as P

    pe = torch.from_numpy(P.embed_nd(ids)[0, 0])
    host_cpus = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    threads = torch.get_num_threads()
    for _ in range(CPU_WARMUPS):
        cb.plain_attention(qkv, qs, ks, pe, w.num_heads)
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        cb.plain_attention(qkv, qs, ks, pe, w.num_heads)
        times.append(time.perf_counter() - t0)
    times.sort()
    p50 = times[len(times) // 2]
    return {"value": round(w.attend_flops() / p50 / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
            "host_cpus": host_cpus, "cpu_model": cpu_model(), "kind": "port", "ms": round(p50 * 1e3, 1),
            "sample": f"full {w.name} step (qk norm+RoPE+sdpa, all {w.num_heads} heads, f32 torch CPU on "
                      f"{threads} threads), p50 of {reps} after {CPU_WARMUPS} warm-up steps"}


def projection_operands(p, dev):
    """The projection's calibrated int8 operands: (x, qw, xq, a_scale)."""
    from flicker_amd import w8a8, workloads

    x_cpu, w_cpu = workloads.make_projection(p)
    x, wt = x_cpu.to(dev), w_cpu.to(dev)
    qw = w8a8.quantize_linear(wt, w8a8.absmax_cols(x))
    xq, a_scale = w8a8.quantize_act(x, qw.inv_smooth)
    return x, qw, xq, a_scale


SHARE_GPUS = 8


def head_share_leg(w, qkv_heads, timed) -> dict:
    """attend on one GPU's share of a head-parallel run over SHARE_GPUS GPUs (heads / 8 of
    them, full sequence): the grid is then too small to fill the GPU, so kernels.attend takes
    its key-split path.  Timed as planned and with the split off."""
    import torch
    from flicker_amd import _lib, kernels
    heads = w.num_heads // SHARE_GPUS
    q, k, v = (t[:, :heads].contiguous() for t in qkv_heads)
    o = torch.empty_like(q)
    splits, _ = _lib.attend_plan(w.batch, heads, w.length)
    flops = 4 * w.batch * heads * w.length * w.length * w.head_dim
    for _ in range(20):
        kernels.attend(q, k, v, out=o)
    split_ms = timed(lambda i: kernels.attend(q, k, v, out=o), 200)
    plain_ms = timed(lambda i: kernels.attend(q, k, v, out=o, splits=1), 200)
    return {"heads": heads, "of_gpus": SHARE_GPUS, "splits": splits, "avg_launch_us": round(split_ms * 1e3, 2),
            "achieved": round(flops / (split_ms * 1e-3) / 1e12, 1), "unit": "TFLOP/s",
            "unsplit_us": round(plain_ms * 1e3, 2)}


def workload_leg(name: str, kernel_timed, dev) -> dict:
    """qk_prep and attend at another Klein configuration, timed like the headline legs: each
    kernel alone, back to back over rotating buffer sets (more than twice the Infinity Cache),
    after its clock settle; the smaller of eager launches and a replayed HIP graph.  For the
    stressed batch (5% of the QKV channels x8) the load-time logit-bound check runs on the
    norm scales and the runtime logit maximum of head 0 is compared with the bound."""
    import torch

    from flicker_amd import kernels, loader, rope, workloads

    w = workloads.WORKLOADS[name]
    qkv_cpu = workloads.make_qkv(w)
    qs, ks = (t.to(dev) for t in workloads.make_scales(w))
    freqs = rope.rope_lanes(workloads.make_ids(w), workloads.q_gain(w), device=dev)
    act_bytes = qkv_cpu.numel() * 2
    n_sets = max(2, -(-2 * INFINITY_CACHE_BYTES // (2 * act_bytes + act_bytes // 3)))
    sets = []
    for _ in range(n_sets):
        out = tuple(torch.empty((w.batch, w.num_heads, w.length, w.head_dim), dtype=torch.bfloat16, device=dev)
                    for _ in range(3))
        sets.append((qkv_cpu.to(dev), out, torch.empty_like(out[0])))
    del qkv_cpu

    def run_qk(i):
        qkv, out, _ = sets[i % n_sets]
        kernels.qk_prep(qkv, qs, ks, freqs, w.num_heads, out=out)

    def run_attend(i):
        _, out, o = sets[i % n_sets]
        kernels.attend(*out, out=o)

    for i in range(n_sets):
        run_qk(i)
    n = max(20, min(200, int(0.2 / (w.attend_flops() / 1.2e15))))
    qk_ms = kernel_timed(run_qk, n, f"{name}/qk_prep")
    at_ms = kernel_timed(run_attend, n, f"{name}/attend")
    at = w.attend_flops() / (at_ms * 1e-3) / 1e12
    gbs = w.qk_prep_bytes() / (qk_ms * 1e-3) / 1e9
    rec = {"config": f"B={w.batch}, {w.num_txt} text + {w.height}x{w.width} image tokens = L {w.length}, "
                     f"{w.num_heads}x{w.head_dim} heads" + (f", {w.stress_fraction:.0%} of QKV channels x8"
                                                            if w.stress_fraction else ""),
           "buffer_sets": n_sets, "launches": n,
           "attend": {"avg_launch_us": round(at_ms * 1e3, 2), "achieved": round(at, 1), "unit": "TFLOP/s",
                      "frac": round(at / BF16_DENSE_PEAK_TFLOPS, 4), "flops_per_launch": w.attend_flops(),
                      "kernel": " + ".join(kernels.attend_kernels(w.batch, w.num_heads, w.length))},
           "qk_prep": {"avg_launch_us": round(qk_ms * 1e3, 2), "achieved": round(gbs, 1), "unit": "GB/s",
                       "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_launch": w.qk_prep_bytes()}}
    if w.stress_fraction:
        bound = float(kernels.logit_bound(qs.float().cpu(), ks.float().cpu()))
        qn, kn = qs.float().cpu(), ks.float().cpu()   # the same scales in every block of the stack
        double = {f"{s}_attn.norm.{n}.scale": t.expand(5, -1) for s in ("img", "txt")
                  for n, t in (("query_norm", qn), ("key_norm", kn))}
        single = {"norm.query_norm.scale": qn.expand(20, -1), "norm.key_norm.scale": kn.expand(20, -1)}
        loader.check_logit_bound({"double_blocks": double, "single_blocks": single})
        q, k, _ = sets[0][1]
        logits = q[0, 0].float() @ k[0, 0].float().T   # q carries the 1/sqrt(D) gain: these are attend's logits
        rec["logit_bound"] = {"bound": round(bound, 3), "runtime_max_head0": round(float(logits.abs().max()), 3),
                              "limit": kernels.EXP_LIMIT, "check_logit_bound": "passed"}
    del sets
    torch.cuda.empty_cache()
    return rec


def vendor_leg(w, qkv_sets, attend_us, gemm_us, args, timed, dev) -> dict:
    """The same operations through ROCm's own libraries, for comparison: torch's fused SDPA
    (the flash backend only, no fallback to the unfused math path) on the same rotating
    head-major q, k, v as attend, with scale 1 as attend applies (q carries the 1/sqrt(d)
    gain); hipBLASLt's int8 GEMM (torch._int_mm, int32 output, no rescale) and its bf16
    GEMM (the unquantised projection, what the reference's nn.Linear runs) on the
    projection's operands.  Eager back-to-back launches."""
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    from flicker_amd import workloads

    out = {}
    n = min(args.kernel_launches, 50)

    def leg(name, fn):
        # A comparison leg never costs the bench line: a library that fails here (no kernel
        # in the installed torch for this shape) is recorded as such.
        try:
            out[name] = fn()
        except Exception as e:  # noqa: BLE001
            out[name] = {"error": f"{type(e).__name__}: {str(e)[:200]}"}

    def sdpa():
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
            for i in range(10):
                F.scaled_dot_product_attention(*qkv_sets[i % len(qkv_sets)], scale=1.0)
            ms = timed(lambda i: F.scaled_dot_product_attention(*qkv_sets[i % len(qkv_sets)], scale=1.0), n)
        tflops = w.attend_flops() / (ms * 1e-3) / 1e12
        return {"avg_launch_us": round(ms * 1e3, 2), "achieved": round(tflops, 1), "unit": "TFLOP/s",
                "attend_speedup": round(ms * 1e3 / attend_us, 3),
                "fa_library": str(torch.backends.cuda.preferred_rocm_fa_library())}

    leg("sdpa_flash", sdpa)
    if args.no_w8a8:
        return out
    p = workloads.PROJECTIONS[args.projection]
    x, qw, xq, _ = projection_operands(p, dev)

    def int_mm():
        b = qw.wq_t.t()   # (K, N), column-major: hipBLASLt's preferred int8 layout
        for _ in range(10):
            torch._int_mm(xq, b)
        ms = timed(lambda i: torch._int_mm(xq, b), n)
        return {"avg_launch_us": round(ms * 1e3, 2), "achieved": round(p.gemm_ops() / (ms * 1e-3) / 1e12, 1),
                "unit": "TOP/s", "output": "int32", "w8a8_gemm_speedup": round(ms * 1e3 / gemm_us, 3)}

    def linear():
        wb = workloads.make_projection(p)[1].t().contiguous().to(dev)   # nn.Linear's (out, in) weight
        for _ in range(10):
            F.linear(x, wb)
        ms = timed(lambda i: F.linear(x, wb), n)
        return {"avg_launch_us": round(ms * 1e3, 2), "achieved": round(p.gemm_ops() / (ms * 1e-3) / 1e12, 1),
                "unit": "TFLOP/s", "w8a8_gemm_speedup": round(ms * 1e3 / gemm_us, 3)}

    leg("int_mm", int_mm)
    leg("bf16_linear", linear)
    return out


def w8a8_leg(args, timed, dev) -> dict:
    """The int8 SmoothQuant QKV projection feeding qk_prep (X (M, 3072) -> Y (M, 9216)):
    activation quantisation and the int8-MFMA GEMM, each timed back to back."""
    import torch

    from flicker_amd import w8a8, workloads

    p = workloads.PROJECTIONS[args.projection]
    x, qw, xq, a_scale = projection_operands(p, dev)
    ys = [torch.empty((p.tokens, p.out_features), dtype=torch.bfloat16, device=dev) for _ in range(2)]
    for i in range(20):
        w8a8.gemm(xq, a_scale, qw.wq_t, qw.w_scale, out=ys[i % 2])
    gemm_ms = timed(lambda i: w8a8.gemm(xq, a_scale, qw.wq_t, qw.w_scale, out=ys[i % 2]), args.kernel_launches,
                    "w8a8_gemm")
    quant_ms = timed(lambda i: w8a8.quantize_act(x, qw.inv_smooth), args.kernel_launches)
    tops = p.gemm_ops() / (gemm_ms * 1e-3) / 1e12
    # The projection feeding qk_prep: the GEMM + qk_prep pair, and the fused kernel whose
    # epilogue does qk_prep (flk_w8a8_qk_prep), on the projection's tokens as one sequence.
    from flicker_amd import kernels, rope
    from flicker_amd.rope import sequence_ids
    w_attn = workloads.WORKLOADS["klein_1024"]
    heads = p.out_features // (3 * w_attn.head_dim)
    qs, ks = (t.to(dev) for t in workloads.make_scales(w_attn))
    n_txt = min(w_attn.num_txt, p.tokens)
    side = int(round((p.tokens - n_txt) ** 0.5))
    ids = sequence_ids(n_txt, side, (p.tokens - n_txt) // max(side, 1)) if p.tokens > n_txt else sequence_ids(n_txt, 0, 0)
    freqs = rope.rope_lanes(ids, workloads.q_gain(w_attn), device=dev)
    qkv_out = [tuple(torch.empty((1, heads, p.tokens, 128), dtype=torch.bfloat16, device=dev) for _ in range(3))
               for _ in range(2)]
    x3 = x.view(1, p.tokens, p.hidden)
    lib = __import__("flicker_amd._lib", fromlist=["lib"])

    def fused(i):
        o = qkv_out[i % 2]
        stream = lib.stream_of(x)   # the current stream at call time (a capture stream under graph timing)
        lib.check(lib.lib().flk_w8a8_qk_prep(
            xq.data_ptr(), qw.wq_t.data_ptr(), a_scale.data_ptr(), qw.w_scale.data_ptr(), p.hidden,
            freqs.cos.data_ptr(), freqs.sin.data_ptr(), freqs.cos.stride(0), qs.data_ptr(), ks.data_ptr(), 0,
            freqs.q_gain, 1, p.tokens, heads, 128, o[0].data_ptr(), o[1].data_ptr(), o[2].data_ptr(),
            p.tokens, 0, stream), "flk_w8a8_qk_prep")

    def unfused(i):
        y = ys[i % 2]
        w8a8.gemm(xq, a_scale, qw.wq_t, qw.w_scale, out=y)
        kernels.qk_prep(y.view(1, p.tokens, p.out_features), qs, ks, freqs, heads, out=qkv_out[i % 2])

    fused_ms = timed(fused, args.kernel_launches, "w8a8_qk_prep_fused")
    unfused_ms = timed(unfused, args.kernel_launches)
    # The block input's modulate (LayerNorm, scale, shift) fused into the quantisation.
    g = torch.Generator().manual_seed(6)
    shift = (0.3 * torch.randn(1, p.hidden, generator=g)).to(torch.bfloat16).to(dev)
    scale = (0.1 * torch.randn(1, p.hidden, generator=g)).to(torch.bfloat16).to(dev)
    mod_ms = timed(lambda i: w8a8.quantize_act_modulated(x3, shift, scale, qw.inv_smooth), args.kernel_launches)
    # A block's whole attention section on this path (modules.py:128-133 + 157 for one stream):
    # modulate + int8 quantisation, the projection with qk_prep in its epilogue, attention
    # with merge_heads in its epilogue -- three launches.
    merged = [torch.empty((1, p.tokens, heads * 128), dtype=torch.bfloat16, device=dev) for _ in range(2)]

    def section(i):
        o = qkv_out[i % 2]
        w8a8.qk_prep(x3, qw, qs, ks, freqs, heads, out=o, modulation=(shift, scale))
        kernels.attend_merged(*o, out=merged[i % 2])

    section(0)
    section_ms = timed(section, args.kernel_launches)
    # A double block's two projections (modules.py:127-139): the first 512 tokens as the text
    # stream with its own weight, the rest as the image stream, each modulated, into one joint
    # q/k/v buffer -- two fused launches, or one for both (w8a8.qk_prep_pair).
    double = None
    if p.tokens > w_attn.num_txt:
        from flicker_amd.kernels import Freqs
        n_txt = w_attn.num_txt
        _, w_cpu = workloads.make_projection(p)
        qw_txt = w8a8.quantize_linear((-w_cpu).to(dev), w8a8.absmax_cols(x3[:, :n_txt]))
        txt = (x3[:, :n_txt], qw_txt, qs, ks, Freqs(freqs.cos[:n_txt], freqs.sin[:n_txt], freqs.q_gain))
        img = (x3[:, n_txt:], qw, qs, ks, Freqs(freqs.cos[n_txt:], freqs.sin[n_txt:], freqs.q_gain))

        def two(i):
            o = qkv_out[i % 2]
            w8a8.qk_prep(*txt, heads, out=o, out_offset=0, modulation=(shift, scale))
            w8a8.qk_prep(*img, heads, out=o, out_offset=n_txt, modulation=(shift, scale))

        def pair(i):
            w8a8.qk_prep_pair(txt, img, heads, out=qkv_out[i % 2], modulation=((shift, scale), (shift, scale)))

        def section2(i):   # the whole double-block attention section on this path
            from flicker_amd import modules
            modules.double_attention_int8(txt[0], img[0], qw_txt, qw, (qs, ks), (qs, ks), freqs, heads,
                                          modulation=((shift, scale), (shift, scale)))

        two(0)
        pair(0)
        section2(0)
        double = {"text_tokens": n_txt, "image_tokens": p.tokens - n_txt,
                  "two_launches_us": round(timed(two, args.kernel_launches) * 1e3, 2),
                  "pair_us": round(timed(pair, args.kernel_launches) * 1e3, 2),
                  "section_us": round(timed(section2, args.kernel_launches) * 1e3, 2),
                  "what": "modulate+quantise per stream, then the fused projection + qk_prep of both "
                          "streams: two launches of each, or one (the _pair entry points); section_us "
                          "adds the joint attend_merged (modules.double_attention_int8)"}
    del x3
    return {"workload": f"{p.name}: X ({p.tokens}, {p.hidden}) bf16 with {p.outlier_fraction:.0%} outlier "
                        f"channels x{p.outlier_gain:g}, W ({p.hidden}, {p.out_features}) ~ N(0, 0.02)",
            "roofline": {"bound": "mfma", "achieved": round(tops, 1), "peak": INT8_DENSE_PEAK_TOPS,
                         "unit": "TOP/s", "frac": round(tops / INT8_DENSE_PEAK_TOPS, 4), "kernel": "w8a8_gemm_kernel",
                         "ops_per_launch": p.gemm_ops(), "avg_launch_us": round(gemm_ms * 1e3, 2)},
            "quantize_act_us": round(quant_ms * 1e3, 2),
            "modulate_quantize_act_us": round(mod_ms * 1e3, 2),
            "gemm_then_qk_prep_us": round(unfused_ms * 1e3, 2),
            "fused_gemm_qk_prep_us": round(fused_ms * 1e3, 2),
            "block_section_us": round(section_ms * 1e3, 2),
            "block_section": "modulate+quantise -> int8 projection with qk_prep epilogue -> attend_merged",
            "double_block_projection": double,
            "dtype": "int8 operands, int32 accumulate, bf16 out"}


def _trace_rows(directory: str) -> list:
    """(kernel, blocks, start ns, end ns) of every dispatch in a kernel trace, in start order."""
    files = glob.glob(os.path.join(directory, "**", "*kernel_trace.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no kernel_trace.csv under {directory}")
    rows = []
    for f in files:
        for r in csv.DictReader(open(f)):
            name = r["Kernel_Name"].replace("void ", "", 1).replace("(anonymous namespace)::", "").split("(")[0]
            blocks = 1
            for a in "XYZ":
                blocks *= int(r["Grid_Size_" + a]) // max(1, int(r["Workgroup_Size_" + a]))
            rows.append((name, blocks, int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    rows.sort(key=lambda t: t[2])
    return rows


def ingest_trace(directory: str, min_run: int = 100, min_share: float = 0.002) -> str:
    """Markdown tables of a kernel trace: each run of >= min_run consecutive dispatches of one
    kernel and grid (a bench leg) with its mean duration and start-to-start period, then every
    kernel and grid with its dispatch statistics and share of the summed kernel time."""
    import statistics
    rows = _trace_rows(directory)
    out = ["| kernel | blocks | launches in the run | mean duration (us) | period start to start (us) |",
           "|---|---|---|---|---|"]
    run = []
    for r in rows + [None]:
        if run and (r is None or r[:2] != run[-1][:2]):
            if len(run) >= min_run:
                d = [(e - s) / 1e3 for _, _, s, e in run]
                period = (run[-1][2] - run[0][2]) / (len(run) - 1) / 1e3
                out.append(f"| `{run[0][0]}` | {run[0][1]} | {len(run)} | {sum(d) / len(d):.1f} | {period:.1f} |")
            run = []
        if r is not None:
            run.append(r)
    groups: dict = {}
    for name, blocks, s, e in rows:
        groups.setdefault((name, blocks), []).append((e - s) / 1e3)
    total = sum(sum(v) for v in groups.values())
    out += ["", "| kernel | blocks | calls | avg (us) | median (us) | min (us) | max (us) | share |",
            "|---|---|---|---|---|---|---|---|"]
    for (name, blocks), d in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
        if sum(d) < min_share * total:
            continue
        out.append(f"| `{name}` | {blocks} | {len(d)} | {sum(d) / len(d):.1f} | {statistics.median(d):.1f} | "
                   f"{min(d):.1f} | {max(d):.1f} | {100 * sum(d) / total:.2f}% |")
    return "\n".join(out)


def main() -> int:
    args = parse()
    if args.ingest_trace:
        print(ingest_trace(args.ingest_trace))
        return 0
    if args.ingest_mfma:
        summary = ingest_mfma(args.ingest_mfma, args.workload)
        with open(mfma_file(args.workload), "w") as f:
            json.dump(summary, f, indent=1)
        print(json.dumps({k: {m: round(v[m], 4) for m in ("mfma_busy", "sclk_ghz", "duration_us")}
                          for k, v in summary["kernels"].items()}))
        return 0
    if args.ingest_pmc:
        summary = ingest_pmc(args.ingest_pmc[0], args.ingest_pmc[1], args.workload)
        os.makedirs(os.path.dirname(traffic_file(args.workload)), exist_ok=True)
        with open(traffic_file(args.workload), "w") as f:
            json.dump(summary, f, indent=1)
        print(json.dumps(summary))
        return 0
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
    positions = rope.position_ids(ids, workloads.q_gain(w), device=dev)

    act_bytes = qkv_cpu.numel() * 2
    set_bytes = 2 * act_bytes + act_bytes // 3
    n_sets = max(2, -(-2 * INFINITY_CACHE_BYTES // set_bytes))
    sets = []
    for _ in range(n_sets):
        qkv = qkv_cpu.to(dev)
        out = tuple(torch.empty((w.batch, w.num_heads, w.length, w.head_dim), dtype=torch.bfloat16, device=dev)
                    for _ in range(3))
        o = torch.empty_like(out[0])
        sets.append((qkv, out, o))
    copies = []
    calib_gemm = None
    if args.only == "calibrate":
        for _ in range(4):
            copies.append((torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev).fill_(1),
                           torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev)))
        if not args.no_w8a8:   # the plain int8 GEMM too, for its traffic
            from flicker_amd import w8a8
            proj = workloads.PROJECTIONS[args.projection]
            _, cqw, cxq, ca = projection_operands(proj, dev)
            cy = torch.empty((proj.tokens, proj.out_features), dtype=torch.bfloat16, device=dev)
            calib_gemm = lambda: w8a8.gemm(cxq, ca, cqw.wq_t, cqw.w_scale, out=cy)  # noqa: E731

    def run_qk(i):
        qkv, out, _ = sets[i % n_sets]
        kernels.qk_prep(qkv, qs, ks, freqs, w.num_heads, out=out)

    def run_qk_ids(i):   # the same qk_prep with its RoPE lanes computed from the ids in-kernel
        qkv, out, _ = sets[i % n_sets]
        kernels.qk_prep(qkv, qs, ks, positions, w.num_heads, out=out)

    def run_attend(i):
        _, out, o = sets[i % n_sets]
        kernels.attend(*out, out=o)

    def step(i):
        run_qk(i)
        run_attend(i)
        if copies:
            src, dst = copies[i % len(copies)]
            dst.copy_(src)
        if calib_gemm is not None:
            calib_gemm()

    def timed(fn, n, name=None):
        """Average ms per call of n back-to-back calls between one pair of HIP events on the
        launch stream (torch's current stream, which the kernels are enqueued on)."""
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(n):
            fn(i)
        e1.record()
        e1.synchronize()
        return e0.elapsed_time(e1) / n

    def timed_graph(fn, n):
        """Average ms per call of fn with 2 * n_sets calls (every buffer set twice) captured
        into one HIP graph, replayed until about n calls have run, between one pair of HIP
        events.  Leaves out the Python enqueue of each call, which is longer than a short
        kernel (~16 us for qk_prep's host-side checks) and would otherwise be what is timed."""
        calls = 2 * n_sets
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):   # first calls outside the capture (allocator, plans)
            for i in range(calls):
                fn(i)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(calls):
                fn(i)
        graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()   # the GPU idled during the capture: replays until its clock is back
        while time.perf_counter() - t0 < args.leg_warmup_s:
            graph.replay()
            torch.cuda.synchronize()
        reps = max(1, -(-n // calls))
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            graph.replay()
        e1.record()
        e1.synchronize()
        return e0.elapsed_time(e1) / (reps * calls)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    # Clock warm-up: untimed steps for a fixed time, so the timed region starts at the GPU's
    # working clock whatever --warmup is (a few steps leave it ramping for ~1 s).
    clock_t0 = time.perf_counter()
    clock_steps = 0
    while time.perf_counter() - clock_t0 < args.clock_warmup_s:
        for _ in range(50):
            step(clock_steps)
            clock_steps += 1
        torch.cuda.synchronize()
    clock_warmup_s = time.perf_counter() - clock_t0 if clock_steps else 0.0
    step_ms = timed(step, args.steps)
    # Per-kernel launch durations: each kernel alone, back to back over the same rotating
    # buffers in a replayed HIP graph (what a rocprofv3 kernel trace of the same command
    # reports per dispatch, plus the small gaps between graph nodes).
    n_kernel = args.kernel_launches
    legs = {}   # per-leg (eager, graph) ms, for the record

    def timed_min(fn, n, name=None):
        """The smaller of the two GPU-inclusive timings: eager back-to-back launches (exact
        when the GPU is the bottleneck, inflated by the Python enqueue for short kernels) and
        a replayed HIP graph (no enqueue, but ~2 us between graph nodes)."""
        eager = timed(fn, n)
        graph = timed_graph(fn, n)
        if name:
            legs[name] = {"eager_us": round(eager * 1e3, 2), "graph_us": round(graph * 1e3, 2)}
        return min(eager, graph)

    def settled(timing):
        """`timing` preceded by back-to-back calls for --leg-warmup-s seconds: a leg often
        follows host-side setup during which the GPU idled and its clock fell, and the clock
        takes a fraction of a second of load to recover."""
        def run(fn, n, name=None):
            t0, i = time.perf_counter(), 0
            while time.perf_counter() - t0 < args.leg_warmup_s:
                for _ in range(10):
                    fn(i)
                    i += 1
                torch.cuda.synchronize()
            return timing(fn, n, name) if name else timing(fn, n)
        return run

    kernel_timed = settled(timed if args.eager_kernel_timing else timed_min)
    qk_ms = kernel_timed(run_qk, n_kernel, "qk_prep") if args.only == "step" else step_ms
    at_ms = kernel_timed(run_attend, n_kernel, "attend") if args.only == "step" else step_ms
    qk_gbs = w.qk_prep_bytes() / (qk_ms * 1e-3) / 1e9
    qk_ids_ms = kernel_timed(run_qk_ids, n_kernel, "qk_prep_ids") if args.only == "step" else None
    at_tflops = w.attend_flops() / (at_ms * 1e-3) / 1e12

    def p50_launch_us(fn, reps: int = 30) -> float:
        """The reference's method (tools/bench.py:21,25-33): the median of single calls, each
        between its own pair of events (reads high for short kernels: the events' own cost)."""
        durs = []
        for i in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn(i)
            e1.record()
            e1.synchronize()
            durs.append(e0.elapsed_time(e1) * 1e3)
        durs.sort()
        return round(durs[len(durs) // 2], 2)

    at_p50 = p50_launch_us(run_attend) if args.only == "step" else None
    qk_p50 = p50_launch_us(run_qk) if args.only == "step" else None

    traffic = {}
    if os.path.exists(traffic_file(w.name)):
        with open(traffic_file(w.name)) as f:
            traffic = json.load(f)["kernels"]
    source = os.path.relpath(traffic_file(w.name), ROOT) if traffic else None
    mfma = {}
    if os.path.exists(mfma_file(w.name)):
        with open(mfma_file(w.name)) as f:
            mfma = json.load(f)["kernels"]
    mfma_source = os.path.relpath(mfma_file(w.name), ROOT) if mfma else None

    def mfma_fields(kernel: str) -> dict:
        if kernel not in mfma:
            return {}
        return {"mfma_busy": round(mfma[kernel]["mfma_busy"], 4), "sclk_ghz": round(mfma[kernel]["sclk_ghz"], 3),
                "mfma_source": mfma_source}

    result = {
        "metric": METRIC,
        "value": round(at_tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "clock_warmup_s": round(clock_warmup_s, 2),
        "clock_warmup_steps": clock_steps,
        "kernel_launches": n_kernel if args.only == "step" else None,
        "leg_warmup_s": args.leg_warmup_s,
        "kernel_timing": "eager back-to-back launches" if args.eager_kernel_timing else
                         "min of eager back-to-back launches and a replayed HIP graph",
        "kernel_timings": legs or None,
        "ms_per_step": round(step_ms, 4),
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
                     "traffic": round(traffic["attend"]["traffic_bytes"]) if traffic else None,
                     "traffic_source": source,
                     "kernel": " + ".join(kernels.attend_kernels(w.batch, w.num_heads, w.length)),
                     "flops_per_launch": w.attend_flops(), "avg_launch_us": round(at_ms * 1e3, 2),
                     "p50_launch_us": at_p50,
                     **mfma_fields("attend")},
        "qk_prep": {"roofline": {"bound": "hbm", "achieved": round(qk_gbs, 1), "peak": HBM_PEAK_GBS,
                                 "unit": "GB/s", "frac": round(qk_gbs / HBM_PEAK_GBS, 4),
                                 "traffic": round(traffic["qk_prep"]["traffic_bytes"]) if traffic else None,
                                 "traffic_source": source, "kernel": "qk_prep_kernel",
                                 "bytes_per_launch": w.qk_prep_bytes(), "avg_launch_us": round(qk_ms * 1e3, 2),
                                 "p50_launch_us": qk_p50}},
    }
    if qk_ids_ms is not None:
        ids_gbs = w.qk_prep_bytes(tables=False) / (qk_ids_ms * 1e-3) / 1e9
        result["qk_prep"]["position_ids"] = {
            "avg_launch_us": round(qk_ids_ms * 1e3, 2), "bytes_per_launch": w.qk_prep_bytes(tables=False),
            "achieved": round(ids_gbs, 1), "unit": "GB/s", "frac": round(ids_gbs / HBM_PEAK_GBS, 4)}
    if args.only == "step" and w.num_heads % SHARE_GPUS == 0:
        result["head_share"] = head_share_leg(w, sets[0][1], kernel_timed)
    if not args.no_w8a8 and args.only == "step":
        result["w8a8"] = w8a8_leg(args, kernel_timed, dev)
        proj = workloads.PROJECTIONS[args.projection]
        result["w8a8"]["roofline"].update(mfma_fields("w8a8_gemm"))
        result["w8a8"]["roofline"]["bytes_per_launch"] = proj.gemm_bytes()
        if "w8a8_gemm" in traffic and proj.tokens == w.batch * w.length:
            result["w8a8"]["roofline"]["traffic"] = round(traffic["w8a8_gemm"]["traffic_bytes"])
            result["w8a8"]["roofline"]["traffic_source"] = source
    if args.workloads and args.only == "step":
        result["workloads"] = {name: workload_leg(name, kernel_timed, dev)
                               for name in args.workloads.split(",") if name and name != w.name}
    if not args.no_vendor and args.only == "step":
        gemm_us = result["w8a8"]["roofline"]["avg_launch_us"] if "w8a8" in result else None
        result["vendor"] = vendor_leg(w, [s[1] for s in sets], at_ms * 1e3, gemm_us, args, settled(timed), dev)
    if not args.no_cpu_baseline and args.only == "step":
        result["cpu_baseline"] = cpu_baseline(w, qkv_cpu, qs_cpu, ks_cpu, ids, args.cpu_reps)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
