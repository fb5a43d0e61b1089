"""Benchmark of the ragged-batch attention path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config C2] [--no-cpu-baseline]

A step is one decode step of the BASELINE headline workload (C2, Llama-3-8B shape): append the
step's new K/V row of each of the 64 sequences into the paged pool (sp_kv_append), then paged
decode attention over every sequence's context (sp_paged_decode). Inputs are resident in HBM
before the timed region starts. Prints one JSON line:
  value      algorithmic bytes of the step (append + decode) / measured step time, GB/s
  roofline   the decode launch: algorithmic bytes / its average duration (HIP events on the
             launch stream) against MI355X's 8 TB/s HBM peak
  cpu_baseline  the oracle's C port of the reference's decode op sequence (f32, OpenMP) timed
             on this host on the same workload
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
METRIC = "paged-decode HBM GB/s (% of peak) + ragged-prefill TFLOP/s, Llama-3-8B shape"


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="C2", choices=["C2", "C4", "C5", "C1"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="approximate CPU time budget of the cpu_baseline leg")
    ap.add_argument("--secondary", action="store_true",
                    help="also time the other decode configs (C4, C5) and report them")
    return ap.parse_args()


def traffic_from_profiles(kernel_tag: str):
    """HBM bytes per decode launch measured by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE,
    scaled by the copy-kernel calibration), read from the committed summary if present."""
    p = ROOT / "profiles" / f"{kernel_tag}_pmc.md"
    if not p.exists():
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", p.read_text())
    return float(m.group(1)) if m else None


def time_decode_config(w, steps: int, warmup: int):
    import torch
    import sketchpad_amd as sp
    from sketchpad_amd import workloads as W

    t = W.make_decode_tensors(w)
    lay = w.layout()
    max_ctx = w.max_context_len
    ws = sp.alloc_decode_workspace(w.num_seqs, w.hq, max_ctx, w.window_left, lay)
    scale = w.head_dim ** -0.5
    stream = torch.cuda.current_stream()

    def append():
        sp.kv_append(t["k_pool"], t["v_pool"], lay, t["k_new"], t["v_new"], t["slot_mapping"],
                     stream=stream.cuda_stream)

    def decode():
        sp.paged_decode(t["out"], t["q"], t["k_pool"], t["v_pool"], lay, t["block_tables"],
                        t["context_lens"], max_ctx, scale, window_left=w.window_left,
                        workspace=ws, stream=stream.cuda_stream)

    for _ in range(warmup):
        append()
        decode()
    torch.cuda.synchronize()

    # whole-step timing
    t0 = time.perf_counter()
    for _ in range(steps):
        append()
        decode()
    torch.cuda.synchronize()
    step_s = (time.perf_counter() - t0) / steps

    # per-launch timing of the decode with HIP events on the launch stream
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    for a, b in ev:
        append()
        a.record(stream)
        decode()
        b.record(stream)
    torch.cuda.synchronize()
    dec_ms = [a.elapsed_time(b) for a, b in ev]
    return {
        "step_s": step_s,
        "decode_ms_avg": float(np.mean(dec_ms)),
        "decode_ms_min": float(np.min(dec_ms)),
        "decode_bytes": w.decode_bytes(),
        "append_bytes": w.append_bytes(),
        "tensors": t,
    }


def cpu_baseline(w, t, budget_s: float):
    """Time the oracle's C port of the reference's decode op sequence on this host."""
    import torch
    from oracle import oracle as O

    threads = min(16, os.cpu_count() or 1)
    kp = t["k_pool"].float().cpu().numpy()
    vp = t["v_pool"].float().cpu().numpy()
    q = t["q"].float().cpu().numpy()
    kn = t["k_new"].float().cpu().numpy()
    vn = t["v_new"].float().cpu().numpy()
    out = np.empty_like(q)
    olay = O.make_layout(w.num_blocks, w.num_layers, w.layer, w.hkv, w.block_size, w.head_dim)
    reps, spent = 0, 0.0
    while spent < budget_s and reps < 100:
        t0 = time.perf_counter()
        O.cpu_decode_baseline(out, q, kn, vn, kp, vp, olay, w.block_tables, w.context_lens,
                              scale=w.head_dim ** -0.5, window_left=w.window_left,
                              threads=threads)
        spent += time.perf_counter() - t0
        reps += 1
    per_step = spent / reps
    bytes_step = w.decode_bytes() + w.append_bytes()
    return {
        "value": round(bytes_step / per_step / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{w.name}: {reps} full decode steps ({w.num_seqs} seqs, append + gather + "
                   f"repeat_kv + matmul/softmax/matmul, f32), {per_step * 1e3:.1f} ms/step"),
    }


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not supported "
              "(the path's sharding is described in DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    import torch
    from sketchpad_amd import workloads as W

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    w = W.DECODE_CONFIGS[args.config]()
    r = time_decode_config(w, args.steps, args.warmup)
    step_bytes = r["decode_bytes"] + r["append_bytes"]
    value = step_bytes / r["step_s"] / 1e9
    achieved = r["decode_bytes"] / (r["decode_ms_avg"] * 1e-3) / 1e9
    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["step_s"] * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": w.dtype,
        "data": "synthetic",
        "config": {
            "workload": f"{w.name}: append + paged decode, B={w.num_seqs}, Hq={w.hq}, "
                        f"Hkv={w.hkv}, D={w.head_dim}, BS={w.block_size}, "
                        f"L~U[{int(w.context_lens.min())},{int(w.context_lens.max())}] "
                        f"(sum {int(w.context_lens.sum())}), seed {w.seed:#x}",
            "tokens_attended": int(w.attended_keys().sum()),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic_from_profiles(f"paged_decode_{args.config.lower()}"),
            "kernel": "paged_decode_kernel + decode_combine_kernel (one sp_paged_decode call)",
            "algorithmic_bytes": r["decode_bytes"],
            "avg_ms": round(r["decode_ms_avg"], 5),
        },
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(w, r["tensors"], args.cpu_seconds)
    del r
    if args.secondary:
        sec = {}
        for name in ("C4", "C5", "C1"):
            if name == args.config:
                continue
            wx = W.DECODE_CONFIGS[name]()
            rx = time_decode_config(wx, max(5, args.steps // 2), 2)
            gbs = rx["decode_bytes"] / (rx["decode_ms_avg"] * 1e-3) / 1e9
            sec[name] = {"decode_ms": round(rx["decode_ms_avg"], 5), "decode_GBs": round(gbs, 2),
                         "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
            del rx
        line["secondary"] = sec
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
