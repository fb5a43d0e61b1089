"""Benchmark of the ragged-batch attention path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config C2] [--no-cpu-baseline]
                    [--no-prefill] [--secondary]
    python bench.py --calibrate-copy    # plain 512 MiB device copies (HBM counter calibration)

A step is one decode step of the headline workload (C2, Llama-3-8B shape): append the
step's new K/V row of each of the 64 sequences into the paged pool, then paged decode attention
over every sequence's context, both in one sp_paged_append_decode call (the append runs inside
the decode kernel; ms_per_step_separate_calls times the same step as sp_kv_append followed by
sp_paged_decode). Inputs are resident in HBM before the timed region starts. Prints one JSON
line:
  value      algorithmic bytes of the step (append + decode) / measured step time, GB/s
  roofline   the decode call: algorithmic bytes / its average duration (HIP events on the
             launch stream around K back-to-back calls) against MI355X's 8 TB/s HBM peak
  cpu_baseline  the oracle's C port of the reference's decode op sequence (f32, OpenMP) timed
             on this host on the same workload
  prefill    the C3 ragged causal prefill (sp_varlen_prefill, bf16 MFMA): average launch time
             over 10 back-to-back launches (and over 50: sustained MFMA load lowers the clock),
             TFLOP/s over the unmasked (query, key) pairs and the fraction of the 2.5 PFLOP/s
             dense bf16 peak, the C3 append, the C3 RoPE-fused append (sp_rope_kv_append: K
             rotated into the pool, V copied, Q rotated in place), the oracle's prefill port
             on a bounded sample, and (long_sequence) the same kernel on one causal
             8,192-token sequence at C3's heads
  polar_decode  the same decode step on PolarQuant-compressed pools (sp_polar_kv_append +
             sp_polar_paged_decode): launch time, algorithmic bytes (2 + D/2 per cached
             vector), GB/s, fraction of HBM peak, and the speed-up over the dense decode
  configs    C4 (one mixed iteration through sp_ragged_paged_attention: the prefill half's
             fraction of the bf16 MFMA peak, the decode half's fraction of HBM, the call against
             the serial bound) and the C5 / C1 decode calls' fractions of HBM
  gemma4_d256  head dim 256 (Gemma-4's sliding layers, 16 / 8 heads, 1024-key window): a paged
             decode batch and a windowed varlen prefill, with their roofline fractions
  gemma4_d512  head dim 512 (Gemma-4's global layers, 16 / 8 heads, causal, no window): the same
             two legs
Decode legs whose working set is below 512 MB (C5's window, the PolarQuant pools, C1) rotate
their timed calls over copies of the pools, so that more than 512 MB (twice the 256 MB MALL) of
K/V is read between two reads of the same byte; each reports its working set, the rotation and
the cache-warm time of the same call repeated on one copy beside it.
Each leg runs its W warmup steps and then keeps warming until 0.3 s have passed before its
timed region: a compute-bound kernel timed right after the GPU leaves idle runs at a lower
clock (C4's mixed step measured 298 us after 5 warm calls and 253 us after 400).
The CPU legs run on the threads OMP_NUM_THREADS allots (every CPU this process may use when it
is unset) and on one thread, and report the host's CPU model and counts.
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
MFMA_BF16_PEAK_TFLOPS = 2500.0
MFMA_FP32_PEAK_TFLOPS = 157.3
MIN_WARM_S = 0.3  # minimum warm-up wall time of every GPU leg
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
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run 10 plain 512 MiB device-to-device copies and exit")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the C3 prefill leg (profiling); prints its JSON object")
    ap.add_argument("--mixed-only", action="store_true",
                    help="only the C4 mixed ragged step (profiling); prints its JSON object")
    ap.add_argument("--flash-only", action="store_true",
                    help="only the f32 flash-attention leg (profiling); prints its JSON object")
    ap.add_argument("--no-prefill", action="store_true",
                    help="skip the C3 ragged-prefill leg")
    ap.add_argument("--no-polar", action="store_true",
                    help="skip the PolarQuant compressed-cache decode leg")
    ap.add_argument("--polar-only", action="store_true",
                    help="only the decode config's PolarQuant leg (profiling)")
    ap.add_argument("--decode-leg", choices=["C1", "C4", "C5"],
                    help="only that config's decode leg, timed as in the default line (pool "
                         "copies rotated past the MALL), for profiling; prints its JSON object")
    ap.add_argument("--gemma-only", action="store_true",
                    help="only the Gemma-4 decode and prefill legs, head dims 256 and 512 "
                         "(profiling)")
    ap.add_argument("--layer", action="store_true",
                    help="also time a whole attention layer (projections + RoPE append + "
                         "attention) on the C2 decode step and the C3 prefill")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the C4 mixed step and the C5 / C1 decode legs")
    ap.add_argument("--secondary", action="store_true",
                    help="also time C4's halves on their own, f32 flash attention and a layer")
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

    def append_decode():
        sp.paged_append_decode(t["out"], t["q"], t["k_pool"], t["v_pool"], lay, t["k_new"],
                               t["v_new"], t["block_tables"], t["context_lens"], max_ctx, scale,
                               window_left=w.window_left, workspace=ws,
                               stream=stream.cuda_stream)

    _warm(lambda: (append(), decode(), append_decode()), warmup)
    torch.cuda.synchronize()

    # whole-step timing: the step as one sp_paged_append_decode call, and as the two calls
    # sp_kv_append + sp_paged_decode
    def step_time(fn):
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps

    step_s = step_time(append_decode)
    step_s_separate = step_time(lambda: (append(), decode()))

    # the decode call's duration: HIP events on the launch stream around `steps` back-to-back calls
    dec_avg, dec_min = _event_times(stream, decode, steps)
    return {
        "step_s": step_s,
        "step_s_separate": step_s_separate,
        "decode_ms_avg": dec_avg,
        "decode_ms_min": dec_min,
        "decode_bytes": w.decode_bytes(),
        "append_bytes": w.append_bytes(),
        "tensors": t,
    }


def time_polar_decode(w, t, steps: int, warmup: int):
    """The same decode step on PolarQuant pools: sp_polar_kv_append of the step's rows, then
    sp_polar_paged_decode. Every slot of the pool holds an encoded random row first."""
    import torch
    import sketchpad_amd as sp
    from sketchpad_amd import workloads as W

    lay = w.layout()
    kp, vp = sp.alloc_polar_pools(lay)
    dt = W.torch_dtype(w.dtype)
    g = torch.Generator(device="cuda").manual_seed(w.seed)
    total = w.num_blocks * w.block_size
    for s0 in range(0, total, 16384):
        n = min(16384, total - s0)
        k = torch.randn(n, w.hkv, w.head_dim, generator=g, device="cuda").to(dt)
        v = torch.randn(n, w.hkv, w.head_dim, generator=g, device="cuda").to(dt)
        sp.polar_kv_append(kp, vp, lay, k, v,
                           torch.arange(s0, s0 + n, dtype=torch.int32, device="cuda"))
    max_ctx = w.max_context_len
    ws = sp.alloc_decode_workspace(w.num_seqs, w.hq, max_ctx, w.window_left, lay)
    scale = w.head_dim ** -0.5
    stream = torch.cuda.current_stream()
    db = w.polar_decode_bytes()
    # copies of the compressed pools for the past-the-MALL timing (rotation_copies)
    copies = rotation_copies(db)
    pools = [(kp, vp)] + [(kp.clone(), vp.clone()) for _ in range(copies - 1)]

    def append():
        sp.polar_kv_append(kp, vp, lay, t["k_new"], t["v_new"], t["slot_mapping"],
                           stream=stream.cuda_stream)

    def decode_on(kx, vx):
        return lambda: sp.polar_paged_decode(t["out"], t["q"], kx, vx, lay, t["block_tables"],
                                             t["context_lens"], max_ctx, scale,
                                             window_left=w.window_left, workspace=ws,
                                             stream=stream.cuda_stream)

    decode = decode_on(kp, vp)
    calls = [decode_on(kx, vx) for kx, vx in pools]
    _warm(lambda: (append(), [c() for c in calls]), warmup)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        append()
        decode()
    torch.cuda.synchronize()
    step_s = (time.perf_counter() - t0) / steps
    reps = max(steps, 4 * copies)
    dec_ms = _rotated_event_ms(stream, calls, reps)
    warm_ms = _rotated_event_ms(stream, calls[:1], reps)
    app_ms, _ = _event_times(stream, append, steps)
    return {
        "ms_per_step": round(step_s * 1e3, 4),
        "decode_ms": round(dec_ms, 5),
        "decode_bytes": db,
        "decode_GBs": round(db / (dec_ms * 1e-3) / 1e9, 2),
        "frac_hbm": round(db / (dec_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "working_set_bytes": db,
        "rotation": {"pool_copies": copies, "bytes_between_reuse": db * max(copies - 1, 1),
                     "protocol": "consecutive calls of the timed region read different copies of "
                                 "the compressed pools (more than 512 MB between two reads of "
                                 "the same byte)"},
        "decode_ms_cache_warm": round(warm_ms, 5),
        "append_ms": round(app_ms, 5),
        "append_bytes": w.polar_append_bytes(),
        "kernel": "polar_decode_kernel + decode_combine_kernel (one sp_polar_paged_decode call)",
    }


def host_cpu():
    """This host's CPU: model name, logical CPUs, the CPUs this process may run on, and the
    threads the CPU legs use: OMP_NUM_THREADS when set (the GPU box allots each GPU's job a
    share of its cores through it), else every CPU this process may run on."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        allowed = len(os.sched_getaffinity(0))
    except AttributeError:
        allowed = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS", "")
    threads = int(env) if env.isdigit() and int(env) > 0 else allowed
    return {"model": model, "nproc": os.cpu_count(), "affinity": allowed, "threads": threads,
            "threads_from": "OMP_NUM_THREADS" if env.isdigit() and int(env) > 0 else "affinity"}


def _timed_reps(fn, budget_s: float, max_reps: int, min_reps: int = 1):
    reps, spent = 0, 0.0
    while (spent < budget_s or reps < min_reps) and reps < max_reps:
        t0 = time.perf_counter()
        fn()
        spent += time.perf_counter() - t0
        reps += 1
    return spent / reps, reps


def cpu_baseline(w, t, budget_s: float):
    """Time the oracle's C port of the reference's decode op sequence on this host: full decode
    steps of the workload, on the host's allotted threads and on one thread."""
    import torch
    from oracle import oracle as O

    cpu = host_cpu()
    threads = cpu["threads"]
    kp = t["k_pool"].float().cpu().numpy()
    vp = t["v_pool"].float().cpu().numpy()
    q = t["q"].float().cpu().numpy()
    kn = t["k_new"].float().cpu().numpy()
    vn = t["v_new"].float().cpu().numpy()
    out = np.empty_like(q)
    olay = O.make_layout(w.num_blocks, w.num_layers, w.layer, w.hkv, w.block_size, w.head_dim)
    def step(nt):
        return lambda: O.cpu_decode_baseline(out, q, kn, vn, kp, vp, olay, w.block_tables,
                                             w.context_lens, scale=w.head_dim ** -0.5,
                                             window_left=w.window_left, threads=nt)

    per_step, reps = _timed_reps(step(threads), budget_s * 2 / 3, 100)
    per_1, reps_1 = _timed_reps(step(1), budget_s / 3, 20)
    bytes_step = w.decode_bytes() + w.append_bytes()
    return {
        "value": round(bytes_step / per_step / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{w.name}: {reps} full decode steps ({w.num_seqs} seqs, append + gather + "
                   f"repeat_kv + matmul/softmax/matmul, f32), {per_step * 1e3:.1f} ms/step on "
                   f"{threads} threads; {reps_1} on 1 thread, {per_1 * 1e3:.1f} ms/step"),
        "value_1_thread": round(bytes_step / per_1 / 1e9, 3),
        "host": cpu,
    }


def _warm(step, warmup: int):
    """`warmup` calls of step(), then more rounds of them until MIN_WARM_S has passed."""
    import torch
    t0 = time.perf_counter()
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    while time.perf_counter() - t0 < MIN_WARM_S:
        for _ in range(max(warmup, 1)):
            step()
        torch.cuda.synchronize()


def _event_times(stream, fn, reps: int):
    """Milliseconds per fn() call with HIP events recorded on the launch stream: the average over
    one timed region of `reps` back-to-back calls (what the roofline uses), and the minimum of
    `reps` individually bracketed calls (each bracket adds the event packets' own overhead)."""
    import torch
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(reps):
        fn()
    b.record(stream)
    torch.cuda.synchronize()
    avg = a.elapsed_time(b) / reps
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(reps)]
    for x, y in ev:
        x.record(stream)
        fn()
        y.record(stream)
    torch.cuda.synchronize()
    return float(avg), float(np.min([x.elapsed_time(y) for x, y in ev]))


MALL_CLEAR_BYTES = 512 << 20  # twice the 256 MB MALL


def rotation_copies(working_set: int) -> int:
    """Pool copies a timed region rotates over so that, between two reads of the same byte, more
    than 512 MB (twice the 256 MB MALL) of other K/V is read: one copy when a call's own working
    set is that large, else enough for the calls in between."""
    if working_set >= MALL_CLEAR_BYTES:
        return 1
    return 1 + -(-MALL_CLEAR_BYTES // working_set)


def _rotated_event_ms(stream, calls, reps: int):
    """ms per call of a HIP-event region of `reps` back-to-back calls, call i being
    calls[i % len(calls)] (each on its own copy of the pools)."""
    import torch
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for i in range(reps):
        calls[i % len(calls)]()
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


def time_decode_rotated(w, steps: int, warmup: int, softcap: float = 0.0):
    """A decode config's sp_paged_decode call timed past the MALL: the region rotates over
    rotation_copies(working set) copies of the K/V pools (same tables and contexts), so no call
    reads K/V a recent call left in the 256 MB MALL. Also reports the same call repeated on one
    copy (cache-warm) beside it. softcap > 0: sp_paged_decode_softcap."""
    import torch
    import sketchpad_amd as sp
    from sketchpad_amd import workloads as W

    t = W.make_decode_tensors(w)
    lay = w.layout()
    ws_bytes = w.decode_bytes()
    copies = rotation_copies(ws_bytes)
    pools = [(t["k_pool"], t["v_pool"])] + [(t["k_pool"].clone(), t["v_pool"].clone())
                                             for _ in range(copies - 1)]
    max_ctx = w.max_context_len
    ws = sp.alloc_decode_workspace(w.num_seqs, w.hq, max_ctx, w.window_left, lay)
    scale = w.head_dim ** -0.5
    stream = torch.cuda.current_stream()

    def call(kp, vp):
        return lambda: sp.paged_decode(t["out"], t["q"], kp, vp, lay, t["block_tables"],
                                       t["context_lens"], max_ctx, scale,
                                       window_left=w.window_left, workspace=ws,
                                       softcap=softcap, stream=stream.cuda_stream)

    calls = [call(kp, vp) for kp, vp in pools]
    _warm(lambda: [c() for c in calls], warmup)
    torch.cuda.synchronize()
    reps = max(steps, 4 * copies)
    ms = _rotated_event_ms(stream, calls, reps)
    warm_ms = _rotated_event_ms(stream, calls[:1], reps)
    return {"decode_ms": ms, "decode_ms_cache_warm": warm_ms, "decode_bytes": ws_bytes,
            "working_set_bytes": ws_bytes, "rotation_copies": copies,
            "bytes_between_reuse": ws_bytes * max(copies - 1, 1)}


def time_prefill_c3(steps: int, warmup: int):
    """C3: append every token's K/V into the paged pool, then ragged causal prefill over the
    packed stream (sp_varlen_prefill). Returns per-launch times of both."""
    import torch
    import sketchpad_amd as sp
    from sketchpad_amd import workloads as W

    w = W.prefill_c3()
    t = W.make_prefill_tensors(w)
    lay = sp.layout(t["num_blocks"], 1, 0, w.hkv, w.block_size, w.head_dim)
    stream = torch.cuda.current_stream()
    s = stream.cuda_stream

    def append():
        sp.kv_append(t["k_pool"], t["v_pool"], lay, t["k"], t["v"], t["slot_mapping"], stream=s)

    def prefill():
        sp.varlen_prefill(t["out"], t["q"], t["k"], t["v"], t["cu_seqlens"], t["cu_seqlens"],
                          w.max_seqlen, w.head_dim ** -0.5, stream=s)

    _warm(lambda: (append(), prefill()), warmup)
    torch.cuda.synchronize()
    # RoPE fused into the append: rotate K into the pool, copy V, rotate Q in place, one pass
    cos, sin = sp.rope_tables(int(w.lens.max()), w.head_dim, 500000.0)
    cos_d, sin_d = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
    positions = torch.from_numpy(
        np.concatenate([np.arange(L) for L in w.lens]).astype(np.int32)).cuda()
    q_rope = t["q"].clone()

    def rope_append():
        sp.rope_kv_append(t["k_pool"], t["v_pool"], lay, t["k"], t["v"], positions,
                          t["slot_mapping"], cos_d, sin_d, q=q_rope, stream=s)

    rope_append()
    torch.cuda.synchronize()
    # Sustained MFMA load lowers the clock within a few ms (per-launch times climb from ~150 to
    # ~185 us over 50 back-to-back C3 launches), so the roofline is a 10-launch region and the
    # sustained figure is reported beside it.
    pf_ms, pf_min = _event_times(stream, prefill, 10)
    pf_sus, _ = _event_times(stream, prefill, max(50, steps))
    ap_ms, _ = _event_times(stream, append, steps)
    ra_ms, _ = _event_times(stream, rope_append, steps)
    flops = w.flops()
    tflops = flops / (pf_ms * 1e-3) / 1e12
    e = 2
    append_bytes = w.total_tokens * w.hkv * w.head_dim * e * 2 * 2 + w.total_tokens * 4
    # K, V rows read and written, Q rows read and written, slot + position, one table row each
    rope_bytes = (w.total_tokens * (w.hkv * 4 + w.hq * 2) * w.head_dim * e
                  + w.total_tokens * (8 + w.head_dim * 4))
    return w, {
        "workload": f"{w.name}: B={w.num_seqs}, lens={[int(x) for x in w.lens]} "
                    f"(sum {w.total_tokens}), Hq={w.hq}, Hkv={w.hkv}, D={w.head_dim}, causal, "
                    f"seed {w.seed:#x}",
        "ms": round(pf_ms, 5),
        "ms_min": round(pf_min, 5),
        "ms_sustained_50": round(pf_sus, 5),
        "tflops": round(tflops, 2),
        "tflops_sustained_50": round(flops / (pf_sus * 1e-3) / 1e12, 2),
        "roofline": {
            "bound": "mfma",
            "achieved": round(tflops, 2),
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
            "kernel": "prefill_k32_kernel<bf16,128> (one sp_varlen_prefill call)",
            "algorithmic_flops": flops,
        },
        "append": {"ms": round(ap_ms, 5), "bytes": append_bytes,
                   "GBs": round(append_bytes / (ap_ms * 1e-3) / 1e9, 2)},
        "rope_append": {"ms": round(ra_ms, 5), "bytes": rope_bytes,
                        "GBs": round(rope_bytes / (ra_ms * 1e-3) / 1e9, 2)},
    }


def time_prefill_long(steps: int):
    """C3's heads and head dim on one long sequence: a causal 8,192-token prefill (32 / 8 heads,
    D 128, bf16) through sp_varlen_prefill, for the kernel's MFMA fraction on long key walks
    beside C3's short ones (same warm-up and 10-launch region as the C3 leg)."""
    import torch
    import sketchpad_amd as sp
    from sketchpad_amd import workloads as W

    c3 = W.prefill_c3()
    w = W.PrefillWorkload("causal-8192-llama3-8b-heads", c3.seed + 100, np.array([8192], np.int32),
                          c3.hq, c3.hkv, c3.head_dim, c3.dtype)
    t = W.make_prefill_tensors(w, with_pool=False)
    stream = torch.cuda.current_stream()

    def prefill():
        sp.varlen_prefill(t["out"], t["q"], t["k"], t["v"], t["cu_seqlens"], t["cu_seqlens"],
                          w.max_seqlen, w.head_dim ** -0.5, stream=stream.cuda_stream)

    _warm(prefill, 3)
    torch.cuda.synchronize()
    ms, ms_min = _event_times(stream, prefill, max(10, steps))
    tflops = w.flops() / (ms * 1e-3) / 1e12
    return {"workload": f"{w.name}: B=1, L=8192, Hq={w.hq}, Hkv={w.hkv}, D={w.head_dim}, causal",
            "ms": round(ms, 5), "ms_min": round(ms_min, 5), "tflops": round(tflops, 2),
            "frac_mfma": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
            "kernel": "prefill_k32_kernel<bf16,128> (one sp_varlen_prefill call)"}


GEMMA4_LOGIT_SOFTCAP = 50.0  # attn_logit_softcap (crates/sketchpad-llm/src/gemma4.rs:96)


def time_gemma4(steps: int, head_dim: int):
    """Gemma-4's two attention shapes, 16 query / 8 KV heads (gemma4.rs:82-107): head dim 256
    (the sliding-window layers, a 1024-key window) and 512 (the global layers, causal with no
    window). The paged decode (decode_gemma4_d256 / _d512, timed past the MALL) and the causal
    varlen prefill (prefill_gemma4_d256 / _d512, TFLOP/s over the visible pairs), each as Gemma-4
    runs it (logit soft cap 50, the *_softcap entry points) and without the cap."""
    import torch
    import sketchpad_amd as sp
    from sketchpad_amd import workloads as W

    cap = GEMMA4_LOGIT_SOFTCAP
    if head_dim == 256:
        dw, w = W.decode_gemma4_d256(), W.prefill_gemma4_d256()
        kernel = "prefill_wide_kernel<bf16,256,false{}>"
    else:
        dw, w = W.decode_gemma4_d512(), W.prefill_gemma4_d512()
        kernel = "prefill_d512_kernel<bf16,false{}>"
    name = f"gemma4-d{head_dim}"
    dec = time_decode_leg(name, steps, dw)
    dec_cap = time_decode_leg(name, steps, dw, softcap=cap)
    t = W.make_prefill_tensors(w, with_pool=False)
    stream = torch.cuda.current_stream()

    def prefill(softcap):
        return lambda: sp.varlen_prefill(t["out"], t["q"], t["k"], t["v"], t["cu_seqlens"],
                                         t["cu_seqlens"], w.max_seqlen, w.head_dim ** -0.5,
                                         window_left=w.window_left, softcap=softcap,
                                         stream=stream.cuda_stream)

    window = f"window_left {w.window_left}" if w.window_left >= 0 else "no window"
    res = {}
    for key, c in (("prefill", 0.0), ("prefill_softcap", cap)):
        fn = prefill(c)
        _warm(fn, 3)
        torch.cuda.synchronize()
        ms, _ = _event_times(stream, fn, max(10, steps))
        tflops = w.flops() / (ms * 1e-3) / 1e12
        res[key] = {"workload": f"{w.name}: B={w.num_seqs}, lens={[int(x) for x in w.lens]}, "
                                f"Hq={w.hq}, Hkv={w.hkv}, D={w.head_dim}, causal, {window}, "
                                f"logit softcap {c:g}",
                    "ms": round(ms, 5), "flops": w.flops(), "tflops": round(tflops, 2),
                    "frac_mfma": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                    "kernel": kernel.format(",true" if c else "")}
    dec_cap["logit_softcap"] = cap
    return {"decode": dec, "decode_softcap": dec_cap, **res}


def time_layer(steps: int, warmup: int, hidden: int = 4096):
    """One whole attention layer of the Llama-3-8B shape (hidden 4096): q and k|v projections
    (sp_linear), RoPE fused into the append (sp_rope_kv_append), attention, o projection — on the
    C2 decode step (64 tokens, sp_paged_decode) and on the C3 prefill (9,476 tokens,
    sp_paged_prefill through the pool). Returns per-part HIP-event times; random weights,
    synthetic inputs."""
    import torch
    import sketchpad_amd as sp
    from sketchpad_amd import workloads as W

    stream = torch.cuda.current_stream()
    s = stream.cuda_stream
    res = {}
    for name in ("decode_C2", "prefill_C3"):
        if name == "decode_C2":
            w = W.decode_c2()
            t = W.make_decode_tensors(w)
            T, hq, hkv, d = w.num_seqs, w.hq, w.hkv, w.head_dim
            lay = w.layout()
            positions = torch.from_numpy((w.context_lens - 1).astype(np.int32)).cuda()
            slots, k_pool, v_pool = t["slot_mapping"], t["k_pool"], t["v_pool"]
            ws = sp.alloc_decode_workspace(T, hq, w.max_context_len, -1, lay)
            rows = w.max_context_len
            attn_bytes = w.decode_bytes()
        else:
            w = W.prefill_c3()
            t = W.make_prefill_tensors(w)
            T, hq, hkv, d = w.total_tokens, w.hq, w.hkv, w.head_dim
            lay = sp.layout(t["num_blocks"], 1, 0, hkv, w.block_size, d)
            positions = torch.from_numpy(
                np.concatenate([np.arange(L) for L in w.lens]).astype(np.int32)).cuda()
            slots, k_pool, v_pool = t["slot_mapping"], t["k_pool"], t["v_pool"]
            rows = int(w.lens.max())
        dt = W.torch_dtype("bf16")
        g = torch.Generator(device="cuda").manual_seed(7)
        x = torch.randn(T, hidden, generator=g, device="cuda").to(dt)
        # weights [out, in]
        wq = (torch.randn(hq * d, hidden, generator=g, device="cuda") * hidden ** -0.5).to(dt)
        wkv = (torch.randn(2 * hkv * d, hidden, generator=g, device="cuda") * hidden ** -0.5).to(dt)
        wo = (torch.randn(hidden, hq * d, generator=g, device="cuda") * (hq * d) ** -0.5).to(dt)
        q = torch.empty(T, hq, d, dtype=dt, device="cuda")
        kv = torch.empty(T, 2 * hkv * d, dtype=dt, device="cuda")
        attn = torch.empty(T, hq, d, dtype=dt, device="cuda")
        out = torch.empty(T, hidden, dtype=dt, device="cuda")
        lws = sp.alloc_linear_workspace([(T, hidden, hq * d), (T, hidden, 2 * hkv * d),
                                         (T, hq * d, hidden)])
        cos, sin = sp.rope_tables(rows, d, 500000.0)
        cos_d, sin_d = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()

        def qkv():
            sp.linear(q, x, wq, workspace=lws, stream=s)
            sp.linear(kv, x, wkv, workspace=lws, stream=s)

        def rope_append():
            sp.rope_kv_append(k_pool, v_pool, lay, kv[:, :hkv * d], kv[:, hkv * d:], positions,
                              slots, cos_d, sin_d, q=q, token_stride=2 * hkv * d, head_stride=d,
                              stream=s)

        if name == "decode_C2":
            def attention():
                sp.paged_decode(attn, q, k_pool, v_pool, lay, t["block_tables"],
                                t["context_lens"], w.max_context_len, d ** -0.5, workspace=ws,
                                stream=s)
        else:
            lens_d = torch.from_numpy(w.lens.astype(np.int32)).cuda()
            pws = sp.alloc_paged_prefill_workspace(w.num_seqs, w.max_seqlen, hq, lay,
                                                   t["block_tables"].shape[1])

            def attention():  # the new tokens attend through the pool they were appended to
                sp.paged_prefill(attn, q, k_pool, v_pool, lay, t["block_tables"], t["cu_seqlens"],
                                 lens_d, w.max_seqlen, d ** -0.5, workspace=pws, stream=s)

        def o_proj():
            sp.linear(out, attn.view(T, hq * d), wo, workspace=lws, stream=s)

        def layer():
            qkv()
            rope_append()
            attention()
            o_proj()

        _warm(layer, warmup)
        torch.cuda.synchronize()
        n = max(10, steps // 2)
        parts = {k: _event_times(stream, f, n)[0]
                 for k, f in (("qkv_proj", qkv), ("rope_append", rope_append),
                              ("attention", attention), ("o_proj", o_proj), ("layer", layer))}
        wbytes = hidden * (hq + 2 * hkv) * d * 2
        obytes = hq * d * hidden * 2
        entry = {k + "_ms": round(v, 5) for k, v in parts.items()}
        entry["tokens"] = T
        entry["qkv_proj_TFLOPs"] = round(2 * T * hidden * (hq + 2 * hkv) * d /
                                         (parts["qkv_proj"] * 1e-3) / 1e12, 2)
        entry["o_proj_TFLOPs"] = round(2 * T * hq * d * hidden / (parts["o_proj"] * 1e-3) / 1e12, 2)
        entry["qkv_proj_weight_GBs"] = round(wbytes / (parts["qkv_proj"] * 1e-3) / 1e9, 2)
        entry["o_proj_weight_GBs"] = round(obytes / (parts["o_proj"] * 1e-3) / 1e9, 2)
        if name == "decode_C2":
            entry["attention_GBs"] = round(attn_bytes / (parts["attention"] * 1e-3) / 1e9, 2)
        else:
            entry["attention_TFLOPs"] = round(w.flops() / (parts["attention"] * 1e-3) / 1e12, 2)
        entry["attention_share"] = round(parts["attention"] / parts["layer"], 3)
        res[name] = entry
        del t
    return res


def time_chunked_c4(steps: int, warmup: int):
    """C4 prefill half: 4 chunks of 512 new tokens against paged contexts (sp_paged_prefill)."""
    import torch
    import sketchpad_amd as sp
    from sketchpad_amd import workloads as W

    w = W.chunked_prefill_c4()
    t = W.make_chunked_tensors(w)
    lay = sp.layout(t["num_blocks"], 1, 0, w.hkv, w.block_size, w.head_dim)
    stream = torch.cuda.current_stream()
    s = stream.cuda_stream
    sp.kv_append(t["k_pool"], t["v_pool"], lay, t["k_new"], t["v_new"], t["slot_mapping"],
                 stream=s)

    # the workspace lets sp_paged_prefill split the long contexts' keys over workgroups
    ws = sp.alloc_paged_prefill_workspace(w.num_seqs, w.max_seqlen_q, w.hq, lay,
                                          t["block_tables"].shape[1])

    def run(workspace):
        def prefill():
            sp.paged_prefill(t["out"], t["q"], t["k_pool"], t["v_pool"], lay, t["block_tables"],
                             t["cu_seqlens_q"], t["context_lens"], w.max_seqlen_q,
                             w.head_dim ** -0.5, workspace=workspace, stream=s)

        _warm(prefill, warmup)
        torch.cuda.synchronize()
        return _event_times(stream, prefill, steps)[0]

    ms_unsplit = run(None)
    ms = run(ws)
    tflops = w.flops() / (ms * 1e-3) / 1e12
    return {"ms": round(ms, 5), "tflops": round(tflops, 2),
            "frac_mfma": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
            "workspace_bytes": 0 if ws is None else ws.numel(),
            "ms_without_key_split": round(ms_unsplit, 5)}


def time_flash_f32(steps: int, warmup: int, b: int = 2, h: int = 8, s: int = 4096, d: int = 64):
    """sp_flash_attention in f32 (the reference flash_attention's element type) on a dense
    non-causal [2, 8, 4096, 64] batch (self-attention at a diffusion UNet's 64x64 latent):
    TFLOP/s (4 B H S^2 D) against the 157.3 TFLOP/s dense fp32 MFMA peak."""
    import torch
    import sketchpad_amd as sp

    g = torch.Generator(device="cuda").manual_seed(7)
    q, k, v = (torch.randn(b, h, s, d, generator=g, device="cuda") for _ in range(3))
    out = torch.empty_like(q)
    stream = torch.cuda.current_stream()

    def attn():
        sp.flash_attention(out, q, k, v, d ** -0.5, causal=False, stream=stream.cuda_stream)

    _warm(attn, warmup)
    torch.cuda.synchronize()
    ms, _ = _event_times(stream, attn, steps)
    tflops = 4 * b * h * s * s * d / (ms * 1e-3) / 1e12
    return {"shape": [b, h, s, d], "ms": round(ms, 4), "tflops": round(tflops, 2),
            "frac_fp32_mfma": round(tflops / MFMA_FP32_PEAK_TFLOPS, 4)}


def cpu_prefill_baseline(w, budget_s: float):
    """The oracle's C port of the reference's prefill op sequence ([Hq, L, L] f32 scores per
    sequence) on the whole C3 workload (all eight sequences), on the host's allotted threads and
    on one thread."""
    import torch
    from oracle import oracle as O
    from sketchpad_amd import workloads as W

    cpu = host_cpu()
    threads = cpu["threads"]
    t = W.make_prefill_tensors(w, device="cpu", with_pool=False)
    q, k, v = (t[n].float().numpy() for n in ("q", "k", "v"))
    out = np.empty_like(q)

    def run(nt):
        return lambda: O.cpu_prefill_baseline(out, q, k, v, w.cu_seqlens, hq=w.hq, hkv=w.hkv,
                                              d=w.head_dim, scale=w.head_dim ** -0.5,
                                              threads=nt)

    per, reps = _timed_reps(run(threads), budget_s * 2 / 3, 50)
    per_1, reps_1 = _timed_reps(run(1), budget_s / 3, 5)
    return {"value": round(w.flops() / per / 1e12, 5), "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": f"the whole C3 batch ({w.num_seqs} sequences, {w.total_tokens} tokens): "
                      f"{reps} causal prefills (repeat_kv + [Hq,L,L] f32 scores + mask + softmax "
                      f"+ matmul per sequence), {per * 1e3:.1f} ms each on {threads} threads; "
                      f"{reps_1} on 1 thread, {per_1 * 1e3:.1f} ms",
            "value_1_thread": round(w.flops() / per_1 / 1e12, 5),
            "host": cpu}


def time_mixed_c4(steps: int, warmup: int):
    """C4, one scheduler iteration as one ragged batch over one pool:
    append the 2,176 new tokens, then sp_ragged_paged_attention (chunked prefill over the 4
    chunks on the caller's stream, decode over the 128 one-token sequences on the library's side
    stream, forked and joined with events so the two overlap). Reports the attention call,
    its two halves timed on their own, the prefill's fraction of the bf16 MFMA peak, the
    decode's fraction of HBM, and the whole call against the serial bound
    F / 2.5 PFLOP/s + B / 8 TB/s and the overlapped bound max(F / 2.5 PFLOP/s, B / 8 TB/s)."""
    import torch
    import sketchpad_amd as sp
    from sketchpad_amd import workloads as W

    w = W.mixed_c4()
    t = W.make_mixed_tensors(w)
    lay = sp.layout(t["num_blocks"], 1, 0, w.hkv, w.block_size, w.head_dim)
    stream = torch.cuda.current_stream()
    s = stream.cuda_stream
    P, T0 = w.num_prefill_seqs, w.num_prefill_tokens
    pmax, dmax = int(w.chunk_lens.max()), int(w.decode_lens.max())
    mb = t["block_tables"].shape[1]
    ws = sp.alloc_ragged_workspace(w.num_seqs, P, pmax, dmax, w.hq, lay, mb)
    scale = w.head_dim ** -0.5

    def append():
        sp.kv_append(t["k_pool"], t["v_pool"], lay, t["k_new"], t["v_new"], t["slot_mapping"],
                     stream=s)

    def attention():
        sp.ragged_paged_attention(t["out"], t["q"], t["k_pool"], t["v_pool"], lay,
                                  t["block_tables"], t["cu_seqlens_q"], t["context_lens"],
                                  num_prefill_seqs=P, num_prefill_tokens=T0,
                                  prefill_max_seqlen_q=pmax, decode_max_context_len=dmax,
                                  scale=scale, workspace=ws, stream=s)

    def prefill_half():
        sp.paged_prefill(t["out"][:T0], t["q"][:T0], t["k_pool"], t["v_pool"], lay,
                         t["block_tables"][:P], t["cu_seqlens_q"], t["context_lens"][:P], pmax,
                         scale, workspace=ws, stream=s)

    def decode_half():
        sp.paged_decode(t["out"][T0:], t["q"][T0:], t["k_pool"], t["v_pool"], lay,
                        t["block_tables"][P:], t["context_lens"][P:], dmax, scale, workspace=ws,
                        stream=s)

    _warm(lambda: (append(), attention()), warmup)
    torch.cuda.synchronize()
    at_ms, _ = _event_times(stream, attention, steps)
    ap_ms, _ = _event_times(stream, append, steps)
    pf_ms, _ = _event_times(stream, prefill_half, steps)
    dc_ms, _ = _event_times(stream, decode_half, steps)
    F, B = w.prefill_flops(), w.decode_bytes()
    bound_ms = (F / (MFMA_BF16_PEAK_TFLOPS * 1e12) + B / (HBM_PEAK_GBS * 1e9)) * 1e3
    overlap_ms = max(F / (MFMA_BF16_PEAK_TFLOPS * 1e12), B / (HBM_PEAK_GBS * 1e9)) * 1e3
    pf_tf = F / (pf_ms * 1e-3) / 1e12
    dc_gbs = B / (dc_ms * 1e-3) / 1e9
    return {
        "workload": f"{w.name}: {P} chunks of {list(map(int, w.chunk_lens))} new tokens on "
                    f"contexts {list(map(int, w.ctx_before))} + {w.num_decode_seqs} decode seqs "
                    f"L~U[{int(w.decode_lens.min())},{int(w.decode_lens.max())}], Hq={w.hq}, "
                    f"Hkv={w.hkv}, D={w.head_dim}, one pool, seed {w.seed:#x}",
        "attention_ms": round(at_ms, 5),
        "append_ms": round(ap_ms, 5),
        "prefill_ms": round(pf_ms, 5),
        "prefill_tflops": round(pf_tf, 2),
        "prefill_frac_mfma": round(pf_tf / MFMA_BF16_PEAK_TFLOPS, 4),
        "prefill_flops": F,
        "decode_ms": round(dc_ms, 5),
        "decode_GBs": round(dc_gbs, 2),
        "decode_frac_hbm": round(dc_gbs / HBM_PEAK_GBS, 4),
        "decode_bytes": B,
        "serial_bound_ms": round(bound_ms, 5),
        "frac_of_serial_bound": round(bound_ms / at_ms, 4),
        "overlap_bound_ms": round(overlap_ms, 5),
        "frac_of_overlap_bound": round(overlap_ms / at_ms, 4),
        "kernels": "sp_ragged_paged_attention: prefill_kernel<bf16,128,true> on the caller's "
                   "stream, concurrently with paged_decode_kernel + decode_combine_kernel on "
                   "the side stream",
    }


def time_decode_leg(name: str, steps: int, w=None, softcap: float = 0.0):
    """A decode config's sp_paged_decode call timed past the MALL (time_decode_rotated): ms,
    GB/s over its algorithmic bytes, fraction of HBM, the working set and the rotation used."""
    from sketchpad_amd import workloads as W
    wx = W.DECODE_CONFIGS[name]() if w is None else w
    rx = time_decode_rotated(wx, steps, 2, softcap)
    gbs = rx["decode_bytes"] / (rx["decode_ms"] * 1e-3) / 1e9
    return {"workload": f"{wx.name}: B={wx.num_seqs}, Hq={wx.hq}, Hkv={wx.hkv}, D={wx.head_dim}, "
                        f"{wx.dtype}, window {wx.window_left}, "
                        f"L~U[{int(wx.context_lens.min())},{int(wx.context_lens.max())}]",
            "decode_ms": round(rx["decode_ms"], 5), "decode_bytes": rx["decode_bytes"],
            "decode_GBs": round(gbs, 2), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
            "working_set_bytes": rx["working_set_bytes"],
            "rotation": {"pool_copies": rx["rotation_copies"],
                         "bytes_between_reuse": rx["bytes_between_reuse"],
                         "protocol": "consecutive calls of the timed region read different copies "
                                     "of the pools, so more than 512 MB (twice the MALL) of K/V "
                                     "is read between two reads of the same byte"},
            "decode_ms_cache_warm": round(rx["decode_ms_cache_warm"], 5)}


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not supported "
              "(multi-GPU sharding of the attention path is not built)", file=sys.stderr)
        sys.exit(2)
    import torch
    from sketchpad_amd import workloads as W

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    if args.calibrate_copy:
        # counter calibration: 10 runtime device copies (512 MiB read + 512 MiB written each),
        # then 10 sp_kv_gather calls of one 131,072-token sequence (bf16, 8 KV heads, D 128):
        # 256 MiB of K and 256 MiB of V read from the pools with the 16-byte loads the decode
        # kernel uses, the same bytes written out
        import sketchpad_amd as sp
        src = torch.ones(512 << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        del dst
        tokens, hkv, d, bs = 131072, 8, 128, 16
        lay = sp.layout(tokens // bs, 1, 0, hkv, bs, d)
        kp = torch.randn(tokens // bs, 1, hkv, bs, d, device="cuda").bfloat16()
        vp = torch.randn_like(kp)
        table = torch.randperm(tokens // bs, device="cuda").int()
        ko = torch.empty(hkv, tokens, d, dtype=torch.bfloat16, device="cuda")
        vo = torch.empty_like(ko)
        for _ in range(10):
            sp.kv_gather(ko, vo, kp, vp, lay, table, tokens)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": src.numel(), "copies": 10,
                          "gather_read_bytes": 2 * kp.numel() * 2, "gathers": 10}), flush=True)
        return
    if args.mixed_only:
        print(json.dumps({"C4_mixed": time_mixed_c4(args.steps, args.warmup)}), flush=True)
        return
    if args.flash_only:
        print(json.dumps({"flash_f32": time_flash_f32(args.steps, args.warmup)}), flush=True)
        return
    if args.prefill_only:
        _, pf = time_prefill_c3(args.steps, args.warmup)
        print(json.dumps({"prefill": pf}), flush=True)
        return
    if args.decode_leg:
        print(json.dumps({args.decode_leg: time_decode_leg(args.decode_leg, args.steps)}),
              flush=True)
        return
    if args.gemma_only:
        print(json.dumps({"gemma4_d256": time_gemma4(args.steps, 256),
                          "gemma4_d512": time_gemma4(args.steps, 512)}), flush=True)
        return
    w = W.DECODE_CONFIGS[args.config]()
    if args.polar_only:
        pq = time_polar_decode(w, W.make_decode_tensors(w), args.steps, args.warmup)
        print(json.dumps({"polar_decode": pq}), flush=True)
        return
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
        "ms_per_step_separate_calls": round(r["step_s_separate"] * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": w.dtype,
        "data": "synthetic",
        "config": {
            "workload": f"{w.name}: append + paged decode in one sp_paged_append_decode call, "
                        f"B={w.num_seqs}, Hq={w.hq}, "
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
    if not args.no_polar and w.dtype in ("bf16", "f16"):
        pq = time_polar_decode(w, r["tensors"], args.steps, args.warmup)
        pq["decode_speedup_vs_dense"] = round(r["decode_ms_avg"] / pq["decode_ms"], 3)
        line["polar_decode"] = pq
    del r
    if not args.no_prefill:
        wp, pf = time_prefill_c3(max(10, args.steps // 2), 3)
        if not args.no_cpu_baseline:
            pf["cpu_baseline"] = cpu_prefill_baseline(wp, args.cpu_seconds)
        pf["long_sequence"] = time_prefill_long(10)
        line["prefill"] = pf
    if not args.no_configs:
        # the other benchmark configurations: C4 (one mixed iteration), C5, C1
        cfg = {"C4": time_mixed_c4(max(10, args.steps // 2), 2)}
        for name in ("C5", "C1"):
            if name != args.config:
                cfg[name] = time_decode_leg(name, max(10, args.steps // 2))
        line["configs"] = cfg
        line["gemma4_d256"] = time_gemma4(max(10, args.steps // 2), 256)
        line["gemma4_d512"] = time_gemma4(max(10, args.steps // 2), 512)
    if args.secondary:
        sec = line.setdefault("secondary", {})
        sec["C4-chunked-prefill"] = time_chunked_c4(10, 2)
        sec["C4-decode"] = time_decode_leg("C4", max(5, args.steps // 2))
        sec["flash-attention-f32"] = time_flash_f32(5, 2)
    if args.layer or args.secondary:
        line["layer"] = time_layer(args.steps, 3)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
