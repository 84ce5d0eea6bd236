#!/usr/bin/env python
"""Decode throughput of the SAGA + Atop-N path on one MI355X.

Workload (the headline configuration): a Qwen2.5-1.5B-shaped SAGA decoder
(28 layers, hidden 1536, 12 query / 1 key / 2 value heads, head_dim 128,
vocab 151936), random-init bf16 weights, batch 8, a 32768-token random-id
prompt prefilled at batch 1 and replicated (as speedup.py:146-161), then
`--steps` decode steps with Atop-N N=512 (the first step calibrates),
replayed as HIP graphs.  value = batch * steps / decode wall time.

Also reported on the same line:
  roofline      the dominant kernel (K1, QK scores streaming the K cache):
                algorithmic bytes per launch / its average duration, timed
                with HIP events over a graph of launches on the stream they
                run on, against the 8 TB/s HBM peak;
  attention_call_roofline
                the whole Atop-N fast step (every kernel of one call) at the
                decoder's state: K + the distinct V rows it selects (per batch
                row and value head, counted from the workspace) + Q/O +
                thresholds, over the call's average duration;
  hbm_copy_GBs  a measured device-to-device copy (bytes read + written /
                time), beside the 8 TB/s spec;
  c5            the 128k comparison: batch 4, 131072 positions, SAGA 1K/2V
                with Atop-N N=1024 against dense GQA 2K/2V, attention alone on
                the same seeded N(0,1) caches, microseconds per call and ratio;
  cpu_baseline  the CPU oracle (the reference's fp32 path restated in numpy)
                on all host cores: per-layer decode-attention latency at the
                C1 (b1, 15/1/5 heads, d64, 4096 positions, N=128), C3 (this
                workload) and C5 (b4, 128k, N=1024) shapes, and attention
                tokens/s at C3; the CPU model is printed;
  dense_gqa     the same harness with 2 key / 2 value heads and the dense
                split-L decode kernel (the in-house dense-GQA comparator).

--prefill prints a separate line for the prefill attention kernel (causal,
batch 1, the decoder's head shape) against the bf16 MFMA peak, with torch
SDPA over expanded heads and the CPU oracle beside it.
"""
import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode tokens/sec @1.5B-shape 32k ctx; attn kernel HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def timed_graph(fn, n_launch, repeats=3):
    """Average time (us) of one of `n_launch` fn(i) calls captured in a graph."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(2):
            fn(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n_launch):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    best = None
    for _ in range(repeats):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1000.0 / n_launch
        best = us if best is None else min(best, us)
    return best


def k1_traffic(batch, ctx, shape):
    """HBM bytes per K1 launch from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE passes (profiles/*_counters.json, written by
    --summarize-counters), when they were taken at this workload; else None."""
    import glob
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*_counters.json"))):
        with open(path) as f:
            d = json.load(f)
        w = d.get("workload") or {}
        if (w.get("batch"), w.get("ctx"), w.get("n_q"), w.get("n_k"), w.get("head_dim")) != \
                (batch, ctx, shape.n_q, shape.n_k, shape.head_dim) or w.get("outlier_keys"):
            continue
        for kern, ent in d["kernels"].items():
            if kern.startswith("void saga::qk_scores_kernel<1, %d>" % shape.head_dim) and "traffic_bytes_per_launch" in ent:
                return int(ent["traffic_bytes_per_launch"]), os.path.relpath(path, ROOT)
    return None, None


def decode_rate(model, steps, warmup):
    """Warm-up replays, then exactly `steps` timed replays bracketed by syncs."""
    model.reset()
    for i in range(warmup):
        model.replay(i)
    torch.cuda.synchronize()
    model.reset()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for i in range(steps):
        model.replay(i)
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1)
    return ms / steps, model.batch * steps / (ms / 1000.0), wall


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


# decode-attention shapes of the CPU baseline: b, q_h, k_h, v_h, d, L, N
CPU_SHAPES = {
    "C1": (1, 15, 1, 5, 64, 4096, 128),
    "C5": (4, 12, 1, 2, 128, 131072, 1024),
}


def _cpu_layer_ms(b, q_h, k_h, v_h, d, L, N, budget_s, max_calls=20):
    """Per-layer latency (ms) of the oracle's fast step on N(0,1) fp32 inputs
    after one calibration, as many calls as fit budget_s (at least 2)."""
    from oracle import saga_oracle as O
    rng = np.random.default_rng(0)
    q = rng.standard_normal((b, q_h, 1, d), dtype=np.float32)
    k = rng.standard_normal((b, k_h, L, d), dtype=np.float32)
    v = rng.standard_normal((b, v_h, L, d), dtype=np.float32)
    q2 = q + np.float32(0.3) * rng.standard_normal(q.shape, dtype=np.float32)
    t0 = time.perf_counter()
    _, thr, _ = O.calibrate(q, k, v, None, N, None)
    cal_ms = (time.perf_counter() - t0) * 1e3
    times = []
    t_start = time.perf_counter()
    while len(times) < 2 or (time.perf_counter() - t_start < budget_s and len(times) < max_calls):
        t0 = time.perf_counter()
        O.fast(q2, k, v, thr, None, N, None)
        times.append((time.perf_counter() - t0) * 1e3)
    a = np.asarray(times)
    return {"fast_ms_mean": round(float(a.mean()), 3), "fast_ms_p50": round(float(np.percentile(a, 50)), 3),
            "fast_ms_p90": round(float(np.percentile(a, 90)), 3), "calibration_ms": round(cal_ms, 3),
            "calls": len(times)}


def cpu_baseline(batch, ctx, shape, top_n, layers, budget_s=6.0):
    """The oracle (the reference's fp32 path restated in numpy) on every host
    core: per-layer decode-attention latency at C1, C3 (this workload) and C5,
    and attention tokens/s at C3 (batch / (layers x per-layer fast step))."""
    try:
        from threadpoolctl import threadpool_limits
    except ImportError:  # pragma: no cover
        threadpool_limits = None
    cores = os.cpu_count() or 1
    shapes = dict(CPU_SHAPES)
    shapes["C3"] = (batch, shape.n_q, shape.n_k, shape.n_v, shape.head_dim, ctx + 1, top_n)
    t0 = time.perf_counter()
    per_layer = {}

    def run():
        for name in ("C1", "C3", "C5"):
            per_layer[name] = dict(_cpu_layer_ms(*shapes[name], budget_s), shape=list(shapes[name]))

    if threadpool_limits is not None:
        with threadpool_limits(limits=cores):
            run()
    else:
        run()
    c3 = per_layer["C3"]["fast_ms_p50"]
    return {
        "value": round(batch / (layers * c3 * 1e-3), 3),
        "unit": f"tokens/s (attention only, {layers} layers of the fast step)",
        "cores": cores,
        "kind": "port",
        "cpu_model": cpu_model(),
        "per_layer": per_layer,
        "sample": (f"numpy oracle in fp32 on {cores} threads: after one calibration, repeated fast steps per shape "
                   f"[b, q_h, k_h, v_h, d, L, N] for ~{budget_s:.0f} s each ({time.perf_counter() - t0:.1f} s); "
                   f"value = batch / ({layers} x C3 per-layer median)"),
    }


def hbm_copy_gbs(nbytes=1 << 30, reps=10):
    """A plain device-to-device copy of nbytes: (read + written bytes) / time."""
    src = torch.empty(nbytes // 2, dtype=torch.int16, device="cuda")
    src.fill_(1)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1000.0 / reps
    del src, dst
    return round(2 * nbytes / us / 1e3, 1)


def atopn_call_bytes(model, top_n, kvl, k2_variant=0):
    """Algorithmic bytes of one fast-step call at the decoder's state,
    averaged over its layers: K (b * k_h * kv_len * d * 2) + the distinct V
    rows selected per (batch row, value head) * d * 2 + Q and O + the
    thresholds.  Returns (bytes, distinct V rows per call)."""
    from saga_amd import ops
    s, B = model.shape, model.batch
    q4 = model._q.view(B, s.n_q, 1, s.head_dim)
    L = model.k_cache.shape[3]
    buf_k = min(2 * top_n, L)
    kv = int(kvl[0])
    ws = model.ws["atopn"]
    rows = 0
    for l in range(s.layers):
        ops.atopn_decode(q4, model.k_cache[l], model.v_cache[l], model.table[l], top_n, kv_len=kvl, out=model._attn,
                         workspace=ws, k2_variant=k2_variant)
        kept = ops.atopn_kept_positions(B, s.n_q, s.n_k, L, s.head_dim, buf_k, ws)
        rows += ops.atopn_distinct_value_rows(kept, B, s.n_q, s.n_v, L)
    torch.cuda.synchronize()
    vrows = rows / s.layers
    d2 = s.head_dim * 2
    return B * s.n_k * kv * d2 + vrows * d2 + 2 * B * s.n_q * d2 + 4 * B * s.n_q, vrows


def c5_leg(copies=4, b=4, q_h=12, L=131072, N=1024, d=128, k2_variant=0):
    """Attention alone at the 128k comparison shape: SAGA (1 key / 2 value
    heads, Atop-N N=1024: calibrated on q, timed on a nearby q2) against
    dense GQA (2 key / 2 value heads) on the same seeded N(0,1) caches,
    `copies` distinct caches cycled (the Infinity Cache would hold one)."""
    from saga_amd import _lib, ops
    g = torch.Generator(device="cuda").manual_seed(5)
    q = torch.randn(b, q_h, 1, d, device="cuda", generator=g).to(torch.bfloat16)
    q2 = (q.float() + 0.3 * torch.randn(q.shape, device="cuda", generator=g)).to(torch.bfloat16)
    out = torch.empty(b, q_h, 1, d, device="cuda", dtype=torch.bfloat16)
    kd = [torch.randn(b, 2, L, d, device="cuda", generator=g).to(torch.bfloat16) for _ in range(copies)]
    vd = [torch.randn(b, 2, L, d, device="cuda", generator=g).to(torch.bfloat16) for _ in range(copies)]
    ks = [x[:, :1].contiguous() for x in kd]   # SAGA: the first key head, the same two value heads
    lib = _lib.load()
    wsd = torch.empty(max(lib.saga_dense_workspace_bytes(b, q_h, L, d), 256), dtype=torch.uint8, device="cuda")
    wsa = torch.empty(max(ops.atopn_workspace_bytes(b, q_h, 1, L, d, N, c) for c in (False, True)),
                      dtype=torch.uint8, device="cuda")
    tabs = [torch.zeros(b * q_h, device="cuda") for _ in range(copies)]
    for i in range(copies):
        ops.atopn_calibrate(q, ks[i], vd[i], N, tabs[i], out=out, workspace=wsa)
    saga_us = timed_graph(lambda i: ops.atopn_decode(q2, ks[i % copies], vd[i % copies], tabs[i % copies], N, out=out,
                                                     workspace=wsa, k2_variant=k2_variant), 2 * copies)
    dense_us = timed_graph(lambda i: ops.dense_decode(q2, kd[i % copies], vd[i % copies], out=out, workspace=wsd),
                           2 * copies)
    ops.atopn_decode(q2, ks[0], vd[0], tabs[0], N, out=out, workspace=wsa, k2_variant=k2_variant)
    kept = ops.atopn_kept_positions(b, q_h, 1, L, d, min(2 * N, L), wsa)
    vrows = ops.atopn_distinct_value_rows(kept, b, q_h, 2, L)
    torch.cuda.synchronize()
    qo = 2 * b * q_h * d * 2
    saga_bytes = b * L * d * 2 + vrows * d * 2 + qo + 4 * b * q_h
    dense_bytes = 2 * b * 2 * L * d * 2 + qo
    del kd, vd, ks
    torch.cuda.empty_cache()
    return {"workload": f"attention alone, batch {b}, {L} positions, {q_h} query heads, d{d}: SAGA 1K/2V Atop-N "
                        f"N={N} vs dense GQA 2K/2V, N(0,1) bf16 caches",
            "saga_us": round(saga_us, 2), "dense_us": round(dense_us, 2), "speedup": round(dense_us / saga_us, 3),
            "saga_GBs": round(saga_bytes / saga_us / 1e3, 1), "dense_GBs": round(dense_bytes / dense_us / 1e3, 1),
            "saga_frac": round(saga_bytes / saga_us / 1e3 / HBM_PEAK_GBS, 4),
            "dense_frac": round(dense_bytes / dense_us / 1e3 / HBM_PEAK_GBS, 4),
            "saga_bytes": int(saga_bytes), "dense_bytes": int(dense_bytes), "saga_value_rows": vrows}


def c1_gpu_us(reps=20):
    """The fast step at the C1 shape (b1, 15/1/5 heads, d64, 4096 positions,
    fp32, N=128) on the GPU, microseconds per call (graph of calls)."""
    from saga_amd import ops
    b, q_h, k_h, v_h, d, L, N = CPU_SHAPES["C1"]
    g = torch.Generator(device="cuda").manual_seed(1)
    q = torch.randn(b, q_h, 1, d, device="cuda", generator=g)
    k = torch.randn(b, k_h, L, d, device="cuda", generator=g)
    v = torch.randn(b, v_h, L, d, device="cuda", generator=g)
    tab = torch.zeros(b * q_h, device="cuda")
    ops.atopn_calibrate(q, k, v, N, tab)
    out = torch.empty(b, q_h, 1, d, device="cuda")
    ws = torch.empty(ops.atopn_workspace_bytes(b, q_h, k_h, L, d, N), dtype=torch.uint8, device="cuda")
    return round(timed_graph(lambda i: ops.atopn_decode(q, k, v, tab, N, out=out, workspace=ws), reps), 2)


def profile_kernels(batch, ctx, shape, top_n, launches=8, outlier_keys=0.0, cal_variant=0):
    """Kernels alone at the decode shape, for hardware-counter runs: K1
    (qk_scores) `launches` times, the Atop-N calibration step `launches`
    times (its kernels chosen by cal_variant: 0 by shape, 1 one block per
    row, 2 chunk kernel + row kernel), the whole Atop-N fast step
    `launches` times, the dense decode at the dense-GQA
    comparator's heads `launches` times, then a plain 1 GiB device-to-device
    copy 3 times, whose counters (2 GiB of known traffic per dispatch) scale
    the others'.  Inputs: N(0,1) bf16 caches of ctx + 1 positions; with
    outlier_keys, that fraction of the key rows scaled x8 (the kernel
    sweep's stress case: rows pass far more than buf_k positions)."""
    from saga_amd import ops
    L = ctx + 1
    d = shape.head_dim
    g = torch.Generator(device="cuda").manual_seed(0)
    q = torch.randn(batch, shape.n_q, 1, d, device="cuda", generator=g).to(torch.bfloat16)
    q2 = (q.float() + 0.3 * torch.randn(q.shape, device="cuda", generator=g)).to(torch.bfloat16)
    kf = torch.randn(batch, shape.n_k, L, d, device="cuda", generator=g)
    if outlier_keys > 0:
        kf[torch.rand(batch, shape.n_k, L, device="cuda", generator=g) < outlier_keys] *= 8.0
    k = kf.to(torch.bfloat16)
    del kf
    v = torch.randn(batch, shape.n_v, L, d, device="cuda", generator=g).to(torch.bfloat16)
    kvl = torch.full((batch,), L, dtype=torch.int32, device="cuda")
    for _ in range(launches):
        ops.qk_scores(q, k, kv_len=kvl, with_partials=True)
    tab = torch.zeros(batch * shape.n_q, device="cuda")
    for _ in range(launches):
        ops.atopn_calibrate(q, k, v, top_n, tab, kv_len=kvl, k2_variant=cal_variant)
    ws = torch.empty(ops.atopn_workspace_bytes(batch, shape.n_q, shape.n_k, L, d, top_n), dtype=torch.uint8,
                     device="cuda")
    for _ in range(launches):
        ops.atopn_decode(q2, k, v, tab, top_n, kv_len=kvl, workspace=ws)
    kept = ops.atopn_kept_positions(batch, shape.n_q, shape.n_k, L, d, min(2 * top_n, L), ws)
    vrows = ops.atopn_distinct_value_rows(kept, batch, shape.n_q, shape.n_v, L)
    views = ops.atopn_workspace_views(batch, shape.n_q, shape.n_k, L, d, min(2 * top_n, L), "cuda", fast=True,
                                      workspace=ws)
    over = int((views["sel_total"] > min(2 * top_n, L)).sum())
    kd = torch.randn(batch, 2, L, d, device="cuda", generator=g).to(torch.bfloat16)
    vd = torch.randn(batch, 2, L, d, device="cuda", generator=g).to(torch.bfloat16)
    for _ in range(launches):
        ops.dense_decode(q, kd, vd, kv_len=kvl)
    src = torch.empty(1 << 29, dtype=torch.int16, device="cuda")
    src.fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    d2 = d * 2
    qo = 2 * batch * shape.n_q * d2
    print(json.dumps({
        "launches": launches, "calibration_variant": cal_variant, "batch": batch, "kv_len": L, "n_q": shape.n_q, "n_k": shape.n_k, "n_v": shape.n_v,
        "head_dim": d, "top_n": top_n, "outlier_keys": outlier_keys, "rows_over_buf_k": over,
        "k1_algorithmic_bytes": batch * shape.n_k * L * d2 + batch * shape.n_q * d2,
        "atopn_call_algorithmic_bytes": batch * shape.n_k * L * d2 + vrows * d2 + qo + 4 * batch * shape.n_q,
        "atopn_distinct_value_rows": vrows,
        "dense_algorithmic_bytes": batch * 4 * L * d2 + qo,
        "copy_launches": 3, "copy_bytes_read": src.numel() * 2, "copy_bytes_written": dst.numel() * 2}), flush=True)
    return 0


def summarize_counters(paths, workload=None):
    """Per-kernel averages of the rocprofv3 counter CSVs (*counter_collection.csv)
    under `paths` (one directory per --pmc pass of `bench.py --profile-kernels`;
    a path ending in .log is that run's output, whose JSON line names the
    workload and its algorithmic bytes).
    FETCH_SIZE and WRITE_SIZE (KiB per dispatch) are scaled by what the same
    counter reads on the 1 GiB device-to-device copies of the same run (the
    __amd_rocclr_copyBuffer dispatches of at least half the largest reading):
    bytes = KiB * 1024 * (2^30 B / (copy reading * 1024)).  traffic = scaled
    FETCH + scaled WRITE.  Other counters are averaged as read."""
    import csv
    import glob
    from collections import defaultdict
    vals = defaultdict(lambda: defaultdict(list))  # kernel -> counter -> per-dispatch values
    for p in paths:
        if p.endswith(".log"):  # the --profile-kernels output: its JSON line names the workload
            with open(p) as fh:
                for line in fh:
                    if line.startswith('{"launches"'):
                        w = json.loads(line)
                        workload = {"batch": w["batch"], "ctx": w["kv_len"] - 1, **{k: w[k] for k in w if k not in (
                            "batch", "launches", "copy_launches", "copy_bytes_read", "copy_bytes_written")}}
            continue
        files = glob.glob(os.path.join(p, "**", "*counter_collection.csv"), recursive=True) if os.path.isdir(p) else [p]
        for f in files:
            per = defaultdict(float)
            names = {}
            with open(f) as fh:
                for row in csv.DictReader(fh):
                    key = (row["Dispatch_Id"], row["Counter_Name"])
                    per[key] += float(row["Counter_Value"])
                    names[row["Dispatch_Id"]] = row["Kernel_Name"]
            for (disp, ctr), v in per.items():
                vals[names[disp]][ctr].append(v)
    copy = "__amd_rocclr_copyBuffer"
    scale = {}
    for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
        xs = vals.get(copy, {}).get(ctr, [])
        big = [x for x in xs if xs and x >= 0.5 * max(xs)]
        if big and max(big) > 0:
            scale[ctr] = (1 << 30) / (sum(big) / len(big) * 1024)
    out = {"workload": workload, "copy_kernel": f"{copy}, 1 GiB read + 1 GiB written per dispatch",
           "bytes_per_counter_kib": {k: round(v * 1024, 3) for k, v in scale.items()}, "kernels": {}}
    for kern, ctrs in sorted(vals.items()):
        if "saga::" not in kern:
            continue
        ent = {}
        for ctr, xs in sorted(ctrs.items()):
            ent[ctr] = {"dispatches": len(xs), "avg": round(sum(xs) / len(xs), 3), "min": min(xs), "max": max(xs)}
        if all(c in ent and c in scale for c in ("FETCH_SIZE", "WRITE_SIZE")):
            ent["fetch_bytes"] = int(ent["FETCH_SIZE"]["avg"] * 1024 * scale["FETCH_SIZE"])
            ent["write_bytes"] = int(ent["WRITE_SIZE"]["avg"] * 1024 * scale["WRITE_SIZE"])
            ent["traffic_bytes_per_launch"] = ent["fetch_bytes"] + ent["write_bytes"]
        out["kernels"][kern] = ent
    print(json.dumps(out, indent=1), flush=True)
    return 0


MFMA_BF16_PEAK_TFLOPS = 2500.0


def prefill_bench(ctx, shape, reps=10, no_cpu=False):
    """Prefill attention alone (saga_prefill_attention, the reference's
    sdpa_attention_forward with separate key / value heads) at the decoder's
    head shape, batch 1, a causal prompt of `ctx` tokens, N(0,1) bf16 q/k/v.
    Algorithmic flops: 4 * q_h * d * L (L + 1) / 2 (q.k and p.v over the
    causal triangle).  Beside it: torch SDPA over the repeat_interleave-
    expanded heads (the reference's path), with and without the expansion."""
    from saga_amd import ops
    L, q_h, d = ctx, shape.n_q, shape.head_dim
    g = torch.Generator(device="cuda").manual_seed(0)
    q = torch.randn(1, q_h, L, d, generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn(1, shape.n_k, L, d, generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn(1, shape.n_v, L, d, generator=g, device="cuda").to(torch.bfloat16)
    out = torch.empty(1, L, q_h, d, device="cuda", dtype=torch.bfloat16)

    def timed(fn):
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    ms = timed(lambda: ops.prefill_attention(q, k, v, is_causal=True, out=out))
    flops = 4.0 * q_h * d * L * (L + 1) / 2
    tflops = flops / (ms * 1e-3) / 1e12
    sdpa = torch.nn.functional.scaled_dot_product_attention
    kx, vx = k.repeat_interleave(q_h // shape.n_k, dim=1), v.repeat_interleave(q_h // shape.n_v, dim=1)
    t_sdpa = timed(lambda: sdpa(q, kx, vx, is_causal=True))
    t_sdpa_x = timed(lambda: sdpa(q, k.repeat_interleave(q_h // shape.n_k, dim=1),
                                  v.repeat_interleave(q_h // shape.n_v, dim=1), is_causal=True))
    log(f"prefill attention L={L}: {ms:.3f} ms, {tflops:.1f} TFLOP/s; torch SDPA (expanded heads) {t_sdpa:.3f} ms "
        f"({t_sdpa_x:.3f} ms with the expansion)")
    line = {
        "metric": f"prefill attention TFLOP/s @1.5B-shape {L // 1024}k causal",
        "value": round(tflops, 1), "unit": "TFLOP/s", "n_gpus": 1, "steps": reps, "warmup": 2,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic: N(0,1) q/k/v",
        "config": {"workload": f"SAGA prefill attention, {q_h} query / {shape.n_k} key / {shape.n_v} value heads, "
                               f"d{d}, batch 1, {L} tokens, causal",
                   "global_batch": 1, "seq_len": L, "parallelism": "single GPU"},
        "roofline": {"kernel": "saga::prefill_attn_kernel<bf16,128>", "bound": "mfma", "achieved": round(tflops, 1),
                     "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None,
                     "algorithmic_flops_per_launch": flops},
        "torch_sdpa_expanded": {"ms": round(t_sdpa, 4), "ms_with_expand": round(t_sdpa_x, 4),
                                "speedup_saga": round(t_sdpa_x / ms, 3)},
    }
    if not no_cpu:
        from oracle import saga_oracle as O
        try:
            from threadpoolctl import threadpool_limits
        except ImportError:  # pragma: no cover
            threadpool_limits = None
        cores = min(16, os.cpu_count() or 1)
        Ls = 2048
        rng = np.random.default_rng(0)
        qs = rng.standard_normal((1, q_h, Ls, d), dtype=np.float32)
        ks = rng.standard_normal((1, shape.n_k, Ls, d), dtype=np.float32)
        vs = rng.standard_normal((1, shape.n_v, Ls, d), dtype=np.float32)

        def run():
            n, t0 = 0, time.perf_counter()
            while True:
                O.prefill(qs, ks, vs, is_causal=True)
                n += 1
                secs = time.perf_counter() - t0
                if secs >= 10.0 or n >= 30:
                    return n, secs

        if threadpool_limits is not None:
            with threadpool_limits(limits=cores):
                n, secs = run()
        else:
            n, secs = run()
        fl_s = 4.0 * q_h * d * Ls * (Ls + 1) / 2
        line["cpu_baseline"] = {"value": round(fl_s * n / secs / 1e12, 5), "unit": "TFLOP/s (causal flops)",
                                "cores": cores, "kind": "port",
                                "sample": f"{n} causal prefills of {Ls} tokens, {q_h}/{shape.n_k}/{shape.n_v} heads "
                                          f"d{d}, fp32 numpy oracle, {secs:.1f} s"}
    print(json.dumps(line), flush=True)
    return 0


def sweep(copies=8, k2_variant=0):
    """Attention-only timings on synthetic bf16 caches: every shape is timed
    as a graph of 2 x `copies` launches cycling over `copies` distinct K/V
    caches (the same cache in a row would sit in the 256 MB Infinity Cache).
    Atop-N: the table is calibrated first (N-th largest probability of a
    nearby query), then the fast step is timed.  Bytes are algorithmic: K
    (+ V rows actually selected, counted from the workspace) for Atop-N, K + V
    for dense."""
    from saga_amd import ops
    dev = "cuda"
    grid = []
    for L in (4096, 16384, 65536, 131072):          # lengths x batches, 12Q / 1K / 2V, N = 256
        for b in (1, 8, 32):
            grid.append(("len-batch", b, 12, 1, 2, L, 256))
    for k_h, v_h, q_h in ((1, 2, 12), (1, 4, 12), (2, 2, 12), (2, 4, 12), (1, 8, 16), (2, 8, 16)):
        grid.append(("heads", 8, q_h, k_h, v_h, 16384, 256))   # head groupings
    for N in (64, 256, 1024):
        grid.append(("top-n", 8, 12, 1, 2, 16384, N))
    grid.append(("C5 SAGA", 4, 12, 1, 2, 131072, 1024))
    grid.append(("C5 dense-GQA", 4, 12, 2, 2, 131072, None))
    for tag, b, q_h, k_h, v_h, L, N in grid:
        g = torch.Generator(device=dev).manual_seed(L + b)
        q = torch.randn(b, q_h, 1, 128, device=dev, generator=g).to(torch.bfloat16)
        q2 = (q.float() + 0.3 * torch.randn(q.shape, device=dev, generator=g)).to(torch.bfloat16)
        ncp = max(1, min(copies, int(6e9 // (b * (k_h + v_h) * L * 256))))
        ks, vs = [], []
        for _ in range(ncp):
            k = torch.randn(b, k_h, L, 128, device=dev, generator=g)
            k[:, :, torch.randperm(L, device=dev, generator=g)[: L // 100]] *= 8  # 1% outlier keys
            ks.append(k.to(torch.bfloat16))
            vs.append(torch.randn(b, v_h, L, 128, device=dev, generator=g).to(torch.bfloat16))
        out = torch.empty(b, q_h, 1, 128, device=dev, dtype=torch.bfloat16)
        kv_bytes = b * k_h * L * 256
        if N is None:
            us = timed_graph(lambda i: ops.dense_decode(q2, ks[i % ncp], vs[i % ncp], out=out), 2 * ncp)
            byts = kv_bytes + b * v_h * L * 256
            line = {"sweep": tag, "b": b, "q_h": q_h, "k_h": k_h, "v_h": v_h, "L": L, "kernel": "dense",
                    "us": round(us, 2), "GBs": round(byts / us / 1e3, 1)}
        else:
            tabs = [torch.zeros(b * q_h, device=dev) for _ in range(ncp)]
            for i in range(ncp):
                ops.atopn_calibrate(q, ks[i], vs[i], N, tabs[i])
            us = timed_graph(lambda i: ops.atopn_decode(q2, ks[i % ncp], vs[i % ncp], tabs[i % ncp], N, out=out,
                                                        k2_variant=k2_variant), 2 * ncp)
            k1 = timed_graph(lambda i: ops.qk_scores(q2, ks[i % ncp], with_partials=True), 2 * ncp)
            ws = ops.workspace(torch.device(dev, torch.cuda.current_device()), "atopn",
                               ops.atopn_workspace_bytes(b, q_h, k_h, L, 128, N))
            ops.atopn_decode(q2, ks[0], vs[0], tabs[0], N, out=out, k2_variant=k2_variant, workspace=ws)
            kept = ops.atopn_kept_positions(b, q_h, k_h, L, 128, min(2 * N, L), ws)
            sel = int((kept >= 0).sum())
            vrows = ops.atopn_distinct_value_rows(kept, b, q_h, v_h, L)
            byts = kv_bytes + vrows * 256 + 2 * b * q_h * 256 + 4 * b * q_h
            line = {"sweep": tag, "b": b, "q_h": q_h, "k_h": k_h, "v_h": v_h, "L": L, "N": N, "kernel": "atopn",
                    "us": round(us, 2), "k1_us": round(k1, 2), "k1_GBs": round(kv_bytes / k1 / 1e3, 1),
                    "selected_per_row": round(sel / (b * q_h), 1), "distinct_value_rows": vrows,
                    "GBs": round(byts / us / 1e3, 1), "frac": round(byts / us / 1e3 / HBM_PEAK_GBS, 4)}
        print(json.dumps(line), flush=True)
        del ks, vs
        torch.cuda.empty_cache()
    return 0


def _shapes():
    from saga_amd import decoder as D
    return D


# workloads: the headline (the metric's 1.5B shape at 32k, batch 8, 256 steps,
# N=512) and the SmolLM2-360M-shaped decoder (batch 1, 8192-token prompt, 128
# greedy tokens, N=256; its dense-GQA comparator keeps 5 key/value heads)
MODELS = {
    "qwen2.5-1.5b": dict(name="Qwen2.5-1.5B", shape=lambda: _shapes().QWEN25_15B_SAGA,
                         gqa=lambda: _shapes().QWEN25_15B_GQA, batch=8, ctx=32768, top_n=512, steps=256,
                         metric=None),
    "smollm2-360m": dict(name="SmolLM2-360M", shape=lambda: _shapes().SMOLLM2_360M_SAGA,
                         gqa=lambda: _shapes().SMOLLM2_360M_GQA, batch=1, ctx=8192, top_n=256, steps=128,
                         metric="decode tokens/sec @360M-shape 8k ctx, batch 1"),
}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--model", choices=sorted(MODELS), default="qwen2.5-1.5b",
                    help="workload: the 1.5B-shaped decoder at 32k (the headline) or the SmolLM2-360M-shaped "
                         "decoder at 8k (batch 1, 128 greedy tokens, N=256)")
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=None)
    ap.add_argument("--ctx", type=int, default=None)
    ap.add_argument("--top-n", type=int, default=None)
    ap.add_argument("--no-dense", action="store_true", help="skip the dense-GQA comparator")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-c5", action="store_true", help="skip the 128k SAGA vs dense-GQA attention comparison")
    ap.add_argument("--synthetic-kv", action="store_true", help="fill the caches with N(0,1) instead of a prefill")
    ap.add_argument("--sweep", action="store_true",
                    help="attention kernels alone over a grid of shapes (lengths, batches, head groupings, N) "
                         "and the 128k dense-GQA vs SAGA comparison; one JSON line per shape")
    ap.add_argument("--k2-variant", type=int, choices=(0, 1, 2), default=0,
                    help="fast-step selection + softmax.V kernels: 0 by shape (default), 1 one block per row, "
                         "2 slice kernel + row kernel (identical selections, outputs equal to fp32 rounding)")
    ap.add_argument("--exempt", default="",
                    help="comma-separated layers that run dense attention in the SAGA model (speedup.py:65-66), "
                         "e.g. 0,14 for Qwen2.5-1.5B")
    ap.add_argument("--prefill", action="store_true",
                    help="measure the prefill attention kernel alone (its own JSON line) instead of decode")
    ap.add_argument("--profile-kernels", action="store_true",
                    help="only launch K1 (qk_scores), the whole Atop-N fast step and the dense decode at the "
                         "workload shape, then a 1 GiB device copy: for hardware-counter runs")
    ap.add_argument("--cal-variant", type=int, choices=(0, 1, 2), default=0,
                    help="with --profile-kernels: calibration kernels, 0 by shape (default), 1 one block per row, "
                         "2 chunk kernel + row kernel (identical lists and p*)")
    ap.add_argument("--outlier-keys", type=float, default=0.0, metavar="FRAC",
                    help="with --profile-kernels: scale this fraction of the key rows x8 (rows overflow buf_k)")
    ap.add_argument("--summarize-counters", nargs="+", metavar="DIR",
                    help="summarize rocprofv3 counter CSVs under DIR(s) per kernel, bytes scaled by the copy "
                         "dispatches of the same run (no GPU needed)")
    args = ap.parse_args()
    if args.summarize_counters:
        return summarize_counters(args.summarize_counters)
    if args.gpus != 1:
        print("bench.py measures one GPU: there is no multi-GPU path (the design shards the "
              "caches by sequence, not built); run with --gpus 1", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2

    from saga_amd import ops
    from saga_amd.decoder import SagaDecoder

    mdl = MODELS[args.model]
    SAGA_SHAPE, GQA_SHAPE = mdl["shape"](), mdl["gqa"]()
    for k in ("batch", "ctx", "top_n", "steps"):
        if getattr(args, k) is None:
            setattr(args, k, mdl[k])

    B, ctx, K, W = args.batch, args.ctx, args.steps, args.warmup
    if args.profile_kernels:
        return profile_kernels(B, ctx, SAGA_SHAPE, args.top_n, outlier_keys=args.outlier_keys,
                               cal_variant=args.cal_variant)
    if args.prefill:
        return prefill_bench(ctx, SAGA_SHAPE, no_cpu=args.no_cpu)
    if args.sweep:
        return sweep(k2_variant=args.k2_variant)
    max_len = ctx + K
    torch.manual_seed(0)
    prompt = torch.randint(0, SAGA_SHAPE.vocab, (ctx,), dtype=torch.int64)

    exempt = tuple(int(x) for x in args.exempt.split(",") if x.strip())

    def build(shape, mode):
        m = SagaDecoder(shape, B, max_len, mode=mode, top_n=args.top_n, exempt_layers=exempt if mode == "atopn" else (),
                        k2_variant=args.k2_variant)
        # the step graphs first (they hold no prompt length), then the
        # prompt, as a server that loads the model and then takes a request:
        # the decode steps start right after the prefill's GPU work, not
        # after the host-side capture
        m.capture()
        t0 = time.perf_counter()
        if args.synthetic_kv:
            m.fill_synthetic(ctx)
        else:
            m.prefill(prompt)
        torch.cuda.synchronize()
        log(f"{mode} model: prefill {time.perf_counter() - t0:.2f}s")
        return m

    log(f"SAGA model ({SAGA_SHAPE.n_q}Q/{SAGA_SHAPE.n_k}K/{SAGA_SHAPE.n_v}V, Atop-N)")
    saga = build(SAGA_SHAPE, "atopn")
    ms, tps, wall = decode_rate(saga, K, W)
    log(f"SAGA decode: {ms:.3f} ms/step, {tps:.0f} tokens/s (host wall {wall:.3f}s)")

    # dominant kernel: K1 over the 28 layers' K caches, at the decode shape
    s = saga.shape
    q4 = saga._q.view(B, s.n_q, 1, s.head_dim)
    kvl = torch.full((B,), ctx + 1, dtype=torch.int32, device="cuda")
    nlaunch = 2 * s.layers
    k1_us = timed_graph(lambda i: ops.qk_scores(q4, saga.k_cache[i % s.layers], kv_len=kvl, with_partials=True),
                        nlaunch)
    k1_bytes = B * s.n_k * (ctx + 1) * s.head_dim * 2 + B * s.n_q * s.head_dim * 2
    k1_gbs = k1_bytes / (k1_us * 1e-6) / 1e9
    attn_us = timed_graph(lambda i: ops.atopn_decode(q4, saga.k_cache[i % s.layers], saga.v_cache[i % s.layers],
                                                     saga.table[i % s.layers], args.top_n, kv_len=kvl,
                                                     out=saga._attn, k2_variant=args.k2_variant,
                                                     workspace=saga.ws["atopn"]), nlaunch)
    call_bytes, call_vrows = atopn_call_bytes(saga, args.top_n, kvl, args.k2_variant)
    call_gbs = call_bytes / (attn_us * 1e-6) / 1e9
    log(f"K1 qk_scores: {k1_us:.2f} us/launch, {k1_gbs:.0f} GB/s; Atop-N fast attention {attn_us:.2f} us/layer, "
        f"{call_bytes / 1e6:.1f} MB algorithmic ({call_vrows:.0f} distinct V rows), {call_gbs:.0f} GB/s")
    saga_cache = saga.k_cache.shape, saga.v_cache.shape
    del saga
    torch.cuda.empty_cache()
    copy_gbs = hbm_copy_gbs()
    log(f"device copy: {copy_gbs:.0f} GB/s (read + written)")

    dense = None
    if not args.no_dense:
        log(f"dense-GQA comparator ({GQA_SHAPE.n_q}Q/{GQA_SHAPE.n_k}K/{GQA_SHAPE.n_v}V, dense decode)")
        gqa = build(GQA_SHAPE, "dense")
        d_ms, d_tps, _ = decode_rate(gqa, K, W)
        gs = gqa.shape
        dq = gqa._q.view(B, gs.n_q, 1, gs.head_dim)
        d_attn_us = timed_graph(lambda i: ops.dense_decode(dq, gqa.k_cache[i % gs.layers], gqa.v_cache[i % gs.layers],
                                                           kv_len=kvl, out=gqa._attn), nlaunch)
        dense = {"tokens_per_s": round(d_tps, 1), "ms_per_step": round(d_ms, 4),
                 "attention_us_per_layer": round(d_attn_us, 2), "speedup_saga_vs_dense": round(tps / d_tps, 3)}
        log(f"dense GQA decode: {d_ms:.3f} ms/step, {d_tps:.0f} tokens/s, attention {d_attn_us:.2f} us/layer; "
            f"SAGA speedup {tps / d_tps:.2f}x")
        del gqa
        torch.cuda.empty_cache()

    c5 = None
    if not args.no_c5 and args.model == "qwen2.5-1.5b":
        log("C5: batch 4, 131072 positions, SAGA 1K/2V N=1024 vs dense GQA 2K/2V (attention alone)")
        c5 = c5_leg(k2_variant=args.k2_variant)
        log(f"C5: SAGA {c5['saga_us']} us, dense {c5['dense_us']} us per call -> {c5['speedup']}x")

    cpu = None
    if not args.no_cpu:
        log("CPU baseline (oracle, fp32)")
        cpu = cpu_baseline(B, ctx, SAGA_SHAPE, args.top_n, SAGA_SHAPE.layers)
        gpu_layer = {"C1": c1_gpu_us(), "C3": round(attn_us, 2)}
        if c5 is not None:
            gpu_layer["C5"] = c5["saga_us"]
        cpu["gpu_per_layer_us"] = gpu_layer
        log(f"CPU: {cpu['value']} attention tokens/s on {cpu['cores']} cores ({cpu['cpu_model']}); per layer "
            + ", ".join(f"{k} {v['fast_ms_mean']} ms" for k, v in cpu["per_layer"].items()))

    traffic, traffic_src = k1_traffic(B, ctx, SAGA_SHAPE)
    out = {
        "metric": METRIC if args.model == "qwen2.5-1.5b" else mdl["metric"],
        "value": round(tps, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: random-init weights, random prompt ids" + (", N(0,1) KV cache" if args.synthetic_kv else ""),
        "config": {
            "workload": (f"{mdl['name']}-shaped SAGA decoder ({SAGA_SHAPE.layers} layers, hidden {SAGA_SHAPE.hidden}, "
                         f"{SAGA_SHAPE.n_q}Q/{SAGA_SHAPE.n_k}K/{SAGA_SHAPE.n_v}V heads, d{SAGA_SHAPE.head_dim}, "
                         f"vocab {SAGA_SHAPE.vocab}), batch {B}, {ctx}-token context, {K} decode steps, "
                         f"Atop-N N={args.top_n}" + (f", dense layers {list(exempt)}" if exempt else "")),
            "global_batch": B,
            "seq_len": ctx,
            "parallelism": "single GPU",
            "kv_cache": {"k": list(saga_cache[0]), "v": list(saga_cache[1]), "dtype": "bf16"},
        },
        "roofline": {
            "kernel": f"saga::qk_scores_kernel<bf16,{SAGA_SHAPE.head_dim}> (K1)",
            "bound": "hbm",
            "achieved": round(k1_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(k1_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            "us_per_launch": round(k1_us, 3),
            "algorithmic_bytes_per_launch": k1_bytes,
        },
        "attention_call_roofline": {
            "kernel": "Atop-N fast step, every kernel of one call (saga_atopn_decode)",
            "bound": "hbm",
            "achieved": round(call_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(call_gbs / HBM_PEAK_GBS, 4),
            "us_per_call": round(attn_us, 3),
            "algorithmic_bytes_per_call": int(call_bytes),
            "distinct_value_rows_per_call": round(call_vrows, 1),
        },
        "hbm_copy_GBs": copy_gbs,
        "attention_us_per_layer": round(attn_us, 2),
        "attention_tokens_per_s_gpu": round(B / (attn_us * 1e-6 * SAGA_SHAPE.layers), 1),
        "dense_gqa": dense,
        "c5": c5,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
