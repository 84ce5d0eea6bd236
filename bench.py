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
  cpu_baseline  the CPU oracle (the reference's fp32 path restated in numpy)
                on a bounded sample: one decode step of attention over the
                28 layers at the same shapes, as attention tokens/s;
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
    WRITE_SIZE passes (profiles/k1_qk_scores_*_traffic.json), when they were
    taken at this workload; else None."""
    import glob
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "k1_qk_scores_*_traffic.json"))):
        with open(path) as f:
            d = json.load(f)
        w = d.get("workload", {})
        if (w.get("batch"), w.get("ctx"), w.get("n_q"), w.get("n_k"), w.get("head_dim")) == \
                (batch, ctx, shape.n_q, shape.n_k, shape.head_dim):
            return int(d["traffic_bytes_per_launch"]), os.path.relpath(path, ROOT)
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


def cpu_baseline(batch, ctx, shape, top_n, layers, min_secs=10.0, max_steps=30):
    """The oracle (reference fp32 path) on one decode step of attention."""
    from oracle import saga_oracle as O
    try:
        from threadpoolctl import threadpool_limits
    except ImportError:  # pragma: no cover
        threadpool_limits = None
    cores = min(16, os.cpu_count() or 1)
    rng = np.random.default_rng(0)
    L = ctx + 1
    q = rng.standard_normal((batch, shape.n_q, 1, shape.head_dim), dtype=np.float32)
    k = rng.standard_normal((batch, shape.n_k, L, shape.head_dim), dtype=np.float32)
    v = rng.standard_normal((batch, shape.n_v, L, shape.head_dim), dtype=np.float32)
    q2 = q + np.float32(0.3) * rng.standard_normal(q.shape, dtype=np.float32)

    def run():
        # whole decode steps (a calibration layer + fast layers) until about
        # min_secs of CPU work, at most max_steps
        steps, t0 = 0, time.perf_counter()
        while True:
            _, thr, _ = O.calibrate(q, k, v, None, top_n, None)
            for _ in range(layers - 1):
                O.fast(q2, k, v, thr, None, top_n, None)
            steps += 1
            secs = time.perf_counter() - t0
            if secs >= min_secs or steps >= max_steps:
                return steps, secs

    if threadpool_limits is not None:
        with threadpool_limits(limits=cores):
            steps, secs = run()
    else:
        steps, secs = run()
    return {
        "value": round(batch * steps / secs, 3),
        "unit": f"tokens/s (attention only, {layers} layers)",
        "cores": cores,
        "kind": "port",
        "sample": (f"{steps} decode steps of attention, each {layers} layers (1 calibration + {layers - 1} fast), "
                   f"b{batch} q{shape.n_q}/k{shape.n_k}/v{shape.n_v} d{shape.head_dim} ctx {L}, N={top_n}, fp32, "
                   f"numpy oracle, {secs:.1f} s"),
    }


def profile_kernels(batch, ctx, shape, launches=8):
    """K1 alone at the decode shape (K cache of ctx + 1 positions), then a
    plain 1 GiB device-to-device copy: per-dispatch hardware counters of the
    copy (2 GiB of known traffic) scale those of K1."""
    from saga_amd import ops
    L = ctx + 1
    g = torch.Generator(device="cuda").manual_seed(0)
    q = torch.randn(batch, shape.n_q, 1, shape.head_dim, device="cuda", generator=g).to(torch.bfloat16)
    k = torch.randn(batch, shape.n_k, L, shape.head_dim, device="cuda", generator=g).to(torch.bfloat16)
    kvl = torch.full((batch,), L, dtype=torch.int32, device="cuda")
    for _ in range(launches):
        ops.qk_scores(q, k, kv_len=kvl, with_partials=True)
    src = torch.empty(1 << 29, dtype=torch.int16, device="cuda")
    src.fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    k1_bytes = batch * shape.n_k * L * shape.head_dim * 2 + batch * shape.n_q * shape.head_dim * 2
    print(json.dumps({"k1_launches": launches, "k1_algorithmic_bytes": k1_bytes,
                      "copy_launches": 3, "copy_bytes_read": src.numel() * 2, "copy_bytes_written": dst.numel() * 2}),
          flush=True)
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


def sweep(copies=8):
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
            if b * L <= 32 * 65536:
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
            us = timed_graph(lambda i: ops.atopn_decode(q2, ks[i % ncp], vs[i % ncp], tabs[i % ncp], N, out=out),
                             2 * ncp)
            k1 = timed_graph(lambda i: ops.qk_scores(q2, ks[i % ncp], with_partials=True), 2 * ncp)
            ops.atopn_decode(q2, ks[0], vs[0], tabs[0], N, out=out)
            torch.cuda.synchronize()
            cnt = ops.atopn_workspace_views(b, q_h, k_h, L, 128, min(2 * N, L), dev)["sel_cnt"]
            sel = int(cnt.sum())
            byts = kv_bytes + sel * 256
            line = {"sweep": tag, "b": b, "q_h": q_h, "k_h": k_h, "v_h": v_h, "L": L, "N": N, "kernel": "atopn",
                    "us": round(us, 2), "k1_us": round(k1, 2), "k1_GBs": round(kv_bytes / k1 / 1e3, 1),
                    "selected_per_row": round(sel / (b * q_h), 1), "GBs": round(byts / us / 1e3, 1)}
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
    ap.add_argument("--synthetic-kv", action="store_true", help="fill the caches with N(0,1) instead of a prefill")
    ap.add_argument("--sweep", action="store_true",
                    help="attention kernels alone over a grid of shapes (lengths, batches, head groupings, N) "
                         "and the 128k dense-GQA vs SAGA comparison; one JSON line per shape")
    ap.add_argument("--k2-variant", type=int, choices=(0, 1, 2), default=0,
                    help="fast-step selection + softmax.V kernels: 0 by shape (default), 1 one block per row, "
                         "2 slice kernel + row kernel (results are identical)")
    ap.add_argument("--exempt", default="",
                    help="comma-separated layers that run dense attention in the SAGA model (speedup.py:65-66), "
                         "e.g. 0,14 for Qwen2.5-1.5B")
    ap.add_argument("--prefill", action="store_true",
                    help="measure the prefill attention kernel alone (its own JSON line) instead of decode")
    ap.add_argument("--profile-kernels", action="store_true",
                    help="only launch K1 (qk_scores) at the workload shape and a 1 GiB device copy, "
                         "for hardware-counter runs")
    args = ap.parse_args()
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
        return profile_kernels(B, ctx, SAGA_SHAPE)
    if args.prefill:
        return prefill_bench(ctx, SAGA_SHAPE, no_cpu=args.no_cpu)
    if args.sweep:
        return sweep()
    max_len = ctx + K
    torch.manual_seed(0)
    prompt = torch.randint(0, SAGA_SHAPE.vocab, (ctx,), dtype=torch.int64)

    exempt = tuple(int(x) for x in args.exempt.split(",") if x.strip())

    def build(shape, mode):
        m = SagaDecoder(shape, B, max_len, mode=mode, top_n=args.top_n, exempt_layers=exempt if mode == "atopn" else (),
                        k2_variant=args.k2_variant)
        t0 = time.perf_counter()
        if args.synthetic_kv:
            m.fill_synthetic(ctx)
        else:
            m.prefill(prompt)
        torch.cuda.synchronize()
        log(f"{mode} model: prefill {time.perf_counter() - t0:.2f}s")
        m.capture()
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
                                                     out=saga._attn, k2_variant=args.k2_variant), nlaunch)
    log(f"K1 qk_scores: {k1_us:.2f} us/launch, {k1_gbs:.0f} GB/s; Atop-N fast attention {attn_us:.2f} us/layer")
    saga_cache = saga.k_cache.shape, saga.v_cache.shape
    del saga
    torch.cuda.empty_cache()

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

    cpu = None
    if not args.no_cpu:
        log("CPU baseline (oracle, fp32)")
        cpu = cpu_baseline(B, ctx, SAGA_SHAPE, args.top_n, SAGA_SHAPE.layers)
        log(f"CPU: {cpu['value']} attention tokens/s on {cpu['cores']} cores")

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
        "attention_us_per_layer": round(attn_us, 2),
        "attention_tokens_per_s_gpu": round(B / (attn_us * 1e-6 * SAGA_SHAPE.layers), 1),
        "dense_gqa": dense,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
