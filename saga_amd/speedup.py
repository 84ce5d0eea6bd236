"""Decode-latency harness with the reference's command line (speedup.py).

    python -m saga_amd.speedup --model_path qwen2.5-1.5b --attention full,atopn:512 \
        --batch_sizes 1,8 --seq_lengths 4096,32768 --num_new_tokens 256

What it mirrors (speedup.py:447-700):
  * attention modes: `full` (the split-L dense decode kernel), `vanilla`
    (the base SDPA function for decode: the flash kernel with one query per
    row, speedup.py:76-83), `atopn:N` and
    `atopn_amortized:N` (calibration on the first generated token, fast
    Atop-N steps after it: the amortized schedule of speedup.py:56-75);
  * the grid of batch sizes x sequence lengths x attention modes x merge
    modes, every configuration in its own subprocess (speedup.py:532-610), so
    that each one starts from an empty device; a subprocess that runs out of
    memory is reported as OOM, a crash or time-out as FAILED;
  * per configuration: a prompt of random ids prefilled at batch 1 and
    replicated (speedup.py:146-161), `--num_warmup` untimed and
    `--num_iterations` timed generations of `--num_new_tokens` tokens replayed
    as two captured HIP graphs (calibration step, fast step;
    speedup.py:179-291), per-token latency mean / std / p50 / p90 in ms
    (speedup.py:434-440);
  * `--exempt_layers` (dense attention in those layers, speedup.py:65-66) and
    `--merge_mode merge|baseline` with `--new_heads`: the SAGA model (key
    heads merged) or the plain GQA model;
  * the reference's execution flags (speedup.py:447-476), with the same
    meanings where they apply to this harness:
      --cuda_graph      replay the decode step as the two captured HIP graphs;
                        without it every step's kernels are launched eagerly
                        from Python (the reference's uncompiled/compiled
                        `decode`, speedup.py:164-177);
      --compile_mode, --no_compile
                        accepted and printed; the decode step is hand-written
                        HIP kernels behind the C ABI, so there is nothing for
                        torch.compile to fuse (no-op);
      --calibrate_during_measurement
                        accepted and printed; every measured generation starts
                        with the calibration step in any case, as the
                        reference's measurement loop does (it resets the
                        amortized step count per iteration, speedup.py:380-405);
      --profile_decode, --profile_output
                        torch.profiler around the measured generations only
                        (not warm-up, prefill or capture), one chrome trace per
                        configuration named as the reference names them
                        (speedup.py:640-661).

Models: `--model_path` is a local checkpoint directory (config.json +
safetensors, loaded by saga_amd.checkpoint; merge mode averages its key heads
down to --new_heads unless the checkpoint already has num_key_heads) or the
name of a built-in shape with random-init weights: qwen2.5-1.5b,
smollm2-360m.  No hub downloads.
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time
from dataclasses import replace
from typing import List, Optional, Tuple

BUILTIN = ("qwen2.5-1.5b", "smollm2-360m")


def parse_attention(spec: str) -> List[Tuple[str, Optional[int]]]:
    """speedup.py:484-495: comma-separated modes."""
    modes = []
    for val in spec.split(","):
        val = val.strip().lower()
        if val in ("vanilla", "full"):
            modes.append((val, None))
        elif val.startswith("atopn:") or val.startswith("atopn_amortized:"):
            modes.append(("atopn", int(val.split(":")[1])))
        else:
            raise ValueError(f"Unknown attention mode: {val}")
    return modes


def _label(mode: str, param: Optional[int]) -> str:
    return f"{mode}:{param}" if param is not None else mode


def build_decoder(model_path: str, merge: bool, new_heads: int, batch: int, max_len: int, mode: str,
                  top_n: int, exempt, dtype):
    """The decoder of one configuration (random-init built-in shape or a
    checkpoint directory)."""
    from saga_amd.decoder import (QWEN25_15B_GQA, QWEN25_15B_SAGA, SMOLLM2_360M_GQA, SMOLLM2_360M_SAGA,
                                  SagaDecoder)
    dmode = {"full": "dense", "vanilla": "vanilla"}.get(mode, "atopn")
    if model_path in BUILTIN:
        saga, gqa = ((QWEN25_15B_SAGA, QWEN25_15B_GQA) if model_path == "qwen2.5-1.5b"
                     else (SMOLLM2_360M_SAGA, SMOLLM2_360M_GQA))
        shape = replace(saga, n_k=new_heads) if merge else gqa
        return SagaDecoder(shape, batch, max_len, mode=dmode, top_n=top_n, exempt_layers=exempt, dtype=dtype)
    from saga_amd.checkpoint import load_checkpoint, read_config
    cfg = read_config(model_path)
    num_key_heads = new_heads if merge and "num_key_heads" not in cfg else None
    shape, weights = load_checkpoint(model_path, num_key_heads=num_key_heads, dtype=dtype)
    return SagaDecoder(shape, batch, max_len, mode=dmode, top_n=top_n, exempt_layers=exempt, dtype=dtype,
                       weights=weights)


def trace_name(profile_output: str, merge: bool, mode: str, param: Optional[int], batch: int, seq_len: int) -> str:
    """The decode trace file of one configuration (speedup.py:657-658)."""
    merge_label = "merged" if merge else "baseline"
    return (f"{profile_output.replace('.json', '')}_{merge_label}_{_label(mode, param).replace(':', '_')}"
            f"_bs{batch}_seq{seq_len}.json")


def run_config(args, mode: str, param: Optional[int], batch: int, seq_len: int, merge: bool) -> dict:
    """One configuration in this process: per-token latency statistics."""
    import numpy as np
    import torch
    dtype = {"float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32}[args.dtype]
    exempt = tuple(int(x) for x in args.exempt_layers.split(",") if x.strip())
    n_new = args.num_new_tokens
    m = build_decoder(args.model_path, merge, args.new_heads, batch, seq_len + n_new, mode, param or 512, exempt,
                      dtype)
    torch.manual_seed(0)
    m.prefill(torch.randint(0, m.shape.vocab, (seq_len,), dtype=torch.int64))
    graphs = bool(getattr(args, "cuda_graph", True))
    if graphs:
        m.capture()

    def generate():
        m.reset()
        for i in range(n_new):
            if graphs:
                m.replay(i)
            else:
                m.step(calibrate=(m.mode == "atopn" and i == 0))

    with torch.no_grad():
        for _ in range(args.num_warmup):
            generate()
        torch.cuda.synchronize()
        prof = None
        if getattr(args, "profile_decode", False):
            from torch.profiler import ProfilerActivity, profile
            prof = profile(activities=[ProfilerActivity.CPU, ProfilerActivity.CUDA])
        lat = []
        for _ in range(args.num_iterations):
            torch.cuda.synchronize()
            if prof is not None:
                prof.start()
            t0 = time.perf_counter()
            generate()
            torch.cuda.synchronize()
            lat.append((time.perf_counter() - t0) * 1000.0)
            if prof is not None:
                prof.stop()
                trace = trace_name(args.profile_output, merge, mode, param, batch, seq_len)
                prof.export_chrome_trace(trace)
                prof = None  # the first measured generation is traced (one trace per configuration)
                print(f"decode trace: {trace}", file=sys.stderr, flush=True)
    lat = np.array(lat) / n_new
    return {"mean_ms": float(np.mean(lat)), "std_ms": float(np.std(lat)), "p50_ms": float(np.percentile(lat, 50)),
            "p90_ms": float(np.percentile(lat, 90)), "tokens_per_s": float(batch * 1000.0 / np.mean(lat))}


def _sub_cmd(args, mode, param, batch, seq_len, merge_mode) -> List[str]:
    cmd = [sys.executable, "-m", "saga_amd.speedup", "--model_path", args.model_path,
           "--attention", _label(mode, param), "--batch_sizes", str(batch), "--seq_lengths", str(seq_len),
           "--num_new_tokens", str(args.num_new_tokens), "--num_iterations", str(args.num_iterations),
           "--num_warmup", str(args.num_warmup), "--dtype", args.dtype, "--new_heads", str(args.new_heads),
           "--merge_mode", merge_mode, "--_subprocess_json"]
    if args.exempt_layers:
        cmd += ["--exempt_layers", args.exempt_layers]
    if getattr(args, "cuda_graph", False):
        cmd.append("--cuda_graph")
    if getattr(args, "profile_decode", False):
        cmd += ["--profile_decode", "--profile_output", args.profile_output]
    return cmd


def describe_flags(args) -> str:
    """What the reference's execution flags mean in this harness (printed
    before the grid, as speedup.py:518-528 prints its settings)."""
    lines = [f"Compile: no-op (hand-written HIP kernels; --compile_mode {args.compile_mode}"
             f"{', --no_compile' if args.no_compile else ''} accepted)",
             "CUDA graph: " + ("enabled (HIP graphs: calibration step, fast step)" if args.cuda_graph
                               else "disabled (kernels launched eagerly per step)")]
    if args.calibrate_during_measurement:
        lines.append("Calibration during measurement: on (every measured generation starts with it)")
    if args.profile_decode:
        lines.append(f"Profiling decode: output={args.profile_output}")
    return "\n".join(lines)


def _is_oom(text: str) -> bool:
    return "OutOfMemoryError" in text or "out of memory" in text or "OOM" in text


def build_parser() -> argparse.ArgumentParser:
    """The reference's command line (speedup.py:447-476) plus --timeout."""
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--model_path", default="qwen2.5-1.5b",
                    help="checkpoint directory, or a built-in shape: " + ", ".join(BUILTIN))
    ap.add_argument("--num_warmup", type=int, default=5)
    ap.add_argument("--num_iterations", type=int, default=5)
    ap.add_argument("--seq_lengths", default="65536")
    ap.add_argument("--batch_sizes", default="32")
    ap.add_argument("--dtype", default="bfloat16", choices=["float16", "bfloat16", "float32"])
    ap.add_argument("--new_heads", type=int, default=1, help="key heads of the merged (SAGA) model")
    ap.add_argument("--num_new_tokens", type=int, default=8)
    ap.add_argument("--merge_mode", default="merge", help="merge, baseline or both (comma-separated)")
    ap.add_argument("--attention", default="full", help="full, vanilla, atopn:N, atopn_amortized:N (comma-separated)")
    ap.add_argument("--exempt_layers", default="", help="comma-separated layers that keep dense attention")
    ap.add_argument("--no_compile", action="store_true",
                    help="accepted (no-op): the decode step is hand-written HIP kernels, not torch.compile output")
    ap.add_argument("--compile_mode", default="default", choices=["default", "reduce-overhead", "max-autotune"],
                    help="accepted (no-op), as --no_compile")
    ap.add_argument("--cuda_graph", action="store_true",
                    help="replay each decode step as a captured HIP graph (else launch its kernels eagerly)")
    ap.add_argument("--calibrate_during_measurement", action="store_true",
                    help="accepted: every measured generation starts with the calibration step in any case")
    ap.add_argument("--profile_decode", action="store_true",
                    help="torch.profiler trace of the measured generations only, one file per configuration")
    ap.add_argument("--profile_output", default="decode_trace.json",
                    help="trace file stem (default: decode_trace.json)")
    ap.add_argument("--timeout", type=int, default=600, help="seconds per configuration subprocess")
    ap.add_argument("--_subprocess_json", action="store_true", help=argparse.SUPPRESS)
    return ap


def main(argv=None) -> int:
    args = build_parser().parse_args(argv)

    seq_lengths = [int(x) for x in args.seq_lengths.split(",")]
    batch_sizes = [int(x) for x in args.batch_sizes.split(",")]
    merge_modes = [m.strip().lower() for m in args.merge_mode.split(",")]
    for mm in merge_modes:
        if mm not in ("merge", "baseline"):
            raise ValueError(f"Unknown merge mode: {mm}")
    modes = parse_attention(args.attention)

    if args._subprocess_json:  # one configuration, JSON on stdout
        (mode, param), = modes
        stats = run_config(args, mode, param, batch_sizes[0], seq_lengths[0], merge_modes[0] == "merge")
        print(json.dumps(stats), flush=True)
        return 0

    print(describe_flags(args), flush=True)

    results, failures = {}, []
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ)
    env["PYTHONPATH"] = root + (os.pathsep + env["PYTHONPATH"] if env.get("PYTHONPATH") else "")
    for merge_mode in merge_modes:
        merge_label = "merged" if merge_mode == "merge" else "baseline"
        for mode, param in modes:
            print(f"\n### {merge_label} / {_label(mode, param)} ###", flush=True)
            for batch in batch_sizes:
                for seq_len in seq_lengths:
                    key = (merge_label, _label(mode, param), batch, seq_len)
                    try:
                        r = subprocess.run(_sub_cmd(args, mode, param, batch, seq_len, merge_mode),
                                           capture_output=True, text=True, timeout=args.timeout, env=env, cwd=root)
                    except subprocess.TimeoutExpired:
                        print(f"  BS={batch}, Seq={seq_len}: TIMEOUT", flush=True)
                        failures.append(key)
                        continue
                    stats = None
                    for line in r.stdout.strip().splitlines():
                        if line.startswith("{"):
                            stats = json.loads(line)
                    if r.returncode == 0 and stats is not None:
                        results[key] = stats
                        print(f"  BS={batch}, Seq={seq_len}: {stats['mean_ms']:.2f} ms (P50={stats['p50_ms']:.2f})",
                              flush=True)
                    elif _is_oom(r.stdout + r.stderr):
                        print(f"  BS={batch}, Seq={seq_len}: OOM", flush=True)
                    else:
                        print(f"  BS={batch}, Seq={seq_len}: FAILED (exit {r.returncode})", flush=True)
                        for line in r.stderr.strip().splitlines()[-3:]:
                            print(f"    {line}")
                        failures.append(key)
    print("\n" + "=" * 70)
    print("SUMMARY")
    print("=" * 70)
    print(f"{'Merge':<10} {'Attention':<12} {'BS':<6} {'Seq':<8} {'Mean (ms)':<12} {'P50 (ms)':<12} {'tok/s':<10}")
    print("-" * 72)
    for (merge, attn, bs, seq), s in results.items():
        print(f"{merge:<10} {attn:<12} {bs:<6} {seq:<8} {s['mean_ms']:<12.3f} {s['p50_ms']:<12.3f} "
              f"{s['tokens_per_s']:<10.0f}")
    if failures:
        print(f"\n{len(failures)} configuration(s) FAILED: {failures}")
    return 1 if failures else 0


if __name__ == "__main__":
    sys.exit(main())
