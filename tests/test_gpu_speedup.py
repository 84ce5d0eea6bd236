"""The decode-latency harness end to end on the GPU: a tiny SAGA checkpoint,
two attention modes, each configuration in its own subprocess (the
reference's speedup.py:532-610 isolation), per-token latency statistics in
the summary."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

pytest.importorskip("transformers")
from ckpt_util import save_saga_checkpoint, tiny_hf_model  # noqa: E402

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_harness_runs_each_configuration_in_a_subprocess(tmp_path):
    path = str(tmp_path / "saga")
    save_saga_checkpoint(tiny_hf_model("qwen2", n_kv=2, n_k_shared=1, tie=True, d=64, intermediate=512, vocab=1024),
                         path, n_k=1)
    cmd = [sys.executable, "-m", "saga_amd.speedup", "--model_path", path, "--attention", "full,atopn:16",
           "--batch_sizes", "2", "--seq_lengths", "200", "--num_new_tokens", "4", "--num_warmup", "1",
           "--num_iterations", "2", "--timeout", "100"]
    print("harness:", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=110, cwd=ROOT)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0
    assert "SUMMARY" in r.stdout and "FAILED" not in r.stdout
    rows = [l for l in r.stdout.splitlines() if l.startswith("merged")]
    assert len(rows) == 2 and {l.split()[1] for l in rows} == {"full", "atopn:16"}
    assert all(float(l.split()[4]) > 0 for l in rows)  # mean ms per token


def test_harness_graphs_and_decode_trace(tmp_path):
    """--cuda_graph replays the captured steps; --profile_decode writes one
    chrome trace of the measured generations per configuration, named as the
    reference names them (speedup.py:640-661)."""
    path = str(tmp_path / "saga")
    save_saga_checkpoint(tiny_hf_model("qwen2", n_kv=2, n_k_shared=1, tie=True, d=64, intermediate=512, vocab=1024),
                         path, n_k=1)
    stem = str(tmp_path / "trace.json")
    cmd = [sys.executable, "-m", "saga_amd.speedup", "--model_path", path, "--attention", "atopn:16",
           "--batch_sizes", "2", "--seq_lengths", "200", "--num_new_tokens", "4", "--num_warmup", "1",
           "--num_iterations", "2", "--timeout", "100", "--cuda_graph", "--compile_mode", "default",
           "--calibrate_during_measurement", "--profile_decode", "--profile_output", stem]
    print("harness:", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=110, cwd=ROOT)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0
    assert "CUDA graph: enabled" in r.stdout and "Compile: no-op" in r.stdout
    trace = str(tmp_path / "trace_merged_atopn_16_bs2_seq200.json")
    assert os.path.exists(trace), os.listdir(tmp_path)
    with open(trace) as f:
        assert "traceEvents" in f.read(4096)
