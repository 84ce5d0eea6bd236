"""The decode-latency harness's command line (saga_amd/speedup.py, mirroring
the reference's speedup.py:447-495), on the CPU: attention-mode parsing and
the per-configuration subprocess command."""
import argparse

import pytest

from saga_amd import speedup


def test_attention_modes_parse_like_the_reference():
    assert speedup.parse_attention("full, atopn:512,atopn_amortized:64,vanilla") == [
        ("full", None), ("atopn", 512), ("atopn", 64), ("vanilla", None)]
    with pytest.raises(ValueError):
        speedup.parse_attention("topk:5")


def test_subprocess_command_carries_one_configuration():
    args = argparse.Namespace(model_path="/ckpt", num_new_tokens=8, num_iterations=3, num_warmup=1,
                              dtype="bfloat16", new_heads=1, exempt_layers="0,14")
    cmd = speedup._sub_cmd(args, "atopn", 512, 8, 32768, "merge")
    assert cmd[1:3] == ["-m", "saga_amd.speedup"]
    flat = " ".join(cmd)
    for part in ("--attention atopn:512", "--batch_sizes 8", "--seq_lengths 32768", "--merge_mode merge",
                 "--exempt_layers 0,14", "--_subprocess_json"):
        assert part in flat
    args.exempt_layers = ""
    assert "--exempt_layers" not in speedup._sub_cmd(args, "full", None, 1, 128, "baseline")


def test_bad_merge_mode_is_refused():
    with pytest.raises(ValueError):
        speedup.main(["--merge_mode", "both-ways", "--_subprocess_json"])
