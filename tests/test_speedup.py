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


# The reference's published latency commands, as its documentation gives
# them (eval.md:43-66; run_eval.sh:89-140 runs the same with --batch_sizes
# 1,4,16 and atopn 512 / 1024 / 2048, with and without --exempt_layers).
REFERENCE_COMMANDS = [
    "--model_path ./models/Qwen2.5-1.5B --merge_mode merge --new_heads 1 --attention full "
    "--batch_sizes 1,4,16,32,64 --seq_lengths 4096,8192,16384,32768,65536,131072 "
    "--num_warmup 5 --num_iterations 100 --num_new_tokens 8 --cuda_graph --compile_mode default",
    "--model_path ./models/Qwen2.5-1.5B --merge_mode merge --new_heads 1 --attention atopn:512 "
    "--exempt_layers 0,14 --batch_sizes 1,4,16,32,64 --seq_lengths 4096,8192,16384,32768,65536,131072 "
    "--num_warmup 5 --num_iterations 100 --num_new_tokens 8 --cuda_graph --compile_mode default",
    "--model_path ./models/Qwen2.5-1.5B --merge_mode baseline --attention full "
    "--batch_sizes 1,4,16,32,64 --seq_lengths 4096,8192,16384,32768,65536,131072 "
    "--num_warmup 5 --num_iterations 100 --num_new_tokens 8 --cuda_graph --compile_mode default",
] + [
    f"--model_path ./models/Qwen2.5-1.5B --merge_mode {mm} {'--new_heads 1 ' if mm == 'merge' else ''}"
    f"--attention atopn:{n} --exempt_layers 0,14 --batch_sizes 1,4,16 "
    "--seq_lengths 4096,8192,16384,32768,65536,131072 --num_warmup 5 --num_iterations 100 --num_new_tokens 8 "
    "--cuda_graph --compile_mode default"
    for mm in ("merge", "baseline") for n in (512, 1024, 2048)
]


@pytest.mark.parametrize("line", REFERENCE_COMMANDS)
def test_reference_latency_commands_parse(line):
    args = speedup.build_parser().parse_args(line.split())
    assert args.cuda_graph and args.compile_mode == "default" and not args.no_compile
    modes = speedup.parse_attention(args.attention)
    assert len(modes) == 1 and modes[0][0] in ("full", "atopn")
    assert [int(x) for x in args.seq_lengths.split(",")][-1] == 131072
    assert args.num_new_tokens == 8 and args.num_iterations == 100 and args.num_warmup == 5
    # the graph flag reaches every configuration's subprocess
    mode, param = modes[0]
    cmd = speedup._sub_cmd(args, mode, param, 1, 4096, args.merge_mode)
    assert "--cuda_graph" in cmd
    text = speedup.describe_flags(args)
    assert "CUDA graph: enabled" in text and "Compile: no-op" in text


def test_other_reference_flags():
    args = speedup.build_parser().parse_args(
        ["--no_compile", "--compile_mode", "max-autotune", "--calibrate_during_measurement", "--profile_decode",
         "--profile_output", "run.json", "--attention", "atopn:1024"])
    assert args.no_compile and args.calibrate_during_measurement and args.profile_decode
    text = speedup.describe_flags(args)
    assert "kernels launched eagerly" in text and "Profiling decode: output=run.json" in text
    cmd = speedup._sub_cmd(args, "atopn", 1024, 4, 8192, "merge")
    assert "--cuda_graph" not in cmd and cmd[cmd.index("--profile_output") + 1] == "run.json"
    # the reference's trace naming (speedup.py:657-658)
    assert speedup.trace_name("run.json", True, "atopn", 1024, 4, 8192) == "run_merged_atopn_1024_bs4_seq8192.json"
    assert speedup.trace_name("t.json", False, "full", None, 1, 4096) == "t_baseline_full_bs1_seq4096.json"
    with pytest.raises(SystemExit):
        speedup.build_parser().parse_args(["--compile_mode", "fastest"])
