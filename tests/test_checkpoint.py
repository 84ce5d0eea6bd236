"""SAGA checkpoint loading (saga_amd.checkpoint), on the CPU.

The loaded weights, run through a float64 forward of the decoder layout built
from the oracle's ops, must give transformers' own logits for the same
checkpoint: a plain GQA checkpoint, the same merged to fewer key heads at load
time, and SAGA checkpoints with num_key_heads / num_value_heads in config.json
(lm_eval_saga.py:52-146).  Tied and untied LM heads, Qwen2 (q/k/v bias) and
Llama (no bias).  The head merge is pinned by a closed form, the file
discovery by single-file, indexed and globbed shards, and the refusals by
their error types."""
import json
import os

import numpy as np
import pytest
import torch

from conftest import rel_l2
from saga_amd.checkpoint import load_checkpoint, merge_key_heads, shape_from_config

transformers = pytest.importorskip("transformers")
from ckpt_util import forward64, hf_logits, save_saga_checkpoint, tiny_hf_model  # noqa: E402

IDS = [5, 17, 99, 3, 64, 127, 0, 42, 8, 77]


def _save_hf(model, path):
    model.save_pretrained(path, safe_serialization=True)
    return path


@pytest.mark.parametrize("kind,tie", [("qwen2", True), ("llama", False)])
def test_gqa_checkpoint_matches_transformers(tmp_path, kind, tie):
    model = tiny_hf_model(kind, n_kv=2, n_k_shared=1, tie=tie)
    ref = hf_logits(model, IDS)
    path = _save_hf(model, str(tmp_path / "gqa"))
    shape, w = load_checkpoint(path, dtype=torch.float32)
    assert (shape.n_q, shape.n_k, shape.n_v, shape.head_dim, shape.layers) == (4, 2, 2, 16, 2)
    assert shape.qkv_bias == (kind == "qwen2") and shape.rope_theta == 5e5 and shape.eps == 1e-5
    assert (w["lm_head"] is None) == tie
    assert rel_l2(forward64(shape, w, IDS), ref) < 1e-5
    # the same checkpoint merged to one key head at load time: its two key
    # heads are identical, so the merged model is the same model
    shape1, w1 = load_checkpoint(path, num_key_heads=1, dtype=torch.float32)
    assert (shape1.n_k, shape1.n_v) == (1, 2)
    assert rel_l2(forward64(shape1, w1, IDS), ref) < 1e-5


@pytest.mark.parametrize("kind,tie", [("qwen2", False), ("llama", True)])
def test_saga_checkpoint_matches_transformers(tmp_path, kind, tie):
    """num_key_heads = 1 next to num_key_value_heads = 2: k_proj holds one head."""
    model = tiny_hf_model(kind, n_kv=2, n_k_shared=1, tie=tie)
    ref = hf_logits(model, IDS)
    path = str(tmp_path / "saga")
    save_saga_checkpoint(model, path, n_k=1)
    shape, w = load_checkpoint(path, dtype=torch.float32)
    assert (shape.n_k, shape.n_v) == (1, 2)
    assert w["w_qkv"][0].shape == ((4 + 1 + 2) * 16, 64)
    assert rel_l2(forward64(shape, w, IDS), ref) < 1e-5


def test_saga_checkpoint_with_value_heads(tmp_path):
    """num_value_heads (4) and num_key_heads (1) both differ from
    num_key_value_heads (2, left over from the base model): the explicit
    counts win (train_scratch.py:331-356)."""
    model = tiny_hf_model("qwen2", n_kv=4, n_k_shared=1, tie=True)
    ref = hf_logits(model, IDS)
    path = str(tmp_path / "saga_v")
    save_saga_checkpoint(model, path, n_k=1, n_v=4)
    cfg = json.load(open(os.path.join(path, "config.json")))
    cfg["num_key_value_heads"] = 2
    json.dump(cfg, open(os.path.join(path, "config.json"), "w"))
    shape, w = load_checkpoint(path, dtype=torch.float32)
    assert (shape.n_k, shape.n_v) == (1, 4)
    assert rel_l2(forward64(shape, w, IDS), ref) < 1e-5


def test_merge_key_heads_closed_form():
    """Head h filled with h + 1: groups of consecutive heads average to
    closed-form values (gqa_distill.py:83-91; speedup.py:92-115 is the
    one-head case)."""
    d, hidden = 4, 3
    w = torch.cat([torch.full((d, hidden), float(h + 1)) for h in range(4)])
    b = torch.cat([torch.full((d,), 10.0 * (h + 1)) for h in range(4)])
    w2, b2 = merge_key_heads(w, b, 4, 2, d)
    assert torch.equal(w2, torch.cat([torch.full((d, hidden), 1.5), torch.full((d, hidden), 3.5)]))
    assert torch.equal(b2, torch.cat([torch.full((d,), 15.0), torch.full((d,), 35.0)]))
    w1, b1 = merge_key_heads(w, None, 4, 1, d)
    assert torch.equal(w1, torch.full((d, hidden), 2.5)) and b1 is None
    with pytest.raises(ValueError):
        merge_key_heads(w, b, 4, 3, d)


def test_sharded_checkpoints_load_the_same(tmp_path):
    """model.safetensors, an indexed set of shards and unindexed
    model-*.safetensors shards (lm_eval_saga.py:88-97) give the same weights."""
    from safetensors.torch import load_file, save_file
    model = tiny_hf_model("qwen2", n_kv=2, n_k_shared=2, tie=True)
    single = _save_hf(model, str(tmp_path / "single"))
    _, w0 = load_checkpoint(single)
    sd = load_file(os.path.join(single, "model.safetensors"))
    names = sorted(sd)
    parts = [names[::2], names[1::2]]
    for variant in ("indexed", "globbed"):
        d = tmp_path / variant
        d.mkdir()
        (d / "config.json").write_text((tmp_path / "single" / "config.json").read_text())
        wmap = {}
        for i, part in enumerate(parts):
            fn = f"model-{i + 1:05d}-of-00002.safetensors"
            save_file({k: sd[k] for k in part}, str(d / fn))
            wmap.update({k: fn for k in part})
        if variant == "indexed":
            (d / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": wmap}))
        _, w1 = load_checkpoint(str(d))
        for k in w0:
            a, b = w0[k], w1[k]
            if a is None:
                assert b is None
            elif isinstance(a, list):
                assert all(torch.equal(x, y) for x, y in zip(a, b))
            else:
                assert torch.equal(a, b)


def test_refusals(tmp_path):
    model = tiny_hf_model("llama", n_kv=2, n_k_shared=1, tie=False)
    path = _save_hf(model, str(tmp_path / "m"))
    cfg_path = os.path.join(path, "config.json")
    cfg = json.load(open(cfg_path))
    # a config that claims one key head over a k_proj of two
    json.dump(dict(cfg, num_key_heads=1), open(cfg_path, "w"))
    with pytest.raises(ValueError, match="k_proj"):
        load_checkpoint(path)
    # a RoPE scaling rule the decoder does not implement
    json.dump(dict(cfg, rope_parameters={"rope_theta": 5e5, "rope_type": "llama3", "factor": 8.0}),
              open(cfg_path, "w"))
    with pytest.raises(NotImplementedError):
        load_checkpoint(path)
    # key heads that do not divide the query heads
    with pytest.raises(ValueError):
        shape_from_config(dict(cfg, num_key_heads=3), qkv_bias=False)
    # no weights at all
    os.remove(os.path.join(path, "model.safetensors"))
    with pytest.raises(FileNotFoundError):
        load_checkpoint(path)


def test_transformers4_config_keys():
    """rope_theta at the top level and rope_scaling null (transformers 4.x
    config.json, as Qwen2.5 and SmolLM2 checkpoints ship it)."""
    cfg = {"num_attention_heads": 12, "num_key_value_heads": 2, "num_key_heads": 1, "hidden_size": 1536,
           "num_hidden_layers": 28, "intermediate_size": 8960, "vocab_size": 151936, "rope_theta": 1e6,
           "rope_scaling": None, "rms_norm_eps": 1e-6}
    s = shape_from_config(cfg, qkv_bias=True)
    assert (s.n_q, s.n_k, s.n_v, s.head_dim, s.rope_theta, s.eps) == (12, 1, 2, 128, 1e6, 1e-6)
    from saga_amd.decoder import QWEN25_15B_SAGA
    assert s == QWEN25_15B_SAGA


def test_decoder_takes_loaded_weights_on_cpu(tmp_path):
    """SagaDecoder(weights=...) keeps the loaded tensors (shapes checked, an
    untied LM head kept apart from the embedding) and rejects a wrong shape."""
    from saga_amd.decoder import SagaDecoder
    model = tiny_hf_model("llama", n_kv=2, n_k_shared=1, tie=False)
    path = str(tmp_path / "saga")
    save_saga_checkpoint(model, path, n_k=1)
    shape, w = load_checkpoint(path)
    m = SagaDecoder(shape, batch=2, max_len=64, device="cpu", weights=w, pack_weights=False)
    assert torch.equal(m.w_qkv[1], w["w_qkv"][1]) and torch.equal(m.lm_head, w["lm_head"])
    assert not torch.equal(m.lm_head, m.embed)
    assert m.k_cache.shape == (2, 2, 1, 64, 16) and m.v_cache.shape == (2, 2, 2, 64, 16)
    bad = dict(w, w_o=[t[:, :-16] for t in w["w_o"]])
    with pytest.raises(ValueError, match="w_o"):
        SagaDecoder(shape, batch=2, max_len=64, device="cpu", weights=bad, pack_weights=False)
