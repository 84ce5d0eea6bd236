"""SAGA checkpoint loading: a Hugging Face model directory (config.json +
safetensors) into the decoder's weight layout.

What the reference reads (lm_eval_saga.py:52-146):
  * config.json of a Qwen2 / Llama model; `num_key_heads` and
    `num_value_heads`, when present, are the key-head and value-head counts
    of a SAGA checkpoint (merge_heads.py:225, train_scratch.py:331-356 write
    them); without them both fall back to `num_key_value_heads` (a plain GQA
    checkpoint);
  * the weights from `model.safetensors`, else from every
    `model-*.safetensors` shard (lm_eval_saga.py:88-97; a
    model.safetensors.index.json weight map is honoured too);
  * k_proj [num_key_heads * d, hidden] and v_proj [num_value_heads * d,
    hidden], each with its optional bias, at the checkpoint's own sizes
    (lm_eval_saga.py:101-130), d = hidden_size // num_attention_heads
    (lm_eval_saga.py:99; a config `head_dim` is taken when given).
Pair-merged checkpoints (merge_heads.py:101-202) are saved with q/v/o already
permuted to the merged grouping, so `kv_merge_pairs` is not needed to load
them.  A plain GQA checkpoint can be merged at load time to fewer key heads by
averaging consecutive groups of key heads and their biases
(num_key_heads=..., the reference's merge_key_projection_heads,
gqa_distill.py:59-100 / speedup.py:92-115).

Decoder layout (SagaDecoder._WEIGHT_SHAPES): q, k, v rows concatenated in
w_qkv [(n_q + n_k + n_v) * d, hidden] (zero bias when the model has none),
gate and up rows in w_gu [2 * intermediate, hidden], RMSNorm weights ln1 /
ln2 per layer and ln_f, the embedding, and lm_head (None when tied).
Models with o_proj / MLP biases or a RoPE scaling rule other than the
default are refused, not silently mis-run.
"""
from __future__ import annotations

import glob
import json
import os
from typing import Dict, Optional, Tuple

import torch

from .decoder import DecoderShape


def read_config(path: str) -> dict:
    with open(os.path.join(path, "config.json")) as f:
        return json.load(f)


def _rope_theta(cfg: dict) -> float:
    """RoPE base of a transformers 4.x (rope_theta + rope_scaling) or 5.x
    (rope_parameters) config; only the default (unscaled) rule is supported."""
    rp = cfg.get("rope_parameters") or {}
    scaling = cfg.get("rope_scaling") or {}
    rtype = rp.get("rope_type", scaling.get("rope_type", scaling.get("type", "default")))
    if rtype not in (None, "default"):
        raise NotImplementedError(f"RoPE type {rtype!r}: only the default rotary embedding is supported")
    theta = cfg.get("rope_theta", rp.get("rope_theta"))
    return float(theta if theta is not None else 10000.0)


def shape_from_config(cfg: dict, qkv_bias: bool, num_key_heads: Optional[int] = None) -> DecoderShape:
    """DecoderShape of a checkpoint config (lm_eval_saga.py:60-69)."""
    n_q = int(cfg["num_attention_heads"])
    n_kv = int(cfg.get("num_key_value_heads", n_q))
    n_k = int(cfg.get("num_key_heads", n_kv))
    n_v = int(cfg.get("num_value_heads", n_kv))
    if num_key_heads is not None:
        n_k = int(num_key_heads)
    hidden = int(cfg["hidden_size"])
    head_dim = int(cfg.get("head_dim") or hidden // n_q)
    for name, n in (("key", n_k), ("value", n_v)):
        if n < 1 or n_q % n:
            raise ValueError(f"{n_q} query heads are not a multiple of {n} {name} heads")
    return DecoderShape(layers=int(cfg["num_hidden_layers"]), hidden=hidden, n_q=n_q, n_k=n_k, n_v=n_v,
                        head_dim=head_dim, intermediate=int(cfg["intermediate_size"]), vocab=int(cfg["vocab_size"]),
                        rope_theta=_rope_theta(cfg), eps=float(cfg.get("rms_norm_eps", 1e-6)), qkv_bias=qkv_bias)


def checkpoint_files(path: str) -> list:
    """Safetensors files of a checkpoint directory, in the reference's order
    of preference (lm_eval_saga.py:88-97)."""
    single = os.path.join(path, "model.safetensors")
    if os.path.exists(single):
        return [single]
    index = os.path.join(path, "model.safetensors.index.json")
    if os.path.exists(index):
        with open(index) as f:
            wmap = json.load(f)["weight_map"]
        return [os.path.join(path, n) for n in sorted(set(wmap.values()))]
    shards = sorted(glob.glob(os.path.join(path, "model-*.safetensors")))
    if not shards:
        raise FileNotFoundError(f"no model.safetensors or model-*.safetensors in {path}")
    return shards


class _Tensors:
    """Lazy name -> tensor access over the checkpoint's safetensors files
    (each tensor read once, when asked for)."""

    def __init__(self, files):
        from safetensors import safe_open
        self._where: Dict[str, object] = {}
        self._handles = []
        for fn in files:
            h = safe_open(fn, framework="pt", device="cpu")
            self._handles.append(h)
            for k in h.keys():
                self._where[k] = h

    def __contains__(self, name: str) -> bool:
        return name in self._where

    def keys(self):
        return self._where.keys()

    def get(self, name: str) -> torch.Tensor:
        if name not in self._where:
            raise KeyError(f"checkpoint has no tensor {name!r}")
        return self._where[name].get_tensor(name)


def merge_key_heads(w: torch.Tensor, b: Optional[torch.Tensor], n_from: int, n_to: int,
                    head_dim: int) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """k_proj of n_from heads -> n_to heads, each the mean of a consecutive
    group of n_from / n_to heads (gqa_distill.py:83-91), computed in fp32."""
    if n_to > n_from or n_from % n_to:
        raise ValueError(f"cannot merge {n_from} key heads into {n_to}")
    grp = n_from // n_to
    hidden = w.shape[1]
    wm = w.float().reshape(n_to, grp, head_dim, hidden).mean(1).reshape(n_to * head_dim, hidden).to(w.dtype)
    bm = None
    if b is not None:
        bm = b.float().reshape(n_to, grp, head_dim).mean(1).reshape(n_to * head_dim).to(b.dtype)
    return wm, bm


def load_checkpoint(path: str, num_key_heads: Optional[int] = None,
                    dtype: torch.dtype = torch.bfloat16) -> Tuple[DecoderShape, dict]:
    """(DecoderShape, weights) of a checkpoint directory; weights in the
    decoder's layout, on the CPU in `dtype`.  num_key_heads: merge the
    checkpoint's key heads down to this many at load time."""
    cfg = read_config(path)
    T = _Tensors(checkpoint_files(path))
    pre = "model.layers.{}."
    qkv_bias = pre.format(0) + "self_attn.q_proj.bias" in T
    for extra in ("self_attn.o_proj.bias", "mlp.gate_proj.bias", "mlp.up_proj.bias", "mlp.down_proj.bias"):
        if pre.format(0) + extra in T:
            raise NotImplementedError(f"checkpoint has {extra}: o_proj / MLP biases are not supported")
    stored = shape_from_config(cfg, qkv_bias)  # the heads the tensors hold
    shape = stored if num_key_heads is None else shape_from_config(cfg, qkv_bias, num_key_heads)
    s, d = shape, shape.head_dim
    src_n_k = stored.n_k

    def cast(t):
        return t.to(dtype).contiguous()

    def expect(t, want, name):
        if tuple(t.shape) != tuple(want):
            raise ValueError(f"{name}: checkpoint tensor is {tuple(t.shape)}, the config implies {tuple(want)}")
        return t

    w = {"ln1": [], "ln2": [], "w_qkv": [], "b_qkv": [], "w_o": [], "w_gu": [], "w_d": []}
    for l in range(s.layers):
        p = pre.format(l)
        a = p + "self_attn."
        q = expect(T.get(a + "q_proj.weight"), (s.n_q * d, s.hidden), a + "q_proj.weight")
        k = expect(T.get(a + "k_proj.weight"), (src_n_k * d, s.hidden), a + "k_proj.weight")
        v = expect(T.get(a + "v_proj.weight"), (s.n_v * d, s.hidden), a + "v_proj.weight")
        if qkv_bias:
            qb, kb, vb = (T.get(a + n + "_proj.bias") for n in "qkv")
        else:
            qb = kb = vb = None
        if src_n_k != s.n_k:
            k, kb = merge_key_heads(k, kb, src_n_k, s.n_k, d)
        w["w_qkv"].append(cast(torch.cat([q, k, v], 0)))
        if qkv_bias:
            w["b_qkv"].append(cast(torch.cat([qb, kb, vb], 0)))
        else:
            w["b_qkv"].append(torch.zeros(s.qkv_width, dtype=dtype))
        w["w_o"].append(cast(T.get(a + "o_proj.weight")))
        m = p + "mlp."
        w["w_gu"].append(cast(torch.cat([T.get(m + "gate_proj.weight"), T.get(m + "up_proj.weight")], 0)))
        w["w_d"].append(cast(T.get(m + "down_proj.weight")))
        w["ln1"].append(cast(T.get(p + "input_layernorm.weight")))
        w["ln2"].append(cast(T.get(p + "post_attention_layernorm.weight")))
    w["embed"] = cast(T.get("model.embed_tokens.weight"))
    w["ln_f"] = cast(T.get("model.norm.weight"))
    tied = cfg.get("tie_word_embeddings", False) or "lm_head.weight" not in T
    w["lm_head"] = None if tied else cast(T.get("lm_head.weight"))
    return shape, w
