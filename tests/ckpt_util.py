"""Tiny Hugging Face checkpoints for the checkpoint-loader tests, and a
float64 forward of the decoder weight layout built from the oracle's ops.

A GQA model whose key heads are identical within each group of g = n_kv /
n_k heads computes exactly what a SAGA model with n_k key heads (each the
group's shared head) computes: every query head sees the same key rows.  So
transformers' own forward of such a model is an independent reference for
SAGA checkpoints, which transformers cannot run natively."""
import json
import os

import numpy as np
import torch

from oracle import saga_oracle as O


def tiny_hf_model(kind: str, n_kv: int, n_k_shared: int, tie: bool, seed: int = 0, d: int = 16,
                  intermediate: int = 96, vocab: int = 128):
    """fp32 Qwen2 (q/k/v bias) or Llama (no bias) with 4 query heads of d
    dims, n_kv key/value heads whose key projections (and biases) repeat
    within groups of n_kv / n_k_shared heads, and non-trivial norm weights."""
    from transformers import LlamaConfig, LlamaForCausalLM, Qwen2Config, Qwen2ForCausalLM
    common = dict(hidden_size=4 * d, intermediate_size=intermediate, num_hidden_layers=2, num_attention_heads=4,
                  num_key_value_heads=n_kv, vocab_size=vocab, max_position_embeddings=4096,
                  rope_parameters={"rope_theta": 5e5, "rope_type": "default"}, rms_norm_eps=1e-5,
                  tie_word_embeddings=tie)
    if kind == "qwen2":
        cfg, cls = Qwen2Config(**common), Qwen2ForCausalLM
    else:
        cfg, cls = LlamaConfig(head_dim=d, attention_bias=False, **common), LlamaForCausalLM
    cfg._attn_implementation = "eager"
    torch.manual_seed(seed)
    model = cls(cfg).float().eval()
    g = n_kv // n_k_shared
    with torch.no_grad():
        for name, p in model.named_parameters():  # HF init leaves norms at 1 and biases at 0
            if "norm" in name:
                p.copy_(1 + 0.3 * torch.randn_like(p))
            elif name.endswith("bias"):
                p.copy_(0.1 * torch.randn_like(p))
        for layer in model.model.layers:
            k = layer.self_attn.k_proj
            wk = k.weight.view(n_k_shared, g, d, -1)
            wk.copy_(wk[:, :1].expand_as(wk).clone())
            if k.bias is not None:
                bk = k.bias.view(n_k_shared, g, d)
                bk.copy_(bk[:, :1].expand_as(bk).clone())
    return model


def hf_logits(model, ids) -> np.ndarray:
    with torch.no_grad():
        return model(torch.as_tensor(ids)[None]).logits[0].double().numpy()


def save_saga_checkpoint(model, path: str, n_k: int, n_v=None):
    """A SAGA checkpoint of a tiny_hf_model whose key heads repeat in groups:
    config.json gains num_key_heads (and num_value_heads when given), k_proj
    keeps the first head of every group (merge_heads.py:225 /
    train_scratch.py:331-356 write checkpoints of this form)."""
    from safetensors.torch import save_file
    os.makedirs(path, exist_ok=True)
    cfg = model.config.to_dict()
    n_kv = cfg["num_key_value_heads"]
    d = cfg["hidden_size"] // cfg["num_attention_heads"]
    sd = {k: v.detach().clone().contiguous() for k, v in model.state_dict().items()}
    if cfg.get("tie_word_embeddings"):
        sd.pop("lm_head.weight", None)
    g = n_kv // n_k
    for l in range(cfg["num_hidden_layers"]):
        a = f"model.layers.{l}.self_attn.k_proj."
        sd[a + "weight"] = sd[a + "weight"].view(n_k, g, d, -1)[:, 0].reshape(n_k * d, -1).contiguous()
        if a + "bias" in sd:
            sd[a + "bias"] = sd[a + "bias"].view(n_k, g, d)[:, 0].reshape(-1).contiguous()
    cfg["num_key_heads"] = n_k
    if n_v is not None:
        cfg["num_value_heads"] = n_v
    save_file(sd, os.path.join(path, "model.safetensors"))
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(cfg, f)


def forward64(shape, w, ids) -> np.ndarray:
    """Logits [T, vocab] of the decoder weight layout over a causal prompt,
    in float64 from the oracle's rmsnorm / rope / dense attention / silu_mul
    (attention of position t over positions 0..t)."""
    f = lambda t: t.detach().double().cpu().numpy()
    s, d = shape, shape.head_dim
    T = len(ids)
    pos = np.arange(T)
    x = f(w["embed"])[np.asarray(ids)]
    for l in range(s.layers):
        h = O.rmsnorm(x, f(w["ln1"][l]), s.eps)
        qkv = (h @ f(w["w_qkv"][l]).T + f(w["b_qkv"][l])).reshape(T, s.n_q + s.n_k + s.n_v, d)
        q = O.rope(qkv[:, :s.n_q], pos[:, None], s.rope_theta)
        K = O.rope(qkv[:, s.n_q:s.n_q + s.n_k], pos[:, None], s.rope_theta).transpose(1, 0, 2)[None]
        V = qkv[:, s.n_q + s.n_k:].transpose(1, 0, 2)[None]
        attn = np.stack([O.dense(q[t][None, :, None, :], K[:, :, :t + 1], V[:, :, :t + 1])[0, :, 0]
                         for t in range(T)])
        x = x + attn.reshape(T, -1) @ f(w["w_o"][l]).T
        h = O.rmsnorm(x, f(w["ln2"][l]), s.eps)
        x = x + O.silu_mul(h @ f(w["w_gu"][l]).T) @ f(w["w_d"][l]).T
    head = w["lm_head"] if w.get("lm_head") is not None else w["embed"]
    return O.rmsnorm(x, f(w["ln_f"]), s.eps) @ f(head).T
