"""Seeded input cases shared by the golden-vector generator and the tests.

Inputs are drawn with numpy's PCG64 generator (``default_rng(seed)``), whose
stream is stable across numpy versions, then stored nowhere: every consumer
regenerates them and checks the SHA-256 recorded next to the expected outputs.
bf16 cases round the float32 draws to bfloat16 once (round-to-nearest-even),
and the fp32 references run on those rounded values.
"""
from __future__ import annotations

import hashlib

import numpy as np

# name -> parameters.  b/q_h/k_h/v_h/d/L: shapes; N: Atop-N top_n; mask: None,
# "bool" (HF decode mask, added as 0/1) or "float" (additive, finfo.min for
# masked slots); mask_extra: extra mask columns beyond L (sliced off by the
# reference, attention/attention.py:125); qscale: multiplier on the queries
# (larger -> more peaked softmax); bf16: round inputs to bfloat16.
CASES = {
    # the CPU-runnable single-layer decode step: b1, 15 Q / 1 K / 5 V heads,
    # d64, context 4096, fp32, N(0,1) q/k/v, N=128.
    "c1": dict(seed=1, b=1, q_h=15, k_h=1, v_h=5, d=64, L=4096, N=128, mask=None,
               scaling=None, qscale=1.0, bf16=False),
    "bool_mask": dict(seed=2, b=2, q_h=6, k_h=1, v_h=2, d=64, L=700, N=32, mask="bool",
                      mask_extra=8, scaling=0.1, qscale=1.0, bf16=False),
    "float_mask": dict(seed=3, b=2, q_h=6, k_h=2, v_h=3, d=128, L=300, N=64, mask="float",
                       mask_extra=0, scaling=None, qscale=2.0, bf16=False),
    "short_L": dict(seed=4, b=1, q_h=4, k_h=1, v_h=4, d=64, L=100, N=64, mask=None,
                    scaling=None, qscale=1.0, bf16=False),
    "peaked": dict(seed=5, b=2, q_h=12, k_h=1, v_h=2, d=128, L=2048, N=64, mask=None,
                   scaling=None, qscale=4.0, bf16=False),
    "bf16": dict(seed=6, b=2, q_h=12, k_h=1, v_h=2, d=128, L=1024, N=128, mask=None,
                 scaling=None, qscale=1.0, bf16=True),
    # key row 3 of batch 0 is 30x query head 0 of the fast step: that logit
    # exceeds the tail max by > 88, exp overflows, s = inf, t = inf, nothing
    # passes and the reference's softmax over an all -inf buffer gives NaN.
    "inf_threshold": dict(seed=7, b=1, q_h=4, k_h=1, v_h=2, d=64, L=512, N=32, mask=None,
                          scaling=None, qscale=1.0, bf16=False, plant="inf"),
}


def _round_bf16(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + (((u >> 16) & 1) + 0x7FFF)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32).reshape(x.shape)


def make_inputs(name: str) -> dict:
    """Regenerate the float32 inputs of a case: q1 (calibration query), q2
    (fast-step query), key, value and (optionally) the attention mask."""
    c = CASES[name]
    rng = np.random.default_rng(c["seed"])
    b, q_h, k_h, v_h, d, L = c["b"], c["q_h"], c["k_h"], c["v_h"], c["d"], c["L"]
    q1 = rng.standard_normal((b, q_h, 1, d), dtype=np.float32) * np.float32(c["qscale"])
    q2 = rng.standard_normal((b, q_h, 1, d), dtype=np.float32) * np.float32(c["qscale"])
    key = rng.standard_normal((b, k_h, L, d), dtype=np.float32)
    value = rng.standard_normal((b, v_h, L, d), dtype=np.float32)
    if c.get("plant") == "inf":
        key[0, 0, 3, :] = q2[0, 0, 0, :] * np.float32(30.0)
    out = dict(q1=q1, q2=q2, key=key, value=value)
    if c.get("bf16"):
        out = {k: _round_bf16(v) for k, v in out.items()}
    if c["mask"] is not None:
        Lm = L + c.get("mask_extra", 0)
        valid = np.ones((b, 1, 1, Lm), dtype=bool)
        # batch row i sees positions < L - 5*(i+1): the tail of the static
        # buffer is "unfilled" as in a static KV cache.
        for i in range(b):
            valid[i, :, :, L - 5 * (i + 1):] = False
        if c["mask"] == "bool":
            out["mask"] = valid
        else:
            out["mask"] = np.where(valid, np.float32(0), np.finfo(np.float32).min).astype(np.float32)
    return out


def inputs_sha256(inp: dict) -> str:
    h = hashlib.sha256()
    for k in sorted(inp):
        a = np.ascontiguousarray(inp[k])
        h.update(k.encode())
        h.update(str(a.dtype).encode())
        h.update(a.tobytes())
    return h.hexdigest()
