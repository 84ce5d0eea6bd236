"""CPU oracle for the SAGA + Atop-N decode-attention path (numpy restatement).

TEST INFRASTRUCTURE ONLY.  This module is what the GPU results are checked
against: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The product path (``saga_amd``) never calls it and has no CPU
fallback.

Every function restates one function of the reference (noamelata/SAGA) and
cites the ``file:line`` it follows.  Arithmetic is done in the dtype of the
inputs: float32 inputs give the reference's fp32 path, float64 inputs give the
closed-form (exact-ish) variant used to pin the fp32 results.  bf16 data is
represented as float32 arrays holding bf16-rounded values (``round_bf16``), so
that "the reference fp32 path on the bf16 inputs" is simply the fp32 path.

Conventions shared with the reference:
  * query [b, q_h, l_q, d], key [b, k_h, L, d], value [b, v_h, L, d];
  * query head h reads key head h // (q_h // k_h) and value head
    h // (q_h // v_h) (attention/attention.py:70, 81, 119, 163);
  * rows of the threshold table are r = b_idx * q_h + h
    (attention/attention.py:184-187, 200-201).

How each function is pinned (tests/test_oracle.py):
  qk_scores          golden vectors from the reference + float64 closed form
  logit_threshold    golden vectors (exact fp32 t within 2 ulp) + the
                     identity {softmax(x) > p*} == {x > t} in float64
  threshold_select   golden index sets + brute-force loop + strict '>' cases
  gather_output      golden vectors + float64 per-head loops
  calibrate          golden vectors + brute-force sort / k-th order statistic
  fast               golden vectors (composition of the above)
  dense              golden vectors + torch scaled_dot_product_attention
  prefill            torch scaled_dot_product_attention on repeat_kv-expanded
                     heads (causal, bool and float masks) + causality and
                     single-key closed forms (no reference golden vectors
                     exist for the prefill path)
The only behaviour not pinned by the reference is the overflow rule of
threshold_select (more than k elements pass): the reference keeps a
race-dependent subset (attention/triton_atopn.py:47-53); this oracle and the
HIP kernels keep the first k in ascending index order.  torch.topk's order
among exactly equal probabilities is unspecified (attention/attention.py:182);
the oracle takes the lower index first.
"""
from __future__ import annotations

import math

import numpy as np

TAIL_SIZE = 256          # attention/attention.py:136 (tail_size=256)
PROB_CLAMP = 1e-30       # attention/attention.py:147
RENORM_CLAMP = 1e-12     # attention/attention.py:161
MAX_LAYERS = 128         # attention/attention.py:92


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16 (round-to-nearest-even), kept as float32."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    rounding = ((u >> 16) & 1) + 0x7FFF
    r = ((u + rounding) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32).copy()
    nan = np.isnan(a)
    out[nan] = np.nan
    return out.reshape(np.shape(x))


def _scale(query, scaling):
    return 1 / math.sqrt(query.shape[-1]) if scaling is None else scaling


def qk_scores(query, key, scaling=None, attention_mask=None):
    """Scaled (and masked) logits, attention/attention.py:113-128.

    Returns [b, q_h, l_q, L] in the input dtype.  A boolean mask is added as
    0/1 exactly as ``logits + bool_tensor`` does in torch (:124-126).
    """
    b, q_h, l_q, d = query.shape
    k_h, L = key.shape[1], key.shape[2]
    g = q_h // k_h
    dt = query.dtype
    qg = query.reshape(b, k_h, g * l_q, d)                          # :119
    w = np.matmul(qg, np.swapaxes(key, -1, -2))                    # :120-121
    w = w.reshape(b, q_h, l_q, L) * dt.type(_scale(query, scaling))  # :122
    if attention_mask is not None:                                 # :124-126
        m = np.asarray(attention_mask)[..., :L]
        w = w + m.astype(dt)
    return w


def softmax(x, axis=-1):
    """torch.nn.functional.softmax restated: exp(x - max) / sum."""
    with np.errstate(invalid="ignore", over="ignore"):
        m = np.max(x, axis=axis, keepdims=True)
        e = np.exp(x - m)
        return e / np.sum(e, axis=axis, keepdims=True)


def logit_threshold(attn_logits, softmax_threshold, tail_size=TAIL_SIZE):
    """Softmax-space -> logit-space threshold, attention/attention.py:136-149.

    t = m + log(max(p*, 1e-30) * sum_j exp(x_j - m)), m = max of the last
    min(tail_size, L) logits of the row.
    """
    nr = attn_logits.shape[0] * attn_logits.shape[1]
    L = attn_logits.shape[-1]
    x = attn_logits.reshape(nr, L)
    dt = x.dtype
    tail = min(tail_size, L)                                       # :142
    m = x[:, -tail:].max(axis=-1)                                  # :143
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        s = np.exp(x - m[:, None]).sum(axis=-1, dtype=dt)          # :145
        p = np.maximum(np.asarray(softmax_threshold, dtype=dt).reshape(-1), dt.type(PROB_CLAMP))
        return (m + np.log(p * s)).astype(dt)                      # :147


def _row_thresholds(threshold, n_rows):
    """Threshold broadcast rule of attention/triton_atopn.py:87-96."""
    t = np.asarray(threshold).reshape(-1)
    if t.size == n_rows:
        return t
    if t.size == 1:
        return np.repeat(t, n_rows)
    reps = (n_rows + t.size - 1) // t.size
    return np.tile(t, reps)[:n_rows]


def threshold_select(x, k, threshold):
    """Threshold stream compaction, attention/triton_atopn.py:59-113 (kernel :6-53).

    Per row: the elements with x > t (strict, compared in fp32, :42), capped at
    k.  Unfilled slots hold (-inf, 0) (:82-84).  Order: ascending index; on
    overflow the first k by index are kept (the reference keeps a
    race-dependent subset there).  Returns (values [..., k] in x's dtype,
    indices [..., k] int64, per-row count of passing elements before the cap).
    """
    shape = x.shape
    D = shape[-1]
    x2 = x.reshape(-1, D)
    n = x2.shape[0]
    cmp_dt = np.float64 if x.dtype == np.float64 else np.float32
    t = _row_thresholds(threshold, n).astype(cmp_dt)
    vals = np.full((n, k), -np.inf, dtype=x.dtype)
    idx = np.zeros((n, k), dtype=np.int64)
    counts = np.zeros(n, dtype=np.int64)
    for r in range(n):
        with np.errstate(invalid="ignore"):
            sel = np.nonzero(x2[r].astype(cmp_dt) > t[r])[0]
        counts[r] = sel.size
        keep = sel[:k]
        vals[r, :keep.size] = x2[r, keep]
        idx[r, :keep.size] = keep
    return vals.reshape(shape[:-1] + (k,)), idx.reshape(shape[:-1] + (k,)), counts


def _value_rows(value, q_h, idx):
    """Gather V rows per query head: head h reads value head h // (q_h // v_h).

    attention/attention.py:163-164 (expand over the value group + gather).
    """
    b, v_h = value.shape[0], value.shape[1]
    g_v = q_h // v_h
    vh = np.arange(q_h) // g_v
    bi = np.arange(b)[:, None, None]
    return value[bi, vh[None, :, None], idx]                      # [b, q_h, K, d]


def gather_output(attn_weights_topk, attn_indices, value, query_shape, input_is_logits=False):
    """Sparse softmax . V over the selected rows, attention/attention.py:152-170.

    input_is_logits: softmax over the K-wide buffer (-inf padding -> weight 0,
    an all -inf row -> NaN, :158-159); otherwise renormalise probabilities with
    a 1e-12 floor on the sum (:160-161).
    """
    b, q_h, l_q, d = query_shape
    assert l_q == 1, "decode path: l_q == 1"
    w = attn_weights_topk.reshape(b, q_h, -1)
    K = w.shape[-1]
    dt = np.result_type(w.dtype, value.dtype)
    if input_is_logits:
        p = softmax(w.astype(dt), axis=-1)
    else:
        p = w.astype(dt) / np.maximum(w.sum(axis=-1, keepdims=True, dtype=dt), dt.type(RENORM_CLAMP))
    idx = attn_indices.reshape(b, q_h, K)
    rows = _value_rows(value.astype(dt), q_h, idx)
    out = np.matmul(p[:, :, None, :], rows)                       # :166-168
    return out.reshape(b, q_h, 1, d)


def topk_desc(x, k):
    """Top-k along the last axis, descending; equal values: lower index first."""
    order = np.argsort(-x, axis=-1, kind="stable")[..., :k]
    return np.take_along_axis(x, order, axis=-1), order


def calibrate(query, key, value, attention_mask=None, top_n=256, scaling=None):
    """Calibration step, attention/attention.py:173-189.

    Full softmax, top-k (k = min(top_n, L)), threshold = k-th largest
    probability per row (stored by the reference in
    AMORTIZED_THRESHOLD_TENSOR[layer, :b*q_h]), output = renormalised top-k . V.
    Returns (out [b, q_h, 1, d], threshold [b*q_h], top-k indices [b, q_h, 1, k]).
    """
    b, q_h, l_q, d = query.shape
    L = key.shape[2]
    probs = softmax(qk_scores(query, key, scaling, attention_mask), axis=-1)  # :179
    k = min(top_n, L)                                               # :181
    pk, ik = topk_desc(probs, k)                                    # :182
    thr = pk[:, :, 0, -1].reshape(b * q_h)                          # :184-185
    out = gather_output(pk, ik, value, query.shape, input_is_logits=False)  # :189
    return out, thr, ik


def fast(query, key, value, softmax_threshold, attention_mask=None, top_n=256, scaling=None):
    """Amortized fast step, attention/attention.py:192-209.

    Returns (out [b, q_h, 1, d], logit thresholds [b*q_h], selected indices
    [b, q_h, 1, buf_k], counts [b*q_h]) with buf_k = min(2*top_n, L).
    """
    L = key.shape[2]
    logits = qk_scores(query, key, scaling, attention_mask)        # :198
    t = logit_threshold(logits, softmax_threshold)                  # :203
    buf_k = min(top_n * 2, L)                                       # :205
    vals, idx, counts = threshold_select(logits, buf_k, t)          # :206
    out = gather_output(vals, idx, value, query.shape, input_is_logits=True)  # :208
    return out, t, idx, counts


def dense(query, key, value, attention_mask=None, scaling=None):
    """Dense decode attention, attention/attention.py:64-85 (full_einsum_forward)."""
    b, q_h, l_q, d = query.shape
    v_h, L = value.shape[1], value.shape[2]
    p = softmax(qk_scores(query, key, scaling, attention_mask), axis=-1)       # :79
    pv = p.reshape(b, v_h, (q_h // v_h) * l_q, L)                   # :81
    out = np.matmul(pv, value.astype(p.dtype))                      # :82-83
    return out.reshape(b, q_h, l_q, d)


def prefill(query, key, value, attention_mask=None, scaling=None, is_causal=None):
    """Prefill attention, attention/attention.py:13-53 (sdpa_attention_forward).

    Keys and values are expanded to the query heads by repeat_kv (:24-26:
    query head h reads key head h // (q_h // k_h), value head
    h // (q_h // v_h)); the mask is cut to the key length (:28-30); with
    is_causal None the call is causal iff l_q > 1 and there is no mask
    (:36-37; SDPA's causal mask is top-left: key j <= query i); then SDPA
    (:42-50): softmax(q k^T * scale + mask) v, a bool mask keeping True
    entries.  A query that sees no key gives 0 (torch's math path).
    Returns [b, l_q, q_h, d] (:51, transpose(1, 2))."""
    q = np.asarray(query)
    dt = np.result_type(q.dtype, np.float32)
    q = q.astype(dt)
    b, q_h, l_q, d = q.shape
    k = np.repeat(np.asarray(key, dtype=dt), q_h // key.shape[1], axis=1)      # :24
    v = np.repeat(np.asarray(value, dtype=dt), q_h // value.shape[1], axis=1)  # :25
    L = k.shape[2]
    mask = None if attention_mask is None else np.asarray(attention_mask)[:, :, :, :L]  # :28-30
    if is_causal is None:
        is_causal = l_q > 1 and mask is None                        # :36-37
    x = np.matmul(q, np.swapaxes(k, -1, -2)) * dt.type(_scale(q, scaling))
    if mask is not None:
        x = np.where(mask, x, -np.inf) if mask.dtype == np.bool_ else x + mask.astype(dt)
    if is_causal:
        x = np.where(np.arange(L)[None, :] <= np.arange(l_q)[:, None], x, -np.inf)
    m = x.max(axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0)
    e = np.exp(x - m)
    ssum = e.sum(axis=-1, keepdims=True)
    out = np.matmul(e / np.where(ssum > 0, ssum, 1), v)            # :42-50
    return np.ascontiguousarray(np.swapaxes(out, 1, 2))             # :51


def truncate_kv(key, value, kv_len):
    """Per-batch views key[i, :, :kv_len[i]] used to define the kv_len extension.

    The HIP entry points accept an optional per-batch valid length; its meaning
    is "the reference applied to the key/value truncated to that length".
    """
    return [(key[i:i + 1, :, :int(n)], value[i:i + 1, :, :int(n)]) for i, n in enumerate(kv_len)]


# --------------------------------------------------------------------------
# Decode-step ops around the attention path.  Their reference is the model
# the reference benchmarks (transformers Qwen2, installed version 5.15.0; the
# reference pins 5.3.0, which is not in this container):
#   TF = transformers/models/qwen2/modeling_qwen2.py
# Pinned in tests/test_oracle.py by brute-force loops and identities.

def rope_inv_freq(d, theta):
    """TF:86 inv_freq = 1 / theta^(arange(0, d, 2) / d), computed in fp32."""
    return (1.0 / (np.float32(theta) ** (np.arange(0, d, 2, dtype=np.float32) / np.float32(d)))).astype(np.float32)


def rope(x, pos, theta):
    """TF:97-120 rotate-half RoPE of x [..., d] at integer positions pos
    (broadcast over the leading dims): x*cos + rotate_half(x)*sin with
    cos/sin of cat(freqs, freqs), freqs = pos * inv_freq (fp32)."""
    d = x.shape[-1]
    ang = np.asarray(pos, dtype=np.float32)[..., None] * rope_inv_freq(d, theta)
    c, s = np.cos(ang.astype(np.float64)), np.sin(ang.astype(np.float64))
    x1, x2 = x[..., : d // 2].astype(np.float64), x[..., d // 2:].astype(np.float64)
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1)


def rmsnorm(x, w, eps):
    """TF:247-253 w * x / sqrt(mean(x^2) + eps) over the last axis (float64)."""
    x = np.asarray(x, dtype=np.float64)
    return np.asarray(w, dtype=np.float64) * (x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps))


def silu_mul(gate_up):
    """TF:46-47 act_fn(gate) * up with act = silu, gate_up = [gate | up]."""
    g = np.asarray(gate_up, dtype=np.float64)
    h = g.shape[-1] // 2
    gate, up = g[..., :h], g[..., h:]
    return gate / (1.0 + np.exp(-gate)) * up
