"""SAGA attention module, MI355X build: the reference's attention/attention.py API.

Same public names, signatures, module globals and return conventions as the
reference (noamelata/SAGA, attention/attention.py), so its callers
(speedup.py, lm_eval_saga.py) import this module unchanged.  Decode calls
(l_q == 1) run the HIP kernels of libsaga_amd.so; prefill of bf16 / f16
operands with head_dim 64 / 128 runs the HIP prefill kernel on the
unexpanded caches, other prefill operands torch's
scaled_dot_product_attention, as in the reference (:13-53).

Deliberate differences from the reference (results otherwise agree with its
fp32 path within rounding):
  * scores, softmax and P.V accumulate in fp32 for bf16/f16 inputs (the
    reference rounds logits, exp-sums and probabilities to the input dtype);
  * the calibration threshold stored in AMORTIZED_THRESHOLD_TENSOR is the
    fp32 k-th largest probability (the reference stores the bf16-rounded one
    in bf16 runs);
  * Atop-N selection keeps the first buf_k passing positions in index order
    when more pass (the reference keeps a race-dependent subset);
  * full_einsum_forward with l_q > 1 runs the decode kernel once per batch
    row with that row's l_q queries as its batch (all keys visible, the mask
    added, is_causal ignored, as the reference's einsum does).
"""
import math
from typing import Optional, Tuple

import torch

from .. import _lib, ops
from .. import torch_ops  # noqa: F401  (registers torch.ops.saga.*)

_lib.load()  # fail at import when the HIP library is missing

# The decode entry points below call the kernels through torch.ops.saga.*
# (torch.library custom operators with fake implementations), so that
# torch.compile'd callers (speedup.py:502-508) trace them as graph nodes.
_saga = torch.ops.saga


def _expand_heads(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """[b, h, L, d] -> [b, h * n_rep, L, d]; head j of the result is head j // n_rep."""
    if n_rep == 1:
        return x
    b, h, L, d = x.shape
    return x[:, :, None, :, :].expand(b, h, n_rep, L, d).reshape(b, h * n_rep, L, d)


# =============================================================================
# Prefill (separate key / value head maps)
# =============================================================================

def sdpa_attention_forward(
        module: torch.nn.Module,
        query: torch.Tensor,
        key: torch.Tensor,
        value: torch.Tensor,
        attention_mask: Optional[torch.Tensor],
        dropout: float = 0.0,
        scaling: Optional[float] = None,
        is_causal: Optional[bool] = None,
        **kwargs,
) -> Tuple[torch.Tensor, None]:
    """attention/attention.py:13-53: attention over keys expanded by q_h / k_h
    and values by q_h / v_h (they differ in SAGA).  CUDA bf16 / f16 operands
    with d 64 / 128 run the HIP prefill kernel on the unexpanded caches
    (torch.ops.saga.prefill_attention); other operands keep the reference's
    expansion + torch SDPA.  Returns ([b, l_q, q_h, d] contiguous, None)."""
    mask = attention_mask
    if mask is not None:
        mask = mask[:, :, :, : key.shape[-2]]
    if is_causal is None:
        is_causal = query.shape[2] > 1 and mask is None
    if torch.jit.is_tracing() and isinstance(is_causal, torch.Tensor):
        is_causal = is_causal.item()
    expand = hasattr(module, "num_key_value_groups")
    same_heads = key.shape[-3] == query.shape[-3] and value.shape[-3] == query.shape[-3]
    if (expand or same_heads) and not (is_causal and mask is not None) \
            and ops.prefill_supported(query, key, value, mask, dropout, scaling):
        return _saga.prefill_attention(query, key, value, mask, scaling, bool(is_causal)), None
    if expand:
        n_q = query.shape[-3]
        key = _expand_heads(key, n_q // key.shape[-3])
        value = _expand_heads(value, n_q // value.shape[-3])
    out = torch.nn.functional.scaled_dot_product_attention(
        query.contiguous(), key.contiguous(), value.contiguous(),
        attn_mask=mask, dropout_p=dropout, scale=scaling, is_causal=is_causal)
    return out.transpose(1, 2).contiguous(), None


def register_sdpa():
    """attention/attention.py:56-57: install sdpa_attention_forward as
    transformers' "sdpa" attention implementation."""
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    ALL_ATTENTION_FUNCTIONS["sdpa"] = sdpa_attention_forward


# =============================================================================
# Dense decode attention
# =============================================================================

def full_einsum_forward(query, key, value, attention_mask=None, is_causal=False, scaling=None):
    """attention/attention.py:64-85: softmax(Q K^T * scaling + mask) V with
    separate key / value head grouping (query head h reads key head
    h // (q_h / k_h) and value head h // (q_h / v_h)), on the HIP split-L
    dense kernel.  Returns [b, q_h, l_q, d] in the input dtype.

    l_q > 1: every query attends to all l_kv keys (the reference adds only
    the mask, :75-77, and ignores is_causal).  Each batch row runs the
    kernel once with its l_q queries as the kernel's batch and the row's
    keys and values as stride-0 views (nothing is copied); the mask slice of
    the row is passed the same way."""
    b, q_h, l_q, d = query.shape
    if l_q == 1:
        return _saga.dense_decode(query, key, value, attention_mask, scaling)
    out = torch.empty(b, q_h, l_q, d, dtype=query.dtype, device=query.device)
    k_h, v_h = key.shape[1], value.shape[1]
    for i in range(b):
        qi = query[i].permute(1, 0, 2).unsqueeze(2)                     # [l_q, q_h, 1, d]
        ki = key[i:i + 1].expand(l_q, k_h, key.shape[2], d)             # stride 0 over the queries
        vi = value[i:i + 1].expand(l_q, v_h, value.shape[2], d)
        mi = None
        if attention_mask is not None:
            m = attention_mask[min(i, attention_mask.shape[0] - 1)]     # [1 | q_h, l_q, L']
            mi = m.permute(1, 0, 2).unsqueeze(2)                        # [l_q, 1 | q_h, 1, L']
        out[i] = ops.dense_decode(qi, ki, vi, mi, scaling)[:, :, 0].permute(1, 0, 2)
    return out


# =============================================================================
# Atop-N amortized attention
# =============================================================================

MAX_LAYERS = 128
AMORTIZED_THRESHOLD_TENSOR: Optional[torch.Tensor] = None
EXEMPT_LAYERS: set = set()


def init_amortized_threshold_tensor(device, num_layers, num_rows):
    """attention/attention.py:97-99: per-(layer, row) softmax-space thresholds,
    fp32 zeros, row r = batch * q_h + head."""
    global AMORTIZED_THRESHOLD_TENSOR
    AMORTIZED_THRESHOLD_TENSOR = torch.zeros(num_layers, num_rows, device=device, dtype=torch.float32)


def reset_amortized_state():
    """attention/attention.py:102-105."""
    if AMORTIZED_THRESHOLD_TENSOR is not None:
        AMORTIZED_THRESHOLD_TENSOR.zero_()


def _table_row(layer_idx: int, num_rows: int) -> torch.Tensor:
    if AMORTIZED_THRESHOLD_TENSOR is None:
        raise RuntimeError("AMORTIZED_THRESHOLD_TENSOR is not initialised; call init_amortized_threshold_tensor()")
    if AMORTIZED_THRESHOLD_TENSOR.shape[1] < num_rows:
        raise ValueError(f"threshold table has {AMORTIZED_THRESHOLD_TENSOR.shape[1]} rows, need {num_rows}")
    return AMORTIZED_THRESHOLD_TENSOR[layer_idx, :num_rows]


def _threshold_topk_triton(x: torch.Tensor, k: int, threshold: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """attention/attention.py:108-110 (name kept; HIP-backed)."""
    from .triton_atopn import threshold_topk_fast
    return threshold_topk_fast(x, k, threshold)


def _compute_attn_weights(query, key, scaling, attention_mask):
    """attention/attention.py:113-128 (fp32 scores, returned in the input dtype)."""
    return ops.qk_scores(query, key, attention_mask, scaling).to(query.dtype)


def _compute_attn_probs(query, key, scaling, attention_mask):
    """attention/attention.py:131-133."""
    return torch.nn.functional.softmax(_compute_attn_weights(query, key, scaling, attention_mask), dim=-1)


def _transform_softmax_threshold(attn_logits, softmax_threshold, tail_size=256):
    """attention/attention.py:136-149 (tail_size is fixed at 256 in the kernel)."""
    if tail_size != 256:
        raise NotImplementedError("the HIP threshold kernel uses the reference's tail of 256 positions")
    return ops.logit_threshold(attn_logits.to(torch.float32).contiguous(), softmax_threshold)


def _atopn_gather_and_output(attn_weights_topk, attn_indices, value, query_shape, top_n_attention,
                             input_is_logits=False):
    """attention/attention.py:152-170."""
    return ops.sparse_softmax_pv(attn_weights_topk, attn_indices, value, query_shape,
                                 input_is_logits=input_is_logits, out_dtype=value.dtype)


def approx_top_n_attention_amortized_cal(query, key, value, attention_mask=None, is_causal=False,
                                         top_n_attention: int = 256, scaling=None, layer_idx: int = 0):
    """attention/attention.py:173-189: calibration step.  Full softmax
    statistics, exact top-k (k = min(top_n_attention, L)), the k-th largest
    probability of every row stored in AMORTIZED_THRESHOLD_TENSOR[layer_idx],
    output = renormalised top-k probabilities . V."""
    b, q_h = query.shape[0], query.shape[1]
    row = _table_row(layer_idx, b * q_h)
    return _saga.atopn_calibrate(query, key, value, row, top_n_attention, attention_mask, scaling)


def approx_top_n_attention_amortized(query, key, value, attention_mask=None, is_causal=False,
                                     top_n_attention: int = 256, scaling=None, layer_idx: int = 0):
    """attention/attention.py:192-209: fast step.  Logit threshold from the
    stored softmax thresholds, ordered selection of the logits above it
    (at most 2 * top_n_attention), sparse softmax . V over those rows."""
    b, q_h = query.shape[0], query.shape[1]
    row = _table_row(layer_idx, b * q_h)
    return _saga.atopn_decode(query, key, value, row, top_n_attention, attention_mask, scaling)
