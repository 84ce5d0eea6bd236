"""torch.library operators for the decode attention kernels.

The reference compiles its decode step with torch.compile (speedup.py:502-508,
620-622).  A Python call into the C ABI (ctypes) cannot be traced, so each
kernel entry point is registered as a custom operator with a fake
(meta) implementation: torch.compile then records one graph node per call
instead of breaking the graph, and functionalisation sees that the
calibration step writes its threshold row.

Operators (namespace "saga"):
  * atopn_decode(query, key, value, softmax_threshold, top_n, attention_mask,
    scaling, kv_len) -> out [b, q_h, 1, d]        (attention/attention.py:192-209)
  * atopn_calibrate(query, key, value, threshold_out!, top_n, attention_mask,
    scaling, kv_len) -> out [b, q_h, 1, d]        (attention/attention.py:173-189)
  * dense_decode(query, key, value, attention_mask, scaling, kv_len)
    -> out [b, q_h, 1, d]                         (attention/attention.py:64-85)
  * prefill_attention(query, key, value, attention_mask, scaling, is_causal)
    -> out [b, l_q, q_h, d]                       (attention/attention.py:13-53)
"""
from typing import Optional

import torch

from . import ops


def _out_like(query: torch.Tensor) -> torch.Tensor:
    b, q_h, _, d = query.shape
    return query.new_empty(b, q_h, 1, d)


@torch.library.custom_op("saga::atopn_decode", mutates_args=())
def atopn_decode(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, softmax_threshold: torch.Tensor,
                 top_n: int, attention_mask: Optional[torch.Tensor] = None, scaling: Optional[float] = None,
                 kv_len: Optional[torch.Tensor] = None) -> torch.Tensor:
    return ops.atopn_decode(query, key, value, softmax_threshold, top_n, attention_mask, scaling, kv_len=kv_len)


@atopn_decode.register_fake
def _atopn_decode_fake(query, key, value, softmax_threshold, top_n, attention_mask=None, scaling=None,
                       kv_len=None):
    return _out_like(query)


@torch.library.custom_op("saga::atopn_calibrate", mutates_args=("threshold_out",))
def atopn_calibrate(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, threshold_out: torch.Tensor,
                    top_n: int, attention_mask: Optional[torch.Tensor] = None, scaling: Optional[float] = None,
                    kv_len: Optional[torch.Tensor] = None) -> torch.Tensor:
    return ops.atopn_calibrate(query, key, value, top_n, threshold_out, attention_mask, scaling, kv_len=kv_len)


@atopn_calibrate.register_fake
def _atopn_calibrate_fake(query, key, value, threshold_out, top_n, attention_mask=None, scaling=None,
                          kv_len=None):
    return _out_like(query)


@torch.library.custom_op("saga::dense_decode", mutates_args=())
def dense_decode(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                 attention_mask: Optional[torch.Tensor] = None, scaling: Optional[float] = None,
                 kv_len: Optional[torch.Tensor] = None) -> torch.Tensor:
    return ops.dense_decode(query, key, value, attention_mask, scaling, kv_len=kv_len)


@dense_decode.register_fake
def _dense_decode_fake(query, key, value, attention_mask=None, scaling=None, kv_len=None):
    return _out_like(query)


@torch.library.custom_op("saga::prefill_attention", mutates_args=())
def prefill_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                      attention_mask: Optional[torch.Tensor] = None, scaling: Optional[float] = None,
                      is_causal: bool = False) -> torch.Tensor:
    return ops.prefill_attention(query, key, value, attention_mask, scaling, is_causal)


@prefill_attention.register_fake
def _prefill_attention_fake(query, key, value, attention_mask=None, scaling=None, is_causal=False):
    b, q_h, l_q, d = query.shape
    return query.new_empty(b, l_q, q_h, d)
