"""Threshold selection, MI355X build of the reference's attention/triton_atopn.py.

The module name is kept so that callers importing ``attention.triton_atopn``
(speedup.py clears ``_BUFFER_CACHE``) run unchanged; there is no Triton here.
``threshold_topk_fast`` runs the HIP ordered-compaction kernel
(saga_threshold_select in libsaga_amd.so).
"""
import torch

from .. import ops

# (rows, k, device, dtype) -> (values, int64 indices), reused across calls so
# that the call is capturable in a HIP graph after the first one
# (attention/triton_atopn.py:56, 73-81).
_BUFFER_CACHE = {}


def threshold_topk_fast(
    x: torch.Tensor,
    k: int,
    threshold: torch.Tensor,
    block_size: int = 1024,
) -> tuple[torch.Tensor, torch.Tensor]:
    """attention/triton_atopn.py:59-113.

    Per row of x [..., D]: the elements with x > threshold (strict, compared
    in fp32), at most k, in ascending index order; unfilled slots are
    (-inf, 0).  threshold: one value per row, a single value, or a shorter
    vector repeated over the rows.  Returns views of cached buffers
    (values in x's dtype, int64 indices), shape x.shape[:-1] + (k,), which
    the next call with the same shape overwrites -- as in the reference.
    block_size is accepted for signature compatibility; the HIP kernel tiles
    each row itself.
    """
    D = x.shape[-1]
    rows = x.numel() // D
    key = (rows, k, x.device, x.dtype)
    if key not in _BUFFER_CACHE:
        _BUFFER_CACHE[key] = (
            torch.empty(rows, k, device=x.device, dtype=x.dtype),
            torch.empty(rows, k, device=x.device, dtype=torch.int64),
        )
    out_values, out_indices = _BUFFER_CACHE[key]
    return ops.threshold_select(x, k, threshold, out_values=out_values, out_indices=out_indices)
