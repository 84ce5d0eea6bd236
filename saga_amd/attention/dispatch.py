"""Decode-time attention dispatch of the reference's drivers, on the HIP kernels.

The reference routes every attention call of a transformers model through a
function installed as ALL_ATTENTION_FUNCTIONS["sdpa"]:

  * speedup.py:43-85 (sdpa_attention_forward_dispatch): by ATTENTION_MODE
    ("vanilla" | "full" | "atopn"); in "atopn" a step counter kept at layer 0
    sends the first decode step after a prefill to the calibration path and
    later steps to the fast path; EXEMPT_LAYERS run dense attention; a
    prefill (l_q > 1) resets the counter and runs the base SDPA forward;
  * lm_eval_saga.py:152-214 (sdpa_attention_forward): the same with the
    threshold table created lazily at the first decode step, recalibration
    on the first step and every 32 steps after it, and a prefill resetting
    the threshold table as well.

Both policies live in SagaDispatcher; the module-level names mirror
speedup.py's globals and function so that its call sites read the same.
Decode calls return [b, 1, q_h, d] contiguous and None, as the reference's
(speedup.py:85).
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import attention as A

# lm_eval_saga.py:35-38: layers whose 256-position tail underestimates the
# row max (exp overflow -> inf threshold -> NaN output), run dense.
MODEL_EXEMPT_LAYERS = {
    "qwen2.5-1.5b": {0, 14},
    "llama-3.2-1b": {0},
}


def default_exempt_layers(model_name: str) -> set:
    """lm_eval_saga.py:35-38 lookup: substring match, case-insensitive."""
    name = model_name.lower()
    for key, layers in MODEL_EXEMPT_LAYERS.items():
        if key in name:
            return set(layers)
    return set()


class SagaDispatcher:
    """Callable with the transformers attention-function signature.

    policy="speedup": calibrate on the first decode step after a prefill
    (speedup.py:59-75).  policy="lm_eval": calibrate on the first step and
    every `recalibrate_every` steps after it, create the threshold table
    lazily, reset it on prefill (lm_eval_saga.py:165-212).
    mode: "vanilla" (base SDPA for every call), "full" (dense decode kernel)
    or "atopn".
    """

    def __init__(self, mode: str = "atopn", top_n: Optional[int] = 256, policy: str = "speedup",
                 recalibrate_every: int = 32):
        if mode not in ("vanilla", "full", "atopn"):
            raise ValueError(f"mode must be 'vanilla', 'full' or 'atopn', got {mode!r}")
        if policy not in ("speedup", "lm_eval"):
            raise ValueError(f"policy must be 'speedup' or 'lm_eval', got {policy!r}")
        self.mode, self.top_n, self.policy, self.recalibrate_every = mode, top_n, policy, recalibrate_every
        self.step = 0  # decode steps since the last prefill, counted at layer 0

    def _calibrate_now(self) -> bool:
        if self.policy == "speedup":
            return self.step <= 1
        return self.step <= 1 or self.step % self.recalibrate_every == 1

    def __call__(self, module, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                 attention_mask: Optional[torch.Tensor] = None, dropout: float = 0.0,
                 scaling: Optional[float] = None, is_causal: Optional[bool] = None,
                 **kwargs) -> Tuple[torch.Tensor, None]:
        layer_idx = getattr(module, "layer_idx", 0) if module is not None else 0
        l_q = query.shape[-2]
        mask = attention_mask
        if mask is not None:
            mask = mask[:, :, :, : key.shape[-2]].to(query.device)
        if l_q > 1 or self.mode == "vanilla":
            # prefill (or vanilla mode): base SDPA; a prefill restarts the step count
            if l_q > 1 and layer_idx == 0:
                self.step = 0
                if self.policy == "lm_eval" and self.mode == "atopn":
                    A.reset_amortized_state()
            return A.sdpa_attention_forward(module, query, key, value, attention_mask, dropout=dropout,
                                            scaling=scaling, is_causal=is_causal, **kwargs)
        if self.mode == "full":
            out = A.full_einsum_forward(query, key, value, mask, scaling=scaling)
        else:
            if layer_idx == 0:
                self.step += 1
                if self.policy == "lm_eval" and A.AMORTIZED_THRESHOLD_TENSOR is None:
                    A.init_amortized_threshold_tensor(query.device, A.MAX_LAYERS, query.shape[0] * query.shape[1])
            if layer_idx in A.EXEMPT_LAYERS:
                out = A.full_einsum_forward(query, key, value, mask, scaling=scaling)
            elif self._calibrate_now():
                out = A.approx_top_n_attention_amortized_cal(query, key, value, mask, scaling=scaling,
                                                             top_n_attention=self.top_n, layer_idx=layer_idx)
            else:
                out = A.approx_top_n_attention_amortized(query, key, value, mask, scaling=scaling,
                                                         top_n_attention=self.top_n, layer_idx=layer_idx)
        return out.transpose(1, 2).contiguous(), None

    def register(self) -> "SagaDispatcher":
        """Install as transformers' "sdpa" attention (speedup.py:497,
        lm_eval_saga.py:214)."""
        from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
        ALL_ATTENTION_FUNCTIONS["sdpa"] = self
        return self


# speedup.py:36-39 globals and :43-85 function, same names
TOP_N_ATTENTION = None
ATTENTION_MODE = "vanilla"
_DISPATCHER = SagaDispatcher(mode="vanilla", top_n=None, policy="speedup")


def sdpa_attention_forward_dispatch(module, query, key, value, attention_mask=None, dropout=0.0, scaling=None,
                                    is_causal=None, **kwargs) -> Tuple[torch.Tensor, None]:
    """speedup.py:43-85, reading this module's ATTENTION_MODE and
    TOP_N_ATTENTION at every call (the reference's drivers assign them)."""
    _DISPATCHER.mode = ATTENTION_MODE
    _DISPATCHER.top_n = TOP_N_ATTENTION
    return _DISPATCHER(module, query, key, value, attention_mask, dropout=dropout, scaling=scaling,
                       is_causal=is_causal, **kwargs)
