"""ctypes binding of libsaga_amd.so (declarations: include/saga_amd.h).

The library is built in-tree by ``python -m saga_amd.build``.  Loading fails
loudly when it is missing: there is no CPU or torch fallback for the decode
path.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsaga_amd.so")

DTYPE_F32, DTYPE_BF16, DTYPE_F16, DTYPE_BOOL, DTYPE_I32, DTYPE_I64 = range(6)
_TORCH_DTYPES = {
    torch.float32: DTYPE_F32,
    torch.bfloat16: DTYPE_BF16,
    torch.float16: DTYPE_F16,
    torch.bool: DTYPE_BOOL,
    torch.int32: DTYPE_I32,
    torch.int64: DTYPE_I64,
}

SAGA_OK = 0
ERRORS = {-1: "invalid argument", -2: "unsupported", -3: "workspace", -4: "HIP runtime"}


class SagaTensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("ndim", ctypes.c_int32),
        ("shape", ctypes.c_int64 * 4),
        ("stride", ctypes.c_int64 * 4),
    ]


class AtopnLayout(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in (
        "scores", "scores_ld", "part_max", "part_sum", "part_tail", "nparts", "thresh",
        "sel_idx", "sel_val", "sel_cnt", "sel_total", "nslice", "slice_cap", "slice_idx", "slice_val",
        "slice_cnt", "slice_pre", "slice_o", "slice_ml", "row_part", "row_cnt", "total_bytes")]


# Every symbol include/saga_amd.h declares, with its ctypes signature.
_P = ctypes.c_void_p
_T = ctypes.POINTER(SagaTensor)
_I64 = ctypes.c_int64
_SIGS = {
    "saga_version": (ctypes.c_int, []),
    "saga_last_error": (ctypes.c_char_p, []),
    "saga_qk_scores": (ctypes.c_int, [_T, _T, _T, _P, ctypes.c_float, _T, _P, _P, _P]),
    "saga_logit_threshold": (ctypes.c_int, [_T, _P, _P, _P, _P]),
    "saga_threshold_select": (ctypes.c_int, [_T, _P, _I64, _I64, _T, _P, _P, _P]),
    "saga_sparse_softmax_pv": (ctypes.c_int, [_T, _T, _T, ctypes.c_int32, _T, _P]),
    "saga_qk_nparts": (ctypes.c_int64, [_I64, _I64, _I64]),
    "saga_atopn_workspace_bytes": (ctypes.c_size_t, [_I64, _I64, _I64, _I64, _I64, _I64]),
    "saga_atopn_workspace_layout": (ctypes.c_int, [_I64, _I64, _I64, _I64, _I64, _I64,
                                                   ctypes.POINTER(AtopnLayout)]),
    "saga_atopn_decode": (ctypes.c_int, [_T, _T, _T, _T, _P, ctypes.c_float, _I64, _P, _T, _P, ctypes.c_size_t, _P]),
    "saga_atopn_decode_ex": (ctypes.c_int, [_T, _T, _T, _T, _P, ctypes.c_float, _I64, _P, _T, ctypes.c_int32, _P,
                                            ctypes.c_size_t, _P]),
    "saga_atopn_decode_noalloc": (ctypes.c_int, [_T, _T, _T, _T, _P, ctypes.c_float, _I64, _P, _T, _P]),
    "saga_atopn_calibrate": (ctypes.c_int, [_T, _T, _T, _T, _P, ctypes.c_float, _I64, _P, _T, _P, ctypes.c_size_t, _P]),
    "saga_atopn_calibrate_ex": (ctypes.c_int, [_T, _T, _T, _T, _P, ctypes.c_float, _I64, _P, _T, ctypes.c_int32, _P,
                                               ctypes.c_size_t, _P]),
    "saga_dense_workspace_bytes": (ctypes.c_size_t, [_I64, _I64, _I64, _I64]),
    "saga_dense_decode": (ctypes.c_int, [_T, _T, _T, _T, _P, ctypes.c_float, _T, _P, ctypes.c_size_t, _P]),
    "saga_rope_kv_append": (ctypes.c_int, [_T, _I64, _I64, _I64, ctypes.c_float, _P, _P, _T, _T, _T, _P]),
    "saga_rmsnorm": (ctypes.c_int, [_T, _T, ctypes.c_float, _T, _P]),
    "saga_silu_mul": (ctypes.c_int, [_T, _T, _P]),
    "saga_gemv_workspace_bytes": (ctypes.c_size_t, [_I64, _I64, _I64]),
    "saga_gemv": (ctypes.c_int, [_T, _T, _T, ctypes.c_float, ctypes.c_int32, _T, _P, ctypes.c_size_t, _P]),
    "saga_gemv_rope_kv": (ctypes.c_int, [_T, _T, _T, ctypes.c_float, _I64, _I64, _I64, ctypes.c_float, _P, _P,
                                         _T, _T, _T, _P, _P]),
    "saga_rope_table": (ctypes.c_int, [_P, _I64, _I64, ctypes.c_float, _P, _P]),
    "saga_embed_rope": (ctypes.c_int, [_P, _T, _T, _P, _I64, ctypes.c_float, _P, _P]),
    "saga_advance_positions": (ctypes.c_int, [_P, _P, _I64, _P]),
    "saga_argmax_workspace_bytes": (ctypes.c_size_t, [_I64, _I64]),
    "saga_argmax": (ctypes.c_int, [_T, _P, _P, ctypes.c_size_t, _P]),
    "saga_prefill_attention": (ctypes.c_int, [_T, _T, _T, _T, ctypes.c_float, ctypes.c_int32, ctypes.c_int64, _T, _P]),
}
GEMV_STORE, GEMV_ADD, GEMV_SILU_PAIRS = 0, 1, 2
K2_AUTO, K2_ROW_BLOCK, K2_SLICE_ROW = 0, 1, 2
NOALLOC_SCRATCH_BYTES = 64 << 20

_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Load libsaga_amd.so once and attach the declared signatures."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise ImportError(
                    f"{LIB_PATH} is not built; run `python -m saga_amd.build` "
                    "(the SAGA decode path has no CPU fallback)")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in _SIGS.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    if rc != SAGA_OK:
        msg = load().saga_last_error().decode(errors="replace")
        raise RuntimeError(f"saga_amd {what}: {ERRORS.get(rc, rc)}: {msg}")


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _TORCH_DTYPES[dt]
    except KeyError:
        raise TypeError(f"saga_amd: unsupported dtype {dt}") from None


def tensor(t: torch.Tensor | None):
    """saga_tensor descriptor of a torch tensor (None -> NULL)."""
    if t is None:
        return None
    if t.dim() > 4:
        raise ValueError("saga_amd: at most 4 dims")
    d = SagaTensor()
    d.data = t.data_ptr()
    d.dtype = dtype_code(t.dtype)
    d.ndim = max(t.dim(), 1)
    shape = list(t.shape) or [1]
    stride = list(t.stride()) or [1]
    for i in range(d.ndim):
        d.shape[i] = shape[i]
        d.stride[i] = stride[i]
    return ctypes.byref(d)


def ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def atopn_layout(b: int, q_h: int, k_h: int, L: int, d: int, buf_k: int) -> AtopnLayout:
    lay = AtopnLayout()
    check(load().saga_atopn_workspace_layout(b, q_h, k_h, L, d, buf_k, ctypes.byref(lay)), "workspace_layout")
    return lay
