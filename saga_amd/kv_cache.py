"""KV-cache layout, allocation and capacity planning for SAGA decoders.

The reference keeps separate per-layer key and value caches, K [B, k_h, Lmax,
d] and V [B, v_h, Lmax, d] (speedup.py:119-139, the StaticCache layout of
transformers cache_utils.py:455-487), with k_h < v_h in SAGA models.  This
build keeps the same per-layer layout and stores all layers in one tensor per
kind: K [layers, B, k_h, Lmax, d] and V [layers, B, v_h, Lmax, d].
  * contiguous, so each layer's cache is a view in the reference layout (the
    kernels take it in place; a d = 128 bf16 row is 256 bytes);
  * each tensor starts 256-byte aligned (caching allocator blocks are);
  * one allocation per kind: the 28 layers of a 1.5B-shaped model at batch
    8 and 32k context are two tensors of 1.9 and 3.8 GB.

plan_capacity() answers how long a context, or how large a batch, fits on one
GPU next to the decode weights and workspaces: an MI355X has 288 GB of HBM3E.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

HBM_BYTES_MI355X = 288 * 10**9


def _es(dtype) -> int:
    return torch.tensor([], dtype=dtype).element_size()


def kv_cache_bytes(shape, batch: int, max_len: int, dtype=torch.bfloat16) -> int:
    """Bytes of the K and V caches of every layer."""
    return shape.layers * batch * (shape.n_k + shape.n_v) * max_len * shape.head_dim * _es(dtype)


def decode_weight_bytes(shape, dtype=torch.bfloat16, decode_copies: bool = True) -> int:
    """Weights of a decoder of this shape: embedding (tied LM head), per-layer
    q/k/v (+ bias), o, gate/up and down projections, norms.  decode_copies:
    plus the decode-layout copies the skinny GEMM reads (norm-folded q/k/v and
    gate/up, packed o and down, normed LM head)."""
    es = _es(dtype)
    s = shape
    per_layer = (s.qkv_width * s.hidden + s.qkv_width + s.hidden * s.n_q * s.head_dim + 2 * s.intermediate * s.hidden
                 + s.hidden * s.intermediate + 2 * s.hidden)
    base = (s.vocab * s.hidden + s.layers * per_layer + s.hidden) * es
    if not decode_copies:
        return base
    copies = (s.layers * (s.qkv_width * s.hidden + 2 * s.intermediate * s.hidden + s.hidden * s.n_q * s.head_dim
                          + s.hidden * s.intermediate) + s.vocab * s.hidden) * es
    return base + copies


def decode_workspace_bytes(shape, batch: int, max_len: int, top_n: int) -> int:
    """Atop-N and dense decode workspaces of one layer call (shared by all
    layers) plus the per-step activations and the threshold table."""
    from . import _lib
    lib = _lib.load()
    s = shape
    ws = lib.saga_atopn_workspace_bytes(batch, s.n_q, s.n_k, max_len, s.head_dim, min(2 * top_n, max_len))
    ws += lib.saga_dense_workspace_bytes(batch, s.n_q, max_len, s.head_dim)
    ws += lib.saga_gemv_workspace_bytes(batch, s.hidden, s.intermediate)
    ws += s.layers * batch * s.n_q * 4
    ws += batch * (3 * s.hidden + s.qkv_width + 2 * s.intermediate + s.vocab) * 2
    return int(ws)


@dataclass(frozen=True)
class CapacityPlan:
    batch: int
    max_len: int
    kv_bytes: int
    weight_bytes: int
    workspace_bytes: int
    budget_bytes: int

    @property
    def total_bytes(self) -> int:
        return self.kv_bytes + self.weight_bytes + self.workspace_bytes

    def __str__(self) -> str:
        g = 1e9
        return (f"batch {self.batch} x {self.max_len} positions: KV {self.kv_bytes / g:.1f} GB + weights "
                f"{self.weight_bytes / g:.1f} GB + workspaces {self.workspace_bytes / g:.2f} GB = "
                f"{self.total_bytes / g:.1f} of {self.budget_bytes / g:.0f} GB")


def plan_capacity(shape, batch: Optional[int] = None, max_len: Optional[int] = None, budget_bytes: Optional[int] = None,
                  reserve_fraction: float = 0.05, top_n: int = 512, dtype=torch.bfloat16,
                  align: int = 256) -> CapacityPlan:
    """The largest max_len for a given batch, or the largest batch for a given
    max_len (give exactly one), that fits budget_bytes (default: the current
    device's total memory, else 288 GB) minus reserve_fraction, next to the
    decode weights (with their decode copies) and workspaces.  max_len is
    rounded down to a multiple of `align` positions."""
    if (batch is None) == (max_len is None):
        raise ValueError("give exactly one of batch and max_len")
    if budget_bytes is None:
        budget_bytes = (torch.cuda.get_device_properties(0).total_memory if torch.cuda.is_available()
                        else HBM_BYTES_MI355X)
    avail = int(budget_bytes * (1 - reserve_fraction))
    wbytes = decode_weight_bytes(shape, dtype)

    def fits(b: int, L: int) -> Optional[CapacityPlan]:
        kv = kv_cache_bytes(shape, b, L, dtype)
        ws = decode_workspace_bytes(shape, b, L, top_n)
        if kv + wbytes + ws > avail:
            return None
        return CapacityPlan(b, L, kv, wbytes, ws, budget_bytes)

    best = None
    if batch is not None:
        lo, hi = 0, 1
        while fits(batch, hi * align) is not None and hi < (1 << 24):
            lo, hi = hi, hi * 2
        while hi - lo > 1:  # largest multiple of align that fits
            mid = (lo + hi) // 2
            if fits(batch, mid * align) is not None:
                lo = mid
            else:
                hi = mid
        best = fits(batch, lo * align) if lo > 0 else None
    else:
        lo, hi = 0, 1
        while fits(hi, max_len) is not None and hi < (1 << 20):
            lo, hi = hi, hi * 2
        while hi - lo > 1:
            mid = (lo + hi) // 2
            if fits(mid, max_len) is not None:
                lo = mid
            else:
                hi = mid
        best = fits(lo, max_len) if lo > 0 else None
    if best is None:
        raise MemoryError(f"nothing fits: weights alone are {wbytes / 1e9:.1f} GB of {avail / 1e9:.0f} GB")
    return best


class KVCache:
    """K [layers, B, k_h, Lmax, d] and V [layers, B, v_h, Lmax, d], zero-filled;
    layer(l) returns the reference-layout views (k [B, k_h, Lmax, d],
    v [B, v_h, Lmax, d])."""

    def __init__(self, shape, batch: int, max_len: int, device="cuda", dtype=torch.bfloat16,
                 check_free: bool = True):
        dev = torch.device(device)
        need = kv_cache_bytes(shape, batch, max_len, dtype)
        if check_free and dev.type == "cuda":
            free, _ = torch.cuda.mem_get_info(dev)
            if need > 0.8 * free:
                raise MemoryError(f"KV cache of {need / 2**30:.1f} GiB does not fit in {free / 2**30:.1f} GiB free "
                                  f"HBM (plan_capacity() gives the largest batch / context)")
        d = shape.head_dim
        self.k = torch.zeros(shape.layers, batch, shape.n_k, max_len, d, device=dev, dtype=dtype)
        self.v = torch.zeros(shape.layers, batch, shape.n_v, max_len, d, device=dev, dtype=dtype)
        self.batch, self.max_len = batch, max_len

    @property
    def nbytes(self) -> int:
        return self.k.numel() * self.k.element_size() + self.v.numel() * self.v.element_size()

    def layer(self, l: int):
        return self.k[l], self.v[l]
