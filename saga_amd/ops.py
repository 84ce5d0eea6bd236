"""Tensor-level operations of the SAGA + Atop-N decode path on MI355X.

Each function validates torch tensors, makes sure they live on a ROCm device,
and calls one C-ABI entry point of libsaga_amd.so on the current stream.
Nothing here computes on the CPU.

Workspaces: a caller may pass its own (`workspace=`, a uint8 device tensor of
at least the entry point's *_workspace_bytes); otherwise one is taken from a
cache keyed by (device, stream, kind), grown when needed and reused (the
counterpart of the reference's _BUFFER_CACHE, attention/triton_atopn.py:56,
73-84), so calls are capturable in a HIP graph after a warm-up call on the
same stream.  Calls on different streams never share a cached workspace.  A
cached workspace grows by at least half its size when a call needs more, so
a need that grows step by step (a decode whose cache length grows with every
token) reallocates a logarithmic number of times.  A replaced workspace that
was handed out during a graph capture is kept alive until clear_workspaces(),
because the graph still holds its address; any other is freed at once.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

from . import _lib

_WORKSPACES: dict = {}  # (device, stream handle, kind) -> uint8 tensor
_CAPTURED: set = set()  # keys whose current workspace was handed out during a graph capture
_RETIRED: list = []     # replaced workspaces that a captured graph may use, alive until clear_workspaces()


def _need_gpu(*ts: Optional[torch.Tensor]) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                f"saga_amd: tensors must be on a ROCm GPU (got {t.device}); the decode path has no CPU fallback")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"saga_amd: tensors on different devices ({dev}, {t.device})")
    return dev


def _device(device) -> torch.device:
    dev = torch.device(device)
    if dev.type == "cuda" and dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    return dev


def grown_size(old: int, need: int) -> int:
    """Bytes of a cached workspace replacing one of `old` bytes for a call
    needing `need`: at least 1.5x the old size, so that a need growing in
    small steps replaces the workspace O(log(final / first)) times."""
    return max(int(need), old + old // 2, 256)


def _replace(key, ws: Optional[torch.Tensor], need: int, alloc) -> torch.Tensor:
    """The cache's policy, without the device: a replaced workspace is kept
    (in _RETIRED) only if it was handed out while a graph was being captured."""
    if ws is not None and key in _CAPTURED:
        _RETIRED.append(ws)
    _CAPTURED.discard(key)
    new = alloc(grown_size(0 if ws is None else ws.numel(), need))
    _WORKSPACES[key] = new
    return new


def workspace(device: torch.device, kind: str, nbytes: int, stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
    """uint8 workspace of at least nbytes for calls on `stream` (default: the
    device's current stream), cached per (device, stream, kind).  A cached
    workspace too small for a call is replaced by one at least 1.5x larger;
    the old one stays allocated until clear_workspaces() if a graph was
    captured while it was handed out, else it is freed."""
    dev = _device(device)
    if stream is None:
        stream = torch.cuda.current_stream(dev)
    key = (dev, stream.cuda_stream, kind)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = _replace(key, ws, nbytes, lambda n: torch.empty(n, dtype=torch.uint8, device=dev))
    if torch.cuda.is_current_stream_capturing():
        _CAPTURED.add(key)
    return ws


def clear_workspaces() -> None:
    """Free every cached workspace (speedup.py:427-428 clears the reference's
    _BUFFER_CACHE between configurations).  A HIP graph captured with cached
    workspaces must not be replayed afterwards."""
    _WORKSPACES.clear()
    _CAPTURED.clear()
    _RETIRED.clear()


def _take_workspace(given: Optional[torch.Tensor], device, kind: str, nbytes: int) -> torch.Tensor:
    if given is None:
        return workspace(device, kind, nbytes)
    if given.device != device or given.dtype != torch.uint8 or not given.is_contiguous() or given.numel() < nbytes:
        raise ValueError(f"saga_amd: {kind} workspace must be a contiguous uint8 tensor of >= {nbytes} bytes "
                         f"on {device}")
    return given


def _scale(query: torch.Tensor, scaling: Optional[float]) -> float:
    # attention/attention.py:117
    return 1 / math.sqrt(query.size(-1)) if scaling is None else float(scaling)


def _vec_ready(t: torch.Tensor) -> torch.Tensor:
    """Rows must have a unit innermost stride and 16-byte aligned strides."""
    es = t.element_size()
    ok = t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all(
        (s * es) % 16 == 0 for s, n in zip(t.stride()[:-1], t.shape[:-1]) if n > 1)
    return t if ok else t.contiguous()


def _mask_view(mask: Optional[torch.Tensor], L: int) -> Optional[torch.Tensor]:
    if mask is None:
        return None
    if mask.dim() != 4:
        raise ValueError(f"saga_amd: attention mask must be 4-D [b, 1|q_h, 1, L'], got {tuple(mask.shape)}")
    return mask[:, :, :, :L]


def _kv_len(kv_len: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    if kv_len is None:
        return None
    if kv_len.dtype != torch.int32 or not kv_len.is_contiguous():
        raise ValueError("saga_amd: kv_len must be a contiguous int32 tensor [b]")
    return kv_len


def qk_scores(query, key, attention_mask=None, scaling=None, kv_len=None, with_partials=False):
    """Scaled, masked logits [b, q_h, 1, L] in fp32 (attention/attention.py:113-128).

    with_partials: also return the max and sum of exp(x - max) of each part
    of the row [b*q_h, saga_qk_nparts(b, k_h, L)]: part c covers the 16-position
    tiles [c*T/P, (c+1)*T/P), T = ceil(L/16), P parts (possibly none).
    """
    dev = _need_gpu(query, key, attention_mask, kv_len)
    lib = _lib.load()
    query, key = _vec_ready(query), _vec_ready(key)
    b, q_h, _, _ = query.shape
    L = key.shape[2]
    mask = _mask_view(attention_mask, L)
    # rows padded to 16 bytes (the kernel's vector stores), returned as a view
    scores = torch.empty(b, q_h, 1, (L + 3) // 4 * 4, dtype=torch.float32, device=dev)[..., :L]
    pm = ps = None
    if with_partials:
        nparts = lib.saga_qk_nparts(b, key.shape[1], L)
        pm = torch.empty(b * q_h, nparts, dtype=torch.float32, device=dev)
        ps = torch.empty_like(pm)
    _lib.check(lib.saga_qk_scores(_lib.tensor(query), _lib.tensor(key), _lib.tensor(mask), _lib.ptr(_kv_len(kv_len)),
                                  _scale(query, scaling), _lib.tensor(scores), _lib.ptr(pm), _lib.ptr(ps),
                                  _lib.stream_of(query)), "qk_scores")
    return (scores, pm, ps) if with_partials else scores


def logit_threshold(scores, softmax_threshold, kv_len=None):
    """Logit-space threshold per row (attention/attention.py:136-149)."""
    dev = _need_gpu(scores, softmax_threshold, kv_len)
    b, q_h = scores.shape[0], scores.shape[1]
    pstar = softmax_threshold.reshape(-1).to(torch.float32).contiguous()
    if pstar.numel() != b * q_h:
        raise ValueError("saga_amd: softmax_threshold must have b*q_h entries")
    out = torch.empty(b * q_h, dtype=torch.float32, device=dev)
    _lib.check(_lib.load().saga_logit_threshold(_lib.tensor(scores), _lib.ptr(_kv_len(kv_len)), _lib.ptr(pstar),
                                                _lib.ptr(out), _lib.stream_of(scores)), "logit_threshold")
    return out


def threshold_select(x, k, threshold, out_values=None, out_indices=None, with_counts=False):
    """Ordered threshold compaction (attention/triton_atopn.py:59-113).

    Returns (values [..., k] in x's dtype, int64 indices [..., k]) and, with
    with_counts, the per-row number of passing elements before the cap.
    """
    dev = _need_gpu(x, threshold)
    D = x.shape[-1]
    xf = x.reshape(-1, D).contiguous()
    rows = xf.shape[0]
    thr = threshold.reshape(-1).to(torch.float32).contiguous()
    if out_values is None:
        out_values = torch.empty(rows, k, dtype=x.dtype, device=dev)
    if out_indices is None:
        out_indices = torch.empty(rows, k, dtype=torch.int64, device=dev)
    counts = torch.empty(rows, dtype=torch.int32, device=dev) if with_counts else None
    _lib.check(_lib.load().saga_threshold_select(_lib.tensor(xf), _lib.ptr(thr), thr.numel(), k,
                                                 _lib.tensor(out_values), _lib.ptr(out_indices), _lib.ptr(counts),
                                                 _lib.stream_of(x)), "threshold_select")
    shape = tuple(x.shape[:-1]) + (k,)
    vals, idx = out_values.reshape(shape), out_indices.reshape(shape)
    return (vals, idx, counts) if with_counts else (vals, idx)


def sparse_softmax_pv(weights, indices, value, query_shape, input_is_logits=False, out_dtype=None):
    """Softmax / renormalisation over K selected entries, then . V
    (attention/attention.py:152-170).  Returns [b, q_h, 1, d]."""
    dev = _need_gpu(weights, indices, value)
    b, q_h, l_q, d = query_shape
    if l_q != 1:
        raise NotImplementedError("saga_amd: sparse softmax.V is the decode path (l_q == 1)")
    K = weights.shape[-1]
    w = weights.reshape(b, q_h, 1, K).contiguous()
    idx = indices.reshape(b, q_h, 1, K).contiguous()
    value = _vec_ready(value)
    out = torch.empty(b, q_h, 1, d, dtype=out_dtype or value.dtype, device=dev)
    _lib.check(_lib.load().saga_sparse_softmax_pv(_lib.tensor(w), _lib.tensor(idx), _lib.tensor(value),
                                                  1 if input_is_logits else 0, _lib.tensor(out),
                                                  _lib.stream_of(value)), "sparse_softmax_pv")
    return out


def _decode_prep(query, key, value, attention_mask, kv_len):
    dev = _need_gpu(query, key, value, attention_mask, kv_len)
    query, key, value = _vec_ready(query), _vec_ready(key), _vec_ready(value)
    if query.shape[2] != 1:
        raise NotImplementedError("saga_amd: the HIP decode kernels take l_q == 1")
    return dev, query, key, value, _mask_view(attention_mask, key.shape[2])


def atopn_workspace_bytes(b: int, q_h: int, k_h: int, L: int, d: int, top_n: int, calibrate: bool = False) -> int:
    """Bytes of the workspace of one fast step (or calibration step) call."""
    buf_k = min(top_n, L) if calibrate else min(2 * top_n, L)
    return int(_lib.load().saga_atopn_workspace_bytes(b, q_h, k_h, L, d, buf_k))


def atopn_decode(query, key, value, softmax_threshold, top_n, attention_mask=None, scaling=None, kv_len=None,
                 out=None, out_dtype=None, workspace=None, k2_variant=_lib.K2_AUTO):
    """Atop-N fast step (attention/attention.py:192-209).

    softmax_threshold: fp32 [b*q_h] (a row of the threshold table).
    k2_variant: the kernels of the selection + softmax.V (results are
    identical in every variant; see saga_atopn_decode_ex)."""
    dev, query, key, value, mask = _decode_prep(query, key, value, attention_mask, kv_len)
    b, q_h, _, d = query.shape
    L = key.shape[2]
    if softmax_threshold.dtype != torch.float32 or not softmax_threshold.is_contiguous() \
            or softmax_threshold.numel() < b * q_h:
        raise ValueError("saga_amd: softmax_threshold must be contiguous fp32 with b*q_h entries")
    if out is None:
        out = torch.empty(b, q_h, 1, d, dtype=out_dtype or query.dtype, device=dev)
    lib = _lib.load()
    ws = _take_workspace(workspace, dev, "atopn", atopn_workspace_bytes(b, q_h, key.shape[1], L, d, top_n))
    _lib.check(lib.saga_atopn_decode_ex(_lib.tensor(query), _lib.tensor(key), _lib.tensor(value), _lib.tensor(mask),
                                        _lib.ptr(_kv_len(kv_len)), _scale(query, scaling), int(top_n),
                                        _lib.ptr(softmax_threshold), _lib.tensor(out), int(k2_variant), _lib.ptr(ws),
                                        ws.numel(), _lib.stream_of(query)), "atopn_decode")
    return out


def atopn_decode_noalloc(query, key, value, softmax_threshold, top_n, attention_mask=None, scaling=None, kv_len=None,
                         out=None):
    """atopn_decode on the library's static per-GPU scratch
    (saga_atopn_decode_noalloc): no workspace is allocated or passed, so the
    call allocates nothing when `out` is given.  Calls that may overlap on
    one GPU race on that scratch; shapes whose workspace exceeds it raise."""
    dev, query, key, value, mask = _decode_prep(query, key, value, attention_mask, kv_len)
    b, q_h, _, d = query.shape
    if softmax_threshold.dtype != torch.float32 or not softmax_threshold.is_contiguous() \
            or softmax_threshold.numel() < b * q_h:
        raise ValueError("saga_amd: softmax_threshold must be contiguous fp32 with b*q_h entries")
    if out is None:
        out = torch.empty(b, q_h, 1, d, dtype=query.dtype, device=dev)
    _lib.check(_lib.load().saga_atopn_decode_noalloc(
        _lib.tensor(query), _lib.tensor(key), _lib.tensor(value), _lib.tensor(mask), _lib.ptr(_kv_len(kv_len)),
        _scale(query, scaling), int(top_n), _lib.ptr(softmax_threshold), _lib.tensor(out), _lib.stream_of(query)),
        "atopn_decode_noalloc")
    return out


def atopn_calibrate(query, key, value, top_n, threshold_out, attention_mask=None, scaling=None, kv_len=None,
                    out=None, out_dtype=None, workspace=None, k2_variant=_lib.K2_AUTO):
    """Atop-N calibration step (attention/attention.py:173-189).

    threshold_out: fp32 [b*q_h], receives the k-th largest probability per row.
    k2_variant: one block per row, or chunk kernel + row kernel (the same
    list and p* in every variant; see saga_atopn_calibrate_ex).
    """
    dev, query, key, value, mask = _decode_prep(query, key, value, attention_mask, kv_len)
    b, q_h, _, d = query.shape
    L = key.shape[2]
    if threshold_out.dtype != torch.float32 or not threshold_out.is_contiguous() or threshold_out.numel() < b * q_h:
        raise ValueError("saga_amd: threshold_out must be contiguous fp32 with b*q_h entries")
    if out is None:
        out = torch.empty(b, q_h, 1, d, dtype=out_dtype or query.dtype, device=dev)
    lib = _lib.load()
    ws = _take_workspace(workspace, dev, "atopn", atopn_workspace_bytes(b, q_h, key.shape[1], L, d, top_n, True))
    _lib.check(lib.saga_atopn_calibrate_ex(_lib.tensor(query), _lib.tensor(key), _lib.tensor(value),
                                           _lib.tensor(mask), _lib.ptr(_kv_len(kv_len)), _scale(query, scaling),
                                           int(top_n), _lib.ptr(threshold_out), _lib.tensor(out), int(k2_variant),
                                           _lib.ptr(ws), ws.numel(), _lib.stream_of(query)), "atopn_calibrate")
    return out


def dense_decode(query, key, value, attention_mask=None, scaling=None, kv_len=None, out=None, out_dtype=None,
                 workspace=None):
    """Dense decode attention (attention/attention.py:64-85, l_q == 1)."""
    dev, query, key, value, mask = _decode_prep(query, key, value, attention_mask, kv_len)
    b, q_h, _, d = query.shape
    L = key.shape[2]
    if out is None:
        out = torch.empty(b, q_h, 1, d, dtype=out_dtype or query.dtype, device=dev)
    lib = _lib.load()
    ws = _take_workspace(workspace, dev, "dense", lib.saga_dense_workspace_bytes(b, q_h, L, d))
    _lib.check(lib.saga_dense_decode(_lib.tensor(query), _lib.tensor(key), _lib.tensor(value), _lib.tensor(mask),
                                     _lib.ptr(_kv_len(kv_len)), _scale(query, scaling), _lib.tensor(out),
                                     _lib.ptr(ws), ws.numel(), _lib.stream_of(query)), "dense_decode")
    return out


_PREFILL_MASK_DTYPES = (torch.bool, torch.float32, torch.bfloat16, torch.float16)


def prefill_supported(query, key, value, attention_mask=None, dropout: float = 0.0, scaling=None) -> bool:
    """Whether prefill_attention takes these operands (else the caller keeps
    torch SDPA, as the reference does for every prefill)."""
    return ((scaling is None or 0 < scaling < float("inf")) and query.is_cuda and query.dim() == 4 and query.dtype in (torch.bfloat16, torch.float16)
            and key.dtype == query.dtype and value.dtype == query.dtype and query.shape[-1] in (64, 128)
            and not dropout and query.shape[1] % key.shape[1] == 0 and query.shape[1] % value.shape[1] == 0
            and (attention_mask is None or (attention_mask.dim() == 4 and attention_mask.dtype in _PREFILL_MASK_DTYPES
                                            and attention_mask.shape[2] in (1, query.shape[2]))))


def prefill_attention(query, key, value, attention_mask=None, scaling=None, is_causal=None, causal_offset: int = 0,
                      out=None):
    """Prefill attention with separate key / value head counts
    (attention/attention.py:13-53: torch SDPA over keys expanded by q_h / k_h
    and values by q_h / v_h), one HIP kernel over the unexpanded caches.

    query [b, q_h, Lq, d], key [b, k_h, Lk, d], value [b, v_h, Lk, d] (bf16 /
    f16, d 64 or 128); attention_mask [b|1, q_h|1, Lq|1, >= Lk] (bool keeps
    True, float is added), cut to Lk as the reference does (:28-30).
    is_causal None: causal iff Lq > 1 and there is no mask (:36-37); causal
    means key j <= query i + causal_offset (SDPA: causal_offset 0).
    Returns out [b, Lq, q_h, d]: the reference's output after its transpose."""
    dev = _need_gpu(query, key, value, attention_mask)
    query, key, value = _vec_ready(query), _vec_ready(key), _vec_ready(value)
    b, q_h, Lq, d = query.shape
    Lk = key.shape[2]
    mask = attention_mask
    if mask is not None:
        if mask.dim() != 4:
            raise ValueError(f"saga_amd: attention mask must be 4-D, got {tuple(mask.shape)}")
        mask = mask[:, :, :, :Lk]
        if mask.shape[2] == 1 and Lq > 1:
            mask = mask.expand(-1, -1, Lq, -1)
    if is_causal is None:
        is_causal = Lq > 1 and mask is None
    if is_causal and mask is not None:
        raise ValueError("saga_amd: a mask and is_causal cannot both be given (as in torch SDPA)")
    if out is None:
        out = torch.empty(b, Lq, q_h, d, dtype=query.dtype, device=dev)
    if out.numel() == 0:
        return out
    if Lk == 0:
        return out.zero_()
    _lib.check(_lib.load().saga_prefill_attention(_lib.tensor(query), _lib.tensor(key), _lib.tensor(value),
                                                  _lib.tensor(mask), _scale(query, scaling), 1 if is_causal else 0,
                                                  int(causal_offset), _lib.tensor(out), _lib.stream_of(query)),
               "prefill_attention")
    return out


def atopn_kept_positions(b: int, q_h: int, k_h: int, L: int, d: int, buf_k: int, workspace: torch.Tensor):
    """The fast step's kept positions of every row after a call on
    `workspace`, on the device: int32 [b*q_h, buf_k] in ascending order,
    padded with -1 past each row's count."""
    lay = _lib.atopn_layout(b, q_h, k_h, L, d, buf_k)
    nr, ns, cap = b * q_h, lay.nslice, lay.slice_cap
    ws = workspace
    cnt = ws[lay.slice_cnt:lay.slice_cnt + nr * ns * 4].view(torch.int32).reshape(nr, ns).clamp(max=cap)
    sidx = ws[lay.slice_idx:lay.slice_idx + nr * ns * cap * 4].view(torch.int32).reshape(nr, ns, cap)
    valid = torch.arange(cap, device=ws.device)[None, None, :] < cnt[:, :, None]
    rank = torch.cumsum(valid.reshape(nr, -1).to(torch.int32), dim=1).reshape(nr, ns, cap)
    valid &= rank <= buf_k  # the ordered cap: the first buf_k by position
    out = torch.full((nr, buf_k), -1, dtype=torch.int32, device=ws.device)
    dest = (rank - 1).clamp(min=0)
    rows = torch.arange(nr, device=ws.device)[:, None, None].expand(nr, ns, cap)
    out[rows[valid], dest[valid]] = sidx[valid]
    return out


def atopn_distinct_value_rows(kept: torch.Tensor, b: int, q_h: int, v_h: int, L: int) -> int:
    """Distinct V rows a fast step reads: the union of kept positions over the
    query heads sharing each (batch, value head)."""
    nr = b * q_h
    r = torch.arange(nr, device=kept.device)[:, None].expand_as(kept)
    group = (r // q_h) * v_h + (r % q_h) // (q_h // v_h)
    valid = kept >= 0
    key = group[valid].to(torch.int64) * L + kept[valid].to(torch.int64)
    return int(torch.unique(key).numel())


def atopn_workspace_views(b: int, q_h: int, k_h: int, L: int, d: int, buf_k: int, device, fast: bool = True,
                          workspace=None, rows=None) -> dict:
    """An Atop-N workspace after a call, for inspection (valid until the next
    call on it; default: the cached one of the device's current stream):
    logit thresholds (fast step), kept / passing counts, the selected
    positions and logits in ascending order, and the scores.  The calibration
    step (fast=False) writes its list to sel_idx / sel_val; the fast step
    keeps it in per-slice lists, concatenated here in slice order and cut at
    buf_k (host copies).  rows: only these score rows, as host tensors (for
    large shapes)."""
    lay = _lib.atopn_layout(b, q_h, k_h, L, d, buf_k)
    dev = _device(device)
    ws = workspace if workspace is not None else \
        _WORKSPACES[(dev, torch.cuda.current_stream(dev).cuda_stream, "atopn")]
    nr = b * q_h

    def view(off, n, dt):
        es = torch.tensor([], dtype=dt).element_size()
        return ws[off:off + n * es].view(dt)

    out = {
        "thresh": view(lay.thresh, nr, torch.float32),
        "sel_cnt": view(lay.sel_cnt, nr, torch.int32),
        "sel_total": view(lay.sel_total, nr, torch.int32),
        "sel_idx": view(lay.sel_idx, nr * buf_k, torch.int32).reshape(nr, buf_k),
        "sel_val": view(lay.sel_val, nr * buf_k, torch.float32).reshape(nr, buf_k),
        "scores": view(lay.scores, nr * lay.scores_ld, torch.float32).reshape(nr, lay.scores_ld)[:, :L],
    }
    sel = list(range(nr)) if rows is None else [int(r) for r in rows]
    if rows is not None:
        ri = torch.tensor(sel, device=ws.device, dtype=torch.int64)
        out = {k: v.index_select(0, ri).cpu() for k, v in out.items()}
    if fast:
        ns, cap = lay.nslice, lay.slice_cap
        ri = torch.tensor(sel, device=ws.device, dtype=torch.int64)
        cnt = view(lay.slice_cnt, nr * ns, torch.int32).reshape(nr, ns).index_select(0, ri).cpu()
        sidx = view(lay.slice_idx, nr * ns * cap, torch.int32).reshape(nr, ns, cap).index_select(0, ri).cpu()
        sval = view(lay.slice_val, nr * ns * cap, torch.float32).reshape(nr, ns, cap).index_select(0, ri).cpu()
        idx = torch.full((len(sel), buf_k), -1, dtype=torch.int32)
        val = torch.full((len(sel), buf_k), float("nan"))
        for j in range(len(sel)):
            keep = [min(int(cnt[j, s]), cap) for s in range(ns)]
            rj = torch.cat([sidx[j, s, :keep[s]] for s in range(ns)])[:buf_k]
            rv = torch.cat([sval[j, s, :keep[s]] for s in range(ns)])[:buf_k]
            idx[j, :rj.numel()] = rj
            val[j, :rv.numel()] = rv
        out["sel_idx"], out["sel_val"] = idx, val
    return out


# ----------------------------------------------------------- decode-step ops

def rope_kv_append(qkv, n_q, n_k, n_v, theta, pos, k_cache, v_cache, batch=None, q_out=None):
    """RoPE on the new tokens' q and k, k/v appended into the separate caches
    (transformers models/qwen2/modeling_qwen2.py:211-214 + cache update).
    qkv [N, (n_q+n_k+n_v)*d]; pos int32 [N]; batch int32 [N] or None.
    Returns q_out [N, n_q, d]."""
    dev = _need_gpu(qkv, pos, k_cache, v_cache, batch)
    d = k_cache.shape[-1]
    if q_out is None:
        q_out = torch.empty(qkv.shape[0], n_q, d, dtype=qkv.dtype, device=dev)
    for t, name in ((pos, "pos"), (batch, "batch")):
        if t is not None and (t.dtype != torch.int32 or not t.is_contiguous()):
            raise ValueError(f"saga_amd: {name} must be a contiguous int32 tensor")
    _lib.check(_lib.load().saga_rope_kv_append(_lib.tensor(qkv), n_q, n_k, n_v, float(theta), _lib.ptr(pos),
                                               _lib.ptr(batch), _lib.tensor(q_out), _lib.tensor(k_cache),
                                               _lib.tensor(v_cache), _lib.stream_of(qkv)), "rope_kv_append")
    return q_out


def rmsnorm(x, weight, eps, out=None):
    """weight * x / sqrt(mean(x^2) + eps) over the last dim of x [N, H]."""
    _need_gpu(x, weight)
    out = torch.empty_like(x) if out is None else out
    _lib.check(_lib.load().saga_rmsnorm(_lib.tensor(x), _lib.tensor(weight), float(eps), _lib.tensor(out),
                                        _lib.stream_of(x)), "rmsnorm")
    return out


def silu_mul(gate_up, out=None):
    """silu(gate) * up for gate_up = [gate | up] of shape [N, 2H] -> [N, H]."""
    _need_gpu(gate_up)
    n, h2 = gate_up.shape
    out = torch.empty(n, h2 // 2, dtype=gate_up.dtype, device=gate_up.device) if out is None else out
    _lib.check(_lib.load().saga_silu_mul(_lib.tensor(gate_up), _lib.tensor(out), _lib.stream_of(gate_up)), "silu_mul")
    return out


def pack_gemv_weight(w: torch.Tensor, tile_rows: int = 16) -> torch.Tensor:
    """W [N, K] -> a packed layout that gemv and gemv_rope_kv also accept:
    every MFMA fragment is 1 KB contiguous (one DRAM region per load).
    tile_rows 16: [N/16, K/32, 16, 32], fragment = 16 rows x 32 columns.
    tile_rows 8: [N/8, K/64, 512], fragment row 8h + r = W row 8t + r at
    columns [64j + 32h, 64j + 32h + 32): weights of few 16-row tiles (the
    1536-row projections) spread over twice the workgroups, for at most 8
    rows of x."""
    N, K = w.shape
    if N % 16 or K % 32:
        raise ValueError("saga_amd: packing needs N % 16 == 0 and K % 32 == 0")
    if tile_rows == 16:
        return w.reshape(N // 16, 16, K // 32, 32).permute(0, 2, 1, 3).contiguous()
    if tile_rows != 8:
        raise ValueError("saga_amd: tile_rows must be 16 or 8")
    if K % 64:
        raise ValueError("saga_amd: 8-row packing needs K % 64 == 0")
    return w.reshape(N // 8, 8, K // 64, 2, 32).permute(0, 2, 3, 1, 4).reshape(N // 8, K // 64, 512).contiguous()


def _gemv_n(w: torch.Tensor) -> int:
    return w.shape[0] * {4: 16, 3: 8}.get(w.dim(), 1)


def gemv(x, w, bias=None, rms_eps=None, epilogue="store", out=None, split_k=True, workspace=None):
    """Skinny projection for decode (x [M <= 32, K] bf16, w [N, K] bf16, or
    packed by pack_gemv_weight):
    y = s * x @ w.T (+ bias), s = 1/sqrt(mean(x^2) + rms_eps) per row when
    rms_eps is given (RMSNorm fused, norm weight folded into w).
    epilogue: "store", "add" (out += result, in place) or "silu_pairs" (w rows
    interleaved gate/up; out = silu(gate) * up, [M, N/2]).  split_k: pass
    the cached workspace, so that long-row weights with few tiles are read
    split over K (deterministic two-kernel reduction); workspace: a caller's
    own instead of the cached one."""
    _need_gpu(x, w, bias, out)
    codes = {"store": _lib.GEMV_STORE, "add": _lib.GEMV_ADD, "silu_pairs": _lib.GEMV_SILU_PAIRS}
    code = codes[epilogue]
    M, N = x.shape[0], _gemv_n(w)
    if out is None:
        if code == _lib.GEMV_ADD:
            raise ValueError("saga_amd: epilogue 'add' needs out")
        out = torch.empty(M, N // 2 if code == _lib.GEMV_SILU_PAIRS else N, dtype=x.dtype, device=x.device)
    eps = -1.0 if rms_eps is None else float(rms_eps)
    lib = _lib.load()
    need = lib.saga_gemv_workspace_bytes(M, N, x.shape[1]) if split_k else 0
    ws = _take_workspace(workspace, x.device, "gemv", need) if need else None
    _lib.check(lib.saga_gemv(_lib.tensor(x), _lib.tensor(w), _lib.tensor(bias), eps, code, _lib.tensor(out),
                             _lib.ptr(ws), ws.numel() if ws is not None else 0, _lib.stream_of(x)), "gemv")
    return out


def rope_pair_order(n_q, n_k, n_v, d, device=None):
    """Row permutation of a fused [q | k | v] projection (heads of d rows)
    that puts every q and k head in rotary-pair order [0, d/2, 1, d/2+1, ...]
    and leaves the v heads in place: w_pairs = w[order], bias_pairs = bias[order]
    (the layout gemv_rope_kv expects)."""
    half = d // 2
    pair = torch.stack([torch.arange(half), torch.arange(half) + half], dim=1).reshape(-1)
    parts = [pair + h * d for h in range(n_q + n_k)]
    parts += [torch.arange(d) + (n_q + n_k + h) * d for h in range(n_v)]
    return torch.cat(parts).to(device=device)


def gemv_rope_kv(x, w_pairs, bias_pairs, n_q, n_k, n_v, theta, pos, k_cache, v_cache, rms_eps=None, batch=None,
                 q_out=None, rope_table=None):
    """Fused q/k/v projection + RoPE + KV-cache append for M <= 32 new tokens:
    the same results as gemv(x, w, bias) followed by rope_kv_append, with w
    and bias given in rope_pair_order.  rope_table: rope_table(pos, d, theta)
    of the same positions (the rotations computed once for several layers),
    or None.  Returns q_out [M, n_q, d]."""
    dev = _need_gpu(x, w_pairs, bias_pairs, pos, k_cache, v_cache, batch, q_out, rope_table)
    d = k_cache.shape[-1]
    if q_out is None:
        q_out = torch.empty(x.shape[0], n_q, d, dtype=x.dtype, device=dev)
    for t, name in ((pos, "pos"), (batch, "batch")):
        if t is not None and (t.dtype != torch.int32 or not t.is_contiguous()):
            raise ValueError(f"saga_amd: {name} must be a contiguous int32 tensor")
    if rope_table is not None and (rope_table.dtype != torch.float32 or not rope_table.is_contiguous()
                                   or tuple(rope_table.shape) != (x.shape[0], d // 2, 2)):
        raise ValueError("saga_amd: rope_table must be a contiguous float32 [M, d/2, 2] tensor")
    eps = -1.0 if rms_eps is None else float(rms_eps)
    _lib.check(_lib.load().saga_gemv_rope_kv(_lib.tensor(x), _lib.tensor(w_pairs), _lib.tensor(bias_pairs), eps,
                                             n_q, n_k, n_v, float(theta), _lib.ptr(pos), _lib.ptr(batch),
                                             _lib.tensor(q_out), _lib.tensor(k_cache), _lib.tensor(v_cache),
                                             _lib.ptr(rope_table), _lib.stream_of(x)), "gemv_rope_kv")
    return q_out


def rope_table(pos, d, theta, out=None):
    """Rotations of the token rows at positions pos (int32 [M]): fp32
    [M, d/2, 2] with out[n, i] = (cos, sin)(pos[n] * theta^(-2i/d)), the
    angles rope_kv_append and gemv_rope_kv use."""
    dev = _need_gpu(pos, out)
    if pos.dtype != torch.int32 or not pos.is_contiguous() or pos.dim() != 1:
        raise ValueError("saga_amd: pos must be a contiguous int32 [M] tensor")
    if out is None:
        out = torch.empty(pos.shape[0], d // 2, 2, dtype=torch.float32, device=dev)
    elif out.dtype != torch.float32 or not out.is_contiguous() or tuple(out.shape) != (pos.shape[0], d // 2, 2):
        raise ValueError("saga_amd: out must be a contiguous float32 [M, d/2, 2] tensor")
    _lib.check(_lib.load().saga_rope_table(_lib.ptr(pos), pos.shape[0], d, float(theta), _lib.ptr(out),
                                           _lib.stream_of(pos)), "rope_table")
    return out


def embed_rope(tokens, embed, out, pos=None, d=None, theta=None, rope_table=None):
    """The opening of a decode step in one launch: out[b] = embed[tokens[b]]
    (tokens int64 [B], embed [V, H], out [B, H]; an id outside [0, V) gives
    a NaN row) and, when rope_table (fp32 [B, d/2, 2]) is given, the rows'
    rotations at positions pos (int32 [B]) as rope_table() computes them."""
    _need_gpu(tokens, embed, out, pos, rope_table)
    if tokens.dtype != torch.int64 or not tokens.is_contiguous() or tokens.shape != (out.shape[0],):
        raise ValueError("saga_amd: tokens must be a contiguous int64 [B] tensor")
    if rope_table is not None:
        if pos is None or pos.dtype != torch.int32 or not pos.is_contiguous() or pos.shape != tokens.shape:
            raise ValueError("saga_amd: pos must be a contiguous int32 [B] tensor")
        if (rope_table.dtype != torch.float32 or not rope_table.is_contiguous()
                or tuple(rope_table.shape) != (out.shape[0], d // 2, 2)):
            raise ValueError("saga_amd: rope_table must be a contiguous float32 [B, d/2, 2] tensor")
    _lib.check(_lib.load().saga_embed_rope(_lib.ptr(tokens), _lib.tensor(embed), _lib.tensor(out), _lib.ptr(pos),
                                           int(d or 0), float(theta or 0.0), _lib.ptr(rope_table),
                                           _lib.stream_of(out)), "embed_rope")
    return out


def advance_positions(pos, kv_len=None):
    """pos += 1 and kv_len += 1 (int32 [B] tensors) in one launch: the close
    of a decode step."""
    _need_gpu(pos, kv_len)
    for t in (pos, kv_len):
        if t is not None and (t.dtype != torch.int32 or not t.is_contiguous() or t.shape != pos.shape):
            raise ValueError("saga_amd: pos and kv_len must be contiguous int32 tensors of one shape")
    _lib.check(_lib.load().saga_advance_positions(_lib.ptr(pos), _lib.ptr(kv_len), pos.numel(), _lib.stream_of(pos)),
               "advance_positions")


def argmax_rows(x, out=None, workspace=None):
    """First index of each row's maximum (bf16 [rows, N]) -> int64 [rows]."""
    _need_gpu(x, out)
    out = torch.empty(x.shape[0], dtype=torch.int64, device=x.device) if out is None else out
    lib = _lib.load()
    need = lib.saga_argmax_workspace_bytes(x.shape[0], x.shape[1])
    ws = _take_workspace(workspace, x.device, "argmax", need) if need else None
    _lib.check(lib.saga_argmax(_lib.tensor(x), _lib.ptr(out), _lib.ptr(ws), ws.numel() if ws is not None else 0,
                               _lib.stream_of(x)), "argmax")
    return out
