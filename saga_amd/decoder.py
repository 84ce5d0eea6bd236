"""Decode harness: a Qwen2/Llama-shaped decoder on the SAGA decode path.

The counterpart of the reference's benchmark machinery (speedup.py:119-440):
separate key-head / value-head KV caches (initialize_kv_cache, :119-139), a
batch-1 prefill replicated to the whole batch (prefill, :146-161), and decode
steps captured as two HIP graphs -- one for the Atop-N calibration step and
one for the fast steps -- replayed once per token (capture_cuda_graphs /
decode_with_graph, :179-291).  Weights are random by default (the benchmarked
models' shapes) or come from a SAGA checkpoint (saga_amd.checkpoint,
SagaDecoder.from_pretrained).

Per layer and step (7 launches): q/k/v projection with the RMSNorm and bias
fused -> RoPE + cache append -> attention (Atop-N: scores, then
select + softmax.V; or dense) -> o_proj accumulated into the residual stream
-> [gate, up] projection with the RMSNorm and silu(gate)*up fused -> down
projection accumulated into the residual stream.  Projections use the
saga_amd skinny GEMM (batch <= 32; hipBLASLt otherwise), the LM head is
followed by a row argmax kernel.  Positions advance on the device, so one
captured graph serves every step.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, replace
from typing import Optional

import torch

from . import ops
from .attention.attention import sdpa_attention_forward
from .kv_cache import KVCache, kv_cache_bytes  # noqa: F401  (kv_cache_bytes re-exported)


@dataclass(frozen=True)
class DecoderShape:
    """Transformer shape; n_k / n_v are SAGA's separate key / value head counts."""
    layers: int
    hidden: int
    n_q: int
    n_k: int
    n_v: int
    head_dim: int
    intermediate: int
    vocab: int
    rope_theta: float
    eps: float
    qkv_bias: bool = True

    @property
    def qkv_width(self) -> int:
        return (self.n_q + self.n_k + self.n_v) * self.head_dim


# Qwen2.5-1.5B with one key head and two value heads (SAGA); the dense-GQA
# comparator keeps the original two key/value heads.
QWEN25_15B_SAGA = DecoderShape(28, 1536, 12, 1, 2, 128, 8960, 151936, 1e6, 1e-6, True)
QWEN25_15B_GQA = replace(QWEN25_15B_SAGA, n_k=2)
# SmolLM2-360M with 1 key head / 5 value heads (Llama: no q/k/v bias).
SMOLLM2_360M_SAGA = DecoderShape(32, 960, 15, 1, 5, 64, 2560, 49152, 1e5, 1e-5, False)
SMOLLM2_360M_GQA = replace(SMOLLM2_360M_SAGA, n_k=5)


def gemv_tile_rows(shape: DecoderShape, batch: int) -> int:
    """Weight tile rows of the q/k/v, o and down projections: 8-row tiles
    (packed [N/8, K/64, 512]: twice the workgroups of 16-row tiles) when the
    batch is at most 8 rows and every one of those weights has K % 64 == 0
    (q/k/v: hidden, o: n_q * head_dim, down: intermediate), else 16."""
    ks = (shape.hidden, shape.n_q * shape.head_dim, shape.intermediate)
    return 8 if batch <= 8 and all(k % 64 == 0 for k in ks) else 16


class _HeadGroups(torch.nn.Module):
    """Stand-in for the HF attention module passed to sdpa_attention_forward."""
    num_key_value_groups = 1


class SagaDecoder:
    """Qwen2 / Llama-shaped decoder with SAGA attention on MI355X: random-init
    weights, or a checkpoint's (weights=..., from_pretrained).

    mode: "atopn" (calibration + fast Atop-N steps), "dense" (every layer on
    the split-L dense decode kernel; with n_k == n_v this is plain GQA) or
    "vanilla" (every layer through sdpa_attention_forward, the drop-in for
    the model's own SDPA function that the reference's vanilla mode calls
    for decode, speedup.py:76-83: the flash prefill kernel over the
    unexpanded caches with one query per row and a kv_len mask, built on the
    device).  exempt_layers run dense in "atopn" mode
    (attention/attention.py:94, speedup.py:65-66).
    With packed decode weights (pack_weights) the row-major projection
    weights are released after packing unless keep_source_weights: the
    prefill then unpacks one layer's weights at a time.  k2_variant picks the
    fast step's selection + softmax.V kernels (ops.atopn_decode).
    """

    def __init__(self, shape: DecoderShape, batch: int, max_len: int, mode: str = "atopn", top_n: int = 512,
                 exempt_layers=(), device="cuda", dtype=torch.bfloat16, seed: int = 0, fuse_rope: bool = True,
                 pack_weights: bool = True, weights: Optional[dict] = None, keep_source_weights: bool = False,
                 k2_variant: int = 0):
        if mode not in ("atopn", "dense", "vanilla"):
            raise ValueError(f"mode must be 'atopn', 'dense' or 'vanilla', got {mode!r}")
        self.shape, self.batch, self.max_len, self.mode, self.top_n = shape, batch, max_len, mode, top_n
        self.exempt = set(exempt_layers)
        self.device, self.dtype = torch.device(device), dtype
        g = torch.Generator(device=self.device).manual_seed(seed)
        s, d = shape, shape.head_dim

        if weights is not None:
            self._take_weights(weights)
        else:
            def w(*size, std=0.02):
                return (torch.randn(*size, generator=g, device=self.device, dtype=torch.float32) * std).to(dtype)

            self.embed = w(s.vocab, s.hidden)
            self.lm_head = self.embed  # tied
            self.ln1 = [torch.ones(s.hidden, device=self.device, dtype=dtype) for _ in range(s.layers)]
            self.ln2 = [torch.ones(s.hidden, device=self.device, dtype=dtype) for _ in range(s.layers)]
            self.w_qkv = [w(s.qkv_width, s.hidden) for _ in range(s.layers)]
            self.b_qkv = [w(s.qkv_width) if s.qkv_bias else torch.zeros(s.qkv_width, device=self.device, dtype=dtype)
                          for _ in range(s.layers)]
            self.w_o = [w(s.hidden, s.n_q * d) for _ in range(s.layers)]
            self.w_gu = [w(2 * s.intermediate, s.hidden) for _ in range(s.layers)]
            self.w_d = [w(s.hidden, s.intermediate) for _ in range(s.layers)]
            self.ln_f = torch.ones(s.hidden, device=self.device, dtype=dtype)
        # separate key-head and value-head caches [layer][batch, heads, max_len, d]
        self.kv = KVCache(s, batch, max_len, self.device, dtype)
        self.k_cache, self.v_cache = self.kv.k, self.kv.v
        # Atop-N threshold table, rows = batch * n_q (attention/attention.py:92-99)
        self.table = torch.zeros(max(s.layers, 1), batch * s.n_q, device=self.device, dtype=torch.float32)
        # static decode-step state (fixed addresses for graph replay)
        self.tokens = torch.zeros(batch, dtype=torch.int64, device=self.device)
        self.pos = torch.zeros(batch, dtype=torch.int32, device=self.device)
        self.kv_len = torch.zeros(batch, dtype=torch.int32, device=self.device)
        self._positions = torch.arange(max_len, dtype=torch.int32, device=self.device)  # vanilla mode's mask
        self._x = torch.empty(batch, s.hidden, device=self.device, dtype=dtype)
        self._h = torch.empty(batch, s.hidden, device=self.device, dtype=dtype)
        self._qkv = torch.empty(batch, s.qkv_width, device=self.device, dtype=dtype)
        self._q = torch.empty(batch, s.n_q, d, device=self.device, dtype=dtype)
        self._rope = torch.empty(batch, d // 2, 2, device=self.device, dtype=torch.float32)  # the step's rotations
        self._attn = torch.empty(batch, s.n_q, 1, d, device=self.device, dtype=dtype)
        self._gu = torch.empty(batch, 2 * s.intermediate, device=self.device, dtype=dtype)
        self._act = torch.empty(batch, s.intermediate, device=self.device, dtype=dtype)
        self._logits = torch.empty(batch, s.vocab, device=self.device, dtype=dtype)
        # decode projections: the skinny-GEMM kernel for up to 32 token rows
        self.use_gemv = (batch <= 32 and dtype == torch.bfloat16 and s.hidden % 32 == 0 and s.intermediate % 32 == 0
                         and (s.n_q * d) % 32 == 0 and s.qkv_width % 16 == 0 and s.vocab % 16 == 0)
        # q/k/v projection, RoPE and cache append in one launch (pair-ordered rows)
        self.fuse_rope = fuse_rope and self.use_gemv and d % 16 == 0
        self.pack_weights = pack_weights
        self.keep_source_weights = keep_source_weights
        self.k2_variant = k2_variant
        self.prepare_kernel_weights()
        self._alloc_workspaces()
        self.graph_cal: Optional[torch.cuda.CUDAGraph] = None
        self.graph_fast: Optional[torch.cuda.CUDAGraph] = None
        self.prompt_len = 0

    # (attribute, shape as a function of the decoder shape) of every weight
    _WEIGHT_SHAPES = {
        "embed": lambda s: (s.vocab, s.hidden),
        "lm_head": lambda s: (s.vocab, s.hidden),
        "ln_f": lambda s: (s.hidden,),
        "ln1": lambda s: (s.hidden,),
        "ln2": lambda s: (s.hidden,),
        "w_qkv": lambda s: (s.qkv_width, s.hidden),
        "b_qkv": lambda s: (s.qkv_width,),
        "w_o": lambda s: (s.hidden, s.n_q * s.head_dim),
        "w_gu": lambda s: (2 * s.intermediate, s.hidden),
        "w_d": lambda s: (s.hidden, s.intermediate),
    }
    _PER_LAYER = ("ln1", "ln2", "w_qkv", "b_qkv", "w_o", "w_gu", "w_d")

    def _take_weights(self, weights: dict) -> None:
        """Weights given as tensors in the decoder's layout (one per name of
        _WEIGHT_SHAPES; per-layer names hold a list; lm_head None = tied),
        moved to the decoder's device and dtype, shapes checked."""
        s = self.shape
        for name, shape_of in self._WEIGHT_SHAPES.items():
            want = tuple(shape_of(s))
            val = weights.get(name)
            if name == "lm_head" and val is None:
                continue
            if val is None:
                raise KeyError(f"weights: missing {name!r}")
            vals = val if name in self._PER_LAYER else [val]
            if name in self._PER_LAYER and len(vals) != s.layers:
                raise ValueError(f"weights: {name!r} has {len(vals)} layers, the shape {s.layers}")
            out = []
            for t in vals:
                if tuple(t.shape) != want:
                    raise ValueError(f"weights: {name!r} is {tuple(t.shape)}, the shape needs {want}")
                out.append(t.to(device=self.device, dtype=self.dtype).contiguous())
            setattr(self, name, out if name in self._PER_LAYER else out[0])
        if weights.get("lm_head") is None:
            self.lm_head = self.embed

    @classmethod
    def from_pretrained(cls, path: str, batch: int, max_len: int, num_key_heads: Optional[int] = None,
                        **kwargs) -> "SagaDecoder":
        """A decoder with the weights of a SAGA (or plain GQA) checkpoint
        directory: config.json + safetensors (saga_amd.checkpoint).
        num_key_heads merges a checkpoint's key heads at load time."""
        from .checkpoint import load_checkpoint
        shape, weights = load_checkpoint(path, num_key_heads=num_key_heads)
        return cls(shape, batch, max_len, weights=weights, **kwargs)

    def prepare_kernel_weights(self) -> None:
        """Decode-layout copies of the weights for the skinny GEMM: RMSNorm
        weights folded into the following projection (w * diag(norm)), gate
        and up rows interleaved (gate_0, up_0, gate_1, ...) so one output tile
        holds both halves of silu(gate) * up, and a normed LM head; with
        pack_weights every decode weight in the packed MFMA-fragment layout
        (ops.pack_gemv_weight), after which the row-major projection weights
        are released (keep_source_weights keeps them)."""
        if not self.use_gemv:
            return
        if self.w_qkv is None:
            raise RuntimeError("prepare_kernel_weights: the row-major weights were released after packing "
                               "(construct with keep_source_weights=True to fold new norm weights)")
        s = self.shape
        with torch.no_grad():
            self.kw_qkv = [(self.w_qkv[l].float() * self.ln1[l].float()).to(self.dtype) for l in range(s.layers)]
            self.kb_qkv = self.b_qkv
            if self.fuse_rope:
                order = ops.rope_pair_order(s.n_q, s.n_k, s.n_v, s.head_dim, device=self.device)
                self.kw_qkv = [w.index_select(0, order).contiguous() for w in self.kw_qkv]
                self.kb_qkv = [b.index_select(0, order).contiguous() for b in self.b_qkv]
                self._unpair = torch.argsort(order)
            self.kw_gu = []
            for l in range(s.layers):
                w = (self.w_gu[l].float() * self.ln2[l].float()).to(self.dtype)
                self.kw_gu.append(torch.stack([w[:s.intermediate], w[s.intermediate:]], dim=1)
                                  .reshape(2 * s.intermediate, s.hidden).contiguous())
            self.kw_lm = (self.lm_head.float() * self.ln_f.float()).to(self.dtype)
            self.kw_o = list(self.w_o)
            self.kw_d = list(self.w_d)
            if self.pack_weights:
                # MFMA-fragment order: every fragment 1 KB contiguous.  The
                # projections of few 16-row tiles (q/k/v, o, down: 96-120 at
                # the 1.5B shape) in 8-row tiles when the batch allows (<= 8
                # rows: twice the workgroups, no split over K)
                pk = ops.pack_gemv_weight
                rows8 = gemv_tile_rows(s, self.batch)
                self.kw_qkv = [pk(w, rows8) for w in self.kw_qkv]
                self.kw_gu = [pk(w) for w in self.kw_gu]
                self.kw_o = [pk(w, rows8) for w in self.w_o]
                self.kw_d = [pk(w, rows8) for w in self.w_d]
                self.kw_lm = pk(self.kw_lm)
                if not self.keep_source_weights:
                    self.w_qkv = self.w_o = self.w_gu = self.w_d = None
                    if self.lm_head is not self.embed:
                        self.lm_head = None
                    self._ones = torch.ones(s.hidden, device=self.device, dtype=self.dtype)

    def _alloc_workspaces(self) -> None:
        """The decoder's own workspaces (never the shared cache: the captured
        graphs hold their addresses for the decoder's lifetime)."""
        s, B, L, d = self.shape, self.batch, self.max_len, self.shape.head_dim
        lib = ops._lib.load() if self.device.type == "cuda" else None
        self.ws = {}
        if lib is None:
            return

        def buf(n):
            return torch.empty(max(int(n), 256), dtype=torch.uint8, device=self.device)

        self.ws["atopn"] = buf(max(ops.atopn_workspace_bytes(B, s.n_q, s.n_k, L, d, self.top_n, cal)
                                   for cal in (True, False)))
        self.ws["dense"] = buf(lib.saga_dense_workspace_bytes(B, s.n_q, L, d))
        if self.use_gemv:
            shapes = ((s.qkv_width, s.hidden), (s.hidden, s.n_q * d), (2 * s.intermediate, s.hidden),
                      (s.hidden, s.intermediate), (s.vocab, s.hidden))
            self.ws["gemv"] = buf(max(lib.saga_gemv_workspace_bytes(B, n, k) for n, k in shapes))
            self.ws["argmax"] = buf(lib.saga_argmax_workspace_bytes(B, s.vocab))

    @staticmethod
    def _unpack(w: torch.Tensor) -> torch.Tensor:
        """Row-major [N, K] of a packed weight: [N/16, K/32, 16, 32] or, in
        8-row tiles, [N/8, K/64, 512] (ops.pack_gemv_weight)."""
        if w.dim() == 2:
            return w
        if w.dim() == 3:
            n8, k64 = w.shape[0], w.shape[1]
            return w.reshape(n8, k64, 2, 8, 32).permute(0, 3, 1, 2, 4).reshape(n8 * 8, k64 * 64)
        n16, k32 = w.shape[0], w.shape[1]
        return w.permute(0, 2, 1, 3).reshape(n16 * 16, k32 * 32)

    def _prefill_layer(self, l: int):
        """(norm-1 weight, w_qkv, b_qkv, qkv column order, w_o, norm-2 weight,
        w_gu, gate/up interleaved) for the prefill of layer l: the row-major
        originals, or, once released, the unpacked decode copies (norms
        folded in, q/k rows in rotary-pair order, gate/up interleaved)."""
        if self.w_qkv is not None:
            return self.ln1[l], self.w_qkv[l], self.b_qkv[l], None, self.w_o[l], self.ln2[l], self.w_gu[l], False
        unpair = self._unpair if self.fuse_rope else None
        return (self._ones, self._unpack(self.kw_qkv[l]), self.kb_qkv[l], unpair, self._unpack(self.kw_o[l]),
                self._ones, self._unpack(self.kw_gu[l]), True)

    # ------------------------------------------------------------------ prefill
    @torch.no_grad()
    def prefill(self, prompt: torch.Tensor, chunk: int = 8192) -> None:
        """Run a batch-1 prompt through the model, fill cache row 0 and copy it
        to every batch row (speedup.py:146-161); the next token (argmax of the
        last position) is the first decode input of every row."""
        s, d = self.shape, self.shape.head_dim
        T = int(prompt.numel())
        if T + 1 > self.max_len:
            raise ValueError("prompt does not fit the cache")
        x = self.embed.index_select(0, prompt.to(self.device).reshape(-1))
        pos = torch.arange(T, device=self.device, dtype=torch.int32)
        zeros = torch.zeros(T, device=self.device, dtype=torch.int32)
        mod = _HeadGroups()
        for l in range(s.layers):
            n1, w_qkv, b_qkv, unpair, w_o, n2, w_gu, interleaved = self._prefill_layer(l)
            h = ops.rmsnorm(x, n1, s.eps)
            qkv = torch.addmm(b_qkv, h, w_qkv.t())
            if unpair is not None:
                qkv = qkv.index_select(1, unpair)
            q = ops.rope_kv_append(qkv, s.n_q, s.n_k, s.n_v, s.rope_theta, pos, self.k_cache[l], self.v_cache[l],
                                   batch=zeros)
            k = self.k_cache[l, 0:1, :, :T]
            v = self.v_cache[l, 0:1, :, :T]
            # the HIP prefill kernel when ops.prefill_supported holds for these
            # operands, else torch SDPA (attention/attention.py:13-53)
            o, _ = sdpa_attention_forward(mod, q.transpose(0, 1).unsqueeze(0), k, v, None, is_causal=True)
            x = torch.addmm(x, o.reshape(T, s.n_q * d), w_o.t())
            w_d = self.w_d[l] if self.w_d is not None else self._unpack(self.kw_d[l])
            for c0 in range(0, T, chunk):
                xc = x[c0:c0 + chunk]
                gu = torch.mm(ops.rmsnorm(xc, n2, s.eps), w_gu.t())
                if interleaved:  # (gate_0, up_0, gate_1, ...) -> [gate | up]
                    gu = gu.view(gu.shape[0], s.intermediate, 2).transpose(1, 2).reshape(gu.shape[0], -1)
                xc.addmm_(ops.silu_mul(gu), w_d.t())
            del w_qkv, w_o, w_gu, w_d
        if self.lm_head is not None:
            last = ops.rmsnorm(x[-1:], self.ln_f, s.eps)
            first = torch.mm(last, self.lm_head.t()).argmax(dim=-1)
        else:
            first = torch.mm(ops.rmsnorm(x[-1:], self._ones, s.eps), self._unpack(self.kw_lm).t()).argmax(dim=-1)
        self.k_cache[:, 1:, :, :T] = self.k_cache[:, 0:1, :, :T]
        self.v_cache[:, 1:, :, :T] = self.v_cache[:, 0:1, :, :T]
        self.prompt_len = T
        self.reset()
        self._first_token = first
        self.tokens.fill_(0)
        self.tokens.copy_(first.expand(self.batch))

    def fill_synthetic(self, prompt_len: int, seed: int = 1) -> None:
        """Fill the cache with N(0,1) keys/values of prompt_len positions
        instead of a prefill (tests and kernel-level runs)."""
        g = torch.Generator(device=self.device).manual_seed(seed)
        for c in (self.k_cache, self.v_cache):
            c[..., :prompt_len, :] = torch.randn(c[..., :prompt_len, :].shape, generator=g, device=self.device,
                                                 dtype=torch.float32).to(self.dtype)
        self.prompt_len = prompt_len
        self._first_token = torch.zeros(1, dtype=torch.int64, device=self.device)
        self.reset()

    def reset(self) -> None:
        """Rewind the decode state to just after the prompt."""
        self.pos.fill_(self.prompt_len)
        self.kv_len.fill_(self.prompt_len + 1)
        if hasattr(self, "_first_token"):
            self.tokens.copy_(self._first_token.expand(self.batch))

    # ------------------------------------------------------------------- decode
    @torch.no_grad()
    def step(self, calibrate: bool) -> None:
        """One decode step for every batch row (static buffers only)."""
        s, d, B = self.shape, self.shape.head_dim, self.batch
        ws = self.ws
        x = self._x
        # the token rows' embeddings and their rotations (once for all layers)
        ops.embed_rope(self.tokens, self.embed, x, self.pos, d, s.rope_theta,
                       rope_table=self._rope if self.fuse_rope else None)
        q4 = self._q.view(B, s.n_q, 1, d)
        for l in range(s.layers):
            if self.fuse_rope:
                ops.gemv_rope_kv(x, self.kw_qkv[l], self.kb_qkv[l], s.n_q, s.n_k, s.n_v, s.rope_theta, self.pos,
                                 self.k_cache[l], self.v_cache[l], rms_eps=s.eps, q_out=self._q,
                                 rope_table=self._rope)
            else:
                if self.use_gemv:
                    ops.gemv(x, self.kw_qkv[l], bias=self.b_qkv[l], rms_eps=s.eps, out=self._qkv, workspace=ws.get("gemv"))
                else:
                    ops.rmsnorm(x, self.ln1[l], s.eps, out=self._h)
                    torch.addmm(self.b_qkv[l], self._h, self.w_qkv[l].t(), out=self._qkv)
                ops.rope_kv_append(self._qkv, s.n_q, s.n_k, s.n_v, s.rope_theta, self.pos, self.k_cache[l],
                                   self.v_cache[l], q_out=self._q)
            K, V = self.k_cache[l], self.v_cache[l]
            if self.mode == "vanilla":
                self._vanilla_attention(q4, K, V)
            elif self.mode == "dense" or l in self.exempt:
                ops.dense_decode(q4, K, V, kv_len=self.kv_len, out=self._attn, workspace=ws["dense"])
            elif calibrate:
                ops.atopn_calibrate(q4, K, V, self.top_n, self.table[l], kv_len=self.kv_len, out=self._attn,
                                    workspace=ws["atopn"])
            else:
                ops.atopn_decode(q4, K, V, self.table[l], self.top_n, kv_len=self.kv_len, out=self._attn,
                                 workspace=ws["atopn"], k2_variant=self.k2_variant)
            if self.use_gemv:
                ops.gemv(self._attn.view(B, s.n_q * d), self.kw_o[l], epilogue="add", out=x, workspace=ws["gemv"])
                ops.gemv(x, self.kw_gu[l], rms_eps=s.eps, epilogue="silu_pairs", out=self._act, workspace=ws["gemv"])
                ops.gemv(self._act, self.kw_d[l], epilogue="add", out=x, workspace=ws["gemv"])
            else:
                x.addmm_(self._attn.view(B, s.n_q * d), self.w_o[l].t())
                ops.rmsnorm(x, self.ln2[l], s.eps, out=self._h)
                torch.mm(self._h, self.w_gu[l].t(), out=self._gu)
                ops.silu_mul(self._gu, out=self._act)
                x.addmm_(self._act, self.w_d[l].t())
        if self.use_gemv:
            ops.gemv(x, self.kw_lm, rms_eps=s.eps, out=self._logits, workspace=ws["gemv"])
            ops.argmax_rows(self._logits, out=self.tokens, workspace=ws["argmax"])
        else:
            ops.rmsnorm(x, self.ln_f, s.eps, out=self._h)
            torch.mm(self._h, self.lm_head.t(), out=self._logits)
            torch.argmax(self._logits, dim=-1, out=self.tokens)
        ops.advance_positions(self.pos, self.kv_len)

    def _vanilla_attention(self, q4: torch.Tensor, K: torch.Tensor, V: torch.Tensor) -> None:
        """speedup.py:76-83, vanilla mode: the decode step through the base
        SDPA function (sdpa_attention_forward), the cache's unfilled slots
        masked off (position < kv_len[b], built on the device)."""
        B, s = self.batch, self.shape
        keep = (self._positions[None, :] < self.kv_len[:, None])[:, None, None, :]
        o, _ = sdpa_attention_forward(_HeadGroups(), q4, K, V, keep, is_causal=False)  # [B, 1, n_q, d]
        self._attn.view(B, s.n_q, s.head_dim).copy_(o.view(B, s.n_q, s.head_dim))

    def capture(self) -> None:
        """Capture the calibration and fast steps as HIP graphs (after an eager
        warm-up that allocates every workspace)."""
        side = torch.cuda.Stream(self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            for cal in (True, False):
                self.reset()
                self.step(cal)
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        self.reset()
        graphs = []
        for cal in (True, False):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self.step(cal)
            graphs.append(g)
        self.graph_cal, self.graph_fast = graphs
        torch.cuda.synchronize(self.device)

    def replay(self, i: int) -> None:
        """Step i of a generation: the calibration graph first (Atop-N), then fast steps."""
        if self.mode == "atopn" and i == 0:
            self.graph_cal.replay()
        else:
            self.graph_fast.replay()

    @torch.no_grad()
    def generate(self, prompt: torch.Tensor, max_new_tokens: int, graphs: bool = True) -> torch.Tensor:
        """Greedy generation for every batch row from a batch-1 prompt (the
        reference benchmark's protocol, speedup.py:146-193): prefill, then
        max_new_tokens decode steps (calibration first in Atop-N mode).
        Returns the generated ids [batch, max_new_tokens]: the token picked
        after the prompt, then the pick of every decode step but the last.
        graphs: replay the captured HIP graphs (captured on first use), else
        run the steps eagerly (same kernels, same results)."""
        if max_new_tokens < 1:
            return torch.empty(self.batch, 0, dtype=torch.int64, device=self.device)
        if int(prompt.numel()) + max_new_tokens > self.max_len:
            raise ValueError("prompt + max_new_tokens does not fit the cache (max_len)")
        self.prefill(prompt)
        if graphs and self.graph_fast is None:
            self.capture()  # leaves the state rewound to just after the prompt
        out = torch.empty(self.batch, max_new_tokens, dtype=torch.int64, device=self.device)
        out[:, 0] = self.tokens
        for i in range(max_new_tokens - 1):
            if graphs:
                self.replay(i)
            else:
                self.step(calibrate=(self.mode == "atopn" and i == 0))
            out[:, i + 1] = self.tokens
        return out
