"""HIP prefill attention (saga_prefill_attention) vs the oracle's restatement
of the reference prefill (attention/attention.py:13-53: SDPA over
repeat_kv-expanded key and value heads).

bf16 / f16 outputs against the float64 oracle on the same (rounded) inputs:
max-abs 2e-2 and rel-L2 5e-3.  P is rounded to the input dtype before the
P.V product, as in torch's flash kernels; transformers' own bf16 SDPA errors
are printed beside ours at the larger shapes.  Shapes cover asymmetric key /
value heads, lengths that are not multiples of the 64-key tile or the query
block, bool and float masks (broadcast over heads, wider than the keys),
non-causal calls, a causal chunk after cached positions (causal_offset), one
query, one key, f16, strided query / output views, and the reference-API
module's dispatch to the kernel."""
import numpy as np
import pytest
import torch

from conftest import rel_l2
from oracle import saga_oracle as O
from saga_amd import ops

pytestmark = pytest.mark.gpu

MAX_ABS, REL_L2 = 2e-2, 5e-3


def _inputs(seed, b, q_h, k_h, v_h, Lq, Lk, d, dtype=torch.bfloat16):
    g = torch.Generator(device="cuda").manual_seed(seed)
    mk = lambda *s: torch.randn(*s, generator=g, device="cuda", dtype=torch.float32).to(dtype)
    return mk(b, q_h, Lq, d), mk(b, k_h, Lk, d), mk(b, v_h, Lk, d)


def _np(t):
    return t.detach().to(torch.float64).cpu().numpy()


def _check(out, ref, what):
    got = _np(out)
    err_abs, err_l2 = float(np.max(np.abs(got - ref))), rel_l2(got, ref)
    print(f"{what}: max-abs {err_abs:.2e} rel-L2 {err_l2:.2e}", flush=True)
    assert np.isfinite(got).all(), what
    assert err_abs < MAX_ABS and err_l2 < REL_L2, (what, err_abs, err_l2)


CASES = [
    # b, q_h, k_h, v_h, Lq, Lk, d, causal
    (1, 12, 1, 2, 300, 300, 128, True),    # Qwen2.5-1.5B SAGA heads
    (2, 15, 1, 5, 200, 200, 64, True),     # SmolLM2-360M SAGA heads
    (1, 4, 2, 4, 130, 257, 128, False),    # more value heads than key heads, ragged
    (3, 6, 3, 2, 65, 65, 64, True),        # more key heads than value heads
    (1, 2, 1, 1, 1, 97, 128, False),       # one query
    (1, 2, 1, 2, 33, 1, 64, False),        # one key
    (2, 8, 8, 8, 129, 129, 128, True),     # plain multi-head
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "b{}_q{}k{}v{}_Lq{}_Lk{}_d{}_{}".format(
    *c[:7], "causal" if c[7] else "full"))
def test_prefill_matches_oracle(case):
    b, q_h, k_h, v_h, Lq, Lk, d, causal = case
    print(f"prefill {case}", flush=True)
    q, k, v = _inputs(1, b, q_h, k_h, v_h, Lq, Lk, d)
    out = ops.prefill_attention(q, k, v, is_causal=causal)
    torch.cuda.synchronize()
    assert out.shape == (b, Lq, q_h, d) and out.dtype == q.dtype
    _check(out, O.prefill(_np(q), _np(k), _np(v), None, None, causal), f"prefill {case}")


@pytest.mark.parametrize("mdt", [torch.bool, torch.float32, torch.bfloat16])
def test_prefill_masks(mdt):
    """Masks [b, 1, Lq, Lk + 5] (broadcast over heads, cut to the keys) and
    [1, q_h, Lq, Lk]: bool keeps True, float is added (SDPA semantics)."""
    b, q_h, k_h, v_h, Lq, Lk, d = 2, 6, 1, 3, 77, 140, 128
    print(f"prefill mask {mdt}", flush=True)
    q, k, v = _inputs(2, b, q_h, k_h, v_h, Lq, Lk, d)
    g = torch.Generator(device="cuda").manual_seed(3)
    for shape in ((b, 1, Lq, Lk + 5), (1, q_h, Lq, Lk)):
        r = torch.rand(*shape, generator=g, device="cuda")
        if mdt == torch.bool:
            m = r < 0.6
            m[..., 0] = True
        else:
            m = torch.where(r < 0.3, torch.full_like(r, -float("inf")), torch.randn_like(r)).to(mdt)
            m[..., 0] = 0
        m[..., 3, :] = False if mdt == torch.bool else -float("inf")  # a query that sees no key: 0
        out = ops.prefill_attention(q, k, v, attention_mask=m, scaling=0.1)
        torch.cuda.synchronize()
        ref = O.prefill(_np(q), _np(k), _np(v), m.cpu().numpy() if mdt == torch.bool else _np(m), 0.1, False)
        _check(out, ref, f"mask {mdt} {shape}")
        assert not out[:, 3].any()


def test_prefill_causal_offset_chunk():
    """A chunk of 50 queries after 250 cached positions: causal_offset 250
    equals the oracle with the explicit mask key <= 250 + i."""
    b, q_h, k_h, v_h, Lq, Lk, d = 1, 12, 1, 2, 50, 300, 128
    q, k, v = _inputs(4, b, q_h, k_h, v_h, Lq, Lk, d)
    out = ops.prefill_attention(q, k, v, is_causal=True, causal_offset=Lk - Lq)
    torch.cuda.synchronize()
    mask = np.arange(Lk)[None, None, None, :] <= (Lk - Lq + np.arange(Lq))[None, None, :, None]
    _check(out, O.prefill(_np(q), _np(k), _np(v), mask, None, False), "causal_offset 250")


def test_prefill_f16():
    q, k, v = _inputs(5, 2, 12, 1, 2, 190, 190, 128, dtype=torch.float16)
    out = ops.prefill_attention(q, k, v, is_causal=True)
    torch.cuda.synchronize()
    assert out.dtype == torch.float16
    _check(out, O.prefill(_np(q), _np(k), _np(v), None, None, True), "f16")


def test_prefill_strided_views():
    """The decoder's layout: queries [T, q_h, d] viewed as [1, q_h, T, d],
    caches [B, h, Lmax, d] cut to T, output written into a wider buffer."""
    T, q_h, d, Lmax = 333, 12, 128, 512
    g = torch.Generator(device="cuda").manual_seed(6)
    qt = torch.randn(T, q_h, d, generator=g, device="cuda").to(torch.bfloat16)
    kc = torch.randn(2, 1, Lmax, d, generator=g, device="cuda").to(torch.bfloat16)
    vc = torch.randn(2, 2, Lmax, d, generator=g, device="cuda").to(torch.bfloat16)
    q, k, v = qt.transpose(0, 1).unsqueeze(0), kc[1:2, :, :T], vc[1:2, :, :T]
    big = torch.full((1, T, q_h + 4, d), 7.0, device="cuda", dtype=torch.bfloat16)
    out = ops.prefill_attention(q, k, v, is_causal=True, out=big[:, :, 2:2 + q_h])
    torch.cuda.synchronize()
    assert out.data_ptr() == big[:, :, 2:].data_ptr()
    assert (big[:, :, :2] == 7).all() and (big[:, :, 2 + q_h:] == 7).all()
    _check(out, O.prefill(_np(q), _np(k), _np(v), None, None, True), "strided")


@pytest.mark.parametrize("L,d,q_h,k_h,v_h", [(4096, 128, 12, 1, 2), (2048, 64, 15, 1, 5)])
def test_prefill_long_vs_torch_fp32(L, d, q_h, k_h, v_h):
    """Long causal prefill vs torch SDPA in fp32 on the expanded heads (the
    oracle's float64 loop would take minutes at this size)."""
    print(f"prefill long L={L} d={d}", flush=True)
    q, k, v = _inputs(7, 1, q_h, k_h, v_h, L, L, d)
    out = ops.prefill_attention(q, k, v, is_causal=True)
    kx = k.float().repeat_interleave(q_h // k_h, dim=1)
    vx = v.float().repeat_interleave(q_h // v_h, dim=1)
    ref = torch.nn.functional.scaled_dot_product_attention(q.float(), kx, vx, is_causal=True).transpose(1, 2)
    tb = torch.nn.functional.scaled_dot_product_attention(q, kx.to(q.dtype), vx.to(q.dtype),
                                                          is_causal=True).transpose(1, 2)
    torch.cuda.synchronize()
    r = _np(ref)
    print(f"  torch bf16 SDPA: max-abs {float(np.max(np.abs(_np(tb) - r))):.2e} rel-L2 {rel_l2(_np(tb), r):.2e}")
    _check(out, r, f"long L={L} d={d}")


def test_reference_api_dispatches_to_the_kernel(monkeypatch):
    """sdpa_attention_forward (attention/attention.py:13-53) with a
    transformers-style module runs the HIP kernel for bf16 d-128 prefill and
    gives the expanded-SDPA result; fp32 operands keep torch SDPA."""
    from saga_amd.attention import attention as A
    calls = []
    real = ops.prefill_attention
    monkeypatch.setattr(ops, "prefill_attention", lambda *a, **kw: calls.append(1) or real(*a, **kw))

    class Mod(torch.nn.Module):
        num_key_value_groups = 6

    q, k, v = _inputs(8, 1, 12, 1, 2, 200, 200, 128)
    out, _ = A.sdpa_attention_forward(Mod(), q, k, v, None)
    torch.cuda.synchronize()
    assert calls and out.shape == (1, 200, 12, 128) and out.is_contiguous()
    _check(out, O.prefill(_np(q), _np(k), _np(v)), "reference API")
    calls.clear()
    out32, _ = A.sdpa_attention_forward(Mod(), q.float(), k.float(), v.float(), None)
    assert not calls
    assert rel_l2(_np(out32), _np(out)) < REL_L2


def test_prefill_rejects_bad_operands():
    q, k, v = _inputs(9, 1, 6, 4, 2, 16, 16, 128)  # 6 query heads over 4 key heads
    with pytest.raises(Exception, match="multiple"):
        ops.prefill_attention(q, k, v)
    q, k, v = _inputs(9, 1, 4, 1, 2, 16, 16, 128)
    m = torch.ones(1, 1, 16, 16, dtype=torch.bool, device="cuda")
    with pytest.raises(ValueError):
        ops.prefill_attention(q, k, v, attention_mask=m, is_causal=True)
    q96, k96, v96 = _inputs(9, 1, 4, 1, 2, 16, 16, 96)
    with pytest.raises(Exception, match="head_dim"):
        ops.prefill_attention(q96, k96, v96)
