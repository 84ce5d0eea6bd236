"""Decode-step kernels and the decode harness on the GPU.

rope_kv_append / rmsnorm / silu_mul vs the oracle's restatement of the
transformers Qwen2 ops; the harness's graph-replayed steps vs eager steps;
one decode step of a tiny random decoder vs a float64 reference built from the
oracle (attention via the oracle's dense / Atop-N functions).
"""
import numpy as np
import pytest
import torch

from conftest import rel_l2
from gpu_util import dev, host
from oracle import saga_oracle as O
from saga_amd import ops

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dt,H", [(torch.bfloat16, 1536), (torch.float32, 960), (torch.float16, 100)])
def test_embed_rope_and_advance(dt, H):
    """The step's opening (embedding rows + rotation table in one launch)
    equals index_select and rope_table bit for bit (16-byte and element
    copies); an id outside the vocabulary gives a NaN row; the step's close
    adds one to every position and cache length."""
    V, B, d = 5000, 4, 128
    g = torch.Generator(device="cuda").manual_seed(3)
    emb = torch.randn(V, H, device="cuda", generator=g).to(dt)
    toks = torch.tensor([0, 4999, 17, 2500], device="cuda", dtype=torch.int64)
    pos = torch.tensor([0, 32767, 5, 131071], device="cuda", dtype=torch.int32)
    x = torch.empty(B, H, device="cuda", dtype=dt)
    table = torch.empty(B, d // 2, 2, device="cuda", dtype=torch.float32)
    ops.embed_rope(toks, emb, x, pos, d, 1e6, rope_table=table)
    torch.cuda.synchronize()
    assert torch.equal(x, emb.index_select(0, toks))
    assert torch.equal(table, ops.rope_table(pos, d, 1e6))
    ops.embed_rope(torch.tensor([1, -1, 5000, 2], device="cuda"), emb, x)  # no table
    torch.cuda.synchronize()
    assert torch.equal(x[0], emb[1]) and torch.equal(x[3], emb[2])
    assert torch.isnan(x[1].float()).all() and torch.isnan(x[2].float()).all()
    kv = pos + 1
    ops.advance_positions(pos, kv)
    ops.advance_positions(pos)
    torch.cuda.synchronize()
    assert pos.tolist() == [2, 32769, 7, 131073] and kv.tolist() == [2, 32769, 7, 131073]


def test_rope_kv_append_matches_oracle():
    rng = np.random.default_rng(40)
    N, n_q, n_k, n_v, d, B, Lmax = 5, 12, 1, 2, 128, 3, 4096
    qkv = O.round_bf16(rng.standard_normal((N, (n_q + n_k + n_v) * d), dtype=np.float32))
    pos = np.array([0, 7, 4095, 33, 1000], dtype=np.int32)
    batch = np.array([0, 1, 2, 1, 0], dtype=np.int32)
    kc = torch.zeros(B, n_k, Lmax, d, device="cuda", dtype=torch.bfloat16)
    vc = torch.zeros(B, n_v, Lmax, d, device="cuda", dtype=torch.bfloat16)
    q = host(ops.rope_kv_append(dev(qkv, "bf16"), n_q, n_k, n_v, 1e6, torch.from_numpy(pos).cuda(), kc, vc,
                                batch=torch.from_numpy(batch).cuda()))
    x = qkv.reshape(N, n_q + n_k + n_v, d)
    q_ref = O.rope(x[:, :n_q], pos[:, None], 1e6)
    k_ref = O.rope(x[:, n_q:n_q + n_k], pos[:, None], 1e6)
    assert np.max(np.abs(q - q_ref)) < 2e-2 and rel_l2(q, q_ref) < 4e-3
    kh, vh = host(kc), host(vc)
    for n in range(N):
        assert rel_l2(kh[batch[n], :, pos[n]], k_ref[n]) < 4e-3
        np.testing.assert_array_equal(vh[batch[n], :, pos[n]], x[n, n_q + n_k:])
    assert np.count_nonzero(kh) == N * n_k * d and np.count_nonzero(vh) == N * n_v * d


def test_rope_out_of_range_position_writes_nothing():
    kc = torch.zeros(1, 1, 16, 64, device="cuda", dtype=torch.bfloat16)
    vc = torch.zeros(1, 2, 16, 64, device="cuda", dtype=torch.bfloat16)
    qkv = torch.randn(1, 4 * 64, device="cuda", dtype=torch.bfloat16)
    q = ops.rope_kv_append(qkv, 1, 1, 2, 1e4, torch.tensor([16], dtype=torch.int32, device="cuda"), kc, vc)
    assert torch.isnan(q).all() and not kc.any() and not vc.any()


def test_rmsnorm_and_silu_mul_match_oracle():
    rng = np.random.default_rng(41)
    x = O.round_bf16(rng.standard_normal((8, 1536), dtype=np.float32))
    w = O.round_bf16(rng.standard_normal(1536, dtype=np.float32))
    y = host(ops.rmsnorm(dev(x, "bf16"), dev(w, "bf16"), 1e-6))
    ref = O.rmsnorm(x, w, 1e-6)
    assert rel_l2(y, ref) < 4e-3
    gu = O.round_bf16(rng.standard_normal((8, 2 * 8960), dtype=np.float32))
    a = host(ops.silu_mul(dev(gu, "bf16")))
    assert rel_l2(a, O.silu_mul(gu)) < 4e-3


def _tiny_model(mode, top_n=16, keep_source_weights=False, batch=2):
    from saga_amd.decoder import DecoderShape, SagaDecoder
    shape = DecoderShape(layers=3, hidden=256, n_q=4, n_k=1, n_v=2, head_dim=64, intermediate=512, vocab=1024,
                         rope_theta=1e4, eps=1e-6, qkv_bias=True)
    m = SagaDecoder(shape, batch=batch, max_len=600, mode=mode, top_n=top_n,
                    exempt_layers=(0,) if mode == "atopn" else (), keep_source_weights=keep_source_weights)
    return m


@pytest.mark.parametrize("mode", ["atopn", "dense", "vanilla"])
def test_graph_replay_equals_eager_steps(mode):
    m = _tiny_model(mode)
    m.prefill(torch.randint(0, 1024, (500,), generator=torch.Generator().manual_seed(7)))
    m.capture()
    m.reset()
    for i in range(4):
        m.replay(i)
    torch.cuda.synchronize()
    toks_graph = m.tokens.clone()
    k_graph = m.k_cache[:, :, :, 500:504].clone()
    m.reset()
    for i in range(4):
        m.step(calibrate=(i == 0))
    torch.cuda.synchronize()
    assert torch.equal(toks_graph, m.tokens)
    assert torch.equal(k_graph, m.k_cache[:, :, :, 500:504])
    assert int(m.pos[0]) == 504 and int(m.kv_len[0]) == 505


@pytest.mark.parametrize("mode", ["atopn", "dense"])
def test_graphs_captured_before_the_prompt(mode):
    """The step graphs hold no prompt length: captured on an empty cache
    (bench.py captures before the prefill), they replay the steps of a
    500-token prompt and then of a 300-token one exactly as eager steps do."""
    m = _tiny_model(mode)
    m.capture()
    for T, seed in ((500, 7), (300, 8)):
        m.prefill(torch.randint(0, 1024, (T,), generator=torch.Generator().manual_seed(seed)))
        m.reset()
        for i in range(4):
            m.replay(i)
        torch.cuda.synchronize()
        toks_graph = m.tokens.clone()
        k_graph = m.k_cache[:, :, :, T:T + 4].clone()
        m.reset()
        for i in range(4):
            m.step(calibrate=(mode == "atopn" and i == 0))
        torch.cuda.synchronize()
        assert torch.equal(toks_graph, m.tokens), T
        assert torch.equal(k_graph, m.k_cache[:, :, :, T:T + 4]), T
        assert int(m.pos[0]) == T + 4 and int(m.kv_len[0]) == T + 5


@pytest.mark.parametrize("batch", [2, 24])
def test_one_decode_step_vs_float64_reference(batch):
    """One dense decode step of the harness recomputed on the host in float64:
    embed, rmsnorm, projections, RoPE, cache append, attention, MLP, LM head.
    (Dense attention: an Atop-N top-k boundary could flip under the bf16
    rounding of the intermediates; selection is checked by its own tests.)
    Batch 24: the projections' 17-32-row kernels (two token tiles per weight
    fragment) and 16-row weight tiles."""
    m = _tiny_model("dense", keep_source_weights=True, batch=batch)
    g = torch.Generator(device="cuda").manual_seed(5)
    for t in m.ln1 + m.ln2 + [m.ln_f]:  # non-trivial norm weights: exercises their folding
        t.copy_((1 + 0.3 * torch.randn(t.shape, generator=g, device="cuda")).to(t.dtype))
    m.prepare_kernel_weights()
    assert m.use_gemv
    prompt_len = 400
    m.fill_synthetic(prompt_len)
    toks = [3, 1023] + [(37 * i + 11) % 1024 for i in range(batch - 2)]
    m.tokens.copy_(torch.tensor(toks, device="cuda"))
    s = m.shape
    f = lambda t: t.detach().to(torch.float64).cpu().numpy()
    kc0, vc0 = f(m.k_cache), f(m.v_cache)
    m.step(calibrate=True)
    torch.cuda.synchronize()
    x = f(m.embed)[toks]
    for l in range(s.layers):
        h = O.rmsnorm(x, f(m.ln1[l]), s.eps)
        qkv = h @ f(m.w_qkv[l]).T + f(m.b_qkv[l])
        qkv = qkv.reshape(batch, s.n_q + s.n_k + s.n_v, s.head_dim)
        q = O.rope(qkv[:, :s.n_q], prompt_len, s.rope_theta)
        k_new = O.rope(qkv[:, s.n_q:s.n_q + s.n_k], prompt_len, s.rope_theta)
        K, V = kc0[l][:, :, :prompt_len + 1].copy(), vc0[l][:, :, :prompt_len + 1].copy()
        K[:, :, prompt_len] = k_new
        V[:, :, prompt_len] = qkv[:, s.n_q + s.n_k:]
        q4 = q[:, :, None, :]
        attn = O.dense(q4, K, V)
        x = x + attn.reshape(batch, -1) @ f(m.w_o[l]).T
        h = O.rmsnorm(x, f(m.ln2[l]), s.eps)
        x = x + O.silu_mul(h @ f(m.w_gu[l]).T) @ f(m.w_d[l]).T
    logits = O.rmsnorm(x, f(m.ln_f), s.eps) @ f(m.embed).T
    got = f(m._logits)
    assert rel_l2(got, logits) < 3e-2
    # bf16 rounding of intermediates may flip a near-tie argmax; compare when the margin is clear
    for r in range(batch):
        top2 = np.sort(logits[r])[-2:]
        if top2[1] - top2[0] > 0.05:
            assert int(m.tokens[r]) == int(np.argmax(logits[r]))


def test_fused_rope_projection_equals_unfused_step():
    """The decode step with the q/k/v projection, RoPE and cache append fused
    in one launch writes the caches and logits of the unfused step."""
    from saga_amd.decoder import DecoderShape, SagaDecoder
    shape = DecoderShape(layers=2, hidden=256, n_q=4, n_k=1, n_v=2, head_dim=64, intermediate=512, vocab=1024,
                         rope_theta=1e4, eps=1e-6, qkv_bias=True)
    ms = [SagaDecoder(shape, batch=3, max_len=300, mode="dense", fuse_rope=f) for f in (True, False)]
    assert ms[0].fuse_rope and not ms[1].fuse_rope
    for m in ms:
        m.fill_synthetic(200)
        m.tokens.copy_(torch.tensor([5, 77, 1000], device="cuda"))
        m.step(calibrate=True)
    torch.cuda.synchronize()
    for a, b in ((ms[0].k_cache, ms[1].k_cache), (ms[0].v_cache, ms[1].v_cache), (ms[0]._logits, ms[1]._logits)):
        assert torch.allclose(a.float(), b.float(), rtol=2 ** -7, atol=1e-3)


def test_packed_weights_decode_step_identical():
    """The decoder with its decode weights packed (the default) produces the
    caches and logits of the row-major decoder bit for bit."""
    from saga_amd.decoder import DecoderShape, SagaDecoder
    shape = DecoderShape(layers=2, hidden=256, n_q=4, n_k=1, n_v=2, head_dim=64, intermediate=512, vocab=1024,
                         rope_theta=1e4, eps=1e-6, qkv_bias=True)
    ms = [SagaDecoder(shape, batch=3, max_len=300, mode="atopn", pack_weights=p) for p in (True, False)]
    assert ms[0].kw_gu[0].dim() == 4 and ms[1].kw_gu[0].dim() == 2
    for m in ms:
        m.fill_synthetic(200)
        m.tokens.copy_(torch.tensor([5, 77, 1000], device="cuda"))
        m.step(calibrate=True)
        m.step(calibrate=False)
    torch.cuda.synchronize()
    for a, b in ((ms[0].k_cache, ms[1].k_cache), (ms[0].v_cache, ms[1].v_cache), (ms[0]._logits, ms[1]._logits)):
        assert torch.equal(a, b)


def test_vanilla_mode_matches_dense_mode():
    """The harness's vanilla mode (speedup.py:76-83: decode through the base
    SDPA function, here the flash kernel with one query per row and a
    device-built kv_len mask) and its full mode (the split-L dense decode
    kernel) compute the same attention: one decode step of the same
    weights and prompt gives the same logits to bf16 rounding."""
    prompt = torch.randint(0, 1024, (400,), generator=torch.Generator().manual_seed(3))
    logits = {}
    for mode in ("dense", "vanilla"):
        m = _tiny_model(mode)
        m.prefill(prompt)
        m.step(calibrate=False)
        m.step(calibrate=False)
        torch.cuda.synchronize()
        logits[mode] = m._logits.float().cpu().numpy()
    assert rel_l2(logits["vanilla"], logits["dense"]) < 2e-2
