"""Seeded shape sweeps of the non-selection kernels at their size boundaries:
prefill attention against torch fp32 SDPA on expanded heads, dense decode,
the calibration step, the skinny GEMM (every epilogue, packed and row-major
W, split-K), the fused projection + RoPE + KV append, and one decode step of
small decoders against a float64 host forward.  The bars are those of the
per-kernel tests."""
import numpy as np
import pytest
import torch

from conftest import rel_l2
from gpu_util import dev, host, qkv
from oracle import saga_oracle as O
from saga_amd import ops

pytestmark = pytest.mark.gpu

GROUPS = [(12, 1, 2), (15, 1, 5), (8, 2, 4), (6, 3, 1), (4, 2, 2), (16, 1, 1), (8, 4, 2), (16, 1, 8)]  # q, k, v


@pytest.mark.parametrize("seed", range(12))
def test_prefill_sweep(seed):
    rng = np.random.default_rng(70000 + seed)
    q_h, k_h, v_h = GROUPS[seed % len(GROUPS)]
    d = (128, 64)[seed % 2]
    dt = (torch.bfloat16, torch.float16)[(seed // 2) % 2]
    b = int(rng.integers(1, 4))
    Lk = int(rng.choice([1, 31, 64, 65, 255, 257, 700, 1500]))
    Lq = int(rng.choice([1, 64, 65, Lk, max(1, Lk // 2)]))
    causal = seed % 3 != 0
    off = Lk - Lq if causal and Lk >= Lq else 0
    print(f"prefill sweep seed={seed} b={b} q/k/v={q_h}/{k_h}/{v_h} d={d} Lq={Lq} Lk={Lk} causal={causal}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(b, q_h, Lq, d, generator=g, device="cuda").to(dt)
    k = torch.randn(b, k_h, Lk, d, generator=g, device="cuda").to(dt)
    v = torch.randn(b, v_h, Lk, d, generator=g, device="cuda").to(dt)
    out = ops.prefill_attention(q, k, v, is_causal=causal, causal_offset=off)
    kx, vx = k.float().repeat_interleave(q_h // k_h, 1), v.float().repeat_interleave(q_h // v_h, 1)
    mask = None
    if causal:
        mask = torch.arange(Lk, device="cuda")[None, :] <= (off + torch.arange(Lq, device="cuda"))[:, None]
    ref = torch.nn.functional.scaled_dot_product_attention(q.float(), kx, vx, attn_mask=mask).transpose(1, 2)
    if mask is not None:  # a query that sees no key gets 0
        ref = torch.where(mask.any(-1)[None, :, None, None], ref, torch.zeros_like(ref))
    torch.cuda.synchronize()
    got, r = host(out), host(ref)
    assert np.isfinite(got).all()
    assert float(np.max(np.abs(got - r))) < 2e-2 and rel_l2(got, r) < 5e-3


@pytest.mark.parametrize("seed", range(8))
def test_dense_decode_sweep(seed):
    rng = np.random.default_rng(71000 + seed)
    q_h, k_h, v_h = GROUPS[seed % len(GROUPS)]
    d = (64, 128)[seed % 2]
    b = int(rng.integers(1, 4))
    L = int(rng.choice([1, 15, 17, 511, 513, 2047, 5000, 16385]))
    dt = ("bf16", "f16")[seed % 2]
    (q, k, v), (qd, kd, vd) = qkv(rng, b, q_h, k_h, v_h, d, L, dt)
    lens = rng.integers(1, L + 1, size=b).astype(np.int32) if seed % 3 == 0 else None
    print(f"dense sweep seed={seed} b={b} q/k/v={q_h}/{k_h}/{v_h} d={d} L={L} kv_len={lens}", flush=True)
    kvl = None if lens is None else torch.from_numpy(lens).cuda()
    out = host(ops.dense_decode(qd, kd, vd, kv_len=kvl, out_dtype=torch.float32))
    for i in range(b):
        n = L if lens is None else int(lens[i])
        assert rel_l2(out[i:i + 1], O.dense(q[i:i + 1], k[i:i + 1, :, :n], v[i:i + 1, :, :n])) < 1e-3


@pytest.mark.parametrize("seed", range(8))
def test_calibration_sweep(seed):
    rng = np.random.default_rng(72000 + seed)
    q_h, k_h, v_h = GROUPS[seed % len(GROUPS)]
    d = (128, 64)[seed % 2]
    b = int(rng.integers(1, 4))
    L = int(rng.choice([1, 17, 257, 1025, 4097, 12289]))
    N = int(rng.choice([1, 7, 256, 1000, 4096]))
    dt = ("bf16", "f16", "f32")[seed % 3]
    (q, k, v), (qd, kd, vd) = qkv(rng, b, q_h, k_h, v_h, d, L, dt, outliers=0.01 * (seed % 2))
    print(f"calibration sweep seed={seed} b={b} q/k/v={q_h}/{k_h}/{v_h} d={d} L={L} N={N} {dt}", flush=True)
    table = torch.zeros(b * q_h, device="cuda")
    cal = host(ops.atopn_calibrate(qd, kd, vd, N, table, out_dtype=torch.float32))
    kk = min(N, L)
    views = ops.atopn_workspace_views(b, q_h, k_h, L, d, kk, "cuda:0", fast=False)
    idx, cnt = views["sel_idx"].cpu().numpy(), views["sel_cnt"].cpu().numpy()
    rc, rt, ridx = O.calibrate(q, k, v, None, N, None)
    np.testing.assert_allclose(host(table), rt, rtol=1e-4, atol=1e-30)
    assert rel_l2(cal, rc) < (1e-5 if dt == "f32" else 1e-3)
    ridx = np.asarray(ridx).reshape(b * q_h, -1)
    for r in range(b * q_h):
        assert cnt[r] == kk
        assert len(set(idx[r, :kk].tolist()) ^ set(ridx[r, :kk].tolist())) <= 2  # a swap at the k-th boundary


@pytest.mark.parametrize("seed", range(18))
def test_gemv_sweep(seed):
    """Seeded shapes, epilogues and W layouts (row-major, 16-row packed, and
    8-row packed for at most 8 token rows) against the float64 product."""
    rng = np.random.default_rng(90000 + seed)
    M = int(rng.integers(1, 33))
    K = 32 * int(rng.choice([1, 2, 5, 48, 63, 280]))
    N = 16 * int(rng.choice([1, 2, 7, 96, 120, 560, 1120]))
    epi = ("store", "add", "silu_pairs")[seed % 3]
    if epi == "silu_pairs" and N % 32:
        N += 16
    rms, split = bool(seed % 2), seed % 5 != 0
    layout = ("rows", "packed16", "packed8")[(seed // 2) % 3]
    if layout == "packed8":
        M = min(M, 8)
        K += K % 64
    use_bias = epi != "silu_pairs" and seed % 4 == 1
    print(f"gemv sweep seed={seed} M={M} K={K} N={N} {epi} rms={rms} {layout} split={split}", flush=True)
    x = O.round_bf16(rng.standard_normal((M, K), dtype=np.float32))
    w = O.round_bf16(rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.05))
    b = O.round_bf16(rng.standard_normal(N, dtype=np.float32))
    wd = dev(w, "bf16")
    if layout != "rows":
        wd = ops.pack_gemv_weight(wd, 8 if layout == "packed8" else 16)
    xs = x.astype(np.float64)
    if rms:
        xs = xs / np.sqrt((xs ** 2).mean(-1, keepdims=True) + 1e-6)
    full = xs @ w.astype(np.float64).T
    eps = 1e-6 if rms else None
    bias = dev(b, "bf16") if use_bias else None
    if epi == "store":
        y = host(ops.gemv(dev(x, "bf16"), wd, bias=bias, rms_eps=eps, split_k=split))
        ref = full + (b if use_bias else 0)
    elif epi == "add":
        y0 = O.round_bf16(rng.standard_normal((M, N), dtype=np.float32))
        out = dev(y0, "bf16")
        ops.gemv(dev(x, "bf16"), wd, bias=bias, rms_eps=eps, epilogue="add", out=out, split_k=split)
        y, ref = host(out), y0 + full + (b if use_bias else 0)
    else:
        y = host(ops.gemv(dev(x, "bf16"), wd, rms_eps=eps, epilogue="silu_pairs", split_k=split))
        ref = O.silu_mul(np.concatenate([full[:, 0::2], full[:, 1::2]], axis=1))
    assert np.isfinite(y).all() and rel_l2(y, ref) < 4e-3


@pytest.mark.parametrize("seed", range(9))
def test_rope_kv_projection_sweep(seed):
    rng = np.random.default_rng(110000 + seed)
    M = int(rng.integers(1, 33))
    if seed % 3 == 1:  # 8-row packed weights take at most 8 token rows
        M = min(M, 8)
    n_q, n_k, n_v = GROUPS[seed % len(GROUPS)]
    d = (64, 128)[seed % 2]
    K = 32 * int(rng.choice([5, 30, 48]))
    theta = (1e4, 1e6)[seed % 2]
    B, Lmax = M + int(rng.integers(0, 4)), int(rng.choice([16, 257, 2048]))
    print(f"rope sweep seed={seed} M={M} q/k/v={n_q}/{n_k}/{n_v} d={d} K={K} B={B} Lmax={Lmax}", flush=True)
    N = (n_q + n_k + n_v) * d
    x = O.round_bf16(rng.standard_normal((M, K), dtype=np.float32))
    w = O.round_bf16(rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.05))
    b = O.round_bf16(rng.standard_normal(N, dtype=np.float32))
    pos = torch.from_numpy(rng.integers(0, Lmax, M).astype(np.int32)).cuda()
    batch = torch.from_numpy(rng.permutation(B)[:M].astype(np.int32)).cuda()
    xd, wd, bd = dev(x, "bf16"), dev(w, "bf16"), dev(b, "bf16")
    kc = torch.zeros(B, n_k, Lmax, d, device="cuda", dtype=torch.bfloat16)
    vc = torch.zeros(B, n_v, Lmax, d, device="cuda", dtype=torch.bfloat16)
    order = ops.rope_pair_order(n_q, n_k, n_v, d, device="cuda")
    wo = wd[order].contiguous()
    if seed % 3 == 0:
        wo = ops.pack_gemv_weight(wo)
    elif seed % 3 == 1 and M <= 8 and K % 64 == 0:
        wo = ops.pack_gemv_weight(wo, 8)
    table = ops.rope_table(pos, d, theta) if seed % 2 == 0 else None
    q = ops.gemv_rope_kv(xd, wo, bd[order].contiguous(), n_q, n_k, n_v, theta, pos, kc, vc, rms_eps=1e-6,
                         batch=batch, rope_table=table)
    torch.cuda.synchronize()
    xs = x.astype(np.float64)
    xs = xs / np.sqrt((xs ** 2).mean(-1, keepdims=True) + 1e-6)
    proj = (xs @ w.astype(np.float64).T + b).reshape(M, n_q + n_k + n_v, d)
    p = host(pos).astype(np.int64)
    assert rel_l2(host(q), O.rope(proj[:, :n_q], p[:, None], theta)) < 4e-3
    kh, vh, bt = host(kc), host(vc), host(batch).astype(np.int64)
    k_ref = O.rope(proj[:, n_q:n_q + n_k], p[:, None], theta)
    for m in range(M):
        assert rel_l2(kh[bt[m], :, p[m]], k_ref[m]) < 4e-3
        assert rel_l2(vh[bt[m], :, p[m]], proj[m, n_q + n_k:]) < 4e-3
    written = np.zeros((B, Lmax), bool)
    written[bt, p] = True
    assert not kh.transpose(0, 2, 1, 3)[~written].any() and not vh.transpose(0, 2, 1, 3)[~written].any()


@pytest.mark.parametrize("seed", range(4))
def test_small_decoder_step_sweep(seed):
    from saga_amd.decoder import DecoderShape, SagaDecoder
    rng = np.random.default_rng(150000 + seed)
    n_q, n_k, n_v = GROUPS[seed % len(GROUPS)]
    d = (64, 128)[seed % 2]
    hidden, inter = n_q * d, int(rng.choice([256, 1024, 2560]))
    vocab = (1024, 4099, 8192, 49152)[seed]
    layers, B = int(rng.integers(1, 4)), int(rng.integers(1, 5))
    max_len = int(rng.choice([64, 600]))
    plen = int(rng.integers(1, max_len - 1))
    print(f"decoder sweep seed={seed} L={layers} h={hidden} q/k/v={n_q}/{n_k}/{n_v} d={d} V={vocab} B={B} plen={plen}",
          flush=True)
    shape = DecoderShape(layers=layers, hidden=hidden, n_q=n_q, n_k=n_k, n_v=n_v, head_dim=d, intermediate=inter,
                         vocab=vocab, rope_theta=1e4, eps=1e-6, qkv_bias=bool(seed % 2))
    m = SagaDecoder(shape, batch=B, max_len=max_len, mode="dense", keep_source_weights=True)
    g = torch.Generator(device="cuda").manual_seed(seed)
    for t in m.ln1 + m.ln2 + [m.ln_f]:
        t.copy_((1 + 0.3 * torch.randn(t.shape, generator=g, device="cuda")).to(t.dtype))
    m.prepare_kernel_weights()
    m.fill_synthetic(plen)
    toks = rng.integers(0, vocab, B)
    m.tokens.copy_(torch.tensor(toks, device="cuda"))
    f = lambda t: t.detach().to(torch.float64).cpu().numpy()
    kc0, vc0 = f(m.k_cache), f(m.v_cache)
    m.step(calibrate=True)
    torch.cuda.synchronize()
    x = f(m.embed)[toks]
    for l in range(layers):
        h = O.rmsnorm(x, f(m.ln1[l]), shape.eps)
        qkv_ = (h @ f(m.w_qkv[l]).T + f(m.b_qkv[l])).reshape(B, n_q + n_k + n_v, d)
        q = O.rope(qkv_[:, :n_q], plen, shape.rope_theta)
        K, V = kc0[l][:, :, :plen + 1].copy(), vc0[l][:, :, :plen + 1].copy()
        K[:, :, plen] = O.rope(qkv_[:, n_q:n_q + n_k], plen, shape.rope_theta)
        V[:, :, plen] = qkv_[:, n_q + n_k:]
        x = x + O.dense(q[:, :, None, :], K, V).reshape(B, -1) @ f(m.w_o[l]).T
        h = O.rmsnorm(x, f(m.ln2[l]), shape.eps)
        x = x + O.silu_mul(h @ f(m.w_gu[l]).T) @ f(m.w_d[l]).T
    logits = O.rmsnorm(x, f(m.ln_f), shape.eps) @ f(m.lm_head).T
    assert rel_l2(f(m._logits), logits) < 3e-2
    for r in range(B):
        top2 = np.sort(logits[r])[-2:]
        if top2[1] - top2[0] > 0.05:
            assert int(m.tokens[r]) == int(np.argmax(logits[r]))
