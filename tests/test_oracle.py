"""Pins of the CPU oracle (oracle/saga_oracle.py).

Three kinds of checks, each chosen so that a plausible slip in the oracle
(wrong head mapping, >= instead of >, dropped mask, wrong tail, missing
clamp, unrenormalised probabilities) fails at least one of them:
  * golden vectors written by the reference's own functions
    (tests/golden/make_golden.py),
  * float64 closed forms / identities / library routines,
  * brute-force loops on tiny inputs,
plus planted mistakes that must be caught by those checks.
"""
import math

import numpy as np
import pytest
import torch

import cases
from conftest import rel_l2, set_diff_outside_band
from oracle import saga_oracle as O

ALL_CASES = list(cases.CASES)


def _inputs(name):
    inp = cases.make_inputs(name)
    return inp, cases.CASES[name]


@pytest.mark.parametrize("name", ALL_CASES)
def test_fixture_inputs_regenerate(name, golden):
    g = golden(name)
    inp, _ = _inputs(name)
    assert str(g["sha256"]) == cases.inputs_sha256(inp)


def _ref(g, key, bf16):
    return g[key + "_f32ref"] if bf16 else g[key]


@pytest.mark.parametrize("name", ALL_CASES)
def test_oracle_matches_reference_golden(name, golden):
    """Oracle fp32 path vs the reference's fp32 outputs on the same inputs."""
    g = golden(name)
    inp, c = _inputs(name)
    bf = c["bf16"]
    m = inp.get("mask")
    N, sc = c["N"], c["scaling"]

    full = O.dense(inp["q2"], inp["key"], inp["value"], m, sc)
    assert rel_l2(full, _ref(g, "full_out", bf)) < 1e-5

    out, thr, ik = O.calibrate(inp["q1"], inp["key"], inp["value"], m, N, sc)
    assert rel_l2(out, _ref(g, "cal_out", bf)) < 1e-5
    np.testing.assert_allclose(thr, _ref(g, "cal_threshold", bf), rtol=2e-6, atol=0)
    np.testing.assert_array_equal(np.sort(ik.reshape(thr.size, -1), axis=-1), _ref(g, "cal_idx_sorted", bf))

    L = inp["key"].shape[2]
    buf_k = min(2 * N, L)
    logits = O.qk_scores(inp["q2"], inp["key"], sc, m).reshape(thr.size, L)
    for tag, table in (("fast", _ref(g, "cal_threshold", bf)), ("zero", np.zeros_like(thr))):
        o, t, idx, cnt = O.fast(inp["q2"], inp["key"], inp["value"], table, m, N, sc)
        t_ref = _ref(g, f"{tag}_t", bf)
        fin = np.isfinite(t_ref)
        np.testing.assert_array_equal(np.isfinite(t), fin)
        np.testing.assert_allclose(t[fin], t_ref[fin], rtol=1e-6, atol=1e-6)
        idx_ref = _ref(g, f"{tag}_idx", bf)
        cnt_ref = _ref(g, f"{tag}_count", bf)
        idx2 = idx.reshape(thr.size, buf_k)
        for r in range(thr.size):
            band = 1e-5 * max(1.0, abs(float(t_ref[r]))) if fin[r] else 0.0
            sel = idx2[r, :min(cnt[r], buf_k)]
            sel_ref = idx_ref[r, :min(cnt_ref[r], buf_k)]
            if cnt[r] <= buf_k and cnt_ref[r] <= buf_k:
                assert not set_diff_outside_band(sel, sel_ref, logits[r], t_ref[r], band)
            else:  # overflow: ordered rule keeps the first buf_k by index
                np.testing.assert_array_equal(sel, sel_ref)
        o_ref = _ref(g, f"{tag}_out", bf)
        np.testing.assert_array_equal(np.isnan(o), np.isnan(o_ref))
        ok = ~np.isnan(o_ref)
        assert rel_l2(o[ok], o_ref[ok]) < 1e-5

    if "fast_logits" in g.files:
        assert rel_l2(O.qk_scores(inp["q2"], inp["key"], sc, m), g["fast_logits"]) < 1e-6


def test_reference_bf16_chain_is_far_from_fp32_path(golden):
    """Recorded behaviour of the reference: its own bf16 chain differs from
    its fp32 path by more than the 1e-3 rel-L2 bar (bf16 rounding of logits,
    exp-sums and probabilities).  The HIP kernels accumulate in fp32 and are
    held to the fp32 path instead."""
    g = golden("bf16")
    assert rel_l2(g["cal_out"], g["cal_out_f32ref"]) > 1e-2
    assert rel_l2(g["fast_out"], g["fast_out_f32ref"]) > 1e-2
    assert rel_l2(g["full_out"], g["full_out_f32ref"]) > 1e-3


# ---------------------------------------------------------------- closed forms

def _rand(rng, *shape):
    return rng.standard_normal(shape)


@pytest.mark.parametrize("q_h,k_h,v_h", [(6, 1, 2), (6, 2, 3), (6, 3, 1), (4, 4, 4)])
def test_qk_scores_brute_force(q_h, k_h, v_h):
    rng = np.random.default_rng(11)
    b, d, L = 2, 8, 13
    q = _rand(rng, b, q_h, 1, d)
    k = _rand(rng, b, k_h, L, d)
    mask = rng.standard_normal((b, 1, 1, L + 3))
    s = O.qk_scores(q, k, 0.37, mask)
    g = q_h // k_h
    for bi in range(b):
        for h in range(q_h):
            for l in range(L):
                ref = sum(q[bi, h, 0, j] * k[bi, h // g, l, j] for j in range(d)) * 0.37 + mask[bi, 0, 0, l]
                assert abs(s[bi, h, 0, l] - ref) < 1e-12


def test_qk_scores_bool_mask_adds_one():
    """torch adds a bool mask as 0/1 (attention/attention.py:124-126)."""
    rng = np.random.default_rng(12)
    q, k = _rand(rng, 1, 2, 1, 4), _rand(rng, 1, 1, 5, 4)
    mask = np.array([True, False, True, True, False, True])[None, None, None, :]
    plain = O.qk_scores(q, k, 1.0)
    masked = O.qk_scores(q, k, 1.0, mask)
    np.testing.assert_allclose(masked - plain, np.broadcast_to(mask[..., :5].astype(float), plain.shape))
    torch_sum = torch.from_numpy(plain) + torch.from_numpy(mask[..., :5].copy())
    np.testing.assert_allclose(masked, torch_sum.numpy())


def test_threshold_identity_float64():
    """{x > t} == {softmax(x) > p*} away from ties: the m of the transform cancels."""
    rng = np.random.default_rng(13)
    for L in (50, 256, 1000):
        x = rng.standard_normal((1, 3, 1, L)) * 3
        p = softmax64(x.reshape(3, L))
        pstar = np.sort(p, axis=-1)[:, -17] * 1.000001
        t = O.logit_threshold(x, pstar)
        for r in range(3):
            lhs = set(np.nonzero(x.reshape(3, L)[r] > t[r])[0])
            rhs = set(np.nonzero(p[r] > pstar[r])[0])
            assert lhs == rhs


def softmax64(x):
    e = np.exp(x - x.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


def test_threshold_tail_and_clamp():
    rng = np.random.default_rng(14)
    # L < 256: the tail is the whole row, so m = max and t = log(p*) + logsumexp(x)
    x = rng.standard_normal((1, 2, 1, 100))
    pstar = np.array([1e-3, 0.2])
    t = O.logit_threshold(x, pstar)
    lse = np.log(np.exp(x.reshape(2, 100)).sum(-1))
    np.testing.assert_allclose(t, np.log(pstar) + lse, rtol=1e-12)
    # L > 256 with the true max outside the tail: m is the tail max, t unchanged mathematically
    y = rng.standard_normal((1, 1, 1, 600))
    y[0, 0, 0, 10] = 9.0
    ty = O.logit_threshold(y, np.array([1e-2]))
    m_tail = y[0, 0, 0, -256:].max()
    s = np.exp(y.reshape(-1) - m_tail).sum()
    np.testing.assert_allclose(ty, m_tail + np.log(1e-2 * s), rtol=1e-12)
    # p* = 0 clamps to 1e-30
    t0 = O.logit_threshold(x, np.zeros(2))
    np.testing.assert_allclose(t0, np.log(1e-30) + lse, rtol=1e-12)


def test_threshold_select_brute_force_and_strict():
    rng = np.random.default_rng(15)
    x = rng.standard_normal((3, 40)).astype(np.float32)
    thr = np.array([0.1, x[1, 7], -5.0], dtype=np.float32)  # row 1: one element equals t
    vals, idx, cnt = O.threshold_select(x, 8, thr)
    for r in range(3):
        sel = [i for i in range(40) if x[r, i] > thr[r]]
        assert cnt[r] == len(sel)
        kept = sel[:8]
        assert list(idx[r, :len(kept)]) == kept
        assert np.all(idx[r, len(kept):] == 0) and np.all(np.isneginf(vals[r, len(kept):]))
        np.testing.assert_array_equal(vals[r, :len(kept)], x[r, kept])
    assert 7 not in set(idx[1, :min(cnt[1], 8)])  # equality is not selected


def test_threshold_select_broadcast_rules():
    """attention/triton_atopn.py:87-96: per row, scalar, repeated."""
    x = np.arange(24, dtype=np.float32).reshape(6, 4)
    _, _, c_row = O.threshold_select(x, 4, np.arange(6, dtype=np.float32) * 4 + 1)
    assert list(c_row) == [2] * 6
    _, _, c_sc = O.threshold_select(x, 4, np.array([10.0], dtype=np.float32))
    assert list(c_sc) == [0, 0, 1, 4, 4, 4]
    _, _, c_rep = O.threshold_select(x, 4, np.array([100.0, -1.0], dtype=np.float32))
    assert list(c_rep) == [0, 4, 0, 4, 0, 4]


def test_gather_output_brute_force():
    rng = np.random.default_rng(16)
    b, q_h, v_h, L, d, K = 2, 6, 3, 30, 5, 7
    v = rng.standard_normal((b, v_h, L, d))
    idx = rng.integers(0, L, size=(b, q_h, 1, K))
    w = rng.standard_normal((b, q_h, 1, K))
    w[0, 1, 0, 3:] = -np.inf  # padding
    out = O.gather_output(w, idx, v, (b, q_h, 1, d), input_is_logits=True)
    probs = np.abs(w)
    probs[np.isinf(probs)] = 0
    outp = O.gather_output(probs, idx, v, (b, q_h, 1, d), input_is_logits=False)
    g_v = q_h // v_h
    for bi in range(b):
        for h in range(q_h):
            ww = w[bi, h, 0]
            e = np.exp(ww - ww.max())
            p = e / e.sum()
            ref = sum(p[j] * v[bi, h // g_v, idx[bi, h, 0, j]] for j in range(K))
            np.testing.assert_allclose(out[bi, h, 0], ref, rtol=1e-12)
            pp = probs[bi, h, 0] / max(probs[bi, h, 0].sum(), 1e-12)
            refp = sum(pp[j] * v[bi, h // g_v, idx[bi, h, 0, j]] for j in range(K))
            np.testing.assert_allclose(outp[bi, h, 0], refp, rtol=1e-12)
    w[1, 2, 0, :] = -np.inf
    out_nan = O.gather_output(w, idx, v, (b, q_h, 1, d), input_is_logits=True)
    assert np.all(np.isnan(out_nan[1, 2])) and not np.any(np.isnan(out_nan[0]))


def test_calibrate_brute_force():
    rng = np.random.default_rng(17)
    b, q_h, k_h, v_h, L, d, N = 1, 4, 1, 2, 64, 8, 10
    q, k, v = _rand(rng, b, q_h, 1, d), _rand(rng, b, k_h, L, d), _rand(rng, b, v_h, L, d)
    out, thr, ik = O.calibrate(q, k, v, None, N, None)
    logits = O.qk_scores(q, k).reshape(q_h, L)
    for h in range(q_h):
        p = softmax64(logits[h])
        order = sorted(range(L), key=lambda i: -p[i])[:N]
        assert thr[h] == pytest.approx(sorted(p)[-N], rel=1e-12)
        assert set(ik[0, h, 0]) == set(order)
        ref = sum(p[i] * v[0, h // (q_h // v_h), i] for i in order) / sum(p[i] for i in order)
        np.testing.assert_allclose(out[0, h, 0], ref, rtol=1e-12)


@pytest.mark.parametrize("q_h,k_h,v_h", [(6, 1, 2), (6, 2, 3), (4, 4, 4), (15, 1, 5)])
def test_dense_matches_torch_sdpa(q_h, k_h, v_h):
    rng = np.random.default_rng(18)
    b, d, L = 2, 16, 37
    q, k, v = _rand(rng, b, q_h, 1, d), _rand(rng, b, k_h, L, d), _rand(rng, b, v_h, L, d)
    mask = np.where(rng.random((b, 1, 1, L)) < 0.2, -np.inf, 0.0)
    mask[:, :, :, 0] = 0.0
    ours = O.dense(q, k, v, mask, 0.3)
    tq = torch.from_numpy(q)
    tk = torch.from_numpy(k).repeat_interleave(q_h // k_h, dim=1)
    tv = torch.from_numpy(v).repeat_interleave(q_h // v_h, dim=1)
    ref = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, attn_mask=torch.from_numpy(mask), scale=0.3)
    np.testing.assert_allclose(ours, ref.numpy(), rtol=1e-10, atol=1e-12)


def test_fast_path_recovers_calibration_set_float64():
    """With the query of the calibration step, t equals the k-th largest logit
    mathematically, so the fast step selects the top-(k-1) or, when rounding
    puts t just below that logit, the top-k."""
    rng = np.random.default_rng(19)
    q, k, v = _rand(rng, 1, 3, 1, 16), _rand(rng, 1, 1, 300, 16), _rand(rng, 1, 3, 300, 16)
    N = 20
    _, thr, ik = O.calibrate(q, k, v, None, N, None)
    _, _, idx, cnt = O.fast(q, k, v, thr, None, N, None)
    for h in range(3):
        n = int(cnt[h])
        assert n in (N - 1, N)
        top = [int(i) for i in ik[0, h, 0, :n]]
        assert sorted(top) == list(idx[0, h, 0, :n])


def test_kv_len_truncation_definition():
    rng = np.random.default_rng(20)
    k, v = _rand(rng, 2, 1, 50, 4), _rand(rng, 2, 2, 50, 4)
    parts = O.truncate_kv(k, v, [30, 50])
    assert parts[0][0].shape == (1, 1, 30, 4) and parts[1][1].shape == (1, 2, 50, 4)


# ----------------------------------------------------------- planted mistakes

def test_planted_head_mapping_mistake_is_caught(golden):
    """Using value head h % v_h instead of h // (q_h / v_h) must break the golden check."""
    g = golden("float_mask")
    inp, c = _inputs("float_mask")
    orig = O._value_rows

    def wrong(value, q_h, idx):
        b, v_h = value.shape[0], value.shape[1]
        vh = np.arange(q_h) % v_h
        return value[np.arange(b)[:, None, None], vh[None, :, None], idx]

    O._value_rows = wrong
    try:
        out, _, _ = O.calibrate(inp["q1"], inp["key"], inp["value"], inp["mask"], c["N"], c["scaling"])
    finally:
        O._value_rows = orig
    assert rel_l2(out, g["cal_out"]) > 1e-2


def test_planted_non_strict_compare_is_caught():
    x = np.array([[1.0, 2.0, 3.0]], dtype=np.float32)
    _, _, cnt = O.threshold_select(x, 3, np.array([2.0], dtype=np.float32))
    assert cnt[0] == 1                       # strict
    assert int((x >= 2.0).sum()) == 2        # a '>=' oracle would report 2


def test_planted_missing_mask_is_caught(golden):
    g = golden("bool_mask")
    inp, c = _inputs("bool_mask")
    out_no_mask = O.dense(inp["q2"], inp["key"], inp["value"], None, c["scaling"])
    assert rel_l2(out_no_mask, g["full_out"]) > 1e-3


def test_planted_tail_mistake_is_caught(golden):
    """Taking the max over the whole row instead of the last 256 logits
    changes t where the true max lies outside the tail (inf case)."""
    g = golden("inf_threshold")
    inp, c = _inputs("inf_threshold")
    logits = O.qk_scores(inp["q2"], inp["key"], c["scaling"])
    x = logits.reshape(-1, logits.shape[-1])
    m_full = x.max(-1)
    with np.errstate(over="ignore"):
        t_full = m_full + np.log(np.maximum(g["cal_threshold"], 1e-30) * np.exp(x - m_full[:, None]).sum(-1))
    assert np.isinf(g["fast_t"][0]) and np.isfinite(t_full[0])


def test_planted_unrenormalised_probs_is_caught(golden):
    g = golden("c1")
    inp, c = _inputs("c1")
    probs = O.softmax(O.qk_scores(inp["q1"], inp["key"], None), axis=-1)
    pk, ik = O.topk_desc(probs, c["N"])
    rows = O._value_rows(inp["value"], 15, ik.reshape(1, 15, -1))
    raw = np.matmul(pk.reshape(1, 15, 1, -1), rows).reshape(g["cal_out"].shape)
    assert rel_l2(raw, g["cal_out"]) > 1e-2


# ------------------------------------------------------- decode-step op pins

def test_rope_is_a_rotation_with_the_hf_frequencies():
    rng = np.random.default_rng(30)
    d, theta = 8, 1e4
    x = rng.standard_normal((3, d))
    pos = np.array([0, 1, 37])
    y = O.rope(x, pos, theta)
    np.testing.assert_allclose(y[0], x[0])                      # position 0: identity
    np.testing.assert_allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1))  # rotation
    inv = 1.0 / theta ** (np.arange(0, d, 2) / d)
    for n, p in enumerate(pos):                                 # brute force per pair (i, i + d/2)
        for i in range(d // 2):
            a = p * inv[i]
            assert abs(y[n, i] - (x[n, i] * math.cos(a) - x[n, i + d // 2] * math.sin(a))) < 1e-5
            assert abs(y[n, i + d // 2] - (x[n, i + d // 2] * math.cos(a) + x[n, i] * math.sin(a))) < 1e-5
    # relative-position property of rotate-half RoPE: <R(p)q, R(p+k)k'> depends only on k
    q, k = rng.standard_normal(d), rng.standard_normal(d)
    dots = [float(O.rope(q, p, theta) @ O.rope(k, p + 5, theta)) for p in (0, 3, 11)]
    np.testing.assert_allclose(dots, dots[0], rtol=1e-5)


def test_rmsnorm_and_silu_mul_closed_forms():
    rng = np.random.default_rng(31)
    x = rng.standard_normal((2, 6))
    w = rng.standard_normal(6)
    y = O.rmsnorm(x, w, 1e-6)
    np.testing.assert_allclose(((y / w) ** 2).mean(axis=-1), 1.0, rtol=1e-5)
    gu = rng.standard_normal((2, 8))
    ref = [[gu[n, i] * (1 / (1 + math.exp(-gu[n, i]))) * gu[n, 4 + i] for i in range(4)] for n in range(2)]
    np.testing.assert_allclose(O.silu_mul(gu), ref)
    t = torch.from_numpy(gu[:, :4])
    np.testing.assert_allclose(O.silu_mul(gu), (torch.nn.functional.silu(t) * torch.from_numpy(gu[:, 4:])).numpy())


def _sdpa_expanded(q, k, v, mask, scale, is_causal):
    """torch's own SDPA (float64, CPU) over repeat_interleave-expanded heads,
    [b, l_q, q_h, d]."""
    q_h = q.shape[1]
    tk = torch.from_numpy(k).repeat_interleave(q_h // k.shape[1], dim=1)
    tv = torch.from_numpy(v).repeat_interleave(q_h // v.shape[1], dim=1)
    tm = None if mask is None else torch.from_numpy(mask)
    out = torch.nn.functional.scaled_dot_product_attention(torch.from_numpy(q), tk, tv, attn_mask=tm, scale=scale,
                                                           is_causal=is_causal)
    return out.transpose(1, 2).numpy()


@pytest.mark.parametrize("q_h,k_h,v_h", [(6, 1, 2), (6, 2, 3), (4, 4, 4), (15, 1, 5)])
@pytest.mark.parametrize("kind", ["causal", "full", "bool", "float", "causal_short_q", "masked_row"])
def test_prefill_matches_torch_sdpa(q_h, k_h, v_h, kind):
    rng = np.random.default_rng(31)
    b, d = 2, 16
    Lq, Lk = (5, 37) if kind == "causal_short_q" else (37, 37)
    q, k, v = _rand(rng, b, q_h, Lq, d), _rand(rng, b, k_h, Lk, d), _rand(rng, b, v_h, Lk, d)
    mask, causal = None, kind.startswith("causal")
    if kind in ("bool", "masked_row"):
        mask = rng.random((b, 1, Lq, Lk + 3)) < 0.7  # wider than Lk: cut by the function (:28-30)
        mask[..., 0] = True
        if kind == "masked_row":
            mask[1, 0, 4] = False  # a query that sees no key
    elif kind == "float":
        mask = np.where(rng.random((b, q_h, Lq, Lk)) < 0.3, -np.inf, rng.standard_normal((b, q_h, Lq, Lk)))
        mask[..., 0] = 0.0
    ours = O.prefill(q, k, v, mask, 0.3, causal)
    ref = _sdpa_expanded(q, k, v, None if mask is None else mask[..., :Lk], 0.3, causal)
    assert ours.shape == (b, Lq, q_h, d)
    np.testing.assert_allclose(ours, ref, rtol=1e-10, atol=1e-12)
    if kind == "masked_row":
        assert not ours[1, 4].any()


def test_prefill_default_causal_rule():
    """is_causal None: causal for l_q > 1 without a mask (attention/attention.py:36-37)."""
    rng = np.random.default_rng(32)
    q, k, v = _rand(rng, 1, 2, 6, 8), _rand(rng, 1, 1, 6, 8), _rand(rng, 1, 2, 6, 8)
    np.testing.assert_array_equal(O.prefill(q, k, v), O.prefill(q, k, v, is_causal=True))
    assert not np.allclose(O.prefill(q, k, v), O.prefill(q, k, v, is_causal=False))
    one = O.prefill(q[:, :, :1], k, v)  # l_q == 1: not causal
    np.testing.assert_array_equal(one, O.prefill(q[:, :, :1], k, v, is_causal=False))


def test_prefill_causality_and_single_key():
    """Causal output at query i does not depend on keys / values after i;
    query 0 of a causal call sees one key, so its output is that value row of
    its value head."""
    rng = np.random.default_rng(33)
    q, k, v = _rand(rng, 1, 6, 20, 8), _rand(rng, 1, 1, 20, 8), _rand(rng, 1, 3, 20, 8)
    out = O.prefill(q, k, v, is_causal=True)
    k2, v2 = k.copy(), v.copy()
    k2[:, :, 11:] = rng.standard_normal(k2[:, :, 11:].shape)
    v2[:, :, 11:] = rng.standard_normal(v2[:, :, 11:].shape)
    out2 = O.prefill(q, k2, v2, is_causal=True)
    np.testing.assert_array_equal(out[:, :11], out2[:, :11])
    assert not np.allclose(out[:, 11:], out2[:, 11:])
    for h in range(6):
        np.testing.assert_allclose(out[0, 0, h], v[0, h // 2, 0], rtol=1e-12)
