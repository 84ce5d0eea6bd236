"""QK scores, per-part partials and the logit threshold on the GPU vs the oracle.

saga_qk_scores replaces _compute_attn_weights (attention/attention.py:113-128),
saga_logit_threshold replaces _transform_softmax_threshold (:136-149).
The oracle runs in float64 on the same (dtype-representable) inputs; the
kernel accumulates in fp32, so the tolerance is relative to the largest
|q|.|k| * scale (fp32 rounding of a d-term dot product).
"""
import numpy as np
import pytest
import torch

from gpu_util import dev, host, qkv
from oracle import saga_oracle as O
from saga_amd import ops

pytestmark = pytest.mark.gpu

SHAPES = [  # b, q_h, k_h, v_h, d, L
    (1, 15, 1, 5, 64, 4096),
    (2, 12, 1, 2, 128, 1000),
    (3, 6, 2, 3, 128, 257),
    (2, 16, 1, 2, 128, 33),
    (1, 8, 8, 8, 64, 300),
    (1, 1, 1, 1, 128, 1),
]


def _mask(rng, kind, b, q_h, L):
    if kind is None:
        return None, None
    valid = rng.random((b, 1, 1, L + 5)) > 0.1
    if kind == "bool":
        return valid, torch.from_numpy(valid).cuda()
    m = np.where(valid, 0.0, -np.inf).astype(np.float32)
    m[..., 0] = 0.0
    return m, torch.from_numpy(m).cuda()


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("mask_kind", [None, "bool", "float"])
def test_scores_and_partials(dt, shape, mask_kind):
    b, q_h, k_h, v_h, d, L = shape
    print(f"scores dt={dt} shape={shape} mask={mask_kind}", flush=True)
    rng = np.random.default_rng(sum(shape))
    (q, k, _), (qd, kd, _) = qkv(rng, b, q_h, k_h, v_h, d, L, dt)
    m_np, m_t = _mask(rng, mask_kind, b, q_h, L)
    scale = 0.0883
    s, pm, ps = ops.qk_scores(qd, kd, m_t, scale, with_partials=True)
    ref = O.qk_scores(q.astype(np.float64), k.astype(np.float64), scale, m_np)
    got = host(s)
    tol = 2e-6 * d * float(np.abs(q).max() * np.abs(k).max() * scale) + 1e-6
    fin = np.isfinite(ref)
    np.testing.assert_array_equal(np.isfinite(got), fin)
    assert np.max(np.abs(got[fin] - ref[fin])) <= tol
    # partials are exact functions of the kernel's own scores
    x = got.reshape(b * q_h, L)
    T, nparts = (L + 15) // 16, pm.shape[1]
    pm, ps = host(pm), host(ps)
    for c in range(nparts):
        # part c: tiles [c*T/nparts, (c+1)*T/nparts) of 16 positions (4 K1 waves)
        t0, t1 = c * T // nparts, (c + 1) * T // nparts
        assert 0 <= t1 - t0 <= 24
        if t1 == t0:
            assert np.isneginf(pm[:, c]).all() and (ps[:, c] == 0).all()
            continue
        blk = x[:, 16 * t0:min(16 * t1, L)].astype(np.float64)
        mx = blk.max(axis=1)
        np.testing.assert_array_equal(pm[:, c], mx.astype(np.float32))
        with np.errstate(invalid="ignore"):
            sm = np.where(np.isneginf(mx), 0.0, np.exp(blk - mx[:, None]).sum(axis=1))
        np.testing.assert_allclose(ps[:, c], sm, rtol=2e-5)


@pytest.mark.parametrize("shape", SHAPES)
def test_kv_len_truncates(shape):
    b, q_h, k_h, v_h, d, L = shape
    rng = np.random.default_rng(7)
    (q, k, _), (qd, kd, _) = qkv(rng, b, q_h, k_h, v_h, d, L, "bf16")
    lens = rng.integers(1, L + 1, size=b).astype(np.int32)
    s = host(ops.qk_scores(qd, kd, None, None, kv_len=torch.from_numpy(lens).cuda()))
    full = host(ops.qk_scores(qd, kd))
    for i, n in enumerate(lens):
        np.testing.assert_array_equal(s[i, :, :, :n], full[i, :, :, :n])
        assert np.all(np.isneginf(s[i, :, :, n:]))


@pytest.mark.parametrize("L", [1, 100, 256, 257, 5000])
def test_logit_threshold_matches_oracle_on_same_scores(L):
    rng = np.random.default_rng(L)
    b, q_h = 2, 6
    x = rng.standard_normal((b, q_h, 1, L), dtype=np.float32) * np.float32(3)
    pstar = rng.random(b * q_h).astype(np.float32) * np.float32(0.01)
    pstar[0] = 0.0  # clamp to 1e-30
    t = host(ops.logit_threshold(dev(x), torch.from_numpy(pstar).cuda()))
    ref = O.logit_threshold(x.astype(np.float64), pstar.astype(np.float64))
    np.testing.assert_allclose(t, ref, rtol=2e-6, atol=2e-6)
