"""Dense split-L decode on the GPU vs the oracle (full_einsum_forward,
attention/attention.py:64-85), including the dense-GQA comparator shape."""
import numpy as np
import pytest
import torch

from conftest import rel_l2
from gpu_util import host, qkv, randn
from oracle import saga_oracle as O
from saga_amd import ops

pytestmark = pytest.mark.gpu

SHAPES = [  # b, q_h, k_h, v_h, d, L
    (1, 15, 1, 5, 64, 4096),
    (2, 12, 1, 2, 128, 1000),
    (2, 12, 2, 2, 128, 777),
    (3, 6, 2, 3, 128, 257),
    (1, 8, 8, 8, 64, 40),
    (2, 12, 2, 1, 128, 300),
    (8, 12, 2, 2, 128, 33024),
    # one key head below batch 4: the query heads split over two units that
    # read the same key head (each half spanning two value heads; one each)
    (1, 12, 1, 4, 64, 5000),
    (3, 16, 1, 2, 128, 2500),
]


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", SHAPES)
def test_dense_matches_oracle(dt, shape):
    b, q_h, k_h, v_h, d, L = shape
    print(f"dense dt={dt} shape={shape}", flush=True)
    rng = np.random.default_rng(sum(shape) + 1)
    (q, k, v), (qd, kd, vd) = qkv(rng, b, q_h, k_h, v_h, d, L, dt, qscale=2.0)
    out32 = host(ops.dense_decode(qd, kd, vd, out_dtype=torch.float32))
    ref = O.dense(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64))
    assert rel_l2(out32, ref) < (1e-5 if dt == "f32" else 1e-4)
    if dt != "f32":
        out16 = host(ops.dense_decode(qd, kd, vd))
        assert np.max(np.abs(out16 - ref)) < 2e-2


def test_dense_with_masks():
    rng = np.random.default_rng(5)
    b, q_h, k_h, v_h, d, L = 2, 12, 1, 2, 128, 600
    (q, k, v), (qd, kd, vd) = qkv(rng, b, q_h, k_h, v_h, d, L, "bf16")
    valid = rng.random((b, 1, 1, L + 3)) > 0.3
    for m in (valid, np.where(valid, 0.0, -np.inf).astype(np.float32)):
        out = host(ops.dense_decode(qd, kd, vd, torch.from_numpy(m).cuda(), 0.1, out_dtype=torch.float32))
        ref = O.dense(q, k, v, m, 0.1)
        assert rel_l2(out, ref) < 1e-4


def test_workspace_reuse_across_shapes():
    """Calls of different shapes share one cached workspace; the arrival
    counters live in a fixed region, so a later call never sees stale data
    of an earlier layout (regression test)."""
    rng = np.random.default_rng(6)
    shapes = [(8, 12, 2, 2, 128, 20000), (2, 12, 1, 2, 128, 1000), (1, 15, 1, 5, 64, 4096), (2, 12, 1, 2, 128, 1000)]
    for shape in shapes:
        b, q_h, k_h, v_h, d, L = shape
        (q, k, v), (qd, kd, vd) = qkv(rng, b, q_h, k_h, v_h, d, L, "bf16")
        out = host(ops.dense_decode(qd, kd, vd, out_dtype=torch.float32))
        assert rel_l2(out, O.dense(q, k, v)) < 1e-4, shape
        table = torch.full((b * q_h,), 2e-4, device="cuda")
        fast = host(ops.atopn_decode(qd, kd, vd, table, 128, out_dtype=torch.float32))
        ref, _, _, _ = O.fast(q, k, v, host(table), None, 128, None)
        assert rel_l2(fast, ref) < 1e-3, shape


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("mask_kind", [None, "bool", "float"])
def test_full_einsum_forward_several_queries(dt, mask_kind):
    """full_einsum_forward with l_q > 1 (attention/attention.py:64-85): every
    query attends to all keys plus the mask (is_causal is ignored, as in the
    reference), query head h reading key head h // (q_h / k_h) and value
    head h // (q_h / v_h); a bool mask adds 1.0 where true."""
    from saga_amd.attention import attention as A
    rng = np.random.default_rng(17 + (mask_kind is not None))
    b, q_h, k_h, v_h, d, L, l_q = 3, 12, 1, 2, 128, 700, 5
    q, qd = randn(rng, (b, q_h, l_q, d), dt)
    (_, k, v), (_, kd, vd) = qkv(rng, b, q_h, k_h, v_h, d, L, dt)
    m = None
    if mask_kind == "bool":
        m = rng.random((b, 1, l_q, L + 4)) > 0.4
    elif mask_kind == "float":
        m = rng.standard_normal((1, q_h, l_q, L), dtype=np.float32)
    md = None if m is None else torch.from_numpy(m).cuda()
    out = A.full_einsum_forward(qd, kd, vd, md, is_causal=True, scaling=0.09)
    assert tuple(out.shape) == (b, q_h, l_q, d) and out.dtype == qd.dtype
    ref = O.dense(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64), m, 0.09)
    got = host(out)
    assert rel_l2(got, ref) < (1e-5 if dt == "f32" else 5e-3)
    if dt != "f32":
        assert np.max(np.abs(got - ref)) < 2e-2
