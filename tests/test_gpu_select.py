"""Threshold selection on the GPU vs the oracle: bit-exact on identical inputs.

saga_threshold_select replaces the Triton kernel of
attention/triton_atopn.py:6-53 / threshold_topk_fast (:59-113).  On the same
x and thresholds the selected indices, their order (ascending), the values,
the per-row counts and the (-inf, 0) padding must be identical.
"""
import numpy as np
import pytest
import torch

from gpu_util import TORCH_DT, dev, host, round_to
from oracle import saga_oracle as O
from saga_amd import ops

pytestmark = pytest.mark.gpu


def _thresholds(x, rng):
    rows = x.shape[0]
    t = np.quantile(x, 0.97, axis=1).astype(np.float32)
    t[0] = x[0, rng.integers(0, x.shape[1])]      # an element equal to t: strict '>' excludes it
    if rows > 2:
        t[1] = -np.inf                              # everything passes (overflow when k < D)
        t[2] = np.inf                               # nothing passes
    if rows > 3:
        t[3] = np.quantile(x[3], 0.5)
    return t


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("D,k", [(1, 1), (7, 3), (1024, 64), (1025, 1025), (16384, 512), (16385, 16385),
                                 (40000, 1024), (131072, 2048)])
def test_select_matches_oracle_exactly(dt, D, k):
    print(f"select dt={dt} D={D} k={k}", flush=True)
    rng = np.random.default_rng(D * 7 + k)
    rows = 5
    x = round_to(rng.standard_normal((rows, D), dtype=np.float32), dt)
    t = _thresholds(x, rng)
    vals, idx, cnt = ops.threshold_select(dev(x, dt), k, torch.from_numpy(t).cuda(), with_counts=True)
    ov, oi, oc = O.threshold_select(x, k, t)
    np.testing.assert_array_equal(idx.cpu().numpy(), oi)
    np.testing.assert_array_equal(host(vals), ov)
    np.testing.assert_array_equal(cnt.cpu().numpy(), oc)
    assert vals.dtype == TORCH_DT[dt]


def test_select_threshold_broadcast_and_nan():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((6, 3000), dtype=np.float32)
    x[2, 100:110] = np.nan
    for thr in (np.array([0.5], np.float32), np.array([2.0, -0.5], np.float32),
                np.linspace(-1, 2, 6).astype(np.float32)):
        vals, idx, cnt = ops.threshold_select(dev(x), 256, torch.from_numpy(thr).cuda(), with_counts=True)
        ov, oi, oc = O.threshold_select(x, 256, thr)
        np.testing.assert_array_equal(idx.cpu().numpy(), oi)
        np.testing.assert_array_equal(cnt.cpu().numpy(), oc)


def test_select_is_deterministic_and_shapes_follow_input():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((2, 3, 1, 20000), dtype=np.float32)
    xt = dev(x)
    t = torch.full((6,), 1.5, device="cuda")
    v1, i1 = ops.threshold_select(xt, 1024, t)
    v2, i2 = ops.threshold_select(xt, 1024, t)
    assert v1.shape == (2, 3, 1, 1024) and i1.dtype == torch.int64
    assert torch.equal(i1, i2) and torch.equal(v1, v2)


def test_triton_atopn_api_caches_buffers():
    import attention.triton_atopn as T
    T._BUFFER_CACHE.clear()
    x = torch.randn(4, 1, 1, 5000, device="cuda", dtype=torch.bfloat16)
    thr = torch.zeros(4, device="cuda")
    v1, i1 = T.threshold_topk_fast(x, 300, thr)
    p1 = i1.data_ptr()
    v2, i2 = T.threshold_topk_fast(x, 300, thr)
    assert i2.data_ptr() == p1 and len(T._BUFFER_CACHE) == 1
    ov, oi, oc = O.threshold_select(host(x), 300, np.zeros(4, np.float32))
    np.testing.assert_array_equal(i2.cpu().numpy(), oi)
    np.testing.assert_array_equal(host(v2), ov)
