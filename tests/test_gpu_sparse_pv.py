"""Sparse softmax . V on the GPU vs the oracle.

saga_sparse_softmax_pv replaces _atopn_gather_and_output
(attention/attention.py:152-170): logits mode (softmax over the K-wide
buffer, -inf padding weighs 0, an all -inf row gives NaN) and probability
mode (renormalise with a 1e-12 floor).  fp32 output vs the float64 oracle.
"""
import numpy as np
import pytest
import torch

from gpu_util import dev, host, randn
from oracle import saga_oracle as O
from saga_amd import ops

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("b,q_h,v_h,d,L,K", [(1, 15, 5, 64, 4096, 256), (2, 12, 2, 128, 3000, 1024),
                                              (2, 6, 3, 128, 50, 7), (1, 4, 4, 64, 700, 129),
                                              (1, 12, 2, 128, 33024, 2048)])
@pytest.mark.parametrize("logits", [True, False])
def test_sparse_pv_matches_oracle(dt, b, q_h, v_h, d, L, K, logits):
    print(f"sparse_pv dt={dt} b={b} q_h={q_h} v_h={v_h} d={d} L={L} K={K} logits={logits}", flush=True)
    rng = np.random.default_rng(L + K)
    v, vd = randn(rng, (b, v_h, L, d), dt)
    idx = rng.integers(0, L, size=(b, q_h, 1, K)).astype(np.int64)
    if logits:
        w = (rng.standard_normal((b, q_h, 1, K)) * 2).astype(np.float32)
        w[0, 0, 0, K // 2:] = -np.inf  # padding
        if q_h > 1:
            w[0, 1, 0, :] = -np.inf    # nothing selected -> NaN row
    else:
        w = rng.random((b, q_h, 1, K)).astype(np.float32) * np.float32(0.01)
        w[0, 0, 0, 3:] = 0.0
    out = ops.sparse_softmax_pv(dev(w), torch.from_numpy(idx).cuda(), vd, (b, q_h, 1, d),
                                input_is_logits=logits, out_dtype=torch.float32)
    ref = O.gather_output(w.astype(np.float64), idx, v.astype(np.float64), (b, q_h, 1, d), input_is_logits=logits)
    got = host(out)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    np.testing.assert_allclose(got[ok], ref[ok], rtol=1e-5, atol=1e-6)


def test_sparse_pv_out_of_range_index_poisons_row():
    rng = np.random.default_rng(9)
    v, vd = randn(rng, (1, 2, 100, 128), "bf16")
    idx = np.zeros((1, 4, 1, 8), dtype=np.int64)
    idx[0, 2, 0, 5] = 100  # == L
    w = np.zeros((1, 4, 1, 8), dtype=np.float32)
    out = host(ops.sparse_softmax_pv(dev(w), torch.from_numpy(idx).cuda(), vd, (1, 4, 1, 128),
                                     input_is_logits=True, out_dtype=torch.float32))
    assert np.all(np.isnan(out[0, 2])) and not np.any(np.isnan(out[0, [0, 1, 3]]))
