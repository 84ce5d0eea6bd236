"""KV-cache layout and capacity planning (CPU)."""
import pytest
import torch

from saga_amd.decoder import QWEN25_15B_SAGA, QWEN25_15B_GQA, DecoderShape
from saga_amd.kv_cache import HBM_BYTES_MI355X, KVCache, decode_weight_bytes, kv_cache_bytes, plan_capacity


def test_cache_bytes_headline_shape():
    # 28 layers x 8 rows x (1 + 2) heads x 33024 positions x 128 x 2 B
    assert kv_cache_bytes(QWEN25_15B_SAGA, 8, 33024) == 28 * 8 * 3 * 33024 * 128 * 2
    # the dense-GQA comparator holds 4 heads: 4/3 of the SAGA cache
    assert kv_cache_bytes(QWEN25_15B_GQA, 8, 33024) * 3 == kv_cache_bytes(QWEN25_15B_SAGA, 8, 33024) * 4


def test_weight_bytes_count_every_matrix():
    s = QWEN25_15B_SAGA
    base = decode_weight_bytes(s, decode_copies=False)
    # tied embedding 151936 x 1536 and 28 layers of q/k/v, o, gate/up, down
    per_layer = 1920 * 1536 + 1920 + 1536 * 1536 + 2 * 8960 * 1536 + 1536 * 8960 + 2 * 1536
    assert base == 2 * (151936 * 1536 + 28 * per_layer + 1536)
    assert decode_weight_bytes(s) > base


def test_plan_capacity_is_the_largest_fit():
    s = QWEN25_15B_SAGA
    plan = plan_capacity(s, batch=8, budget_bytes=HBM_BYTES_MI355X)
    assert plan.total_bytes <= HBM_BYTES_MI355X * 0.95
    # 28 layers x 8 rows x 3 heads x 256 B = 172 KB per position: ~1.5M positions at batch 8
    assert plan.max_len % 256 == 0 and 1_400_000 < plan.max_len < 1_700_000
    # 256 more positions no longer fit (the workspaces only grow with the context)
    more = kv_cache_bytes(s, 8, plan.max_len + 256) + plan.weight_bytes + plan.workspace_bytes
    assert more > HBM_BYTES_MI355X * 0.95
    bplan = plan_capacity(s, max_len=131072, budget_bytes=HBM_BYTES_MI355X)
    assert 85 <= bplan.batch <= 100 and bplan.total_bytes <= HBM_BYTES_MI355X * 0.95
    assert "GB" in str(bplan)
    with pytest.raises(ValueError):
        plan_capacity(s, batch=8, max_len=1024)
    tiny = DecoderShape(2, 64, 4, 1, 2, 64, 128, 256, 1e4, 1e-6)
    with pytest.raises(MemoryError):
        plan_capacity(QWEN25_15B_SAGA, batch=1, budget_bytes=10**9)
    assert plan_capacity(tiny, batch=1, budget_bytes=10**8).max_len > 0


def test_kv_cache_layer_views_are_the_reference_layout():
    tiny = DecoderShape(3, 64, 4, 1, 2, 64, 128, 256, 1e4, 1e-6)
    kv = KVCache(tiny, batch=2, max_len=40, device="cpu")
    k, v = kv.layer(1)
    assert k.shape == (2, 1, 40, 64) and v.shape == (2, 2, 40, 64)
    assert k.is_contiguous() and v.is_contiguous()
    assert kv.nbytes == kv_cache_bytes(tiny, 2, 40)
    assert k.data_ptr() == kv.k.data_ptr() + 1 * 2 * 1 * 40 * 64 * 2
