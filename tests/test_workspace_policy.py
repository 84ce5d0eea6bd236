"""The ops-level workspace cache's growth and retirement policy, on the CPU
(no device: the cache's replacement step is driven with a CPU allocator)."""
import torch

from saga_amd import ops
from saga_amd.decoder import QWEN25_15B_SAGA, DecoderShape, gemv_tile_rows


def _fresh():
    ops.clear_workspaces()


def test_growing_need_reallocates_logarithmically_and_frees_uncaptured():
    """A decode whose cache grows by 16 positions per step (the fast-step
    workspace of 8 rows x 12 heads x d128, 32k -> 36k positions): the old
    policy kept one dead buffer per growth (11 GB over 4096 tokens)."""
    _fresh()
    key = ("cpu", 0, "atopn")
    alloc = lambda n: torch.empty(n, dtype=torch.uint8)
    need0 = 40_000_000
    sizes = []
    for step in range(400):
        need = need0 + step * 16 * 12_000  # grows with L
        ws = ops._WORKSPACES.get(key)
        if ws is None or ws.numel() < need:
            ws = ops._replace(key, ws, need, alloc)
            sizes.append(ws.numel())
        assert ops._WORKSPACES[key].numel() >= need
    # 40 -> 60 -> 90 -> 135 MB for a final need of 117 MB (the old policy: 256 buffers)
    assert len(sizes) <= 4, sizes
    assert sizes[-1] < 1.5 * (need0 + 399 * 16 * 12_000)
    assert ops._RETIRED == []  # nothing was handed out under capture: every replaced buffer is freed
    _fresh()


def test_workspace_handed_out_under_capture_is_retired_not_freed():
    _fresh()
    key = ("cpu", 0, "atopn")
    alloc = lambda n: torch.empty(n, dtype=torch.uint8)
    a = ops._replace(key, None, 1000, alloc)
    ops._CAPTURED.add(key)  # what workspace() records when it hands `a` out during a capture
    b = ops._replace(key, a, 5000, alloc)
    assert ops._RETIRED == [a] and b.numel() >= 5000
    # b was not handed out under capture: replacing it frees it
    c = ops._replace(key, b, 9000, alloc)
    assert len(ops._RETIRED) == 1 and ops._RETIRED[0] is a and c.numel() >= 9000
    _fresh()
    assert ops._RETIRED == [] and ops._CAPTURED == set()


def test_grown_size():
    assert ops.grown_size(0, 10) == 256
    assert ops.grown_size(0, 1000) == 1000
    assert ops.grown_size(1000, 1001) == 1500
    assert ops.grown_size(1000, 4000) == 4000


def test_gemv_tile_rows_needs_every_k_a_multiple_of_64():
    assert gemv_tile_rows(QWEN25_15B_SAGA, 8) == 8
    assert gemv_tile_rows(QWEN25_15B_SAGA, 9) == 16
    # o_proj's K = n_q * head_dim = 9 * 96 = 864 = 32 (mod 64): 16-row tiles
    odd = DecoderShape(2, 1024, 9, 1, 3, 96, 2048, 1000, 1e4, 1e-6)
    assert (odd.n_q * odd.head_dim) % 64 == 32
    assert gemv_tile_rows(odd, 4) == 16
