"""Skinny GEMM (decode projections) and row argmax on the GPU vs float64."""
import numpy as np
import pytest
import torch

from conftest import rel_l2
from gpu_util import dev, host
from oracle import saga_oracle as O
from saga_amd import ops

pytestmark = pytest.mark.gpu

SHAPES = [(8, 1536, 1792), (8, 1536, 1536), (8, 1536, 17920), (8, 8960, 1536), (1, 960, 1344), (16, 1536, 4096),
          (3, 64, 32), (8, 2560, 960)]


def _data(rng, M, K, N):
    x = O.round_bf16(rng.standard_normal((M, K), dtype=np.float32))
    w = O.round_bf16(rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.05))
    b = O.round_bf16(rng.standard_normal(N, dtype=np.float32))
    return x, w, b


@pytest.mark.parametrize("M,K,N", SHAPES)
@pytest.mark.parametrize("rms", [False, True])
def test_gemv_store_and_bias(M, K, N, rms):
    rng = np.random.default_rng(M * K + N)
    x, w, b = _data(rng, M, K, N)
    y = host(ops.gemv(dev(x, "bf16"), dev(w, "bf16"), bias=dev(b, "bf16"), rms_eps=1e-6 if rms else None))
    xs = x.astype(np.float64)
    if rms:
        xs = xs / np.sqrt((xs ** 2).mean(-1, keepdims=True) + 1e-6)
    ref = xs @ w.astype(np.float64).T + b
    assert rel_l2(y, ref) < 4e-3


@pytest.mark.parametrize("M,K,N", SHAPES)
def test_gemv_add_in_place(M, K, N):
    rng = np.random.default_rng(M + K + N)
    x, w, _ = _data(rng, M, K, N)
    y0 = O.round_bf16(rng.standard_normal((M, N), dtype=np.float32))
    out = dev(y0, "bf16")
    ops.gemv(dev(x, "bf16"), dev(w, "bf16"), epilogue="add", out=out)
    ref = y0 + x.astype(np.float64) @ w.astype(np.float64).T
    assert rel_l2(host(out), ref) < 4e-3


@pytest.mark.parametrize("M,K,N", [(8, 1536, 17920), (1, 960, 5120), (4, 64, 64)])
def test_gemv_silu_pairs(M, K, N):
    rng = np.random.default_rng(7 + N)
    x, w, _ = _data(rng, M, K, N)
    y = host(ops.gemv(dev(x, "bf16"), dev(w, "bf16"), rms_eps=1e-5, epilogue="silu_pairs"))
    xs = x.astype(np.float64)
    xs = xs / np.sqrt((xs ** 2).mean(-1, keepdims=True) + 1e-5)
    full = xs @ w.astype(np.float64).T           # rows interleaved (gate_i, up_i)
    gu = np.concatenate([full[:, 0::2], full[:, 1::2]], axis=1)
    assert rel_l2(y, O.silu_mul(gu)) < 4e-3


def test_gemv_rejects_bad_shapes():
    x = torch.zeros(17, 64, device="cuda", dtype=torch.bfloat16)
    w = torch.zeros(32, 64, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="16 rows"):
        ops.gemv(x, w)
    with pytest.raises(RuntimeError, match="N % 16"):
        ops.gemv(x[:4], torch.zeros(20, 64, device="cuda", dtype=torch.bfloat16))


@pytest.mark.parametrize("N", [1, 1000, 151936])
def test_argmax_rows_first_max(N):
    rng = np.random.default_rng(N)
    x = O.round_bf16(rng.standard_normal((8, N), dtype=np.float32))
    if N > 10:
        x[3, 5] = x[3, N - 2] = 100.0  # tie: first index wins
    got = ops.argmax_rows(dev(x, "bf16")).cpu().numpy()
    np.testing.assert_array_equal(got, np.argmax(x, axis=1))
