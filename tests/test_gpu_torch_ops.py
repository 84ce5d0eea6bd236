"""The torch.library operators on the GPU: torch.library.opcheck (schema,
fake and real implementations agree) and torch.compile of the reference's
attention calls with fullgraph=True (no graph break at the kernels), equal to
eager execution."""
import numpy as np
import pytest
import torch

from gpu_util import qkv

pytestmark = pytest.mark.gpu


def _inputs():
    rng = np.random.default_rng(41)
    (_, _, _), (q, k, v) = qkv(rng, 2, 12, 1, 2, 128, 700, "bf16")
    return q, k, v


def test_opcheck_all_ops():
    import saga_amd.torch_ops  # noqa: F401
    q, k, v = _inputs()
    t = torch.full((24,), 1e-3, device="cuda")
    torch.library.opcheck(torch.ops.saga.atopn_decode, (q, k, v, t, 64))
    torch.library.opcheck(torch.ops.saga.atopn_calibrate, (q, k, v, t.clone(), 64))
    torch.library.opcheck(torch.ops.saga.dense_decode, (q, k, v))


def test_compiled_reference_api_equals_eager(monkeypatch):
    import attention.attention as A
    monkeypatch.setattr(A, "AMORTIZED_THRESHOLD_TENSOR", A.AMORTIZED_THRESHOLD_TENSOR)
    q, k, v = _inputs()
    A.init_amortized_threshold_tensor("cuda", A.MAX_LAYERS, 24)

    def step(q, k, v):
        cal = A.approx_top_n_attention_amortized_cal(q, k, v, top_n_attention=64, layer_idx=2)
        fast = A.approx_top_n_attention_amortized(q, k, v, top_n_attention=64, layer_idx=2)
        dense = A.full_einsum_forward(q, k, v)
        return cal, fast, dense

    eager = step(q, k, v)
    table_eager = A.AMORTIZED_THRESHOLD_TENSOR.clone()
    A.reset_amortized_state()
    compiled = torch.compile(step, backend="aot_eager", fullgraph=True)(q, k, v)
    torch.cuda.synchronize()
    for a, b in zip(eager, compiled):
        assert torch.equal(a, b)
    assert torch.equal(A.AMORTIZED_THRESHOLD_TENSOR, table_eager)
