"""torch.library registration of the decode kernels (CPU: schemas and fake
shapes; the GPU half is in test_gpu_torch_ops.py).  The reference compiles
its decode step (speedup.py:502-508), so the kernels must trace as graph
nodes; fake (meta) implementations give torch.compile the output shapes."""
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import saga_amd.torch_ops  # noqa: F401


def _fake_inputs(b=2, q_h=12, k_h=1, v_h=2, L=300, d=128):
    q = torch.empty(b, q_h, 1, d, dtype=torch.bfloat16, device="cuda")
    k = torch.empty(b, k_h, L, d, dtype=torch.bfloat16, device="cuda")
    v = torch.empty(b, v_h, L, d, dtype=torch.bfloat16, device="cuda")
    t = torch.empty(b * q_h, device="cuda")
    return q, k, v, t


def test_ops_are_registered_with_their_mutations():
    for name in ("atopn_decode", "atopn_calibrate", "dense_decode"):
        assert hasattr(torch.ops.saga, name)
    schema = torch.ops.saga.atopn_calibrate.default._schema
    mutated = [a.name for a in schema.arguments if a.alias_info is not None and a.alias_info.is_write]
    assert mutated == ["threshold_out"]
    for name in ("atopn_decode", "dense_decode"):
        s = getattr(torch.ops.saga, name).default._schema
        assert not any(a.alias_info is not None and a.alias_info.is_write for a in s.arguments)


def test_fake_implementations_give_the_output_shape():
    with FakeTensorMode():
        q, k, v, t = _fake_inputs()
        for out in (torch.ops.saga.atopn_decode(q, k, v, t, 64),
                    torch.ops.saga.atopn_calibrate(q, k, v, t, 64),
                    torch.ops.saga.dense_decode(q, k, v)):
            assert out.shape == (2, 12, 1, 128) and out.dtype == torch.bfloat16 and out.device.type == "cuda"
        q32, k32, v32, t32 = (x.float() if x.dtype == torch.bfloat16 else x for x in _fake_inputs(1, 15, 1, 5, 40, 64))
        assert torch.ops.saga.atopn_decode(q32, k32, v32, t32, 8).shape == (1, 15, 1, 64)
