"""saga_atopn_decode_noalloc through the C ABI: the Atop-N fast step on the
library's static per-GPU scratch, no workspace argument.  Its output must
equal saga_atopn_decode's (the same kernels on the same inputs) on
consecutive calls that reuse the scratch -- the second one smaller, with a
mask and ragged kv_len -- and a shape whose workspace exceeds the scratch is
refused before any launch."""
import ctypes

import numpy as np
import pytest
import torch

from gpu_util import qkv
from saga_amd import _lib

pytestmark = pytest.mark.gpu


def _decode(lib, fn, q, k, v, table, N, out, mask=None, kv_len=None, ws=None):
    stream = _lib.stream_of(q)
    args = [_lib.tensor(q), _lib.tensor(k), _lib.tensor(v), _lib.tensor(mask), _lib.ptr(kv_len), 1.0 / np.sqrt(q.shape[-1]),
            N, _lib.ptr(table), _lib.tensor(out)]
    if fn == "saga_atopn_decode":
        args += [_lib.ptr(ws), ws.numel()]
    rc = getattr(lib, fn)(*args, stream)
    return rc


def _case(seed, b, q_h, k_h, v_h, L, N, masked=False):
    rng = np.random.default_rng(seed)
    (_, _, _), (qd, kd, vd) = qkv(rng, b, q_h, k_h, v_h, 128, L, "bf16", outliers=0.01)
    table = torch.from_numpy(rng.uniform(1e-4, 2e-3, b * q_h).astype(np.float32)).cuda()
    mask = kv_len = None
    if masked:
        mask = torch.from_numpy(rng.random((b, 1, 1, L + 5)) < 0.9).cuda()
        kv_len = torch.from_numpy(rng.integers(1, L + 1, b).astype(np.int32)).cuda()
    return qd, kd, vd, table, mask, kv_len


def test_noalloc_equals_workspace_entry_point_on_consecutive_calls():
    lib = _lib.load()
    shapes = [(101, 8, 12, 1, 2, 8192, 512, False),   # then a smaller call reusing the scratch,
              (102, 2, 12, 1, 2, 3000, 64, True),     # with a bool mask and ragged kv_len,
              (103, 8, 12, 1, 2, 33024, 512, False)]  # then the 1.5B-shape decode at 32k positions
    for seed, b, q_h, k_h, v_h, L, N, masked in shapes:
        print(f"noalloc case seed={seed} b={b} L={L} N={N} masked={masked}", flush=True)
        qd, kd, vd, table, mask, kv_len = _case(seed, b, q_h, k_h, v_h, L, N, masked)
        out_na = torch.full((b, q_h, 1, 128), float("nan"), device="cuda", dtype=torch.float32)
        out_ws = torch.full_like(out_na, float("nan"))
        buf_k = min(2 * N, L)
        need = lib.saga_atopn_workspace_bytes(b, q_h, k_h, L, 128, buf_k)
        assert 0 < need <= _lib.NOALLOC_SCRATCH_BYTES
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        assert _decode(lib, "saga_atopn_decode_noalloc", qd, kd, vd, table, N, out_na, mask, kv_len) == 0, \
            lib.saga_last_error()
        assert _decode(lib, "saga_atopn_decode", qd, kd, vd, table, N, out_ws, mask, kv_len, ws) == 0, \
            lib.saga_last_error()
        torch.cuda.synchronize()
        assert torch.equal(torch.isnan(out_na), torch.isnan(out_ws))
        ok = ~torch.isnan(out_ws)
        assert ok.any()
        assert torch.equal(out_na[ok], out_ws[ok])


def test_noalloc_refuses_shapes_past_the_scratch():
    lib = _lib.load()
    b, q_h, k_h, v_h, L, N = 32, 12, 1, 2, 131072, 1024
    assert lib.saga_atopn_workspace_bytes(b, q_h, k_h, L, 128, 2 * N) > _lib.NOALLOC_SCRATCH_BYTES
    # descriptors only: refused before any device access, so no tensors are allocated
    q = torch.empty(b, q_h, 1, 128, device="cuda", dtype=torch.bfloat16)
    k = torch.empty(b, k_h, 1, 128, device="cuda", dtype=torch.bfloat16).expand(b, k_h, L, 128)
    v = torch.empty(b, v_h, 1, 128, device="cuda", dtype=torch.bfloat16).expand(b, v_h, L, 128)
    out = torch.empty(b, q_h, 1, 128, device="cuda", dtype=torch.bfloat16)
    table = torch.zeros(b * q_h, device="cuda")
    rc = _decode(lib, "saga_atopn_decode_noalloc", q, k, v, table, N, out)
    assert rc == -3 and b"static scratch" in lib.saga_last_error()


def test_noalloc_under_hip_graph_capture():
    """The entry point's purpose: calls inside a captured HIP graph, which
    cannot allocate.  The graph (two decode calls of different shapes) is
    replayed several times, with eager calls that reuse the scratch and
    in-place input changes between replays; every replay must equal the
    workspace entry point on the inputs of that moment."""
    lib = _lib.load()
    cases = [_case(201, 8, 12, 1, 2, 8192, 512), _case(202, 2, 12, 1, 2, 3000, 64, masked=True)]
    Ns = (512, 64)
    outs = [torch.empty(c[0].shape[0], 12, 1, 128, device="cuda", dtype=torch.float32) for c in cases]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # eager warm-up on the capture stream: the scratch address is looked up here
        for (qd, kd, vd, table, mask, kv_len), N, out in zip(cases, Ns, outs):
            assert _decode(lib, "saga_atopn_decode_noalloc", qd, kd, vd, table, N, out, mask, kv_len) == 0
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for (qd, kd, vd, table, mask, kv_len), N, out in zip(cases, Ns, outs):
            assert _decode(lib, "saga_atopn_decode_noalloc", qd, kd, vd, table, N, out, mask, kv_len) == 0, \
                lib.saga_last_error()
    other = _case(203, 4, 12, 1, 2, 20000, 256)
    other_out = torch.empty(4, 12, 1, 128, device="cuda", dtype=torch.float32)
    rng = np.random.default_rng(7)
    for rep in range(4):
        print(f"noalloc graph replay {rep}", flush=True)
        if rep >= 2:  # new queries in place: the replay must follow them
            for qd, *_ in cases:
                qd.copy_(torch.from_numpy(rng.standard_normal(tuple(qd.shape), dtype=np.float32)).to(qd.dtype).cuda())
        for o in outs:
            o.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for (qd, kd, vd, table, mask, kv_len), N, out in zip(cases, Ns, outs):
            b, L = qd.shape[0], kd.shape[2]
            ws = torch.empty(lib.saga_atopn_workspace_bytes(b, 12, 1, L, 128, min(2 * N, L)), dtype=torch.uint8,
                             device="cuda")
            ref = torch.full_like(out, float("nan"))
            assert _decode(lib, "saga_atopn_decode", qd, kd, vd, table, N, ref, mask, kv_len, ws) == 0
            torch.cuda.synchronize()
            assert torch.equal(torch.isnan(out), torch.isnan(ref))
            ok = ~torch.isnan(ref)
            assert ok.any() and torch.equal(out[ok], ref[ok]), rep
        # an eager call between replays overwrites the shared scratch
        qd, kd, vd, table, mask, kv_len = other
        assert _decode(lib, "saga_atopn_decode_noalloc", qd, kd, vd, table, 256, other_out) == 0
        torch.cuda.synchronize()
    del g
