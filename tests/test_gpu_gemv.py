"""Skinny GEMM (decode projections) and row argmax on the GPU vs float64."""
import numpy as np
import pytest
import torch

from conftest import rel_l2
from gpu_util import dev, host
from oracle import saga_oracle as O
from saga_amd import _lib, ops

pytestmark = pytest.mark.gpu

SHAPES = [(8, 1536, 1792), (8, 1536, 1536), (8, 1536, 17920), (8, 8960, 1536), (1, 960, 1344), (16, 1536, 4096),
          (32, 1536, 1920), (17, 8960, 1536), (24, 4096, 64), (32, 64, 32),
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


@pytest.mark.parametrize("M,K,N", [(8, 1536, 17920), (1, 960, 5120), (4, 64, 64), (32, 1536, 17920)])
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
    x = torch.zeros(33, 64, device="cuda", dtype=torch.bfloat16)
    w = torch.zeros(32, 64, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="32 rows"):
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


@pytest.mark.parametrize("M,K,n_q,n_k,n_v,d", [(8, 1536, 12, 1, 2, 128), (1, 960, 15, 1, 5, 64), (16, 512, 4, 2, 2, 64),
                                             (32, 1536, 12, 1, 2, 128), (19, 960, 15, 1, 5, 64)])
def test_gemv_rope_kv_matches_unfused(M, K, n_q, n_k, n_v, d):
    """Projection + RoPE + cache append in one launch == gemv then
    rope_kv_append (the projection is rounded to bf16 before the rotation in
    both), and both match the oracle's RoPE of the float64 projection."""
    rng = np.random.default_rng(M * 7 + K)
    N = (n_q + n_k + n_v) * d
    x, w, b = _data(rng, M, K, N)
    B, Lmax = max(16, M), 2048
    pos = torch.from_numpy(rng.integers(0, Lmax, M).astype(np.int32)).cuda()
    batch = torch.from_numpy(rng.permutation(B)[:M].astype(np.int32)).cuda()
    xd, wd, bd = dev(x, "bf16"), dev(w, "bf16"), dev(b, "bf16")
    caches = [torch.zeros(B, h, Lmax, d, device="cuda", dtype=torch.bfloat16) for h in (n_k, n_v, n_k, n_v)]
    qkv = ops.gemv(xd, wd, bias=bd, rms_eps=1e-6)
    q_ref = ops.rope_kv_append(qkv, n_q, n_k, n_v, 1e6, pos, caches[0], caches[1], batch=batch)
    order = ops.rope_pair_order(n_q, n_k, n_v, d, device="cuda")
    q = ops.gemv_rope_kv(xd, wd[order].contiguous(), bd[order].contiguous(), n_q, n_k, n_v, 1e6, pos,
                         caches[2], caches[3], rms_eps=1e-6, batch=batch)
    torch.cuda.synchronize()
    for a, r in ((q, q_ref), (caches[2], caches[0]), (caches[3], caches[1])):
        assert torch.allclose(a.float(), r.float(), rtol=2 ** -7, atol=1e-6)
    # against the oracle: float64 projection, RoPE in float64
    xs = x.astype(np.float64)
    xs = xs / np.sqrt((xs ** 2).mean(-1, keepdims=True) + 1e-6)
    proj = (xs @ w.astype(np.float64).T + b).reshape(M, n_q + n_k + n_v, d)
    p = host(pos).astype(np.int64)
    assert rel_l2(host(q), O.rope(proj[:, :n_q], p[:, None], 1e6)) < 4e-3
    kh, vh, bt = host(caches[2]), host(caches[3]), host(batch).astype(np.int64)
    k_ref = O.rope(proj[:, n_q:n_q + n_k], p[:, None], 1e6)
    for m in range(M):
        assert rel_l2(kh[bt[m], :, p[m]], k_ref[m]) < 4e-3
        assert rel_l2(vh[bt[m], :, p[m]], proj[m, n_q + n_k:]) < 4e-3


@pytest.mark.parametrize("d,theta", [(128, 1e6), (64, 1e5)])
def test_rope_table_against_float64(d, theta):
    """table[n, i] = (cos, sin) of the fp32 angle pos[n] * theta^(-2i/d)
    (transformers computes the angle in fp32 the same way), against float64
    cos / sin of that angle: positions 0 .. 131071 and a negative one."""
    pos = np.array([0, 1, 7, 4095, 32767, 32768, 65536 + 3, 131071, -5], dtype=np.int32)
    got = host(ops.rope_table(torch.from_numpy(pos).cuda(), d, theta))
    assert got.shape == (pos.size, d // 2, 2)
    inv = (1.0 / np.power(np.float32(theta), np.arange(0, d, 2, dtype=np.float32) / np.float32(d))).astype(np.float32)
    ang = (pos[:, None].astype(np.float32) * inv[None, :]).astype(np.float64)
    # the angles of pos <= 2^17 are within 2^-7 rad of representable: a one-ulp
    # difference in theta^(-2i/d) moves them by at most 2^17 * 2^-24 = 2^-7
    tol = 2.0 ** -7 + 1e-6
    np.testing.assert_allclose(got[..., 0], np.cos(ang), atol=tol)
    np.testing.assert_allclose(got[..., 1], np.sin(ang), atol=tol)
    small = np.abs(pos) <= 64  # angles below 64 rad: no room for the ulp argument
    np.testing.assert_allclose(got[small, :, 0], np.cos(ang[small]), atol=2e-6)
    np.testing.assert_allclose(got[small, :, 1], np.sin(ang[small]), atol=2e-6)


@pytest.mark.parametrize("M,K,n_q,n_k,n_v,d", [(8, 1536, 12, 1, 2, 128), (1, 960, 15, 1, 5, 64), (32, 1536, 12, 1, 2, 128)])
def test_gemv_rope_kv_with_table_identical(M, K, n_q, n_k, n_v, d):
    """The fused projection with the step's rotation table (computed once for
    all layers) writes the same bits as with the rotations computed in its
    epilogue; positions past 32k included."""
    rng = np.random.default_rng(M * 13 + K)
    N = (n_q + n_k + n_v) * d
    x, w, b = _data(rng, M, K, N)
    B, Lmax = max(16, M), 40000
    pos = torch.from_numpy(rng.integers(0, Lmax, M).astype(np.int32)).cuda()
    pos[0] = Lmax - 1
    batch = torch.from_numpy(rng.permutation(B)[:M].astype(np.int32)).cuda()
    order = ops.rope_pair_order(n_q, n_k, n_v, d, device="cuda")
    wd, bd = dev(w, "bf16")[order].contiguous(), dev(b, "bf16")[order].contiguous()
    xd = dev(x, "bf16")
    table = ops.rope_table(pos, d, 1e6)
    outs = []
    for tab in (None, table):
        caches = [torch.zeros(B, h, Lmax, d, device="cuda", dtype=torch.bfloat16) for h in (n_k, n_v)]
        q = ops.gemv_rope_kv(xd, wd, bd, n_q, n_k, n_v, 1e6, pos, caches[0], caches[1], rms_eps=1e-6, batch=batch,
                             rope_table=tab)
        torch.cuda.synchronize()
        outs.append([q] + caches)
    for a, r in zip(outs[0], outs[1]):
        assert torch.equal(a.view(torch.int16), r.view(torch.int16))
    with pytest.raises(ValueError, match="rope_table"):
        ops.gemv_rope_kv(xd, wd, bd, n_q, n_k, n_v, 1e6, pos, caches[0], caches[1], rms_eps=1e-6, batch=batch,
                         rope_table=table[:, :-1].contiguous())


def test_rope_pair_order_is_a_permutation():
    order = ops.rope_pair_order(3, 1, 2, 8)
    assert sorted(order.tolist()) == list(range(6 * 8))
    assert order[:8].tolist() == [0, 4, 1, 5, 2, 6, 3, 7] and order[32:].tolist() == list(range(32, 48))


@pytest.mark.parametrize("M", [8, 32, 23])
@pytest.mark.parametrize("epilogue", ["store", "add", "silu_pairs"])
@pytest.mark.parametrize("rms", [False, True])
def test_gemv_split_k_matches_single_pass_and_is_deterministic(M, epilogue, rms):
    """Long rows with few tiles (the down projection shape) go through the
    split-K path; it agrees with the one-workgroup-per-tile path and repeats
    bit for bit."""
    rng = np.random.default_rng(77 + M)
    K, N = 8960, 1536
    x, w, _ = _data(rng, M, K, N)
    xd, wd = dev(x, "bf16"), dev(w, "bf16")
    assert _lib.load().saga_gemv_workspace_bytes(M, N, K) > 0
    y0 = dev(O.round_bf16(rng.standard_normal((M, N // 2 if epilogue == "silu_pairs" else N), dtype=np.float32)),
             "bf16")
    outs = []
    for split in (False, True, True):
        y = y0.clone()
        outs.append(ops.gemv(xd, wd, rms_eps=1e-6 if rms else None, epilogue=epilogue, out=y, split_k=split))
    torch.cuda.synchronize()
    assert torch.equal(outs[1], outs[2])
    assert torch.allclose(outs[0].float(), outs[1].float(), rtol=2 ** -7, atol=2e-3)


# (5, 32, 64): one 32-column block, whose size-1 dim keeps torch's stride
@pytest.mark.parametrize("M,K,N", [(8, 1536, 1920), (8, 1536, 17920), (8, 8960, 1536), (3, 64, 32), (8, 1536, 151936),
                                   (5, 32, 64), (32, 1536, 1920), (29, 8960, 1536), (32, 1536, 151936)])
@pytest.mark.parametrize("epilogue", ["store", "add", "silu_pairs"])
def test_packed_weights_give_identical_results(M, K, N, epilogue):
    """W in the packed MFMA-fragment layout [N/16, K/32, 16, 32] feeds the same
    fragments in the same order: every epilogue (and the split-K path of
    the long-row shape) returns bit-identical outputs."""
    rng = np.random.default_rng(M * 7 + N)
    x, w, b = _data(rng, M, K, N)
    xd, wd = dev(x, "bf16"), dev(w, "bf16")
    wp = ops.pack_gemv_weight(wd)
    assert wp.shape == (N // 16, K // 32, 16, 32)
    # the packing is the fragment order: fragment (t, j) = rows 16t.., columns 32j..
    assert torch.equal(wp[1, 2], wd[16:32, 64:96]) if N >= 32 and K >= 96 else True
    y0 = dev(O.round_bf16(rng.standard_normal((M, N // 2 if epilogue == "silu_pairs" else N), dtype=np.float32)),
             "bf16")
    bias = dev(b, "bf16") if epilogue == "store" else None
    for rms in (None, 1e-6):
        ya = ops.gemv(xd, wd, bias=bias, rms_eps=rms, epilogue=epilogue, out=y0.clone())
        yb = ops.gemv(xd, wp, bias=bias, rms_eps=rms, epilogue=epilogue, out=y0.clone())
        torch.cuda.synchronize()
        assert torch.equal(ya, yb)


@pytest.mark.parametrize("M,K,N", [(8, 1536, 1536), (8, 8960, 1536), (8, 1536, 1920), (5, 960, 2560), (1, 64, 32),
                                   (7, 2560, 960)])
@pytest.mark.parametrize("epilogue", ["store", "add", "silu_pairs"])
def test_packed8_weights_match_float64(M, K, N, epilogue):
    """W in 8-row tiles [N/8, K/64, 512] (the two 32-column halves of a
    64-column step in one MFMA, folded across lanes): every epilogue, with
    and without the fused RMS scale, agrees with the float64 product as the
    16-row layout does (its sums run in another order: equal to rounding,
    not bit-identical), and repeats bit for bit."""
    rng = np.random.default_rng(M * 11 + N + K)
    x, w, b = _data(rng, M, K, N)
    xd, wd = dev(x, "bf16"), dev(w, "bf16")
    w8 = ops.pack_gemv_weight(wd, 8)
    assert w8.shape == (N // 8, K // 64, 512)
    y0 = O.round_bf16(rng.standard_normal((M, N // 2 if epilogue == "silu_pairs" else N), dtype=np.float32))
    bias = dev(b, "bf16") if epilogue == "store" else None
    for rms in (None, 1e-6):
        xs = x.astype(np.float64)
        if rms:
            xs = xs / np.sqrt((xs ** 2).mean(-1, keepdims=True) + rms)
        prod = xs @ w.astype(np.float64).T
        if epilogue == "store":
            ref = prod + b
        elif epilogue == "add":
            ref = prod + y0
        else:
            g, u = prod[:, 0::2], prod[:, 1::2]
            ref = g / (1 + np.exp(-g)) * u
        outs = [ops.gemv(xd, w8, bias=bias, rms_eps=rms, epilogue=epilogue, out=dev(y0, "bf16")) for _ in range(2)]
        y16 = ops.gemv(xd, ops.pack_gemv_weight(wd), bias=bias, rms_eps=rms, epilogue=epilogue, out=dev(y0, "bf16"))
        torch.cuda.synchronize()
        assert torch.equal(outs[0], outs[1])
        got = host(outs[0])
        assert rel_l2(got, ref) < 4e-3 and rel_l2(host(y16), ref) < 4e-3
        assert np.max(np.abs(got - ref)) <= 2 ** -7 * np.max(np.abs(ref)) + 1e-3
        assert torch.allclose(outs[0].float(), y16.float(), rtol=2 ** -7, atol=2e-3)


def test_packed8_rope_kv_and_row_limit():
    """The fused q/k/v projection + RoPE + cache append on 8-row tiles equals
    the 16-row layout to rounding; more than 8 rows of x are refused."""
    rng = np.random.default_rng(83)
    M, K, n_q, n_k, n_v, d = 8, 1536, 12, 1, 2, 128
    x, w, b = _data(rng, M, K, (n_q + n_k + n_v) * d)
    xd, wd, bd = dev(x, "bf16"), dev(w, "bf16"), dev(b, "bf16")
    pos = torch.arange(M, dtype=torch.int32, device="cuda") * 3 + 1
    outs = []
    for rows in (16, 8):
        kc = torch.zeros(M, n_k, 64, d, dtype=torch.bfloat16, device="cuda")
        vc = torch.zeros(M, n_v, 64, d, dtype=torch.bfloat16, device="cuda")
        q = ops.gemv_rope_kv(xd, ops.pack_gemv_weight(wd, rows), bd, n_q, n_k, n_v, 1e6, pos, kc, vc, rms_eps=1e-6,
                             rope_table=ops.rope_table(pos, d, 1e6))
        outs.append((q, kc, vc))
    torch.cuda.synchronize()
    for a, c in zip(outs[0], outs[1]):
        assert torch.allclose(a.float(), c.float(), rtol=2 ** -7, atol=2e-3)
        assert a.float().abs().sum() > 0
    x9 = dev(O.round_bf16(rng.standard_normal((9, 64), dtype=np.float32)), "bf16")
    with pytest.raises(RuntimeError, match="at most 8 rows"):
        ops.gemv(x9, ops.pack_gemv_weight(wd[:32, :64].contiguous(), 8))


def test_packed_rope_kv_projection_identical():
    rng = np.random.default_rng(81)
    M, K, n_q, n_k, n_v, d = 8, 1536, 12, 1, 2, 128
    x, w, b = _data(rng, M, K, (n_q + n_k + n_v) * d)
    xd, wd, bd = dev(x, "bf16"), dev(w, "bf16"), dev(b, "bf16")
    pos = torch.arange(M, dtype=torch.int32, device="cuda") * 3 + 1
    outs = []
    for wt in (wd, ops.pack_gemv_weight(wd)):
        kc = torch.zeros(M, n_k, 64, d, dtype=torch.bfloat16, device="cuda")
        vc = torch.zeros(M, n_v, 64, d, dtype=torch.bfloat16, device="cuda")
        q = ops.gemv_rope_kv(xd, wt, bd, n_q, n_k, n_v, 1e6, pos, kc, vc, rms_eps=1e-6)
        outs.append((q, kc, vc))
    torch.cuda.synchronize()
    for a, c in zip(outs[0], outs[1]):
        assert torch.equal(a, c)


@pytest.mark.parametrize("N", [4097, 151936])
def test_argmax_two_pass_ties_across_chunks(N):
    """The two-pass argmax (chunks of 4096 per workgroup) keeps the first
    index of the maximum when it repeats in later chunks, and agrees with
    the one-workgroup-per-row pass (no workspace)."""
    rng = np.random.default_rng(N)
    x = O.round_bf16(rng.standard_normal((5, N), dtype=np.float32))
    x[0, [N - 1, 4096, 5000 % N]] = 30.0          # tie: first one wins
    x[1, :] = -1.0                                 # all equal -> index 0
    x[2, [3, N - 2]] = 7.0
    xd = dev(x, "bf16")
    got = ops.argmax_rows(xd).cpu().numpy()
    np.testing.assert_array_equal(got, np.argmax(x, axis=1))
    lib = _lib.load()
    assert lib.saga_argmax_workspace_bytes(5, N) > 0
    one = torch.empty(5, dtype=torch.int64, device="cuda")
    _lib.check(lib.saga_argmax(_lib.tensor(xd), _lib.ptr(one), None, 0, _lib.stream_of(xd)), "argmax")
    np.testing.assert_array_equal(one.cpu().numpy(), got)


def test_split_k_shapes_share_one_workspace():
    """Split-K calls of different shapes, one after the other on the cached
    workspace (the tile counters sit at a fixed offset and are left at zero):
    each matches its single-pass result."""
    rng = np.random.default_rng(90)
    for M, K, N in [(8, 2560, 960), (8, 8960, 1536), (32, 8960, 1536), (4, 2560, 960), (8, 8960, 1536), (2, 4096, 256),
                    (17, 2560, 960)]:
        x, w, _ = _data(rng, M, K, N)
        xd, wd = dev(x, "bf16"), dev(w, "bf16")
        for rms in (None, 1e-6):
            a = ops.gemv(xd, wd, rms_eps=rms, split_k=False)
            b = ops.gemv(xd, wd, rms_eps=rms, split_k=True)
            torch.cuda.synchronize()
            assert torch.allclose(a.float(), b.float(), rtol=2 ** -7, atol=2e-3), (M, K, N, rms)
