"""C ABI of libsaga_amd.so on the CPU: it loads, exports every symbol the
header declares, sizes workspaces, and rejects bad arguments with an error
code and message before anything is launched (no GPU needed)."""
import ctypes
import os
import re

import pytest

from saga_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "saga_amd.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(saga_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_symbols()
    assert len(names) >= 12
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib._SIGS), "ctypes signatures and header declarations differ"
    assert lib.saga_version() == 100


def _t(shape, dtype=_lib.DTYPE_BF16, data=0x100000, strides=None):
    d = _lib.SagaTensor()
    d.data = data
    d.dtype = dtype
    d.ndim = len(shape)
    if strides is None:
        strides, acc = [], 1
        for n in reversed(shape):
            strides.insert(0, acc)
            acc *= n
    for i, (n, s) in enumerate(zip(shape, strides)):
        d.shape[i] = n
        d.stride[i] = s
    return d


def _call_decode(q, k, v, out, mask=None, top_n=8, ws=0x200000, nbytes=1 << 30, fn="saga_atopn_decode"):
    lib = _lib.load()
    return getattr(lib, fn)(ctypes.byref(q), ctypes.byref(k), ctypes.byref(v),
                            ctypes.byref(mask) if mask is not None else None, None, 0.125, top_n,
                            ctypes.c_void_p(0x300000), ctypes.byref(out), ctypes.c_void_p(ws), nbytes, None)


def _err():
    return _lib.load().saga_last_error().decode()


GOOD = dict(q=(2, 12, 1, 128), k=(2, 1, 64, 128), v=(2, 2, 64, 128), out=(2, 12, 1, 128))


def _good():
    return {n: _t(s) for n, s in GOOD.items()}


@pytest.mark.parametrize("mutate,code,needle", [
    (lambda a: a.__setitem__("q", _t((2, 12, 2, 128))), -2, "l_q == 1"),
    (lambda a: a.__setitem__("k", _t((2, 5, 64, 128))), -1, "multiple of k_h"),
    (lambda a: a.__setitem__("v", _t((2, 5, 64, 128))), -1, "multiple of v_h"),
    (lambda a: a.__setitem__("v", _t((2, 2, 63, 128))), -1, "value: shape"),
    (lambda a: a.update(q=_t((2, 12, 1, 96)), k=_t((2, 1, 64, 96)), v=_t((2, 2, 64, 96)),
                        out=_t((2, 12, 1, 96))), -2, "head_dim"),
    (lambda a: a.update(q=_t((2, 32, 1, 128)), out=_t((2, 32, 1, 128))), -2, "q_h / k_h"),
    (lambda a: a.__setitem__("k", _t((2, 1, 64, 128), dtype=_lib.DTYPE_F32)), -1, "dtype differs"),
    (lambda a: a.__setitem__("q", _t((2, 12, 1, 128), data=0x100002)), -1, "16-byte aligned"),
    (lambda a: a.__setitem__("k", _t((2, 1, 64, 128), strides=(64 * 130, 64 * 130, 130, 1))), -1, "multiple of 16"),
    (lambda a: a.__setitem__("out", _t((2, 12, 1, 64))), -1, "out: shape"),
    (lambda a: a.__setitem__("q", _t((2, 12, 1, 128), data=0)), -1, "null data"),
])
def test_decode_argument_errors(mutate, code, needle):
    a = _good()
    mutate(a)
    rc = _call_decode(a["q"], a["k"], a["v"], a["out"])
    assert rc == code, _err()
    assert needle in _err()


def test_decode_rejects_bad_mask_and_topn_and_workspace():
    a = _good()
    rc = _call_decode(a["q"], a["k"], a["v"], a["out"], mask=_t((2, 1, 1, 63), dtype=_lib.DTYPE_BOOL))
    assert rc == -1 and "mask" in _err()
    rc = _call_decode(a["q"], a["k"], a["v"], a["out"], mask=_t((2, 1, 1, 64), dtype=_lib.DTYPE_I32))
    assert rc == -1 and "mask: dtype" in _err()
    rc = _call_decode(a["q"], a["k"], a["v"], a["out"], top_n=0)
    assert rc == -1 and "top_n" in _err()
    rc = _call_decode(a["q"], a["k"], a["v"], a["out"], nbytes=100)
    assert rc == -3 and "workspace" in _err()
    rc = _call_decode(a["q"], a["k"], a["v"], a["out"], ws=0x200010)
    assert rc == -3 and "aligned" in _err()


def test_decode_ex_checks_the_k2_variant():
    """saga_atopn_decode_ex takes the K2 kernels per call (no process-wide
    switch): variants 0-2 pass validation (the fake pointers then fail only
    at the launch, for want of a device), anything else is refused before."""
    lib = _lib.load()
    a = _good()

    def call(variant, nbytes=1 << 30):
        return lib.saga_atopn_decode_ex(ctypes.byref(a["q"]), ctypes.byref(a["k"]), ctypes.byref(a["v"]), None, None,
                                        0.125, 8, ctypes.c_void_p(0x300000), ctypes.byref(a["out"]), variant,
                                        ctypes.c_void_p(0x200000), nbytes, None)

    for bad in (-1, 3, 7):
        assert call(bad) == -1 and "k2_variant" in _err()
    for good in (_lib.K2_AUTO, _lib.K2_ROW_BLOCK, _lib.K2_SLICE_ROW):
        assert call(good, nbytes=100) == -3 and "workspace" in _err()  # validated up to the workspace check
    assert not hasattr(lib, "saga_set_k2_mode") and not hasattr(lib, "saga_set_fused_fast_step")


def test_calibrate_ex_checks_the_variant():
    """saga_atopn_calibrate_ex takes the calibration kernels per call, with
    the same variant values and checks as saga_atopn_decode_ex."""
    lib = _lib.load()
    a = _good()

    def call(variant, nbytes=1 << 30):
        return lib.saga_atopn_calibrate_ex(ctypes.byref(a["q"]), ctypes.byref(a["k"]), ctypes.byref(a["v"]), None,
                                           None, 0.125, 8, ctypes.c_void_p(0x300000), ctypes.byref(a["out"]), variant,
                                           ctypes.c_void_p(0x200000), nbytes, None)

    for bad in (-1, 3, 7):
        assert call(bad) == -1 and "k2_variant" in _err()
    for good in (_lib.K2_AUTO, _lib.K2_ROW_BLOCK, _lib.K2_SLICE_ROW):
        assert call(good, nbytes=100) == -3 and "workspace" in _err()


def test_null_descriptor_is_an_error_not_a_crash():
    lib = _lib.load()
    rc = lib.saga_atopn_decode(None, None, None, None, None, 1.0, 8, None, None, None, 0, None)
    assert rc == -1 and "null" in _err()
    rc = lib.saga_threshold_select(None, None, 0, 4, None, None, None, None)
    assert rc == -1


def test_threshold_select_argument_errors():
    lib = _lib.load()
    x = _t((4, 100), dtype=_lib.DTYPE_F32)
    vals = _t((4, 8), dtype=_lib.DTYPE_F32)
    bad_vals = _t((4, 8), dtype=_lib.DTYPE_BF16)
    thr = ctypes.c_void_p(0x400000)
    idx = ctypes.c_void_p(0x500000)
    assert lib.saga_threshold_select(ctypes.byref(x), thr, 0, 8, ctypes.byref(vals), idx, None, None) == -1
    assert lib.saga_threshold_select(ctypes.byref(x), thr, 4, 8, ctypes.byref(bad_vals), idx, None, None) == -1
    assert "dtype must match" in _err()
    assert lib.saga_threshold_select(ctypes.byref(x), thr, 4, 9, ctypes.byref(vals), idx, None, None) == -1
    strided = _t((2, 2, 100), dtype=_lib.DTYPE_F32, strides=(1000, 100, 1))
    assert lib.saga_threshold_select(ctypes.byref(strided), thr, 4, 8, ctypes.byref(vals), idx, None, None) == -1
    assert "collapsible" in _err()


def test_workspace_sizes_and_layout():
    lib = _lib.load()
    lay = _lib.atopn_layout(8, 12, 1, 33024, 128, 1024)
    offs = [lay.scores, lay.part_max, lay.part_sum, lay.thresh, lay.sel_idx, lay.sel_val, lay.sel_cnt,
            lay.sel_total]
    assert offs == sorted(offs) and all(o % 256 == 0 for o in offs)
    assert lay.scores_ld % 16 == 0 and lay.scores_ld >= 33024
    assert lay.nparts == lib.saga_qk_nparts(8, 1, 33024)
    assert lay.total_bytes == lib.saga_atopn_workspace_bytes(8, 12, 1, 33024, 128, 1024)
    assert lay.part_max - lay.scores >= 96 * 33024 * 4
    assert lib.saga_dense_workspace_bytes(8, 12, 33024, 128) > 0
    bad = _lib.AtopnLayout()
    assert lib.saga_atopn_workspace_layout(0, 12, 1, 10, 128, 4, ctypes.byref(bad)) == -1


@pytest.mark.parametrize("b", [1, 4, 8, 32])
@pytest.mark.parametrize("k_h", [1, 2])
def test_qk_part_plan(b, k_h):
    """K1 splits each (batch, key head) row into 4n balanced ranges of at most
    6 sixteen-position tiles (n partials, one per block of 4 waves), in whole
    rounds of 3072 resident waves up to the rounding to blocks."""
    lib = _lib.load()
    for L in (1, 15, 16, 17, 100, 4096, 32769, 33024, 131072, 131328):
        n = lib.saga_qk_nparts(b, k_h, L)
        T = (L + 15) // 16
        assert 1 <= n and 4 * n <= T + 3
        assert -(-T // (4 * n)) <= 6
        rounds = -(-(b * k_h * -(-T // 6)) // 3072)
        assert b * k_h * 4 * n <= rounds * 3072 + 3 * b * k_h
    assert lib.saga_qk_nparts(8, 1, 33024) == 96
    assert lib.saga_qk_nparts(0, 1, 10) == 0


def test_gemv_split_plan():
    """Split-K only for weights with few 16-row tiles and long rows."""
    lib = _lib.load()
    assert lib.saga_gemv_workspace_bytes(8, 1536, 8960) > 0       # MLP down projection
    assert lib.saga_argmax_workspace_bytes(8, 151936) == 8 * 38 * 8  # 38 chunks of 4096, (value, index) each
    assert lib.saga_argmax_workspace_bytes(8, 4096) == 0             # one chunk: single pass
    for n, k in ((17920, 1536), (1920, 1536), (1536, 1536), (151936, 1536)):
        assert lib.saga_gemv_workspace_bytes(8, n, k) == 0


def test_ops_refuse_cpu_tensors():
    import torch
    from saga_amd import ops
    q = torch.zeros(1, 2, 1, 64)
    k = torch.zeros(1, 1, 8, 64)
    v = torch.zeros(1, 2, 8, 64)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.dense_decode(q, k, v)
    import attention.attention as A
    A.init_amortized_threshold_tensor("cpu", A.MAX_LAYERS, 2)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        A.approx_top_n_attention_amortized(q, k, v, top_n_attention=4)


def test_gemv_packed_weight_layout_checks():
    """A 4-D w is the packed layout [N/16, K/32, 16, 32]: K must match x,
    the tensor must be contiguous, 16-byte aligned; errors come back before
    any launch."""
    lib = _lib.load()
    x = _t((8, 1536))
    y = _t((8, 1920))

    def call(w):
        return lib.saga_gemv(ctypes.byref(x), ctypes.byref(w), None, -1.0, 0, ctypes.byref(y), None, 0, None)

    assert call(_t((120, 47, 16, 32))) == -1 and "packed" in _err()          # K / 32 = 48 expected
    assert call(_t((120, 48, 32, 16))) == -1 and "packed" in _err()          # fragment dims swapped
    bad = _t((120, 48, 16, 32), strides=(48 * 512, 512, 1, 16))               # transposed fragments
    assert call(bad) == -1 and "packed" in _err()
    assert call(_t((120, 48, 16, 32), data=0x100008)) == -1 and "aligned" in _err()
    assert call(_t((120, 48, 16, 16))) == -1


def test_gemv_packed8_weight_layout_checks():
    """A 3-D w is the 8-row-tile layout [N/8, K/64, 512]: K must match x, the
    tensor must be contiguous and 16-byte aligned, x at most 8 rows; errors
    come back before any launch."""
    lib = _lib.load()
    y = _t((8, 1920))

    def call(w, x=_t((8, 1536))):
        return lib.saga_gemv(ctypes.byref(x), ctypes.byref(w), None, -1.0, 0, ctypes.byref(y), None, 0, None)

    assert call(_t((240, 23, 512))) == -1 and "8-row" in _err()                    # K / 64 = 24 expected
    assert call(_t((240, 24, 256))) == -1 and "8-row" in _err()                    # fragment of 512
    assert call(_t((240, 24, 512), strides=(24 * 512, 1, 24))) == -1 and "8-row" in _err()
    assert call(_t((240, 24, 512), data=0x100008)) == -1 and "aligned" in _err()
    assert call(_t((240, 24, 512)), x=_t((9, 1536))) == -2 and "at most 8 rows" in _err()


def test_pack_gemv_weight_8_row_tiles_on_cpu():
    """pack_gemv_weight(w, 8)[t, j, 32 r + c] = w[8t + r % 8, 64j + 32 (r // 8) + c],
    and the decoder's unpacking inverts both layouts."""
    import torch
    from saga_amd import ops
    from saga_amd.decoder import SagaDecoder
    w = torch.arange(32 * 192, dtype=torch.float32).reshape(32, 192)
    p = ops.pack_gemv_weight(w, 8)
    assert p.shape == (4, 3, 512)
    for t, j, r, c in [(0, 0, 0, 0), (3, 2, 15, 31), (1, 1, 8, 5), (2, 0, 7, 30)]:
        assert p[t, j, 32 * r + c] == w[8 * t + r % 8, 64 * j + 32 * (r // 8) + c]
    for rows in (16, 8):
        assert torch.equal(SagaDecoder._unpack(ops.pack_gemv_weight(w, rows)), w)
    with pytest.raises(ValueError, match="K % 64"):
        ops.pack_gemv_weight(torch.zeros(16, 96), 8)


def test_embed_rope_and_advance_argument_errors():
    """The step's opening and close check their operands before any launch."""
    lib = _lib.load()
    emb, x = _t((5000, 1536)), _t((8, 1536))
    tok = ctypes.c_void_p(0x100000)
    assert lib.saga_embed_rope(None, ctypes.byref(emb), ctypes.byref(x), None, 0, 0.0, None, None) == -1
    assert "tokens" in _err()
    assert lib.saga_embed_rope(tok, ctypes.byref(emb), ctypes.byref(_t((8, 1024))), None, 0, 0.0, None, None) == -1
    assert "[B, H]" in _err()
    assert lib.saga_embed_rope(tok, ctypes.byref(emb), ctypes.byref(_t((8, 1536), dtype=_lib.DTYPE_F32)), None, 0,
                               0.0, None, None) == -1
    tab = ctypes.c_void_p(0x200000)
    assert lib.saga_embed_rope(tok, ctypes.byref(emb), ctypes.byref(x), None, 128, 1e6, tab, None) == -1
    assert "pos" in _err()
    assert lib.saga_embed_rope(tok, ctypes.byref(emb), ctypes.byref(x), tok, 127, 1e6, tab, None) == -1
    assert lib.saga_embed_rope(tok, ctypes.byref(emb), ctypes.byref(x), tok, 128, 1e6, ctypes.c_void_p(0x200008),
                               None) == -1 and "aligned" in _err()
    assert lib.saga_advance_positions(None, None, 4, None) == -1
    assert lib.saga_advance_positions(None, None, -1, None) == -1
    assert lib.saga_advance_positions(None, None, 0, None) == 0
