"""Parity at the kernel-sweep corners and at the 128k dense-GQA comparison
shape, with full-size bf16 caches.

Kernel sweep (head_dim 128, keys N(0,1) with 1 % of the rows scaled x8 to
stress the threshold, as the sweep's synthetic caches): batch 32 at 64k and
128k positions, batch 8 at 64k and 128k with N in {64, 1024}, and the head
groupings k_h in {1, 2} x v_h in {2, 4, 8} at 16k.  Dense GQA at the 128k
comparison shape: batch 4, 12 query / 2 key / 2 value heads.

Inputs are drawn on the GPU; the oracle (the reference's fp32 path) runs on
sampled batch rows.  Batch rows never interact, so the oracle on a one-row
sub-batch is the reference on that row.  Checked: calibration thresholds and
outputs; the fast step's thresholds, its ordered selection rule on its own
fp32 scores (exact), its sets against the oracle's outside a near-tie band
(overflowing rows: the ordered lists up to the first near-tie position), and
its outputs against the reference fp32 gather . V on the GPU's selection
(rel-L2 1e-3 on the fp32 output, max-abs 2e-2 on the bf16 output)."""
import zlib

import numpy as np
import pytest
import torch

from conftest import rel_l2, set_diff_outside_band
from oracle import saga_oracle as O
from saga_amd import ops

pytestmark = pytest.mark.gpu

C4 = {  # name: b, q_h, k_h, v_h, L, N
    "b32_64k_N256": (32, 12, 1, 2, 65536, 256),
    "b32_128k_N256": (32, 12, 1, 2, 131072, 256),
    "b8_64k_N64": (8, 12, 1, 2, 65536, 64),
    "b8_64k_N1024": (8, 12, 1, 2, 65536, 1024),
    "b8_128k_N64": (8, 12, 1, 2, 131072, 64),
    "b8_128k_N1024": (8, 12, 1, 2, 131072, 1024),
    "k1_v4_16k": (8, 12, 1, 4, 16384, 256),
    "k1_v8_16k": (8, 16, 1, 8, 16384, 256),
    "k2_v2_16k": (8, 12, 2, 2, 16384, 256),
    "k2_v4_16k": (8, 12, 2, 4, 16384, 256),
    "k2_v8_16k": (8, 16, 2, 8, 16384, 256),
}
D = 128


def _inputs(seed, b, q_h, k_h, v_h, L):
    """bf16 q1, q2 (= q1 + 0.3 noise), K with 1 % outlier rows x8, V, drawn on the GPU."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    q1 = torch.randn(b, q_h, 1, D, device="cuda", generator=g).to(torch.bfloat16)
    q2 = (q1.float() + 0.3 * torch.randn(b, q_h, 1, D, device="cuda", generator=g)).to(torch.bfloat16)
    k = torch.empty(b, k_h, L, D, device="cuda", dtype=torch.bfloat16)
    v = torch.empty(b, v_h, L, D, device="cuda", dtype=torch.bfloat16)
    for i in range(b):  # one batch row at a time: bounded fp32 temporaries
        kf = torch.randn(k_h, L, D, device="cuda", generator=g)
        out = torch.rand(k_h, L, device="cuda", generator=g) < 0.01
        kf[out] *= 8.0
        k[i] = kf.to(torch.bfloat16)
        v[i] = torch.randn(v_h, L, D, device="cuda", generator=g).to(torch.bfloat16)
    return q1, q2, k, v


def _host(t):
    return t.float().cpu().numpy()


def _sample_rows(b):
    return sorted({0, b // 2, b - 1})


@pytest.mark.parametrize("name", list(C4))
def test_sweep_corner_vs_oracle(name):
    b, q_h, k_h, v_h, L, N = C4[name]
    print(f"c4 corner {name}: b={b} q/k/v={q_h}/{k_h}/{v_h} L={L} N={N}", flush=True)
    q1, q2, k, v = _inputs(zlib.crc32(name.encode()), b, q_h, k_h, v_h, L)
    nr, buf_k = b * q_h, min(2 * N, L)
    table = torch.zeros(nr, device="cuda")
    cal = _host(ops.atopn_calibrate(q1, k, v, N, table, out_dtype=torch.float32))
    out32 = _host(ops.atopn_decode(q2, k, v, table, N, out_dtype=torch.float32))
    out16 = _host(ops.atopn_decode(q2, k, v, table, N, out_dtype=torch.bfloat16))
    torch.cuda.synchronize()
    thr = _host(table)
    batch_rows = _sample_rows(b)
    rows = [i * q_h + j for i in batch_rows for j in range(q_h)]
    views = ops.atopn_workspace_views(b, q_h, k_h, L, D, buf_k, "cuda:0", rows=rows)
    views = {k_: (v_.numpy() if isinstance(v_, torch.Tensor) else v_) for k_, v_ in views.items()}
    g_v = q_h // v_h
    flips = overflow = 0
    for bi_pos, i in enumerate(batch_rows):
        qi1, qi2, ki, vi = _host(q1[i:i + 1]), _host(q2[i:i + 1]), _host(k[i:i + 1]), _host(v[i:i + 1])
        r0 = i * q_h
        ref_cal, rt, _ = O.calibrate(qi1, ki, vi, None, N, None)
        np.testing.assert_allclose(thr[r0:r0 + q_h], rt, rtol=1e-4)
        assert rel_l2(cal[i], ref_cal[0]) < 1e-3
        _, t_ref, idx_ref, cnt_ref = O.fast(qi2, ki, vi, thr[r0:r0 + q_h], None, N, None)
        logits = O.qk_scores(qi2, ki).reshape(q_h, L)
        for j in range(q_h):
            vr = bi_pos * q_h + j  # row in the sampled views
            x, t = views["scores"][vr], views["thresh"][vr]
            # the ordered rule on the GPU's own fp32 scores and threshold: exact
            passing = np.nonzero(x > t)[0]
            assert views["sel_total"][vr] == passing.size
            kept = min(passing.size, buf_k)
            assert views["sel_cnt"][vr] == kept
            sel = views["sel_idx"][vr, :kept]
            np.testing.assert_array_equal(sel, passing[:kept])
            np.testing.assert_allclose(t, t_ref[j], rtol=1e-5, atol=1e-5)
            sel_ref = idx_ref.reshape(q_h, buf_k)[j, :min(int(cnt_ref[j]), buf_k)]
            band = 1e-4 * max(1.0, abs(float(t_ref[j])))
            if cnt_ref[j] > buf_k or passing.size > buf_k:
                overflow += 1
                near = np.nonzero(np.abs(x - t_ref[j]) <= band)[0]
                first = near[0] if near.size else L
                np.testing.assert_array_equal(sel[sel < first], sel_ref[sel_ref < first])
            else:
                assert not set_diff_outside_band(sel, sel_ref, x, t_ref[j], band)
                flips += len(set(sel.tolist()) ^ set(sel_ref.tolist()))
                # the reference fp32 path's own output (its own selection), whatever the flips
                vh = j // g_v
                direct = O.gather_output(logits[j, sel_ref][None, None, None, :],
                                         sel_ref[None, None, None, :].astype(np.int64), vi[:, vh:vh + 1],
                                         (1, 1, 1, D), input_is_logits=True).reshape(D)
                assert rel_l2(out32[i, j, 0], direct) < 1e-3, (i, j, flips)
                assert np.max(np.abs(out16[i, j, 0] - direct)) < 2e-2, (i, j, flips)
            # the reference fp32 gather . V on the GPU's own selection
            vh = j // g_v
            ref = O.gather_output(logits[j, sel][None, None, None, :], sel[None, None, None, :].astype(np.int64),
                                  vi[:, vh:vh + 1], (1, 1, 1, D), input_is_logits=True).reshape(D)
            assert rel_l2(out32[i, j, 0], ref) < 1e-3, (i, j, kept)
            assert np.max(np.abs(out16[i, j, 0] - ref)) < 2e-2, (i, j, kept)
    print(f"  flips={flips} overflowing_rows={overflow} mean_kept={views['sel_cnt'].mean():.1f}", flush=True)


def test_dense_gqa_at_the_128k_comparison_shape():
    """The in-house dense-GQA comparator (full_einsum_forward,
    attention/attention.py:64-85) at batch 4, 131072 positions, 12 query /
    2 key / 2 value heads, against the oracle's dense path on sampled rows."""
    b, q_h, k_h, v_h, L = 4, 12, 2, 2, 131072
    q1, _, k, v = _inputs(77, b, q_h, k_h, v_h, L)
    out32 = _host(ops.dense_decode(q1, k, v, out_dtype=torch.float32))
    out16 = _host(ops.dense_decode(q1, k, v, out_dtype=torch.bfloat16))
    torch.cuda.synchronize()
    for i in _sample_rows(b):
        ref = O.dense(_host(q1[i:i + 1]), _host(k[i:i + 1]), _host(v[i:i + 1]))
        assert rel_l2(out32[i], ref[0]) < 1e-3
        assert np.max(np.abs(out16[i] - ref[0])) < 2e-2
