"""The dispatcher inside a transformers model, as the reference's drivers
install it (speedup.py:497: ALL_ATTENTION_FUNCTIONS["sdpa"] = dispatcher).

A tiny random-init Qwen2 (4 query heads, 1 key/value head, d64) runs a
600-token prefill and greedy decode steps; every decode-step attention call
goes to the HIP kernels.  Dense mode and the Atop-N calibration step with
N >= L (every position kept) must reproduce transformers' own SDPA logits;
every fast and calibration step after it, inside the model, equals the
oracle's amortized step (the reference's fp32 path) on the same operands and
threshold-table row."""
import pytest
import torch

from conftest import rel_l2

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")


def _model():
    from transformers import Qwen2Config, Qwen2ForCausalLM
    cfg = Qwen2Config(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                      num_key_value_heads=1, vocab_size=1024, max_position_embeddings=4096, rope_theta=1e4)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(0)
    return Qwen2ForCausalLM(cfg).to("cuda", torch.bfloat16).eval()


@torch.no_grad()
def _greedy(model, ids, steps):
    out = model(ids, use_cache=True)
    pkv, logits = out.past_key_values, [out.logits[:, -1].float()]
    tok = out.logits[:, -1].argmax(-1, keepdim=True)
    for _ in range(steps):
        out = model(tok, past_key_values=pkv, use_cache=True)
        pkv = out.past_key_values
        logits.append(out.logits[:, -1].float())
        tok = out.logits[:, -1].argmax(-1, keepdim=True)
    return logits


@pytest.fixture
def restore_sdpa(monkeypatch):
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    from saga_amd.attention import attention as A
    monkeypatch.setattr(A, "EXEMPT_LAYERS", set())
    orig = ALL_ATTENTION_FUNCTIONS["sdpa"]
    yield orig
    ALL_ATTENTION_FUNCTIONS["sdpa"] = orig


def test_dense_and_calibration_match_transformers(restore_sdpa):
    from saga_amd.attention import attention as A
    from saga_amd.attention.dispatch import SagaDispatcher
    model = _model()
    ids = torch.randint(0, 1024, (2, 600), device="cuda")
    ref = _greedy(model, ids, 3)

    calls = []
    disp = SagaDispatcher(mode="full").register()
    orig_full = A.full_einsum_forward

    def spy_full(*a, **k):
        calls.append("full")
        return orig_full(*a, **k)

    A.full_einsum_forward = spy_full
    try:
        dense = _greedy(model, ids, 3)
    finally:
        A.full_einsum_forward = orig_full
    assert calls.count("full") == 3 * 2  # 3 decode steps x 2 layers
    for a, b in zip(dense, ref):
        assert rel_l2(a.cpu().numpy(), b.cpu().numpy()) < 2e-2

    A.init_amortized_threshold_tensor("cuda", A.MAX_LAYERS, 2 * 4)
    disp = SagaDispatcher(mode="atopn", top_n=4096, policy="speedup").register()
    atopn = _greedy(model, ids, 3)
    assert disp.step == 3
    # step 1 calibrates with N >= L: every position kept, renormalised = softmax
    assert rel_l2(atopn[1].cpu().numpy(), ref[1].cpu().numpy()) < 2e-2
    for lg in atopn:
        assert torch.isfinite(lg).all()
    A.reset_amortized_state()


def _f32(t):
    return None if t is None else t.detach().float().cpu().numpy()


def test_atopn_fast_steps_run_on_kernels(restore_sdpa):
    """lm_eval's policy (recalibration every 2 steps) inside the model: every
    Atop-N call's output against the oracle on the call's own operands -- the
    calibration step's output and stored threshold, and each fast step's
    output given the table row the kernels read."""
    import numpy as np
    from oracle import saga_oracle as O
    from saga_amd.attention import attention as A
    from saga_amd.attention.dispatch import SagaDispatcher
    model = _model()
    ids = torch.randint(0, 1024, (1, 700), device="cuda")
    A.init_amortized_threshold_tensor("cuda", A.MAX_LAYERS, 4)
    disp = SagaDispatcher(mode="atopn", top_n=64, policy="lm_eval", recalibrate_every=2).register()
    calls = []
    orig_cal, orig_fast = A.approx_top_n_attention_amortized_cal, A.approx_top_n_attention_amortized

    def spy(kind, fn):
        def wrapped(query, key, value, attention_mask=None, is_causal=False, top_n_attention=256, scaling=None,
                    layer_idx=0):
            row = _f32(A.AMORTIZED_THRESHOLD_TENSOR[layer_idx, :query.shape[0] * query.shape[1]])
            out = fn(query, key, value, attention_mask, is_causal=is_causal, top_n_attention=top_n_attention,
                     scaling=scaling, layer_idx=layer_idx)
            stored = _f32(A.AMORTIZED_THRESHOLD_TENSOR[layer_idx, :query.shape[0] * query.shape[1]])
            calls.append((kind, _f32(query), _f32(key), _f32(value), _f32(attention_mask), scaling, top_n_attention,
                          row, stored, _f32(out)))
            return out
        return wrapped

    A.approx_top_n_attention_amortized_cal = spy("cal", orig_cal)
    A.approx_top_n_attention_amortized = spy("fast", orig_fast)
    try:
        logits = _greedy(model, ids, 5)
    finally:
        A.approx_top_n_attention_amortized_cal, A.approx_top_n_attention_amortized = orig_cal, orig_fast
    assert disp.step == 5
    assert (A.AMORTIZED_THRESHOLD_TENSOR[:2, :4] > 0).all()
    for lg in logits:
        assert torch.isfinite(lg).all()
    kinds = [c[0] for c in calls]
    assert kinds.count("cal") >= 2 and kinds.count("fast") >= 4, kinds
    for kind, q, k, v, mask, sc, N, row, stored, out in calls:
        if kind == "cal":
            ref, thr, _ = O.calibrate(q, k, v, mask, N, sc)
            np.testing.assert_allclose(stored, thr, rtol=1e-4)
        else:
            ref, _, _, _ = O.fast(q, k, v, row, mask, N, sc)
        # bf16 operands (the oracle runs in fp32 on the same rounded values)
        assert np.max(np.abs(out - ref)) < 2e-2 and rel_l2(out, ref) < 2e-2, kind
    A.reset_amortized_state()
