"""Routing of the decode-time dispatcher (speedup.py:43-85,
lm_eval_saga.py:152-214) on the CPU: the attention functions are replaced by
recorders, so only the host logic runs (step counter at layer 0, exempt
layers, calibration schedule, prefill reset, output layout)."""
import pytest
import torch

from saga_amd.attention import attention as A
from saga_amd.attention import dispatch as D


class _Layer:
    def __init__(self, i):
        self.layer_idx = i


@pytest.fixture
def calls(monkeypatch):
    log = []

    def rec(name):
        def f(q, k, v, *args, **kw):
            log.append((name, kw.get("layer_idx")))
            return torch.arange(q.numel(), dtype=torch.float32).reshape(q.shape)
        return f

    def base(module, q, k, v, mask, **kw):
        log.append(("sdpa", module.layer_idx))
        return q.transpose(1, 2).contiguous(), None

    monkeypatch.setattr(A, "full_einsum_forward", rec("full"))
    monkeypatch.setattr(A, "approx_top_n_attention_amortized_cal", rec("cal"))
    monkeypatch.setattr(A, "approx_top_n_attention_amortized", rec("fast"))
    monkeypatch.setattr(A, "sdpa_attention_forward", base)
    monkeypatch.setattr(A, "reset_amortized_state", lambda: log.append(("reset", None)))
    monkeypatch.setattr(A, "init_amortized_threshold_tensor", lambda dev, n, r: log.append(("init", r)))
    monkeypatch.setattr(A, "AMORTIZED_THRESHOLD_TENSOR", None)
    monkeypatch.setattr(A, "EXEMPT_LAYERS", {1})
    return log


def _run(fn, l_q, layers=3, b=2, q_h=4, d=8, L=16):
    outs = []
    for i in range(layers):
        q = torch.zeros(b, q_h, l_q, d)
        k = torch.zeros(b, 1, L, d)
        out, none = fn(_Layer(i), q, k, torch.zeros(b, 2, L, d), torch.ones(b, 1, l_q, L + 5, dtype=torch.bool),
                       scaling=0.1)
        assert none is None and out.shape == (b, l_q, q_h, d) and out.is_contiguous()
        outs.append(out)
    return outs


def test_speedup_policy(calls):
    disp = D.SagaDispatcher(mode="atopn", top_n=8, policy="speedup")
    _run(disp, 5)
    for _ in range(3):
        _run(disp, 1)
    _run(disp, 5)
    _run(disp, 1)
    names = [c[0] for c in calls]
    assert names == ["sdpa"] * 3 + ["cal", "full", "cal"] + ["fast", "full", "fast"] * 2 + ["sdpa"] * 3 + \
        ["cal", "full", "cal"]
    assert [c[1] for c in calls if c[0] in ("cal", "fast")][:2] == [0, 2]


def test_lm_eval_policy_recalibrates(calls):
    disp = D.SagaDispatcher(mode="atopn", top_n=8, policy="lm_eval", recalibrate_every=2)
    _run(disp, 5)
    for _ in range(4):
        _run(disp, 1)
    names = [c[0] for c in calls]
    # prefill resets the table; the first decode step creates it (8 rows = b*q_h)
    assert names[:4] == ["reset", "sdpa", "sdpa", "sdpa"]
    assert calls[4] == ("init", 8)
    decode = [n for n in names[5:] if n != "init"]
    assert decode == ["cal", "full", "cal", "fast", "full", "fast", "cal", "full", "cal", "fast", "full", "fast"]


def test_full_and_vanilla_modes(calls):
    _run(D.SagaDispatcher(mode="full"), 1)
    _run(D.SagaDispatcher(mode="vanilla"), 1)
    assert [c[0] for c in calls] == ["full"] * 3 + ["sdpa"] * 3


def test_decode_output_is_transposed(calls):
    disp = D.SagaDispatcher(mode="full")
    out = _run(disp, 1, layers=1)[0]
    ref = torch.arange(2 * 4 * 8, dtype=torch.float32).reshape(2, 4, 1, 8).transpose(1, 2)
    assert torch.equal(out, ref)


def test_module_level_mirror_reads_globals(calls, monkeypatch):
    monkeypatch.setattr(D, "ATTENTION_MODE", "atopn")
    monkeypatch.setattr(D, "TOP_N_ATTENTION", 8)
    monkeypatch.setattr(D, "_DISPATCHER", D.SagaDispatcher(mode="vanilla", top_n=None))
    _run(D.sdpa_attention_forward_dispatch, 1)
    assert [c[0] for c in calls] == ["cal", "full", "cal"]


def test_default_exempt_layers():
    assert D.default_exempt_layers("Qwen/Qwen2.5-1.5B-Instruct") == {0, 14}
    assert D.default_exempt_layers("meta-llama/Llama-3.2-1B") == {0}
    assert D.default_exempt_layers("gpt2") == set()
