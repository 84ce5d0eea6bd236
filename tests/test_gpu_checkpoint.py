"""A SAGA checkpoint loaded into the decoder and decoded on the kernels.

SagaDecoder.from_pretrained reads a checkpoint written the way the
reference's tools write them (config.json num_key_heads, k_proj of one head;
lm_eval_saga.py:52-146).  After the batch-1 prefill, decode steps on the
kernels (skinny GEMM, fused RoPE + cache append, attention) must give the
logits of a float64 forward of the same bf16 weights over the same tokens (the
prompt and the tokens the decoder chose).  Dense mode: every step.  Atop-N
mode: the calibration step with N above the context, which keeps every
position; the fast steps after it may drop positions below the calibrated
probability (attention/attention.py:181-185, 203-206), so their selection is
left to the attention parity tests."""
import numpy as np
import pytest
import torch

from conftest import rel_l2

pytestmark = pytest.mark.gpu

pytest.importorskip("transformers")
from ckpt_util import forward64, save_saga_checkpoint, tiny_hf_model  # noqa: E402


@pytest.mark.parametrize("kind,tie,mode", [("qwen2", True, "dense"), ("llama", False, "dense"),
                                           ("qwen2", True, "atopn"), ("llama", False, "atopn")])
def test_loaded_checkpoint_decodes_like_float64_forward(tmp_path, kind, tie, mode):
    from saga_amd.checkpoint import load_checkpoint
    from saga_amd.decoder import SagaDecoder
    model = tiny_hf_model(kind, n_kv=2, n_k_shared=1, tie=tie, d=64, intermediate=512, vocab=1024)
    path = str(tmp_path / "saga")
    save_saga_checkpoint(model, path, n_k=1)
    shape, w = load_checkpoint(path)  # the bf16 weights the decoder holds
    print(f"checkpoint {kind} tie={tie} mode={mode}: {shape}", flush=True)
    m = SagaDecoder.from_pretrained(path, batch=2, max_len=256, mode=mode, top_n=512)
    assert (m.shape.n_k, m.shape.n_v) == (1, 2) and m.use_gemv and m.fuse_rope
    rng = np.random.default_rng(7)
    ids = [int(t) for t in rng.integers(0, 1024, 120)]
    m.prefill(torch.tensor(ids))
    hf16 = model.to(torch.bfloat16)  # transformers' own bf16 forward, for scale
    for i in range(3 if mode == "dense" else 1):
        ids.append(int(m.tokens[0]))
        m.step(calibrate=(i == 0))
        torch.cuda.synchronize()
        got = m._logits.float().cpu().numpy()
        ref = forward64(shape, w, ids)[-1]
        err = rel_l2(got[0], ref)
        with torch.no_grad():
            hf = hf16(torch.tensor(ids)[None]).logits[0, -1].double().numpy()
        print(f"  step {i}: rel_l2 {err:.4f} (transformers bf16: {rel_l2(hf, ref):.4f})", flush=True)
        assert np.array_equal(got[0], got[1])  # both batch rows hold the same sequence
        assert err < 1.5e-2, (i, err)  # measured 0.004-0.005, transformers bf16 0.005-0.007
        top2 = np.sort(ref)[-2:]
        if top2[1] - top2[0] > 0.05:  # bf16 rounding may flip a near tie
            assert int(m.tokens[0]) == int(np.argmax(ref))


def test_generate_graphs_equal_eager_steps(tmp_path):
    """SagaDecoder.generate on a loaded checkpoint: the replayed HIP graphs
    give the tokens of eager steps, and the first token is the prefill's
    argmax of the float64 forward when its margin is clear."""
    from saga_amd.checkpoint import load_checkpoint
    from saga_amd.decoder import SagaDecoder
    model = tiny_hf_model("llama", n_kv=2, n_k_shared=1, tie=False, d=64, intermediate=512, vocab=1024)
    path = str(tmp_path / "saga")
    save_saga_checkpoint(model, path, n_k=1)
    m = SagaDecoder.from_pretrained(path, batch=3, max_len=256, mode="atopn", top_n=512)
    prompt = torch.tensor(np.random.default_rng(9).integers(0, 1024, 90))
    g = m.generate(prompt, 8)
    e = m.generate(prompt, 8, graphs=False)
    torch.cuda.synchronize()
    assert g.shape == (3, 8) and torch.equal(g, e)
    assert torch.equal(g[0], g[1]) and torch.equal(g[0], g[2])
    shape, w = load_checkpoint(path)
    ref = forward64(shape, w, [int(t) for t in prompt])[-1]
    top2 = np.sort(ref)[-2:]
    if top2[1] - top2[0] > 0.05:
        assert int(g[0, 0]) == int(np.argmax(ref))
