"""Pins for the oracle's end-to-end restatement of TorchEngine.prefill (oracle/engine_ref.py):
the reference's own engine tests (tests/test_torch_engine.py:36-74, tests/test_mlx_engine.py:
24-99), run on CPU with a tiny random-init Qwen2 model instead of a downloaded checkpoint. Also
checks that the PyTorch-ROCm baseline engine (chunkkv_amd.baseline) is the same op sequence."""

import numpy as np
import pytest
import torch

from chunkkv_amd.baseline import TorchOpsEngine
from chunkkv_amd.types import BlendConfig, ChunkKV, Placement
from oracle import engine_ref as R
from tests.helpers import StubTokenizer, tiny_qwen2


@pytest.fixture(scope="module")
def model():
    return tiny_qwen2(layers=3, hidden=128, heads=4, kv=2, inter=256, vocab=300, seed=1)


@pytest.fixture(scope="module")
def parts():
    rng = np.random.default_rng(1)
    t = lambda n: rng.integers(1, 299, n).tolist()  # noqa: E731
    return dict(sys=t(9), a=t(23), b=t(19), q=t(7))


def chunk_of(res, s, e):
    return ChunkKV([k[:, :, s:e].contiguous() for k in res["keys"]], [v[:, :, s:e].contiguous() for v in res["values"]], s)


def kl(p, q):
    p, q = torch.log_softmax(p.float(), -1), torch.log_softmax(q.float(), -1)
    return (p.exp() * (p - q)).sum(-1).mean().item()


def test_no_cache_matches_hf_forward(model, parts):
    toks = parts["sys"] + parts["a"] + parts["b"] + parts["q"]
    with torch.inference_mode():
        ref = model(torch.tensor([toks])).logits[0]
    out = R.prefill(model, toks, logits_from=0)
    torch.testing.assert_close(out["logits"], ref, atol=2e-3, rtol=0)
    assert out["stats"]["prefill_token_equiv"] == len(toks)


def test_same_position_reuse(model, parts):
    toks = parts["sys"] + parts["a"] + parts["b"] + parts["q"]
    s = len(parts["sys"])
    first = R.prefill(model, toks)
    ca = chunk_of(first, s, s + len(parts["a"]))
    exact = R.prefill(model, toks, [Placement(ca, s, exact=True)], BlendConfig())
    torch.testing.assert_close(exact["logits"], first["logits"], atol=2e-3, rtol=0)
    naive = R.prefill(model, toks, [Placement(ca, s)], BlendConfig(full_first_layer=False))
    torch.testing.assert_close(naive["logits"], first["logits"], atol=2e-3, rtol=0)
    assert naive["stats"]["prefill_token_equiv"] == len(toks) - len(parts["a"])


def test_moved_chunks_full_recompute_and_blend(model, parts):
    s = len(parts["sys"])
    first = R.prefill(model, parts["sys"] + parts["a"] + parts["b"] + parts["q"])
    ca = chunk_of(first, s, s + len(parts["a"]))
    cb = chunk_of(first, s + len(parts["a"]), s + len(parts["a"]) + len(parts["b"]))
    toks2 = parts["sys"] + parts["b"] + parts["a"] + parts["q"]
    with torch.inference_mode():
        fwd = model(torch.tensor([toks2])).logits[0, -1:]
    pl = [Placement(cb, s), Placement(ca, s + len(parts["b"]))]
    full = R.prefill(model, toks2, pl, BlendConfig(recompute_ratio=1.0))
    naive = R.prefill(model, toks2, pl, BlendConfig(full_first_layer=False))
    blend = R.prefill(model, toks2, pl, BlendConfig(recompute_ratio=0.3))
    assert kl(fwd, full["logits"]) < 1e-4
    assert kl(fwd, blend["logits"]) < kl(fwd, naive["logits"])
    assert naive["stats"]["prefill_token_equiv"] < blend["stats"]["prefill_token_equiv"] < len(toks2)
    # the budget: 2 chunks, round(0.3*19)=6 and round(0.3*23)=7, plus 2 sinks each
    n_fresh = len(toks2) - len(parts["a"]) - len(parts["b"])
    assert blend["stats"]["recomputed_cached_tokens"] == 6 + 7 + 4
    assert len(blend["sel"]["keep_abs"]) == n_fresh + 17


def test_exact_chunk_skips_layer0(model, parts):
    s = len(parts["sys"])
    first = R.prefill(model, parts["sys"] + parts["a"] + parts["b"] + parts["q"])
    ca = chunk_of(first, s, s + len(parts["a"]))
    other = R.prefill(model, parts["sys"] + parts["b"] + parts["q"])
    cb = chunk_of(other, s, s + len(parts["b"]))
    toks = parts["sys"] + parts["a"] + parts["b"] + parts["q"]
    with torch.inference_mode():
        fwd = model(torch.tensor([toks])).logits[0, -1:]
    out = R.prefill(model, toks, [Placement(ca, s, exact=True), Placement(cb, s + len(parts["a"]), ratio=1.0)], BlendConfig())
    assert kl(fwd, out["logits"]) < 1e-4
    assert out["stats"]["prefill_token_equiv"] == len(toks) - len(parts["a"])


def test_full_budget_with_leading_exact_chunk(model, parts):
    first = R.prefill(model, parts["a"] + parts["b"] + parts["q"])
    ca = chunk_of(first, 0, len(parts["a"]))
    s = len(parts["sys"])
    other = R.prefill(model, parts["sys"] + parts["b"] + parts["q"])
    cb = chunk_of(other, s, s + len(parts["b"]))
    toks = parts["a"] + parts["b"] + parts["q"]
    with torch.inference_mode():
        fwd = model(torch.tensor([toks])).logits[0, -1:]
    out = R.prefill(model, toks, [Placement(ca, 0, exact=True), Placement(cb, len(parts["a"]), ratio=1.0)], BlendConfig())
    assert kl(fwd, out["logits"]) < 1e-4
    assert out["stats"]["prefill_token_equiv"] == len(toks) - len(parts["a"])


def test_logits_at_non_recomputed_positions_raise(model, parts):
    s = len(parts["sys"])
    first = R.prefill(model, parts["sys"] + parts["a"] + parts["q"])
    ca = chunk_of(first, s, s + len(parts["a"]))
    with pytest.raises(ValueError):
        R.prefill(model, parts["sys"] + parts["a"] + parts["q"], [Placement(ca, s, exact=True)], BlendConfig(), logits_from=s)


def test_rocm_baseline_is_the_same_op_sequence(model, parts):
    """TorchOpsEngine on CPU with torch's own inv_freq and argsort = the oracle with an unstable
    argsort: identical results, bit for bit."""
    s = len(parts["sys"])
    first = R.prefill(model, parts["sys"] + parts["a"] + parts["b"] + parts["q"])
    ca = chunk_of(first, s, s + len(parts["a"]))
    cb = chunk_of(first, s + len(parts["a"]), s + len(parts["a"]) + len(parts["b"]))
    toks2 = parts["sys"] + parts["b"] + parts["a"] + parts["q"]
    pl = [Placement(cb, s), Placement(ca, s + len(parts["b"]))]
    cfg = BlendConfig(recompute_ratio=0.3, n_sink=3, escalate_threshold=1e9)
    eng = TorchOpsEngine(model, StubTokenizer())
    a = eng.prefill(toks2, pl, cfg, logits_from=len(toks2) - 3)
    b = R.prefill(model, toks2, pl, cfg, logits_from=len(toks2) - 3, tie_stable=False)
    assert torch.equal(a.logits, b["logits"])
    assert a.stats == b["stats"]
    for x, y in zip(a.keys, b["keys"]):
        assert torch.equal(x, y)
