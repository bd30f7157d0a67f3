"""End-to-end properties at the full 8k request shape on a random-init Qwen2.5-7B architecture
(bf16): 24 chunks x 320 tokens prefilled on their own and placed in a shuffled order, then a
512-token uncached tail and a 64-token query (N = 8256), as in the benchmark.

- recompute_ratio 1.0 keeps every cached token, so every layer recomputes every position: the
  blend prefill must give exactly the no-cache prefill of the same tokens (same kernels, same
  rows), and the stats' closed forms hold (reference tests/test_torch_engine.py:61-64 states the
  same equivalence with a KL bound).
- recompute_ratio 0.3 against the reference op sequence on PyTorch-ROCm (TorchOpsEngine): the
  same stats (2304 pooled + 96 sinks + 576 uncached kept) and next-token distributions within a
  KL bound (the two differ in attention kernels and the correctly rounded cos/sin only).
- recompute_ratio 0.3 against the oracle on the engine's own layer-1 device inputs (the model's
  real activations at N = 8256): the deviation, the kept set, layer 1's cache after the scatter
  and the gathered rows of layers 2-27, bit for bit.
"""

import numpy as np
import pytest
import torch

from chunkkv_amd.baseline import TorchOpsEngine
from chunkkv_amd.engine import HipEngine
from chunkkv_amd.planner import plan_request
from chunkkv_amd.types import BlendConfig, Placement
from oracle import oracle as O
from tests.helpers import StubTokenizer, random_qwen25_7b

pytestmark = pytest.mark.gpu
DEV = "cuda"
L_CHUNK, N_CHUNKS, TAIL = 320, 24, 576


@pytest.fixture(scope="module")
def setup():
    model = random_qwen25_7b(DEV)
    eng = HipEngine(model, StubTokenizer())
    g = torch.Generator().manual_seed(3)
    pool = []
    for _ in range(N_CHUNKS):
        toks = torch.randint(0, 152064, (L_CHUNK,), generator=g).tolist()
        pool.append((toks, eng.prefill(toks).chunk(0, L_CHUNK)))
    tokens, placements = [], []
    for c in torch.randperm(N_CHUNKS, generator=g).tolist():
        placements.append(Placement(pool[c][1], len(tokens)))
        tokens += pool[c][0]
    tokens += torch.randint(0, 152064, (TAIL,), generator=g).tolist()
    yield model, eng, tokens, placements
    del eng, model, pool
    torch.cuda.empty_cache()


def _kl(p, q):
    p, q = torch.log_softmax(p.float(), -1), torch.log_softmax(q.float(), -1)
    return (p.exp() * (p - q)).sum(-1).mean().item()


def test_full_size_ratio_one_equals_full_prefill(setup):
    model, eng, tokens, placements = setup
    N = len(tokens)
    blend = eng.prefill(tokens, placements, BlendConfig(recompute_ratio=1.0, n_sink=4))
    full = eng.prefill(tokens)
    assert blend.stats["cached_tokens"] == N_CHUNKS * L_CHUNK
    assert blend.stats["recomputed_cached_tokens"] == N_CHUNKS * L_CHUNK
    assert blend.stats["prefill_token_equiv"] == N
    assert torch.equal(blend.logits, full.logits)
    for li in (0, 1, 2, 27):
        assert torch.equal(blend.keys[li], full.keys[li]) and torch.equal(blend.values[li], full.values[li])


def test_full_size_blend_matches_reference_ops(setup):
    model, eng, tokens, placements = setup
    cfg = BlendConfig(recompute_ratio=0.3, n_sink=4)
    a = eng.prefill(tokens, placements, cfg)
    b = TorchOpsEngine(model, StubTokenizer()).prefill(tokens, placements, cfg)
    assert a.stats["recomputed_cached_tokens"] == b.stats["recomputed_cached_tokens"] == 2304 + 96
    assert a.stats["prefill_token_equiv"] == b.stats["prefill_token_equiv"]
    kl = _kl(b.logits, a.logits)
    print(f"KL(reference ops || HipEngine) at the last position: {kl:.3e}")
    assert kl < 1e-2


def _oracle_layer(plan, li, N, H, D, theta):
    """Layer li's base cache as the oracle gathers it (uncovered rows left at zero)."""
    Ko = np.zeros((1, H, N, D), dtype=np.uint16)
    Vo = np.zeros_like(Ko)
    ks = [[O.to_numpy(ch.keys[li])[0]] for ch in plan.chunks]
    vs = [[O.to_numpy(ch.values[li])[0]] for ch in plan.chunks]
    assert O.rerope_gather(Ko, Vo, ks, vs, plan.segments, theta) == 0
    return Ko[0], Vo[0]


def test_full_size_layer1_repair_matches_oracle(setup):
    """The 8k request's layer-1 repair on the engine's own device inputs (the model's layer-1 k/v
    and the gathered base cache), against the oracle: diff/norm, the kept set, rel_dev, layer 1's
    cache after the scatter, and the dropped rows of layers 2, 13 and 27, all bit-exact."""
    model, eng, tokens, placements = setup
    N, H, D, theta = len(tokens), eng.n_kv, eng.head_dim, eng.theta
    cfg = BlendConfig(recompute_ratio=0.3, n_sink=4)
    eng.trace = {}
    res = eng.prefill(tokens, placements, cfg)
    tr, eng.trace = eng.trace, None
    plan = plan_request(N, placements, cfg.n_sink, cfg.recompute_ratio)
    n_keep = tr["n_keep"]
    assert n_keep == plan.n_keep == 2976

    k, v = O.to_numpy(tr["k"])[0], O.to_numpy(tr["v"])[0]
    K, V = O.to_numpy(tr["K"])[0], O.to_numpy(tr["V"])[0]
    flags, local = O.to_numpy(tr["flags"]), O.to_numpy(tr["local"])
    # the base cache the deviation read: every cached row gathered as the oracle does
    K1o, V1o = _oracle_layer(plan, 1, N, H, D, theta)
    np.testing.assert_array_equal(K[:, plan.cached], K1o[:, plan.cached])
    np.testing.assert_array_equal(V[:, plan.cached], V1o[:, plan.cached])

    d_o, n_o = O.deviation(k, v, K, V, flags, local)
    np.testing.assert_array_equal(O.to_numpy(tr["diff"]).view(np.uint32), d_o.view(np.uint32))
    np.testing.assert_array_equal(O.to_numpy(tr["norm"]).view(np.uint32), n_o.view(np.uint32))
    want = O.select(d_o, n_o, flags, local, plan.spans, None)
    sel = tr["sel"]
    np.testing.assert_array_equal(O.to_numpy(sel.keep_abs)[:n_keep], want["keep_abs"])
    np.testing.assert_array_equal(O.to_numpy(sel.keep_local)[:n_keep], want["keep_local"])
    np.testing.assert_array_equal(O.to_numpy(sel.keep_rank), want["keep_rank"])
    np.testing.assert_array_equal(O.to_numpy(sel.rel_dev).view(np.uint32), want["rel_dev"].view(np.uint32))
    np.testing.assert_array_equal(O.to_numpy(sel.counts)[:6], want["counts"][:6])
    assert [c["rel_dev"] for c in res.stats["chunks"]] == want["rel_dev"].tolist()

    # layer 1 after the scatter: kept rows = the fresh rows, every other cached row = base cache
    ka, kl = want["keep_abs"], want["keep_local"]
    K1, V1 = O.to_numpy(res.keys[1])[0], O.to_numpy(res.values[1])[0]
    np.testing.assert_array_equal(K1[:, ka], k[:, kl])
    np.testing.assert_array_equal(V1[:, ka], v[:, kl])
    dropped = plan.cached & (want["keep_rank"] < 0)
    np.testing.assert_array_equal(K1[:, dropped], K1o[:, dropped])
    np.testing.assert_array_equal(V1[:, dropped], V1o[:, dropped])

    # layers 2..27: the cached rows of the dropped positions, re-rotated and gathered
    for li in (2, 13, 27):
        Klo, Vlo = _oracle_layer(plan, li, N, H, D, theta)
        Kg, Vg = O.to_numpy(res.keys[li])[0], O.to_numpy(res.values[li])[0]
        np.testing.assert_array_equal(Kg[:, dropped], Klo[:, dropped])
        np.testing.assert_array_equal(Vg[:, dropped], Vlo[:, dropped])


def test_full_size_layer1_four_launches_identical(setup):
    """The 8k request with layer 1 as four launches (base cache, deviation, selection, kept-row
    scatter): the same caches and logits as the one-call default, bit for bit."""
    model, eng, tokens, placements = setup
    cfg = BlendConfig(recompute_ratio=0.3, n_sink=4)
    a = HipEngine(model, StubTokenizer(), layer1="four_launches").prefill(tokens, placements, cfg)
    b = eng.prefill(tokens, placements, cfg)
    assert torch.equal(a.logits, b.logits) and a.stats == b.stats
    for li in (0, 1, 2, 27):
        assert torch.equal(a.keys[li], b.keys[li]) and torch.equal(a.values[li], b.values[li])


def test_full_size_sdpa_mode_matches_reference_ops(setup):
    """HipEngine(attention="sdpa"): every KV-repair kernel, torch's fused SDPA kernels for the
    attention and torch's norm/MLP, against the reference op sequence at the 8k request: the same
    stats, next-token distributions within the KL bound."""
    model, _, tokens, placements = setup
    cfg = BlendConfig(recompute_ratio=0.3, n_sink=4)
    a = HipEngine(model, StubTokenizer(), attention="sdpa").prefill(tokens, placements, cfg)
    b = TorchOpsEngine(model, StubTokenizer()).prefill(tokens, placements, cfg)
    for k in ("cached_tokens", "recomputed_cached_tokens", "prefill_token_equiv"):
        assert a.stats[k] == b.stats[k], k
    assert a.stats["recomputed_cached_tokens"] == 2304 + 96
    kl = _kl(b.logits, a.logits)
    print(f"KL(reference ops || HipEngine sdpa) at the last position: {kl:.3e}")
    assert kl < 1e-2
