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
"""

import pytest
import torch

from chunkkv_amd.baseline import TorchOpsEngine
from chunkkv_amd.engine import HipEngine
from chunkkv_amd.types import BlendConfig, Placement
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
