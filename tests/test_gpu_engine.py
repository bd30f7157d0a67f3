"""End-to-end parity of HipEngine (HIP KV repair on the GPU) with the oracle's CPU restatement of
TorchEngine.prefill and with the reference op sequence on PyTorch-ROCm, on tiny random-init
Qwen2 models (fp32 and bf16), mirroring the reference's engine tests
(tests/test_torch_engine.py:36-74, tests/test_mlx_engine.py:24-99)."""

import copy

import numpy as np
import pytest
import torch

from chunkkv_amd.baseline import TorchOpsEngine
from chunkkv_amd.engine import HipEngine
from chunkkv_amd.types import BlendConfig, ChunkKV, Placement
from oracle import engine_ref as R
from oracle import oracle as O
from tests.helpers import StubTokenizer, tiny_qwen2

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def models():
    cpu = tiny_qwen2(layers=4, hidden=256, heads=4, kv=2, inter=512, vocab=512, seed=0)
    gpu = copy.deepcopy(cpu).to(DEV)
    return cpu, gpu


@pytest.fixture(scope="module")
def parts():
    rng = np.random.default_rng(0)
    t = lambda n: rng.integers(1, 511, n).tolist()  # noqa: E731
    return dict(sys=t(11), a=t(37), b=t(29), q=t(9))


def _kl(p, q):
    p, q = torch.log_softmax(p.float(), -1), torch.log_softmax(q.float(), -1)
    return (p.exp() * (p - q)).sum(-1).mean().item()


def _cpu_chunk(ch):
    return ChunkKV([k.detach().cpu() for k in ch.keys], [v.detach().cpu() for v in ch.values], ch.start)


def assert_same_selection(got, ref, tokens, placements, cfg):
    """Kept sets agree except for candidates whose deviation is within 1e-4 of the top-k
    threshold (the GPU and CPU models round layer-0/1 activations differently)."""
    from chunkkv_amd.planner import plan_request

    ref_set = set(ref["sel"]["keep_abs"].tolist())
    diffset = set(got.tolist()) ^ ref_set
    if not diffset:
        return
    plan = plan_request(len(tokens), placements, cfg.n_sink, cfg.recompute_ratio)
    cand = np.zeros(len(tokens), dtype=bool)
    for s0, L, _, pooled in plan.spans:
        if pooled:
            cand[s0 : s0 + L] = True
    cand &= ~(~plan.cached | plan.sink)
    d = ref["sel"]["diff"].double().numpy()
    thr = np.sort(d[cand])[::-1][plan.budget - 1]
    assert all(cand[p] and abs(d[p] - thr) <= 1e-4 * thr for p in diffset), (diffset, thr)


def _swap_setup(eng, parts):
    s = len(parts["sys"])
    first = eng.prefill(parts["sys"] + parts["a"] + parts["b"] + parts["q"])
    ca = first.chunk(s, s + len(parts["a"]))
    cb = first.chunk(s + len(parts["a"]), s + len(parts["a"]) + len(parts["b"]))
    toks2 = parts["sys"] + parts["b"] + parts["a"] + parts["q"]
    return toks2, [Placement(cb, s), Placement(ca, s + len(parts["b"]))]


def _to_cpu_placements(pl):
    return [Placement(_cpu_chunk(p.chunk), p.start, p.ratio, p.exact) for p in pl]


def test_no_cache_prefill_matches_hf_forward(models, parts):
    cpu, gpu = models
    eng = HipEngine(gpu, StubTokenizer())
    toks = parts["sys"] + parts["a"] + parts["b"] + parts["q"]
    with torch.inference_mode():
        ref = gpu(torch.tensor([toks], device=DEV)).logits[0]
    out = eng.prefill(toks, logits_from=0)
    torch.testing.assert_close(out.logits, ref, atol=2e-3, rtol=0)
    assert out.stats["prefill_token_equiv"] == len(toks)


@pytest.mark.parametrize("attention", ["reference", "fused"])
@pytest.mark.parametrize("ratio", [0.3, 1.0])
def test_blend_matches_oracle_engine(models, parts, attention, ratio):
    cpu, gpu = models
    eng = HipEngine(gpu, StubTokenizer(), attention=attention)
    toks2, pl = _swap_setup(eng, parts)
    cfg = BlendConfig(recompute_ratio=ratio, n_sink=4)
    eng.trace = {}
    out = eng.prefill(toks2, pl, cfg)
    tr, eng.trace = eng.trace, None
    ref = R.prefill(cpu, toks2, _to_cpu_placements(pl), cfg, inv_freq=eng.inv_freq.cpu())
    for key in ("tokens", "cached_tokens", "recomputed_cached_tokens", "prefill_token_equiv"):
        assert out.stats[key] == ref["stats"][key], key
    for a, b in zip(out.stats["chunks"], ref["stats"]["chunks"]):
        assert (a["start"], a["length"], a["escalated"]) == (b["start"], b["length"], b["escalated"])
        assert a["rel_dev"] == pytest.approx(b["rel_dev"], rel=1e-3)
    tol = 2e-3 if attention == "reference" else 5e-3
    torch.testing.assert_close(out.logits.cpu(), ref["logits"], atol=tol, rtol=0)
    # the engine's own layer-1 selection equals the C oracle's on the same device inputs
    n = tr["n_keep"]
    got = O.to_numpy(tr["sel"].keep_abs)[:n]
    want = O.select(O.to_numpy(tr["diff"]), O.to_numpy(tr["norm"]), O.to_numpy(tr["flags"]), O.to_numpy(tr["local"]),
                    O.to_numpy(tr["spans"]).reshape(-1, 4), cfg.escalate_threshold)
    np.testing.assert_array_equal(got, want["keep_abs"])
    # and the CPU reference's set, up to deviations tied within fp32 rounding
    assert_same_selection(got, ref, toks2, pl, cfg)


@pytest.mark.parametrize("ratio", [0.3, 0.0])
def test_side_stream_and_one_stream_builds_identical(models, parts, ratio):
    """Layers 2..L-1 built by the side-stream gather of dropped rows + per-layer scatters, or by
    one assemble launch per layer on the main stream: the same caches, bit for bit."""
    _, gpu = models
    a = HipEngine(gpu, StubTokenizer(), overlap=True)
    b = HipEngine(gpu, StubTokenizer())
    assert a.overlap and not b.overlap
    toks2, pl = _swap_setup(a, parts)
    cfg = BlendConfig(recompute_ratio=ratio, n_sink=4)
    ra, rb = a.prefill(toks2, pl, cfg), b.prefill(toks2, pl, cfg)
    torch.cuda.synchronize()
    assert len(ra.keys) > 2
    for x, y in zip(ra.keys + ra.values, rb.keys + rb.values):
        assert torch.equal(x, y)
    assert torch.equal(ra.logits, rb.logits)


@pytest.mark.parametrize("mode", ["four_launches", "fused_select"])
@pytest.mark.parametrize("thr", [None, 0.05])
def test_layer1_paths_build_identical(models, parts, thr, mode):
    """Layer 1's repair as one call (ckv_layer1_repair, the default), as the base-cache gather plus
    the deviation, the selection and the kept-row scatter, or with the deviation and selection as
    ckv_deviation_select: the same caches, logits and stats, bit for bit, with and without an
    escalation threshold."""
    _, gpu = models
    a = HipEngine(gpu, StubTokenizer(), layer1=mode)
    b = HipEngine(gpu, StubTokenizer())
    assert b.layer1 == "one_call"
    toks2, pl = _swap_setup(a, parts)
    cfg = BlendConfig(recompute_ratio=0.3, n_sink=4, escalate_threshold=thr)
    ra, rb = a.prefill(toks2, pl, cfg), b.prefill(toks2, pl, cfg)
    torch.cuda.synchronize()
    for x, y in zip(ra.keys + ra.values, rb.keys + rb.values):
        assert torch.equal(x, y)
    assert torch.equal(ra.logits, rb.logits)
    assert ra.stats == rb.stats


def test_blend_matches_rocm_reference_ops(models, parts):
    """Same device, same model, reference SDPA call: only the KV repair differs."""
    from chunkkv_amd.baseline import torch_base_kv

    _, gpu = models
    hip = HipEngine(gpu, StubTokenizer(), attention="reference")
    ref = TorchOpsEngine(gpu, StubTokenizer())
    toks2, pl = _swap_setup(hip, parts)
    cfg = BlendConfig(recompute_ratio=0.3, n_sink=2)
    hip.trace = {}
    a = hip.prefill(toks2, pl, cfg)
    tr, hip.trace = hip.trace, None
    b = ref.prefill(toks2, pl, cfg)
    for key in ("tokens", "cached_tokens", "recomputed_cached_tokens", "prefill_token_equiv"):
        assert a.stats[key] == b.stats[key], key
    assert _kl(b.logits, a.logits) < 1e-5
    # the layer-1 base cache built by the HIP gather vs the reference's torch ops
    K1, V1 = torch_base_kv(pl, 1, len(toks2), hip.n_kv, hip.head_dim, torch.float32, ref.inv_freq, DEV)
    cached = torch.zeros(len(toks2), dtype=torch.bool)
    for p in pl:
        cached[p.start : p.start + p.chunk.length] = True
    # within one bf16 ulp (2**-8 relative), the re-RoPE contract; torch's fp32 pow/cos are not
    # correctly rounded, so the two differ by a few fp32 ulps
    got, want = tr["K"][:, :, cached], K1[:, :, cached]
    assert ((got - want).abs() <= 2.0**-8 * want.abs() + 1e-6 * want.abs().max()).all()
    assert torch.equal(tr["V"][:, :, cached], V1[:, :, cached])


def test_full_recompute_matches_forward_and_blend_beats_naive(models, parts):
    """reference tests/test_torch_engine.py:52-65."""
    _, gpu = models
    eng = HipEngine(gpu, StubTokenizer())
    toks2, pl = _swap_setup(eng, parts)
    with torch.inference_mode():
        fwd = gpu(torch.tensor([toks2], device=DEV)).logits[0, -1:]
    full = eng.prefill(toks2, pl, BlendConfig(recompute_ratio=1.0))
    naive = eng.prefill(toks2, pl, BlendConfig(full_first_layer=False))
    blend = eng.prefill(toks2, pl, BlendConfig(recompute_ratio=0.3))
    assert _kl(fwd, full.logits) < 1e-4
    assert _kl(fwd, blend.logits) < _kl(fwd, naive.logits)
    assert naive.stats["prefill_token_equiv"] < blend.stats["prefill_token_equiv"] < len(toks2)


def test_exact_reuse_and_stats_closed_forms(models, parts):
    """reference tests/test_torch_engine.py:44-49 and tests/test_mlx_engine.py:32-39, 70-99."""
    _, gpu = models
    eng = HipEngine(gpu, StubTokenizer())
    s = len(parts["sys"])
    toks = parts["sys"] + parts["a"] + parts["b"] + parts["q"]
    first = eng.prefill(toks)
    ca = first.chunk(s, s + len(parts["a"]))
    same = eng.prefill(toks, [Placement(ca, s, exact=True)], BlendConfig())
    torch.testing.assert_close(same.logits, first.logits, atol=2e-3, rtol=0)
    assert same.stats["prefill_token_equiv"] == len(toks) - len(parts["a"])
    naive = eng.prefill(toks, [Placement(ca, s)], BlendConfig(full_first_layer=False))
    assert naive.stats["prefill_token_equiv"] == len(toks) - len(parts["a"])
    # exact chunk at 0 + moved chunk at ratio 1.0: equals the full forward, exact never recomputed
    other = eng.prefill(parts["sys"] + parts["b"] + parts["q"])
    cb = other.chunk(s, s + len(parts["b"]))
    toks3 = parts["a"] + parts["b"] + parts["q"]
    a0 = eng.prefill(toks3).chunk(0, len(parts["a"]))
    with torch.inference_mode():
        fwd = gpu(torch.tensor([toks3], device=DEV)).logits[0, -1:]
    out = eng.prefill(toks3, [Placement(a0, 0, exact=True), Placement(cb, len(parts["a"]), ratio=1.0)], BlendConfig())
    assert _kl(fwd, out.logits) < 1e-4
    assert out.stats["prefill_token_equiv"] == len(toks3) - len(parts["a"])


def test_escalation_and_errors(models, parts):
    _, gpu = models
    eng = HipEngine(gpu, StubTokenizer())
    toks2, pl = _swap_setup(eng, parts)
    out = eng.prefill(toks2, pl, BlendConfig(escalate_threshold=0.0))  # every chunk escalates
    assert all(c["escalated"] for c in out.stats["chunks"])
    assert out.stats["recomputed_cached_tokens"] == out.stats["cached_tokens"]
    with pytest.raises(ValueError):
        eng.prefill(toks2, pl, BlendConfig(), logits_from=len(parts["sys"]))  # cached positions not recomputed
    with pytest.raises(ValueError):
        eng.prefill(toks2, [Placement(pl[0].chunk, len(toks2) - 3)], BlendConfig())  # runs past the request


def test_generate_matches_hf_greedy(models, parts):
    """reference tests/test_torch_engine.py:68-74 (logits sharpened so greedy picks are not
    near-ties on a random model)."""
    _, base = models
    gpu = copy.deepcopy(base)
    with torch.no_grad():
        gpu.model.norm.weight.mul_(20.0)
    eng = HipEngine(gpu, StubTokenizer())
    toks = parts["sys"] + parts["a"] + parts["q"]
    ours = eng.generate(eng.prefill(toks), max_tokens=8)
    with torch.inference_mode():
        ref = gpu.generate(torch.tensor([toks], device=DEV), max_new_tokens=8, do_sample=False,
                           attention_mask=torch.ones(1, len(toks), dtype=torch.long, device=DEV))[0, len(toks):]
    ref = [t for t in ref.tolist() if t not in eng.eos]
    assert ours == ref[: len(ours)] and len(ours) > 0


@pytest.mark.parametrize("heads,kv", [(4, 4), (8, 2)])
def test_bf16_generate_on_preallocated_cache_matches_concat_decode(heads, kv):
    """bf16 decode on the preallocated slab (in-place row writes, positions-masked attention)
    gives the same greedy tokens as the reference-style torch.cat decode over the same prefill
    (logits sharpened so greedy picks are not near-ties)."""
    from chunkkv_amd.model import DecoderPieces

    gpu = tiny_qwen2(layers=3, hidden=512, heads=heads, kv=kv, inter=1024, vocab=512, seed=6, dtype=torch.bfloat16).to(DEV)
    with torch.no_grad():
        gpu.model.norm.weight.mul_(20.0)
    eng = HipEngine(gpu, StubTokenizer())
    assert eng._native_attention
    rng = np.random.default_rng(6)
    res = eng.prefill(rng.integers(1, 511, 300).tolist())
    ours = eng.generate(res, max_tokens=12)  # device loop, HIP graph replays
    ref = DecoderPieces.generate(eng, res, max_tokens=12)
    assert len(ours) > 0 and ours == ref
    eng.decode_graphs = False
    assert eng.generate(res, max_tokens=12) == ours  # the same steps issued eagerly


@pytest.mark.parametrize("attention,heads,kv", [("reference", 4, 4), ("fused", 4, 4), ("fused", 8, 2)])
def test_bf16_blend_matches_rocm_reference_ops(attention, heads, kv):
    """bf16 model: HipEngine (reference SDPA call, or the fused path with the positions-masked
    matrix-core attention at head_dim 128 and 64 with GQA) vs the reference op sequence."""
    gpu = tiny_qwen2(layers=3, hidden=512, heads=heads, kv=kv, inter=1024, vocab=512, seed=3, dtype=torch.bfloat16).to(DEV)
    hip = HipEngine(gpu, StubTokenizer(), attention=attention)
    assert hip._native_attention
    ref = TorchOpsEngine(gpu, StubTokenizer())
    rng = np.random.default_rng(3)
    t = lambda n: rng.integers(1, 511, n).tolist()  # noqa: E731
    parts = dict(sys=t(20), a=t(64), b=t(48), q=t(8))
    toks2, pl = _swap_setup(hip, parts)
    cfg = BlendConfig(recompute_ratio=0.3, n_sink=4)
    a, b = hip.prefill(toks2, pl, cfg), ref.prefill(toks2, pl, cfg)
    assert a.stats["recomputed_cached_tokens"] == b.stats["recomputed_cached_tokens"]
    assert _kl(b.logits, a.logits) < 1e-3
    # with an exact placement (its rows never recomputed, gathered at layer 0 as well) and an
    # escalation threshold (the kept count read back from the device)
    sys_chunk = hip.prefill(parts["sys"]).chunk(0, len(parts["sys"]))
    pl2 = [Placement(sys_chunk, 0, exact=True)] + pl
    cfg2 = BlendConfig(recompute_ratio=0.3, n_sink=4, escalate_threshold=0.05)
    a2, b2 = hip.prefill(toks2, pl2, cfg2), ref.prefill(toks2, pl2, cfg2)
    for key in ("cached_tokens", "recomputed_cached_tokens", "prefill_token_equiv"):
        assert a2.stats[key] == b2.stats[key], key
    assert [c["escalated"] for c in a2.stats["chunks"]] == [c["escalated"] for c in b2.stats["chunks"]]
    assert _kl(b2.logits, a2.logits) < 1e-3


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fused_decoder_steps_match_the_model_modules(dtype):
    """The fused residual-add + RMSNorm and gated-product kernels (with the MLP's residual add
    deferred to the next norm) against the same engine running the model's own modules: same
    selection and stats, logits and decode within floating-point rounding."""
    gpu = tiny_qwen2(layers=3, hidden=512, heads=8, kv=2, inter=1024, vocab=512, seed=8, dtype=dtype).to(DEV)
    with torch.no_grad():
        gpu.model.norm.weight.mul_(20.0)
    fused, plain = HipEngine(gpu, StubTokenizer()), HipEngine(gpu, StubTokenizer())
    assert fused._fused_mlp
    plain._fused_mlp = False
    rng = np.random.default_rng(8)
    t = lambda n: rng.integers(1, 511, n).tolist()  # noqa: E731
    parts = dict(sys=t(20), a=t(64), b=t(48), q=t(8))
    toks2, pl = _swap_setup(plain, parts)
    cfg = BlendConfig(recompute_ratio=0.3, n_sink=4)
    a, b = fused.prefill(toks2, pl, cfg, logits_from=len(toks2) - 5), plain.prefill(toks2, pl, cfg, logits_from=len(toks2) - 5)
    for key in ("cached_tokens", "recomputed_cached_tokens", "prefill_token_equiv"):
        assert a.stats[key] == b.stats[key], key
    for ca, cb in zip(a.stats["chunks"], b.stats["chunks"]):
        assert ca["rel_dev"] == pytest.approx(cb["rel_dev"], rel=1e-2 if dtype == torch.bfloat16 else 1e-5)
    assert _kl(b.logits, a.logits) < (1e-4 if dtype == torch.bfloat16 else 1e-8)
    # layer 0 recomputes a fixed set of rows from the embeddings through the first norm
    torch.testing.assert_close(a.keys[0], b.keys[0], atol=0.05 if dtype == torch.bfloat16 else 1e-5, rtol=0)
    assert fused.generate(a, max_tokens=8) == plain.generate(a, max_tokens=8)


def test_shift_keys_api(models):
    _, gpu = models
    eng = HipEngine(gpu, StubTokenizer())
    k = torch.randn(1, 2, 10, 64, device=DEV)
    assert eng.shift_keys(k, 0) is k
    back = eng.shift_keys(eng.shift_keys(k, 37), -37)
    torch.testing.assert_close(back, k, atol=1e-5, rtol=0)


def test_repair_step_graph_replay_matches_eager():
    """The KV-repair step as the engine issues it (assemble L0; base cache, deviation, selection
    and scatter at L1; side-stream gather of the dropped rows of L2.. joined with the per-layer
    scatters), captured into one HIP graph across both streams and replayed several times with
    eager work in between: every replay gives the eager result (no memset nodes are recorded),
    and that result equals the one-stream build with one assemble launch per layer."""
    from chunkkv_amd import ops
    from chunkkv_amd.planner import local_index, plan_request

    rng = np.random.default_rng(5)
    H, D, L, C, n_layers = 4, 128, 64, 6, 4
    N = C * L + 16
    chunks = [ChunkKV([torch.randn(1, H, L, D, device=DEV).bfloat16() for _ in range(n_layers)],
                      [torch.randn(1, H, L, D, device=DEV).bfloat16() for _ in range(n_layers)], int(rng.integers(0, 900)))
              for _ in range(C)]
    pl = [Placement(chunks[c], i * L) for i, c in enumerate(rng.permutation(C))]
    plan = plan_request(N, pl, 4, 0.3)
    tab = np.concatenate([np.array([[k.data_ptr(), v.data_ptr()] for k, v in zip(c.keys, c.values)], dtype=np.uint64).reshape(-1)
                          for c in plan.chunks])
    tab_d = torch.from_numpy(tab.view(np.int64)).to(DEV)
    segs = torch.from_numpy(plan.all_segments.reshape(-1)).to(DEV)  # cached runs first
    n_c, n_all = len(plan.segments), len(plan.all_segments)
    flags = torch.from_numpy(plan.flags).to(DEV)
    local = torch.from_numpy(local_index(N, plan.layer0_idx)).to(DEV)
    spans = torch.from_numpy(plan.spans.reshape(-1)).to(DEV)
    n_keep = plan.n_keep
    fk = torch.randn(1, H, N, D, device=DEV).bfloat16()
    fv = torch.randn(1, H, N, D, device=DEV).bfloat16()
    side = torch.cuda.Stream()

    def make(two_streams):
        Ks = torch.empty((n_layers, 1, H, N, D), dtype=torch.bfloat16, device=DEV)
        Vs = torch.empty_like(Ks)
        state = {}

        def step():
            ops.assemble_layer(Ks[0], Vs[0], tab_d, n_layers, 0, segs, n_all, plan.max_all_seg_tokens, fk, fv, local, 1e6)
            ops.assemble_layer(Ks[1], Vs[1], tab_d, n_layers, 1, segs, n_c, plan.max_seg_tokens, None, None, None, 1e6)
            diff, norm = ops.deviation(fk, fv, Ks[1], Vs[1], flags, local)
            sel = state["sel"] = ops.select(diff, norm, flags, local, spans, None, state.get("sel"))
            rows = sel.keep_abs[:n_keep]
            ops.scatter_rows(Ks[1], Vs[1], fk[:, :, :n_keep], fv[:, :, :n_keep], rows)
            if two_streams:
                main = torch.cuda.current_stream()
                side.wait_stream(main)
                with torch.cuda.stream(side):
                    ops.rerope_gather(Ks, Vs, tab_d, segs, n_c, plan.max_seg_tokens, 1e6, layers=(2, n_layers),
                                      skip=sel.keep_rank)
                for li in range(2, n_layers):
                    ops.scatter_rows(Ks[li], Vs[li], fk[:, :, :n_keep], fv[:, :, :n_keep], rows)
                main.wait_stream(side)
            else:
                for li in range(2, n_layers):
                    ops.assemble_layer(Ks[li], Vs[li], tab_d, n_layers, li, segs, n_all, plan.max_all_seg_tokens,
                                       fk[:, :, :n_keep], fv[:, :, :n_keep], sel.keep_rank, 1e6)

        return Ks, Vs, state, step

    Ks, Vs, state, step = make(True)
    Ks.fill_(7.0)  # every row is written: no 7.0 may survive
    Vs.fill_(7.0)
    step()
    torch.cuda.synchronize()
    eager = (Ks.clone(), Vs.clone(), state["sel"].keep_abs[:n_keep].clone())
    assert not (Ks == 7.0).all(dim=-1).any()
    Ks1, Vs1, _, step1 = make(False)
    step1()
    torch.cuda.synchronize()
    assert torch.equal(Ks1, eager[0]) and torch.equal(Vs1, eager[1])

    warm = torch.cuda.Stream()
    warm.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(warm):
        step()
    torch.cuda.current_stream().wait_stream(warm)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for _ in range(3):
        Ks.fill_(7.0)
        Vs.fill_(7.0)
        state["sel"].keep_abs.fill_(-1)
        state["sel"].keep_rank.fill_(-1)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(Ks, eager[0]) and torch.equal(Vs, eager[1])
        assert torch.equal(state["sel"].keep_abs[:n_keep], eager[2])


@pytest.mark.parametrize("attention", ["reference", "fused"])
def test_config1_qwen25_05b_shape_matches_oracle(attention):
    """Config 1: Qwen2.5-0.5B architecture (24 layers, hidden 896, 14 Q / 2 KV heads, head_dim 64,
    theta 1e6, vocab 151936, intermediate 4864, tied embeddings), random init, fp32. Four chunks of
    256 random ids prefilled at 0..1023, placed in a shuffled order, plus a 32-token query;
    15% recompute with 4 sinks. HipEngine on the GPU vs the oracle on the CPU, same chunk bytes."""
    from transformers import Qwen2Config, Qwen2ForCausalLM

    cfg = Qwen2Config(vocab_size=151936, hidden_size=896, intermediate_size=4864, num_hidden_layers=24,
                      num_attention_heads=14, num_key_value_heads=2, max_position_embeddings=32768, rope_theta=1e6,
                      tie_word_embeddings=True, rms_norm_eps=1e-6)
    torch.manual_seed(0)
    cpu = Qwen2ForCausalLM(cfg).eval()
    gpu = copy.deepcopy(cpu).to(DEV)
    eng = HipEngine(gpu, StubTokenizer(), attention=attention)
    rng = np.random.default_rng(1)
    docs = [rng.integers(0, 151936, 256).tolist() for _ in range(4)]
    first = eng.prefill(sum(docs, []))
    chunks = [first.chunk(i * 256, (i + 1) * 256) for i in range(4)]
    order = rng.permutation(4).tolist()
    query = rng.integers(0, 151936, 32).tolist()
    tokens = sum((docs[i] for i in order), []) + query
    pl = [Placement(chunks[i], k * 256) for k, i in enumerate(order)]
    bc = BlendConfig(recompute_ratio=0.15, n_sink=4)
    eng.trace = {}
    out = eng.prefill(tokens, pl, bc)
    tr, eng.trace = eng.trace, None
    ref = R.prefill(cpu, tokens, _to_cpu_placements(pl), bc, inv_freq=eng.inv_freq.cpu())
    assert out.stats["cached_tokens"] == 1024 and out.stats["recomputed_cached_tokens"] == 16 + 4 * 38
    for key in ("tokens", "cached_tokens", "recomputed_cached_tokens", "prefill_token_equiv"):
        assert out.stats[key] == ref["stats"][key], key
    for a, b in zip(out.stats["chunks"], ref["stats"]["chunks"]):
        assert (a["start"], a["length"], a["escalated"]) == (b["start"], b["length"], b["escalated"])
        assert a["rel_dev"] == pytest.approx(b["rel_dev"], rel=1e-3)
    n = tr["n_keep"]
    got = O.to_numpy(tr["sel"].keep_abs)[:n]
    want = O.select(O.to_numpy(tr["diff"]), O.to_numpy(tr["norm"]), O.to_numpy(tr["flags"]), O.to_numpy(tr["local"]),
                    O.to_numpy(tr["spans"]).reshape(-1, 4), None)
    np.testing.assert_array_equal(got, want["keep_abs"])
    assert_same_selection(got, ref, tokens, pl, bc)
    assert _kl(ref["logits"], out.logits.cpu()) < 1e-4


def test_chunk_address_memo_follows_replaced_layers(models, parts):
    """A stored chunk whose layer tensor is replaced must not be gathered from the old address."""
    _, gpu = models
    eng = HipEngine(gpu, StubTokenizer())
    toks2, pl = _swap_setup(eng, parts)
    cfg = BlendConfig(recompute_ratio=0.3, n_sink=2)
    first = eng.prefill(toks2, pl, cfg)
    ch = pl[0].chunk
    old = ch.keys[2]
    ch.keys[2] = old.clone() * 0.5  # a new tensor object with different contents
    second = eng.prefill(toks2, pl, cfg)
    ch.keys[2] = old
    third = eng.prefill(toks2, pl, cfg)
    assert not torch.equal(first.keys[2], second.keys[2])
    assert torch.equal(first.keys[2], third.keys[2]) and torch.equal(first.logits, third.logits)
