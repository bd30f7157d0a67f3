"""GPU parity of each HIP kernel against the C oracle on the same seeded inputs.

Bar: gather, scatter and the selected index set bit-exact; deviation
bit-exact under the fixed summation order; re-RoPE keys within one bf16 ulp (fp32 keys within
a few fp32 ulps: cos/sin come from different libraries on host and device).
"""

import numpy as np
import pytest
import torch

from chunkkv_amd import _native, ops
from chunkkv_amd.planner import plan_request
from oracle import oracle as O
from tests.helpers import bf16_ulp_distance

pytestmark = pytest.mark.gpu
DEV = "cuda"
THETA = 1e6


def dev(a):
    return O.from_numpy(a, DEV)


def host(t):
    return O.to_numpy(t)


def rand_elems(rng, shape, bf16, scale=1.0):
    a = (rng.standard_normal(shape) * scale).astype(np.float32)
    return O.f32_to_bf16_bits(a) if bf16 else a


def assert_keys_close(got, want, bf16, frac_exact=None):
    """Re-rotated keys: the kernel and the oracle use the same correctly rounded cos/sin table
    and IEEE fp32 products/sums, so they agree bit-for-bit (well inside the 1-ulp contract)."""
    if bf16:
        d = bf16_ulp_distance(got, want)
        assert d.max() == 0, f"max ulp distance {d.max()} at {np.argwhere(d == d.max())[:3].tolist()}"
    else:
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("theta", [1e4, 5e5, 1e6])
def test_inv_freq_kernel_bit_exact(D, theta):
    got = host(ops.inv_freq(D, theta, DEV))
    np.testing.assert_array_equal(got.view(np.uint32), O.inv_freq(D, theta).view(np.uint32))


@pytest.mark.parametrize("bf16", [True, False])
@pytest.mark.parametrize("D", [64, 128])
def test_shift_keys_kernel(bf16, D):
    rng = np.random.default_rng(D + bf16)
    x = rand_elems(rng, (1, 4, 300, D), bf16)
    xt = dev(x)
    assert ops.shift_keys(xt, 0, THETA) is xt
    for delta in [1, -1, 37, 4096, -4096, 123457]:
        got = host(ops.shift_keys(xt, delta, THETA))
        assert_keys_close(got, O.shift_keys(x, delta, THETA), bf16)


def _gather_case(rng, bf16, n_layers, H, D, lens, N, overlap=False):
    class C:  # minimal ChunkKV stand-in for the planner
        def __init__(self, L, start):
            self.keys = [np.zeros((1, H, L, D))]
            self.start = start

    class P:
        def __init__(self, chunk, start, exact=False):
            self.chunk, self.start, self.exact, self.ratio = chunk, start, exact, None

    chunks = [C(L, int(rng.integers(0, 5000))) for L in lens]
    for i, c in enumerate(chunks):
        c.idx = i  # position in ks/vs; plan.chunks lists chunks in placement order
    # place chunks at shuffled non-overlapping slots (or overlapping ones)
    order = rng.permutation(len(chunks))
    pos, placements = 0, []
    for i in order:
        placements.append(P(chunks[i], pos, exact=bool(rng.random() < 0.2)))
        pos += lens[i] - (lens[i] // 3 if overlap else 0) + int(rng.integers(0, 5))
    assert pos <= N
    plan = plan_request(N, placements, 4, 0.3)
    ks = [[rand_elems(rng, (H, L, D), bf16) for _ in range(n_layers)] for L in lens]
    vs = [[rand_elems(rng, (H, L, D), bf16) for _ in range(n_layers)] for L in lens]
    return plan, ks, vs


def _run_gather(plan, ks, vs, n_layers, H, D, N, bf16):
    dt = torch.bfloat16 if bf16 else torch.float32
    src = [([dev(k) for k in kl], [dev(v) for v in vl]) for kl, vl in zip(ks, vs)]
    # chunk order in the plan follows first appearance; map back to the list index
    tab = np.zeros((len(plan.chunks), n_layers, 2), dtype=np.uint64)
    for ci, ch in enumerate(plan.chunks):
        kl, vl = src[ch.idx]
        for l in range(n_layers):
            tab[ci, l, 0] = kl[l].data_ptr()
            tab[ci, l, 1] = vl[l].data_ptr()
    sentinel = -7.0
    K = torch.full((n_layers, 1, H, N, D), sentinel, dtype=dt, device=DEV)
    V = torch.full_like(K, sentinel)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    tab_t = torch.from_numpy(tab.view(np.int64)).to(DEV)
    segs_t = torch.from_numpy(plan.segments.reshape(-1)).to(DEV)
    ops.rerope_gather(K, V, tab_t, segs_t, len(plan.segments), plan.max_seg_tokens, THETA, err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    # oracle, same segments (chunk indices refer to plan.chunks order)
    okl = [ks[ch.idx] for ch in plan.chunks]
    ovl = [vs[ch.idx] for ch in plan.chunks]
    npdt = np.uint16 if bf16 else np.float32
    sent = O.f32_to_bf16_bits(np.float32([sentinel]))[0] if bf16 else np.float32(sentinel)
    Ko = np.full((n_layers, H, N, D), sent, dtype=npdt)
    Vo = np.full_like(Ko, sent)
    assert O.rerope_gather(Ko, Vo, okl, ovl, plan.segments, THETA) == 0
    return host(K).reshape(n_layers, H, N, D), host(V).reshape(n_layers, H, N, D), Ko, Vo, src


@pytest.mark.parametrize("bf16", [True, False])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("overlap", [False, True])
def test_rerope_gather_matches_oracle(bf16, D, overlap):
    rng = np.random.default_rng(100 + D + 2 * bf16 + overlap)
    n_layers, H = 3, 2
    lens = [40, 70, 33, 64, 1, 97]
    N = sum(lens) + 40
    plan, ks, vs = _gather_case(rng, bf16, n_layers, H, D, lens, N, overlap)
    Kg, Vg, Ko, Vo, _ = _run_gather(plan, ks, vs, n_layers, H, D, N, bf16)
    np.testing.assert_array_equal(Vg, Vo)  # values: pure copies
    rot = np.zeros(N, dtype=bool)
    for s, n, c, s0, L, delta in plan.segments:
        if delta != 0:
            rot[s : s + n] = True
    np.testing.assert_array_equal(Kg[:, :, ~rot], Ko[:, :, ~rot])  # delta 0 and untouched rows
    assert_keys_close(Kg[:, :, rot], Ko[:, :, rot], bf16)


@pytest.mark.parametrize("layers", [(0, 3), (1, 3), (2, 2)])
def test_rerope_gather_layer_range_with_skip_map(layers):
    """Layers [begin, end) only, rows of positions with skip >= 0 untouched: equals the oracle's
    full gather on exactly the remaining rows."""
    bf16, D = True, 128
    rng = np.random.default_rng(300 + layers[0])
    n_layers, H = 3, 2
    lens = [40, 70, 33, 64, 1, 97]
    N = sum(lens) + 40
    plan, ks, vs = _gather_case(rng, bf16, n_layers, H, D, lens, N, True)
    _, _, Ko, Vo, src = _run_gather(plan, ks, vs, n_layers, H, D, N, bf16)
    skip = np.full(N, -1, dtype=np.int32)
    kept = np.flatnonzero(rng.random(N) < 0.4)
    skip[kept] = np.arange(len(kept), dtype=np.int32)
    tab = np.zeros((len(plan.chunks), n_layers, 2), dtype=np.uint64)
    for ci, ch in enumerate(plan.chunks):
        for l in range(n_layers):
            tab[ci, l] = src[ch.idx][0][l].data_ptr(), src[ch.idx][1][l].data_ptr()
    K = torch.full((n_layers, 1, H, N, D), -7.0, dtype=torch.bfloat16, device=DEV)
    V = torch.full_like(K, -7.0)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    ops.rerope_gather(K, V, torch.from_numpy(tab.view(np.int64)).to(DEV), dev(plan.segments.reshape(-1)),
                      len(plan.segments), plan.max_seg_tokens, THETA, err, layers=layers, skip=dev(skip))
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    Kg, Vg = host(K).reshape(n_layers, H, N, D), host(V).reshape(n_layers, H, N, D)
    sent = O.f32_to_bf16_bits(np.float32([-7.0]))[0]
    want_k, want_v = np.full_like(Ko, sent), np.full_like(Vo, sent)
    rows = np.flatnonzero(skip < 0)
    for l in range(*layers):
        want_k[l][:, rows], want_v[l][:, rows] = Ko[l][:, rows], Vo[l][:, rows]
    np.testing.assert_array_equal(Kg, want_k)
    np.testing.assert_array_equal(Vg, want_v)


@pytest.mark.parametrize("lens,pattern", [
    ([300, 700, 257, 1, 64], "per_segment"),  # several 256-token ranking rounds per segment
    ([40, 70, 33, 64, 1, 97], "all_or_none"),  # whole segments kept or gathered
    ([5000, 30], "per_segment"),               # past the compacted path's segment limit
])
def test_rerope_gather_skip_map_uneven_selection(lens, pattern):
    """Skip maps as a selection leaves them: the kept share differs per segment (0% to 100%), so
    the gathered rows of a segment are ranked across several rounds, some segments gather
    nothing and some everything. Every remaining row equals the oracle's full gather; kept rows
    stay untouched."""
    bf16, D, layers = True, 64, (1, 3)
    rng = np.random.default_rng(sum(lens))
    n_layers, H = 3, 2
    N = sum(lens) + 5 * len(lens)
    plan, ks, vs = _gather_case(rng, bf16, n_layers, H, D, lens, N, False)
    _, _, Ko, Vo, src = _run_gather(plan, ks, vs, n_layers, H, D, N, bf16)
    keep = rng.random(N) < 0.5  # uncached positions are irrelevant to the gather
    for i, (s0, n, *_rest) in enumerate(plan.segments):
        share = rng.choice([0.0, 0.05, 0.5, 0.95, 1.0]) if pattern == "per_segment" else float(i % 2)
        keep[s0 : s0 + n] = rng.random(n) < share
    skip = np.where(keep, 0, -1).astype(np.int32)
    tab = np.zeros((len(plan.chunks), n_layers, 2), dtype=np.uint64)
    for ci, ch in enumerate(plan.chunks):
        for l in range(n_layers):
            tab[ci, l] = src[ch.idx][0][l].data_ptr(), src[ch.idx][1][l].data_ptr()
    K = torch.full((n_layers, 1, H, N, D), -7.0, dtype=torch.bfloat16, device=DEV)
    V = torch.full_like(K, -7.0)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    ops.rerope_gather(K, V, torch.from_numpy(tab.view(np.int64)).to(DEV), dev(plan.segments.reshape(-1)),
                      len(plan.segments), plan.max_seg_tokens, THETA, err, layers=layers, skip=dev(skip))
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    Kg, Vg = host(K).reshape(n_layers, H, N, D), host(V).reshape(n_layers, H, N, D)
    sent = O.f32_to_bf16_bits(np.float32([-7.0]))[0]
    want_k, want_v = np.full_like(Ko, sent), np.full_like(Vo, sent)
    rows = np.flatnonzero(skip < 0)
    for l in range(*layers):
        want_k[l][:, rows], want_v[l][:, rows] = Ko[l][:, rows], Vo[l][:, rows]
    np.testing.assert_array_equal(Kg, want_k)
    np.testing.assert_array_equal(Vg, want_v)


@pytest.mark.parametrize("bf16,D", [(True, 128), (False, 64)])
def test_rerope_gather_many_segments(bf16, D):
    """Launches of 64 or more segments take the segment-fastest launch shape: 80 ragged segments
    (1-40 tokens), every layer without a skip map and layers 1-2 with one, against the oracle."""
    rng = np.random.default_rng(640 + D)
    n_layers, H = 3, 2
    lens = [int(x) for x in rng.integers(1, 41, 80)]
    N = sum(lens) + 5 * len(lens)
    plan, ks, vs = _gather_case(rng, bf16, n_layers, H, D, lens, N, False)
    assert len(plan.segments) >= 64
    Kg, Vg, Ko, Vo, src = _run_gather(plan, ks, vs, n_layers, H, D, N, bf16)
    np.testing.assert_array_equal(Vg, Vo)
    rot = np.zeros(N, dtype=bool)
    for s0, n, c, _s, _L, delta in plan.segments:
        if delta != 0:
            rot[s0 : s0 + n] = True
    np.testing.assert_array_equal(Kg[:, :, ~rot], Ko[:, :, ~rot])
    assert_keys_close(Kg[:, :, rot], Ko[:, :, rot], bf16)
    dt = torch.bfloat16 if bf16 else torch.float32
    skip = np.where(rng.random(N) < 0.3, 0, -1).astype(np.int32)
    tab = np.zeros((len(plan.chunks), n_layers, 2), dtype=np.uint64)
    for ci, ch in enumerate(plan.chunks):
        for l in range(n_layers):
            tab[ci, l] = src[ch.idx][0][l].data_ptr(), src[ch.idx][1][l].data_ptr()
    K = torch.full((n_layers, 1, H, N, D), -7.0, dtype=dt, device=DEV)
    V = torch.full_like(K, -7.0)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    ops.rerope_gather(K, V, torch.from_numpy(tab.view(np.int64)).to(DEV), dev(plan.segments.reshape(-1)),
                      len(plan.segments), plan.max_seg_tokens, THETA, err, layers=(1, 3), skip=dev(skip))
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    Ks, Vs = host(K).reshape(n_layers, H, N, D), host(V).reshape(n_layers, H, N, D)
    rows = np.flatnonzero(skip < 0)
    sent = O.f32_to_bf16_bits(np.float32([-7.0]))[0] if bf16 else np.float32(-7.0)
    for l in range(n_layers):
        if l == 0:
            assert (Ks[0] == sent).all() and (Vs[0] == sent).all()
            continue
        np.testing.assert_array_equal(Ks[l][:, rows], Kg[l][:, rows])
        np.testing.assert_array_equal(Vs[l][:, rows], Vg[l][:, rows])
        kept = np.flatnonzero(skip >= 0)
        assert (Ks[l][:, kept] == sent).all() and (Vs[l][:, kept] == sent).all()


def _rope_rows(x, pos, theta):
    """x (..., n, D) fp32 rotated at positions pos (n,) (rotate-half, torch_engine.py:46-54): angles
    in fp64, the rotation in fp32."""
    D = x.shape[-1]
    inv = theta ** (-torch.arange(0, D, 2, dtype=torch.float64, device=x.device) / D)
    ang = pos.to(torch.float64)[:, None] * inv[None, :]
    c, s = ang.cos().float(), ang.sin().float()
    x1, x2 = x[..., : D // 2], x[..., D // 2 :]
    return torch.cat((x1 * c - x2 * s, x1 * s + x2 * c), -1)


def test_rerope_gather_config2_full_size():
    """Re-RoPE + gather at the Qwen2.5-7B KV shape (the re-RoPE microbenchmark's workload): 28
    layers, 4 heads, D=128, bf16, theta 1e6; 16 chunks x 256 tokens whose keys are N(0,1) vectors
    x rotated at their original positions p_c + t, moved by delta_c ~ U[-4096, 4096] to slot
    dst_c of a 4096-token cache (p_c = dst_c - delta_c, negative for some chunks: RoPE is defined
    there too). Bit-exact against the oracle; and the gathered keys equal x rotated at the new
    positions dst_c + t (the shift property of torch_engine.py:56-59, the reference's
    tests/test_rerope.py::test_shift_moves_keys_to_new_offset) within the rounding of the two
    steps: each element off by at most 2^-7 r, r the radius of its (x_i, x_i+D/2) pair (the rotations
    preserve it; the cached keys' bf16 rounding and the result's each add 2^-9 r, the fp32 shift
    angle at |delta| <= 4096 at most 2.5e-4 r)."""
    rng = np.random.default_rng(2)
    n_layers, H, D, L, C = 28, 4, 128, 256, 16
    N = L * C
    dst = rng.permutation(C) * L
    deltas = rng.integers(-4096, 4097, C)
    g = torch.Generator(device=DEV).manual_seed(2)
    t = torch.arange(L, device=DEV)
    X = torch.randn((C, n_layers, 1, H, L, D), generator=g, device=DEV)
    Kc = torch.empty((C, n_layers, 1, H, L, D), dtype=torch.bfloat16, device=DEV)
    for c in range(C):
        Kc[c] = _rope_rows(X[c], int(dst[c] - deltas[c]) + t, THETA).to(torch.bfloat16)
    Vc = torch.randn((C, n_layers, 1, H, L, D), generator=g, device=DEV).to(torch.bfloat16)
    segs = np.array([[dst[c], L, c, 0, L, deltas[c]] for c in range(C)], dtype=np.int32)
    tab = np.zeros((C, n_layers, 2), dtype=np.uint64)
    for c in range(C):
        for l in range(n_layers):
            tab[c, l, 0] = Kc[c, l].data_ptr()
            tab[c, l, 1] = Vc[c, l].data_ptr()
    K = torch.empty((n_layers, 1, H, N, D), dtype=torch.bfloat16, device=DEV)
    V = torch.empty_like(K)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    ops.rerope_gather(K, V, torch.from_numpy(tab.view(np.int64)).to(DEV), torch.from_numpy(segs.reshape(-1)).to(DEV),
                      C, L, THETA, err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    # the shift property, every layer and chunk
    for c in range(C):
        want = _rope_rows(X[c], int(dst[c]) + t, THETA)  # (n_layers, 1, H, L, D)
        r = torch.sqrt(X[c][..., : D // 2] ** 2 + X[c][..., D // 2 :] ** 2)
        got = K[:, :, :, dst[c] : dst[c] + L].float()
        bad = (got - want).abs() > 2.0 ** -7 * torch.cat((r, r), -1) + 1e-6
        assert not bad.any(), f"chunk {c} (delta {deltas[c]}): {int(bad.sum())} keys off"
    del X
    Kc_h, Vc_h = host(Kc), host(Vc)
    Ko = np.empty((n_layers, H, N, D), dtype=np.uint16)
    Vo = np.empty_like(Ko)
    okl = [[Kc_h[c, l, 0] for l in range(n_layers)] for c in range(C)]
    ovl = [[Vc_h[c, l, 0] for l in range(n_layers)] for c in range(C)]
    assert O.rerope_gather(Ko, Vo, okl, ovl, segs, THETA) == 0
    np.testing.assert_array_equal(host(V).reshape(Vo.shape), Vo)
    assert_keys_close(host(K).reshape(Ko.shape), Ko, True)


def test_rerope_gather_flags_bad_segment_without_writing():
    H, D, N = 2, 64, 32
    src = torch.randn((1, H, 8, D), device=DEV)
    tab = torch.tensor([src.data_ptr(), src.data_ptr()], dtype=torch.int64, device=DEV)
    segs = torch.tensor([28, 8, 0, 0, 8, 5], dtype=torch.int32, device=DEV)  # runs past N
    K = torch.zeros((1, 1, H, N, D), device=DEV)
    V = torch.zeros_like(K)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    ops.rerope_gather(K, V, tab, segs, 1, 8, THETA, err)
    torch.cuda.synchronize()
    assert int(err.item()) == _native.DEVICE_ERR_RANGE
    assert not K.any() and not V.any()


def _deviation_case(rng, N, H, D, bf16, token_major_v=True):
    """Config-3 style: cached = fresh + per-chunk lognormal(-3, 1) noise."""
    n_chunks = max(1, N // 256)
    sigma = np.exp(rng.normal(-3.0, 1.0, n_chunks)).astype(np.float32)
    fresh_k = rng.standard_normal((H, N, D)).astype(np.float32)
    fresh_v = rng.standard_normal((H, N, D)).astype(np.float32)
    sig_tok = np.repeat(sigma, int(np.ceil(N / n_chunks)))[:N][None, :, None]
    K = fresh_k + sig_tok * rng.standard_normal((H, N, D)).astype(np.float32)
    V = fresh_v + sig_tok * rng.standard_normal((H, N, D)).astype(np.float32)
    conv = (lambda a: O.f32_to_bf16_bits(a)) if bf16 else (lambda a: a.astype(np.float32))
    return conv(fresh_k), conv(fresh_v), conv(K), conv(V)


@pytest.mark.parametrize("bf16", [True, False])
@pytest.mark.parametrize("N", [1, 77, 8192])
@pytest.mark.parametrize("H,D", [(4, 128), (2, 64), (4, 64)])
def test_deviation_bit_exact(bf16, N, H, D):
    """Every row layout of the deviation kernel: one vector of each row per lane (bf16 4 x 128),
    fewer vectors than lanes (2 x 64, 4 x 64) and several per lane (fp32 4 x 128)."""
    rng = np.random.default_rng(N + bf16 + 7 * D + H)
    k, v, K, V = _deviation_case(rng, N, H, D, bf16)
    flags = (rng.random(N) < 0.9).astype(np.uint8)
    active = np.sort(rng.choice(N, max(1, int(N * 0.85)), replace=False))
    local = np.full(N, -1, dtype=np.int32)
    local[active] = np.arange(len(active))
    kf, vf = k[:, active], v[:, active]
    kt = dev(kf)[None]
    # fresh v as the engine produces it: a token-major (1, n, H, D) buffer viewed as (1, H, n, D)
    vt = dev(np.ascontiguousarray(vf.transpose(1, 0, 2)))[None].transpose(1, 2)
    assert vt.stride(2) == H * D  # token stride of the token-major buffer
    diff, norm = ops.deviation(kt, vt, dev(K)[None], dev(V)[None], dev(flags), dev(local))
    od, on = O.deviation(kf, vf, K, V, flags, local)
    np.testing.assert_array_equal(host(diff).view(np.uint32), od.view(np.uint32))
    np.testing.assert_array_equal(host(norm).view(np.uint32), on.view(np.uint32))


def _spans(n_chunks, L, ratio, n_sink, N):
    flags = np.zeros(N, dtype=np.uint8)
    spans = []
    for c in range(n_chunks):
        s = c * L
        flags[s : s + L] |= 1
        flags[s : s + min(n_sink, L)] |= 2
        spans.append((s, L, int(round(ratio * L)), int(ratio > 0)))
    return flags, np.array(spans, dtype=np.int32).reshape(-1, 4)


def _check_select(diff, norm, flags, local, spans, thr):
    got = ops.select(dev(diff), dev(norm), dev(flags), dev(local), dev(spans.reshape(-1)), thr)
    want = O.select(diff, norm, flags, local, spans, thr)
    counts = host(got.counts)
    np.testing.assert_array_equal(counts[:6], want["counts"][:6])
    n = int(counts[0])
    np.testing.assert_array_equal(host(got.keep_abs)[:n], want["keep_abs"])
    np.testing.assert_array_equal(host(got.keep_local)[:n], want["keep_local"])
    C = len(spans)
    np.testing.assert_array_equal(host(got.rel_dev)[:C].view(np.uint32), want["rel_dev"].view(np.uint32))
    np.testing.assert_array_equal(host(got.escalated)[:C], want["escalated"])
    np.testing.assert_array_equal(host(got.keep_rank), want["keep_rank"])
    return want


@pytest.mark.parametrize("ratio", [0.15, 0.3, 0.5])
def test_select_config3_bit_exact(ratio):
    """32 chunks x 256 tokens, 4 sinks each, deviations from the config-3 noise model."""
    rng = np.random.default_rng(int(ratio * 100))
    N, H, D = 8192, 4, 128
    k, v, K, V = _deviation_case(rng, N, H, D, True)
    flags, spans = _spans(32, 256, ratio, 4, N)
    local = np.arange(N, dtype=np.int32)
    diff, norm = O.deviation(k, v, K, V, flags, local)
    want = _check_select(diff, norm, flags, local, spans, None)
    expect_keep = {0.15: 1344, 0.3: 2592, 0.5: 4224}[ratio]
    assert want["counts"][0] == expect_keep


@pytest.mark.parametrize("seed", range(6))
def test_select_planted_ties_and_escalation(seed):
    rng = np.random.default_rng(1000 + seed)
    n_chunks, L, tail = int(rng.integers(1, 40)), int(rng.integers(5, 300)), int(rng.integers(0, 100))
    N = n_chunks * L + tail
    flags, spans = _spans(n_chunks, L, float(rng.choice([0.0, 0.1, 0.3, 1.0, 2.0])), int(rng.integers(0, 6)), N)
    levels = rng.gamma(2.0, 1.0, 7).astype(np.float32)
    diff = levels[rng.integers(0, 7, N)]  # heavy ties
    if seed % 2:
        diff[rng.integers(0, N, 5)] = np.nan
        diff[rng.integers(0, N, 5)] = 0.0
    norm = (np.abs(diff) + rng.gamma(3.0, 1.0, N)).astype(np.float32)
    local = np.full(N, -1, dtype=np.int32)
    act = np.sort(rng.choice(N, int(N * 0.95), replace=False))
    local[act] = np.arange(len(act))
    thr = None if seed < 3 else float(np.nanmedian(diff) / np.mean(norm))
    _check_select(diff, norm, flags, local, spans, thr)


@pytest.mark.parametrize("N_chunks", [4, 40, 130])
def test_select_nan_candidates_rank_after_finite(N_chunks):
    """A budget that reaches past the finite candidates into NaN ones. The kernels' rule: NaN
    ranks below every finite deviation (0 included) and NaN candidates are taken lowest index
    first, so every finite candidate is kept, then the lowest-index NaN candidates. (The
    reference's argsort(-where(cand, diff, -1)) would instead reach the non-candidates' +1
    entries before any NaN, in an unstable order, and keep arbitrary non-candidates.)"""
    rng = np.random.default_rng(77 + N_chunks)
    L = 64
    N = N_chunks * L + 16
    flags, spans = _spans(N_chunks, L, 0.9, 4, N)  # budget 58 of 60 candidates per chunk
    diff = rng.gamma(2.0, 1.0, N).astype(np.float32)
    cand = np.zeros(N, dtype=bool)
    for s0, ln, _, _ in spans:
        cand[s0 + 4 : s0 + ln] = True
    cand_pos = np.flatnonzero(cand)
    nan_pos = np.sort(rng.choice(cand_pos, 5 * N_chunks, replace=False))
    diff[nan_pos] = np.nan
    diff[rng.choice(np.setdiff1d(cand_pos, nan_pos), N_chunks, replace=False)] = 0.0
    norm = (np.nan_to_num(diff) + 1).astype(np.float32)
    local = np.arange(N, dtype=np.int32)
    want = _check_select(diff, norm, flags, local, spans, None)
    budget = int(want["counts"][2])
    n_finite = int(cand.sum()) - len(nan_pos)
    assert budget > n_finite  # the budget reaches into the NaN candidates
    kept = set(want["keep_abs"].tolist())
    assert set(np.setdiff1d(cand_pos, nan_pos).tolist()) <= kept
    assert [p for p in nan_pos.tolist() if p in kept] == nan_pos[: budget - n_finite].tolist()


@pytest.mark.parametrize("N", [1, 31, 32, 33, 64, 1023, 1024, 1025, 8256, 16384, 16385, 33792, 131072])
def test_select_sizes(N):
    rng = np.random.default_rng(N)
    L = max(1, N // 3)
    n_chunks = N // L
    flags, spans = _spans(n_chunks, L, 0.3, 2, N)
    diff = rng.gamma(2.0, 1.0, N).astype(np.float32)
    norm = (diff + 1).astype(np.float32)
    _check_select(diff, norm, flags, np.arange(N, dtype=np.int32), spans, None)


@pytest.mark.parametrize("flags_off", [4, 1])
@pytest.mark.parametrize("N", [1025, 8256, 16000, 20000, 33000])
def test_select_misaligned_inputs(N, flags_off):
    """diff, norm and local one element into their buffers (4-byte, not 16-byte aligned), flags
    4 or 1 bytes in: the selecting threads load their runs from one address per array instead of
    16-byte vectors, the flags as aligned words (4-byte aligned flags) or byte by byte, in every
    register bucket from 4 to 16 positions per thread and the L2 form above 16384 positions; same
    result as the oracle."""
    rng = np.random.default_rng(N + flags_off)
    L = 250
    flags, spans = _spans(N // L, L, 0.3, 4, N)
    diff = rng.gamma(2.0, 1.0, N).astype(np.float32)
    norm = (diff + 1).astype(np.float32)
    local = np.arange(N, dtype=np.int32)

    def at(a, off):
        buf = torch.zeros(len(a) + off + 16, dtype=dev(a[:1]).dtype, device=DEV)
        buf[off : off + len(a)] = dev(a)
        return buf[off : off + len(a)]

    d, n, f, lo = at(diff, 1), at(norm, 1), at(flags, flags_off), at(local, 1)
    assert d.data_ptr() % 16 and lo.data_ptr() % 16 and f.data_ptr() % 4 == flags_off % 4
    got = ops.select(d, n, f, lo, dev(spans.reshape(-1)), None)
    want = O.select(diff, norm, flags, local, spans, None)
    counts = host(got.counts)
    np.testing.assert_array_equal(counts[:6], want["counts"][:6])
    k = int(counts[0])
    np.testing.assert_array_equal(host(got.keep_abs)[:k], want["keep_abs"])
    np.testing.assert_array_equal(host(got.keep_local)[:k], want["keep_local"])
    np.testing.assert_array_equal(host(got.keep_rank), want["keep_rank"])
    np.testing.assert_array_equal(host(got.rel_dev)[: len(spans)].view(np.uint32), want["rel_dev"].view(np.uint32))


@pytest.mark.parametrize("bf16", [True, False])
def test_scatter_bit_exact(bf16):
    rng = np.random.default_rng(7 + bf16)
    H, N, D = 4, 3000, 128
    n = 977
    K = rand_elems(rng, (H, N, D), bf16)
    V = rand_elems(rng, (H, N, D), bf16)
    k = rand_elems(rng, (H, n, D), bf16)
    v = rand_elems(rng, (H, n, D), bf16)
    rows = np.sort(rng.choice(N, n, replace=False)).astype(np.int64)
    Kt, Vt = dev(K)[None].contiguous(), dev(V)[None].contiguous()
    vt = dev(np.ascontiguousarray(v.transpose(1, 0, 2)))[None].transpose(1, 2)  # token-major like v_proj
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    ops.scatter_rows(Kt, Vt, dev(k)[None], vt, dev(rows), err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    assert O.scatter_rows(K, V, k, v, rows) == 0
    np.testing.assert_array_equal(host(Kt)[0], K)
    np.testing.assert_array_equal(host(Vt)[0], V)


def test_scatter_flags_out_of_range_row():
    H, N, D = 2, 16, 64
    K = torch.zeros((1, H, N, D), device=DEV)
    V = torch.zeros_like(K)
    k = torch.ones((1, H, 2, D), device=DEV)
    rows = torch.tensor([3, 16], dtype=torch.int64, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    ops.scatter_rows(K, V, k, k.clone(), rows, err)
    torch.cuda.synchronize()
    assert int(err.item()) == _native.DEVICE_ERR_RANGE
    assert K[0, :, 3].eq(1).all() and int(K.count_nonzero()) == H * D


def _assemble_case(seed, bf16, D, overlap, active_frac, layer=1):
    """Oracle gather of every layer + oracle scatter of the active rows of `layer` (the
    reference's base cache + overwrite pair) against one assemble launch."""
    rng = np.random.default_rng(seed)
    n_layers, H = 3, 2
    lens = [40, 70, 33, 64, 1, 97]
    N = sum(lens) + 40
    plan, ks, vs = _gather_case(rng, bf16, n_layers, H, D, lens, N, overlap)
    Kg, Vg, Ko, Vo, src = _run_gather(plan, ks, vs, n_layers, H, D, N, bf16)
    # active: every uncached position plus a random share of the cached ones
    act = ~plan.cached | (rng.random(N) < active_frac)
    active = np.flatnonzero(act).astype(np.int64)
    n = len(active)
    k = rand_elems(rng, (H, n, D), bf16)
    v = rand_elems(rng, (H, n, D), bf16)
    Kw, Vw = Ko[layer].copy(), Vo[layer].copy()
    assert O.scatter_rows(Kw, Vw, k, v, active) == 0
    local = np.full(N, -1, dtype=np.int32)
    local[active] = np.arange(n, dtype=np.int32)
    return plan, src, k, v, local, Kw, Vw, n_layers, H, N


def _assemble_run(plan, src, k, v, local, n_layers, H, N, D, bf16, layer, segs=None, fill=-7.0):
    dt = torch.bfloat16 if bf16 else torch.float32
    tab = np.zeros((len(plan.chunks), n_layers, 2), dtype=np.uint64)
    for ci, ch in enumerate(plan.chunks):
        kl, vl = src[ch.idx]
        for l in range(n_layers):
            tab[ci, l, 0] = kl[l].data_ptr()
            tab[ci, l, 1] = vl[l].data_ptr()
    segs = plan.all_segments if segs is None else segs
    K = torch.full((1, H, N, D), fill, dtype=dt, device=DEV)
    V = torch.full_like(K, fill)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    vt = None if v is None else dev(np.ascontiguousarray(v.transpose(1, 0, 2)))[None].transpose(1, 2)
    ops.assemble_layer(K, V, torch.from_numpy(tab.view(np.int64)).to(DEV), n_layers, layer,
                       dev(segs.reshape(-1)), len(segs), int(segs[:, 1].max()) if len(segs) else 0,
                       None if k is None else dev(k)[None], vt, None if local is None else dev(local), THETA, err)
    torch.cuda.synchronize()
    return host(K)[0], host(V)[0], int(err.item())


@pytest.mark.parametrize("bf16", [True, False])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("overlap", [False, True])
@pytest.mark.parametrize("active_frac", [0.0, 0.3, 1.0])
def test_assemble_matches_gather_then_scatter(bf16, D, overlap, active_frac):
    layer = 1
    plan, src, k, v, local, Kw, Vw, n_layers, H, N = _assemble_case(
        500 + D + 2 * bf16 + overlap + int(active_frac * 10), bf16, D, overlap, active_frac, layer)
    Kg, Vg, e = _assemble_run(plan, src, k, v, local, n_layers, H, N, D, bf16, layer)
    assert e == 0
    np.testing.assert_array_equal(Vg, Vw)
    assert_keys_close(Kg, Kw, bf16)  # bit-exact: same arithmetic as the gather


@pytest.mark.parametrize("layer", [0, 2])
def test_assemble_gather_only_matches_gather(layer):
    """local = NULL: the cached segments only, as the gather of that layer; other rows untouched."""
    bf16, D = True, 128
    rng = np.random.default_rng(77 + layer)
    n_layers, H = 3, 2
    lens = [40, 70, 33, 64, 1, 97]
    N = sum(lens) + 40
    plan, ks, vs = _gather_case(rng, bf16, n_layers, H, D, lens, N, False)
    _, _, Ko, Vo, src = _run_gather(plan, ks, vs, n_layers, H, D, N, bf16)
    Kg, Vg, e = _assemble_run(plan, src, None, None, None, n_layers, H, N, D, bf16, layer, segs=plan.segments)
    assert e == 0
    np.testing.assert_array_equal(Vg, Vo[layer])
    np.testing.assert_array_equal(Kg, Ko[layer])  # sentinel rows outside cached runs too


def test_assemble_flags_uncached_inactive_row():
    """An uncached position with no active row has no source: flagged, its row left as it was."""
    bf16, D = True, 64
    plan, src, k, v, local, Kw, Vw, n_layers, H, N = _assemble_case(9, bf16, D, False, 0.2)
    p = int(np.flatnonzero(~plan.cached)[0])
    local = local.copy()
    local[p] = -1
    Kg, Vg, e = _assemble_run(plan, src, k, v, local, n_layers, H, N, D, bf16, 1)
    assert e == _native.DEVICE_ERR_RANGE
    sent = O.f32_to_bf16_bits(np.float32([-7.0]))[0]
    assert (Kg[:, p] == sent).all() and (Vg[:, p] == sent).all()
    others = np.ones(N, dtype=bool)
    others[p] = False
    np.testing.assert_array_equal(Vg[:, others], Vw[:, others])


def test_assemble_flags_bad_segment():
    bf16, D = True, 64
    plan, src, k, v, local, Kw, Vw, n_layers, H, N = _assemble_case(11, bf16, D, False, 0.2)
    segs = plan.all_segments.copy()
    segs[0, 2] = len(plan.chunks)  # chunk index past the table
    _, _, e = _assemble_run(plan, src, k, v, local, n_layers, H, N, D, bf16, 1, segs=segs)
    assert e == _native.DEVICE_ERR_RANGE
