"""Pins for the C oracle (oracle/ckv_oracle.c) against checks that do not restate its code:
closed forms, the reference's own re-RoPE tolerances (src tests/test_rerope.py:10-27), fp64
brute force, the reference's torch expressions evaluated by torch, and library sorts."""

from decimal import Decimal, getcontext

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import bf16_ulp_distance, rope_reference_f64

THETAS = [1e4, 5e5, 1e6]
DIMS = [64, 128, 256]


def exact_inv_freq(theta: float, D: int) -> np.ndarray:
    """theta ** fp32(-2i/D), evaluated with 40-digit decimals and rounded once to fp32."""
    getcontext().prec = 40
    t = Decimal(float(np.float32(theta)))
    out = []
    for i in range(D // 2):
        e = Decimal(float(np.float32(-2 * i) / np.float32(D)))
        out.append(np.float32(float((e * t.ln()).exp())))
    return np.array(out, dtype=np.float32)


@pytest.mark.parametrize("D", DIMS)
@pytest.mark.parametrize("theta", THETAS)
def test_inv_freq_is_correctly_rounded_closed_form(D, theta):
    got = O.inv_freq(D, theta)
    assert got[0] == 1.0
    assert np.all(np.diff(got) < 0)
    np.testing.assert_array_equal(got.view(np.uint32), exact_inv_freq(theta, D).view(np.uint32))
    # torch's fp32 pow (the reference's evaluator) agrees to within one ulp
    ref = (theta ** (-torch.arange(0, D, 2, dtype=torch.float32) / D)).numpy()
    assert np.max(np.abs(ref.view(np.int32).astype(np.int64) - got.view(np.int32))) <= 1


def test_zero_shift_is_identity():  # reference tests/test_rerope.py:25-27
    k = np.random.default_rng(0).standard_normal((1, 2, 4, 64)).astype(np.float32)
    assert O.shift_keys(k, 0, 1e6) is k


def test_shift_from_zero_matches_textbook_rope():  # reference tests/test_rerope.py:10-12
    rng = np.random.default_rng(1)
    x = rng.standard_normal((2, 1, 64)).astype(np.float32)
    for p in range(5, 15):
        got = O.shift_keys(x, p, 1e6)
        want = rope_reference_f64(x, np.array([p]), 1e6)
        np.testing.assert_allclose(got, want, atol=1e-5)


def test_shift_moves_keys_to_new_offset():  # reference tests/test_rerope.py:15-17
    rng = np.random.default_rng(2)
    x = rng.standard_normal((1, 2, 10, 64))
    k5 = rope_reference_f64(x, np.arange(5, 15), 1e6).astype(np.float32)
    k42 = rope_reference_f64(x, np.arange(42, 52), 1e6)
    np.testing.assert_allclose(O.shift_keys(k5, 37, 1e6), k42, atol=1e-4)


def test_shift_round_trip():  # reference tests/test_rerope.py:20-22
    rng = np.random.default_rng(3)
    k = rope_reference_f64(rng.standard_normal((1, 2, 10, 64)), np.arange(3, 13), 1e6).astype(np.float32)
    back = O.shift_keys(O.shift_keys(k, 37, 1e6), -37, 1e6)
    np.testing.assert_allclose(back, k, atol=1e-5)


@pytest.mark.parametrize("D", [64, 128])
def test_shift_bf16_within_one_ulp_of_f64_rotation(D):
    """Same fp32 angle as the contract, rotation in fp64, one rounding: <= 1 bf16 ulp."""
    rng = np.random.default_rng(4 + D)
    x32 = rng.standard_normal((4, 64, D)).astype(np.float32)
    xb = O.f32_to_bf16_bits(x32)
    inv = exact_inv_freq(1e6, D)
    for delta in [1, -1, 777, -4096, 4096, 2900]:
        got = O.shift_keys(xb, delta, 1e6)
        ang = (np.float32(delta) * inv).astype(np.float32).astype(np.float64)
        xf = O.bf16_bits_to_f32(xb).astype(np.float64)
        a, b = xf[..., : D // 2], xf[..., D // 2 :]
        want = np.concatenate([a * np.cos(ang) - b * np.sin(ang), a * np.sin(ang) + b * np.cos(ang)], axis=-1)
        dist = bf16_ulp_distance(got, O.f32_to_bf16_bits(want.astype(np.float32)))
        assert dist.max() <= 1
        assert (dist == 0).mean() > 0.99


def test_shift_preserves_pair_norms():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 50, 128)).astype(np.float32)
    y = O.shift_keys(x, 1234, 1e6)
    n0 = x[..., :64] ** 2 + x[..., 64:] ** 2
    n1 = y[..., :64] ** 2 + y[..., 64:] ** 2
    np.testing.assert_allclose(n1, n0, rtol=1e-5, atol=1e-6)


def _random_chunks(rng, n_chunks, n_layers, H, D, L, bf16):
    ks, vs = [], []
    for _ in range(n_chunks):
        kl, vl = [], []
        for _ in range(n_layers):
            a = rng.standard_normal((H, L, D)).astype(np.float32)
            b = rng.standard_normal((H, L, D)).astype(np.float32)
            kl.append(O.f32_to_bf16_bits(a) if bf16 else a)
            vl.append(O.f32_to_bf16_bits(b) if bf16 else b)
        ks.append(kl)
        vs.append(vl)
    return ks, vs


@pytest.mark.parametrize("bf16", [True, False])
def test_rerope_gather_equals_per_segment_shift(bf16):
    rng = np.random.default_rng(6)
    n_layers, H, D, L, N = 3, 2, 64, 40, 200
    ks, vs = _random_chunks(rng, 3, n_layers, H, D, L, bf16)
    # segments: (dst_start, n, chunk, src_start, src_len, delta)
    segs = np.array([[0, 40, 0, 0, L, 0], [50, 30, 1, 10, L, 37], [100, 40, 2, 0, L, -1000], [160, 40, 0, 0, L, 4000]],
                    dtype=np.int32)
    dt = np.uint16 if bf16 else np.float32
    Kd = np.zeros((n_layers, H, N, D), dtype=dt)
    Vd = np.zeros_like(Kd)
    assert O.rerope_gather(Kd, Vd, ks, vs, segs, 1e6) == 0
    Kw = np.zeros_like(Kd)
    Vw = np.zeros_like(Vd)
    for l in range(n_layers):
        for dst, n, c, s0, _, delta in segs:
            Kw[l, :, dst : dst + n] = O.shift_keys(ks[c][l][:, s0 : s0 + n], int(delta), 1e6)
            Vw[l, :, dst : dst + n] = vs[c][l][:, s0 : s0 + n]
    np.testing.assert_array_equal(Kd, Kw)
    np.testing.assert_array_equal(Vd, Vw)


def test_rerope_gather_rejects_bad_segment():
    rng = np.random.default_rng(7)
    ks, vs = _random_chunks(rng, 1, 1, 1, 64, 8, False)
    Kd = np.zeros((1, 1, 16, 64), dtype=np.float32)
    Vd = np.zeros_like(Kd)
    bad = np.array([[12, 8, 0, 0, 8, 3]], dtype=np.int32)  # runs past N
    assert O.rerope_gather(Kd, Vd, ks, vs, bad, 1e6) == 1
    assert not Kd.any()


# ---- deviation -------------------------------------------------------------------------


def _dev_inputs(rng, H=4, D=128, N=96, bf16=True, frac_active=0.8):
    active = np.sort(rng.choice(N, int(N * frac_active), replace=False))
    n = len(active)
    cached = rng.random(N) < 0.8
    flags = cached.astype(np.uint8)
    k = rng.standard_normal((H, n, D)).astype(np.float32)
    v = rng.standard_normal((H, n, D)).astype(np.float32)
    K = rng.standard_normal((H, N, D)).astype(np.float32)
    V = rng.standard_normal((H, N, D)).astype(np.float32)
    # cached rows near the fresh ones for a realistic spread of deviations
    K[:, active] = k + 0.05 * rng.standard_normal(k.shape).astype(np.float32)
    V[:, active] = v + 0.05 * rng.standard_normal(v.shape).astype(np.float32)
    if bf16:
        k, v, K, V = (O.f32_to_bf16_bits(a) for a in (k, v, K, V))
    local = np.full(N, -1, dtype=np.int32)
    local[active] = np.arange(n)
    return k, v, K, V, flags, local, active, cached


@pytest.mark.parametrize("bf16", [True, False])
def test_deviation_matches_f64_brute_force(bf16):
    rng = np.random.default_rng(8)
    k, v, K, V, flags, local, active, cached = _dev_inputs(rng, bf16=bf16)
    diff, norm = O.deviation(k, v, K, V, flags, local)
    kf, vf, Kf, Vf = (O.as_f32(a).astype(np.float64) for a in (k, v, K, V))
    for p in range(K.shape[1]):
        j = local[p]
        if j < 0:
            assert diff[p] == 0 and norm[p] == 0
            continue
        Kc = Kf[:, p] if cached[p] else 0.0
        Vc = Vf[:, p] if cached[p] else 0.0
        dk = kf[:, j] - Kc
        dv = vf[:, j] - Vc
        if bf16:  # the reference subtracts in bf16: one rounding of the fp32 difference
            dk = O.bf16_bits_to_f32(O.f32_to_bf16_bits(dk.astype(np.float32))).astype(np.float64)
            dv = O.bf16_bits_to_f32(O.f32_to_bf16_bits(dv.astype(np.float32))).astype(np.float64)
        else:
            dk = dk.astype(np.float32).astype(np.float64)
            dv = dv.astype(np.float32).astype(np.float64)
        want_d = (dk**2).sum() + (dv**2).sum()
        want_n = (kf[:, j] ** 2).sum() + (vf[:, j] ** 2).sum()
        assert abs(diff[p] - want_d) <= 2e-6 * want_d + 1e-30
        assert abs(norm[p] - want_n) <= 2e-6 * want_n


def test_deviation_matches_reference_torch_expression():
    """torch_engine.py:118-120 evaluated by torch on the same bf16 data, within fp32 sum order."""
    rng = np.random.default_rng(9)
    k, v, K, V, flags, local, active, cached = _dev_inputs(rng, N=128, frac_active=1.0)
    flags[:] = 1
    diff, norm = O.deviation(k, v, K, V, flags, local)
    tk, tv, tK, tV = (O.from_numpy(a)[None] for a in (k, v, K, V))
    act = torch.from_numpy(active)
    d = ((tk - tK[:, :, act]).float() ** 2).sum(dim=(0, 1, 3))
    d += ((tv - tV[:, :, act]).float() ** 2).sum(dim=(0, 1, 3))
    n = (tk.float() ** 2).sum(dim=(0, 1, 3)) + (tv.float() ** 2).sum(dim=(0, 1, 3))
    np.testing.assert_allclose(diff[active], d.numpy(), rtol=3e-6)
    np.testing.assert_allclose(norm[active], n.numpy(), rtol=3e-6)


def test_deviation_exact_invariants():
    rng = np.random.default_rng(10)
    k, v, K, V, flags, local, active, cached = _dev_inputs(rng, bf16=False)
    d1, n1 = O.deviation(k, v, K, V, flags, local)
    d2, n2 = O.deviation(2 * k, 2 * v, 2 * K, 2 * V, flags, local)  # powers of two scale exactly
    np.testing.assert_array_equal(d2, 4 * d1)
    np.testing.assert_array_equal(n2, 4 * n1)
    Kc, Vc = K.copy(), V.copy()
    Kc[:, active] = k
    Vc[:, active] = v
    f = np.ones_like(flags)
    d0, _ = O.deviation(k, v, Kc, Vc, f, local)
    assert not d0.any()


# ---- selection -------------------------------------------------------------------------


def _sel_case(rng, n_chunks=12, L=40, tail=30, ratio=0.3, n_sink=4, ties=True):
    N = n_chunks * L + tail
    flags = np.zeros(N, dtype=np.uint8)
    spans = []
    for c in range(n_chunks):
        s = c * L
        flags[s : s + L] |= 1
        flags[s : s + n_sink] |= 2
        spans.append((s, L, int(round(ratio * L)), 1 if ratio > 0 else 0))
    diff = rng.gamma(2.0, 1.0, N).astype(np.float32)
    if ties:  # plant runs of equal deviations that straddle the selection boundary
        vals = np.sort(diff)[::-1]
        b = sum(sp[2] for sp in spans)
        thr = vals[min(b + n_chunks * n_sink, N - 1)]
        idx = rng.choice(N, N // 6, replace=False)
        diff[idx] = thr
    norm = (diff + rng.gamma(5.0, 1.0, N)).astype(np.float32)
    local = np.arange(N, dtype=np.int32)
    return diff, norm, flags, local, np.array(spans, dtype=np.int32)


def _lexsort_select(diff, flags, spans, budget_cap=True):
    """Independent restatement of the tie contract with numpy.lexsort."""
    N = len(diff)
    keep = ((flags & 1) == 0) | ((flags & 2) != 0)
    pool = np.zeros(N, dtype=bool)
    budget = 0
    for s, L, b, pooled in spans:
        if pooled:
            pool[s : s + L] = True
            budget += b
    cand = np.flatnonzero(pool & ~keep)
    budget = min(budget, len(cand))
    order = np.lexsort((cand, -diff[cand].astype(np.float64)))  # diff desc, index asc
    keep[cand[order[:budget]]] = True
    return np.flatnonzero(keep)


@pytest.mark.parametrize("ratio", [0.15, 0.3, 0.5, 1.0, 0.0])
def test_select_matches_lexsort_and_stable_argsort(ratio):
    rng = np.random.default_rng(11)
    diff, norm, flags, local, spans = _sel_case(rng, ratio=ratio)
    got = O.select(diff, norm, flags, local, spans, None)
    want = _lexsort_select(diff, flags, spans)
    np.testing.assert_array_equal(got["keep_abs"], want)
    # the reference expression (torch_engine.py:143-146) with a stable sort gives the same set
    t = torch.from_numpy(diff)
    keep = torch.from_numpy(((flags & 1) == 0) | ((flags & 2) != 0))
    pool = torch.zeros(len(diff), dtype=torch.bool)
    budget = 0
    for s, L, b, pooled in spans:
        if pooled:
            pool[s : s + L] = True
            budget += int(b)
    budget = min(budget, int((pool & ~keep).sum()))
    if budget > 0:
        top = torch.argsort(-torch.where(pool & ~keep, t, torch.full_like(t, -1.0)), stable=True)[:budget]
        keep[top] = True
    np.testing.assert_array_equal(got["keep_abs"], keep.nonzero().squeeze(1).numpy())
    assert got["counts"][0] == len(want)
    assert got["counts"][2] == budget


def test_select_rel_dev_and_escalation():
    rng = np.random.default_rng(12)
    diff, norm, flags, local, spans = _sel_case(rng, ties=False)
    rel64 = np.array([diff[s : s + L].astype(np.float64).sum() / norm[s : s + L].astype(np.float64).sum() for s, L, _, _ in spans])
    thr = float(np.median(rel64))
    got = O.select(diff, norm, flags, local, spans, thr)
    np.testing.assert_allclose(got["rel_dev"], rel64, rtol=1e-5)
    esc = got["escalated"].astype(bool)
    np.testing.assert_array_equal(esc, got["rel_dev"].astype(np.float64) > thr)
    keep = set(got["keep_abs"].tolist())
    for (s, L, _, _), e in zip(spans, esc):
        span = set(range(s, s + L))
        assert span <= keep if e else len(span & keep) < L
    # escalated chunks leave the pool: the budget counts only the others
    assert got["counts"][5] == sum(b for (s, L, b, p), e in zip(spans, esc) if not e)


def test_select_budget_cap_with_sinks():
    """ratio 1.0 asks for more tokens than remain after the sinks (cf. test_mlx_engine.py:86-99)."""
    rng = np.random.default_rng(13)
    diff, norm, flags, local, spans = _sel_case(rng, n_chunks=3, L=20, tail=5, ratio=1.0, n_sink=4)
    got = O.select(diff, norm, flags, local, spans, None)
    assert got["counts"][5] == 60 and got["counts"][2] == 48  # requested 3*20, capped at 3*(20-4)
    np.testing.assert_array_equal(got["keep_abs"], np.arange(65))


def test_select_uncomputed_tokens_are_counted():
    rng = np.random.default_rng(14)
    diff, norm, flags, local, spans = _sel_case(rng, ties=False)
    local = local.copy()
    local[:5] = -1  # first sinks were never computed
    got = O.select(diff, norm, flags, local, spans, None)
    kept_uncomputed = np.isin(got["keep_abs"], np.arange(5)).sum()
    assert kept_uncomputed >= 4  # the four sinks at least
    assert got["counts"][4] == kept_uncomputed
    assert (got["keep_local"] >= 0).all()


def test_select_nan_ranks_last():
    diff = np.array([1.0, np.nan, 3.0, 2.0, np.nan, 0.5], dtype=np.float32)
    flags = np.ones(6, dtype=np.uint8)
    spans = np.array([[0, 6, 4, 1]], dtype=np.int32)
    got = O.select(diff, np.ones(6, np.float32), flags, np.arange(6, dtype=np.int32), spans, None)
    np.testing.assert_array_equal(got["keep_abs"], [0, 2, 3, 5])


def test_scatter_rows_brute_force():
    rng = np.random.default_rng(15)
    H, N, D, n = 2, 50, 64, 17
    K = rng.standard_normal((H, N, D)).astype(np.float32)
    V = rng.standard_normal((H, N, D)).astype(np.float32)
    k = rng.standard_normal((H, n, D)).astype(np.float32)
    v = rng.standard_normal((H, n, D)).astype(np.float32)
    rows = rng.choice(N, n, replace=False).astype(np.int64)
    Kw, Vw = K.copy(), V.copy()
    for j, t in enumerate(rows):
        for h in range(H):
            Kw[h, t] = k[h, j]
            Vw[h, t] = v[h, j]
    assert O.scatter_rows(K, V, k, v, rows) == 0
    np.testing.assert_array_equal(K, Kw)
    np.testing.assert_array_equal(V, Vw)


@pytest.mark.parametrize("Hq,Hkv,D,N,n", [(4, 4, 64, 40, 40), (14, 2, 64, 97, 31), (28, 4, 128, 150, 57)])
def test_attention_active_matches_reference_sdpa_call(Hq, Hkv, D, N, n):
    """The oracle against the reference's own call (torch_engine.py:157, :68-72): a boolean mask
    active[:, None] >= arange(N) and SDPA with enable_gqa, fp32 on the CPU."""
    import torch.nn.functional as F

    rng = np.random.default_rng(Hq + N)
    q = rng.standard_normal((Hq, n, D)).astype(np.float32)
    K = rng.standard_normal((Hkv, N, D)).astype(np.float32)
    V = rng.standard_normal((Hkv, N, D)).astype(np.float32)
    active = np.sort(rng.choice(N, n, replace=False))
    got = O.attention_active(q, K, V, active)
    act = torch.from_numpy(active)
    mask = act[:, None] >= torch.arange(N)[None, :]
    want = F.scaled_dot_product_attention(torch.from_numpy(q)[None], torch.from_numpy(K)[None],
                                          torch.from_numpy(V)[None], attn_mask=mask, enable_gqa=True)
    np.testing.assert_allclose(got, want[0].transpose(0, 1).numpy(), atol=2e-5, rtol=0)


def test_attention_active_closed_forms():
    """Position 0 sees only row 0 (output = V[0]); equal scores average the visible rows; a row
    far above the others takes all the weight."""
    D, N = 64, 10
    q = np.zeros((1, 3, D), np.float32)
    K = np.zeros((1, N, D), np.float32)
    V = np.arange(N * D, dtype=np.float32).reshape(1, N, D)
    out = O.attention_active(q, K, V, np.array([0, 4, 9]))
    np.testing.assert_array_equal(out[0, 0], V[0, 0])
    np.testing.assert_allclose(out[1, 0], V[0, :5].mean(axis=0))
    np.testing.assert_allclose(out[2, 0], V[0].mean(axis=0))
    K[0, 7, 0] = 1000.0
    q[0, 2, 0] = 1.0
    out = O.attention_active(q, K, V, np.array([0, 4, 9]))
    np.testing.assert_allclose(out[2, 0], V[0, 7])


def test_rope_equal_positions_is_shift_keys():
    """Every row at position p is a shift by p (the same fp32 angle, the same rotation)."""
    rng = np.random.default_rng(31)
    x = O.f32_to_bf16_bits(rng.standard_normal((3, 20, 128)).astype(np.float32))
    for p in (1, 37, 4096, 32767, -5):
        got = O.rope(x, np.full(20, p), 1e6)
        np.testing.assert_array_equal(got, O.shift_keys(x, p, 1e6))


def test_rope_matches_reference_torch_expression():
    """torch_engine.py:53-54 + :46-51 on the CPU in torch (its own fp32 cos/sin): within one bf16
    ulp; position 0 goes through the formula (signed zeros included) like torch."""
    rng = np.random.default_rng(32)
    H, n, D, theta = 4, 300, 128, 1e6
    x = O.f32_to_bf16_bits(rng.standard_normal((H, n, D)).astype(np.float32))
    x[0, 0, :4] = O.f32_to_bf16_bits(np.float32([-0.0, 0.0, -0.0, 1.0]))
    pos = np.concatenate([[0], np.sort(rng.choice(np.arange(1, 32768), n - 1, replace=False))])
    got = O.rope(x, pos, theta)
    inv = torch.from_numpy(O.inv_freq(D, theta))
    xt = O.from_numpy(x)
    ang = torch.from_numpy(pos).float()[:, None] * inv[None, :]
    cos, sin = ang.cos(), ang.sin()
    x32 = xt.float()
    x1, x2 = x32[..., : D // 2], x32[..., D // 2 :]
    want = O.to_numpy(torch.cat([x1 * cos - x2 * sin, x1 * sin + x2 * cos], dim=-1).to(torch.bfloat16))
    assert bf16_ulp_distance(got, want).max() <= 1
    np.testing.assert_array_equal(got[:, 0], want[:, 0])  # position 0: cos 1, sin 0 exactly


def test_rope_fp64_rotation_and_composition():
    rng = np.random.default_rng(33)
    H, n, D, theta = 2, 64, 64, 1e4
    x = rng.standard_normal((H, n, D)).astype(np.float32)
    pos = rng.integers(0, 20000, n)
    got = O.rope(x, pos, theta)
    inv = O.inv_freq(D, theta).astype(np.float64)
    ang = (pos.astype(np.float32)[:, None] * O.inv_freq(D, theta)[None, :]).astype(np.float64)
    x1, x2 = x[..., : D // 2].astype(np.float64), x[..., D // 2 :].astype(np.float64)
    want = np.concatenate([x1 * np.cos(ang) - x2 * np.sin(ang), x1 * np.sin(ang) + x2 * np.cos(ang)], -1)
    np.testing.assert_allclose(got, want, atol=2e-5, rtol=0)
    del inv
    a, b = rng.integers(0, 500, n), rng.integers(0, 500, n)
    np.testing.assert_allclose(O.rope(O.rope(x, a, theta), b, theta), O.rope(x, a + b, theta), atol=1e-4, rtol=0)


def _hf_rmsnorm(hidden, weight, eps, dtype):
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RMSNorm

    m = Qwen2RMSNorm(hidden, eps=eps).to(dtype)
    with torch.no_grad():
        m.weight.copy_(weight)
    return m


@pytest.mark.parametrize("bf16", [True, False])
def test_add_rmsnorm_matches_hf_module(bf16):
    """The model's own module (transformers Qwen2RMSNorm) after torch's residual add, on the CPU:
    the residual sum is bit-exact, the normalised row within one ulp (sum order and rsqrt are
    torch's there)."""
    rng = np.random.default_rng(41)
    rows, hidden, eps = 33, 896, 1e-6
    dt = torch.bfloat16 if bf16 else torch.float32
    ht = torch.from_numpy(rng.standard_normal((rows, hidden)).astype(np.float32) * 3).to(dt)
    dt_ = torch.from_numpy(rng.standard_normal((rows, hidden)).astype(np.float32)).to(dt)
    wt = torch.from_numpy(rng.uniform(0.5, 2.0, hidden).astype(np.float32)).to(dt)
    s_want = ht + dt_
    y_want = _hf_rmsnorm(hidden, wt, eps, dt)(s_want).detach()
    s, y = O.add_rmsnorm(O.to_numpy(ht), O.to_numpy(dt_), O.to_numpy(wt), eps)
    np.testing.assert_array_equal(s, O.to_numpy(s_want))
    if bf16:
        dist = bf16_ulp_distance(y, O.to_numpy(y_want))
        assert dist.max() <= 1 and (dist > 0).mean() < 0.01
    else:
        np.testing.assert_allclose(y, y_want.numpy(), rtol=2e-6, atol=0)
    # no residual: the norm of h alone
    s0, y0 = O.add_rmsnorm(O.to_numpy(ht), None, O.to_numpy(wt), eps)
    np.testing.assert_array_equal(s0, O.to_numpy(ht))
    y0_want = O.to_numpy(_hf_rmsnorm(hidden, wt, eps, dt)(ht).detach())
    if bf16:
        assert bf16_ulp_distance(y0, y0_want).max() <= 1
    else:
        np.testing.assert_allclose(y0, y0_want, rtol=2e-6, atol=0)


def test_add_rmsnorm_closed_form():
    """A constant row c normalises to c / sqrt(c^2 + eps) (times the weight); the weight is
    applied per column, not per row; rows are independent."""
    hidden, eps = 256, 1e-6
    h = np.full((3, hidden), 2.0, dtype=np.float32)
    h[1] *= -1
    h[2] = np.arange(hidden, dtype=np.float32) - 100
    w = np.linspace(0.5, 1.5, hidden).astype(np.float32)
    _, y = O.add_rmsnorm(h, None, w, eps)
    np.testing.assert_allclose(y[0], w * 2.0 / np.sqrt(4.0 + eps), rtol=1e-6)
    np.testing.assert_allclose(y[1], -y[0], rtol=0, atol=0)
    x = h[2].astype(np.float64)
    np.testing.assert_allclose(y[2], w * x / np.sqrt((x**2).mean() + eps), rtol=1e-6)


def test_silu_mul_matches_torch_and_closed_forms():
    rng = np.random.default_rng(42)
    g = torch.from_numpy(rng.standard_normal((17, 512)).astype(np.float32) * 4).to(torch.bfloat16)
    u = torch.from_numpy(rng.standard_normal((17, 512)).astype(np.float32)).to(torch.bfloat16)
    g[0, :4] = torch.tensor([0.0, -0.0, 80.0, -80.0])
    got = O.silu_mul(O.to_numpy(g), O.to_numpy(u))
    want = O.to_numpy(torch.nn.functional.silu(g) * u)
    dist = bf16_ulp_distance(got, want)
    assert dist.max() <= 1 and (dist > 0).mean() < 0.01
    x = np.linspace(-6, 6, 101).astype(np.float32)
    one = np.ones_like(x)
    s = O.silu_mul(x, one)
    assert s[50] == 0.0
    np.testing.assert_allclose(s - O.silu_mul(-x, one), x, rtol=1e-6, atol=1e-6)  # silu(x) - silu(-x) = x
    np.testing.assert_allclose(O.silu_mul(x, 2 * one), 2 * s, rtol=0, atol=0)
