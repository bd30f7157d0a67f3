"""ckv_deviation_select (the layer-1 deviation, then the pooled top-k, sinks and compaction from
the candidate histogram the deviation counts, torch_engine.py:117-153) and ckv_scatter_kept_rows (the k/v compaction folded into the scatter,
:152 and :155-156) against the oracle, bit for bit: diff/norm, keep_abs, keep_local, keep_rank,
rel_dev, escalated and the counts. Cases: the config-3 and config-4 shapes, every shape of the
selection spread over many workgroups up to 36864 positions and the single-workgroup forms,
escalation and flags without the pooled bit (the histogram is then not used: same result),
exact placements, heavy ties and NaN deviations, the workspace left zeroed across calls of
different sizes, and replays of a captured HIP graph."""

import numpy as np
import pytest
import torch

from chunkkv_amd import _native, ops
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
H, D = 4, 128
CACHED, SINK, EXACT, POOLED = 1, 2, 4, 8


def _layout(N, chunks, n_sink, ratio, exact=()):
    """chunks: list of (start, length); exact: indices of exact placements. Returns flags, spans,
    local (active = every non-exact position)."""
    flags = np.zeros(N, dtype=np.uint8)
    spans = []
    for i, (s, L) in enumerate(chunks):
        flags[s : s + L] |= CACHED
        if i in exact:
            flags[s : s + L] |= EXACT
            continue
        flags[s : s + min(n_sink, L)] |= SINK
        r = ratio if np.isscalar(ratio) else ratio[i]
        if r > 0:
            flags[s : s + L] |= POOLED
        spans.append((s, L, int(round(r * L)), int(r > 0)))
    active = np.flatnonzero((flags & EXACT) == 0)
    local = np.full(N, -1, dtype=np.int32)
    local[active] = np.arange(len(active), dtype=np.int32)
    return flags, np.array(spans, dtype=np.int32).reshape(-1, 4), local, active


def _rows(rng, N, sigma_tok):
    """Fresh rows and a cache that differs from them by sigma_tok per position (bf16 bits)."""
    fk = rng.standard_normal((H, N, D)).astype(np.float32)
    fv = rng.standard_normal((H, N, D)).astype(np.float32)
    s = sigma_tok[None, :, None].astype(np.float32)
    K = fk + s * rng.standard_normal((H, N, D)).astype(np.float32)
    V = fv + s * rng.standard_normal((H, N, D)).astype(np.float32)
    b = O.f32_to_bf16_bits
    return b(fk), b(fv), b(K), b(V)


def _chunk_sigma(rng, N, chunks):
    sig = np.ones(N, dtype=np.float32)
    for s, L in chunks:
        sig[s : s + L] = np.exp(rng.normal(-3.0, 1.0))
    return sig


def _at(a, off):
    """a on the device, off elements into a larger buffer (alignment of that offset)."""
    buf = torch.zeros(len(a) + off + 16, dtype=torch.from_numpy(a[:1]).dtype, device=DEV)
    buf[off : off + len(a)] = torch.from_numpy(a).to(DEV)
    return buf[off : off + len(a)]


def _run_and_check(k, v, K, V, flags, local, active, spans, thr, ws=None, expect_top=None, offsets=(0, 0)):
    """Fused call on the device vs the oracle's deviation + selection. offsets: flags and local
    that many elements into their buffers."""
    kf, vf = k[:, active], v[:, active]
    kt = O.from_numpy(kf, DEV)[None]
    # fresh v as the engine has it: a token-major buffer viewed (1, H, n, D)
    vt = O.from_numpy(np.ascontiguousarray(vf.transpose(1, 0, 2)), DEV)[None].transpose(1, 2)
    ws = ops.deviation_select_workspace(DEV) if ws is None else ws
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    Kt, Vt = O.from_numpy(K, DEV)[None], O.from_numpy(V, DEV)[None]
    diff, norm, sel = ops.deviation_select(kt, vt, Kt, Vt, _at(flags, offsets[0]), _at(local, offsets[1]),
                                           O.from_numpy(spans.reshape(-1), DEV), thr, ws, err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    d_o, n_o = O.deviation(kf, vf, K, V, flags, local)
    np.testing.assert_array_equal(O.to_numpy(diff).view(np.uint32), d_o.view(np.uint32))
    np.testing.assert_array_equal(O.to_numpy(norm).view(np.uint32), n_o.view(np.uint32))
    want = O.select(d_o, n_o, flags, local, spans, thr)
    counts = O.to_numpy(sel.counts)
    np.testing.assert_array_equal(counts[:7], want["counts"][:7])
    n = int(counts[0])
    np.testing.assert_array_equal(O.to_numpy(sel.keep_abs)[:n], want["keep_abs"])
    np.testing.assert_array_equal(O.to_numpy(sel.keep_local)[:n], want["keep_local"])
    np.testing.assert_array_equal(O.to_numpy(sel.keep_rank), want["keep_rank"])
    C = len(spans)
    np.testing.assert_array_equal(O.to_numpy(sel.rel_dev)[:C].view(np.uint32), want["rel_dev"].view(np.uint32))
    np.testing.assert_array_equal(O.to_numpy(sel.escalated)[:C], want["escalated"])
    if expect_top is not None:
        assert int(counts[_native.COUNT_TOP_HISTOGRAM]) & 1 == int(expect_top)
    assert not ws.any(), "the workspace must be left zeroed"
    return want, (kt, vt, sel)


@pytest.mark.parametrize("ratio", [0.15, 0.3, 0.5])
def test_config3_shape(ratio):
    rng = np.random.default_rng(int(ratio * 100))
    N = 8192
    chunks = [(c * 256, 256) for c in range(32)]
    flags, spans, local, active = _layout(N, chunks, 4, ratio)
    k, v, K, V = _rows(rng, N, _chunk_sigma(rng, N, chunks))
    want, _ = _run_and_check(k, v, K, V, flags, local, active, spans, None, expect_top=True)
    assert want["counts"][0] == {0.15: 1344, 0.3: 2592, 0.5: 4224}[ratio]


def test_config4_shape_and_kept_row_scatter():
    """24 chunks x 320 + 576 uncached at 30 %, then the kept rows scattered from the fresh rows
    through keep_local (the compaction folded in)."""
    rng = np.random.default_rng(4)
    N = 24 * 320 + 576
    chunks = [(c * 320, 320) for c in range(24)]
    flags, spans, local, active = _layout(N, chunks, 4, 0.3)
    k, v, K, V = _rows(rng, N, _chunk_sigma(rng, N, chunks))
    want, (kt, vt, sel) = _run_and_check(k, v, K, V, flags, local, active, spans, None, expect_top=True)
    n = int(want["counts"][0])
    assert n == 2976
    Kt, Vt = O.from_numpy(K, DEV)[None].contiguous(), O.from_numpy(V, DEV)[None].contiguous()
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    ops.scatter_kept_rows(Kt, Vt, kt, vt, sel.keep_abs[:n], sel.keep_local[:n], err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    Kw, Vw = K.copy(), V.copy()
    rows = want["keep_abs"].astype(np.int64)
    assert O.scatter_rows(Kw, Vw, np.ascontiguousarray(k[:, active][:, want["keep_local"]]),
                          np.ascontiguousarray(v[:, active][:, want["keep_local"]]), rows) == 0
    np.testing.assert_array_equal(O.to_numpy(Kt)[0], Kw)
    np.testing.assert_array_equal(O.to_numpy(Vt)[0], Vw)


@pytest.mark.parametrize("N", [1, 16, 17, 77, 1024, 1025, 2048, 2049, 4099, 9216, 9217, 12288, 18432, 18433, 24577,
                               32832, 33792, 36864, 36865])
def test_sizes(N):
    """Every shape of the spread selection (256 threads x 2, 4, 9 groups of four positions, 512 x 9,
    18), the boundaries between them, and the single-workgroup L2 form above 36864 positions."""
    rng = np.random.default_rng(N)
    L = max(1, min(256, N // 3))
    chunks = [(c * L, L) for c in range(max(1, (N - 5) // L))] if N > 5 else [(0, N)]
    flags, spans, local, active = _layout(N, chunks, 2, 0.3)
    k, v, K, V = _rows(rng, N, _chunk_sigma(rng, N, chunks))
    _run_and_check(k, v, K, V, flags, local, active, spans, None, expect_top=N <= 36864)


@pytest.mark.parametrize("thr_mode", ["none_escalate", "some_escalate"])
def test_escalation(thr_mode):
    """With a threshold no chunk crosses, the histogram path runs; once chunks escalate it does
    not (their positions leave the candidates) and the result is still the oracle's."""
    rng = np.random.default_rng(31)
    N = 40 * 128 + 64
    chunks = [(c * 128, 128) for c in range(40)]
    flags, spans, local, active = _layout(N, chunks, 4, 0.3)
    sig = _chunk_sigma(rng, N, chunks)
    k, v, K, V = _rows(rng, N, sig)
    thr = 10.0 if thr_mode == "none_escalate" else float(np.median(sig[: 40 * 128]) ** 2 * 0.5)
    want, _ = _run_and_check(k, v, K, V, flags, local, active, spans, thr, expect_top=thr_mode == "none_escalate")
    assert (want["escalated"].sum() > 0) == (thr_mode == "some_escalate")


def test_flags_without_pooled_bit_and_exact_placements():
    """Flags without the pooled bit: the histogram is empty, the selection ignores it, same result.
    Exact placements (cached, never computed, not pooled) and per-placement ratios, including 0,
    keep the histogram path."""
    rng = np.random.default_rng(8)
    N = 30 * 200 + 100
    chunks = [(c * 200, 200) for c in range(30)]
    ratios = [0.0 if c % 7 == 3 else 0.25 for c in range(30)]
    flags, spans, local, active = _layout(N, chunks, 3, ratios, exact={5, 11, 12})
    k, v, K, V = _rows(rng, N, _chunk_sigma(rng, N, chunks))
    want, _ = _run_and_check(k, v, K, V, flags, local, active, spans, None, expect_top=True)
    no_pool = flags & ~np.uint8(POOLED)
    want2, _ = _run_and_check(k, v, K, V, no_pool, local, active, spans, None, expect_top=False)
    np.testing.assert_array_equal(want["keep_abs"], want2["keep_abs"])


@pytest.mark.parametrize("offsets", [(1, 1), (4, 1), (2, 3)])
@pytest.mark.parametrize("N", [4099, 8256, 9217, 32832])
def test_misaligned_flags_and_local(N, offsets):
    """Flags and local indices not 16-byte aligned (1, 2 or 4 bytes / 1 or 3 elements into their
    buffers): the spread selection loads them element by element instead of as words and
    vectors; same result as the oracle."""
    rng = np.random.default_rng(N + 7 * offsets[0])
    L = 256
    chunks = [(c * L, L) for c in range(N // L - 1)]
    flags, spans, local, active = _layout(N, chunks, 4, 0.3)
    k, v, K, V = _rows(rng, N, _chunk_sigma(rng, N, chunks))
    _run_and_check(k, v, K, V, flags, local, active, spans, None, expect_top=True, offsets=offsets)


def test_ties_and_nan_deviations():
    """Fresh rows equal to the cached ones (deviation 0, all tied), rows repeated across
    positions (equal deviations), and NaN rows: ties go to the lower position, NaN last."""
    rng = np.random.default_rng(12)
    N = 16 * 256
    chunks = [(c * 256, 256) for c in range(16)]
    flags, spans, local, active = _layout(N, chunks, 4, 0.6)
    k, v, K, V = _rows(rng, N, _chunk_sigma(rng, N, chunks))
    same = rng.choice(N, 900, replace=False)
    k[:, same], v[:, same] = K[:, same], V[:, same]  # deviation 0
    rep = rng.choice(N, 600, replace=False)
    k[:, rep], v[:, rep], K[:, rep], V[:, rep] = k[:, :1], v[:, :1], K[:, :1], V[:, :1]  # one repeated value
    nan = rng.choice(N, 40, replace=False)
    k[:, nan, 5] = 0x7FC0  # bf16 NaN
    want, _ = _run_and_check(k, v, K, V, flags, local, active, spans, None, expect_top=True)
    d_o = O.deviation(k[:, active], v[:, active], K, V, flags, local)[0]
    assert np.isnan(d_o).sum() >= 30 and (d_o == 0).sum() >= 600


def test_workspace_shared_by_calls_of_different_sizes():
    """One workspace, several calls in a row (the second smaller), each result the oracle's and
    the workspace zero after each."""
    rng = np.random.default_rng(21)
    ws = ops.deviation_select_workspace(DEV)
    for N, L in ((9000, 300), (3000, 100), (9000, 300)):
        chunks = [(c * L, L) for c in range(N // L - 1)]
        flags, spans, local, active = _layout(N, chunks, 4, 0.3)
        k, v, K, V = _rows(rng, N, _chunk_sigma(rng, N, chunks))
        _run_and_check(k, v, K, V, flags, local, active, spans, None, ws=ws, expect_top=True)


def test_graph_replays_match_eager():
    """Captured once, replayed three times with eager work between the replays: every replay's
    outputs equal the eager call's (the kernel clears its own workspace, no memset node)."""
    rng = np.random.default_rng(99)
    N = 24 * 320 + 576
    chunks = [(c * 320, 320) for c in range(24)]
    flags, spans, local, active = _layout(N, chunks, 4, 0.3)
    k, v, K, V = _rows(rng, N, _chunk_sigma(rng, N, chunks))
    kt = O.from_numpy(k[:, active], DEV)[None]
    vt = O.from_numpy(v[:, active], DEV)[None]
    Kt, Vt = O.from_numpy(K, DEV)[None], O.from_numpy(V, DEV)[None]
    fl, lo, sp = O.from_numpy(flags, DEV), O.from_numpy(local, DEV), O.from_numpy(spans.reshape(-1), DEV)
    ws = ops.deviation_select_workspace(DEV)
    d0, n0, s0 = ops.deviation_select(kt, vt, Kt, Vt, fl, lo, sp, None, ws)
    n = 2976  # keep_abs is defined for the kept count only
    eager = [t.clone() for t in (d0, n0, s0.keep_abs[:n], s0.keep_rank, s0.counts)]
    outs = (torch.empty_like(d0), torch.empty_like(n0))
    sel = ops._new_selection(N, len(spans), kt.device)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ops.deviation_select(kt, vt, Kt, Vt, fl, lo, sp, None, ws, out=sel, diff_norm=outs)
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.deviation_select(kt, vt, Kt, Vt, fl, lo, sp, None, ws, out=sel, diff_norm=outs)
    for _ in range(3):
        for t in (outs[0], outs[1], sel.keep_abs, sel.keep_rank, sel.counts):
            t.fill_(-1)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = (outs[0], outs[1], sel.keep_abs[:n], sel.keep_rank, sel.counts)
        for a, b in zip(got, eager):
            assert torch.equal(a, b)
        assert not ws.any()


def test_scatter_kept_rows_flags_bad_source_row():
    Kt = torch.zeros((1, 2, 16, 64), dtype=torch.bfloat16, device=DEV)
    Vt = torch.zeros_like(Kt)
    k = torch.ones((1, 2, 4, 64), dtype=torch.bfloat16, device=DEV)
    dst = torch.tensor([1, 5], dtype=torch.int64, device=DEV)
    src = torch.tensor([3, 4], dtype=torch.int64, device=DEV)  # 4 is past the 4 source rows
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    ops.scatter_kept_rows(Kt, Vt, k, k.clone(), dst, src, err)
    torch.cuda.synchronize()
    assert int(err.item()) == _native.DEVICE_ERR_RANGE
    assert (Kt[0, :, 1] == 1).all() and not Kt[0, :, 5].any()
