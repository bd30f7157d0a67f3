"""ckv_layer1_repair (layer 1's base cache, deviation, selection and kept-row scatter in one call,
torch_engine.py:96-103 and :117-156) against the same work done by the four launches it replaces
(ckv_rerope_gather_layers, ckv_deviation, ckv_select, ckv_scatter_kept_rows) and against the
oracle, bit for bit: the layer's K/V cache, diff/norm, keep_abs, keep_local, keep_rank, rel_dev,
escalated and the counts.

Cases: the 8k request's shape (24 chunks x 320 at shuffled positions + 576 uncached, 30 %), the
config-3 shape at 15/30/50 %, the replay's 32,832-token request,
small requests with exact and overlapping placements at head_dim 64 in bf16 and fp32, requests
with no placement, with every position exact (no fresh row), of one token and a ragged one, an
escalation threshold, a threshold bin ranked directly and one refined by radix passes, deviations
that tie (one histogram bin holding every candidate: more radix rounds, then equal keys ranked by
position), NaN deviations, one workspace across calls of
different sizes (the histogram is left zeroed), and replays of a captured HIP graph.

ckv_layer1_repair_gather (the same repair, whole layers of the later layers' base cache gathered
beside the selection, the dropped rows of the others with the kept rows' scatter) against
layer1_repair + rerope_gather (with and without the skip map) at the 8k, config-3 and replay
shapes, the edge requests, every element type / head size / head count the whole-layer gather is
built for, and graph replays; the gathered layers also against the oracle.

ckv_rerope_gather_layers_kept (that call's last launch alone) against rerope_gather(skip) then
scatter_kept_rows, with the kept-row count from the device or the host, at the 8k and replay
shapes and the edge requests, and with an out-of-range source row (skipped and flagged)."""

import numpy as np
import pytest
import torch

from chunkkv_amd import _native, ops
from chunkkv_amd.planner import local_index, plan_request
from chunkkv_amd.types import ChunkKV, Placement
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
THETA = 1e6
SENT = -7.0


class Request:
    """A blend request as the engine sees it at layer 1: chunk store (n_layers columns), plan,
    descriptors on the device and the fresh rows (cached rows + per-chunk noise)."""

    def __init__(self, seed, chunk_lens, starts, N, ratio=0.3, n_sink=4, H=4, D=128, dtype=torch.bfloat16,
                 n_layers=2, layer=1, exact=(), pool=None, noise=None, ratios=None, zero_store=False):
        g = torch.Generator(device=DEV).manual_seed(seed)
        rng = np.random.default_rng(seed)
        self.H, self.D, self.dtype, self.n_layers, self.layer, self.N = H, D, dtype, n_layers, layer, N
        self.zero_store = zero_store
        if pool is None:
            pool = [self._chunk(g, rng, L) for L in chunk_lens]
        self.pool = pool
        self.placements = [
            Placement(pool[c], s, exact=(i in exact), ratio=None if ratios is None else ratios[i])
            for i, (c, s) in enumerate(starts)
        ]
        plan = plan_request(N, self.placements, n_sink, ratio)
        self.plan = plan
        tab = np.array([[[k.data_ptr(), v.data_ptr()] for k, v in zip(ch.keys, ch.values)] for ch in plan.chunks],
                       dtype=np.uint64)
        self.tab = torch.from_numpy(tab.reshape(-1).view(np.int64)).to(DEV)
        self.segs = torch.from_numpy(plan.segments.reshape(-1).copy()).to(DEV)
        self.n_segs = len(plan.segments)
        self.flags_np = plan.flags
        self.local_np = local_index(N, plan.layer0_idx)
        self.flags = torch.from_numpy(self.flags_np).to(DEV)
        self.local = torch.from_numpy(self.local_np).to(DEV)
        self.spans = torch.from_numpy(plan.spans.reshape(-1).copy()).to(DEV)
        self.err = torch.zeros(1, dtype=torch.int32, device=DEV)
        # fresh rows of the active positions: the re-rotated cached row plus per-chunk noise
        # (uncached positions: random), k contiguous, v token-major as v_proj leaves it
        base_k, base_v = self.gather_reference()[:2]
        n_act = len(plan.layer0_idx)
        act = torch.from_numpy(plan.layer0_idx).to(DEV)
        cached = torch.from_numpy(plan.cached).to(DEV)[act][None, None, :, None]
        sig = torch.ones(N, device=DEV)
        for p in self.placements:
            L = int(p.chunk.keys[0].shape[2])
            s = float(torch.exp(torch.randn((), generator=g, device=DEV) - 3.0)) if noise is None else noise
            sig[p.start : p.start + L] = s
        sig = sig[act][None, None, :, None]
        rnd = lambda: torch.randn((1, H, n_act, D), generator=g, device=DEV)  # noqa: E731
        bk, bv = base_k[:, :, act].float(), base_v[:, :, act].float()
        self.k = torch.where(cached, bk + sig * rnd(), rnd()).to(dtype)
        v_rows = torch.where(cached, bv + sig * rnd(), rnd()).to(dtype)
        self.v = v_rows.transpose(1, 2).contiguous().transpose(1, 2)

    def _chunk(self, g, rng, L):
        mk = lambda: (torch.zeros((1, self.H, L, self.D), device=DEV) if self.zero_store  # noqa: E731
                      else torch.randn((1, self.H, L, self.D), generator=g, device=DEV)).to(self.dtype)
        keys = [mk() for _ in range(self.n_layers)]
        values = [mk() for _ in range(self.n_layers)]
        return ChunkKV(keys, values, int(rng.integers(0, 4096)))

    def gather_reference(self):
        """Layer `layer` of a slab filled by ckv_rerope_gather_layers (sentinel elsewhere)."""
        K = torch.full((self.n_layers, 1, self.H, self.N, self.D), SENT, dtype=self.dtype, device=DEV)
        V = torch.full_like(K, SENT)
        if self.n_segs:
            ops.rerope_gather(K, V, self.tab, self.segs, self.n_segs, self.plan.max_seg_tokens, THETA, self.err,
                              layers=(self.layer, self.layer + 1))
        return K[self.layer], V[self.layer], K, V

    def four_launches(self, thr):
        K, V, _, _ = self.gather_reference()
        K, V = K.clone(), V.clone()
        diff, norm = ops.deviation(self.k, self.v, K, V, self.flags, self.local, self.err)
        sel = ops.select(diff, norm, self.flags, self.local, self.spans, thr)
        n = int(sel.counts[0].item())
        ops.scatter_kept_rows(K, V, self.k, self.v, sel.keep_abs[:n], sel.keep_local[:n], self.err)
        return K, V, diff, norm, sel

    def fused(self, thr, ws, out=None):
        K = torch.full((1, self.H, self.N, self.D), 3.0, dtype=self.dtype, device=DEV)
        V = torch.full_like(K, 3.0)
        diff, norm, sel = ops.layer1_repair(K, V, self.tab, self.n_layers, self.layer, self.segs, self.n_segs,
                                            self.k, self.v, self.flags, self.local, self.spans, thr, THETA, ws,
                                            self.err, out)
        return K, V, diff, norm, sel


def _bits(t):
    return O.to_numpy(t)


def _same(a, b, what):
    np.testing.assert_array_equal(_bits(a), _bits(b), err_msg=what)


def check(req: Request, thr=None, ws=None, oracle=True):
    """Fused vs the four launches (and the oracle when asked), bit for bit; returns the counts."""
    ws = ops.layer1_repair_workspace(DEV) if ws is None else ws
    Kr, Vr, dr, nr, sr = req.four_launches(thr)
    Kf, Vf, df, nf, sf = req.fused(thr, ws)
    torch.cuda.synchronize()
    assert int(req.err.item()) == 0, f"device status {int(req.err.item())}"
    N, C = req.N, len(req.plan.spans)
    cr, cf = _bits(sr.counts), _bits(sf.counts)
    np.testing.assert_array_equal(cf[:7], cr[:7], err_msg="counts")
    n = int(cr[0])
    _same(df.view(torch.int32), dr.view(torch.int32), "diff")
    _same(nf.view(torch.int32), nr.view(torch.int32), "norm")
    _same(sf.keep_abs[:n], sr.keep_abs[:n], "keep_abs")
    _same(sf.keep_local[:n], sr.keep_local[:n], "keep_local")
    _same(sf.keep_rank, sr.keep_rank, "keep_rank")
    if C:
        _same(sf.rel_dev[:C].view(torch.int32), sr.rel_dev[:C].view(torch.int32), "rel_dev")
        _same(sf.escalated[:C], sr.escalated[:C], "escalated")
    _same(Kf, Kr, "K cache")
    _same(Vf, Vr, "V cache")
    if oracle:
        Ko = np.full((1, req.H, N, req.D), 0, dtype=np.uint16 if req.dtype == torch.bfloat16 else np.float32)
        Vo = np.zeros_like(Ko)
        ks = [[_bits(ch.keys[req.layer])[0]] for ch in req.plan.chunks]
        vs = [[_bits(ch.values[req.layer])[0]] for ch in req.plan.chunks]
        if req.n_segs:
            assert O.rerope_gather(Ko, Vo, ks, vs, req.plan.segments, THETA) == 0
        act = req.plan.layer0_idx
        k_np = _bits(req.k)[0]
        v_np = np.ascontiguousarray(_bits(req.v.contiguous())[0])
        d_o, n_o = O.deviation(k_np, v_np, Ko[0], Vo[0], req.flags_np, req.local_np)
        np.testing.assert_array_equal(_bits(df).view(np.uint32), d_o.view(np.uint32))
        want = O.select(d_o, n_o, req.flags_np, req.local_np, req.plan.spans, thr)
        np.testing.assert_array_equal(cf[:7], want["counts"][:7])
        np.testing.assert_array_equal(_bits(sf.keep_abs)[:n], want["keep_abs"])
        np.testing.assert_array_equal(_bits(sf.keep_rank), want["keep_rank"])
        ka, kl = want["keep_abs"], want["keep_local"]
        K1, V1 = Ko[0].copy(), Vo[0].copy()
        K1[:, ka], V1[:, ka] = k_np[:, kl], v_np[:, kl]
        np.testing.assert_array_equal(_bits(Kf)[0], K1)
        np.testing.assert_array_equal(_bits(Vf)[0], V1)
        assert len(act) == len(req.local_np[req.local_np >= 0])
    return cf


def _shuffled(rng, n_chunks, L, tail):
    order = rng.permutation(n_chunks)
    return [(int(c), int(j * L)) for j, c in enumerate(order)], n_chunks * L + tail


def test_8k_request_shape():
    """24 chunks x 320 at shuffled positions + 576 uncached positions, 30 % + 4 sinks: 8256
    positions, six per wavefront (T = 6), 2976 kept rows."""
    rng = np.random.default_rng(8)
    starts, N = _shuffled(rng, 24, 320, 576)
    req = Request(8, [320] * 24, starts, N)
    counts = check(req)
    assert counts[0] == 2976 and req.plan.n_keep == 2976


@pytest.mark.parametrize("N_tail", [0, 576])
def test_uncorrelated_rows_in_histogram_copies(N_tail):
    """Fresh rows that do not follow the cached ones (noise 30 x the rows' own scale: every
    deviation within a few percent of the others, most candidates in a few histogram bins) at
    sizes where the layer-1 pass counts into four histogram copies (above 2048 positions): the
    call, its merged form and the oracle agree bit for bit."""
    rng = np.random.default_rng(11 + N_tail)
    starts, N = _shuffled(rng, 24, 320, N_tail)
    req = Request(11 + N_tail, [320] * 24, starts, N, noise=30.0, n_layers=4)
    check(req)
    _, _, sm, _ = _merged_vs_separate(req)
    assert int(sm.counts[0].item()) == req.plan.n_keep


@pytest.mark.parametrize("ratio", [0.15, 0.3, 0.5])
def test_config3_shape(ratio):
    """32 chunks x 256 in order (shift 0 keeps the keys bit for bit), T = 4."""
    starts = [(c, c * 256) for c in range(32)]
    req = Request(int(ratio * 100), [256] * 32, starts, 8192, ratio=ratio)
    counts = check(req)
    assert counts[0] == {0.15: 1344, 0.3: 2592, 0.5: 4224}[ratio]


def test_replay_request_shape_tiles_beyond_the_grid():
    """128 chunks of 256 drawn with replacement (Zipf 1.1) from 24, + 64 query positions: 32,832
    positions, more tiles than workgroups (reloaded rows), chunks repeated at several shifts."""
    rng = np.random.default_rng(55)
    zipf = 1.0 / np.arange(1, 25) ** 1.1
    ids = rng.choice(24, 128, p=zipf / zipf.sum())
    starts = [(int(c), j * 256) for j, c in enumerate(ids)]
    req = Request(55, [256] * 24, starts, 128 * 256 + 64, ratio=0.15)
    counts = check(req, oracle=False)
    assert counts[0] == req.plan.n_keep


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_small_exact_and_overlapping_head_dim_64(dtype):
    """0.5B KV shape (2 heads x 64): an exact placement (never recomputed: cached rows only),
    overlapping placements (the later one wins), a ratio-0 placement, uncached gaps."""
    lens = [40, 33, 50, 29, 61]
    starts = [(0, 5), (1, 60), (2, 80), (3, 150), (4, 190)]  # 2 overlaps 1 (80 < 93)
    req = Request(3, lens, starts, 270, H=2, D=64, dtype=dtype, n_layers=3, layer=1, exact=(3,),
                  ratios=[0.3, 0.5, None, 0.0, 0.25])
    assert req.plan.has_overlap and req.plan.exact.any()
    check(req)


@pytest.mark.parametrize("case", ["no_placements", "every_position_exact", "one_token", "ragged"])
def test_edge_requests(case):
    """No placement (no segment, no span: every position uncached and kept); one exact placement
    covering the request (no fresh row, nothing kept: the scatter reads nothing); a one-token
    request (its only position a sink); a 33-token chunk at offset 3 of 40 positions."""
    lens, starts, N, exact, keep = {
        "no_placements": ([], [], 7, (), 7),
        "every_position_exact": ([50], [(0, 0)], 50, (0,), 0),
        "one_token": ([1], [(0, 0)], 1, (), 1),
        "ragged": ([33], [(0, 3)], 40, (), None),
    }[case]
    req = Request(40 + N, lens, starts, N, exact=exact)
    counts = check(req)
    assert counts[0] == req.plan.n_keep
    if keep is not None:
        assert counts[0] == keep


def test_escalation_threshold():
    """Chunks whose relative deviation passes the threshold keep every position and leave the
    pool; the threshold sits between the chunks' noise levels."""
    rng = np.random.default_rng(7)
    starts, N = _shuffled(rng, 12, 128, 100)
    req = Request(7, [128] * 12, starts, N, ratio=0.3)
    rel = O.to_numpy(req.four_launches(None)[4].rel_dev)[:12]
    thr = float(np.median(rel))
    counts = check(req, thr=thr)
    esc = int((rel > thr).sum())
    assert 0 < esc < 12 and counts[0] > req.plan.n_keep


def test_tied_deviations_rank_by_position():
    """Fresh rows equal to the cached ones: every candidate's deviation is 0, below the
    histogram's window, so the selection runs its full radix passes; the lowest positions win."""
    starts = [(c, c * 256) for c in range(48)]
    req = Request(11, [256] * 48, starts, 48 * 256 + 64, ratio=0.3, noise=0.0)
    counts = check(req, oracle=False)
    assert counts[_native.COUNT_TOP_HISTOGRAM] == 0


def test_quantised_deviations_tie_inside_the_list():
    """Three distinct deviation values (a zero store, fresh rows zero but for one element of 0.5, 1
    or 2): the ties at the threshold go by position."""
    starts = [(c, c * 64) for c in range(16)]
    req = Request(12, [64] * 16, starts, 16 * 64 + 8, ratio=0.5, noise=0.0, zero_store=True)
    k = req.k.clone()
    cached = torch.from_numpy(req.plan.cached[req.plan.layer0_idx]).to(DEV)
    mag = torch.tensor([0.5, 1.0, 2.0], device=DEV)[torch.arange(k.shape[2], device=DEV) % 3]
    k[0, 0, :, 0] = torch.where(cached, mag, k[0, 0, :, 0].float()).to(k.dtype)
    req.k = k
    counts = check(req)
    assert counts[_native.COUNT_TOP_HISTOGRAM] & 1 == 1


def _refresh_rows(req, sig):
    """Fresh rows = the cached rows + sig[position] x N(0, 1) (uncached positions random)."""
    g = torch.Generator(device=DEV).manual_seed(77)
    base_k, base_v = req.gather_reference()[:2]
    act = torch.from_numpy(req.plan.layer0_idx).to(DEV)
    cached = torch.from_numpy(req.plan.cached).to(DEV)[act][None, None, :, None]
    sig = sig[None, None, :, None]
    rnd = lambda: torch.randn((1, req.H, len(act), req.D), generator=g, device=DEV)  # noqa: E731
    req.k = torch.where(cached, base_k[:, :, act].float() + sig * rnd(), rnd()).to(req.dtype)
    v_rows = torch.where(cached, base_v[:, :, act].float() + sig * rnd(), rnd()).to(req.dtype)
    req.v = v_rows.transpose(1, 2).contiguous().transpose(1, 2)


def test_threshold_bin_ranked_directly():
    """A noise level per position spread over decades: few candidates share the threshold's
    histogram bin, so they are ranked directly (counts[7] bit 1), bit-exact with the oracle."""
    starts = [(c, c * 256) for c in range(24)]
    req = Request(21, [256] * 24, starts, 24 * 256 + 64, ratio=0.3)
    g = torch.Generator(device=DEV).manual_seed(21)
    _refresh_rows(req, torch.exp(2.0 * torch.randn(len(req.plan.layer0_idx), generator=g, device=DEV)))
    counts = check(req)
    assert counts[_native.COUNT_TOP_HISTOGRAM] == 3


def test_threshold_bin_refined_by_radix_passes():
    """One noise level everywhere: every candidate's deviation lies within a few percent, a few
    1/64-octave bins hold them all, and the threshold's bin is refined by radix passes (counts[7]
    bit 1 clear)."""
    starts = [(c, c * 256) for c in range(24)]
    req = Request(22, [256] * 24, starts, 24 * 256 + 64, ratio=0.3)
    _refresh_rows(req, torch.full((len(req.plan.layer0_idx),), 0.05, device=DEV))
    counts = check(req)
    assert counts[_native.COUNT_TOP_HISTOGRAM] == 1


@pytest.mark.parametrize("sig,top", [(3e5, 0), (None, 1)])
def test_threshold_beyond_the_histogram_window(sig, top):
    """Deviations above the histogram's window (about 2^40): with every candidate there the
    threshold's bin is an edge bin and the selection runs its full radix passes (counts[7] 0);
    with a few positions there and the rest spread over decades the threshold bin is interior
    (the edge bin only counts above it). Both bit-exact with the oracle."""
    starts = [(c, c * 256) for c in range(24)]
    req = Request(23, [256] * 24, starts, 24 * 256 + 64, ratio=0.3)
    n = len(req.plan.layer0_idx)
    if sig is None:
        g = torch.Generator(device=DEV).manual_seed(23)
        s = torch.exp(1.5 * torch.randn(n, generator=g, device=DEV))
        s[::97] = 3e5  # deviations ~1e14, in the top edge bin
    else:
        s = torch.full((n,), sig, device=DEV)
    _refresh_rows(req, s)
    counts = check(req)
    assert counts[_native.COUNT_TOP_HISTOGRAM] & 1 == top


def test_nan_deviations_rank_last():
    starts = [(c, c * 200) for c in range(10)]
    req = Request(13, [200] * 10, starts, 2100, ratio=0.4)
    k = req.k.clone()
    k[0, 1, 5:40, 3] = float("nan")
    req.k = k
    check(req)


def test_one_workspace_across_sizes():
    """The selection leaves the histogram zeroed: calls of any size follow each other on one
    workspace (the replay-size call counts no histogram)."""
    ws = ops.layer1_repair_workspace(DEV)
    for seed, (n_ch, L, tail) in enumerate([(24, 320, 576), (3, 50, 17), (136, 256, 0), (32, 256, 0), (6, 100, 300)]):
        rng = np.random.default_rng(100 + seed)
        starts, N = _shuffled(rng, n_ch, L, tail)
        check(Request(100 + seed, [L] * n_ch, starts, N), ws=ws, oracle=False)
        assert not ws.any()


def test_graph_replays():
    """One captured launch replayed three times, eager work and a synchronisation between the
    replays, each replay's outputs equal to the eager call's."""
    rng = np.random.default_rng(30)
    starts, N = _shuffled(rng, 24, 320, 576)
    req = Request(30, [320] * 24, starts, N)
    ws = ops.layer1_repair_workspace(DEV)
    Kr, Vr, dr, nr, sr = req.fused(None, ws)
    torch.cuda.synchronize()
    K = torch.zeros_like(Kr)
    V = torch.zeros_like(Vr)
    out = ops._new_selection(N, len(req.plan.spans), DEV)
    dn = (torch.empty_like(dr), torch.empty_like(nr))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ops.layer1_repair(K, V, req.tab, req.n_layers, req.layer, req.segs, req.n_segs, req.k, req.v, req.flags,
                          req.local, req.spans, None, THETA, ws, req.err, out, dn)
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.layer1_repair(K, V, req.tab, req.n_layers, req.layer, req.segs, req.n_segs, req.k, req.v, req.flags,
                          req.local, req.spans, None, THETA, ws, req.err, out, dn)
    for i in range(3):
        K.fill_(float(i))
        out.keep_rank.fill_(-5)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert int(req.err.item()) == 0
        _same(K, Kr, f"K, replay {i}")
        _same(V, Vr, f"V, replay {i}")
        _same(dn[0].view(torch.int32), dr.view(torch.int32), f"diff, replay {i}")
        _same(out.keep_rank, sr.keep_rank, f"keep_rank, replay {i}")
        n = int(sr.counts[0].item())
        _same(out.keep_abs[:n], sr.keep_abs[:n], f"keep_abs, replay {i}")
        _same(out.counts[:7], sr.counts[:7], f"counts, replay {i}")


def _merged_vs_separate(req, thr=None, ws=None, layers=None):
    """ckv_layer1_repair_gather (layer `req.layer` repaired; the first layers of `layers` gathered
    whole beside the selection, the kept rows' scatter and the gather of the dropped rows of the
    others in one launch) against layer1_repair + rerope_gather(layers, skip=keep_rank), and
    rerope_gather(layers) for the layers gathered whole: every layer of both slabs, the diff/norm
    and the selection, bit for bit. Returns (K, V, selection, number of layers gathered whole)."""
    L = req.n_layers
    layers = (req.layer + 1, L) if layers is None else layers
    ws = ops.layer1_repair_workspace(DEV) if ws is None else ws
    shape = (L, 1, req.H, req.N, req.D)
    Ks, Vs = torch.full(shape, SENT, dtype=req.dtype, device=DEV), torch.full(shape, -SENT, dtype=req.dtype, device=DEV)
    Km, Vm = Ks.clone(), Vs.clone()
    ds, ns, ss = ops.layer1_repair(Ks[req.layer], Vs[req.layer], req.tab, L, req.layer, req.segs, req.n_segs, req.k,
                                   req.v, req.flags, req.local, req.spans, thr, THETA, ws, req.err)
    if req.n_segs:
        ops.rerope_gather(Ks, Vs, req.tab, req.segs, req.n_segs, req.plan.max_seg_tokens, THETA, req.err,
                          layers=layers, skip=ss.keep_rank)
    dm, nm, sm = ops.layer1_repair_gather(Km, Vm, req.tab, req.layer, layers, req.segs, req.n_segs,
                                          req.plan.max_seg_tokens, req.k, req.v, req.flags, req.local, req.spans, thr,
                                          THETA, ws, req.err)
    torch.cuda.synchronize()
    assert int(req.err.item()) == 0, f"device status {int(req.err.item())}"
    assert not ws.any()
    n = int(ss.counts[0].item())
    _same(sm.counts[:7], ss.counts[:7], "counts")
    _same(dm.view(torch.int32), ds.view(torch.int32), "diff")
    _same(nm.view(torch.int32), ns.view(torch.int32), "norm")
    _same(sm.keep_abs[:n], ss.keep_abs[:n], "keep_abs")
    _same(sm.keep_local[:n], ss.keep_local[:n], "keep_local")
    _same(sm.keep_rank, ss.keep_rank, "keep_rank")
    Kd, Vd = torch.full(shape, SENT, dtype=req.dtype, device=DEV), torch.full(shape, -SENT, dtype=req.dtype, device=DEV)
    if req.n_segs:
        ops.rerope_gather(Kd, Vd, req.tab, req.segs, req.n_segs, req.plan.max_seg_tokens, THETA, req.err,
                          layers=layers)
    torch.cuda.synchronize()
    # the leading layers of the range gathered whole, as the library reports them
    n_pre = ops.layer1_repair_gather_whole_layers(req.N, len(req.plan.spans), thr, req.n_segs, req.plan.max_seg_tokens,
                                                  layers, req.H, req.D, req.dtype)
    assert 0 <= n_pre <= layers[1] - layers[0]
    for li in range(L):
        whole = layers[0] <= li < layers[0] + n_pre
        _same(Km[li], Kd[li] if whole else Ks[li], f"K layer {li}")
        _same(Vm[li], Vd[li] if whole else Vs[li], f"V layer {li}")
    return Km, Vm, sm, n_pre


def test_merged_gather_8k_request_shape():
    """The 8k request's shape with 5 layers: layer 1 repaired, the dropped rows of layers 2-4
    gathered in the scatter's launch; layer 0 left as it was. The gathered layers also match the
    oracle: every cached row re-rotated except the kept ones, which keep the slab's fill."""
    rng = np.random.default_rng(81)
    starts, N = _shuffled(rng, 24, 320, 576)
    req = Request(81, [320] * 24, starts, N, n_layers=5)
    Km, Vm, sm, n_pre = _merged_vs_separate(req)
    assert int(sm.counts[0].item()) == 2976
    assert n_pre == 2  # ~8 KiB of traffic a position: two whole layers of 31.5 MB
    kept = _bits(sm.keep_rank) >= 0
    ks = [[_bits(ch.keys[li])[0] for li in range(5)] for ch in req.plan.chunks]
    vs = [[_bits(ch.values[li])[0] for li in range(5)] for ch in req.plan.chunks]
    for li in (2, 4):
        Ko = np.full((req.H, N, req.D), 0, dtype=np.uint16)
        Vo = np.zeros_like(Ko)
        assert O.rerope_gather(Ko[None], Vo[None], [[c[li]] for c in ks], [[c[li]] for c in vs], req.plan.segments,
                               THETA) == 0
        gathered = req.plan.cached & (~kept | (li < 2 + n_pre))
        np.testing.assert_array_equal(_bits(Km[li])[0][:, gathered], Ko[:, gathered], err_msg=f"K layer {li}")
        np.testing.assert_array_equal(_bits(Vm[li])[0][:, gathered], Vo[:, gathered], err_msg=f"V layer {li}")
        sent = _bits(torch.tensor(SENT, dtype=req.dtype))
        assert (_bits(Km[li])[0][:, ~gathered] == sent).all()


@pytest.mark.parametrize("ratio", [0.15, 0.5])
def test_merged_gather_config3_shape(ratio):
    starts = [(c, c * 256) for c in range(32)]
    req = Request(90 + int(ratio * 100), [256] * 32, starts, 8192, ratio=ratio, n_layers=4)
    assert _merged_vs_separate(req)[3] == 2  # both layers of the range: ~8 KiB a position


def test_merged_gather_replay_request_shape():
    """The replay's 32,832-position request (128 chunks of 256 drawn from 24, + 64 query
    positions), 3 layers, chunks repeated at several shifts."""
    rng = np.random.default_rng(56)
    zipf = 1.0 / np.arange(1, 25) ** 1.1
    ids = rng.choice(24, 128, p=zipf / zipf.sum())
    starts = [(int(c), j * 256) for j, c in enumerate(ids)]
    req = Request(56, [256] * 24, starts, 128 * 256 + 64, ratio=0.15, n_layers=3)
    assert _merged_vs_separate(req)[3] == 0  # above 16384 positions: the spread selection


@pytest.mark.parametrize("case", ["threshold", "small_f32", "no_placements", "every_position_exact", "empty_layers"])
def test_merged_gather_edges(case):
    """An escalation threshold (the single-workgroup selection), fp32 at head_dim 64 with an
    exact and overlapping placements, no placement (nothing to gather: the launch scatters only),
    every position exact (nothing kept: the launch gathers only), and an empty layer range."""
    if case == "threshold":
        rng = np.random.default_rng(9)
        starts, N = _shuffled(rng, 12, 128, 100)
        req = Request(9, [128] * 12, starts, N, ratio=0.3, n_layers=4)
        rel = O.to_numpy(req.four_launches(None)[4].rel_dev)[:12]
        _merged_vs_separate(req, thr=float(np.median(rel)))
        return
    if case == "small_f32":
        req = Request(4, [40, 33, 50, 29, 61], [(0, 5), (1, 60), (2, 80), (3, 150), (4, 190)], 270, H=2, D=64,
                      dtype=torch.float32, n_layers=4, exact=(3,), ratios=[0.3, 0.5, None, 0.0, 0.25])
    elif case == "no_placements":
        req = Request(5, [], [], 7, n_layers=3)
    elif case == "every_position_exact":
        req = Request(6, [50], [(0, 0)], 50, exact=(0,), n_layers=3)
    else:
        req = Request(7, [64] * 4, [(c, c * 64) for c in range(4)], 260, n_layers=2)
        _merged_vs_separate(req, layers=(2, 2))
        return
    _merged_vs_separate(req)


@pytest.mark.parametrize("dtype,D,H,whole", [(torch.bfloat16, 64, 4, True), (torch.bfloat16, 64, 8, True),
                                              (torch.bfloat16, 128, 1, True), (torch.bfloat16, 128, 2, True),
                                              (torch.float32, 128, 2, True), (torch.float32, 64, 4, True),
                                              (torch.bfloat16, 64, 3, False)])
def test_merged_gather_whole_layers_every_shape(dtype, D, H, whole):
    """The whole layers beside the selection at every element type and head size it is built
    for, head counts from 1 to 8 within the call's 1024-byte rows (a wavefront's rows are one
    head's: with a head count that does not divide 16 no layer is gathered whole); ragged chunk
    lengths leave partial items at the segments' ends."""
    rng = np.random.default_rng(D + H)
    lens = [int(x) for x in rng.integers(40, 300, 14)]
    starts, pos = [], 0
    for c in rng.permutation(14):
        starts.append((int(c), pos))
        pos += lens[c]
    req = Request(D + H, lens, starts, pos + 37, H=H, D=D, dtype=dtype, n_layers=5)
    n_pre = _merged_vs_separate(req)[3]
    assert (n_pre > 0) == whole, n_pre


def test_merged_gather_graph_replays():
    """ckv_layer1_repair_gather captured once (the whole-layer gather beside the selection
    included) and replayed three times, the slabs refilled between replays: every replay equals
    the eager call, every layer."""
    rng = np.random.default_rng(31)
    starts, N = _shuffled(rng, 24, 320, 576)
    req = Request(31, [320] * 24, starts, N, n_layers=5)
    ws = ops.layer1_repair_workspace(DEV)
    shape = (5, 1, req.H, N, req.D)
    Ke, Ve = torch.full(shape, SENT, dtype=req.dtype, device=DEV), torch.full(shape, -SENT, dtype=req.dtype, device=DEV)
    de, ne, se = ops.layer1_repair_gather(Ke, Ve, req.tab, 1, (2, 5), req.segs, req.n_segs, req.plan.max_seg_tokens,
                                          req.k, req.v, req.flags, req.local, req.spans, None, THETA, ws, req.err)
    torch.cuda.synchronize()
    K, V = torch.empty_like(Ke), torch.empty_like(Ve)
    out = ops._new_selection(N, len(req.plan.spans), DEV)
    dn = (torch.empty_like(de), torch.empty_like(ne))
    call = lambda: ops.layer1_repair_gather(K, V, req.tab, 1, (2, 5), req.segs, req.n_segs,  # noqa: E731
                                            req.plan.max_seg_tokens, req.k, req.v, req.flags, req.local, req.spans,
                                            None, THETA, ws, req.err, out, dn)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    for i in range(3):
        K.fill_(SENT)
        V.fill_(-SENT)
        out.keep_rank.fill_(-5)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert int(req.err.item()) == 0
        for li in range(5):
            _same(K[li], Ke[li], f"K layer {li}, replay {i}")
            _same(V[li], Ve[li], f"V layer {li}, replay {i}")
        _same(out.keep_rank, se.keep_rank, f"keep_rank, replay {i}")
        _same(dn[0].view(torch.int32), de.view(torch.int32), f"diff, replay {i}")
    assert not ws.any()


def _kept_vs_separate(req, layers, kept_layer=1, device_count=True):
    """ckv_rerope_gather_layers_kept after a selection against rerope_gather(layers,
    skip=keep_rank) then scatter_kept_rows into layer `kept_layer`: every layer of the slabs bit
    for bit. With device_count the kept-row count is the selection's device count and n_keep its
    upper bound N (the launch shape ckv_layer1_repair_gather uses); otherwise the host count."""
    L = req.n_layers
    ws = ops.layer1_repair_workspace(DEV)
    scratch = torch.empty((1, req.H, req.N, req.D), dtype=req.dtype, device=DEV)
    _, _, sel = ops.layer1_repair(scratch, torch.empty_like(scratch), req.tab, L, req.layer, req.segs, req.n_segs,
                                  req.k, req.v, req.flags, req.local, req.spans, None, THETA, ws, req.err)
    torch.cuda.synchronize()
    n = int(sel.counts[0].item())
    shape = (L, 1, req.H, req.N, req.D)
    Ks, Vs = torch.full(shape, SENT, dtype=req.dtype, device=DEV), torch.full(shape, -SENT, dtype=req.dtype, device=DEV)
    Km, Vm = Ks.clone(), Vs.clone()
    if req.n_segs:
        ops.rerope_gather(Ks, Vs, req.tab, req.segs, req.n_segs, req.plan.max_seg_tokens, THETA, req.err,
                          layers=layers, skip=sel.keep_rank)
    ops.scatter_kept_rows(Ks[kept_layer], Vs[kept_layer], req.k, req.v, sel.keep_abs[:n], sel.keep_local[:n], req.err)
    # with no segment the table and descriptors are empty (NULL): the launch scatters only
    ops.rerope_gather_layers_kept(Km, Vm, req.tab, req.segs, req.n_segs, req.plan.max_seg_tokens, THETA, layers, sel.keep_rank,
                                  kept_layer, req.k, req.v, sel.keep_abs, sel.keep_local, req.N if device_count else n,
                                  sel.counts[:1] if device_count else None, req.err)
    torch.cuda.synchronize()
    assert int(req.err.item()) == 0, f"device status {int(req.err.item())}"
    for li in range(L):
        _same(Km[li], Ks[li], f"K layer {li}")
        _same(Vm[li], Vs[li], f"V layer {li}")
    return Km, Vm, sel


@pytest.mark.parametrize("device_count", [True, False])
def test_gather_layers_kept_8k_request_shape(device_count):
    """The request step's last KV-repair launch called alone: the 8k request's kept rows of
    layer 1 beside the dropped rows of layers 2-5; the kept layer's rows also match the
    oracle's selection applied to the fresh rows."""
    rng = np.random.default_rng(83)
    starts, N = _shuffled(rng, 24, 320, 576)
    req = Request(83, [320] * 24, starts, N, n_layers=6)
    Km, _, sel = _kept_vs_separate(req, (2, 6), device_count=device_count)
    n = int(sel.counts[0].item())
    assert n == 2976
    ka, kl = _bits(sel.keep_abs)[:n], _bits(sel.keep_local)[:n]
    np.testing.assert_array_equal(_bits(Km[1])[0][:, ka], _bits(req.k)[0][:, kl])
    sent = _bits(torch.tensor(SENT, dtype=req.dtype))
    rest = np.ones(N, dtype=bool)
    rest[ka] = False
    assert (_bits(Km[1])[0][:, rest] == sent).all()


@pytest.mark.parametrize("case", ["kept_layer_first", "small_f32", "no_placements", "every_position_exact",
                                  "empty_layers", "replay_shape"])
def test_gather_layers_kept_edges(case):
    """The kept layer before the gathered range, fp32 at head_dim 64 with exact and overlapping
    placements, no placement (the launch scatters only), nothing kept (the launch gathers only),
    an empty layer range, and the replay's 32,832-position request (128 segments: the
    segment-fastest gather shape)."""
    if case == "kept_layer_first":
        rng = np.random.default_rng(12)
        starts, N = _shuffled(rng, 12, 128, 100)
        req = Request(12, [128] * 12, starts, N, n_layers=4, layer=0)
        _kept_vs_separate(req, (1, 4), kept_layer=0)
        return
    if case == "small_f32":
        req = Request(14, [40, 33, 50, 29, 61], [(0, 5), (1, 60), (2, 80), (3, 150), (4, 190)], 270, H=2, D=64,
                      dtype=torch.float32, n_layers=4, exact=(3,), ratios=[0.3, 0.5, None, 0.0, 0.25])
    elif case == "no_placements":
        req = Request(15, [], [], 7, n_layers=3)
    elif case == "every_position_exact":
        req = Request(16, [50], [(0, 0)], 50, exact=(0,), n_layers=3)
    elif case == "empty_layers":
        req = Request(17, [64] * 4, [(c, c * 64) for c in range(4)], 260, n_layers=3)
        _kept_vs_separate(req, (2, 2))
        return
    else:
        rng = np.random.default_rng(57)
        zipf = 1.0 / np.arange(1, 25) ** 1.1
        ids = rng.choice(24, 128, p=zipf / zipf.sum())
        req = Request(57, [256] * 24, [(int(c), j * 256) for j, c in enumerate(ids)], 128 * 256 + 64, ratio=0.15,
                      n_layers=3)
    _kept_vs_separate(req, (2, req.n_layers))


def test_gather_layers_kept_flags_an_out_of_range_source_row():
    """A kept row whose source row is past the fresh rows is skipped and flagged; every other row
    of the launch is written as the separate launches write it."""
    rng = np.random.default_rng(18)
    starts, N = _shuffled(rng, 8, 128, 60)
    req = Request(18, [128] * 8, starts, N, n_layers=3)
    ws = ops.layer1_repair_workspace(DEV)
    scratch = torch.empty((1, req.H, N, req.D), dtype=req.dtype, device=DEV)
    _, _, sel = ops.layer1_repair(scratch, torch.empty_like(scratch), req.tab, 3, 1, req.segs, req.n_segs, req.k,
                                  req.v, req.flags, req.local, req.spans, None, THETA, ws, req.err)
    torch.cuda.synchronize()
    n = int(sel.counts[0].item())
    assert n > 2
    bad = sel.keep_local.clone()
    bad[1] = req.k.shape[2]  # one past the last fresh row
    shape = (3, 1, req.H, N, req.D)
    K, V = torch.full(shape, SENT, dtype=req.dtype, device=DEV), torch.full(shape, -SENT, dtype=req.dtype, device=DEV)
    ops.rerope_gather_layers_kept(K, V, req.tab, req.segs, req.n_segs, req.plan.max_seg_tokens, THETA, (2, 3),
                                  sel.keep_rank, 1, req.k, req.v, sel.keep_abs, bad, n, None, req.err)
    torch.cuda.synchronize()
    assert int(req.err.item()) == _native.DEVICE_ERR_RANGE
    req.err.zero_()
    ka, kl = _bits(sel.keep_abs)[:n], _bits(sel.keep_local)[:n]
    good = np.arange(n) != 1
    np.testing.assert_array_equal(_bits(K[1])[0][:, ka[good]], _bits(req.k)[0][:, kl[good]])
    sent = _bits(torch.tensor(SENT, dtype=req.dtype))
    assert (_bits(K[1])[0][:, ka[1]] == sent).all()
