"""ckv_deviation_select_noalloc (the library's static scratch array instead of a caller workspace)
against ckv_deviation_select with a workspace, through the C ABI, bit for bit: the call captured
into a HIP graph as the process's first noalloc call (the scratch address looked up under
capture) and again after an eager call, each graph replayed three times; two eager calls in a
row on the same GPU, the second with a smaller request (and the oracle); a request above the
histogram's reach (more than 36864 positions: the scratch array is not used)."""

import numpy as np
import pytest
import torch

from chunkkv_amd import _native, ops
from chunkkv_amd._native import lib
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
H, D = 4, 128


def _case(seed, n_chunks, L, tail, ratio):
    rng = np.random.default_rng(seed)
    N = n_chunks * L + tail
    flags = np.zeros(N, dtype=np.uint8)
    spans = []
    for c in range(n_chunks):
        s = c * L
        flags[s : s + L] |= 1 | 8  # cached, pooled
        flags[s : s + 4] |= 2  # sinks
        spans.append((s, L, int(round(ratio * L)), 1))
    spans = np.array(spans, dtype=np.int32)
    local = np.arange(N, dtype=np.int32)
    sig = np.ones(N, dtype=np.float32)
    for c in range(n_chunks):
        sig[c * L : (c + 1) * L] = np.exp(rng.normal(-3.0, 1.0))
    fk = rng.standard_normal((H, N, D)).astype(np.float32)
    fv = rng.standard_normal((H, N, D)).astype(np.float32)
    K = fk + sig[None, :, None] * rng.standard_normal((H, N, D)).astype(np.float32)
    V = fv + sig[None, :, None] * rng.standard_normal((H, N, D)).astype(np.float32)
    b = O.f32_to_bf16_bits
    return N, b(fk), b(fv), b(K), b(V), flags, local, spans


def _noalloc(kt, vt, Kt, Vt, fl, lo, sp, C, N, out, diff, norm, err):
    rc = lib().ckv_deviation_select_noalloc(
        kt.data_ptr(), kt.stride(1), kt.stride(2), vt.data_ptr(), vt.stride(1), vt.stride(2), Kt.data_ptr(),
        Vt.data_ptr(), N * D, fl.data_ptr(), lo.data_ptr(), N, kt.shape[2], H, D, _native.DTYPE_BF16, sp.data_ptr(), C,
        0, 0.0, diff.data_ptr(), norm.data_ptr(), out.keep_abs.data_ptr(), out.keep_local.data_ptr(),
        out.keep_rank.data_ptr(), out.rel_dev.data_ptr(), out.escalated.data_ptr(), out.counts.data_ptr(),
        err.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rc == _native.CKV_OK


def _inputs(seed, n_chunks, L, tail, ratio=0.3):
    N, k, v, K, V, flags, local, spans = _case(seed, n_chunks, L, tail, ratio)
    kt = O.from_numpy(k, DEV)[None]
    vt = O.from_numpy(np.ascontiguousarray(v.transpose(1, 0, 2)), DEV)[None].transpose(1, 2)
    Kt, Vt = O.from_numpy(K, DEV)[None], O.from_numpy(V, DEV)[None]
    fl, lo, sp = O.from_numpy(flags, DEV), O.from_numpy(local, DEV), O.from_numpy(spans.reshape(-1), DEV)
    return N, len(spans), kt, vt, Kt, Vt, fl, lo, sp


def _same_as(out, diff, norm, d_ws, n_ws, s_ws, what):
    n = int(s_ws.counts[0].item())
    assert torch.equal(diff.view(torch.int32), d_ws.view(torch.int32)), what
    assert torch.equal(norm.view(torch.int32), n_ws.view(torch.int32)), what
    assert torch.equal(out.counts, s_ws.counts), what
    assert torch.equal(out.keep_abs[:n], s_ws.keep_abs[:n]) and torch.equal(out.keep_local[:n], s_ws.keep_local[:n])
    assert torch.equal(out.keep_rank, s_ws.keep_rank), what
    assert torch.equal(out.rel_dev.view(torch.int32), s_ws.rel_dev.view(torch.int32)), what
    assert torch.equal(out.escalated, s_ws.escalated), what


def test_noalloc_captured_first_then_after_an_eager_call():
    """Captured as the first noalloc call of the process, replayed three times (the outputs
    poisoned and eager work between replays); then an eager call and a second capture of a smaller
    request, replayed three times; every replay equal to the workspace entry point."""
    for seed, n_chunks, L, tail, eager_first in ((5, 24, 320, 576, False), (6, 12, 200, 40, True)):
        N, C, kt, vt, Kt, Vt, fl, lo, sp = _inputs(seed, n_chunks, L, tail)
        print(f"capture: N={N}, eager call first: {eager_first}", flush=True)
        ws = ops.deviation_select_workspace(DEV)
        d_ws, n_ws, s_ws = ops.deviation_select(kt, vt, Kt, Vt, fl, lo, sp, None, ws)
        out = ops._new_selection(N, C, kt.device)
        diff = torch.empty(N, dtype=torch.float32, device=DEV)
        norm = torch.empty(N, dtype=torch.float32, device=DEV)
        err = torch.zeros(1, dtype=torch.int32, device=DEV)
        if eager_first:
            _noalloc(kt, vt, Kt, Vt, fl, lo, sp, C, N, out, diff, norm, err)
            torch.cuda.synchronize()
            _same_as(out, diff, norm, d_ws, n_ws, s_ws, "eager call")
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            with torch.cuda.graph(g, stream=side):
                _noalloc(kt, vt, Kt, Vt, fl, lo, sp, C, N, out, diff, norm, err)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        for i in range(3):
            out.keep_rank.fill_(-5)
            out.counts.fill_(-1)
            diff.fill_(float("nan"))
            _ = torch.randn(1 << 20, device=DEV).sum()  # eager work between replays
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert int(err.item()) == 0
            _same_as(out, diff, norm, d_ws, n_ws, s_ws, f"replay {i}")
        del g


def test_noalloc_matches_workspace_entry_two_calls():
    for seed, n_chunks, L, tail in ((1, 24, 320, 576), (2, 12, 200, 40)):  # the second call smaller
        N, k, v, K, V, flags, local, spans = _case(seed, n_chunks, L, tail, 0.3)
        print(f"call: N={N}, {n_chunks} chunks of {L}", flush=True)
        kt = O.from_numpy(k, DEV)[None]
        vt = O.from_numpy(np.ascontiguousarray(v.transpose(1, 0, 2)), DEV)[None].transpose(1, 2)
        Kt, Vt = O.from_numpy(K, DEV)[None], O.from_numpy(V, DEV)[None]
        fl, lo, sp = O.from_numpy(flags, DEV), O.from_numpy(local, DEV), O.from_numpy(spans.reshape(-1), DEV)
        C = len(spans)
        ws = ops.deviation_select_workspace(DEV)
        d_ws, n_ws, s_ws = ops.deviation_select(kt, vt, Kt, Vt, fl, lo, sp, None, ws)
        out = ops._new_selection(N, C, kt.device)
        diff = torch.empty(N, dtype=torch.float32, device=DEV)
        norm = torch.empty(N, dtype=torch.float32, device=DEV)
        err = torch.zeros(1, dtype=torch.int32, device=DEV)
        _noalloc(kt, vt, Kt, Vt, fl, lo, sp, C, N, out, diff, norm, err)
        torch.cuda.synchronize()
        assert int(err.item()) == 0
        n = int(s_ws.counts[0].item())
        assert int(out.counts[_native.COUNT_TOP_HISTOGRAM].item()) & 1 == 1  # the scratch-backed path ran
        assert torch.equal(diff.view(torch.int32), d_ws.view(torch.int32))
        assert torch.equal(norm.view(torch.int32), n_ws.view(torch.int32))
        assert torch.equal(out.counts, s_ws.counts)
        assert torch.equal(out.keep_abs[:n], s_ws.keep_abs[:n]) and torch.equal(out.keep_local[:n], s_ws.keep_local[:n])
        assert torch.equal(out.keep_rank, s_ws.keep_rank)
        assert torch.equal(out.rel_dev.view(torch.int32), s_ws.rel_dev.view(torch.int32))
        assert torch.equal(out.escalated, s_ws.escalated)
        want = O.select(*O.deviation(k, v, K, V, flags, local), flags, local, spans, None)
        np.testing.assert_array_equal(O.to_numpy(out.keep_abs)[:n], want["keep_abs"])


def test_noalloc_above_the_histogram_reach():
    """40,000 positions (more than the 36864 the histogram paths take): the selection counts its
    own digits and the scratch array is not touched; the same outputs as the workspace entry."""
    N, C, kt, vt, Kt, Vt, fl, lo, sp = _inputs(7, 160, 250, 0)
    assert N == 40000
    ws = ops.deviation_select_workspace(DEV)
    d_ws, n_ws, s_ws = ops.deviation_select(kt, vt, Kt, Vt, fl, lo, sp, None, ws)
    out = ops._new_selection(N, C, kt.device)
    diff = torch.empty(N, dtype=torch.float32, device=DEV)
    norm = torch.empty(N, dtype=torch.float32, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    _noalloc(kt, vt, Kt, Vt, fl, lo, sp, C, N, out, diff, norm, err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    assert int(out.counts[_native.COUNT_TOP_HISTOGRAM].item()) & 1 == 0  # no histogram
    _same_as(out, diff, norm, d_ws, n_ws, s_ws, "40,000 positions")
