"""Blend-prefill KV-repair benchmark on one MI355X.

    python bench.py [--steps K] [--warmup W] [--ttft-requests R] [--cpu-seconds S]

Workload (the Qwen2.5-7B 8k-context blend prefill): 28 layers, 4 KV heads, head_dim 128,
bf16, rope theta 1e6; a request of N = 8256 tokens = 24 cached chunks of 320 tokens placed at
shuffled positions (each chunk computed at its own original offset, so every placement shifts
its keys), then a 512-token uncached tail and a 64-token query; 30% recompute, 4 sinks per chunk.

A step is one request's whole KV repair with every input already resident in HBM, issued as
HipEngine issues it (30 launches in order on one stream): layer 0's fresh rows written into its
cache; layer 1's repair with the base cache of layers 2-27 as one ckv_layer1_repair_gather call
of three launches (the cached rows of layer 1 re-rotated into its cache with the deviation; the
selection of 2304 pooled + 96 sinks + 576 uncached = 2976 kept rows, with layers 2-3 gathered
whole by the CUs the single-workgroup selection leaves idle; the scatter of layer 1's kept rows
with the gather of the cached rows of the 5280 dropped positions of layers 4-27); then the
fresh rows of layers 2-27 (they overwrite the kept rows of layers 2-3). The fresh rows are
written by ckv_rope_qkv as in the engine (k rotated to its position, v copied, straight into
the cache rows); the engine's launch also rotates q for the attention, which the step leaves
out as the reference's KV-repair bytes do.
The unit of work is one request's KV repair as the reference's op sequence moves it (re-RoPE +
gather of every cached row of all 28 layers, the layer-0 scatter of all 8256 rows, the
deviation, the scatters of layers 1-27):
    gather          28 x 24 x 320 x 4 heads x 128 x 2 B x 2 (K,V) x 2 (r+w) =   880,803,840
    deviation       8256 x (4 rows x 1 KiB) + 8256 x 8 B                       =    33,882,624
    scatter L0      8256 x 4096 B                                              =    33,816,576
    scatter L1-27   27 x 2976 x 4096 B                                         =   329,121,792
    total                                                                      = 1,277,624,832
`value` = that total / measured time per step (GB/s), the step replayed from a HIP graph (the
eager time, launch-bound from Python, is reported as ms_per_step_eager; with random layer-1
rows (every deviation within a few percent of the others) as ms_per_step_uncorrelated; layer 1
as ckv_layer1_repair and the dropped rows of layers 2-27 as a separate gather launch as
ms_per_step_separate_gather;
the same launches with the gathers on a second stream (HipEngine(overlap=True)) as
ms_per_step_two_streams; layer 1 as the four launches ckv_layer1_repair replaces (base-cache
gather, deviation, selection, scatter) as ms_per_step_layer1_four_launches; layers 0 and 2-27
built by one assemble launch each as ms_per_step_assemble_variant); the fused flow itself moves
moved_bytes_per_step (moved_gbs). `roofline` is the step's dominant kernel, its last KV-repair
launch of layer 1 (layer 1's kept rows beside the dropped rows of layers 4-27, 531,234,816 B),
called alone through ckv_rerope_gather_layers_kept with the step's inputs and launch shape and
timed live with HIP events around a burst of back-to-back launches on the launch stream; the
gather of the dropped rows of layers 2-27 as one launch (the separate-gather step's) is reported
beside it. Inputs rotate between two independent copies so
consecutive steps do not hit in the 256 MB MALL.

Besides the bandwidth line, the run measures blend-prefill TTFT p50 (prefill + last_logprobs,
the bracket of the reference's bench/replay.py:32-35) over seeded requests of the same shape on
a random-init Qwen2.5-7B-architecture bf16 model, for HipEngine and for the reference-op
sequence on PyTorch-ROCm, and the reference op sequence's KV repair on the host CPU
(cpu_baseline).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

from chunkkv_amd.gemm_tuning import use_tuned_gemms

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "KV-repair HBM GB/s (% of peak) + blend-prefill TTFT p50, Qwen2.5-7B 8k ctx"
PEAK_GBS = 8000.0  # MI355X HBM3E

N_LAYERS, N_KV, HEAD_DIM, THETA = 28, 4, 128, 1e6
CHUNK_LEN, N_CHUNKS, TAIL, QUERY = 320, 24, 512, 64
N_TOKENS = N_CHUNKS * CHUNK_LEN + TAIL + QUERY  # 8256
RATIO, N_SINK = 0.30, 4
ROW_BYTES = N_KV * HEAD_DIM * 2  # one token's K (or V) row set, bf16

GATHER_BYTES = N_LAYERS * N_CHUNKS * CHUNK_LEN * ROW_BYTES * 2 * 2
# HBM bytes per gather launch of this workload from the FETCH_SIZE / WRITE_SIZE counter passes
# (profiles/traffic_rerope_gather_qwen25_7b_8k.md; FETCH_SIZE calibrated against a kernel of
# known traffic). Counters cannot be read inside a timed run, so the measured value is recorded.
GATHER_TRAFFIC_BYTES = 881_089_130
# Same for one gather of the dropped rows of layers 2-27 of the 8k request (FETCH_SIZE median
# 137,468.3 KiB / 0.500023 + WRITE_SIZE median 274,560 KiB; 562,298,880 algorithmic bytes).
DROPPED_TRAFFIC_BYTES = 562_671_568
# rocprofv3 FETCH_SIZE / 0.500023 + WRITE_SIZE of the step's kept rows + dropped rows of layers
# 4-27 launch (266,093,411 B read, 259,392 KiB written)
MERGED_TRAFFIC_BYTES = 266_093_411 + 265_617_408
DEVIATION_BYTES = N_TOKENS * 4 * ROW_BYTES + N_TOKENS * 8


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


class Chunk:
    """ChunkKV-compatible holder whose per-layer tensors are views of one slab."""

    def __init__(self, k_slab, v_slab, start):
        self.keys = list(k_slab.unbind(0))
        self.values = list(v_slab.unbind(0))
        self.start = start

    @property
    def length(self):
        return self.keys[0].shape[2]


class Place:
    def __init__(self, chunk, start, ratio=None, exact=False):
        self.chunk, self.start, self.ratio, self.exact = chunk, start, ratio, exact


def rope_rows(x: torch.Tensor, positions: torch.Tensor, inv_freq: torch.Tensor) -> torch.Tensor:
    ang = positions.float()[:, None] * inv_freq[None, :]
    c, s = ang.cos(), ang.sin()
    a, b = x.float().chunk(2, dim=-1)
    return torch.cat((a * c - b * s, a * s + b * c), dim=-1).to(x.dtype)


def make_request(gen: torch.Generator, dev, inv_freq):
    """Chunks computed at their own offsets, placed at a shuffled order; returns placements."""
    chunks = []
    for _ in range(N_CHUNKS):
        orig = int(torch.randint(0, 8192, (1,), generator=gen))
        x = torch.randn((N_LAYERS, 1, N_KV, CHUNK_LEN, HEAD_DIM), generator=gen).to(dev)
        k = rope_rows(x, torch.arange(orig, orig + CHUNK_LEN, device=dev), inv_freq).to(torch.bfloat16)
        v = torch.randn((N_LAYERS, 1, N_KV, CHUNK_LEN, HEAD_DIM), generator=gen).to(dev).to(torch.bfloat16)
        chunks.append(Chunk(k, v, orig))
    order = torch.randperm(N_CHUNKS, generator=gen).tolist()
    return [Place(chunks[c], i * CHUNK_LEN) for i, c in enumerate(order)]


class RepairWorkload:
    """All device buffers of one request's KV repair (see module docstring)."""

    def __init__(self, seed: int, dev):
        from chunkkv_amd import ops
        from chunkkv_amd.planner import local_index, plan_request

        gen = torch.Generator().manual_seed(seed)
        self.inv = ops.inv_freq(HEAD_DIM, THETA, dev)
        self.placements = make_request(gen, dev, self.inv)
        plan = plan_request(N_TOKENS, self.placements, N_SINK, RATIO)
        assert plan.n_keep == 2976 and plan.budget == 2304
        self.plan = plan
        tab = np.concatenate(
            [np.array([[k.data_ptr(), v.data_ptr()] for k, v in zip(c.keys, c.values)], dtype=np.uint64).reshape(-1)
             for c in plan.chunks]
        )
        self.tab = torch.from_numpy(tab.view(np.int64)).to(dev)
        self.segs = torch.from_numpy(plan.segments.reshape(-1)).to(dev)
        self.segs_all = torch.from_numpy(plan.all_segments.reshape(-1)).to(dev)  # cached runs first
        self.flags = torch.from_numpy(plan.flags).to(dev)
        self.local = torch.from_numpy(local_index(N_TOKENS, plan.layer0_idx)).to(dev)
        self.spans = torch.from_numpy(plan.spans.reshape(-1)).to(dev)
        self.layer0 = torch.from_numpy(plan.layer0_idx.astype(np.int64)).to(dev)
        self.k_slab = torch.empty((N_LAYERS, 1, N_KV, N_TOKENS, HEAD_DIM), dtype=torch.bfloat16, device=dev)
        self.v_slab = torch.empty_like(self.k_slab)
        self.err = torch.zeros(1, dtype=torch.int32, device=dev)
        # Fresh rows: layer 1 = cached rows + per-chunk lognormal(-3, 1) noise (the model's
        # layer-1 K/V differ from the cached ones by a chunk-dependent amount); k is
        # contiguous, v token-major like the v_proj output.
        sigma = torch.exp(torch.randn(N_CHUNKS, generator=gen) - 3.0)
        noise = torch.ones(N_TOKENS)
        for i, p in enumerate(self.placements):
            noise[p.start : p.start + CHUNK_LEN] = sigma[i]
        base_k = torch.zeros((1, N_KV, N_TOKENS, HEAD_DIM))
        base_v = torch.zeros_like(base_k)
        for p in self.placements:
            delta = p.start - p.chunk.start
            ang = (delta * self.inv.cpu())[None, :]
            kc = p.chunk.keys[1].float().cpu()
            a, b = kc.chunk(2, dim=-1)
            base_k[:, :, p.start : p.start + CHUNK_LEN] = torch.cat((a * ang.cos() - b * ang.sin(), a * ang.sin() + b * ang.cos()), -1)
            base_v[:, :, p.start : p.start + CHUNK_LEN] = p.chunk.values[1].float().cpu()
        nk = base_k + noise[None, None, :, None] * torch.randn(base_k.shape, generator=gen)
        nv = base_v + noise[None, None, :, None] * torch.randn(base_v.shape, generator=gen)
        self.fresh = []
        for li in range(N_LAYERS):
            n = N_TOKENS if li < 2 else plan.n_keep
            if li == 1:
                k, v = nk, nv
            else:
                k = torch.randn((1, N_KV, n, HEAD_DIM), generator=gen)
                v = torch.randn((1, N_KV, n, HEAD_DIM), generator=gen)
            k = k.to(torch.bfloat16).to(dev)
            v = v.to(torch.bfloat16).transpose(1, 2).contiguous().to(dev).transpose(1, 2)
            self.fresh.append((k, v))
        # k/v projection outputs (token-major (1, n, H*D), before RoPE) of layers 0 and 2..27:
        # what ckv_rope_qkv turns into cache rows in the engine.
        self.proj = [None if li == 1 else tuple(
            torch.randn((1, N_TOKENS if li == 0 else plan.n_keep, N_KV * HEAD_DIM), generator=gen).to(torch.bfloat16)
            .to(dev) for _ in range(2)) for li in range(N_LAYERS)]
        self.sel = None
        self.ws = ops.deviation_select_workspace(dev)
        self.ws1 = ops.layer1_repair_workspace(dev)
        self.dn = (torch.empty(N_TOKENS, dtype=torch.float32, device=dev),
                   torch.empty(N_TOKENS, dtype=torch.float32, device=dev))
        self.side = torch.cuda.Stream(device=dev)  # default priority

    def gather(self):
        from chunkkv_amd import ops

        ops.rerope_gather(self.k_slab, self.v_slab, self.tab, self.segs, len(self.plan.segments),
                          self.plan.max_seg_tokens, THETA, self.err)

    def assemble(self, li: int):
        """One layer li >= 2 (or 0) as HipEngine builds it: every row written once."""
        from chunkkv_amd import ops

        plan = self.plan
        local = self.local if li == 0 else self.sel.keep_rank
        ops.assemble_layer(self.k_slab[li], self.v_slab[li], self.tab, N_LAYERS, li, self.segs_all,
                           len(plan.all_segments), plan.max_all_seg_tokens, *self.fresh[li], local, THETA, self.err)

    def gather_dropped(self):
        """Layers 2..27 in one launch: the cached rows of every position the selection dropped."""
        from chunkkv_amd import ops

        ops.rerope_gather(self.k_slab, self.v_slab, self.tab, self.segs, len(self.plan.segments),
                          self.plan.max_seg_tokens, THETA, self.err, layers=(2, N_LAYERS), skip=self.sel.keep_rank)

    def gather_kept(self):
        """The step's last KV-repair launch called alone (ckv_rerope_gather_layers_kept, as
        ckv_layer1_repair_gather issues it: the selection's device count, N its bound): layer 1's
        kept rows beside the dropped rows of the layers after those gathered whole."""
        from chunkkv_amd import ops

        k1, v1 = self.fresh[1]
        ops.rerope_gather_layers_kept(self.k_slab, self.v_slab, self.tab, self.segs, len(self.plan.segments),
                                      self.plan.max_seg_tokens, THETA, (2 + whole_layers(self.plan), N_LAYERS),
                                      self.sel.keep_rank, 1, k1, v1, self.sel.keep_abs, self.sel.keep_local, N_TOKENS,
                                      self.sel.counts[:1], self.err)

    def kv_rows(self, li: int):
        """Layer li's fresh rows into its cache as the engine writes them: the k/v part of
        ckv_rope_qkv (k rotated to its position, v copied, straight into the cache rows). The
        engine's launch also rotates q for the attention; the step leaves q out, as the
        reference's KV-repair bytes do."""
        from chunkkv_amd import ops

        pos = self.layer0 if li == 0 else self.sel.keep_abs[: self.plan.n_keep]
        k_in, v_in = self.proj[li]
        ops.rope_qkv(None, k_in, v_in, pos, 0, N_KV, HEAD_DIM, THETA, k_out=self.k_slab[li], v_out=self.v_slab[li],
                     rows=pos, err=self.err)

    layer1_mode = "one"  # as HipEngine: layer 1's whole repair in one call (ckv_layer1_repair)

    def step(self, two_streams: bool = False):
        """One request's KV repair as HipEngine issues it (30 launches, in order on one stream):
        layer 0's fresh rows; layer 1's base cache, deviation, selection and kept rows with the base
        cache of layers 2-27 in one call of three launches (ckv_layer1_repair_gather); the fresh rows
        of layers 2-27. With layer1_mode "separate_gather", layer 1 is ckv_layer1_repair and the
        dropped rows of layers 2-27 a gather launch of their own; with "split", layer 1 is the four
        launches ckv_layer1_repair replaces (base cache, deviation, selection, kept-row scatter).
        two_streams=True issues the gathers on a second stream instead, as HipEngine(overlap=True)
        does (beside the fresh rows they do not touch)."""
        from chunkkv_amd import ops

        plan = self.plan
        main = torch.cuda.current_stream()

        def fork(fn):
            if not two_streams:
                return fn()
            self.side.wait_stream(main)
            with torch.cuda.stream(self.side):
                fn()

        if self.layer1_mode == "one" and not two_streams:
            # as HipEngine: layer 1's repair with the dropped rows of layers 2-27 in its last launch
            self.kv_rows(0)
            self.layer1_gather()
            for li in range(2, N_LAYERS):
                self.kv_rows(li)
            return
        if self.layer1_mode in ("one", "separate_gather"):
            self.kv_rows(0)
            self.layer1_one()
        else:
            fork(lambda: ops.rerope_gather(self.k_slab, self.v_slab, self.tab, self.segs, len(plan.segments),
                                           plan.max_seg_tokens, THETA, self.err, layers=(1, 2)))
            self.kv_rows(0)
            if two_streams:
                main.wait_stream(self.side)
            self.layer1()
        fork(self.gather_dropped)
        for li in range(2, N_LAYERS):
            self.kv_rows(li)
        if two_streams:
            main.wait_stream(self.side)

    def layer1_gather(self):
        """Layer 1's whole repair and the gather of the dropped rows of layers 2-27 in one call of
        three launches (ckv_layer1_repair_gather): the cached rows re-rotated with the deviation,
        the selection, then the kept rows of layer 1 and the dropped rows of layers 2-27 in one
        launch."""
        from chunkkv_amd import ops

        k1, v1 = self.fresh[1]
        _, _, self.sel = ops.layer1_repair_gather(self.k_slab, self.v_slab, self.tab, 1, (2, N_LAYERS), self.segs,
                                                  len(self.plan.segments), self.plan.max_seg_tokens, k1, v1,
                                                  self.flags, self.local, self.spans, None, THETA, self.ws1, self.err,
                                                  self.sel, self.dn)

    def step_separate_gather(self):
        """The step with layer 1's repair and the dropped-row gather as separate calls (the kept
        rows' scatter its own launch)."""
        self.layer1_mode = "separate_gather"
        try:
            self.step()
        finally:
            self.layer1_mode = "one"

    def layer1_one(self):
        """Layer 1's whole repair in one call of three launches: the cached rows re-rotated from the
        chunk store with the deviation, the selection, the kept rows from the fresh rows
        (ckv_layer1_repair)."""
        from chunkkv_amd import ops

        k1, v1 = self.fresh[1]
        _, _, self.sel = ops.layer1_repair(self.k_slab[1], self.v_slab[1], self.tab, N_LAYERS, 1, self.segs,
                                           len(self.plan.segments), k1, v1, self.flags, self.local, self.spans, None,
                                           THETA, self.ws1, self.err, self.sel, self.dn)

    def layer1(self):
        """Layer 1 after its base cache, as three launches: the deviation, the selection, the kept
        rows compacted and scattered into the cache."""
        from chunkkv_amd import ops

        n = self.plan.n_keep
        K, V = self.k_slab[1], self.v_slab[1]
        k1, v1 = self.fresh[1]
        diff, norm = ops.deviation(k1, v1, K, V, self.flags, self.local, self.err)
        self.sel = ops.select(diff, norm, self.flags, self.local, self.spans, None, self.sel)
        ops.scatter_kept_rows(K, V, k1, v1, self.sel.keep_abs[:n], self.sel.keep_local[:n], self.err)

    def step_split(self):
        """The step with layer 1 as the four launches ckv_layer1_repair replaces."""
        self.layer1_mode = "split"
        try:
            self.step()
        finally:
            self.layer1_mode = "one"

    def step_two_streams(self):
        """The same launches with the gathers on a second stream."""
        self.step(two_streams=True)

    def step_assemble(self):
        """Layer 0 and layers 2-27 with one assemble launch each (every row written once, fresh
        rows from k/v tensors), one stream: the alternative when the caller's fresh rows already
        exist as tensors."""
        self._head()
        for li in range(2, N_LAYERS):
            self.assemble(li)

    def _head(self):
        from chunkkv_amd import ops

        plan = self.plan
        K, V = self.k_slab.unbind(0), self.v_slab.unbind(0)
        self.assemble(0)
        ops.assemble_layer(K[1], V[1], self.tab, N_LAYERS, 1, self.segs_all, len(plan.segments), plan.max_seg_tokens,
                           None, None, None, THETA, self.err)
        self.layer1()


def repair_bytes(n_keep: int) -> int:
    """Algorithmic bytes of one request's KV repair (module docstring)."""
    scatter_row = ROW_BYTES * 2 * 2  # K and V rows of one token, read + write
    return GATHER_BYTES + DEVIATION_BYTES + N_TOKENS * scatter_row + (N_LAYERS - 1) * n_keep * scatter_row


PREWARM_S = 0.2  # untimed calls before each timed burst: MI355X clocks ramp up over tens of ms of load


def _timed(fn, n: int, stream) -> float:
    """Average ms of n calls of fn(i), HIP events on `stream` around the whole burst. The burst
    follows PREWARM_S seconds of untimed calls of the same fn, so it is timed at the clocks a
    loaded GPU runs at rather than while they are still rising from idle."""
    t_end, i = time.perf_counter() + PREWARM_S, 0
    while time.perf_counter() < t_end:
        fn(i)
        i += 1
        if i % 8 == 0:
            torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for i in range(n):
        fn(i)
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / n


_REQUEST_STREAMS: list = []


def request_streams(n: int, dev) -> list:
    """n streams for concurrent requests, created once per process, ahead of every other stream,
    and shared by the concurrent measurements (as a server creates its request streams at start-up).
    HIP maps each stream onto one of its hardware queues (GPU_MAX_HW_QUEUES, 4 here) when the
    stream is created, and the mapping depends on the streams created before it: with request
    streams created after other measurements' streams, config 5's rounds took 3.20 ms against
    2.95 ms for the same work."""
    while len(_REQUEST_STREAMS) < n:
        _REQUEST_STREAMS.append(torch.cuda.Stream(device=dev))  # default priority
    return _REQUEST_STREAMS[:n]


def _graph_of(fn):
    """Capture fn() (already run once eagerly) into a HIP graph, warming it on a side stream."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


def bench_repair(steps: int, warmup: int, dev) -> dict:
    """Time the KV-repair step as HipEngine issues it (30 launches on one stream, captured once
    per input set in a HIP graph and replayed; the eager time, launch-bound from Python, layer 1
    as four launches, the two-stream issue and the assemble-per-layer variant are reported too),
    and the dominant kernel (the step's last launch: layer 1's kept rows with the dropped rows of
    layers 4-27) and the separate-gather step's gather of the dropped rows of layers 2-27, each
    from a burst of back-to-back launches."""
    wls = [RepairWorkload(1234 + i, dev) for i in range(2)]
    for i in range(max(warmup, 2)):
        wls[i % 2].step()
        wls[i % 2].step_two_streams()
        wls[i % 2].step_assemble()
        wls[i % 2].step_split()
        wls[i % 2].step_separate_gather()
    torch.cuda.synchronize()
    graphs = [_graph_of(w.step) for w in wls]
    two = [_graph_of(w.step_two_streams) for w in wls]
    asm_graphs = [_graph_of(w.step_assemble) for w in wls]
    split = [_graph_of(w.step_split) for w in wls]
    sep = [_graph_of(w.step_separate_gather) for w in wls]
    stream = torch.cuda.current_stream(dev)
    for g in graphs + two + asm_graphs + split + sep:
        g.replay()
    ms = _timed(lambda i: graphs[i % 2].replay(), steps, stream)
    ms_two = _timed(lambda i: two[i % 2].replay(), steps, stream)
    ms_asm = _timed(lambda i: asm_graphs[i % 2].replay(), steps, stream)
    ms_split = _timed(lambda i: split[i % 2].replay(), steps, stream)
    ms_sep = _timed(lambda i: sep[i % 2].replay(), steps, stream)
    for w in wls:  # the selection state of the one-stream step again
        w.step()
    ms_eager = _timed(lambda i: wls[i % 2].step(), steps, stream)
    gd_ms = _timed(lambda i: wls[i % 2].gather_dropped(), steps, stream)
    for w in wls:  # the selection state of the one-stream step again
        w.step()
    gk_ms = _timed(lambda i: wls[i % 2].gather_kept(), steps, stream)
    n_asm = N_LAYERS - 2
    asm_ms = _timed(lambda i: wls[(i // n_asm) % 2].assemble(2 + i % n_asm), steps * n_asm, stream)
    ms_unc = _uncorrelated_steps(wls, steps, stream, dev)
    assert all(int(w.err.item()) == 0 for w in wls)
    plan = wls[0].plan
    n_keep = plan.n_keep
    assert int(wls[0].sel.counts[0].item()) == n_keep
    nbytes = repair_bytes(n_keep)
    gd_bytes = dropped_bytes(plan)
    gk_bytes = merged_bytes(plan)
    ms_conc = _concurrent_steps(wls, steps, dev)
    return dict(ms_per_step=ms, ms_two=ms_two, ms_asm=ms_asm, ms_split=ms_split, ms_sep=ms_sep, ms_eager=ms_eager,
                ms_unc=ms_unc,
                bytes=nbytes,
                moved=moved_bytes(plan),
                gbs=nbytes / (ms * 1e-3) / 1e9, gd_ms=gd_ms, gd_bytes=gd_bytes, gd_gbs=gd_bytes / (gd_ms * 1e-3) / 1e9,
                gk_ms=gk_ms, gk_bytes=gk_bytes, gk_gbs=gk_bytes / (gk_ms * 1e-3) / 1e9,
                asm_ms=asm_ms, asm_gbs=ASSEMBLE_BYTES / (asm_ms * 1e-3) / 1e9, n_keep=n_keep, ms_conc=ms_conc,
                conc_gbs=CONCURRENT * nbytes / (ms_conc * 1e-3) / 1e9)


CONCURRENT = 4  # requests in flight for the serving-loop variant of the step


def _concurrent_steps(wls, steps: int, dev) -> float:
    """ms per round of CONCURRENT requests' KV repairs, each request's launches on its own stream
    (one stream per request, as a server with concurrent requests issues them), replayed from a
    HIP graph. The single request's step is a chain of dependent launches, most of them too small
    to fill the GPU; independent requests overlap each other's latency."""
    reqs = list(wls) + [RepairWorkload(1234 + len(wls) + i, dev) for i in range(CONCURRENT - len(wls))]
    streams = request_streams(len(reqs), dev)

    def round_():
        main = torch.cuda.current_stream(dev)
        for w, st in zip(reqs, streams):
            st.wait_stream(main)
            with torch.cuda.stream(st):
                w.step()
        for st in streams:
            main.wait_stream(st)

    round_()
    torch.cuda.synchronize()
    g = _graph_of(round_)
    g.replay()
    ms = _timed(lambda i: g.replay(), steps, torch.cuda.current_stream(dev))
    assert all(int(w.err.item()) == 0 for w in reqs)
    for w in wls:  # leave the step's selection state as it was
        w.step()
    torch.cuda.synchronize()
    return ms


def _uncorrelated_steps(wls, steps: int, stream, dev) -> float:
    """ms per step with layer-1 fresh rows that do not follow the cached ones (random rows: every
    deviation within a few percent of the others, so most candidates share a few bins of the
    selection's histogram, its worst case); the workloads' own rows are put back after."""
    gen = torch.Generator(device=dev).manual_seed(99)
    saved = [w.fresh[1] for w in wls]
    for w in wls:
        k1 = w.fresh[1][0]
        ku = torch.randn(k1.shape, generator=gen, device=dev).to(k1.dtype)
        vu = torch.randn(k1.shape, generator=gen, device=dev).to(k1.dtype).transpose(1, 2).contiguous().transpose(1, 2)
        w.fresh[1] = (ku, vu)
        w.step()
    torch.cuda.synchronize()
    graphs = [_graph_of(w.step) for w in wls]
    for g in graphs:
        g.replay()
    ms = _timed(lambda i: graphs[i % 2].replay(), steps, stream)
    assert all(int(w.err.item()) == 0 and int(w.sel.counts[0].item()) == w.plan.n_keep for w in wls)
    for w, f in zip(wls, saved):
        w.fresh[1] = f
        w.step()
    torch.cuda.synchronize()
    return ms


def dropped_bytes(plan) -> int:
    """Algorithmic bytes of the gather of the dropped rows of layers 2..27: every cached row whose
    position the selection did not keep, K and V, read + write."""
    n_uncached = plan.n_tokens - int(plan.cached.sum())
    n_dropped = int(plan.cached.sum()) - (plan.n_keep - n_uncached)
    return (N_LAYERS - 2) * n_dropped * ROW_BYTES * 4


def merged_bytes(plan) -> int:
    """Algorithmic bytes of the step's last KV-repair launch: layer 1's kept rows (fresh rows read,
    cache rows written) and the dropped cached rows of the layers after those gathered whole, K
    and V, read + write."""
    n_uncached = plan.n_tokens - int(plan.cached.sum())
    n_dropped = int(plan.cached.sum()) - (plan.n_keep - n_uncached)
    return (N_LAYERS - 2 - whole_layers(plan)) * n_dropped * ROW_BYTES * 4 + plan.n_keep * ROW_BYTES * 4


def whole_layers(plan) -> int:
    """Layers of 2..27 that ckv_layer1_repair_gather gathers whole beside its selection (kept
    cached rows included, overwritten by the fresh rows after)."""
    from chunkkv_amd import ops

    return ops.layer1_repair_gather_whole_layers(plan.n_tokens, len(plan.spans), None, len(plan.segments),
                                                 plan.max_seg_tokens, (2, N_LAYERS), N_KV, HEAD_DIM, torch.bfloat16)


def moved_bytes(plan) -> int:
    """Algorithmic bytes of the step as HipEngine runs it: each assembled layer reads and writes
    every row once, and the layers gathered whole beside the selection their kept cached rows
    once more; layer 1 reads and writes its cached rows (base cache), then the deviation and
    the scatter of the kept rows."""
    row = ROW_BYTES * 4  # K and V, read + write
    n_cached = int(plan.cached.sum())
    kept_cached = plan.n_keep - (plan.n_tokens - n_cached)
    return ((N_LAYERS - 1) * plan.n_tokens * row + n_cached * row + DEVIATION_BYTES + plan.n_keep * row
            + whole_layers(plan) * kept_cached * row)


ASSEMBLE_BYTES = N_TOKENS * ROW_BYTES * 4  # one assembled layer: 8256 rows of K and V, read + write


def random_qwen25_7b(dev):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    cfg = Qwen2Config(vocab_size=152064, hidden_size=3584, intermediate_size=18944, num_hidden_layers=N_LAYERS,
                      num_attention_heads=28, num_key_value_heads=N_KV, max_position_embeddings=32768,
                      rope_theta=THETA, tie_word_embeddings=False, rms_norm_eps=1e-6)
    torch.manual_seed(0)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(dev):
            model = Qwen2ForCausalLM(cfg)
    finally:
        torch.set_default_dtype(prev)
    return model.eval()


class _Tok:
    eos_token_id = 151645


def bench_ttft(n_requests: int, dev, model=None, n_reference_attention: int = 20) -> dict:
    """TTFT p50 of HipEngine vs the reference op sequence on the same seeded requests; of HipEngine
    with torch's fused SDPA kernels and torch's norm/MLP (attention="sdpa": the KV repair alone on
    the HIP kernels) on all of them; and of HipEngine with the reference's own SDPA call
    (attention="reference", its fp32 math path) on the first n_reference_attention of them. All
    run the model's library GEMMs with the same committed TunableOp selection table (when
    present)."""
    from chunkkv_amd.baseline import TorchOpsEngine
    from chunkkv_amd.engine import HipEngine
    from chunkkv_amd.types import BlendConfig

    if model is None:
        t = time.perf_counter()
        model = random_qwen25_7b(dev)
        log(f"[bench] random-init Qwen2.5-7B architecture ready in {time.perf_counter() - t:.1f}s")
    tuned = use_tuned_gemms()
    log(f"[bench] library GEMMs: {'tuned table (TunableOp, lookup only)' if tuned else 'default heuristics'} "
        "for all engines")
    hip, ref = HipEngine(model, _Tok()), TorchOpsEngine(model, _Tok())
    hip_ref_attn = HipEngine(model, _Tok(), attention="reference")
    hip_sdpa = HipEngine(model, _Tok(), attention="sdpa")
    hip_overlap = HipEngine(model, _Tok(), overlap=True)
    gen = torch.Generator().manual_seed(7)
    vocab = model.config.vocab_size
    # Chunk pool: each chunk prefilled alone at position 0 (its own context), stored like KVStore does.
    pool = []
    for _ in range(2 * N_CHUNKS):
        toks = torch.randint(0, vocab, (CHUNK_LEN,), generator=gen).tolist()
        res = hip.prefill(toks)
        pool.append((toks, res.chunk(0, CHUNK_LEN)))
        del res
    reqs = []
    for _ in range(n_requests + 2):
        pick = torch.randperm(len(pool), generator=gen)[:N_CHUNKS].tolist()
        tokens, placements = [], []
        for c in pick:
            placements.append(Place(pool[c][1], len(tokens)))
            tokens += pool[c][0]
        tokens += torch.randint(0, vocab, (TAIL + QUERY,), generator=gen).tolist()
        reqs.append((tokens, placements))
    cfg = BlendConfig(recompute_ratio=RATIO, n_sink=N_SINK)
    out = {}
    for name, eng, n_req in (("hip", hip, len(reqs)), ("torch_ops", ref, len(reqs)),
                              ("hip_attention_reference", hip_ref_attn, min(len(reqs), n_reference_attention + 2)),
                              ("hip_torch_attention", hip_sdpa, len(reqs)),
                              ("hip_overlap", hip_overlap, min(len(reqs), n_reference_attention + 2))):
        times, stats = [], None
        for i, (tokens, placements) in enumerate(reqs[:n_req]):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            res = eng.prefill(tokens, placements, cfg)
            eng.last_logprobs(res)
            dt = time.perf_counter() - t0
            if i >= 2:
                times.append(dt * 1e3)
            stats = res.stats
            del res
        out[name] = dict(p50=float(np.percentile(times, 50)), p99=float(np.percentile(times, 99)), stats=stats,
                         tuned_gemms=tuned, requests=len(times))
        log(f"[bench] TTFT {name}: p50 {out[name]['p50']:.2f} ms  p99 {out[name]['p99']:.2f} ms")
    del hip, ref, hip_ref_attn, hip_sdpa, hip_overlap
    torch.cuda.empty_cache()
    out["model"] = model
    return out


def bench_cpu(seconds: float) -> dict:
    """The reference's KV-repair op sequence on the host's cores, bounded to ~`seconds`."""
    from types import SimpleNamespace as NS

    from oracle import engine_ref as R

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(99)
    inv = R.reference_inv_freq(THETA, HEAD_DIM)
    chunks = [NS(keys=[torch.randn((1, N_KV, CHUNK_LEN, HEAD_DIM), generator=gen).bfloat16() for _ in range(N_LAYERS)],
                 values=[torch.randn((1, N_KV, CHUNK_LEN, HEAD_DIM), generator=gen).bfloat16() for _ in range(N_LAYERS)],
                 start=int(torch.randint(0, 8192, (1,), generator=gen))) for _ in range(N_CHUNKS)]
    order = torch.randperm(N_CHUNKS, generator=gen).tolist()
    pl = [NS(chunk=chunks[c], start=i * CHUNK_LEN, ratio=None, exact=False) for i, c in enumerate(order)]
    cfg = NS(recompute_ratio=RATIO, n_sink=N_SINK, full_first_layer=True, escalate_threshold=None)
    cached_l, _, sink_l = R.plan_positions(N_TOKENS, pl, N_SINK)
    cached, sink = torch.tensor(cached_l), torch.tensor(sink_l)
    layer0 = torch.arange(N_TOKENS)
    fk = [torch.randn((1, N_KV, N_TOKENS if l < 2 else 2976, HEAD_DIM), generator=gen).bfloat16() for l in range(N_LAYERS)]
    fv = [torch.randn((1, N_KV, N_TOKENS if l < 2 else 2976, HEAD_DIM), generator=gen).bfloat16() for l in range(N_LAYERS)]
    R.repair_step(pl, fk, fv, N_TOKENS, N_KV, HEAD_DIM, torch.bfloat16, inv, cfg, layer0, cached, sink)  # warm-up
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        keep = R.repair_step(pl, fk, fv, N_TOKENS, N_KV, HEAD_DIM, torch.bfloat16, inv, cfg, layer0, cached, sink)
        times.append(time.perf_counter() - t0)
    assert len(keep) == 2976
    med = float(np.median(times))
    return dict(value=repair_bytes(2976) / med / 1e9, unit="GB/s", cores=threads, kind="port", cpu_model=_cpu_model(),
                sample=f"{len(times)} requests of the same workload (one request = 28-layer base_kv + layer-1 "
                       f"deviation/selection + 28 scatters), torch {torch.__version__} CPU eager, median "
                       f"{med * 1e3:.0f} ms/request")


def _workload_line(metric: str, value: float, ms: float, steps: int, warmup: int, config: dict, roofline: dict) -> dict:
    return {
        "metric": metric, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic", "config": config, "pct_of_peak": round(100.0 * value / PEAK_GBS, 2), "roofline": roofline,
    }


def _rooffor(kernel: str, nbytes: int, ms: float) -> dict:
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"kernel": kernel, "bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / PEAK_GBS, 4), "traffic": None, "bytes_per_launch": nbytes, "avg_launch_us": round(ms * 1e3, 2)}


def bench_gather_only(steps: int, warmup: int, dev) -> dict:
    """Re-RoPE + gather microbenchmark at the Qwen2.5-7B KV shape: 28 layers, 4 heads, D=128,
    bf16, 16 chunks x 256 tokens (keys rotated at their original offsets), delta ~ U[-4096, 4096],
    gathered into a 4096-token cache. Bytes per launch = 28 x 4096 x 4 x 1024 = 469,762,048."""
    from chunkkv_amd import ops
    from chunkkv_amd.planner import plan_request

    L, C, N = 256, 16, 4096
    sets = []
    for seed in range(3):  # 3 x (235 MB chunks + 235 MB cache) rotates past the 256 MB MALL
        gen = torch.Generator().manual_seed(seed)
        inv = ops.inv_freq(HEAD_DIM, THETA, dev)
        slots = torch.randperm(C, generator=gen).tolist()
        deltas = torch.randint(-4096, 4097, (C,), generator=gen).tolist()
        pl = []
        for c in range(C):
            orig = slots[c] * L - deltas[c]
            x = torch.randn((N_LAYERS, 1, N_KV, L, HEAD_DIM), generator=gen).to(dev)
            k = rope_rows(x, torch.arange(orig, orig + L, device=dev), inv).to(torch.bfloat16)
            v = torch.randn((N_LAYERS, 1, N_KV, L, HEAD_DIM), generator=gen).to(dev).to(torch.bfloat16)
            pl.append(Place(Chunk(k, v, orig), slots[c] * L))
        plan = plan_request(N, pl, N_SINK, RATIO)
        tab = np.concatenate([np.array([[k.data_ptr(), v.data_ptr()] for k, v in zip(ch.keys, ch.values)],
                                       dtype=np.uint64).reshape(-1) for ch in plan.chunks])
        K = torch.empty((N_LAYERS, 1, N_KV, N, HEAD_DIM), dtype=torch.bfloat16, device=dev)
        sets.append((pl, plan, torch.from_numpy(tab.view(np.int64)).to(dev), torch.from_numpy(plan.segments.reshape(-1)).to(dev),
                     K, torch.empty_like(K)))

    def launch(i):
        _, plan, tab, segs, K, V = sets[i % 3]
        ops.rerope_gather(K, V, tab, segs, len(plan.segments), plan.max_seg_tokens, THETA)

    for i in range(warmup):
        launch(i)
    ms = _timed(launch, steps, torch.cuda.current_stream(dev))
    nbytes = N_LAYERS * C * L * ROW_BYTES * 4
    return _workload_line(
        "re-RoPE + gather HBM GB/s, Qwen2.5-7B KV shape", nbytes / (ms * 1e-3) / 1e9, ms, steps, warmup,
        {"workload": "re-RoPE + gather: 28 layers, 4 KV heads, head_dim 128, bf16, 16 chunks x 256 tokens, "
                     "delta ~ U[-4096, 4096], 4096-token cache", "bytes_per_step": nbytes},
        _rooffor("rerope_gather_kernel<bf16,128>", nbytes, ms))


DEV_SETS = 16  # config-3 input sets rotated per graph replay: 16 x 50 MB > 512 MB, past the 256 MB MALL


def bench_deviation_topk(steps: int, warmup: int, dev) -> dict:
    """Deviation + pooled top-k + scatter microbenchmark: layer-1 fresh vs cached K/V for 32 chunks
    x 256 tokens (8192), 4 heads x 128, bf16; cached = fresh + sigma_c N(0,1), sigma_c ~
    lognormal(-3, 1); pooled top-k at 15/30/50% plus 4 sinks per chunk (ckv_deviation_select: the
    deviation counting the candidate histogram, then the selection starting from it), then the
    kept rows compacted and scattered into the layer's cache (ckv_scatter_kept_rows). Also timed:
    the deviation alone (ckv_deviation, the HBM-bound launch: the roofline) and the deviation and
    selection without the histogram (ckv_deviation + ckv_select). DEV_SETS independent input sets
    (33.6 MB of K/V read and the kept rows written per set, ~800 MB in all) are cycled through
    inside each graph replay, so every launch reads HBM rather than the 256 MB MALL."""
    from chunkkv_amd import ops
    from chunkkv_amd.planner import local_index, plan_request

    N, C, L = 8192, 32, 256
    g = torch.Generator(device=dev).manual_seed(3)
    sets = []
    for _ in range(DEV_SETS):
        fk = torch.randn((1, N_KV, N, HEAD_DIM), generator=g, device=dev)
        fv = torch.randn((1, N_KV, N, HEAD_DIM), generator=g, device=dev)
        sigma = torch.exp(torch.randn(C, generator=g, device=dev) - 3.0).repeat_interleave(L)[None, None, :, None]
        K = (fk + sigma * torch.randn(fk.shape, generator=g, device=dev)).bfloat16()
        V = (fv + sigma * torch.randn(fv.shape, generator=g, device=dev)).bfloat16()
        v = fv.bfloat16().transpose(1, 2).contiguous().transpose(1, 2)  # token-major, as v_proj leaves it
        sets.append(dict(k=fk.bfloat16(), v=v, K=K, V=V, Kd=torch.empty_like(K), Vd=torch.empty_like(V),
                         ws=ops.deviation_select_workspace(dev)))
    pl = [Place(Chunk(torch.empty((1, 1, N_KV, L, HEAD_DIM)), torch.empty((1, 1, N_KV, L, HEAD_DIM)), 0), c * L)
          for c in range(C)]
    out = {}
    stream = torch.cuda.current_stream(dev)
    for ratio in (0.15, 0.30, 0.50):
        plan = plan_request(N, pl, N_SINK, ratio)
        n = plan.n_keep
        flags = torch.from_numpy(plan.flags).to(dev)
        local = torch.from_numpy(local_index(N, plan.layer0_idx)).to(dev)
        spans = torch.from_numpy(plan.spans.reshape(-1)).to(dev)
        sels = [None] * DEV_SETS
        dns = [(torch.empty(N, device=dev), torch.empty(N, device=dev)) for _ in range(DEV_SETS)]

        def dev_sel(i):  # ckv_deviation_select: deviation + histogram, selection from the histogram
            st = sets[i]
            sels[i] = ops.deviation_select(st["k"], st["v"], st["K"], st["V"], flags, local, spans, None, st["ws"],
                                           out=sels[i], diff_norm=dns[i])[2]

        def dev_only(i):  # the deviation launch alone (ckv_deviation)
            st = sets[i]
            ops.deviation(st["k"], st["v"], st["K"], st["V"], flags, local)

        def dev_then_sel(i):  # without the histogram: ckv_deviation + ckv_select
            st = sets[i]
            d_, n_ = ops.deviation(st["k"], st["v"], st["K"], st["V"], flags, local)
            sels[i] = ops.select(d_, n_, flags, local, spans, None, sels[i])

        def scat(i):
            st = sets[i]
            ops.scatter_kept_rows(st["Kd"], st["Vd"], st["k"], st["v"], sels[i].keep_abs[:n], sels[i].keep_local[:n])

        for i in range(DEV_SETS):
            dev_sel(i)
            scat(i)
        # one graph = every input set once (DEV_SETS launches back to back: a replay's own launch
        # cost is spread over them; what remains per launch is the kernel's time and its gaps)
        g_dev = _graph_of(lambda: [dev_sel(i) for i in range(DEV_SETS)])
        # counts[7] bit 0: the counted histogram started the selection (bit 1 says whether its
        # threshold bin was ranked directly, which depends on the ratio)
        assert all(int(sl.counts[0].item()) == n and int(sl.counts[7].item()) & 1 == 1 for sl in sels)
        g_only = _graph_of(lambda: [dev_only(i) for i in range(DEV_SETS)])
        g_two = _graph_of(lambda: [dev_then_sel(i) for i in range(DEV_SETS)])
        g_sc = _graph_of(lambda: [scat(i) for i in range(DEV_SETS)])
        g_both = _graph_of(lambda: [(dev_sel(i), scat(i)) for i in range(DEV_SETS)])
        t_dev = _timed(lambda i: g_dev.replay(), steps, stream) / DEV_SETS
        t_only = _timed(lambda i: g_only.replay(), steps, stream) / DEV_SETS
        t_two = _timed(lambda i: g_two.replay(), steps, stream) / DEV_SETS
        t_sc = _timed(lambda i: g_sc.replay(), steps, stream) / DEV_SETS
        t_both = _timed(lambda i: g_both.replay(), steps, stream) / DEV_SETS
        assert all(int(sl.counts[0].item()) == n for sl in sels)
        out[ratio] = dict(n_keep=n, dev_sel_ms=t_dev, deviation_ms=t_only, dev_sel_without_histogram_ms=t_two,
                          scatter_ms=t_sc, both_ms=t_both, scatter_bytes=n * ROW_BYTES * 4)
    dev_bytes = N * 4 * ROW_BYTES + N * 8
    r30 = out[0.30]
    nb = dev_bytes + r30["scatter_bytes"]
    line = _workload_line(
        "deviation + pooled top-k + scatter HBM GB/s, Qwen2.5-7B KV shape", nb / (r30["both_ms"] * 1e-3) / 1e9,
        r30["both_ms"], steps, warmup,
        {"workload": "layer-1 deviation + pooled top-k (30%) + 4 sinks x 32 chunks x 256 + scatter of the kept rows, "
                     "4 KV heads, head_dim 128, bf16; 16 input sets rotated (cold HBM); ckv_deviation_select (the "
                     "deviation counting the candidate histogram, the selection starting from it: two launches) "
                     "then ckv_scatter_kept_rows; the deviation alone and the two calls without the histogram are "
                     "in ratios", "bytes_per_step": nb},
        _rooffor("deviation_kernel<bf16> (the HBM-bound launch; the selection moves 74 KB)", dev_bytes,
                 r30["deviation_ms"]))
    line["ratios"] = {str(r): {k2: (round(v2, 5) if isinstance(v2, float) else v2) for k2, v2 in o.items()}
                      for r, o in out.items()}
    return line


# Four HipEngine prefills in flight, one host thread each (bench_replay's concurrent TTFT), stopped
# making progress in two of three runs on the GPU (no output for 3 minutes, the run killed) after
# completing in the others at 448-520 ms p50. No kernel of this library waits for another
# workgroup or launch, and no host path of the engine waits across streams without overlap, so the
# stall lies in what the four threads share (the library GEMMs' kernels and the HIP runtime); its
# cause is not found. The measurement runs only when asked for (--concurrent-ttft).
CONCURRENT_TTFT_NOTE = ("4 concurrent 32k prefills (one host thread each) not measured by default: runs of it "
                        "stalled with no progress on the GPU, cause not found; --concurrent-ttft runs it")


def bench_replay(steps: int, warmup: int, dev, n_streams: int = 4, ttft_requests: int = 6, model=None,
                 concurrent_ttft: bool = False) -> dict:
    """Long-context multi-request replay at the Qwen2.5-7B shape: an HBM-resident store of 256
    chunks x 256 tokens x 2 context variants (7.0 GiB); 4 concurrent requests of 128 chunks
    sampled with replacement (Zipf s=1.1) at random order + a 64-token query (32832 tokens), 15%
    recompute + 4 sinks. Each request's KV repair is the engine's launch sequence (layer 0's fresh
    rows; layer 1's repair with the base cache of layers 2-27 as one ckv_layer1_repair_gather call:
    base cache with the deviation, the selection, the kept rows with the gather of the dropped rows
    of layers 2-27; the fresh rows of layers 2-27) on its own HIP stream, with a layer-1 workspace
    and an error flag per request (asserted zero). The rounds are timed with layer-1 rows that
    follow the cached ones (per-chunk noise) and again with uncorrelated random rows (the
    selection's hardest input). Then TTFT p50/p99 of HipEngine.prefill + last_logprobs on requests
    of the same shape (random-init Qwen2.5-7B architecture, bf16; the store's K/V serve as the
    cached chunks), one at a time, and with concurrent_ttft also with 4 requests in flight, each
    from its own host thread (off by default: see CONCURRENT_TTFT_NOTE)."""
    from chunkkv_amd import ops
    from chunkkv_amd.planner import local_index, plan_request

    L, POOL, VARIANTS, PER_REQ, Q = 256, 256, 2, 128, 64
    N = PER_REQ * L + Q
    gen = torch.Generator(device=dev).manual_seed(11)
    store = []
    for _ in range(POOL * VARIANTS):
        k = torch.randn((N_LAYERS, 1, N_KV, L, HEAD_DIM), generator=gen, device=dev).to(torch.bfloat16)
        v = torch.randn((N_LAYERS, 1, N_KV, L, HEAD_DIM), generator=gen, device=dev).to(torch.bfloat16)
        store.append(Chunk(k, v, int(torch.randint(0, 32768, (1,), generator=gen, device=dev).item())))
    log(f"[bench] replay: store of {len(store)} chunks built")
    zipf = 1.0 / np.arange(1, POOL + 1) ** 1.1
    zipf /= zipf.sum()
    rng = np.random.default_rng(11)
    row = N_KV * HEAD_DIM
    reqs, placements_of = [], []
    for r in range(2 * n_streams):
        ids = rng.choice(POOL, PER_REQ, p=zipf) * VARIANTS + rng.integers(0, VARIANTS, PER_REQ)
        pl = [Place(store[i], j * L) for j, i in enumerate(ids)]
        placements_of.append(pl)
        plan = plan_request(N, pl, N_SINK, 0.15)
        tab = np.concatenate([np.array([[k.data_ptr(), v.data_ptr()] for k, v in zip(ch.keys, ch.values)],
                                       dtype=np.uint64).reshape(-1) for ch in plan.chunks])
        K = torch.empty((N_LAYERS, 1, N_KV, N, HEAD_DIM), dtype=torch.bfloat16, device=dev)
        V = torch.empty_like(K)
        tab_d = torch.from_numpy(tab.view(np.int64)).to(dev)
        segs_d = torch.from_numpy(plan.segments.reshape(-1)).to(dev)
        proj = [None if li == 1 else (torch.randn((1, N if li == 0 else plan.n_keep, row), device=dev).bfloat16(),
                                      torch.randn((1, N if li == 0 else plan.n_keep, row), device=dev).bfloat16())
                for li in range(N_LAYERS)]
        # layer-1 fresh rows as the 8k request builds them: each cached position's re-rotated cached
        # row plus noise at a per-chunk level exp(N(-3, 1)), the uncached query rows random, v
        # token-major (uncorrelated random rows put every deviation within a few percent of the
        # others: the selection's slowest case, measured separately)
        ops.rerope_gather(K, V, tab_d, segs_d, len(plan.segments), plan.max_seg_tokens, THETA, layers=(1, 2))
        sig = torch.ones(N, device=dev)
        sig[: PER_REQ * L] = torch.exp(torch.randn(PER_REQ, generator=gen, device=dev) - 3.0).repeat_interleave(L)
        sig = sig[None, None, :, None]
        cached = torch.from_numpy(plan.cached).to(dev)[None, None, :, None]
        rnd = lambda: torch.randn((1, N_KV, N, HEAD_DIM), generator=gen, device=dev)  # noqa: E731
        k1 = torch.where(cached, K[1].float() + sig * rnd(), rnd()).bfloat16()
        v1 = torch.where(cached, V[1].float() + sig * rnd(), rnd()).bfloat16().transpose(1, 2).contiguous()
        reqs.append(dict(plan=plan, tab=tab_d, segs=segs_d, K=K, V=V,
                         flags=torch.from_numpy(plan.flags).to(dev),
                         local=torch.from_numpy(local_index(N, plan.layer0_idx)).to(dev),
                         spans=torch.from_numpy(plan.spans.reshape(-1)).to(dev),
                         layer0=torch.from_numpy(plan.layer0_idx.astype(np.int64)).to(dev), proj=proj,
                         fresh1=(k1, v1.transpose(1, 2)), sel=None,
                         err=torch.zeros(1, dtype=torch.int32, device=dev),
                         ws=ops.layer1_repair_workspace(dev),
                         dn=(torch.empty(N, dtype=torch.float32, device=dev),
                             torch.empty(N, dtype=torch.float32, device=dev))))
    assert reqs[0]["plan"].budget == 4864
    log(f"[bench] replay: {len(reqs)} requests planned")
    streams = request_streams(n_streams, dev)

    def repair(rq):
        """The request's KV repair as HipEngine issues it: layer 0's fresh rows; layer 1's repair
        with the base cache of layers 2-27 (ckv_layer1_repair_gather); layers 2-27's fresh rows."""
        plan, err = rq["plan"], rq["err"]
        K, V = rq["K"].unbind(0), rq["V"].unbind(0)
        nseg, mseg = len(plan.segments), plan.max_seg_tokens
        ops.rope_qkv(None, *rq["proj"][0], rq["layer0"], 0, N_KV, HEAD_DIM, THETA, k_out=K[0], v_out=V[0],
                     rows=rq["layer0"], err=err)
        k1, v1 = rq["fresh1"]
        _, _, rq["sel"] = ops.layer1_repair_gather(rq["K"], rq["V"], rq["tab"], 1, (2, N_LAYERS), rq["segs"], nseg,
                                                   mseg, k1, v1, rq["flags"], rq["local"], rq["spans"], None, THETA,
                                                   rq["ws"], err, rq["sel"], rq["dn"])
        rows = rq["sel"].keep_abs[: plan.n_keep]
        for li in range(2, N_LAYERS):
            ops.rope_qkv(None, *rq["proj"][li], rows, 0, N_KV, HEAD_DIM, THETA, k_out=K[li], v_out=V[li], rows=rows,
                         err=err)

    def round_(i):
        base = (i % 2) * n_streams
        for s_i, s in enumerate(streams):
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                repair(reqs[base + s_i])
        for s in streams:
            torch.cuda.current_stream().wait_stream(s)

    for i in range(max(warmup, 2)):
        round_(i)
    torch.cuda.synchronize()
    ms_eager = _timed(round_, steps, torch.cuda.current_stream(dev))
    # the same rounds replayed from HIP graphs (one per input set), as a serving loop would issue them
    graphs = [_graph_of(lambda i=i: round_(i)) for i in range(2)]
    for g in graphs:
        g.replay()
    ms = _timed(lambda i: graphs[i % 2].replay(), steps, torch.cuda.current_stream(dev))
    log(f"[bench] replay: rounds {ms:.3f} ms (graphs), {ms_eager:.3f} ms (eager)")
    per_req = sum(repair_bytes_for(rq["plan"]) for rq in reqs[:n_streams]) / n_streams
    nbytes = per_req * n_streams
    assert all(int(rq["sel"].counts[0].item()) == rq["plan"].n_keep for rq in reqs)
    assert all(int(rq["err"].item()) == 0 for rq in reqs)
    # The same rounds with uncorrelated layer-1 rows (every fresh row random): every candidate's
    # deviation lies within a few percent of the others, the selection's hardest input.
    for rq in reqs:
        k1 = torch.randn((1, N_KV, N, HEAD_DIM), generator=gen, device=dev).bfloat16()
        v1 = torch.randn((1, N_KV, N, HEAD_DIM), generator=gen, device=dev).bfloat16().transpose(1, 2).contiguous()
        rq["fresh1"] = (k1, v1.transpose(1, 2))
    for i in range(2):
        round_(i)
    graphs_u = [_graph_of(lambda i=i: round_(i)) for i in range(2)]
    for g in graphs_u:
        g.replay()
    ms_uncorr = _timed(lambda i: graphs_u[i % 2].replay(), steps, torch.cuda.current_stream(dev))
    log(f"[bench] replay: rounds with uncorrelated layer-1 rows {ms_uncorr:.3f} ms")
    assert all(int(rq["sel"].counts[0].item()) == rq["plan"].n_keep for rq in reqs)
    assert all(int(rq["err"].item()) == 0 for rq in reqs)
    line = _workload_line(
        "aggregate KV-repair HBM GB/s, 4 concurrent 32k-token requests, Qwen2.5-7B KV shape", nbytes / (ms * 1e-3) / 1e9,
        ms, steps, warmup,
        {"workload": "replay: store 256 chunks x 256 tokens x 2 variants (7.0 GiB HBM); 4 requests x (128 Zipf(1.1) "
                     "chunks + 64-token query) = 32832 tokens each, 15% + 4 sinks, one HIP stream per request",
         "bytes_per_step": int(nbytes), "requests_per_step": n_streams},
        None)
    line["store_gib"] = round(len(store) * N_LAYERS * 2 * N_KV * L * HEAD_DIM * 2 / 2**30, 2)
    line["ms_per_step_eager"] = round(ms_eager, 4)
    line["ms_per_step_uncorrelated"] = round(ms_uncorr, 4)
    line["uncorrelated_over_correlated"] = round(ms_uncorr / ms, 4)
    for rq in reqs:  # free the repair buffers before the model comes in
        rq.clear()
    del reqs, graphs, graphs_u
    torch.cuda.empty_cache()
    if ttft_requests > 0:
        from chunkkv_amd.engine import HipEngine
        from chunkkv_amd.types import BlendConfig

        own_model = model is None
        if own_model:
            model = random_qwen25_7b(dev)
        use_tuned_gemms()
        hip = HipEngine(model, _Tok())
        cfg = BlendConfig(recompute_ratio=0.15, n_sink=N_SINK)
        vocab = model.config.vocab_size
        times = []
        for i in range(ttft_requests + 1):
            tokens = torch.randint(0, vocab, (N,), generator=torch.Generator().manual_seed(100 + i)).tolist()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            res = hip.prefill(tokens, placements_of[i % len(placements_of)], cfg)
            hip.last_logprobs(res)
            dt = time.perf_counter() - t0
            if i:
                times.append(dt * 1e3)
            del res
        line["ttft_p50_ms"] = round(float(np.percentile(times, 50)), 2)
        line["ttft_p99_ms"] = round(float(np.percentile(times, 99)), 2)
        line["ttft_requests"] = len(times)
        log(f"[bench] replay: TTFT of one 32k request p50 {line['ttft_p50_ms']} ms")
        line["ttft_note"] = ("HipEngine; ttft_p50_ms / ttft_p99_ms one request at a time; the reference op "
                             "sequence is not timed at 32k (its math-path SDPA would hold ~120 GB of fp32 scores "
                             "per layer)")
        if concurrent_ttft:
            conc = _concurrent_ttft(model, cfg, placements_of, n_streams, max(ttft_requests, 20), N, vocab, dev)
            line["ttft_p50_ms_concurrent"] = round(float(np.percentile(conc, 50)), 2)
            line["ttft_p99_ms_concurrent"] = round(float(np.percentile(conc, 99)), 2)
            line["ttft_requests_concurrent"] = len(conc)
            line["ttft_note"] += (f"; *_concurrent with {n_streams} requests in flight (one host thread, HipEngine "
                                  "and HIP stream per request, each request's prefill + last_logprobs timed from "
                                  "the round's start)")
        else:
            line["ttft_concurrent_note"] = CONCURRENT_TTFT_NOTE
        del hip
        if own_model:
            del model
        torch.cuda.empty_cache()
    return line


def _concurrent_ttft(model, cfg, placements_of, n_streams: int, rounds: int, N: int, vocab: int, dev) -> list:
    """TTFT (ms) of `rounds` rounds of n_streams concurrent HipEngine prefills + last_logprobs, one
    host thread, engine (weights shared) and request stream per request; a round's requests start
    together (a barrier) and each is timed from the round's start to its own logprobs. One warm-up
    round first. Run only with --concurrent-ttft (CONCURRENT_TTFT_NOTE)."""
    import threading

    from chunkkv_amd.engine import HipEngine

    streams = request_streams(n_streams, dev)
    engines = [HipEngine(model, _Tok()) for _ in range(n_streams)]
    times: list[float] = []
    errors: list[BaseException] = []
    for rnd in range(rounds + 1):
        toks = [torch.randint(0, vocab, (N,), generator=torch.Generator().manual_seed(1000 + rnd * n_streams + j)).tolist()
                for j in range(n_streams)]
        start = threading.Barrier(n_streams + 1)
        t0 = [0.0]
        out = [0.0] * n_streams

        def run(j):
            try:
                torch.cuda.set_device(dev)
                with torch.cuda.stream(streams[j]):
                    start.wait()
                    res = engines[j].prefill(toks[j], placements_of[(rnd * n_streams + j) % len(placements_of)], cfg)
                    engines[j].last_logprobs(res)
                    out[j] = (time.perf_counter() - t0[0]) * 1e3
                    del res
            except BaseException as e:  # reported below, after every thread ended
                errors.append(e)
                start.abort()

        threads = [threading.Thread(target=run, args=(j,)) for j in range(n_streams)]
        for th in threads:
            th.start()
        torch.cuda.synchronize()
        t0[0] = time.perf_counter()
        try:
            start.wait()
        except threading.BrokenBarrierError:
            pass
        for th in threads:
            th.join()
        if errors:
            raise errors[0]
        if rnd:
            times += out
    del engines
    torch.cuda.synchronize()
    return times


def traffic_probe(steps: int, warmup: int, dev) -> dict:
    """Dispatches for the HBM traffic counters (run under rocprofv3 --pmc): `steps` re-RoPE +
    gather launches of the 8k request alternating two input sets, `steps` request steps (the
    fresh-row writes, the layer-1 deviation, selection and scatter as the step issues them),
    `steps` dropped-row gathers, `steps` of the step's last launch called alone (the roofline
    kernel), then `steps` elementwise kernels that read and write exactly
    COPY_BYTES each, whose FETCH_SIZE / WRITE_SIZE calibrate the counters (a plain D2D copy goes to
    the DMA engine and is not counted)."""
    wls = [RepairWorkload(1234 + i, dev) for i in range(2)]
    for i in range(steps):
        wls[i % 2].gather()
    for i in range(max(steps, 2)):
        wls[i % 2].step()  # also the selection output for the launches below
    torch.cuda.synchronize()
    for i in range(steps):
        wls[i % 2].gather_dropped()
    for i in range(steps):
        wls[i % 2].gather_kept()
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device=dev)
    dst = [torch.empty_like(src) for _ in range(2)]
    for i in range(steps):  # one elementwise kernel: reads and writes exactly COPY_BYTES
        torch.mul(src, 1.0, out=dst[i % 2])
    torch.cuda.synchronize()
    return {"workload": "traffic probe", "gather_launches": steps, "copy_bytes": COPY_BYTES, "copies": steps}


COPY_BYTES = 512 << 20


def bench_extract(steps: int, warmup: int, dev) -> dict:
    """Store-put extraction after the 8k Qwen2.5-7B-shape request: the 24 reusable chunk segments
    (320 tokens each) of all 28 layers' K and V copied out of the request slabs, one
    ckv_extract_chunks launch (the reference: PrefillResult.chunk per segment, 2 x 28 `.contiguous()`
    copies each, timed beside it). Bytes per launch = 24 x 320 x 28 x 2 x 1024 x 2 = 880,803,840."""
    from chunkkv_amd import ops

    gen = torch.Generator().manual_seed(9)
    slabs = [tuple(torch.randn((N_LAYERS, 1, N_KV, N_TOKENS, HEAD_DIM), generator=gen).to(torch.bfloat16).to(dev)
                   for _ in range(2)) for _ in range(2)]
    perm = torch.randperm(N_CHUNKS, generator=gen).tolist()
    spans = [(i * CHUNK_LEN, (i + 1) * CHUNK_LEN) for i in perm]
    stream = torch.cuda.current_stream(dev)
    keep = []

    def ours(i):
        K, V = slabs[i % 2]
        keep.append(ops.extract_chunks(K, V, spans))
        if len(keep) > 2:
            keep.pop(0)

    def reference(i):
        K, V = slabs[i % 2]
        keep.append([[K[l][:, :, s:e].contiguous() for l in range(N_LAYERS)] + [V[l][:, :, s:e].contiguous()
                      for l in range(N_LAYERS)] for s, e in spans])
        if len(keep) > 2:
            keep.pop(0)

    # the kernel alone: fixed destination buffers and descriptors, back-to-back launches
    from chunkkv_amd._native import lib

    fixed = [ops.extract_chunks(K, V, spans) for K, V in slabs]
    desc = []
    for bufs in fixed:
        host = np.zeros(N_CHUNKS * 4, dtype=np.int32)
        host[: 2 * N_CHUNKS].view(np.uint64)[:] = [b.data_ptr() for b in bufs]
        host[2 * N_CHUNKS :] = [v for s_, e_ in spans for v in (s_, e_ - s_)]
        desc.append(torch.from_numpy(host).to(dev))

    def kernel_only(i):
        K, V = slabs[i % 2]
        d = desc[i % 2]
        lib().ckv_extract_chunks(K.data_ptr(), V.data_ptr(), N_KV * N_TOKENS * HEAD_DIM, N_TOKENS * HEAD_DIM,
                                 d.data_ptr(), d.data_ptr() + 8 * N_CHUNKS, N_CHUNKS, CHUNK_LEN, N_LAYERS, N_KV,
                                 N_TOKENS, HEAD_DIM, 1, None, torch.cuda.current_stream(dev).cuda_stream)

    for i in range(max(warmup, 2)):
        ours(i)
        reference(i)
        kernel_only(i)
    ms = _timed(ours, steps, stream)
    ms_ref = _timed(reference, steps, stream)
    ms_k = _timed(kernel_only, steps, stream)
    for (K, V), bufs in zip(slabs, fixed):
        for b, (s_, e_) in zip(bufs, spans):
            assert torch.equal(b[0, 5], K[5][:, :, s_:e_]) and torch.equal(b[1, 27], V[27][:, :, s_:e_])
    nb = N_CHUNKS * CHUNK_LEN * N_LAYERS * 2 * ROW_BYTES * 2
    line = _workload_line(
        "store-put extraction, HBM GB/s", nb / (ms * 1e-3) / 1e9, ms, steps, warmup,
        {"workload": "24 reusable segments x 320 tokens of the 8256-token request, 28 layers, 4 KV heads, "
                     "head_dim 128, bf16, one launch (value: the whole PrefillResult.chunks call, incl. the 24 "
                     "buffer allocations and the descriptor copy)"},
        _rooffor("extract_kernel", nb, ms_k))
    line["reference_per_layer_copies_ms"] = round(ms_ref, 4)
    return line


def bench_decode(steps: int, warmup: int, dev) -> dict:
    """Greedy decode after the 8k blend prefill on a random-init Qwen2.5-7B-architecture bf16
    model: 32 new tokens per request (EOS disabled), HipEngine.generate (preallocated slabs,
    in-place k/v rows, positions-masked attention) vs the reference's torch.cat-per-token decode
    (torch_engine.py:180-198) run on the same engine and prefill. Metric: decode tokens/s."""
    from chunkkv_amd.engine import HipEngine
    from chunkkv_amd.model import DecoderPieces
    from chunkkv_amd.types import BlendConfig

    model = random_qwen25_7b(dev)
    use_tuned_gemms()
    hip = HipEngine(model, _Tok())
    hip.eos = set()
    gen = torch.Generator().manual_seed(11)
    vocab = model.config.vocab_size
    pool = []
    for _ in range(N_CHUNKS):
        toks = torch.randint(0, vocab, (CHUNK_LEN,), generator=gen).tolist()
        pool.append((toks, hip.prefill(toks).chunk(0, CHUNK_LEN)))
    tokens, placements = [], []
    for c in torch.randperm(len(pool), generator=gen).tolist():
        placements.append(Place(pool[c][1], len(tokens)))
        tokens += pool[c][0]
    tokens += torch.randint(0, vocab, (TAIL + QUERY,), generator=gen).tolist()
    res = hip.prefill(tokens, placements, BlendConfig(recompute_ratio=RATIO, n_sink=N_SINK))
    n_new = 32
    out = {}
    for name, fn in (("hip", lambda: hip.generate(res, n_new)), ("concat", lambda: DecoderPieces.generate(hip, res, n_new))):
        for _ in range(max(1, warmup)):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        toks_out = [fn() for _ in range(max(1, steps))]
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / max(1, steps)
        out[name] = (dt, toks_out[0])
    agree = sum(a == b for a, b in zip(out["hip"][1], out["concat"][1]))
    tps = n_new / out["hip"][0]
    return {
        "metric": "decode tokens/s after the 8k blend prefill", "value": round(tps, 2), "unit": "tokens/s",
        "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": round(out["hip"][0] * 1e3, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"random-init Qwen2.5-7B architecture, 8256-token blend prefill, {n_new} greedy tokens"},
        "concat_decode_tokens_per_s": round(n_new / out["concat"][0], 2),
        "tokens_equal_to_concat_decode": f"{agree}/{n_new}",
    }


PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 matrix-core peak


def bench_attention(steps: int, warmup: int, dev) -> dict:
    """ckv_attention_active at the Qwen2.5-7B shape (28 query / 4 KV heads, head_dim 128, bf16)
    over an 8256-row cache: the 2976 active rows of layers 2-27 of the 8k request (2400 cached
    positions kept at random + the 576 uncached tail) and all 8256 rows (layers 0-1, plain
    causal). Work = 4 * D flops per visible (query, key) pair and query head (the two products);
    the torch SDPA formulations the engine used before (expanded KV heads + boolean mask;
    is_causal with enable_gqa) are timed beside it."""
    import torch.nn.functional as F

    from chunkkv_amd import ops

    gen = torch.Generator().manual_seed(5)
    Hq = 28
    K = torch.randn((1, N_KV, N_TOKENS, HEAD_DIM), generator=gen).to(torch.bfloat16).to(dev)
    V = torch.randn((1, N_KV, N_TOKENS, HEAD_DIM), generator=gen).to(torch.bfloat16).to(dev)
    stream = torch.cuda.current_stream(dev)
    n_cached = N_CHUNKS * CHUNK_LEN
    cases = {
        "active_2976": torch.cat([torch.randperm(n_cached, generator=gen)[:2400].sort().values,
                                  torch.arange(n_cached, N_TOKENS)]),
        "causal_8256": torch.arange(N_TOKENS),
    }
    out = {}
    for name, active in cases.items():
        active = active.to(dev)
        n = active.numel()
        q = torch.randn((1, Hq, n, HEAD_DIM), generator=gen).to(torch.bfloat16).to(dev)
        flops = 4.0 * HEAD_DIM * Hq * float((active + 1).sum().item())
        for _ in range(warmup):
            ops.attention_active(q, K, V, active)
        ms = _timed(lambda i: ops.attention_active(q, K, V, active), steps, stream)
        if n == N_TOKENS:
            sdpa = lambda i: F.scaled_dot_product_attention(q, K, V, is_causal=True, enable_gqa=True)  # noqa: E731
        else:
            mask = active[:, None] >= torch.arange(N_TOKENS, device=dev)[None, :]
            Ke, Ve = K.repeat_interleave(Hq // N_KV, 1), V.repeat_interleave(Hq // N_KV, 1)
            sdpa = lambda i: F.scaled_dot_product_attention(q, Ke, Ve, attn_mask=mask)  # noqa: E731
        sdpa(0)
        ms_sdpa = _timed(sdpa, steps, stream)
        tf = flops / (ms * 1e-3) / 1e12
        out[name] = {"ms": round(ms, 4), "tflops": round(tf, 1), "frac": round(tf / PEAK_BF16_TFLOPS, 4),
                     "sdpa_ms": round(ms_sdpa, 4), "flops": flops}
    main_case = out["active_2976"]
    return {
        "metric": "positions-masked GQA attention, TFLOP/s", "value": main_case["tflops"], "unit": "TFLOP/s",
        "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": main_case["ms"], "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "Qwen2.5-7B attention shape: 28 q / 4 KV heads, head_dim 128, 8256-row cache; "
                               "2976 active rows (layers 2-27) and 8256 (layers 0-1)"},
        "roofline": {"kernel": "attn_active_kernel<128>", "bound": "mfma", "achieved": main_case["tflops"],
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": main_case["frac"], "traffic": None,
                     "flops_per_launch": main_case["flops"], "avg_launch_us": round(main_case["ms"] * 1e3, 2)},
        "cases": out,
    }


def bench_dropped(steps: int, warmup: int, dev) -> dict:
    """The dominant kernel alone: `steps` back-to-back gathers of the dropped rows of layers 2-27
    (alternating two input sets), timed with HIP events on the launch stream. Its rocprofv3
    kernel average is the same quantity (no other gather launch runs in this workload)."""
    wls = [RepairWorkload(1234 + i, dev) for i in range(2)]
    for w in wls:
        w.step_assemble()  # selection output, without a gather of the dropped rows
    for i in range(warmup):
        wls[i % 2].gather_dropped()
    stream = torch.cuda.current_stream(dev)
    ms = _timed(lambda i: wls[i % 2].gather_dropped(), steps, stream)
    assert all(int(w.err.item()) == 0 for w in wls)
    nb = dropped_bytes(wls[0].plan)
    gbs = nb / (ms * 1e-3) / 1e9
    return _workload_line("gather of the dropped rows, HBM GB/s", gbs, ms, steps, warmup,
                          {"workload": "layers 2-27 of the 8256-token Qwen2.5-7B-shape request: 24 cached chunks x 320, "
                                       "5280 dropped positions"},
                          {"kernel": "rerope_gather_kernel<bf16,128>", "bound": "hbm", "achieved": round(gbs, 1),
                           "peak": PEAK_GBS, "unit": "GB/s", "frac": round(gbs / PEAK_GBS, 4),
                           "traffic": DROPPED_TRAFFIC_BYTES, "bytes_per_launch": nb, "avg_launch_us": round(ms * 1e3, 2)})


def bench_layer1_32k(steps: int, warmup: int, dev) -> dict:
    """Layer 1's repair of one 32,832-token request alone, as the engine issues it
    (ckv_layer1_repair_gather: the layer-1 pass counting the candidate histogram, the selection
    spread over 129 slice workgroups, the kept rows with the dropped rows of two later layers):
    128 chunks x 256 tokens drawn from a pool of 64 (4 layers held) + a 64-token query, 15 %
    recompute + 4 sinks; layer-1 rows that follow the cached ones (per-chunk noise exp(N(-3, 1)))
    and uncorrelated random rows (every deviation within a few percent of the others), each set
    timed from HIP-graph replays of `steps` back-to-back calls. Run under rocprofv3 for the
    per-kernel times (the selection is `select_slices_kernel<9, false, false>`)."""
    from chunkkv_amd import ops
    from chunkkv_amd.planner import local_index, plan_request

    L, POOL, PER_REQ, Q, NL = 256, 64, 128, 64, 4
    N = PER_REQ * L + Q
    gen = torch.Generator(device=dev).manual_seed(3)
    store = [Chunk(torch.randn((NL, 1, N_KV, L, HEAD_DIM), generator=gen, device=dev).bfloat16(),
                   torch.randn((NL, 1, N_KV, L, HEAD_DIM), generator=gen, device=dev).bfloat16(), 1000 + 7 * i)
             for i in range(POOL)]
    rng = np.random.default_rng(3)
    pl = [Place(store[i], j * L) for j, i in enumerate(rng.choice(POOL, PER_REQ))]
    plan = plan_request(N, pl, N_SINK, 0.15)
    tab = np.concatenate([np.array([[k.data_ptr(), v.data_ptr()] for k, v in zip(c.keys, c.values)],
                                   dtype=np.uint64).reshape(-1) for c in plan.chunks])
    tab = torch.from_numpy(tab.view(np.int64)).to(dev)
    segs = torch.from_numpy(plan.segments.reshape(-1)).to(dev)
    flags = torch.from_numpy(plan.flags).to(dev)
    local = torch.from_numpy(local_index(N, plan.layer0_idx)).to(dev)
    spans = torch.from_numpy(plan.spans.reshape(-1)).to(dev)
    K = torch.empty((NL, 1, N_KV, N, HEAD_DIM), dtype=torch.bfloat16, device=dev)
    V = torch.empty_like(K)
    ops.rerope_gather(K, V, tab, segs, len(plan.segments), plan.max_seg_tokens, THETA, layers=(1, 2))
    sig = torch.exp(torch.randn(PER_REQ, generator=gen, device=dev) - 3.0).repeat_interleave(L)
    sig = torch.cat([sig, torch.ones(Q, device=dev)])[None, None, :, None]
    cached = torch.from_numpy(plan.cached).to(dev)[None, None, :, None]
    rnd = lambda: torch.randn((1, N_KV, N, HEAD_DIM), generator=gen, device=dev)  # noqa: E731
    rows = {
        "correlated": (torch.where(cached, K[1].float() + sig * rnd(), rnd()).bfloat16(),
                       torch.where(cached, V[1].float() + sig * rnd(), rnd()).bfloat16()),
        "uncorrelated": (rnd().bfloat16(), rnd().bfloat16()),
    }
    ws = ops.layer1_repair_workspace(dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    sel = ops._new_selection(N, len(plan.spans), dev)
    dn = (torch.empty(N, device=dev), torch.empty(N, device=dev))
    stream = torch.cuda.current_stream(dev)
    out = {}
    for name, (k1, v1) in rows.items():
        def call():
            ops.layer1_repair_gather(K, V, tab, 1, (2, NL), segs, len(plan.segments), plan.max_seg_tokens, k1, v1,
                                     flags, local, spans, None, THETA, ws, err, sel, dn)
        for _ in range(max(warmup, 2)):
            call()
        torch.cuda.synchronize()
        g = _graph_of(call)
        g.replay()
        out[name] = _timed(lambda i: g.replay(), steps, stream)
        assert int(err.item()) == 0 and int(sel.counts[0].item()) == plan.n_keep
    ms = out["correlated"]
    line = _workload_line("layer-1 repair of one 32,832-token request, us per call", ms * 1e3, ms, steps, warmup,
                          {"workload": "one 32,832-token request (128 chunks x 256 + 64 query, 15 % + 4 sinks), "
                                       "Qwen2.5-7B KV shape, ckv_layer1_repair_gather with two later layers"}, None)
    line["higher_is_better"] = False
    line["unit"] = "us"
    line.pop("pct_of_peak")
    line["us_per_call_uncorrelated"] = round(out["uncorrelated"] * 1e3, 2)
    return line


def repair_bytes_for(plan) -> int:
    """Algorithmic repair bytes of a request plan (gather of every cached row, deviation over the
    layer-0 active set, scatters of layer 0 and layers 1..L-1)."""
    row = ROW_BYTES
    n_cached_rows = int(plan.cached.sum())
    n0 = len(plan.layer0_idx)
    return (N_LAYERS * n_cached_rows * row * 4 + n0 * 4 * row + plan.n_tokens * 8 + n0 * row * 4
            + (N_LAYERS - 1) * plan.n_keep * row * 4)


def _config_summary(line: dict) -> dict:
    """The figures of one microbenchmark line kept in the default line's `configs`."""
    out = {"workload": line["config"]["workload"], "bytes_per_step": line["config"].get("bytes_per_step"),
           "ms_per_step": line["ms_per_step"], "gbs": line["value"], "pct_of_peak": line["pct_of_peak"]}
    if line.get("roofline"):
        rf = line["roofline"]
        out["roofline"] = {k: rf[k] for k in ("kernel", "achieved", "peak", "frac", "bytes_per_launch", "avg_launch_us")
                           if k in rf}
    for k in ("ratios", "store_gib", "ms_per_step_eager", "ms_per_step_uncorrelated", "uncorrelated_over_correlated",
              "ttft_p50_ms", "ttft_p99_ms", "ttft_requests", "ttft_p50_ms_concurrent", "ttft_p99_ms_concurrent",
              "ttft_requests_concurrent", "ttft_note", "ttft_concurrent_note"):
        if k in line:
            out[k] = line[k]
    return out


def _cpu_model() -> str:
    """The host CPU's model name with its family/model/stepping numbers (a virtualised host may
    report only the brand, e.g. "AMD EPYC"; the numbers still name the generation)."""
    info: dict[str, str] = {}
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if not ln.strip():
                    break  # the first processor's block is enough
                key, _, val = ln.partition(":")
                info.setdefault(key.strip(), val.strip())
    except OSError:
        return "unknown"
    name = info.get("model name", "unknown")
    nums = [f"{k} {info[k]}" for k in ("cpu family", "model", "stepping") if k in info]
    return f"{name} ({', '.join(nums)})" if nums else name


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--ttft-requests", type=int, default=50)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the config-2, config-3 and config-5 sub-measurements of the default line")
    ap.add_argument("--replay-ttft-requests", type=int, default=20)
    ap.add_argument("--concurrent-ttft", action="store_true",
                    help="config 5: also time 4 concurrent HipEngine prefills (one host thread each; off by default)")
    ap.add_argument("--workload", default="request",
                    choices=["request", "gather", "deviation", "replay", "traffic", "dropped", "attention", "extract",
                             "decode", "layer1_32k"],
                    help="request: the 8k Qwen2.5-7B blend-prefill KV repair (default); gather / deviation / replay: "
                         "the re-RoPE+gather, deviation+top-k+scatter and 4x32k replay microbenchmarks")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    request_streams(CONCURRENT, dev)  # the first streams of the process
    if args.workload != "request":
        fn = {"gather": bench_gather_only, "deviation": bench_deviation_topk, "replay": bench_replay,
              "traffic": traffic_probe, "dropped": bench_dropped, "attention": bench_attention,
              "extract": bench_extract, "decode": bench_decode, "layer1_32k": bench_layer1_32k}[args.workload]
        if args.workload == "replay":
            print(json.dumps(bench_replay(args.steps, args.warmup, dev, ttft_requests=args.replay_ttft_requests,
                                          concurrent_ttft=args.concurrent_ttft)),
                  flush=True)
        else:
            print(json.dumps(fn(args.steps, args.warmup, dev)), flush=True)
        return

    r = bench_repair(args.steps, args.warmup, dev)
    log(f"[bench] KV repair {r['gbs']:.1f} GB/s ({r['ms_per_step']:.3f} ms/step graph, {r['ms_two']:.3f} ms two "
        f"streams, {r['ms_asm']:.3f} ms assemble variant, {r['ms_split']:.3f} ms layer 1 as four launches, "
        f"{r['ms_eager']:.3f} ms eager); last launch {r['gk_gbs']:.1f} GB/s ({r['gk_ms'] * 1e3:.1f} us); "
        f"dropped-row gather {r['gd_gbs']:.1f} GB/s ({r['gd_ms'] * 1e3:.1f} us); "
        f"assemble {r['asm_gbs']:.1f} GB/s ({r['asm_ms'] * 1e3:.2f} us)")
    configs = {}
    if not args.no_configs:
        sub_steps = min(args.steps, 30)
        configs["config2_rerope_gather"] = _config_summary(bench_gather_only(sub_steps, args.warmup, dev))
        log(f"[bench] config 2 {configs['config2_rerope_gather']}")
        configs["config3_deviation_topk_scatter"] = _config_summary(bench_deviation_topk(sub_steps, args.warmup, dev))
        log(f"[bench] config 3 {configs['config3_deviation_topk_scatter']}")
        # before the 8k TTFT runs, like the sub-measurements above; it builds its own model
        configs["config5_replay"] = _config_summary(
            bench_replay(min(args.steps, 20), args.warmup, dev, ttft_requests=args.replay_ttft_requests,
                         concurrent_ttft=args.concurrent_ttft))
        log(f"[bench] config 5 {configs['config5_replay']}")
    ttft = bench_ttft(args.ttft_requests, dev) if args.ttft_requests > 0 else None
    model = ttft.pop("model") if ttft is not None else None
    del model
    torch.cuda.empty_cache()
    cpu = bench_cpu(args.cpu_seconds) if args.cpu_seconds > 0 else None

    line = {
        "metric": METRIC,
        "value": round(r["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 4),
        "ms_per_step_eager": round(r["ms_eager"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "blend-prefill KV repair, Qwen2.5-7B KV shape (28 layers, 4 KV heads, head_dim 128, bf16), "
                        "8256-token request: 24 cached chunks x 320 at shuffled positions + 512 uncached + 64 query, "
                        "30% recompute, 4 sinks",
            "tokens": N_TOKENS,
            "kept_rows": r["n_keep"],
            "bytes_per_step": r["bytes"],
            "bytes_per_step_note": "KV-repair bytes of one request as the reference's op sequence moves them "
                                   "(value = these bytes / step time); the fused path moves moved_bytes_per_step",
            "moved_bytes_per_step": r["moved"],
        },
        "pct_of_peak": round(100.0 * r["gbs"] / PEAK_GBS, 2),
        "moved_gbs": round(r["moved"] / (r["ms_per_step"] * 1e-3) / 1e9, 2),
        "pct_of_peak_moved": round(100.0 * r["moved"] / (r["ms_per_step"] * 1e-3) / 1e9 / PEAK_GBS, 2),
        "ms_per_step_two_streams": round(r["ms_two"], 4),
        "ms_per_step_assemble_variant": round(r["ms_asm"], 4),
        "ms_per_step_layer1_four_launches": round(r["ms_split"], 4),
        "ms_per_step_separate_gather": round(r["ms_sep"], 4),
        "ms_per_step_uncorrelated": round(r["ms_unc"], 4),
        "concurrent_requests": {"requests": CONCURRENT, "ms_per_round": round(r["ms_conc"], 4),
                                "gbs": round(r["conc_gbs"], 1), "pct_of_peak": round(100.0 * r["conc_gbs"] / PEAK_GBS, 2),
                                "note": "the same request's KV repair, CONCURRENT independent requests in flight on "
                                        "their own streams (one HIP graph per round); value is the single-request step"},
        "roofline": {
            "kernel": "rerope_gather_kernel<bf16,128,GatherSkip,kept rows> (the step's last launch: layer 1's kept "
                      "rows + dropped rows of layers 4-27)",
            "bound": "hbm",
            "achieved": round(r["gk_gbs"], 1),
            "peak": PEAK_GBS,
            "unit": "GB/s",
            "frac": round(r["gk_gbs"] / PEAK_GBS, 4),
            "traffic": MERGED_TRAFFIC_BYTES,
            "traffic_source": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, "
                              "profiles/traffic_request_step_kernels_qwen25_7b_8k.md",
            "bytes_per_launch": r["gk_bytes"],
            "avg_launch_us": round(r["gk_ms"] * 1e3, 2),
        },
        "dropped_row_gather_layers_2_27": {
            "kernel": "rerope_gather_kernel<bf16,128,GatherSkip> (the separate-gather step's launch)",
            "achieved": round(r["gd_gbs"], 1), "frac": round(r["gd_gbs"] / PEAK_GBS, 4),
            "traffic": DROPPED_TRAFFIC_BYTES, "bytes_per_launch": r["gd_bytes"],
            "avg_launch_us": round(r["gd_ms"] * 1e3, 2),
        },
        "assemble_kernel": {"bytes_per_launch": ASSEMBLE_BYTES, "avg_launch_us": round(r["asm_ms"] * 1e3, 2),
                            "achieved_gbs": round(r["asm_gbs"], 1)},
        "cpu_baseline": cpu,
    }
    if ttft is not None:
        line["ttft_p50_ms"] = round(ttft["hip"]["p50"], 2)
        line["ttft_p99_ms"] = round(ttft["hip"]["p99"], 2)
        line["ttft_p50_ms_torch_ops"] = round(ttft["torch_ops"]["p50"], 2)
        line["ttft_gemm_selection"] = "committed TunableOp table" if ttft["hip"]["tuned_gemms"] else "default heuristics"
        line["ttft_p99_ms_torch_ops"] = round(ttft["torch_ops"]["p99"], 2)
        line["ttft_requests"] = args.ttft_requests
        # KV repair on the HIP kernels, attention on PyTorch-ROCm with the reference's own SDPA call
        line["ttft_p50_ms_attention_reference"] = round(ttft["hip_attention_reference"]["p50"], 2)
        line["ttft_p99_ms_attention_reference"] = round(ttft["hip_attention_reference"]["p99"], 2)
        line["ttft_requests_attention_reference"] = ttft["hip_attention_reference"]["requests"]
        # KV repair on the HIP kernels, attention on torch's fused SDPA kernels, norm/MLP on torch
        line["ttft_p50_ms_torch_attention"] = round(ttft["hip_torch_attention"]["p50"], 2)
        line["ttft_p99_ms_torch_attention"] = round(ttft["hip_torch_attention"]["p99"], 2)
        # the same engine with the dropped-row gather on a side stream (HipEngine(overlap=True))
        line["ttft_p50_ms_side_stream"] = round(ttft["hip_overlap"]["p50"], 2)
    if configs:
        line["configs"] = configs
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
