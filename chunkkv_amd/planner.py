"""Host-side request planning for the blend-prefill KV-repair path.

Everything here is integer bookkeeping on the host, vectorised with numpy (the reference does
it with Python loops over every position: src/chunkkv/engine/base.py:63-73 and
src/chunkkv/engine/torch_engine.py:89-94, :106, :128-142):

* per-position flags cached / exact / sink / pooled and the index lists fresh_idx, layer0_idx;
* gather segments: one per run of positions owned by the same placement, the last placement
  winning where placements overlap (the reference assigns slices in placement order);
* the layer-1 selection spans of the non-exact placements with their token budgets
  ``int(round(ratio * length))`` (Python round-half-even) and ``pooled = ratio > 0``;
* the selection outcome sizes that do not depend on the deviation (all of them when no
  escalation threshold is set), which lets the engine size tensors without a device sync.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

POS_CACHED = 1
POS_SINK = 2
POS_EXACT = 4
POS_POOLED = 8  # inside a non-exact placement with ratio > 0 (the layer-1 pool, torch_engine.py:137-139)

SEG_FIELDS = 6  # dst_start, n_tokens, chunk, src_start, src_len, delta
SPAN_FIELDS = 4  # start, length, budget, pooled


@dataclass
class RequestPlan:
    n_tokens: int
    cached: np.ndarray  # bool (N,)
    exact: np.ndarray  # bool (N,)
    sink: np.ndarray  # bool (N,)
    flags: np.ndarray  # uint8 (N,) POS_* bits
    fresh_idx: np.ndarray  # int64, positions not covered by any placement
    layer0_idx: np.ndarray  # int64, positions not covered by an exact placement
    segments: np.ndarray  # int32 (S, 6): cached runs (what the gather reads)
    max_seg_tokens: int
    all_segments: np.ndarray  # int32 (S + F, 6): the cached runs, then uncached runs (chunk = -1)
    max_all_seg_tokens: int
    chunks: list  # unique ChunkKV objects, indexed by segments[:, 2]
    spans: np.ndarray  # int32 (C, 4) for the non-exact placements, in placement order
    n_cached: int
    has_overlap: bool
    # Selection sizes that follow from the layout alone (valid when no escalation threshold):
    budget_requested: int = 0
    n_candidates: int = 0
    budget: int = 0
    n_keep: int = 0
    selected_cached: int = 0
    extra: dict = field(default_factory=dict)


def chunk_length(chunk) -> int:
    return int(chunk.keys[0].shape[2])


def round_budget(ratio: float, length: int) -> int:
    """``int(round(ratio * length))`` exactly as the reference computes it (torch_engine.py:139)."""
    return int(round(ratio * length))


def plan_request(n_tokens: int, placements: list, n_sink: int, recompute_ratio: float) -> RequestPlan:
    """Build the per-request plan. Raises ValueError for placements outside [0, n_tokens)."""
    N = int(n_tokens)
    cached = np.zeros(N, dtype=bool)
    exact = np.zeros(N, dtype=bool)
    sink = np.zeros(N, dtype=bool)
    pooled = np.zeros(N, dtype=bool)
    owner = np.full(N, -1, dtype=np.int64)

    chunk_ids: dict[int, int] = {}
    chunks: list = []
    place_chunk = np.empty(len(placements), dtype=np.int64)
    lengths = np.empty(len(placements), dtype=np.int64)
    spans = []
    for i, p in enumerate(placements):
        L = chunk_length(p.chunk)
        s = int(p.start)
        if s < 0 or s + L > N or L < 0:
            raise ValueError(f"placement {i} covers [{s}, {s + L}) outside the request of {N} tokens")
        key = id(p.chunk)
        if key not in chunk_ids:
            chunk_ids[key] = len(chunks)
            chunks.append(p.chunk)
        place_chunk[i] = chunk_ids[key]
        lengths[i] = L
        cached[s : s + L] = True
        owner[s : s + L] = i
        if p.exact:
            exact[s : s + L] = True
        else:
            if n_sink > 0:
                sink[s : s + min(L, n_sink)] = True
            ratio = recompute_ratio if p.ratio is None else p.ratio
            spans.append((s, L, round_budget(ratio, L) if ratio > 0 else 0, 1 if ratio > 0 else 0))
            if ratio > 0:
                pooled[s : s + L] = True

    flags = (cached.astype(np.uint8) * POS_CACHED) | (sink.astype(np.uint8) * POS_SINK) | (
        exact.astype(np.uint8) * POS_EXACT) | (pooled.astype(np.uint8) * POS_POOLED)

    # Runs of equal owner -> gather segments (last placement wins on overlap).
    segments = np.zeros((0, SEG_FIELDS), dtype=np.int32)
    max_seg = 0
    covered = owner >= 0
    if covered.any():
        change = np.empty(N, dtype=bool)
        change[0] = True
        change[1:] = owner[1:] != owner[:-1]
        starts = np.flatnonzero(change & covered)
        ends_mask = np.empty(N, dtype=bool)
        ends_mask[-1] = True
        ends_mask[:-1] = owner[:-1] != owner[1:]
        ends = np.flatnonzero(ends_mask & covered) + 1
        own = owner[starts]
        p_start = np.array([int(placements[k].start) for k in own], dtype=np.int64)
        c_start = np.array([int(placements[k].chunk.start) for k in own], dtype=np.int64)
        segments = np.stack(
            [starts, ends - starts, place_chunk[own], starts - p_start, lengths[own], p_start - c_start], axis=1
        ).astype(np.int32)
        max_seg = int((ends - starts).max())

    # Uncached runs (chunk = -1): their rows always come from the fresh K/V.
    fresh_segs = np.zeros((0, SEG_FIELDS), dtype=np.int32)
    if (~covered).any():
        un = ~covered
        edge = np.diff(np.concatenate(([0], un.astype(np.int8), [0])))
        f_starts = np.flatnonzero(edge == 1)
        f_ends = np.flatnonzero(edge == -1)
        fresh_segs = np.zeros((len(f_starts), SEG_FIELDS), dtype=np.int32)
        fresh_segs[:, 0] = f_starts
        fresh_segs[:, 1] = f_ends - f_starts
        fresh_segs[:, 2] = -1
    all_segments = np.concatenate([segments, fresh_segs]) if len(fresh_segs) else segments
    max_all = int(all_segments[:, 1].max()) if len(all_segments) else 0

    total_len = int(lengths.sum()) if len(placements) else 0
    n_cached = int(cached.sum())
    plan = RequestPlan(
        n_tokens=N,
        cached=cached,
        exact=exact,
        sink=sink,
        flags=flags,
        fresh_idx=np.flatnonzero(~cached),
        layer0_idx=np.flatnonzero(~exact),
        segments=segments,
        max_seg_tokens=max_seg,
        all_segments=all_segments,
        max_all_seg_tokens=max_all,
        chunks=chunks,
        spans=np.asarray(spans, dtype=np.int32).reshape(-1, SPAN_FIELDS),
        n_cached=n_cached,
        has_overlap=total_len != n_cached,
    )
    _static_selection(plan)
    return plan


def _static_selection(plan: RequestPlan) -> None:
    """Selection sizes when no chunk escalates (torch_engine.py:125-147 with rel ignored)."""
    N = plan.n_tokens
    keep = ~plan.cached | plan.sink
    pool = np.zeros(N, dtype=bool)
    requested = 0
    for s, L, b, pooled in plan.spans:
        if pooled:
            pool[s : s + L] = True
            requested += int(b)
    cand = pool & ~keep
    n_cand = int(cand.sum())
    budget = max(0, min(requested, n_cand))
    plan.budget_requested = requested
    plan.n_candidates = n_cand
    plan.budget = budget
    plan.n_keep = int(keep.sum()) + budget
    plan.selected_cached = int((keep & plan.cached).sum()) + budget


def local_index(n_tokens: int, active: np.ndarray) -> np.ndarray:
    """local[p] = row of position p in `active`, -1 elsewhere (torch_engine.py:148-149)."""
    local = np.full(n_tokens, -1, dtype=np.int32)
    local[active] = np.arange(len(active), dtype=np.int32)
    return local


def stats_dict(n_tokens: int, n_cached: int, n_layers: int, layer0: int, selected_cached: int, chunk_stats: list) -> dict:
    """The reference's stats dict (torch_engine.py:167-176)."""
    rest = (n_tokens - n_cached + selected_cached) * (n_layers - 1)
    return {
        "tokens": n_tokens,
        "cached_tokens": n_cached,
        "recomputed_cached_tokens": selected_cached,
        "prefill_token_equiv": (layer0 + rest) / n_layers,
        "chunks": chunk_stats,
    }
