"""Boundary types of the blend-prefill API.

Field names, defaults and semantics follow src/chunkkv/engine/base.py:13-73 so that callers of
the reference engine (runtime, store, bench) can hand these objects, or the reference's own,
to :class:`chunkkv_amd.engine.HipEngine` unchanged. The engine only reads attributes, so the
reference's dataclasses work as well as these.

K/V tensors are (1, n_kv_heads, L, head_dim) with RoPE applied.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Callable


@dataclass
class ChunkKV:
    """Per-layer K/V of one chunk, computed at positions start .. start+length (base.py:13-23)."""

    keys: list[Any]
    values: list[Any]
    start: int

    @property
    def length(self) -> int:
        return self.keys[0].shape[2]


@dataclass
class Placement:
    """A cached chunk placed at a new offset of the request (base.py:26-33)."""

    chunk: ChunkKV
    start: int
    ratio: float | None = None  # this placement's own recompute fraction; None: BlendConfig.recompute_ratio
    exact: bool = False  # KV produced under the identical prefix: kept as is at every layer, layer 0 too


@dataclass
class BlendConfig:
    """Blend-prefill knobs (base.py:36-43)."""

    recompute_ratio: float = 0.15  # per placement, the part of its cached positions re-run in layers 1..L-1
    n_sink: int = 2  # leading positions of every non-exact placement, re-run unconditionally
    full_first_layer: bool = True  # layer 0 over every non-exact position; False: plain reuse, no repair
    escalate_threshold: float | None = None  # a placement whose layer-1 relative deviation exceeds it is re-run whole


@dataclass
class PrefillResult:
    """Prefill output (base.py:46-60). keys/values hold one (1, H, N, D) tensor per layer."""

    logits: Any  # (n, vocab) for the positions in logit_positions
    logit_positions: Any
    keys: list[Any]
    values: list[Any]
    stats: dict = field(default_factory=dict)
    copy: Callable[[Any], Any] = lambda a: a  # detaches a stored chunk's slices from the request's cache buffers
    # Batched extraction hook (spans -> one (2, L, 1, H, len, D) buffer per span); set by HipEngine
    # to its one-launch kernel. None: the per-layer `copy` path of the reference.
    extract: Callable[[list], list] | None = None

    def chunk(self, start: int, end: int) -> ChunkKV:
        return self.chunks([(start, end)])[0]

    def chunks(self, spans: list) -> list[ChunkKV]:
        """ChunkKV copies of several (start, end) segments; with an extraction hook, one launch
        for all layers of all of them."""
        if self.extract is None:
            return [ChunkKV(keys=[self.copy(k[:, :, s:e, :]) for k in self.keys],
                            values=[self.copy(v[:, :, s:e, :]) for v in self.values], start=s) for s, e in spans]
        return [ChunkKV(keys=list(b[0].unbind(0)), values=list(b[1].unbind(0)), start=int(s))
                for b, (s, _) in zip(self.extract(spans), spans)]


def plan_positions(n: int, placements: list, n_sink: int):
    """Per-position flags as Python lists: cached, exact, sink (base.py:63-73).

    Kept for API compatibility; the engine uses the vectorised planner in
    :mod:`chunkkv_amd.planner`, which produces the same flags.
    """
    cached, exact, sink = [False] * n, [False] * n, [False] * n
    for p in placements:
        end = p.start + p.chunk.length
        for i in range(p.start, end):
            cached[i] = True
        if p.exact:
            for i in range(p.start, end):
                exact[i] = True
        else:
            for i in range(p.start, min(end, p.start + n_sink)):
                sink[i] = True
    return cached, exact, sink
