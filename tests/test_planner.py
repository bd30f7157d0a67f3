"""Host planner (chunkkv_amd.planner) against the reference's own list-based planning
(base.py:63-73, restated in chunkkv_amd.types.plan_positions and in the oracle) and the
selection sizes the oracle computes."""

import numpy as np
import pytest

from chunkkv_amd.planner import POS_POOLED, local_index, plan_request, round_budget, stats_dict
from chunkkv_amd.types import BlendConfig, ChunkKV, Placement, plan_positions
from oracle import engine_ref as R
from oracle import oracle as O


class _C:
    def __init__(self, L, start=0):
        self.keys = [np.zeros((1, 1, L, 1))]
        self.values = self.keys
        self.start = start

    @property
    def length(self):
        return self.keys[0].shape[2]


def _random_layout(rng, n_tokens, n_pl, overlap=False, exact_frac=0.2):
    pls = []
    pos = int(rng.integers(0, 10))
    for _ in range(n_pl):
        L = int(rng.integers(1, 60))
        if pos + L > n_tokens:
            break
        pls.append(Placement(_C(L, int(rng.integers(0, 500))), pos, ratio=[None, 0.0, 0.5, 1.0][int(rng.integers(0, 4))],
                             exact=bool(rng.random() < exact_frac)))
        pos += L - (int(rng.integers(0, L)) if overlap else 0) + int(rng.integers(0, 8))
    return pls


@pytest.mark.parametrize("seed", range(20))
@pytest.mark.parametrize("overlap", [False, True])
def test_flags_match_reference_lists(seed, overlap):
    rng = np.random.default_rng(seed)
    N = 400
    pls = _random_layout(rng, N, 12, overlap)
    n_sink = int(rng.integers(0, 6))
    plan = plan_request(N, pls, n_sink, 0.15)
    cached, exact, sink = plan_positions(N, pls, n_sink)
    np.testing.assert_array_equal(plan.cached, cached)
    np.testing.assert_array_equal(plan.exact, exact)
    np.testing.assert_array_equal(plan.sink, sink)
    c2, e2, s2 = R.plan_positions(N, pls, n_sink)  # the oracle's independent restatement
    np.testing.assert_array_equal(plan.sink, s2)
    np.testing.assert_array_equal(plan.fresh_idx, [i for i in range(N) if not cached[i]])
    np.testing.assert_array_equal(plan.layer0_idx, [i for i in range(N) if not exact[i]])
    assert plan.has_overlap == (sum(p.chunk.keys[0].shape[2] for p in pls) != sum(cached))
    # the pooled bit: the reference's pool mask before escalation (torch_engine.py:128-139)
    pool = np.zeros(N, dtype=bool)
    for p in pls:
        ratio = 0.15 if p.ratio is None else p.ratio
        if not p.exact and ratio > 0:
            pool[p.start : p.start + p.chunk.keys[0].shape[2]] = True
    np.testing.assert_array_equal((plan.flags & POS_POOLED) != 0, pool)
    np.testing.assert_array_equal(plan.flags & 7, np.asarray(cached) * 1 + np.asarray(sink) * 2 + np.asarray(exact) * 4)


@pytest.mark.parametrize("seed", range(10))
def test_segments_cover_union_last_placement_wins(seed):
    rng = np.random.default_rng(100 + seed)
    N = 300
    pls = _random_layout(rng, N, 10, overlap=True)
    plan = plan_request(N, pls, 2, 0.15)
    owner = np.full(N, -1)
    for i, p in enumerate(pls):
        owner[p.start : p.start + p.chunk.keys[0].shape[2]] = i
    seen = np.full(N, -1)
    for dst, n, c, src, L, delta in plan.segments:
        assert n > 0
        seen[dst : dst + n] = 1
        i = owner[dst]
        assert (owner[dst : dst + n] == i).all()
        p = pls[i]
        assert plan.chunks[c] is p.chunk
        assert src == dst - p.start and L == p.chunk.keys[0].shape[2] and delta == p.start - p.chunk.start
    np.testing.assert_array_equal(seen >= 0, owner >= 0)
    assert plan.max_seg_tokens == (plan.segments[:, 1].max() if len(plan.segments) else 0)


def test_out_of_range_placement_rejected():
    with pytest.raises(ValueError):
        plan_request(10, [Placement(_C(5), 8)], 2, 0.15)
    with pytest.raises(ValueError):
        plan_request(10, [Placement(_C(5), -1)], 2, 0.15)


def test_budget_rounding_is_pythons():
    assert round_budget(0.5, 5) == 2 and round_budget(0.3, 5) == 2 and round_budget(0.15, 256) == 38
    assert round_budget(0.3, 320) == 96 and round_budget(0.15, 10) == 2 and round_budget(0.25, 2) == 0


@pytest.mark.parametrize("ratio, keep", [(0.15, 1344), (0.30, 2592), (0.50, 4224)])
def test_config3_selection_sizes(ratio, keep):
    pls = [Placement(_C(256), c * 256) for c in range(32)]
    plan = plan_request(8192, pls, 4, ratio)
    assert plan.n_keep == keep and plan.selected_cached == keep


def test_config4_selection_sizes():
    pls = [Placement(_C(320, 7), c * 320) for c in range(24)]
    plan = plan_request(8256, pls, 4, 0.30)
    assert (plan.budget, plan.n_keep, plan.selected_cached) == (2304, 2976, 2400)
    assert len(plan.fresh_idx) == 576 and len(plan.segments) == 24


@pytest.mark.parametrize("seed", range(15))
def test_static_sizes_match_oracle_selection(seed):
    rng = np.random.default_rng(200 + seed)
    N = 500
    pls = _random_layout(rng, N, 14, overlap=False)
    n_sink = int(rng.integers(0, 5))
    plan = plan_request(N, pls, n_sink, 0.2)
    diff = rng.gamma(2.0, 1.0, N).astype(np.float32)
    local = local_index(N, plan.layer0_idx)
    got = O.select(diff, diff + 1, plan.flags, local, plan.spans, None)
    c = got["counts"]
    assert (c[0], c[1], c[2], c[3], c[5]) == (plan.n_keep, plan.selected_cached, plan.budget, plan.n_candidates,
                                              plan.budget_requested)
    assert c[4] == 0  # nothing outside layer0_idx is ever kept


def test_stats_closed_forms():
    # tests/test_mlx_engine.py:29 (no cache) and :39 (naive reuse of one chunk of length a)
    assert stats_dict(100, 0, 24, 100, 0, [])["prefill_token_equiv"] == 100
    assert stats_dict(100, 30, 24, 70, 0, [])["prefill_token_equiv"] == 70
    st = stats_dict(100, 30, 24, 100, 10, [{"x": 1}])
    assert st["prefill_token_equiv"] == (100 + (100 - 30 + 10) * 23) / 24 and st["chunks"] == [{"x": 1}]


def test_local_index():
    act = np.array([0, 3, 4, 9])
    np.testing.assert_array_equal(local_index(10, act), [0, -1, -1, 1, 2, -1, -1, -1, -1, 3])


def test_types_mirror_reference_defaults():
    cfg = BlendConfig()
    assert (cfg.recompute_ratio, cfg.n_sink, cfg.full_first_layer, cfg.escalate_threshold) == (0.15, 2, True, None)
    ch = ChunkKV([np.zeros((1, 2, 7, 4))], [np.zeros((1, 2, 7, 4))], 3)
    assert ch.length == 7
    p = Placement(ch, 5)
    assert p.ratio is None and p.exact is False
