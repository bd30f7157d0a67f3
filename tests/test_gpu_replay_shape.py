"""The long-context replay's request shape through the KV-repair kernels, checked against the
oracle: 128 chunks of 256 tokens drawn with replacement (Zipf s=1.1) from a pool, so one chunk
sits at several positions with different shifts, plus a 64-token query (N = 32832); 28 layers,
4 KV heads, head_dim 128, bf16; 15% recompute + 4 sinks (budget 128 x 38 = 4864). The flow is
the engine's: layer 1's base cache, the layer-1 deviation against fresh rows that differ from the
cached ones by a per-chunk noise level, the selection (register path at 33 positions per
thread), the scatter of the kept rows, then the gather of the dropped rows of layers 2-27.
Everything integer or copied is bit-exact; the sums follow the oracle's fixed order, so the
deviation and the selection are bit-exact too.
"""

import numpy as np
import pytest
import torch

from chunkkv_amd import ops
from chunkkv_amd.planner import local_index, plan_request
from chunkkv_amd.types import ChunkKV, Placement
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
L_CH, N_PLACED, POOL, Q = 256, 128, 24, 64
NL, H, D, THETA = 28, 4, 128, 1e6
SENT = -7.0


def _np(t):
    return O.to_numpy(t)


def test_config5_request_repair_matches_oracle():
    rng = np.random.default_rng(55)
    g = torch.Generator(device=DEV).manual_seed(55)
    pool = [
        ChunkKV([torch.randn((1, H, L_CH, D), generator=g, device=DEV).bfloat16() for _ in range(NL)],
                [torch.randn((1, H, L_CH, D), generator=g, device=DEV).bfloat16() for _ in range(NL)],
                int(rng.integers(0, 32768)))
        for _ in range(POOL)
    ]
    zipf = 1.0 / np.arange(1, POOL + 1) ** 1.1
    ids = rng.choice(POOL, N_PLACED, p=zipf / zipf.sum())
    assert len(set(ids.tolist())) < N_PLACED  # chunks repeat at several positions
    placements = [Placement(pool[c], j * L_CH) for j, c in enumerate(ids)]
    N = N_PLACED * L_CH + Q
    plan = plan_request(N, placements, 4, 0.15)
    assert plan.budget == 4864

    tab = np.array([[[k.data_ptr(), v.data_ptr()] for k, v in zip(ch.keys, ch.values)] for ch in plan.chunks],
                   dtype=np.uint64)
    tab_d = torch.from_numpy(tab.reshape(-1).view(np.int64)).to(DEV)
    segs_d = torch.from_numpy(plan.segments.reshape(-1)).to(DEV)
    flags_np = plan.flags
    local_np = local_index(N, plan.layer0_idx)
    flags_d, local_d = torch.from_numpy(flags_np).to(DEV), torch.from_numpy(local_np).to(DEV)
    spans_d = torch.from_numpy(plan.spans.reshape(-1)).to(DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    K = torch.full((NL, 1, H, N, D), SENT, dtype=torch.bfloat16, device=DEV)
    V = torch.full_like(K, SENT)

    # layer 1's base cache, then fresh rows = cached + per-chunk noise (uncached positions random)
    ops.rerope_gather(K, V, tab_d, segs_d, len(plan.segments), plan.max_seg_tokens, THETA, err, layers=(1, 2))
    base_k, base_v = K[1].clone(), V[1].clone()
    sigma = torch.exp(torch.randn(N_PLACED, generator=g, device=DEV) - 3.0)
    noise = torch.ones(N, device=DEV)
    for j in range(N_PLACED):
        noise[j * L_CH : (j + 1) * L_CH] = sigma[j]
    cached = torch.from_numpy(plan.cached).to(DEV)[None, None, :, None]
    rnd = lambda: torch.randn((1, H, N, D), generator=g, device=DEV)  # noqa: E731
    k1 = torch.where(cached, base_k.float() + noise[None, None, :, None] * rnd(), rnd()).bfloat16()
    v1_rows = torch.where(cached, base_v.float() + noise[None, None, :, None] * rnd(), rnd()).bfloat16()
    v1 = v1_rows.transpose(1, 2).contiguous().transpose(1, 2)  # token-major memory, as v_proj leaves it

    diff, norm = ops.deviation(k1, v1, K[1], V[1], flags_d, local_d, err)
    sel = ops.select(diff, norm, flags_d, local_d, spans_d, None)
    n_keep = plan.n_keep
    keep_abs = sel.keep_abs[:n_keep]
    ops.scatter_rows(K[1], V[1], k1.index_select(2, sel.keep_local[:n_keep]),
                     v1.index_select(2, sel.keep_local[:n_keep]), keep_abs, err)
    ops.rerope_gather(K, V, tab_d, segs_d, len(plan.segments), plan.max_seg_tokens, THETA, err, layers=(2, NL),
                      skip=sel.keep_rank)
    torch.cuda.synchronize()
    assert int(err.item()) == 0

    # oracle: layer-1 base cache
    sent = O.f32_to_bf16_bits(np.float32([SENT]))[0]

    def oracle_layer(li):
        Ko = np.full((1, H, N, D), sent, dtype=np.uint16)
        Vo = np.full_like(Ko, sent)
        ks = [[_np(ch.keys[li])[0]] for ch in plan.chunks]
        vs = [[_np(ch.values[li])[0]] for ch in plan.chunks]
        assert O.rerope_gather(Ko, Vo, ks, vs, plan.segments, THETA) == 0
        return Ko[0], Vo[0]

    K1o, V1o = oracle_layer(1)
    np.testing.assert_array_equal(_np(base_k)[0], K1o)
    np.testing.assert_array_equal(_np(base_v)[0], V1o)

    # deviation and selection, bit-exact
    k1_np, v1_np = _np(k1)[0], _np(v1_rows)[0]
    d_o, n_o = O.deviation(k1_np, v1_np, K1o, V1o, flags_np, local_np)
    np.testing.assert_array_equal(diff.cpu().numpy(), d_o)
    np.testing.assert_array_equal(norm.cpu().numpy(), n_o)
    want = O.select(d_o, n_o, flags_np, local_np, plan.spans, None)
    assert int(want["counts"][0]) == n_keep == int(sel.counts[0].item())
    np.testing.assert_array_equal(keep_abs.cpu().numpy(), want["keep_abs"])
    np.testing.assert_array_equal(sel.keep_rank.cpu().numpy(), want["keep_rank"])
    np.testing.assert_array_equal(sel.rel_dev.cpu().numpy(), want["rel_dev"])

    # layer 1 after the scatter: kept rows fresh, the rest the base cache
    ka = want["keep_abs"]
    K1w, V1w = K1o.copy(), V1o.copy()
    K1w[:, ka], V1w[:, ka] = k1_np[:, ka], v1_np[:, ka]
    np.testing.assert_array_equal(_np(K[1])[0], K1w)
    np.testing.assert_array_equal(_np(V[1])[0], V1w)

    # layers 2..27: cached rows of the dropped positions gathered, kept positions untouched
    dropped = plan.cached & (want["keep_rank"] < 0)
    for li in (2, 13, NL - 1):
        Klo, Vlo = oracle_layer(li)
        Kg, Vg = _np(K[li])[0], _np(V[li])[0]
        np.testing.assert_array_equal(Kg[:, dropped], Klo[:, dropped])
        np.testing.assert_array_equal(Vg[:, dropped], Vlo[:, dropped])
        assert (Kg[:, ~dropped] == sent).all() and (Vg[:, ~dropped] == sent).all()
