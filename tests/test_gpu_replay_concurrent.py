"""The long-context replay workload at full size, concurrently: an HBM-resident store of 256
chunks x 256 tokens x 2 context variants (7.0 GiB at the Qwen2.5-7B KV shape: 28 layers, 4 KV
heads, head_dim 128, bf16) and 4 requests of 128 chunks drawn with replacement (Zipf s=1.1) at
shuffled positions plus a 64-token query (N = 32832), 15 % recompute + 4 sinks. Each request's
KV repair is issued on its own HIP stream, all four in flight together, in the launch order of
the engine (layer 0's fresh rows; layer 1's repair as one ckv_layer1_repair call, with a
workspace per request: base cache with the deviation, selection, kept rows; the gather of the
dropped rows of layers 2-27; the fresh rows of layers 2-27). The fresh layer-1 rows are built
beforehand from a base cache of the standalone gather. Every request is then checked against the
oracle, bit for bit: that base cache, diff/norm, the kept set, layer 1 after the repair, the
fresh rows of layers 0 and 27 (RoPE at their positions) and the gathered rows of layers 2 and 27.
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
NL, H, D, THETA = 28, 4, 128, 1e6
L_CH, POOL, VARIANTS, PER_REQ, Q = 256, 256, 2, 128, 64
N = PER_REQ * L_CH + Q
N_REQ = 4


def _build(g, rng, store):
    zipf = 1.0 / np.arange(1, POOL + 1) ** 1.1
    ids = rng.choice(POOL, PER_REQ, p=zipf / zipf.sum()) * VARIANTS + rng.integers(0, VARIANTS, PER_REQ)
    placements = [Placement(store[i], j * L_CH) for j, i in enumerate(ids)]
    plan = plan_request(N, placements, 4, 0.15)
    tab = np.array([[[k.data_ptr(), v.data_ptr()] for k, v in zip(ch.keys, ch.values)] for ch in plan.chunks],
                   dtype=np.uint64)
    rq = dict(
        plan=plan, tab=torch.from_numpy(tab.reshape(-1).view(np.int64)).to(DEV),
        segs=torch.from_numpy(plan.segments.reshape(-1)).to(DEV), flags=torch.from_numpy(plan.flags).to(DEV),
        local=torch.from_numpy(local_index(N, plan.layer0_idx)).to(DEV),
        spans=torch.from_numpy(plan.spans.reshape(-1)).to(DEV),
        layer0=torch.from_numpy(plan.layer0_idx.astype(np.int64)).to(DEV),
        K=torch.empty((NL, 1, H, N, D), dtype=torch.bfloat16, device=DEV),
        err=torch.zeros(1, dtype=torch.int32, device=DEV),
    )
    rq["V"] = torch.empty_like(rq["K"])
    # projections (token-major, before RoPE) of layer 0 and of layer 27's kept rows; layers 2-26 get
    # rows of their own too (their content is not checked, only that they land in the kept rows)
    rq["proj"] = [None if li == 1 else tuple(
        torch.randn((1, N if li == 0 else plan.n_keep, H * D), generator=g, device=DEV).bfloat16() for _ in range(2))
        for li in range(NL)]
    # layer-1 fresh rows: the base cache plus a per-chunk noise level (built after the base cache)
    rq["sigma"] = torch.exp(torch.randn(PER_REQ, generator=g, device=DEV) - 3.0)
    return rq


def _fresh_layer1(g, rq):
    plan = rq["plan"]
    noise = rq["sigma"].repeat_interleave(L_CH)
    noise = torch.cat([noise, torch.ones(Q, device=DEV)])[None, None, :, None]
    cached = torch.from_numpy(plan.cached).to(DEV)[None, None, :, None]
    rnd = lambda: torch.randn((1, H, N, D), generator=g, device=DEV)  # noqa: E731
    K1, V1 = rq["K"][1], rq["V"][1]
    k1 = torch.where(cached, K1.float() + noise * rnd(), rnd()).bfloat16()
    v1_rows = torch.where(cached, V1.float() + noise * rnd(), rnd()).bfloat16()
    rq["k1"], rq["v1_rows"] = k1, v1_rows
    rq["v1"] = v1_rows.transpose(1, 2).contiguous().transpose(1, 2)  # token-major memory, as v_proj leaves it


def _repair(rq):
    """One request's KV repair in the engine's launch order."""
    plan = rq["plan"]
    K, V = rq["K"].unbind(0), rq["V"].unbind(0)
    nseg, mseg, err = len(plan.segments), plan.max_seg_tokens, rq["err"]
    ops.rope_qkv(None, *rq["proj"][0], rq["layer0"], 0, H, D, THETA, k_out=K[0], v_out=V[0], rows=rq["layer0"],
                 err=err)
    diff, norm, sel = ops.layer1_repair(K[1], V[1], rq["tab"], NL, 1, rq["segs"], nseg, rq["k1"], rq["v1"],
                                        rq["flags"], rq["local"], rq["spans"], None, THETA, rq["ws"], err)
    rq["diff"], rq["norm"], rq["sel"] = diff, norm, sel
    rows = sel.keep_abs[: plan.n_keep]
    ops.rerope_gather(rq["K"], rq["V"], rq["tab"], rq["segs"], nseg, mseg, THETA, err, layers=(2, NL),
                      skip=sel.keep_rank)
    for li in range(2, NL):
        ops.rope_qkv(None, *rq["proj"][li], rows, 0, H, D, THETA, k_out=K[li], v_out=V[li], rows=rows, err=err)


def _oracle_layer(plan, li):
    Ko = np.zeros((1, H, N, D), dtype=np.uint16)
    Vo = np.zeros_like(Ko)
    ks = [[O.to_numpy(ch.keys[li])[0]] for ch in plan.chunks]
    vs = [[O.to_numpy(ch.values[li])[0]] for ch in plan.chunks]
    assert O.rerope_gather(Ko, Vo, ks, vs, plan.segments, THETA) == 0
    return Ko[0], Vo[0]


def test_config5_four_concurrent_requests_match_oracle():
    g = torch.Generator(device=DEV).manual_seed(5)
    rng = np.random.default_rng(5)
    store = []
    for _ in range(POOL * VARIANTS):
        k = torch.randn((NL, 1, H, L_CH, D), generator=g, device=DEV).bfloat16()
        v = torch.randn((NL, 1, H, L_CH, D), generator=g, device=DEV).bfloat16()
        store.append(ChunkKV(list(k.unbind(0)), list(v.unbind(0)), int(rng.integers(0, 32768))))
    reqs = [_build(g, rng, store) for _ in range(N_REQ)]
    assert all(rq["plan"].budget == 4864 for rq in reqs)
    assert len({c for rq in reqs for c in map(id, rq["plan"].chunks)}) < N_REQ * PER_REQ  # chunks shared
    # layer 1's base caches first (the fresh layer-1 rows are built from them; layer 1 is then
    # reset to a sentinel, every row of which the repair must rewrite), then every request's
    # repair, the four requests on four streams in flight together
    for rq in reqs:
        plan = rq["plan"]
        ops.rerope_gather(rq["K"], rq["V"], rq["tab"], rq["segs"], len(plan.segments), plan.max_seg_tokens, THETA,
                          rq["err"], layers=(1, 2))
        rq["base_k"], rq["base_v"] = rq["K"][1].clone(), rq["V"][1].clone()
        _fresh_layer1(g, rq)
        rq["K"][1].fill_(-7.0)
        rq["V"][1].fill_(-7.0)
        rq["ws"] = ops.layer1_repair_workspace(DEV)
    main = torch.cuda.current_stream()
    streams = [torch.cuda.Stream() for _ in reqs]  # default priority
    for rq, st in zip(reqs, streams):
        st.wait_stream(main)
        with torch.cuda.stream(st):
            _repair(rq)
    for st in streams:
        main.wait_stream(st)
    torch.cuda.synchronize()

    for r, rq in enumerate(reqs):
        plan = rq["plan"]
        print(f"request {r}: {len(plan.chunks)} distinct chunks, n_keep {plan.n_keep}", flush=True)
        assert int(rq["err"].item()) == 0
        K1o, V1o = _oracle_layer(plan, 1)
        c = plan.cached  # the query rows are written later (layer 1's scatter), not by the gather
        np.testing.assert_array_equal(O.to_numpy(rq["base_k"])[0][:, c], K1o[:, c])
        np.testing.assert_array_equal(O.to_numpy(rq["base_v"])[0][:, c], V1o[:, c])
        flags, local = plan.flags, local_index(N, plan.layer0_idx)
        k1, v1 = O.to_numpy(rq["k1"])[0], O.to_numpy(rq["v1_rows"])[0]
        d_o, n_o = O.deviation(k1, v1, K1o, V1o, flags, local)
        np.testing.assert_array_equal(O.to_numpy(rq["diff"]).view(np.uint32), d_o.view(np.uint32))
        np.testing.assert_array_equal(O.to_numpy(rq["norm"]).view(np.uint32), n_o.view(np.uint32))
        want = O.select(d_o, n_o, flags, local, plan.spans, None)
        n = plan.n_keep
        sel = rq["sel"]
        assert int(want["counts"][0]) == n == int(sel.counts[0].item())
        np.testing.assert_array_equal(O.to_numpy(sel.keep_abs)[:n], want["keep_abs"])
        np.testing.assert_array_equal(O.to_numpy(sel.keep_rank), want["keep_rank"])
        np.testing.assert_array_equal(O.to_numpy(sel.rel_dev).view(np.uint32), want["rel_dev"].view(np.uint32))
        ka = want["keep_abs"]
        dropped = plan.cached & (want["keep_rank"] < 0)
        # layer 1 after the repair: the kept rows fresh, every other row the cached one
        K1, V1 = O.to_numpy(rq["K"][1])[0], O.to_numpy(rq["V"][1])[0]
        np.testing.assert_array_equal(K1[:, ka], k1[:, want["keep_local"]])
        np.testing.assert_array_equal(V1[:, ka], v1[:, want["keep_local"]])
        assert (plan.cached | (want["keep_rank"] >= 0)).all()  # so every row is one of the two
        np.testing.assert_array_equal(K1[:, dropped], K1o[:, dropped])
        np.testing.assert_array_equal(V1[:, dropped], V1o[:, dropped])
        # fresh rows: layer 0 at every position, layer 27 at the kept positions (k rotated, v copied)
        for li, pos in ((0, plan.layer0_idx.astype(np.int64)), (NL - 1, ka)):
            kin = O.to_numpy(rq["proj"][li][0])[0].reshape(len(pos), H, D).transpose(1, 0, 2)
            vin = O.to_numpy(rq["proj"][li][1])[0].reshape(len(pos), H, D).transpose(1, 0, 2)
            Kl, Vl = O.to_numpy(rq["K"][li])[0], O.to_numpy(rq["V"][li])[0]
            np.testing.assert_array_equal(Kl[:, pos], O.rope(kin, pos, THETA))
            np.testing.assert_array_equal(Vl[:, pos], vin)
        # layers 2 and 27: the dropped positions' cached rows
        for li in (2, NL - 1):
            Klo, Vlo = _oracle_layer(plan, li)
            Kg, Vg = O.to_numpy(rq["K"][li])[0], O.to_numpy(rq["V"][li])[0]
            np.testing.assert_array_equal(Kg[:, dropped], Klo[:, dropped])
            np.testing.assert_array_equal(Vg[:, dropped], Vlo[:, dropped])
