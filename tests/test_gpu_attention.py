"""GPU parity of the position-masked GQA attention kernel (ckv_attention_active) against the
fp64 oracle and against torch's own SDPA call with the reference's boolean mask.

Tolerance: bf16 inputs and output; the softmax weights are rounded to bf16 before the second
product (relative error 2^-9 per weight), so with N(0, 1) inputs the output is within
1e-2 absolute of the exact fp64 value (the same bound holds for torch's fused bf16 SDPA).
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from chunkkv_amd import _native, ops
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
ATOL = 1e-2


def _case(seed, Hq, Hkv, D, N, n, sorted_=True, with_ends=True):
    rng = np.random.default_rng(seed)
    q = O.f32_to_bf16_bits(rng.standard_normal((Hq, n, D)).astype(np.float32))
    K = O.f32_to_bf16_bits(rng.standard_normal((Hkv, N, D)).astype(np.float32))
    V = O.f32_to_bf16_bits(rng.standard_normal((Hkv, N, D)).astype(np.float32))
    pos = rng.choice(N, n, replace=False) if n <= N else rng.integers(0, N, n)
    if with_ends and n >= 2:
        pos[0], pos[-1] = 0, N - 1
    pos = np.sort(pos) if sorted_ else pos
    return q, K, V, pos.astype(np.int64)


def _run(q, K, V, pos):
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = ops.attention_active(O.from_numpy(q, DEV)[None], O.from_numpy(K, DEV)[None], O.from_numpy(V, DEV)[None],
                               torch.from_numpy(pos).to(DEV), err=err)
    torch.cuda.synchronize()
    return out, int(err.item())


@pytest.mark.parametrize(
    "Hq,Hkv,D,N,n",
    [
        (28, 4, 128, 8256, 2976),  # Qwen2.5-7B layer >= 2 of the 8k request
        (28, 4, 128, 1000, 1000),  # every position active (plain causal)
        (14, 2, 64, 1056, 200),  # Qwen2.5-0.5B heads
        (8, 1, 128, 77, 1),  # one query, partial tile
        (4, 4, 64, 130, 129),  # no grouping, ragged tiles
        (7, 7, 128, 64, 3),  # exactly one tile
    ],
)
def test_attention_matches_oracle(Hq, Hkv, D, N, n):
    q, K, V, pos = _case(Hq * 1000 + N, Hq, Hkv, D, N, n)
    out, e = _run(q, K, V, pos)
    assert e == 0
    got = out[0].float().cpu().numpy()
    sub = slice(None) if n <= 600 else np.sort(np.random.default_rng(0).choice(n, 600, replace=False))
    want = O.attention_active(q[:, sub], K, V, pos[sub])
    np.testing.assert_allclose(got[sub], want, atol=ATOL, rtol=0)


def test_attention_unsorted_positions_and_matches_torch_sdpa():
    """Positions in any order give the same rows; the result agrees with torch's SDPA on the
    reference's boolean mask with the KV heads expanded."""
    Hq, Hkv, D, N, n = 28, 4, 128, 700, 300
    q, K, V, pos = _case(5, Hq, Hkv, D, N, n, sorted_=False)
    out, e = _run(q, K, V, pos)
    assert e == 0
    perm = np.argsort(pos)
    out2, _ = _run(np.ascontiguousarray(q[:, perm]), K, V, pos[perm])
    assert torch.equal(out[0][torch.from_numpy(perm).to(DEV)], out2[0])
    qt, Kt, Vt = (O.from_numpy(a, DEV)[None] for a in (q, K, V))
    p = torch.from_numpy(pos).to(DEV)
    mask = p[:, None] >= torch.arange(N, device=DEV)[None, :]
    ref = F.scaled_dot_product_attention(qt, Kt.repeat_interleave(7, 1), Vt.repeat_interleave(7, 1), attn_mask=mask)
    torch.testing.assert_close(out[0].float(), ref[0].transpose(0, 1).float(), atol=2 * ATOL, rtol=0)


def test_attention_flags_out_of_range_position():
    q, K, V, pos = _case(9, 4, 2, 64, 50, 10)
    pos[3] = 50
    _, e = _run(q, K, V, pos)
    assert e == _native.DEVICE_ERR_RANGE


def test_attention_strided_query_view():
    """q as the transposed view of a token-major projection output (rows contiguous)."""
    Hq, Hkv, D, N, n = 28, 4, 128, 300, 123
    q, K, V, pos = _case(3, Hq, Hkv, D, N, n)
    qt = O.from_numpy(np.ascontiguousarray(q.transpose(1, 0, 2)), DEV)[None].transpose(1, 2)  # (1, Hq, n, D) view
    assert not qt.is_contiguous()
    out = ops.attention_active(qt, O.from_numpy(K, DEV)[None], O.from_numpy(V, DEV)[None], torch.from_numpy(pos).to(DEV))
    ref, _ = _run(q, K, V, pos)
    assert torch.equal(out, ref)


@pytest.mark.parametrize("Hq,Hkv,D,N,n", [
    (28, 4, 128, 8256, 1),  # decode: grouped rows (7 query heads of a KV head per workgroup)
    (28, 4, 128, 5000, 3),  # grouped, 21 rows
    (16, 2, 128, 777, 16),  # grouped, exactly one workgroup of rows (16 x 8), ragged last split
    (14, 2, 64, 3001, 1),   # grouped at head_dim 64 (Qwen2.5-0.5B decode), ragged last tile
    (14, 2, 64, 3000, 40),  # 280 rows: token rows per query head, split
    (8, 8, 64, 3000, 2),    # no grouping (one query head per KV head): token rows, split
])
def test_attention_split_launch_matches_oracle_and_unsplit(Hq, Hkv, D, N, n):
    """Decode-like shapes split the cache range over workgroups and merge: same result as the
    unsplit launch (up to the merge's fp32 rounding) and the oracle. Launches whose queries share
    KV heads and fit one workgroup put the group's query heads in one workgroup's rows."""
    q, K, V, pos = _case(N + n, Hq, Hkv, D, N, n, with_ends=False)
    pos[-1] = N - 1
    assert _native.lib().ckv_attention_workspace_bytes(n, N, Hq, D, None, None) > 0
    args = (O.from_numpy(q, DEV)[None], O.from_numpy(K, DEV)[None], O.from_numpy(V, DEV)[None], torch.from_numpy(pos).to(DEV))
    split = ops.attention_active(*args)
    whole = ops.attention_active(*args, split=False)
    torch.cuda.synchronize()
    torch.testing.assert_close(split.float(), whole.float(), atol=4e-3, rtol=0)
    np.testing.assert_allclose(split[0].float().cpu().numpy(), O.attention_active(q, K, V, pos), atol=ATOL, rtol=0)
