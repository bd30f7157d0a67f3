"""GPU parity of the fused fresh-token RoPE kernel (ckv_rope_qkv) against the oracle: q and k
rotated bit-exactly (same correctly rounded cos/sin, same fp32 operation order), v copied, rows
placed where `rows` says, other cache rows untouched."""

import numpy as np
import pytest
import torch

from chunkkv_amd import _native, ops
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
THETA = 1e6


def _proj(rng, n, Hq, Hkv, D, bf16):
    """A fused q|k|v projection output (1, n, (Hq + 2 Hkv) D), token-major like F.linear's."""
    a = rng.standard_normal((1, n, (Hq + 2 * Hkv) * D)).astype(np.float32) * 3
    return O.f32_to_bf16_bits(a) if bf16 else a


def _split(lin, Hq, Hkv, D):
    q = lin[..., : Hq * D]
    k = lin[..., Hq * D : (Hq + Hkv) * D]
    v = lin[..., (Hq + Hkv) * D :]
    return q, k, v


def _heads(a, H, D):  # (1, n, H*D) -> (H, n, D)
    return np.ascontiguousarray(a[0].reshape(a.shape[1], H, D).transpose(1, 0, 2))


@pytest.mark.parametrize("bf16,D,Hq,Hkv", [(True, 128, 28, 4), (True, 64, 14, 2), (False, 128, 8, 2), (True, 256, 4, 1)])
def test_rope_qkv_tensor_mode_bit_exact(bf16, D, Hq, Hkv):
    rng = np.random.default_rng(D + Hq)
    n = 333
    lin = _proj(rng, n, Hq, Hkv, D, bf16)
    pos = rng.integers(0, 40000, n)
    pos[0] = 0
    lt = O.from_numpy(lin, DEV)
    q_in, k_in, v_in = _split(lt, Hq, Hkv, D)
    q_out, k_out = ops.rope_qkv(q_in, k_in, None, torch.from_numpy(pos).to(DEV), Hq, Hkv, D, THETA)
    torch.cuda.synchronize()
    qn, kn, _ = _split(lin, Hq, Hkv, D)
    want_q = O.rope(_heads(qn, Hq, D), pos, THETA)  # (Hq, n, D)
    want_k = O.rope(_heads(kn, Hkv, D), pos, THETA)
    np.testing.assert_array_equal(O.to_numpy(q_out)[0].transpose(1, 0, 2), want_q)
    np.testing.assert_array_equal(O.to_numpy(k_out)[0], want_k)


def test_rope_qkv_scatter_into_cache():
    """k and v land in the cache rows of their positions; every other row keeps its value."""
    rng = np.random.default_rng(7)
    Hq, Hkv, D, N, n = 28, 4, 128, 1000, 297
    lin = _proj(rng, n, Hq, Hkv, D, True)
    pos = np.sort(rng.choice(N, n, replace=False))
    lt = O.from_numpy(lin, DEV)
    q_in, k_in, v_in = _split(lt, Hq, Hkv, D)
    K = torch.full((1, Hkv, N, D), -3.0, dtype=torch.bfloat16, device=DEV)
    V = torch.full_like(K, -3.0)
    pt = torch.from_numpy(pos).to(DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    q_out, _ = ops.rope_qkv(q_in, k_in, v_in, pt, Hq, Hkv, D, THETA, k_out=K, v_out=V, rows=pt, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    qn, kn, vn = _split(lin, Hq, Hkv, D)
    Kw = np.full((Hkv, N, D), O.f32_to_bf16_bits(np.float32([-3.0]))[0], dtype=np.uint16)
    Vw = Kw.copy()
    Kw[:, pos] = O.rope(_heads(kn, Hkv, D), pos, THETA)
    Vw[:, pos] = _heads(vn, Hkv, D)
    np.testing.assert_array_equal(O.to_numpy(K)[0], Kw)
    np.testing.assert_array_equal(O.to_numpy(V)[0], Vw)
    np.testing.assert_array_equal(O.to_numpy(q_out)[0].transpose(1, 0, 2), O.rope(_heads(qn, Hq, D), pos, THETA))


def test_rope_qkv_flags_bad_row():
    rng = np.random.default_rng(8)
    Hq, Hkv, D, N, n = 4, 2, 64, 50, 5
    lt = O.from_numpy(_proj(rng, n, Hq, Hkv, D, True), DEV)
    q_in, k_in, v_in = _split(lt, Hq, Hkv, D)
    K = torch.zeros((1, Hkv, N, D), dtype=torch.bfloat16, device=DEV)
    V = torch.zeros_like(K)
    rows = torch.tensor([0, 1, 2, 3, N], dtype=torch.int64, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    ops.rope_qkv(q_in, k_in, v_in, rows.clone(), Hq, Hkv, D, THETA, k_out=K, v_out=V, rows=rows, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) == _native.DEVICE_ERR_RANGE
    assert int(K[0, :, 4:].count_nonzero()) == 0


def test_rope_qkv_kv_only():
    """n_q_heads = 0: k rotated and v copied into the cache rows, no q touched."""
    rng = np.random.default_rng(9)
    Hkv, D, N, n = 4, 128, 500, 123
    lin = _proj(rng, n, 0, Hkv, D, True)
    pos = np.sort(rng.choice(N, n, replace=False))
    lt = O.from_numpy(lin, DEV)
    _, k_in, v_in = _split(lt, 0, Hkv, D)
    K = torch.zeros((1, Hkv, N, D), dtype=torch.bfloat16, device=DEV)
    V = torch.zeros_like(K)
    pt = torch.from_numpy(pos).to(DEV)
    q_out, _ = ops.rope_qkv(None, k_in, v_in, pt, 0, Hkv, D, THETA, k_out=K, v_out=V, rows=pt)
    torch.cuda.synchronize()
    assert q_out is None
    _, kn, vn = _split(lin, 0, Hkv, D)
    np.testing.assert_array_equal(O.to_numpy(K)[0][:, pos], O.rope(_heads(kn, Hkv, D), pos, THETA))
    np.testing.assert_array_equal(O.to_numpy(V)[0][:, pos], _heads(vn, Hkv, D))


@pytest.mark.parametrize("D", [64, 128, 256])
def test_rope_table_matches_oracle(D):
    """ckv_rope_table equals the oracle's cos/sin (read off a rotation of unit vectors: x1 = 1,
    x2 = 0 gives y1 = cos, y2 = sin exactly): every frequency at 65,536 positions."""
    N = 1 << 16
    tab = O.to_numpy(ops.rope_table(N, D, THETA, DEV))
    x = np.zeros((1, N, D), np.float32)
    x[..., : D // 2] = 1.0
    y = O.rope(x, np.arange(N), THETA)[0]
    np.testing.assert_array_equal(tab[..., 0].view(np.uint32), y[:, : D // 2].view(np.uint32))
    np.testing.assert_array_equal(tab[..., 1].view(np.uint32), y[:, D // 2 :].view(np.uint32))


@pytest.mark.parametrize("D,Hq,Hkv", [(128, 28, 4), (64, 0, 2), (256, 2, 1)])
def test_rope_rows_far_and_negative_positions(D, Hq, Hkv):
    """The table-free path (cos/sin evaluated per token) at positions anywhere in int32, negative
    ones included, where angles reach 2^31: q and k bit-exact against the oracle, v copied."""
    rng = np.random.default_rng(D + 7 * Hq)
    n = 700
    pos = rng.integers(-(2**31), 2**31, n)
    pos[:6] = [0, 1, -1, 2**31 - 1, -(2**31), 2**20]
    lin = _proj(rng, n, Hq, Hkv, D, True)
    lt = O.from_numpy(lin, DEV)
    q_in, k_in, v_in = _split(lt, Hq, Hkv, D)
    pt = torch.from_numpy(pos).to(DEV)
    out = torch.zeros((1, Hkv, n, D), dtype=torch.bfloat16, device=DEV)
    vout = torch.zeros_like(out)
    rows = torch.arange(n, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    q, _ = ops.rope_qkv(q_in if Hq else None, k_in, v_in, pt, Hq, Hkv, D, THETA, k_out=out, v_out=vout, rows=rows,
                        err=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    qn, kn, vn = _split(lin, Hq, Hkv, D)
    np.testing.assert_array_equal(O.to_numpy(out)[0], O.rope(_heads(kn, Hkv, D), pos, THETA))
    np.testing.assert_array_equal(O.to_numpy(vout)[0], _heads(vn, Hkv, D))
    if Hq:
        want_q = O.rope(_heads(qn, Hq, D), pos, THETA)
        np.testing.assert_array_equal(O.to_numpy(q)[0], want_q.transpose(1, 0, 2))


def test_rope_qkv_with_table_identical_and_bounds():
    rng = np.random.default_rng(10)
    Hq, Hkv, D, N, n = 28, 4, 128, 900, 400
    lt = O.from_numpy(_proj(rng, n, Hq, Hkv, D, True), DEV)
    q_in, k_in, v_in = _split(lt, Hq, Hkv, D)
    pt = torch.from_numpy(np.sort(rng.choice(N, n, replace=False))).to(DEV)
    tab = ops.rope_table(N, D, THETA, DEV)
    outs = []
    for t in (None, tab):
        K = torch.zeros((1, Hkv, N, D), dtype=torch.bfloat16, device=DEV)
        V = torch.zeros_like(K)
        q, _ = ops.rope_qkv(q_in, k_in, v_in, pt, Hq, Hkv, D, THETA, k_out=K, v_out=V, rows=pt, table=t)
        outs.append((q, K, V))
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    short = ops.rope_table(int(pt.max().item()), D, THETA, DEV)  # one position short
    ops.rope_qkv(q_in, k_in, None, pt, Hq, Hkv, D, THETA, table=short, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) == _native.DEVICE_ERR_RANGE


# (bf16, D, Hkv) per shape of the k/v-only kernel: items per token = 2 Hkv D/2/VEC (VEC = 8 bf16,
# 4 fp32); 64 = one item per lane with the k/v split at lane 32, < 64 one item per lane at most,
# > 64 items strided over the wavefront.
KV_SHAPES = {
    "full_bf16_128": (True, 128, 4), "full_bf16_64": (True, 64, 8), "full_f32_128": (False, 128, 2),
    "one_bf16_128": (True, 128, 2), "one_bf16_64": (True, 64, 3), "one_f32_64": (False, 64, 1),
    "loop_bf16_128": (True, 128, 8), "loop_f32_128": (False, 128, 4),
}


@pytest.mark.parametrize("n", [157, 6145])
@pytest.mark.parametrize("row_mode", ["token", "positions", "indexed"])
@pytest.mark.parametrize("shape", list(KV_SHAPES))
def test_rope_kv_every_row_mode_and_shape(shape, row_mode, n):
    """The k/v-only launch (no q: every layer's cache write) in each shape and row mode: rows
    NULL (row = token index), rows = the positions tensor itself, rows indexed separately from
    the positions. k rotated bit-exactly, v copied, every other cache row untouched; 6145 tokens
    are more wavefronts than the chip holds at once (layer 0 of an 8k request is 8256)."""
    bf16, D, Hkv = KV_SHAPES[shape]
    rng = np.random.default_rng(sum(map(ord, shape + row_mode)) + n)
    N = 700 if n < 700 else 2 * n
    lin = _proj(rng, n, 0, Hkv, D, bf16)
    if row_mode == "positions":
        pos = np.sort(rng.choice(N, n, replace=False))
        rows = pos
    else:
        pos = rng.integers(0, 40000, n)
        pos[0] = 0
        rows = np.arange(n) if row_mode == "token" else rng.choice(N, n, replace=False)
    lt = O.from_numpy(lin, DEV)
    _, k_in, v_in = _split(lt, 0, Hkv, D)
    dt = torch.bfloat16 if bf16 else torch.float32
    K = torch.full((1, Hkv, N, D), -3.0, dtype=dt, device=DEV)
    V = torch.full_like(K, -3.0)
    pt = torch.from_numpy(pos).to(DEV)
    rt = None if row_mode == "token" else pt if row_mode == "positions" else torch.from_numpy(rows).to(DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    ops.rope_qkv(None, k_in, v_in, pt, 0, Hkv, D, THETA, k_out=K, v_out=V, rows=rt, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    _, kn, vn = _split(lin, 0, Hkv, D)
    fill = O.f32_to_bf16_bits(np.float32([-3.0]))[0] if bf16 else np.float32(-3.0)
    Kw = np.full((Hkv, N, D), fill, dtype=np.uint16 if bf16 else np.float32)
    Vw = Kw.copy()
    Kw[:, rows] = O.rope(_heads(kn, Hkv, D), pos, THETA)
    Vw[:, rows] = _heads(vn, Hkv, D)
    np.testing.assert_array_equal(O.to_numpy(K)[0], Kw)
    np.testing.assert_array_equal(O.to_numpy(V)[0], Vw)
