"""ORACLE — test infrastructure only (tests/, __graft_entry__.smoke(), bench.py cpu_baseline).

numpy-facing wrapper of the C restatement in oracle/ckv_oracle.c, plus small helpers to move
bf16 data between torch and numpy (bf16 travels as uint16 bit patterns). Function-by-function
citations of the reference lines are in ckv_oracle.c.

Parity status of each function (how it is pinned is in tests/test_oracle.py):
  inv_freq        pinned: fp64 closed form, exact exponents
  shift_keys      pinned: fp64 rotation (<= 1 bf16 ulp), composition/round trip at the
                  reference's own tolerances (tests/test_rerope.py:15-22), delta=0 identity
  rerope_gather   pinned: per-row equality with shift_keys + bit-exact value copies, brute force
  deviation       pinned: fp64 brute force; exact 4x scaling; zero for identical rows; torch's
                  own .sum(dim=(0,1,3)) within fp32 rounding
  select          pinned: numpy lexsort and torch stable argsort of the reference expression,
                  closed-form budgets/stats of tests/test_mlx_engine.py
  scatter_rows    pinned: brute-force Python loop on small shapes
  rope            pinned: equal positions = shift_keys by that position (bit-exact), torch's
                  own _rope/_rotate expression on the CPU within one bf16 ulp, fp64 rotation
                  within one bf16 ulp, composition rope(rope(x, a), b) ~ rope(x, a + b)
  attention_active pinned: torch's CPU scaled_dot_product_attention with the reference's boolean
                  mask and enable_gqa (the reference call itself), fp32, on small shapes
  add_rmsnorm     pinned: the transformers Qwen2RMSNorm module on the CPU after torch's own
                  residual add (bf16 and fp32, within one ulp), closed form of a constant row
  silu_mul        pinned: torch's CPU F.silu(gate) * up in bf16 (within one bf16 ulp), fp64
                  silu closed forms (silu(0) = 0, odd part x/2)
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "_build" / "libckv_oracle.so"
DT_F32, DT_BF16 = 0, 1
COUNT_N = 8

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            from oracle.build import build

            build()
        _lib = ctypes.CDLL(str(LIB_PATH))
        P, I, L, D = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_double
        sig = {
            "ckvo_inv_freq": [I, D, P],
            "ckvo_shift_keys": [P, L, P, L, I, I, I, I, ctypes.c_int32, D],
            "ckvo_rerope_gather": [P, P, L, L, P, P, I, I, I, I, I, I, D],
            "ckvo_deviation": [P, L, L, P, L, L, P, P, L, P, P, I, I, I, I, I, P, P],
            "ckvo_select": [P, P, P, P, I, P, I, I, D, P, P, P, P, P],
            "ckvo_scatter_rows": [P, P, L, P, L, L, P, L, L, P, I, I, I, I, I],
            "ckvo_rope": [P, L, L, P, L, L, P, I, I, I, I, D],
        }
        for name, args in sig.items():
            fn = getattr(_lib, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int if name != "ckvo_inv_freq" else None
    return _lib


def _p(a: np.ndarray | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if a is None else a.ctypes.data)


def dt_of(a: np.ndarray) -> int:
    if a.dtype == np.uint16:
        return DT_BF16
    if a.dtype == np.float32:
        return DT_F32
    raise TypeError(f"oracle element arrays are float32 or uint16 (bf16 bits), got {a.dtype}")


# ---- bf16 helpers --------------------------------------------------------------------------


def bf16_bits_to_f32(a: np.ndarray) -> np.ndarray:
    return (a.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even, NaN -> 0x7fc0 (torch's rule)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


def to_numpy(t) -> np.ndarray:
    """torch tensor (cpu or device) -> numpy; bf16 becomes uint16 bits."""
    import torch

    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def from_numpy(a: np.ndarray, device=None):
    import torch

    if a.dtype == np.uint16:
        t = torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)
    else:
        t = torch.from_numpy(np.ascontiguousarray(a))
    return t if device is None else t.to(device)


def as_f32(a: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(a) if a.dtype == np.uint16 else a.astype(np.float32)


# ---- restated functions --------------------------------------------------------------------


def inv_freq(head_dim: int, theta: float) -> np.ndarray:
    out = np.empty(head_dim // 2, dtype=np.float32)
    lib().ckvo_inv_freq(head_dim, float(theta), _p(out))
    return out


def shift_keys(x: np.ndarray, delta: int, theta: float) -> np.ndarray:
    """x (..., L, D) -> re-rotated copy (delta == 0 returns x itself, as the reference)."""
    if delta == 0:
        return x
    x = np.ascontiguousarray(x)
    L, D = x.shape[-2], x.shape[-1]
    heads = x.size // max(1, L * D)
    out = np.empty_like(x)
    rc = lib().ckvo_shift_keys(_p(out), L * D, _p(x), L * D, heads, L, D, dt_of(x), int(delta), float(theta))
    assert rc == 0
    return out


def rerope_gather(
    k_dst: np.ndarray, v_dst: np.ndarray, chunks_k: list, chunks_v: list, segments: np.ndarray, theta: float
) -> int:
    """k_dst/v_dst: (n_layers, H, N, D) arrays filled in place. chunks_k[c][l]: (H, L_c, D)."""
    n_layers, H, N, D = k_dst.shape
    keep = []
    tab = np.zeros((len(chunks_k), n_layers, 2), dtype=np.uint64)
    for c, (ks, vs) in enumerate(zip(chunks_k, chunks_v)):
        for l in range(n_layers):
            a, b = np.ascontiguousarray(ks[l]), np.ascontiguousarray(vs[l])
            keep += [a, b]
            tab[c, l, 0] = a.ctypes.data
            tab[c, l, 1] = b.ctypes.data
    segs = np.ascontiguousarray(segments, dtype=np.int32)
    return lib().ckvo_rerope_gather(
        _p(k_dst), _p(v_dst), H * N * D, N * D, _p(tab), _p(segs), len(segs), n_layers, H, N, D, dt_of(k_dst), float(theta)
    )


def rope(x: np.ndarray, positions: np.ndarray, theta: float) -> np.ndarray:
    """x (H, n, D) -> rows rotated to their positions (torch_engine.py:53-54, :46-51)."""
    x = np.ascontiguousarray(x)
    H, n, D = x.shape
    pos = np.ascontiguousarray(positions, dtype=np.int64)
    out = np.empty_like(x)
    rc = lib().ckvo_rope(_p(out), n * D, D, _p(x), n * D, D, _p(pos), H, n, D, dt_of(x), float(theta))
    assert rc == 0
    return out


def deviation(k: np.ndarray, v: np.ndarray, K: np.ndarray, V: np.ndarray, flags: np.ndarray, local: np.ndarray):
    """k, v: (H, n, D) fresh rows; K, V: (H, N, D) cache. Returns (diff, norm) float32 (N,)."""
    k, v, K, V = (np.ascontiguousarray(a) for a in (k, v, K, V))
    H, n, D = k.shape
    N = K.shape[1]
    diff = np.empty(N, dtype=np.float32)
    norm = np.empty(N, dtype=np.float32)
    flags = np.ascontiguousarray(flags, dtype=np.uint8)
    local = np.ascontiguousarray(local, dtype=np.int32)
    rc = lib().ckvo_deviation(
        _p(k), n * D, D, _p(v), n * D, D, _p(K), _p(V), N * D, _p(flags), _p(local), N, n, H, D, dt_of(K), _p(diff), _p(norm)
    )
    assert rc == 0
    return diff, norm


def select(diff, norm, flags, local, spans: np.ndarray, escalate_threshold: float | None):
    """Returns dict(keep_abs, keep_local, rel_dev, escalated, counts) like ckv_select."""
    N = len(diff)
    spans = np.ascontiguousarray(spans, dtype=np.int32).reshape(-1, 4)
    C = len(spans)
    diff = np.ascontiguousarray(diff, dtype=np.float32)
    norm = np.ascontiguousarray(norm, dtype=np.float32)
    flags = np.ascontiguousarray(flags, dtype=np.uint8)
    local = np.ascontiguousarray(local, dtype=np.int32)
    keep_abs = np.zeros(N + 1, dtype=np.int64)
    keep_local = np.zeros(N + 1, dtype=np.int64)
    rel = np.zeros(max(C, 1), dtype=np.float32)
    esc = np.zeros(max(C, 1), dtype=np.uint8)
    counts = np.zeros(COUNT_N, dtype=np.int32)
    has = escalate_threshold is not None
    rc = lib().ckvo_select(
        _p(diff), _p(norm), _p(flags), _p(local), N, _p(spans), C, int(has), float(escalate_threshold) if has else 0.0,
        _p(keep_abs), _p(keep_local), _p(rel), _p(esc), _p(counts),
    )
    assert rc == 0
    n = int(counts[0])
    keep_rank = np.full(N, -1, dtype=np.int32)
    keep_rank[keep_abs[:n]] = np.arange(n, dtype=np.int32)
    return dict(keep_abs=keep_abs[:n], keep_local=keep_local[:n], keep_rank=keep_rank, rel_dev=rel[:C],
                escalated=esc[:C], counts=counts)


def scatter_rows(K: np.ndarray, V: np.ndarray, k: np.ndarray, v: np.ndarray, rows: np.ndarray) -> int:
    """K, V: (H, N, D) in place; k, v: (H, n, D); rows int64 (n,)."""
    H, N, D = K.shape
    n = k.shape[1]
    k, v = np.ascontiguousarray(k), np.ascontiguousarray(v)
    rows = np.ascontiguousarray(rows, dtype=np.int64)
    return lib().ckvo_scatter_rows(_p(K), _p(V), N * D, _p(k), n * D, D, _p(v), n * D, D, _p(rows), n, N, H, D, dt_of(K))


def attention_active(q: np.ndarray, K: np.ndarray, V: np.ndarray, positions: np.ndarray, scale: float | None = None):
    """Masked GQA attention in fp64 (torch_engine.py:157 mask, :68-72 SDPA with enable_gqa).

    q: (Hq, n, D); K, V: (Hkv, N, D) (float32, or uint16 bf16 bits); positions: (n,) ints.
    Query i of head h attends to rows j <= positions[i] of KV head h // (Hq // Hkv).
    Returns (n, Hq, D) float64, token-major like ckv_attention_active."""
    q, K, V = (as_f32(np.asarray(a)).astype(np.float64) for a in (q, K, V))
    Hq, n, D = q.shape
    Hkv, N, _ = K.shape
    G = Hq // Hkv
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    pos = np.asarray(positions, dtype=np.int64)
    visible = pos[:, None] >= np.arange(N)[None, :]
    out = np.empty((n, Hq, D))
    for h in range(Hq):
        s = (q[h] @ K[h // G].T) * scale
        s = np.where(visible, s, -np.inf)
        s -= s.max(axis=1, keepdims=True)
        p = np.exp(s)
        out[:, h] = (p @ V[h // G]) / p.sum(axis=1, keepdims=True)
    return out


def _round_to(x: np.ndarray, bf16: bool) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    return bf16_bits_to_f32(f32_to_bf16_bits(x)) if bf16 else x


def add_rmsnorm(h: np.ndarray, delta: np.ndarray | None, weight: np.ndarray, eps: float):
    """Residual add + RMSNorm of the rows of h (torch_engine.py:71-72 and :113 / :75 through the
    model's RMSNorm modules): s = dtype(h + delta); y = dtype(w * dtype(s * rsqrt(mean(s^2) + eps))).

    h, delta: (rows, hidden) float32 or uint16 bf16 bits; weight (hidden,) of the same kind.
    The sum of squares is taken in fp64 and rounded once to fp32, then scaled by fl32(1/hidden)
    in fp32, eps added in fp32, and rsqrt evaluated in fp64 and rounded once.
    Returns (s, y) in the input representation."""
    bf16 = h.dtype == np.uint16
    s = as_f32(h)
    if delta is not None:
        s = _round_to(s + as_f32(delta), bf16)
    ss = np.float32(np.sum(s.astype(np.float64) ** 2, axis=-1, keepdims=True))
    var = (ss * np.float32(1.0 / np.float32(h.shape[-1]))).astype(np.float32)
    r = (1.0 / np.sqrt((var + np.float32(eps)).astype(np.float32).astype(np.float64))).astype(np.float32)
    y = _round_to(as_f32(weight)[None, :] * _round_to(s * r, bf16), bf16)
    if bf16:
        return f32_to_bf16_bits(s), f32_to_bf16_bits(y)
    return s, y


def silu_mul(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """dtype(dtype(silu(gate)) * up), silu(x) = x / (1 + exp(-x)) in fp64 rounded once to fp32,
    the SiLU-gated MLP product (torch_engine.py:72 via the model's MLP). Inputs and output in the
    input representation (float32 or uint16 bf16 bits)."""
    bf16 = gate.dtype == np.uint16
    g = as_f32(gate).astype(np.float64)
    with np.errstate(over="ignore"):
        silu = (g / (1.0 + np.exp(-g))).astype(np.float32)
    out = _round_to(_round_to(silu, bf16) * as_f32(up), bf16)
    return f32_to_bf16_bits(out) if bf16 else out
