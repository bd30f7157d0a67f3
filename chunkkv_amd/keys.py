"""Token-prefix hashes of the reuse gate and the KV store on the library's native SHA-256.

The reference hashes each prefix with one Python ``update`` per token
(src/chunkkv/store/keys.py:15-20): ``sha256(LE32(len) || LE32(t_0) || ...)``, called once per
segment as ``token_hash(req.tokens[:seg.start])`` by ``ReuseGate.decide``
(src/chunkkv/gate/gate.py:42) and again per stored segment by ``ChunkReuseRuntime.prefill``
(src/chunkkv/runtime.py:89). ``token_hash`` is a drop-in for the reference function;
``token_hash_prefixes`` hashes every prefix a request needs in one native call (prefixes spread
over host threads), so a caller computes them once per request. Both are host code: no GPU.
"""

from __future__ import annotations

import ctypes

import numpy as np

from chunkkv_amd import _native
from chunkkv_amd._native import check, lib


def _as_tokens(tokens) -> np.ndarray:
    a = np.asarray(tokens)
    if a.ndim != 1:
        a = a.reshape(-1)
    if a.dtype != np.int64:
        a = a.astype(np.int64) if a.size else np.zeros(0, dtype=np.int64)
    return np.ascontiguousarray(a)


def _digests(arr: np.ndarray, starts: np.ndarray, n_threads: int) -> bytes:
    out = ctypes.create_string_buffer(32 * len(starts))
    st = lib().ckv_token_hash_prefixes(arr.ctypes.data if arr.size else None, len(arr),
                                       starts.ctypes.data if starts.size else None, len(starts), out, int(n_threads))
    if st == _native.CKV_ERR_OUT_OF_RANGE:
        # the reference's int.to_bytes(4, "little") raises OverflowError for such an id
        bad = arr[: int(starts.max()) if starts.size else 0]
        if ((bad < 0) | (bad > 0xFFFFFFFF)).any():
            raise OverflowError("token id outside [0, 2**32) cannot be encoded in 4 bytes")
    check(st, "ckv_token_hash_prefixes")
    return out.raw


def token_hash(tokens) -> str:
    """sha256 hexdigest of LE32(len(tokens)) followed by each token as LE32, like the reference's
    keys.token_hash (OverflowError for an id outside [0, 2**32))."""
    arr = _as_tokens(tokens)
    return _digests(arr, np.array([len(arr)], dtype=np.int64), 1).hex()


def token_hash_prefixes(tokens, starts, n_threads: int = 0) -> list[str]:
    """[token_hash(tokens[:s]) for s in starts] in one native call. starts follow Python slice
    semantics (negative counts from the end, beyond the end means the whole list)."""
    arr = _as_tokens(tokens)
    n = len(arr)
    s = np.array([len(range(n)[: int(x)]) for x in starts], dtype=np.int64)
    raw = _digests(arr, s, n_threads)
    return [raw[32 * i : 32 * (i + 1)].hex() for i in range(len(s))]
