"""Native token-prefix hashes (ckv_token_hash_prefixes, chunkkv_amd.keys) against the reference's
token_hash (src/chunkkv/store/keys.py:15-20, restated in oracle/keys_ref.py), byte for byte, on
both SHA-256 paths (x86 SHA extensions where the CPU has them, and the portable one); plus the
oracle's own pins. Host code only: these tests need no GPU."""

import hashlib
import os
import struct
import time

import numpy as np
import pytest

from chunkkv_amd import keys
from oracle import keys_ref as R


@pytest.fixture(params=["auto", "portable"])
def sha_path(request, monkeypatch):
    if request.param == "portable":
        monkeypatch.setenv("CKV_SHA256_PORTABLE", "1")
    else:
        monkeypatch.delenv("CKV_SHA256_PORTABLE", raising=False)
    return request.param


# ---- the oracle's pins ----------------------------------------------------------------------


def test_oracle_matches_bulk_formulation():
    """One struct-packed message in one update equals the reference's per-token updates."""
    rng = np.random.default_rng(1)
    for n in (0, 1, 13, 14, 15, 16, 200):
        toks = rng.integers(0, 2**32, n).tolist()
        bulk = hashlib.sha256(struct.pack(f"<I{n}I", n, *toks)).hexdigest()
        assert R.token_hash(toks) == bulk


def test_oracle_message_spelled_out():
    msg = bytes([2, 0, 0, 0, 1, 0, 0, 0, 0xFF, 0xFF, 0xFF, 0xFF])  # LE32(2), LE32(1), LE32(2^32 - 1)
    assert R.token_hash([1, 2**32 - 1]) == hashlib.sha256(msg).hexdigest()
    # FIPS 180-4 example digests pin hashlib itself
    assert hashlib.sha256(b"abc").hexdigest() == "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"
    assert hashlib.sha256(b"").hexdigest() == "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855"


# ---- native against the oracle ------------------------------------------------------------------


@pytest.mark.parametrize("n", list(range(0, 34)) + [47, 48, 49, 100, 1000, 4096, 32832])
def test_token_hash_every_padding_case(sha_path, n):
    """Lengths around every block boundary (message = 4 + 4n bytes; the padding takes one or two
    blocks) and long messages, ids over the full 32-bit range."""
    rng = np.random.default_rng(n)
    toks = rng.integers(0, 2**32, n).tolist()
    if n:
        toks[0], toks[-1] = 0, 2**32 - 1
    assert keys.token_hash(toks) == R.token_hash(toks)


@pytest.mark.parametrize("n_threads", [1, 4, 0])
def test_prefixes_of_a_32k_request(sha_path, n_threads):
    """Every segment start of a 32,832-token request (128 segments of 256 + the query), plus
    0, the full length, duplicates, out of order."""
    rng = np.random.default_rng(7 + n_threads)
    toks = rng.integers(0, 152064, 32832).tolist()
    starts = [256 * i for i in range(129)] + [32832, 0, 5, 5, 31000, 17]
    rng.shuffle(starts)
    got = keys.token_hash_prefixes(toks, starts, n_threads=n_threads)
    assert got == [R.token_hash(toks[:s]) for s in starts]


def test_prefix_slice_semantics():
    """starts as Python slices of the token list, like the reference's tokens[:s]."""
    toks = list(range(1, 40))
    starts = [-3, -100, 0, 39, 50, 1000]
    assert keys.token_hash_prefixes(toks, starts) == [R.token_hash(toks[:s]) for s in starts]
    assert keys.token_hash_prefixes(np.array(toks), [7]) == [R.token_hash(toks[:7])]


def test_out_of_range_ids_raise_like_the_reference():
    for bad in (-1, 2**32):
        toks = [5, 6, bad, 7]
        with pytest.raises(OverflowError):
            R.token_hash(toks)
        with pytest.raises(OverflowError):
            keys.token_hash(toks)
        with pytest.raises(OverflowError):
            keys.token_hash_prefixes(toks, [1, 4])
        # an id beyond the longest prefix is never encoded, by the reference either
        assert keys.token_hash_prefixes(toks, [0, 2]) == [R.token_hash(toks[:0]), R.token_hash(toks[:2])]


def test_prefixes_faster_than_the_reference_loop():
    """The 128 segment prefixes of a 32,832-token request: the reference's per-token loop against
    one native call (the list conversion included)."""
    rng = np.random.default_rng(3)
    toks = rng.integers(0, 152064, 32832).tolist()
    starts = [256 * i for i in range(128)]
    t0 = time.perf_counter()
    want = [R.token_hash(toks[:s]) for s in starts]
    t_ref = time.perf_counter() - t0
    t0 = time.perf_counter()
    got = keys.token_hash_prefixes(toks, starts)
    t_nat = time.perf_counter() - t0
    print(f"reference loop {t_ref * 1e3:.1f} ms, native {t_nat * 1e3:.2f} ms ({t_ref / t_nat:.0f}x), "
          f"{os.cpu_count()} CPUs")
    assert got == want
    assert t_nat < t_ref / 5
