"""Test infrastructure only (the oracle): the reference's token-prefix hash restated.

token_hash follows src/chunkkv/store/keys.py:15-20 step for step: hashlib.sha256 fed the
prefix length as 4 little-endian bytes, then every token id as 4 little-endian bytes, one update
each. It is pinned in tests/test_token_hash.py by an independent formulation (the whole message
packed with struct and hashed in one update), by a message spelled out byte by byte, and by
FIPS 180-4's published SHA-256 digests (hashlib itself).
"""

from __future__ import annotations

import hashlib


def token_hash(tokens: list[int]) -> str:
    """keys.py:15-20."""
    h = hashlib.sha256()
    h.update(len(tokens).to_bytes(4, "little"))
    for t in tokens:
        h.update(t.to_bytes(4, "little"))
    return h.hexdigest()
