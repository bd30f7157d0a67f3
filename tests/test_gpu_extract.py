"""GPU parity of the store-put extraction (ckv_extract_chunks): every layer of every requested
segment copied bit-exactly, each segment into its own buffer, in one launch."""

import ctypes

import numpy as np
import pytest
import torch

from chunkkv_amd import _native, ops
from chunkkv_amd.engine import HipEngine
from chunkkv_amd.types import BlendConfig, Placement
from tests.helpers import StubTokenizer, tiny_qwen2

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 128), (torch.float32, 64)])
def test_extract_matches_slices(dtype, D):
    g = torch.Generator(device=DEV).manual_seed(3)
    L, H, N = 3, 4, 500
    K = torch.randn((L, 1, H, N, D), generator=g, device=DEV).to(dtype)
    V = torch.randn((L, 1, H, N, D), generator=g, device=DEV).to(dtype)
    spans = [(0, 1), (0, N), (17, 333), (N - 1, N), (10, 10), (250, 266)]
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    bufs = ops.extract_chunks(K, V, spans, err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    for (s, e), b in zip(spans, bufs):
        assert b.shape == (2, L, 1, H, e - s, D)
        for l in range(L):
            assert b[0, l].is_contiguous() and torch.equal(b[0, l], K[l][:, :, s:e])
            assert torch.equal(b[1, l], V[l][:, :, s:e])


def test_extract_flags_span_past_the_cache():
    """The host wrapper rejects bad spans; the device check covers callers of the C entry."""
    L, H, N, D = 2, 2, 40, 64
    K = torch.zeros((L, 1, H, N, D), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        ops.extract_chunks(K, K.clone(), [(30, 41)])
    dst = torch.zeros((2, L, 1, H, 11, D), dtype=torch.bfloat16, device=DEV)
    tab = torch.tensor([dst.data_ptr()], dtype=torch.int64, device=DEV)
    spans = torch.tensor([30, 11], dtype=torch.int32, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    rc = _native.lib().ckv_extract_chunks(K.data_ptr(), K.data_ptr(), H * N * D, N * D, tab.data_ptr(), spans.data_ptr(),
                                          1, 11, L, H, N, D, _native.DTYPE_BF16, err.data_ptr(),
                                          ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert rc == 0 and int(err.item()) == _native.DEVICE_ERR_RANGE
    assert int(dst.count_nonzero()) == 0


def test_prefill_result_chunk_uses_one_launch_and_matches_copies():
    """PrefillResult.chunk / chunks of a HipEngine result equal the reference's per-layer
    `.contiguous()` copies (base.py:55-60), and the stored chunk works as a placement again."""
    gpu = tiny_qwen2(layers=3, hidden=512, heads=4, kv=4, inter=1024, vocab=512, seed=4, dtype=torch.bfloat16).to(DEV)
    eng = HipEngine(gpu, StubTokenizer())
    rng = np.random.default_rng(4)
    toks = rng.integers(1, 511, 96).tolist()
    res = eng.prefill(toks)
    assert res.extract is not None
    got = res.chunks([(0, 40), (40, 96)])
    for c, (s, e) in zip(got, [(0, 40), (40, 96)]):
        assert c.start == s and c.length == e - s
        for l in range(3):
            assert torch.equal(c.keys[l], res.keys[l][:, :, s:e].contiguous())
            assert torch.equal(c.values[l], res.values[l][:, :, s:e].contiguous())
            assert c.keys[l].nbytes == res.keys[l][:, :, s:e].contiguous().nbytes
    one = res.chunk(40, 96)
    assert all(torch.equal(a, b) for a, b in zip(one.keys, got[1].keys))
    # the extracted chunk is reusable at a new offset
    out = eng.prefill(toks[40:96] + toks[:8], [Placement(one, 0)], BlendConfig(recompute_ratio=0.3))
    assert out.stats["cached_tokens"] == 56
