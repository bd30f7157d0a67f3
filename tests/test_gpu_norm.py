"""GPU parity of the fused decoder elementwise kernels (ckv_add_rmsnorm, ckv_silu_mul) with the
oracle and with the model's own torch modules on the device.

Bar: the residual sum (one rounding of an exact sum) is bit-exact. The normalised row and the
gated product are floating point: the fp32 sum order of the squares and the rsqrt/exp routines
are the kernel's own, so an intermediate bf16 rounding can land one ulp away; the weight (or
up) factor then scales that ulp before the last rounding, so the bar is two bf16 ulps, with at
most 1% of elements differing at all; fp32 within 2e-6 relative.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from chunkkv_amd import ops
from oracle import oracle as O
from tests.helpers import bf16_ulp_distance

pytestmark = pytest.mark.gpu
DEV = "cuda"
EPS = 1e-6


def _inputs(seed, rows, hidden, bf16):
    rng = np.random.default_rng(seed)
    conv = O.f32_to_bf16_bits if bf16 else (lambda a: a)
    h = conv((rng.standard_normal((rows, hidden)) * 3).astype(np.float32))
    d = conv(rng.standard_normal((rows, hidden)).astype(np.float32))
    w = conv(rng.uniform(0.5, 2.0, hidden).astype(np.float32))
    return h, d, w


def _close(got, want, bf16):
    if bf16:
        dist = bf16_ulp_distance(got, want)
        assert dist.max() <= 2 and (dist > 0).mean() < 0.01, (dist.max(), (dist > 0).mean())
    else:
        np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-30)


@pytest.mark.parametrize(
    "rows,hidden,bf16",
    [
        (2976, 3584, True),  # Qwen2.5-7B, the kept rows of the 8k request
        (1, 3584, True),  # one decode token
        (7, 896, True),  # Qwen2.5-0.5B
        (3, 8192, True),  # widest row (4 vectors per thread)
        (5, 8, True),  # one vector per row
        (9, 640, False),  # fp32 model
        (2, 4096, False),  # widest fp32 row
    ],
)
def test_add_rmsnorm_matches_oracle(rows, hidden, bf16):
    h, d, w = _inputs(rows * 7 + hidden, rows, hidden, bf16)
    s_want, y_want = O.add_rmsnorm(h, d, w, EPS)
    ht, dt, wt = (O.from_numpy(a, DEV) for a in (h, d, w))
    s, y = ops.add_rmsnorm(ht, dt, wt, EPS)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(O.to_numpy(s), s_want)
    _close(O.to_numpy(y), y_want, bf16)
    assert torch.equal(ht, O.from_numpy(h, DEV))  # input untouched without h_out=h
    # no residual
    _, y0 = ops.add_rmsnorm(ht, None, wt, EPS)
    _close(O.to_numpy(y0), O.add_rmsnorm(h, None, w, EPS)[1], bf16)


def test_add_rmsnorm_in_place_matches_torch_modules():
    """In place (h_out = h), as the engine runs it, against the model's own modules on the device:
    h + delta and Qwen2RMSNorm."""
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RMSNorm

    h, d, w = _inputs(3, 300, 3584, True)
    ht, dt, wt = (O.from_numpy(a, DEV) for a in (h, d, w))
    m = Qwen2RMSNorm(3584, eps=EPS).to(DEV, torch.bfloat16)
    with torch.no_grad():
        m.weight.copy_(wt)
        s_want = ht[None] + dt[None]
        y_want = m(s_want)
    s, y = ops.add_rmsnorm(ht[None], dt[None], wt, EPS, h_out=ht[None])
    assert s.data_ptr() == ht.data_ptr()
    assert torch.equal(ht[None], s_want)
    _close(O.to_numpy(y[0]), O.to_numpy(y_want[0]), True)


@pytest.mark.parametrize("rows,width,bf16", [(300, 18944, True), (1, 18944, True), (11, 4864, True), (6, 1024, False)])
def test_silu_mul_matches_oracle(rows, width, bf16):
    rng = np.random.default_rng(rows + width)
    conv = O.f32_to_bf16_bits if bf16 else (lambda a: a)
    g = conv((rng.standard_normal((rows, width)) * 4).astype(np.float32))
    u = conv(rng.standard_normal((rows, width)).astype(np.float32))
    got = ops.silu_mul(O.from_numpy(g, DEV), O.from_numpy(u, DEV))
    torch.cuda.synchronize()
    _close(O.to_numpy(got), O.silu_mul(g, u), bf16)


def test_silu_mul_full_size_and_stacked_views_match_torch():
    """The 8k request's MLP shape (2976 x 18944) against torch's F.silu(gate) * up on the device,
    and the same product from the two halves of one stacked gate|up tensor (strided rows)."""
    torch.manual_seed(0)
    gu = (torch.randn(1, 2976, 2 * 18944, device=DEV) * 3).to(torch.bfloat16)
    gate, up = gu[..., :18944], gu[..., 18944:]
    got = ops.silu_mul(gate, up)
    want = F.silu(gate) * up
    dist = bf16_ulp_distance(O.to_numpy(got), O.to_numpy(want))
    assert dist.max() <= 2 and (dist > 0).mean() < 0.01
    assert torch.equal(ops.silu_mul(gate.contiguous(), up.contiguous()), got)
    # more rows than the kernel's grid height: the row loop covers the rest
    g2 = torch.randn(70000, 16, device=DEV).to(torch.bfloat16)
    u2 = torch.randn(70000, 16, device=DEV).to(torch.bfloat16)
    d2 = bf16_ulp_distance(O.to_numpy(ops.silu_mul(g2, u2)), O.to_numpy(F.silu(g2) * u2))
    assert d2.max() <= 2


def test_fused_ops_reject_bad_layouts():
    h = torch.zeros(4, 100, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        ops.add_rmsnorm(h, None, torch.zeros(100, dtype=torch.bfloat16, device=DEV), EPS)  # 100 % 8
    h = torch.zeros(4, 128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        ops.add_rmsnorm(h, None, torch.zeros(128, dtype=torch.float32, device=DEV), EPS)  # weight dtype
    g = torch.zeros(4, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        ops.silu_mul(g[:, 1:57], g[:, 1:57])  # rows not 16-byte aligned
