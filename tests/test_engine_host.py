"""Host-side pieces of HipEngine that need no GPU: the one-copy stacking of projection weights."""

import torch

from chunkkv_amd.engine import _stack_params


def _linears(bias_pattern, seed=0):
    g = torch.Generator().manual_seed(seed)
    mods = []
    for rows, has_bias in zip((6, 2, 2), bias_pattern):
        m = torch.nn.Linear(5, rows, bias=has_bias)
        with torch.no_grad():
            m.weight.copy_(torch.randn(m.weight.shape, generator=g))
            if has_bias:
                m.bias.copy_(torch.randn(rows, generator=g))
        mods.append(m)
    return mods


def test_stacked_weights_are_stored_once_and_modules_unchanged():
    mods = _linears((True, True, True))
    x = torch.randn(3, 5)
    before = [m(x) for m in mods]
    w = _stack_params(mods, "weight")
    b = _stack_params(mods, "bias")
    assert w.shape == (10, 5) and b.shape == (10,)
    # the modules now read their rows of the stack: same outputs, same storage
    for m, y in zip(mods, before):
        assert torch.equal(m(x), y)
        assert m.weight.untyped_storage().data_ptr() == w.untyped_storage().data_ptr()
        assert m.bias.untyped_storage().data_ptr() == b.untyped_storage().data_ptr()
    assert torch.equal(torch.nn.functional.linear(x, w, b), torch.cat(before, -1))
    # a second stacking of the same model views the first stack instead of copying it
    w2, b2 = _stack_params(mods, "weight"), _stack_params(mods, "bias")
    assert w2.data_ptr() == w.data_ptr() and torch.equal(w2, w)
    assert b2.data_ptr() == b.data_ptr() and torch.equal(b2, b)
    # writes through a module's parameter (e.g. load_state_dict) reach the stack
    with torch.no_grad():
        mods[1].weight.fill_(3.0)
    assert (w[6:8] == 3.0).all()


def test_stacked_bias_with_missing_entries_is_zero_filled():
    mods = _linears((True, False, True), seed=1)
    x = torch.randn(4, 5)
    before = [m(x) for m in mods]
    w, b = _stack_params(mods, "weight"), _stack_params(mods, "bias")
    assert mods[1].bias is None and torch.equal(b[6:8], torch.zeros(2))
    assert torch.equal(torch.nn.functional.linear(x, w, b), torch.cat(before, -1))
    assert _stack_params(_linears((False, False, False)), "bias") is None
