"""ORACLE — test infrastructure only (tests/, __graft_entry__.smoke(), bench.py cpu_baseline).

A CPU restatement of the reference blend prefill, src/chunkkv/engine/torch_engine.py:80-178,
with base.py:63-73 (plan_positions) and :167-176 (stats), written against a Hugging Face
Qwen2-style model. It shares no code with the chunkkv_amd package. The torch op sequence is the
reference's; the only deliberate difference is ``tie_stable`` (default True): the top-k argsort
keeps index order among equal deviations, the tie rule the HIP selection implements (the
reference's unstable argsort leaves it open).

Pinned by tests/test_engine_oracle.py: no-cache prefill == the HF forward (the reference's
tests/test_torch_engine.py:36-41), recompute_ratio=1.0 == the no-cache forward (KL < 1e-4,
:52-65), same-position exact reuse == the first prefill (:44-49), and the closed-form
prefill_token_equiv values of tests/test_mlx_engine.py:29,39,57,83,99.

``repair_step`` restates only the KV-repair ops of one request (base_kv for every layer,
layer-1 deviation/selection, per-layer scatter) on given fresh K/V; bench.py times it on the
host's cores as the CPU baseline.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


class BlendDefaults:
    """BlendConfig defaults (base.py:36-43)."""

    recompute_ratio = 0.15
    n_sink = 2
    full_first_layer = True
    escalate_threshold = None


def reference_inv_freq(theta: float, head_dim: int, device="cpu") -> torch.Tensor:
    """torch_engine.py:33 as torch evaluates it (fp32 pow)."""
    return theta ** (-torch.arange(0, head_dim, 2, device=device, dtype=torch.float32) / head_dim)


def _rotate(x, angles):
    half = x.shape[-1] // 2
    c, s = angles.cos(), angles.sin()
    xf = x.float()
    a, b = xf[..., :half], xf[..., half:]
    return torch.cat([a * c - b * s, a * s + b * c], dim=-1).to(x.dtype)


def shift_keys(keys, delta, inv_freq):
    """torch_engine.py:56-59."""
    if delta == 0:
        return keys
    return _rotate(keys, (delta * inv_freq)[None, :].expand(keys.shape[-2], -1))


def plan_positions(n, placements, n_sink):
    """base.py:63-73."""
    cached, exact, sink = [False] * n, [False] * n, [False] * n
    for p in placements:
        for i in range(p.start, p.start + p.chunk.keys[0].shape[2]):
            cached[i] = True
            if p.exact:
                exact[i] = True
            elif i < p.start + n_sink:
                sink[i] = True
    return cached, exact, sink


def base_kv(placements, li, N, n_kv, head_dim, dtype, inv_freq):
    """torch_engine.py:96-103."""
    K = torch.zeros((1, n_kv, N, head_dim), dtype=dtype)
    V = torch.zeros_like(K)
    for p in placements:
        L = p.chunk.keys[0].shape[2]
        K[:, :, p.start : p.start + L] = shift_keys(p.chunk.keys[li].to(dtype), p.start - p.chunk.start, inv_freq)
        V[:, :, p.start : p.start + L] = p.chunk.values[li].to(dtype)
    return K, V


def layer1_selection(k, v, K, V, active, cached, sink, placements, config, tie_stable=True):
    """torch_engine.py:117-147. Returns (keep_abs, chunk_stats, diff, norm)."""
    N = cached.numel()
    d_act = ((k - K[:, :, active]).float() ** 2).sum(dim=(0, 1, 3))
    d_act += ((v - V[:, :, active]).float() ** 2).sum(dim=(0, 1, 3))
    n_act = (k.float() ** 2).sum(dim=(0, 1, 3)) + (v.float() ** 2).sum(dim=(0, 1, 3))
    diff = torch.zeros(N)
    norm = torch.zeros(N)
    diff[active] = d_act
    norm[active] = n_act
    keep = (~cached) | sink
    pool = torch.zeros(N, dtype=torch.bool)
    budget = 0
    stats = []
    for p in placements:
        if p.exact:
            continue
        L = p.chunk.keys[0].shape[2]
        rel = (diff[p.start : p.start + L].sum() / norm[p.start : p.start + L].sum()).item()
        ratio = config.recompute_ratio if p.ratio is None else p.ratio
        escalated = config.escalate_threshold is not None and rel > config.escalate_threshold
        if escalated:
            keep[p.start : p.start + L] = True
        elif ratio > 0:
            pool[p.start : p.start + L] = True
            budget += int(round(ratio * L))
        stats.append({"start": p.start, "length": L, "rel_dev": rel, "escalated": escalated})
    budget = min(budget, int((pool & ~keep).sum().item()))
    if budget > 0:
        top = torch.argsort(-torch.where(pool & ~keep, diff, torch.full_like(diff, -1.0)), stable=tie_stable)[:budget]
        keep[top] = True
    return keep.nonzero().squeeze(1), stats, diff, norm


@torch.inference_mode()
def prefill(model, tokens, placements=None, config=None, logits_from=None, inv_freq=None, tie_stable=True) -> dict:
    """TorchEngine.prefill on a CPU model. Returns logits, keys, values, stats, plus the
    layer-1 keep_abs / diff / norm for parity checks."""
    placements = placements or []
    config = config or BlendDefaults()
    cfg = model.config
    inner, layers = model.model, model.model.layers
    n_heads, n_kv = cfg.num_attention_heads, cfg.num_key_value_heads
    head_dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // n_heads
    scaling = getattr(cfg, "rope_scaling", None) or {}
    theta = getattr(cfg, "rope_theta", None) or scaling.get("rope_theta") or cfg.rope_parameters["rope_theta"]
    if inv_freq is None:
        inv_freq = reference_inv_freq(theta, head_dim)
    N, n_layers = len(tokens), len(layers)
    logits_from = N - 1 if logits_from is None else logits_from

    cached_l, exact_l, sink_l = plan_positions(N, placements, config.n_sink)
    cached, sink = torch.tensor(cached_l, dtype=torch.bool), torch.tensor(sink_l, dtype=torch.bool)
    fresh_idx = torch.tensor([i for i in range(N) if not cached_l[i]], dtype=torch.long)
    layer0_idx = torch.tensor([i for i in range(N) if not exact_l[i]], dtype=torch.long)
    ar = torch.arange(N)

    def rope(x, pos):
        return _rotate(x, pos.float()[:, None] * inv_freq[None, :])

    active = layer0_idx if config.full_first_layer else fresh_idx
    h = inner.embed_tokens(torch.tensor([tokens]))[:, active]
    keys_out, values_out, chunk_stats, selected_cached = [], [], [], 0
    sel_info = {}
    for li, layer in enumerate(layers):
        attn = layer.self_attn
        x = layer.input_layernorm(h)
        B, L, _ = x.shape
        q = rope(attn.q_proj(x).view(B, L, n_heads, -1).transpose(1, 2), active)
        k = rope(attn.k_proj(x).view(B, L, n_kv, -1).transpose(1, 2), active)
        v = attn.v_proj(x).view(B, L, n_kv, -1).transpose(1, 2)
        K, V = base_kv(placements, li, N, n_kv, head_dim, k.dtype, inv_freq)
        if li == 1 and placements and config.full_first_layer:
            keep_abs, chunk_stats, diff, norm = layer1_selection(k, v, K, V, active, cached, sink, placements, config, tie_stable)
            sel_info = dict(keep_abs=keep_abs, diff=diff, norm=norm, k=k, v=v, K=K.clone(), V=V.clone(), active=active)
            selected_cached = int(cached[keep_abs].sum().item())
            local = torch.full((N,), -1, dtype=torch.long)
            local[active] = torch.arange(len(active))
            sel = local[keep_abs]
            assert bool((sel >= 0).all()), "selected a token that was never computed"
            h, q, k, v = h[:, sel], q[:, :, sel], k[:, :, sel], v[:, :, sel]
            active = keep_abs
        K[:, :, active] = k
        V[:, :, active] = v
        out = F.scaled_dot_product_attention(q, K, V, attn_mask=active[:, None] >= ar[None, :], enable_gqa=True)
        h = h + attn.o_proj(out.transpose(1, 2).reshape(h.shape[0], h.shape[1], -1))
        h = h + layer.mlp(layer.post_attention_layernorm(h))
        keys_out.append(K)
        values_out.append(V)

    want = (active >= logits_from).nonzero().squeeze(1)
    if len(want) != N - logits_from:
        raise ValueError("logits requested for positions that were not recomputed")
    logits = model.lm_head(inner.norm(h[:, want]))[0]
    n_cached = sum(cached_l)
    layer0 = len(layer0_idx) if config.full_first_layer else N - n_cached
    rest = (N - n_cached + selected_cached) * (n_layers - 1)
    stats = {
        "tokens": N,
        "cached_tokens": n_cached,
        "recomputed_cached_tokens": selected_cached,
        "prefill_token_equiv": (layer0 + rest) / n_layers,
        "chunks": chunk_stats,
    }
    return dict(logits=logits, keys=keys_out, values=values_out, stats=stats, active=active, **{"sel": sel_info})


def repair_step(placements, fresh_k, fresh_v, N, n_kv, head_dim, dtype, inv_freq, config, layer0_idx, cached, sink):
    """The KV-repair ops of one request (torch_engine.py:96-103, :117-156), without the model:
    per layer base_kv, at layer 1 the deviation, selection and compaction of the fresh rows,
    then the scatter of the active rows. fresh_k[li]/fresh_v[li]: (1, H, n_active(li), D) with
    n_active = len(layer0_idx) for layers 0-1. Returns the final active set."""
    active = layer0_idx
    for li in range(len(fresh_k)):
        K, V = base_kv(placements, li, N, n_kv, head_dim, dtype, inv_freq)
        k, v = fresh_k[li], fresh_v[li]
        if li == 1:
            keep_abs, _, _, _ = layer1_selection(k, v, K, V, active, cached, sink, placements, config)
            local = torch.full((N,), -1, dtype=torch.long)
            local[active] = torch.arange(len(active))
            sel = local[keep_abs]
            k, v = k[:, :, sel], v[:, :, sel]
            active = keep_abs
        K[:, :, active] = k
        V[:, :, active] = v
    return active
