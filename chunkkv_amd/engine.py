"""HipEngine: drop-in replacement for the reference TorchEngine with the KV-repair path on
hand-written gfx950 kernels.

Public surface = src/chunkkv/engine/torch_engine.py:18-207: constructor ``(model, tokenizer)``,
``load(repo, dtype)``, ``prefill(tokens, placements, config, logits_from) -> PrefillResult``,
``generate``, ``last_logprobs``, ``sync``, ``clear_cache``, ``shift_keys``, ``tokenizer``.
The model's GEMMs, RMSNorm and MLP stay on PyTorch-ROCm (chunkkv_amd.model). The KV repair,
the fresh-token RoPE and the attention run on the HIP kernels:

  reference (torch_engine.py)                        here
  _qkv + _rope/_rotate (:61-66, :53-54, :46-51)      one q|k|v GEMM (stacked weights), then
    and K[:, :, active] = k, V[...] = v (:155-156)     ckv_rope_qkv: q rotated into the layout the
                                                       attention reads, k rotated and v copied
                                                       straight into the cache rows of the active
                                                       positions (layer 1: into tensors, for the
                                                       deviation; its kept rows then go through
                                                       ckv_scatter_kept_rows)
  base_kv (:96-103; ~13 launches per placement and   ckv_rerope_gather_layers (overlap=True: on
    layer, zero-filled cache, every layer)             a side stream): at the start, layer 1's
                                                       base cache (and layer 0's rows of exact
                                                       placements);
                                                       right after the selection, one launch for
                                                       the cached rows of every position the
                                                       selection dropped, layers 2..L-1 at once.
                                                       Rows the fresh K/V overwrite are never
                                                       gathered; with the side stream the main
                                                       stream waits only before the attention
                                                       that reads them
  layer 1: base_kv, deviation (:117-124),            ckv_layer1_repair, one call: the cached rows
    rel/escalation/budget/argsort/nonzero (:125-153;   re-rotated into the cache with the
    one .item() per chunk), K[:, :, active] = k        deviations, the selection (one workgroup),
    (:155-156)                                         the kept rows scattered; the host reads
                                                       nothing back unless a threshold is set.
                                                       layer1="four_launches" / "fused_select":
                                                       the base cache at the start, then
                                                       ckv_deviation + ckv_select (or
                                                       ckv_deviation_select) + ckv_scatter_kept_rows
  h, q = ...[sel] (:152)                             index-selected by the selection's keep_local
  mask + SDPA (:157, :68-72)                         ckv_attention_active: matrix-core
                                                       attention masked by the active positions
                                                       (bf16, head_dim 64/128)
All layers' caches live in one (L, 1, H, N, D) slab; PrefillResult.keys/values are its views.

Attention: the reference calls SDPA with enable_gqa and an explicit boolean (n_active x N) mask,
a combination with no fused kernel on ROCm (it runs the fp32 math path). ``attention="fused"``
(default) keeps the same semantics with fast formulations: bf16 models with head_dim 64 or 128
run every layer on the HIP kernel ckv_attention_active, which reads the positions directly (no
mask tensor, no KV-head expansion). Other models use SDPA with ``is_causal=True`` when every
position is active (the mask is then the plain causal mask) and otherwise expand the KV heads and
pass the boolean mask (built once per active set) without enable_gqa.
``attention="sdpa"`` runs the prefill's attention on torch's fused SDPA kernels (flash or
memory-efficient, selected explicitly so that the math path never runs: K/V heads repeated per
query group, ``is_causal=True`` or the boolean positions mask) and the norms and MLP on torch,
with every KV-repair kernel as in the default: it isolates what the KV repair alone gains
(decode keeps ckv_attention_active). ``attention="reference"`` reproduces the reference's SDPA
call exactly.

Side effect on the caller's model: the constructor stacks each layer's q/k/v weights (and, with
the fused MLP, gate/up) into one tensor per layer and re-points the model's q_proj/k_proj/v_proj
(gate_proj/up_proj) Parameters at row views of it, so the weights are held once and the model
keeps working. Moving or converting the model afterwards (model.to(...), .half()) or assigning
new Parameters to those modules leaves the engine's stacks on the old weights: build the engine
after the model is in its final place and dtype, and build a new one after changing it. A second
engine over the same model views the existing stacks instead of copying them.

Contracts where the reference leaves the result open: the selection breaks deviation ties by
the lower token index (torch's argsort is unstable), deviation sums use a fixed order, and
inv_freq is the correctly rounded fp32 value of the reference's expression (torch's fp32 pow
may be one ulp off). Errors keep the reference's types: NotImplementedError for rope scaling,
ValueError for logits at non-recomputed positions, AssertionError when the selection keeps a
token that was never computed.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

from chunkkv_amd import _native, ops
from chunkkv_amd.model import DecoderPieces
from chunkkv_amd.planner import RequestPlan, local_index, plan_request, stats_dict
from chunkkv_amd.types import BlendConfig, ChunkKV, Placement, PrefillResult, plan_positions  # noqa: F401

_ALIGN = 256

_TORCH_OF = {
    np.dtype(np.uint8): torch.uint8,
    np.dtype(np.int32): torch.int32,
    np.dtype(np.int64): torch.int64,
    np.dtype(np.uint64): torch.int64,  # device addresses; the kernels read them as uint64
}


def _adjacent_rows(ts: list[torch.Tensor]) -> torch.Tensor | None:
    """The tensors as one (sum of rows, ...) view when they already lie back to back in one
    storage (contiguous, same dtype and trailing shape), else None."""
    t0 = ts[0]
    if not all(t.is_contiguous() and t.dtype == t0.dtype and t.shape[1:] == t0.shape[1:] and t.device == t0.device
               and t.untyped_storage().data_ptr() == t0.untyped_storage().data_ptr() for t in ts):
        return None
    for a, b in zip(ts, ts[1:]):
        if b.data_ptr() != a.data_ptr() + a.numel() * a.element_size():
            return None
    rows = sum(t.shape[0] for t in ts)
    return t0.new_empty(0).set_(t0.untyped_storage(), t0.storage_offset(), (rows, *t0.shape[1:]),
                                (t0.stride(0), *t0.stride()[1:]) if t0.dim() > 1 else (1,))


def _stack_params(mods: list, name: str) -> torch.Tensor | None:
    """getattr(m, name) of the given modules stacked along dim 0, stored once: the modules'
    parameters are re-pointed at their rows of the stacked tensor (so the model keeps working and
    its weights are not held twice). Modules without the parameter get zero rows in the stack;
    None when no module has it. Weights that already lie back to back (a previous stacking of
    the same model) are viewed, not copied."""
    ps = [getattr(m, name) for m in mods]
    if all(p is None for p in ps):
        return None
    if all(p is not None for p in ps):
        view = _adjacent_rows([p.data for p in ps])
        if view is not None:
            return view
    ref = next(p for p in ps if p is not None)
    parts = [p.data if p is not None else ref.new_zeros((m.weight.shape[0], *ref.shape[1:])) for p, m in zip(ps, mods)]
    stacked = torch.cat(parts, 0).contiguous()
    row = 0
    for m, p, part in zip(mods, ps, parts):
        n = part.shape[0]
        if p is not None:
            setattr(m, name, torch.nn.Parameter(stacked[row : row + n], requires_grad=p.requires_grad))
        row += n
    return stacked


class HipEngine(DecoderPieces):
    def __init__(self, model, tokenizer, attention: str = "fused", overlap: bool = False,
                 layer1: str = "one_call"):
        if attention not in ("fused", "sdpa", "reference"):
            raise ValueError("attention must be 'fused', 'sdpa' or 'reference'")
        if layer1 not in ("one_call", "four_launches", "fused_select"):
            raise ValueError("layer1 must be 'one_call', 'four_launches' or 'fused_select'")
        # attention: "fused" (default) = ckv_attention_active and the fused norm/MLP kernels;
        # "sdpa" = torch's fused SDPA kernels (flash / memory-efficient, never the math path) for
        # the active rows and torch's RMSNorm and MLP, every KV-repair kernel unchanged (isolates
        # what the KV repair alone gains); "reference" = the reference op sequence's attention
        # (torch_engine.py's masked SDPA) and torch's norm/MLP.
        self.attention = attention
        # Layer 1's repair: "one_call" (default) is ckv_layer1_repair (the cached rows gathered with
        # the deviations, the selection, the kept rows; 3 launches); "four_launches" gathers layer
        # 1's base cache at the start and runs ckv_deviation, ckv_select and ckv_scatter_kept_rows;
        # "fused_select" the same with ckv_deviation_select. Same results, bit for bit. Shapes the
        # one call does not take (rows wider than 1 KiB, head_dim > 128, > 3840 cached runs) use
        # the four launches.
        self.layer1 = layer1
        # overlap=True issues the cached-row gathers on a side stream, joined by events where a
        # layer needs its rows, instead of in order on the main stream (same launches, same rows).
        # Off by default: on MI355X the side stream did not shorten the 8k request's TTFT (42.47 vs
        # 42.38 ms p50) and it lengthens the KV-repair launches' own span (0.320 vs 0.314 ms).
        self.overlap = overlap
        self._side: torch.cuda.Stream | None = None
        self._ws: dict[tuple, torch.Tensor] = {}  # layer-1 workspaces, per (kind, stream)
        # generate(): replay each decode step after the first from a HIP graph (device-side loop)
        self.decode_graphs = True
        # Set to a dict to record the layer-1 selection inputs/outputs (device tensors) of the
        # next prefill, for parity checks; None (default) records nothing.
        self.trace: dict | None = None
        self._init_model(model, tokenizer)
        if self.device.type != "cuda":
            raise ValueError("HipEngine runs on a HIP device: move the model to 'cuda' first")
        _native.lib()  # raises now if the kernels were never built: there is no CPU fallback
        self.kv_dtype = self.layers[0].self_attn.k_proj.weight.dtype
        ops.dtype_code(self.kv_dtype)
        self.inv_freq = ops.inv_freq(self.head_dim, self.theta, self.device)
        # ckv_attention_active covers bf16 caches with head_dim 64 or 128; other models keep SDPA
        self._native_attention = self.kv_dtype == torch.bfloat16 and self.head_dim in (64, 128)
        # One projection GEMM per layer for q, k and v (their weights stacked once, here; the
        # model's own q/k/v parameters become row views of the stack); its token-major output
        # feeds ckv_rope_qkv directly.
        self._w_qkv, self._b_qkv = [], []
        with torch.no_grad():
            for layer in self.layers:
                a = layer.self_attn
                lin = [a.q_proj, a.k_proj, a.v_proj]
                self._w_qkv.append(_stack_params(lin, "weight"))
                self._b_qkv.append(_stack_params(lin, "bias"))
        # The elementwise steps between the GEMMs (residual adds, RMSNorms, the SiLU-gated product)
        # run as ckv_add_rmsnorm / ckv_silu_mul for RMSNorm + SiLU-MLP models; the MLP's output is
        # then added by the next norm (or the final one) instead of right away.
        self._fused_mlp = attention == "fused" and self._fusable(model)
        if self._fused_mlp:
            norm = lambda m: (m.weight, float(m.variance_epsilon))  # noqa: E731
            self._norm_in = [norm(layer.input_layernorm) for layer in self.layers]
            self._norm_post = [norm(layer.post_attention_layernorm) for layer in self.layers]
            self._norm_final = norm(self.inner.norm)
            # gate and up as one GEMM per layer (weights stacked once, here): one launch of twice
            # the width fills the CUs better than two at the prefill shapes; ckv_silu_mul reads
            # the two halves of its output in place. As for q|k|v, the model's gate/up parameters
            # become row views of the stack, so the weights are held once.
            self._w_gu, self._b_gu = [], []
            with torch.no_grad():
                for layer in self.layers:
                    lin = [layer.mlp.gate_proj, layer.mlp.up_proj]
                    self._w_gu.append(_stack_params(lin, "weight"))
                    self._b_gu.append(_stack_params(lin, "bias"))

    _RMSNORMS = ("Qwen2RMSNorm", "LlamaRMSNorm", "MistralRMSNorm")

    def _fusable(self, model) -> bool:
        """RMSNorm modules of weight * (x * rsqrt(mean(x^2) + eps)).to(dtype) and a SiLU-gated MLP,
        in a dtype and width the fused kernels take."""
        if getattr(model.config, "hidden_act", None) != "silu" or self.kv_dtype not in (torch.bfloat16, torch.float32):
            return False
        hidden = model.config.hidden_size
        if hidden % 8 or hidden > (8192 if self.kv_dtype == torch.bfloat16 else 4096):
            return False
        norms = [self.inner.norm] + [m for layer in self.layers for m in (layer.input_layernorm, layer.post_attention_layernorm)]
        if any(type(m).__name__ not in self._RMSNORMS or m.weight.dtype != self.kv_dtype for m in norms):
            return False
        mlps = [layer.mlp for layer in self.layers]
        return all(hasattr(m, "gate_proj") and hasattr(m, "up_proj") and hasattr(m, "down_proj")
                   and m.gate_proj.out_features % 8 == 0 and m.up_proj.out_features == m.gate_proj.out_features
                   and m.up_proj.weight.shape == m.gate_proj.weight.shape for m in mlps)

    def _norm(self, li: int, layer, h, pending):
        """Input of layer li: (h + pending, input_layernorm(h + pending)); pending is the previous
        layer's MLP output when the fused kernels defer its residual add (updated in place)."""
        if not self._fused_mlp:
            return h, layer.input_layernorm(h)
        w, eps = self._norm_in[li]
        return ops.add_rmsnorm(h, pending, w, eps, h_out=h if pending is not None else None)

    def _mlp(self, li: int, layer, h, a):
        """h + a (the attention output after o_proj), then the MLP block (gate and up as one stacked
        GEMM). Returns (h, pending): the fused kernels leave the MLP's output in pending for the
        next norm to add."""
        if not self._fused_mlp:
            h = h + a
            return h + layer.mlp(layer.post_attention_layernorm(h)), None
        w, eps = self._norm_post[li]
        h, x = ops.add_rmsnorm(h, a, w, eps, h_out=h)
        gu = F.linear(x, self._w_gu[li], self._b_gu[li])
        width = gu.shape[-1] // 2
        return h, layer.mlp.down_proj(ops.silu_mul(gu[..., :width], gu[..., width:]))

    def _final_logits(self, h, pending):
        """lm_head(norm(h + pending)) of the given rows (torch_engine.py:75)."""
        if pending is None:
            return self._logits(h)
        w, eps = self._norm_final
        return self.model.lm_head(ops.add_rmsnorm(h.contiguous(), pending.contiguous(), w, eps)[1])

    @classmethod
    def load(cls, repo: str, dtype=torch.bfloat16) -> "HipEngine":
        from transformers import AutoModelForCausalLM, AutoTokenizer

        model = AutoModelForCausalLM.from_pretrained(repo, dtype=dtype).to("cuda")
        return cls(model, AutoTokenizer.from_pretrained(repo))

    def _attend_active(self, li, layer, h, q_tm, K, V, active, ar, masks: dict, err=None):
        """Attention of the active rows over the whole cache (row i sees positions <= active[i]),
        then the MLP block; returns (h, pending) as _mlp does. q_tm: (1, n, Hq, D) token-major, as
        ckv_rope_qkv writes it."""
        n_act, N = active.shape[0], ar.shape[0]
        q = q_tm.transpose(1, 2)  # (1, Hq, n, D) view
        key = (active.data_ptr(), n_act)
        if self.attention == "reference":
            return self._attend(layer, h, q, K, V, active[:, None] >= ar[None, :]), None
        attn = layer.self_attn
        if self._native_attention and self.attention == "fused":
            # positions-only mask on the matrix-core kernel; output already token-major
            o = ops.attention_active(q, K, V, active, err=err)
            return self._mlp(li, layer, h, attn.o_proj(o.view(h.shape[0], h.shape[1], -1)))
        group = self.n_heads // self.n_kv
        if self.attention == "sdpa":
            # torch's fused kernels only: K/V repeated per query group (their GQA form), the
            # causal flag for a full prefill, the positions mask otherwise
            if group > 1:
                K, V = K.repeat_interleave(group, dim=1), V.repeat_interleave(group, dim=1)
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                if n_act == N:
                    o = F.scaled_dot_product_attention(q, K, V, is_causal=True)
                else:
                    if key not in masks:
                        masks.clear()
                        masks[key] = active[:, None] >= ar[None, :]
                    o = F.scaled_dot_product_attention(q, K, V, attn_mask=masks[key])
        elif n_act == N:  # active == arange(N): the mask is exactly the causal mask
            o = F.scaled_dot_product_attention(q, K, V, is_causal=True, enable_gqa=True)
        else:
            if key not in masks:
                masks.clear()
                masks[key] = active[:, None] >= ar[None, :]
            if group > 1:
                K, V = K.repeat_interleave(group, dim=1), V.repeat_interleave(group, dim=1)
            o = F.scaled_dot_product_attention(q, K, V, attn_mask=masks[key])
        return self._mlp(li, layer, h, attn.o_proj(o.transpose(1, 2).reshape(h.shape[0], h.shape[1], -1)))

    def shift_keys(self, keys: torch.Tensor, delta: int) -> torch.Tensor:
        """Move post-RoPE keys by `delta` positions on the HIP kernel (torch_engine.py:56-59)."""
        return ops.shift_keys(keys, delta, self.theta)

    # -- device-side request state --------------------------------------------------------

    def _chunk_pointers(self, chunk, keepalive: list) -> np.ndarray:
        """(n_layers, 2) uint64 device addresses of a chunk's per-layer K and V.

        Conforming chunks (this device, the kv dtype, contiguous (1, H, L, D)) are read in
        place and their table is memoised on the chunk object (chunk tensors are treated as
        immutable once stored, as KVStore entries are); others are converted first.
        """
        n_layers = len(self.layers)
        keys, values = chunk.keys, chunk.values
        if len(keys) != n_layers or len(values) != n_layers:
            raise ValueError(f"chunk has {len(keys)} key / {len(values)} value layers, model has {n_layers}")
        # The memo holds the very tensor objects it was built from and is reused only while every
        # per-layer tensor is still the same object (a replaced layer invalidates it).
        memo = getattr(chunk, "_ckv_ptrs", None)
        if (memo is not None and memo[0] == (self.kv_dtype, self.device) and len(memo[1]) == 2 * n_layers
                and all(a is b for a, b in zip(memo[1], (*keys, *values)))):
            return memo[2]
        want = (1, self.n_kv, keys[0].shape[2], self.head_dim)
        ptrs = np.empty((n_layers, 2), dtype=np.uint64)
        converted = False
        for li in range(n_layers):
            for j, t in enumerate((keys[li], values[li])):
                if tuple(t.shape) != want:
                    raise ValueError(f"chunk layer {li} tensor has shape {tuple(t.shape)}, expected {want}")
                if t.device != self.device or t.dtype != self.kv_dtype or not t.is_contiguous() or t.data_ptr() % 16:
                    t = t.to(device=self.device, dtype=self.kv_dtype).contiguous()
                    keepalive.append(t)
                    converted = True
                ptrs[li, j] = t.data_ptr()
        if not converted:
            try:
                chunk._ckv_ptrs = ((self.kv_dtype, self.device), (*keys, *values), ptrs)
            except AttributeError:
                pass
        return ptrs

    def _upload(self, parts: list[np.ndarray]) -> list[torch.Tensor]:
        """Pack host arrays into one pinned buffer, copy it with one async H2D, return views."""
        offs, total = [], 0
        for a in parts:
            offs.append(total)
            total += (a.nbytes + _ALIGN - 1) // _ALIGN * _ALIGN
        host = torch.empty(max(total, _ALIGN), dtype=torch.uint8, pin_memory=True)
        hv = host.numpy()
        for a, o in zip(parts, offs):
            if a.nbytes:
                hv[o : o + a.nbytes] = np.ascontiguousarray(a).view(np.uint8).reshape(-1)
        dev = host.to(self.device, non_blocking=True)
        return [
            dev[o : o + a.nbytes].view(_TORCH_OF[a.dtype])
            if a.nbytes
            else torch.empty(0, dtype=_TORCH_OF[a.dtype], device=self.device)
            for a, o in zip(parts, offs)
        ]

    def _workspace(self, kind: str) -> torch.Tensor:
        """The layer-1 workspace of `kind` ("one_call" or "fused_select") for torch's current
        stream (zeroed once; every call leaves it zeroed). One per stream, so prefills issued on
        different streams never share one."""
        key = (kind, torch.cuda.current_stream(self.device).cuda_stream)
        ws = self._ws.get(key)
        if ws is None:
            make = ops.layer1_repair_workspace if kind == "one_call" else ops.deviation_select_workspace
            ws = self._ws[key] = make(self.device)
        return ws

    def _one_call_fits(self, plan: RequestPlan) -> bool:
        """Whether ckv_layer1_repair takes this request's layer 1 (its limits)."""
        D, row = self.head_dim, self.n_kv * self.head_dim * torch.finfo(self.kv_dtype).bits // 8
        return (self.layer1 == "one_call" and D <= 128 and D & (D - 1) == 0 and row <= 1024
                and len(plan.segments) <= 3840 and plan.n_tokens <= _native.SELECT_MAX_TOKENS)

    def _project(self, li: int, x: torch.Tensor):
        """q|k|v projection of layer li in one GEMM: views (1, n, H*D) of its token-major output."""
        lin = F.linear(x, self._w_qkv[li], self._b_qkv[li])
        qd, kd = self.n_heads * self.head_dim, self.n_kv * self.head_dim
        return lin[..., :qd], lin[..., qd : qd + kd], lin[..., qd + kd :]

    def _gather(self, k_slab, v_slab, tab_d, segs_d, n_segs, max_seg, layers, skip, err):
        """Cached rows of layers [layers) that no fresh row of that layer overwrites (skip[p] >= 0
        marks the active positions; skip None = every cached row), one launch. With overlap on, it
        runs on the side stream, ordered after everything issued so far; the returned event marks
        its end (None when it ran on the main stream)."""
        if not self.overlap:
            ops.rerope_gather(k_slab, v_slab, tab_d, segs_d, n_segs, max_seg, self.theta, err, layers=layers, skip=skip)
            return None
        main = torch.cuda.current_stream(self.device)
        if self._side is None:
            self._side = torch.cuda.Stream(device=self.device)  # default priority
        side = self._side
        side.wait_stream(main)
        with torch.cuda.stream(side):
            ops.rerope_gather(k_slab, v_slab, tab_d, segs_d, n_segs, max_seg, self.theta, err, layers=layers, skip=skip)
            done = torch.cuda.Event()
            done.record(side)
        for t in (k_slab, v_slab, tab_d, segs_d, err) + ((skip,) if skip is not None else ()):
            t.record_stream(side)  # allocated on the main stream, read or written on the side stream
        return done

    # -- decode ---------------------------------------------------------------------------

    @torch.inference_mode()
    def generate(self, result: PrefillResult, max_tokens: int = 32) -> list[int]:
        """Greedy decode continuing a prefill (torch_engine.py:180-198) on preallocated caches.

        The reference appends each new token with a torch.cat of every layer's whole cache
        (:190-191), re-copying the cache once per token. Here one (L, 1, H, N + max_tokens, D) slab
        per tensor is filled once from the prefill's caches; each step writes the token's rotated
        k and its v into row pos in place (ckv_rope_qkv) and attends over the slab with the
        position as the mask (rows past pos are never read). With the positions-masked attention
        kernel a step reads its token and position from device tensors and writes the next greedy
        token back, so after the first (eager) step every step is one HIP graph replay; the host
        only reads the token, for the EOS test."""
        out: list[int] = []
        nxt = int(result.logits[-1].argmax().item())
        if max_tokens <= 0 or nxt in self.eos:
            return out
        dev, H, D, L = self.device, self.n_kv, self.head_dim, len(self.layers)
        N = result.keys[0].shape[2]
        cap = N + max_tokens
        Ks = torch.empty((L, 1, H, cap, D), dtype=self.kv_dtype, device=dev)
        Vs = torch.empty_like(Ks)
        for li in range(L):
            Ks[li, :, :, :N].copy_(result.keys[li])
            Vs[li, :, :, :N].copy_(result.values[li])
        err = torch.zeros(1, dtype=torch.int32, device=dev)
        device_loop = self._native_attention and self.attention in ("fused", "sdpa")
        tok = torch.tensor([[nxt]], dtype=torch.int64, device=dev)
        where = torch.tensor([N], dtype=torch.int64, device=dev)
        graph = None
        while len(out) < max_tokens and nxt not in self.eos:
            out.append(nxt)
            if not device_loop:
                self._decode_step_sdpa(tok, N + len(out) - 1, Ks, Vs, err)
            elif graph is not None:
                graph.replay()
            else:
                self._decode_step(tok, where, Ks, Vs, err)  # also the warm-up of the capture
                if max_tokens - len(out) >= 2 and self.decode_graphs:
                    graph = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(graph):
                        self._decode_step(tok, where, Ks, Vs, err)
            nxt = int(tok.item())
        if int(err.item()) != 0:
            raise RuntimeError("a decode kernel reported an out-of-range position")
        return out

    def _decode_step(self, tok, where, Ks, Vs, err) -> None:
        """One token (tok: (1, 1) int64 at position where: (1,) int64) through every layer; writes
        the next greedy token into tok and advances where. No host values are read."""
        H, D = self.n_kv, self.head_dim
        h, pending = self.inner.embed_tokens(tok), None
        for li, layer in enumerate(self.layers):
            h, x = self._norm(li, layer, h, pending)
            q_in, k_in, v_in = self._project(li, x)
            q, _ = ops.rope_qkv(q_in, k_in, v_in, where, self.n_heads, H, D, self.theta, k_out=Ks[li], v_out=Vs[li],
                                rows=where, err=err)
            o = ops.attention_active(q.transpose(1, 2), Ks[li], Vs[li], where, err=err)
            h, pending = self._mlp(li, layer, h, layer.self_attn.o_proj(o.view(1, 1, -1)))
        tok.copy_(self._final_logits(h, pending)[0, -1].argmax().view(1, 1))
        where.add_(1)

    def _decode_step_sdpa(self, tok, pos: int, Ks, Vs, err) -> None:
        """_decode_step for models outside the attention kernel's range (SDPA over rows <= pos)."""
        H, D = self.n_kv, self.head_dim
        where = torch.tensor([pos], dtype=torch.int64, device=self.device)
        h, pending = self.inner.embed_tokens(tok), None
        for li, layer in enumerate(self.layers):
            h, x = self._norm(li, layer, h, pending)
            q_in, k_in, v_in = self._project(li, x)
            q, _ = ops.rope_qkv(q_in, k_in, v_in, where, self.n_heads, H, D, self.theta, k_out=Ks[li], v_out=Vs[li],
                                rows=where, err=err)
            o = F.scaled_dot_product_attention(q.transpose(1, 2), Ks[li][:, :, : pos + 1], Vs[li][:, :, : pos + 1],
                                               enable_gqa=True)
            h, pending = self._mlp(li, layer, h, layer.self_attn.o_proj(o.transpose(1, 2).reshape(1, 1, -1)))
        tok.copy_(self._final_logits(h, pending)[0, -1].argmax().view(1, 1))

    # -- main entry -----------------------------------------------------------------------

    @torch.inference_mode()
    def prefill(self, tokens, placements=None, config=None, logits_from=None) -> PrefillResult:
        placements = placements or []
        config = config or BlendConfig()
        N = len(tokens)
        n_layers = len(self.layers)
        logits_from = N - 1 if logits_from is None else logits_from
        dev, H, D = self.device, self.n_kv, self.head_dim

        tokens_np = np.asarray(tokens, dtype=np.int64).reshape(-1)
        # When layer 0's active set is every position (no exact placement), the embedding and
        # layer 0's input norm and q|k|v GEMM need nothing from the request plan: they go out
        # first and run while the host builds the plan.
        first = None
        if config.full_first_layer and not any(getattr(p, "exact", False) for p in placements) or not placements:
            tok_d = torch.from_numpy(tokens_np).to(dev)
            h, x = self._norm(0, self.layers[0], self.inner.embed_tokens(tok_d[None]), None)
            first = self._project(0, x)

        plan: RequestPlan = plan_request(N, placements, config.n_sink, config.recompute_ratio)
        select_layer = bool(placements) and config.full_first_layer and n_layers > 1
        one_call = select_layer and self._one_call_fits(plan)
        active_np = plan.layer0_idx if config.full_first_layer else plan.fresh_idx
        local_np = local_index(N, active_np)
        if first is not None and len(active_np) != N:
            raise AssertionError("layer 0's active set is not every position")

        keepalive: list = []
        tab = np.zeros(0, dtype=np.uint64)
        if plan.chunks:
            tab = np.concatenate([self._chunk_pointers(c, keepalive).reshape(-1) for c in plan.chunks])
        flags_d, local_d, active_d, segs_d, spans_d, tab_d, tok_up = self._upload(
            [plan.flags, local_np, active_np.astype(np.int64), plan.all_segments.reshape(-1), plan.spans.reshape(-1), tab,
             tokens_np if first is None else tokens_np[:0]]
        )
        n_cached_segs = len(plan.segments)
        # layer 1 as one call on the main stream carries the gather of layers 2..'s dropped rows
        merged_gather = one_call and not self.overlap and n_cached_segs > 0 and n_layers > 2

        # Every row of every layer is written below: active rows by ckv_rope_qkv (layer 1: by
        # ckv_scatter_rows), the other cached rows by the gathers.
        k_slab = torch.empty((n_layers, 1, H, N, D), dtype=self.kv_dtype, device=dev)
        v_slab = torch.empty_like(k_slab)
        err = torch.zeros(1, dtype=torch.int32, device=dev)
        keys_out = list(k_slab.unbind(0))
        values_out = list(v_slab.unbind(0))

        active = active_d
        if first is None:
            h = self.inner.embed_tokens(tok_up[None])[:, active]
        ar = torch.arange(N, device=dev)
        masks: dict = {}
        sel = None
        ready: dict[int, torch.cuda.Event | None] = {}  # layer -> its cached rows are in place
        gather = lambda layers, skip: self._gather(  # noqa: E731
            k_slab, v_slab, tab_d, segs_d, n_cached_segs, plan.max_seg_tokens, layers, skip, err)
        # Cached rows that do not depend on the model go out first (overlap=True: beside layer 0):
        # with the selection, layer 0's rows outside its active set (exact placements) and layer
        # 1's base cache (every cached row); without it, every layer's rows outside the one
        # active set. Layers 2.. follow right after the selection.
        if n_cached_segs:
            if select_layer:
                if plan.exact.any():
                    ready[0] = gather((0, 1), local_d)
                if not one_call:
                    ready[1] = gather((1, 2), None)
            else:
                ready[0] = gather((0, n_layers), local_d)
        pending = None  # the previous layer's MLP output, when its residual add is deferred
        for li, layer in enumerate(self.layers):
            if li == 0 and first is not None:
                q_in, k_in, v_in = first
            else:
                h, x = self._norm(li, layer, h, pending)
                q_in, k_in, v_in = self._project(li, x)
            K, V = keys_out[li], values_out[li]
            if li == 1 and select_layer:
                q, k = ops.rope_qkv(q_in, k_in, None, active, self.n_heads, H, D, self.theta, err=err)
                v = v_in.view(1, -1, H, D).transpose(1, 2)
                base = None
                if one_call:
                    if self.trace is not None:  # the base cache the deviations compare against
                        base = (torch.empty_like(K), torch.empty_like(V))
                        ops.assemble_layer(*base, tab_d, n_layers, 1, segs_d, n_cached_segs, plan.max_seg_tokens,
                                           None, None, None, self.theta, err)
                    if merged_gather:  # the kept rows' scatter and layers 2..'s dropped rows in one launch
                        diff, norm, sel = ops.layer1_repair_gather(
                            k_slab, v_slab, tab_d, 1, (2, n_layers), segs_d, n_cached_segs, plan.max_seg_tokens, k, v,
                            flags_d, local_d, spans_d, config.escalate_threshold, self.theta,
                            self._workspace("one_call"), err)
                    else:
                        diff, norm, sel = ops.layer1_repair(K, V, tab_d, n_layers, 1, segs_d, n_cached_segs, k, v,
                                                            flags_d, local_d, spans_d, config.escalate_threshold,
                                                            self.theta, self._workspace("one_call"), err)
                else:
                    if ready.get(1) is not None:
                        torch.cuda.current_stream(dev).wait_event(ready[1])
                    base = (K.clone(), V.clone()) if self.trace is not None else None
                    if self.layer1 == "fused_select":
                        diff, norm, sel = ops.deviation_select(k, v, K, V, flags_d, local_d, spans_d,
                                                               config.escalate_threshold,
                                                               self._workspace("fused_select"), err)
                    else:
                        diff, norm = ops.deviation(k, v, K, V, flags_d, local_d, err)
                        sel = ops.select(diff, norm, flags_d, local_d, spans_d, config.escalate_threshold)
                if config.escalate_threshold is None and not plan.has_overlap:
                    n_keep = plan.n_keep  # fixed by the layout: no device round trip
                else:
                    counts = sel.counts.cpu()
                    if int(counts[_native.COUNT_UNCOMPUTED]) > 0:
                        raise AssertionError("selected a token that was never computed")
                    n_keep = int(counts[_native.COUNT_KEEP])
                n_keep_used = n_keep
                if self.trace is not None:
                    self.trace.update(k=k, v=v, K=base[0], V=base[1], flags=flags_d, local=local_d, spans=spans_d,
                                      diff=diff, norm=norm, sel=sel, n_keep=n_keep)
                rows = sel.keep_local[:n_keep]
                h, q = h.index_select(1, rows), q.index_select(1, rows)
                active = sel.keep_abs[:n_keep]
                if not one_call:
                    ops.scatter_kept_rows(K, V, k, v, active, rows, err)  # k/v compaction folded in
                if n_cached_segs and n_layers > 2 and not merged_gather:
                    ready[2] = gather((2, n_layers), sel.keep_rank)
            else:
                # RoPE of q/k with k and v written straight into this layer's cache rows
                q, _ = ops.rope_qkv(q_in, k_in, v_in, active, self.n_heads, H, D, self.theta, k_out=K, v_out=V,
                                    rows=active, err=err)
                if ready.get(li) is not None:
                    torch.cuda.current_stream(dev).wait_event(ready[li])
            h, pending = self._attend_active(li, layer, h, q, K, V, active, ar, masks, err)

        n_want = N - logits_from
        if 0 <= logits_from <= N and not plan.cached[logits_from:].any():
            # Uncached positions are in every active set, and active sets are sorted, so the
            # requested positions are the last n_want rows.
            tail = slice(h.shape[1] - n_want, None)
            logits = self._final_logits(h[:, tail], None if pending is None else pending[:, tail])[0]
        else:
            want = (active >= logits_from).nonzero().squeeze(1)
            if len(want) != n_want:
                raise ValueError("logits requested for positions that were not recomputed")
            logits = self._final_logits(h[:, want], None if pending is None else pending[:, want])[0]

        chunk_stats: list[dict] = []
        selected_cached = 0
        if sel is not None:
            counts = sel.counts.cpu()
            if int(counts[_native.COUNT_UNCOMPUTED]) > 0:
                raise AssertionError("selected a token that was never computed")
            # Without a device read-back the layers after the selection used the host plan's n_keep:
            # the kernel's own count must agree, or the rows sliced above were the wrong ones.
            if int(counts[_native.COUNT_KEEP]) != n_keep_used:
                raise AssertionError(f"selection kept {int(counts[_native.COUNT_KEEP])} tokens, the plan "
                                     f"{n_keep_used}")
            selected_cached = int(counts[_native.COUNT_SELECTED_CACHED])
            for (s, L, _, _), r, e in zip(plan.spans.tolist(), sel.rel_dev.cpu().tolist(), sel.escalated.cpu().tolist()):
                chunk_stats.append({"start": s, "length": L, "rel_dev": r, "escalated": bool(e)})
        if int(err.item()) != 0:
            raise RuntimeError("a KV-repair kernel reported an out-of-range descriptor")
        del keepalive

        layer0 = len(plan.layer0_idx) if config.full_first_layer else N - plan.n_cached
        stats = stats_dict(N, plan.n_cached, n_layers, layer0, selected_cached, chunk_stats)
        return PrefillResult(logits, torch.arange(logits_from, N), keys_out, values_out, stats,
                             copy=lambda t: t.contiguous(), extract=lambda spans: ops.extract_chunks(k_slab, v_slab, spans))
