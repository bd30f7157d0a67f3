"""torch-facing wrappers of the C-ABI entry points (include/chunkkv_amd.h).

Each wrapper checks shapes, dtypes, devices and 16-byte alignment on the host, passes raw
device pointers and torch's current HIP stream, and maps a non-zero status to an exception.
Every wrapper launches a HIP kernel; none computes anything on the CPU.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from chunkkv_amd import _native
from chunkkv_amd._native import check, lib

_DTYPES = {torch.float32: _native.DTYPE_F32, torch.bfloat16: _native.DTYPE_BF16}


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPES[dtype]
    except KeyError:
        raise TypeError(f"unsupported K/V dtype {dtype}; the HIP kernels take float32 or bfloat16") from None


def _dev(*ts: torch.Tensor) -> torch.device:
    d = ts[0].device
    for t in ts:
        if not t.is_cuda:
            raise ValueError("chunkkv_amd ops run on a HIP device; got a tensor on " + str(t.device))
        if t.device != d:
            raise ValueError(f"tensors on different devices: {t.device} vs {d}")
    return d


_raw_stream = torch._C._cuda_getCurrentRawStream


def _stream(device: torch.device) -> int:
    """torch's current HIP stream on `device` as a raw handle (what hipLaunchKernel takes)."""
    return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())


def _ptr(t: torch.Tensor | None) -> int:
    return 0 if t is None else t.data_ptr()


def _rows_ok(t: torch.Tensor) -> bool:
    """Last dim contiguous, base and every other stride on a 16-byte boundary."""
    eb = t.element_size()
    if t.stride(-1) != 1 or t.data_ptr() % 16:
        return False
    return all((s * eb) % 16 == 0 for s in t.stride()[:-1])


def _rows_view(t: torch.Tensor) -> torch.Tensor:
    return t if _rows_ok(t) else t.contiguous()


def inv_freq(head_dim: int, theta: float, device) -> torch.Tensor:
    """(head_dim/2,) fp32 inverse frequencies from the kernels' own device function (a1)."""
    out = torch.empty(head_dim // 2, dtype=torch.float32, device=device)
    _dev(out)
    check(lib().ckv_inv_freq(_ptr(out), head_dim, float(theta), _stream(out.device)), "ckv_inv_freq")
    return out


def shift_keys(keys: torch.Tensor, delta: int, theta: float) -> torch.Tensor:
    """Re-rotate post-RoPE keys (..., L, D) by `delta` positions (torch_engine.py:56-59).

    delta == 0 returns `keys` itself, like the reference.
    """
    delta = int(delta)
    if delta == 0:
        return keys
    if not -(2**31) <= delta < 2**31:
        raise ValueError("delta does not fit in int32")
    _dev(keys)
    x = keys.contiguous()
    L, D = x.shape[-2], x.shape[-1]
    heads = x.numel() // max(1, L * D)
    out = torch.empty_like(x)
    if x.numel() == 0:
        return out
    check(
        lib().ckv_shift_keys(
            _ptr(out), L * D, _ptr(x), L * D, heads, L, D, dtype_code(x.dtype), delta, float(theta), _stream(x.device)
        ),
        "ckv_shift_keys",
    )
    return out


def rerope_gather(
    k_slab: torch.Tensor,
    v_slab: torch.Tensor,
    src_tab: torch.Tensor,
    segments: torch.Tensor,
    n_segs: int,
    max_seg_tokens: int,
    theta: float,
    err: torch.Tensor | None = None,
    layers: tuple[int, int] | None = None,
    skip: torch.Tensor | None = None,
) -> None:
    """Fill every layer's base K/V from cached chunks (torch_engine.py:96-103), one launch.

    k_slab/v_slab: (n_layers, 1, H, N, D) contiguous. src_tab: uint64/int64 device table
    [(chunk*n_layers + layer)*2 + {0, 1}]. segments: int32 (n_segs, 6) device descriptors.
    layers=(begin, end) limits the launch to those layers; skip (int32 (N,), e.g. a selection's
    keep_rank) leaves the rows of positions with skip[p] >= 0 untouched.
    """
    _dev(k_slab, v_slab, src_tab, segments)
    if not (k_slab.is_contiguous() and v_slab.is_contiguous() and k_slab.shape == v_slab.shape):
        raise ValueError("K/V slabs must be contiguous and of equal shape")
    if k_slab.dtype != v_slab.dtype:
        raise ValueError("K/V slabs must share a dtype")
    n_layers, _, H, N, D = k_slab.shape
    if src_tab.dtype != torch.int64 or src_tab.numel() % (2 * n_layers):
        raise ValueError("src_tab must be int64 with 2 addresses per (chunk, layer)")
    if segments.dtype != torch.int32 or segments.numel() < 6 * int(n_segs):
        raise ValueError("segments must be int32 with 6 fields per segment")
    n_chunks = src_tab.numel() // (2 * n_layers)
    if layers is None and skip is None:
        check(
            lib().ckv_rerope_gather(
                _ptr(k_slab), _ptr(v_slab), H * N * D, N * D, _ptr(src_tab), n_chunks, _ptr(segments), int(n_segs),
                int(max_seg_tokens), n_layers, H, N, D, dtype_code(k_slab.dtype), float(theta), _ptr(err),
                _stream(k_slab.device),
            ),
            "ckv_rerope_gather",
        )
        return
    begin, end = (0, n_layers) if layers is None else (int(layers[0]), int(layers[1]))
    if skip is not None:
        _dev(k_slab, skip)
        if skip.dtype != torch.int32 or skip.numel() != N or not skip.is_contiguous():
            raise ValueError("skip must be int32 (N,) contiguous")
    check(
        lib().ckv_rerope_gather_layers(
            _ptr(k_slab), _ptr(v_slab), H * N * D, N * D, _ptr(src_tab), n_chunks, n_layers, begin, end,
            _ptr(segments), int(n_segs), int(max_seg_tokens), _ptr(skip), H, N, D, dtype_code(k_slab.dtype),
            float(theta), _ptr(err), _stream(k_slab.device),
        ),
        "ckv_rerope_gather_layers",
    )


def rerope_gather_layers_kept(
    k_slab: torch.Tensor,
    v_slab: torch.Tensor,
    src_tab: torch.Tensor,
    segments: torch.Tensor,
    n_segs: int,
    max_seg_tokens: int,
    theta: float,
    layers: tuple[int, int],
    skip: torch.Tensor | None,
    kept_layer: int,
    k: torch.Tensor,
    v: torch.Tensor,
    keep_abs: torch.Tensor,
    keep_local: torch.Tensor,
    n_keep: int,
    n_keep_dev: torch.Tensor | None = None,
    err: torch.Tensor | None = None,
) -> None:
    """rerope_gather(layers=..., skip=...) and scatter_kept_rows into layer `kept_layer` of the
    same slab in ONE launch: K[kept_layer, 0, :, keep_abs[j]] = k[0, :, keep_local[j]] (V likewise)
    for j < n_keep, or j < min(n_keep, n_keep_dev[0]) with a device count (e.g. a selection's
    counts; n_keep is then the upper bound). torch_engine.py:96-103 for the gathered layers,
    :152 and :155-156 for the kept layer, which must lie outside `layers`."""
    _dev(k_slab, v_slab, src_tab, segments, k, v, keep_abs, keep_local)
    if not (k_slab.is_contiguous() and v_slab.is_contiguous() and k_slab.shape == v_slab.shape):
        raise ValueError("K/V slabs must be contiguous and of equal shape")
    n_layers, _, H, N, D = k_slab.shape
    k, v = _rows_view(k), _rows_view(v)
    if k.dtype != k_slab.dtype or v.dtype != k_slab.dtype or v_slab.dtype != k_slab.dtype:
        raise TypeError("fresh rows and slabs must share a dtype")
    if k.dim() != 4 or k.shape[0] != 1 or k.shape[1] != H or k.shape[3] != D or v.shape != k.shape:
        raise ValueError(f"fresh rows {tuple(k.shape)} do not match the slab {tuple(k_slab.shape)}")
    if src_tab.dtype != torch.int64 or src_tab.numel() % (2 * n_layers):
        raise ValueError("src_tab must be int64 with 2 addresses per (chunk, layer)")
    if segments.dtype != torch.int32 or segments.numel() < 6 * int(n_segs):
        raise ValueError("segments must be int32 with 6 fields per segment")
    if keep_abs.dtype != torch.int64 or keep_local.dtype != torch.int64 or not (
            keep_abs.is_contiguous() and keep_local.is_contiguous()):
        raise ValueError("keep_abs / keep_local must be contiguous int64")
    if min(keep_abs.numel(), keep_local.numel()) < int(n_keep):
        raise ValueError("keep_abs / keep_local hold fewer than n_keep rows")
    if skip is not None and (skip.dtype != torch.int32 or skip.numel() != N or not skip.is_contiguous()):
        raise ValueError("skip must be int32 (N,) contiguous")
    if n_keep_dev is not None and (n_keep_dev.dtype != torch.int32 or n_keep_dev.device != k_slab.device):
        raise ValueError("n_keep_dev must be an int32 tensor on the slab's device")
    check(
        lib().ckv_rerope_gather_layers_kept(
            _ptr(k_slab), _ptr(v_slab), H * N * D, N * D, _ptr(src_tab), src_tab.numel() // (2 * n_layers), n_layers,
            int(layers[0]), int(layers[1]), _ptr(segments), int(n_segs), int(max_seg_tokens), _ptr(skip),
            int(kept_layer), _ptr(k), k.stride(1), k.stride(2), _ptr(v), v.stride(1), v.stride(2), _ptr(keep_abs),
            _ptr(keep_local), int(n_keep), _ptr(n_keep_dev), k.shape[2], H, N, D, dtype_code(k_slab.dtype),
            float(theta), _ptr(err), _stream(k_slab.device),
        ),
        "ckv_rerope_gather_layers_kept",
    )


def deviation(
    k: torch.Tensor,
    v: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    flags: torch.Tensor,
    local: torch.Tensor,
    err: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Layer-1 per-position deviation and norm (torch_engine.py:117-124); returns (diff, norm)."""
    _dev(k, v, K, V, flags, local)
    k, v = _rows_view(k), _rows_view(v)
    if K.dtype != k.dtype or V.dtype != k.dtype or v.dtype != k.dtype:
        raise TypeError("fresh and cached K/V must share a dtype")
    _, H, N, D = K.shape
    if not (K.is_contiguous() and V.is_contiguous() and V.shape == K.shape):
        raise ValueError("cached K/V must be contiguous (1, H, N, D)")
    if k.shape[1] != H or k.shape[3] != D or v.shape != k.shape:
        raise ValueError(f"fresh k/v shape {tuple(k.shape)} does not match cache {tuple(K.shape)}")
    if flags.dtype != torch.uint8 or local.dtype != torch.int32 or flags.numel() != N or local.numel() != N:
        raise ValueError("flags must be uint8 (N,) and local int32 (N,)")
    if not (flags.is_contiguous() and local.is_contiguous()):
        raise ValueError("flags and local must be contiguous")
    diff = torch.empty(N, dtype=torch.float32, device=K.device)
    norm = torch.empty(N, dtype=torch.float32, device=K.device)
    check(
        lib().ckv_deviation(
            _ptr(k), k.stride(1), k.stride(2), _ptr(v), v.stride(1), v.stride(2), _ptr(K), _ptr(V), N * D,
            _ptr(flags), _ptr(local), N, k.shape[2], H, D, dtype_code(K.dtype), _ptr(diff), _ptr(norm), _ptr(err),
            _stream(K.device),
        ),
        "ckv_deviation",
    )
    return diff, norm


@dataclass
class Selection:
    keep_abs: torch.Tensor  # int64 (N,), first counts[KEEP] valid, ascending
    keep_local: torch.Tensor  # int64 (N,)
    keep_rank: torch.Tensor  # int32 (N,): rank in keep_abs, -1 if not kept (local map of the new active set)
    rel_dev: torch.Tensor  # float32 (C,)
    escalated: torch.Tensor  # uint8 (C,)
    counts: torch.Tensor  # int32 (COUNT_N,)


def _new_selection(N: int, C: int, dev) -> Selection:
    return Selection(
        keep_abs=torch.empty(N, dtype=torch.int64, device=dev),
        keep_local=torch.empty(N, dtype=torch.int64, device=dev),
        keep_rank=torch.empty(N, dtype=torch.int32, device=dev),
        rel_dev=torch.empty(C, dtype=torch.float32, device=dev),
        escalated=torch.empty(C, dtype=torch.uint8, device=dev),
        counts=torch.empty(_native.COUNT_N, dtype=torch.int32, device=dev),
    )


def select(
    diff: torch.Tensor,
    norm: torch.Tensor,
    flags: torch.Tensor,
    local: torch.Tensor,
    spans: torch.Tensor,
    escalate_threshold: float | None,
    out: Selection | None = None,
) -> Selection:
    """Per-chunk rel/escalation/budget + pooled top-k + sinks + compaction (torch_engine.py:125-153)."""
    _dev(diff, norm, flags, local, spans)
    N = diff.numel()
    if N > _native.SELECT_MAX_TOKENS:
        raise ValueError(f"selection supports at most {_native.SELECT_MAX_TOKENS} tokens, got {N}")
    if spans.dtype != torch.int32 or (spans.numel() % 4):
        raise ValueError("spans must be int32 (C, 4)")
    C = spans.numel() // 4
    dev = diff.device
    if out is None:
        out = _new_selection(N, C, dev)
    has_thr = escalate_threshold is not None
    check(
        lib().ckv_select(
            _ptr(diff), _ptr(norm), _ptr(flags), _ptr(local), N, _ptr(spans), C, int(has_thr),
            float(escalate_threshold) if has_thr else 0.0, _ptr(out.keep_abs), _ptr(out.keep_local),
            _ptr(out.keep_rank), _ptr(out.rel_dev), _ptr(out.escalated), _ptr(out.counts), _stream(dev),
        ),
        "ckv_select",
    )
    return out


def deviation_select_workspace(device) -> torch.Tensor:
    """A zeroed workspace for deviation_select. Every call leaves it zeroed again, so one
    workspace serves any number of calls issued in order (one stream); concurrent calls need one
    each."""
    return torch.zeros(_native.DEVIATION_SELECT_WORKSPACE_BYTES // 4, dtype=torch.int32, device=device)


def deviation_select(
    k: torch.Tensor,
    v: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    flags: torch.Tensor,
    local: torch.Tensor,
    spans: torch.Tensor,
    escalate_threshold: float | None,
    workspace: torch.Tensor,
    err: torch.Tensor | None = None,
    out: Selection | None = None,
    diff_norm: tuple[torch.Tensor, torch.Tensor] | None = None,
) -> tuple[torch.Tensor, torch.Tensor, Selection]:
    """deviation() then select() with the top-k's first digit fused into the deviation
    (torch_engine.py:117-153): the deviation launch also counts the candidates' histogram, and the
    selection starts from it. Returns (diff, norm, selection), bit-identical to the two calls.
    flags must carry the planner's pooled bit for the fast path (without it the result is the
    same, the selection slower). workspace: from deviation_select_workspace(), not shared by
    calls that may run concurrently."""
    _dev(k, v, K, V, flags, local, spans, workspace)
    k, v = _rows_view(k), _rows_view(v)
    if K.dtype != k.dtype or V.dtype != k.dtype or v.dtype != k.dtype:
        raise TypeError("fresh and cached K/V must share a dtype")
    _, H, N, D = K.shape
    if not (K.is_contiguous() and V.is_contiguous() and V.shape == K.shape):
        raise ValueError("cached K/V must be contiguous (1, H, N, D)")
    if k.shape[1] != H or k.shape[3] != D or v.shape != k.shape:
        raise ValueError(f"fresh k/v shape {tuple(k.shape)} does not match cache {tuple(K.shape)}")
    if flags.dtype != torch.uint8 or local.dtype != torch.int32 or flags.numel() != N or local.numel() != N:
        raise ValueError("flags must be uint8 (N,) and local int32 (N,)")
    if not (flags.is_contiguous() and local.is_contiguous()):
        raise ValueError("flags and local must be contiguous")
    if N > _native.SELECT_MAX_TOKENS:
        raise ValueError(f"selection supports at most {_native.SELECT_MAX_TOKENS} tokens, got {N}")
    if spans.dtype != torch.int32 or (spans.numel() % 4):
        raise ValueError("spans must be int32 (C, 4)")
    if (workspace.numel() * workspace.element_size() < _native.DEVIATION_SELECT_WORKSPACE_BYTES
            or not workspace.is_contiguous()):
        raise ValueError("workspace must come from deviation_select_workspace()")
    C = spans.numel() // 4
    dev = K.device
    if diff_norm is None:
        diff_norm = (torch.empty(N, dtype=torch.float32, device=dev), torch.empty(N, dtype=torch.float32, device=dev))
    diff, norm = diff_norm
    if out is None:
        out = _new_selection(N, C, dev)
    has_thr = escalate_threshold is not None
    check(
        lib().ckv_deviation_select(
            _ptr(k), k.stride(1), k.stride(2), _ptr(v), v.stride(1), v.stride(2), _ptr(K), _ptr(V), N * D, _ptr(flags),
            _ptr(local), N, k.shape[2], H, D, dtype_code(K.dtype), _ptr(spans), C, int(has_thr),
            float(escalate_threshold) if has_thr else 0.0, _ptr(diff), _ptr(norm), _ptr(out.keep_abs),
            _ptr(out.keep_local), _ptr(out.keep_rank), _ptr(out.rel_dev), _ptr(out.escalated), _ptr(out.counts),
            _ptr(workspace), workspace.numel() * workspace.element_size(), _ptr(err), _stream(dev),
        ),
        "ckv_deviation_select",
    )
    return diff, norm, out


def layer1_repair_workspace(device) -> torch.Tensor:
    """A zeroed workspace for layer1_repair. Each call leaves it ready for the next, so one
    workspace serves any number of calls issued in order (one stream); concurrent calls need one
    each."""
    return torch.zeros(_native.LAYER1_REPAIR_WORKSPACE_BYTES // 4, dtype=torch.int32, device=device)


def layer1_repair(
    K: torch.Tensor,
    V: torch.Tensor,
    src_tab: torch.Tensor,
    n_layers: int,
    layer: int,
    segments: torch.Tensor,
    n_segs: int,
    k: torch.Tensor,
    v: torch.Tensor,
    flags: torch.Tensor,
    local: torch.Tensor,
    spans: torch.Tensor,
    escalate_threshold: float | None,
    theta: float,
    workspace: torch.Tensor,
    err: torch.Tensor | None = None,
    out: Selection | None = None,
    diff_norm: tuple[torch.Tensor, torch.Tensor] | None = None,
) -> tuple[torch.Tensor, torch.Tensor, Selection]:
    """Layer 1's KV repair in one call of three launches (torch_engine.py:96-103 for this layer,
    :117-156): the cache K/V (1, H, N, D) gets every cached row re-rotated from the chunks (src_tab
    column `layer`, the cached-run segments) and the fresh rows of the kept positions; returns
    (diff, norm, selection), bit-identical to rerope_gather (this layer) + deviation + select +
    scatter_kept_rows. k/v: the fresh rows (1, H, n, D), any row-contiguous strides. workspace: from
    layer1_repair_workspace(), not shared by calls that may run concurrently."""
    k, v, diff, norm, out, C, n_tab = _layer1_args(K, V, src_tab, n_layers, segments, n_segs, k, v, flags, local, spans,
                                                   workspace, out, diff_norm)
    _, H, N, D = K.shape
    has_thr = escalate_threshold is not None
    check(
        lib().ckv_layer1_repair(
            _ptr(K), _ptr(V), N * D, _ptr(src_tab), n_tab, int(n_layers), int(layer), _ptr(segments), int(n_segs),
            _ptr(k), k.stride(1), k.stride(2), _ptr(v), v.stride(1), v.stride(2), k.shape[2], _ptr(flags),
            _ptr(local), N, H, D, dtype_code(K.dtype), float(theta), _ptr(spans), C, int(has_thr),
            float(escalate_threshold) if has_thr else 0.0, _ptr(diff), _ptr(norm), _ptr(out.keep_abs),
            _ptr(out.keep_local), _ptr(out.keep_rank), _ptr(out.rel_dev), _ptr(out.escalated), _ptr(out.counts),
            _ptr(workspace), workspace.numel() * workspace.element_size(), _ptr(err), _stream(K.device),
        ),
        "ckv_layer1_repair",
    )
    return diff, norm, out


def _layer1_args(K, V, src_tab, n_layers, segments, n_segs, k, v, flags, local, spans, workspace, out, diff_norm):
    """Checks shared by layer1_repair and layer1_repair_gather (K/V: one layer's (1, H, N, D)
    cache); allocates the outputs not given."""
    _dev(K, V, src_tab, segments, k, v, flags, local, spans, workspace)
    k, v = _rows_view(k), _rows_view(v)
    if K.dtype != k.dtype or V.dtype != k.dtype or v.dtype != k.dtype:
        raise TypeError("fresh and cached K/V must share a dtype")
    _, H, N, D = K.shape
    if not (K.is_contiguous() and V.is_contiguous() and V.shape == K.shape):
        raise ValueError("cache K/V must be contiguous (1, H, N, D)")
    if k.dim() != 4 or k.shape[1] != H or k.shape[3] != D or v.shape != k.shape:
        raise ValueError(f"fresh k/v shape {tuple(k.shape)} does not match cache {tuple(K.shape)}")
    if flags.dtype != torch.uint8 or local.dtype != torch.int32 or flags.numel() != N or local.numel() != N:
        raise ValueError("flags must be uint8 (N,) and local int32 (N,)")
    if not (flags.is_contiguous() and local.is_contiguous()):
        raise ValueError("flags and local must be contiguous")
    if src_tab.dtype != torch.int64 or src_tab.numel() % (2 * int(n_layers)):
        raise ValueError("src_tab must be int64 with 2 addresses per (chunk, layer)")
    if segments.dtype != torch.int32 or segments.numel() < 6 * int(n_segs):
        raise ValueError("segments must be int32 with 6 fields per segment")
    if spans.dtype != torch.int32 or (spans.numel() % 4):
        raise ValueError("spans must be int32 (C, 4)")
    if (workspace.numel() * workspace.element_size() < _native.LAYER1_REPAIR_WORKSPACE_BYTES
            or not workspace.is_contiguous()):
        raise ValueError("workspace must come from layer1_repair_workspace()")
    C = spans.numel() // 4
    dev = K.device
    if diff_norm is None:
        diff_norm = (torch.empty(N, dtype=torch.float32, device=dev), torch.empty(N, dtype=torch.float32, device=dev))
    diff, norm = diff_norm
    if out is None:
        out = _new_selection(N, C, dev)
    return k, v, diff, norm, out, C, src_tab.numel() // (2 * int(n_layers))


def layer1_repair_gather(
    k_slab: torch.Tensor,
    v_slab: torch.Tensor,
    src_tab: torch.Tensor,
    layer: int,
    layers: tuple[int, int],
    segments: torch.Tensor,
    n_segs: int,
    max_seg_tokens: int,
    k: torch.Tensor,
    v: torch.Tensor,
    flags: torch.Tensor,
    local: torch.Tensor,
    spans: torch.Tensor,
    escalate_threshold: float | None,
    theta: float,
    workspace: torch.Tensor,
    err: torch.Tensor | None = None,
    out: Selection | None = None,
    diff_norm: tuple[torch.Tensor, torch.Tensor] | None = None,
) -> tuple[torch.Tensor, torch.Tensor, Selection]:
    """layer1_repair of layer `layer` of the (L, 1, H, N, D) slabs followed by the base cache of
    layers [layers): the rows of dropped positions as rerope_gather(layers=layers,
    skip=keep_rank) writes them; the rows of kept cached positions re-rotated in the first
    layer1_repair_gather_whole_layers(...) layers of the range (gathered whole beside the
    selection) and untouched in the others. The caller overwrites the kept rows of every gathered
    layer with that layer's fresh rows, which makes both forms the same cache. Three launches."""
    if k_slab.dim() != 5 or v_slab.shape != k_slab.shape or not (k_slab.is_contiguous() and v_slab.is_contiguous()):
        raise ValueError("k_slab/v_slab must be contiguous (L, 1, H, N, D)")
    L, _, H, N, D = k_slab.shape
    b, e = int(layers[0]), int(layers[1])
    if not (0 <= b <= e <= L) or b <= int(layer) < e:
        raise ValueError(f"gather layers {layers} must lie in [0, {L}) and exclude layer {layer}")
    K, V = k_slab[int(layer)], v_slab[int(layer)]
    k, v, diff, norm, out, C, n_tab = _layer1_args(K, V, src_tab, L, segments, n_segs, k, v, flags, local, spans,
                                                   workspace, out, diff_norm)
    has_thr = escalate_threshold is not None
    check(
        lib().ckv_layer1_repair_gather(
            _ptr(k_slab), _ptr(v_slab), H * N * D, N * D, _ptr(src_tab), n_tab, L, int(layer), b, e, _ptr(segments),
            int(n_segs), int(max_seg_tokens), _ptr(k), k.stride(1), k.stride(2), _ptr(v), v.stride(1), v.stride(2),
            k.shape[2], _ptr(flags), _ptr(local), N, H, D, dtype_code(K.dtype), float(theta), _ptr(spans), C,
            int(has_thr), float(escalate_threshold) if has_thr else 0.0, _ptr(diff), _ptr(norm), _ptr(out.keep_abs),
            _ptr(out.keep_local), _ptr(out.keep_rank), _ptr(out.rel_dev), _ptr(out.escalated), _ptr(out.counts),
            _ptr(workspace), workspace.numel() * workspace.element_size(), _ptr(err), _stream(K.device),
        ),
        "ckv_layer1_repair_gather",
    )
    return diff, norm, out


def layer1_repair_gather_whole_layers(n_tokens: int, n_chunks: int, escalate_threshold: float | None, n_segs: int,
                                      max_seg_tokens: int, layers: tuple[int, int], n_heads: int, head_dim: int,
                                      dtype: torch.dtype) -> int:
    """How many leading layers of `layers` layer1_repair_gather writes whole (kept rows included)
    beside its selection for a request of this shape on the current device."""
    return int(lib().ckv_layer1_repair_gather_whole_layers(
        int(n_tokens), int(n_chunks), int(escalate_threshold is not None), int(n_segs), int(max_seg_tokens),
        int(layers[1]) - int(layers[0]), int(n_heads), int(head_dim), dtype_code(dtype)))


def scatter_kept_rows(
    K: torch.Tensor,
    V: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    dst_rows: torch.Tensor,
    src_rows: torch.Tensor,
    err: torch.Tensor | None = None,
) -> None:
    """K[:, :, dst_rows] = k[:, :, src_rows]; V likewise, one launch: the compaction of the kept
    rows and their scatter into the cache (torch_engine.py:152, :155-156). k/v: (1, H, n_src, D)
    with contiguous rows (token-major views included); dst_rows/src_rows: int64, equal length."""
    _dev(K, V, k, v, dst_rows, src_rows)
    k, v = _rows_view(k), _rows_view(v)
    _, H, N, D = K.shape
    if not (K.is_contiguous() and V.is_contiguous() and V.shape == K.shape):
        raise ValueError("cache K/V must be contiguous (1, H, N, D)")
    if k.dtype != K.dtype or v.dtype != K.dtype:
        raise TypeError("fresh rows and cache must share a dtype")
    if k.dim() != 4 or k.shape[0] != 1 or k.shape[1] != H or k.shape[3] != D or v.shape != k.shape:
        raise ValueError(f"fresh rows {tuple(k.shape)} do not match the cache {tuple(K.shape)}")
    n = dst_rows.numel()
    if dst_rows.dtype != torch.int64 or src_rows.dtype != torch.int64 or src_rows.numel() != n:
        raise ValueError("dst_rows and src_rows must be int64 of one length")
    dst_rows, src_rows = dst_rows.contiguous(), src_rows.contiguous()
    check(
        lib().ckv_scatter_kept_rows(
            _ptr(K), _ptr(V), N * D, _ptr(k), k.stride(1), k.stride(2), _ptr(v), v.stride(1), v.stride(2),
            _ptr(dst_rows), _ptr(src_rows), n, k.shape[2], N, H, D, dtype_code(K.dtype), _ptr(err), _stream(K.device),
        ),
        "ckv_scatter_kept_rows",
    )


def assemble_layer(
    K: torch.Tensor,
    V: torch.Tensor,
    src_tab: torch.Tensor,
    n_layers: int,
    layer: int,
    segments: torch.Tensor,
    n_segs: int,
    max_seg_tokens: int,
    k: torch.Tensor | None,
    v: torch.Tensor | None,
    local: torch.Tensor | None,
    theta: float,
    err: torch.Tensor | None = None,
) -> None:
    """One layer's cache with every row written once: fresh row where local[p] >= 0, else the
    re-rotated cached row (the reference's base cache + scatter pair, torch_engine.py:96-103 and
    :155-156). local=None gathers the cached segments only.

    K/V: (1, H, N, D) contiguous. src_tab: the gather's int64 address table (chunk, layer, K/V).
    segments: int32 descriptors, cached runs and (optionally) uncached runs with chunk = -1.
    """
    _dev(K, V, segments)
    _, H, N, D = K.shape
    if not (K.is_contiguous() and V.is_contiguous() and V.shape == K.shape):
        raise ValueError("cache K/V must be contiguous (1, H, N, D)")
    if src_tab.numel() % (2 * n_layers) or src_tab.dtype != torch.int64:
        raise ValueError("src_tab must be int64 with 2 addresses per (chunk, layer)")
    if segments.dtype != torch.int32 or segments.numel() < 6 * int(n_segs):
        raise ValueError("segments must be int32 with 6 fields per segment")
    n_chunks = src_tab.numel() // (2 * n_layers)
    n_fresh = 0
    kst = vst = (0, 0)
    if local is not None:
        _dev(K, local, k, v)
        if local.dtype != torch.int32 or local.numel() != N or not local.is_contiguous():
            raise ValueError("local must be int32 (N,) contiguous")
        k, v = _rows_view(k), _rows_view(v)
        if k.dtype != K.dtype or v.dtype != K.dtype:
            raise TypeError("fresh rows and cache must share a dtype")
        if k.dim() != 4 or k.shape[0] != 1 or k.shape[1] != H or k.shape[3] != D or v.shape != k.shape:
            raise ValueError(f"fresh rows {tuple(k.shape)} do not match the cache {tuple(K.shape)}")
        n_fresh = k.shape[2]
        kst, vst = (k.stride(1), k.stride(2)), (v.stride(1), v.stride(2))
    else:
        k = v = None
    check(
        lib().ckv_assemble_layer(
            _ptr(K), _ptr(V), N * D, _ptr(src_tab), n_chunks, n_layers, int(layer), _ptr(segments), int(n_segs),
            int(max_seg_tokens), _ptr(k), kst[0], kst[1], _ptr(v), vst[0], vst[1], n_fresh, _ptr(local), N, H, D,
            dtype_code(K.dtype), float(theta), _ptr(err), _stream(K.device),
        ),
        "ckv_assemble_layer",
    )


def scatter_rows(
    K: torch.Tensor, V: torch.Tensor, k: torch.Tensor, v: torch.Tensor, rows: torch.Tensor, err: torch.Tensor | None = None
) -> None:
    """K[:, :, rows] = k; V[:, :, rows] = v for one layer (torch_engine.py:155-156)."""
    _dev(K, V, k, v, rows)
    k, v = _rows_view(k), _rows_view(v)
    _, H, N, D = K.shape
    if not (K.is_contiguous() and V.is_contiguous() and V.shape == K.shape):
        raise ValueError("cache K/V must be contiguous (1, H, N, D)")
    if k.dtype != K.dtype or v.dtype != K.dtype:
        raise TypeError("fresh rows and cache must share a dtype")
    n = rows.numel()
    if k.shape != (1, H, n, D) or v.shape != k.shape:
        raise ValueError(f"fresh rows {tuple(k.shape)} do not match ({1}, {H}, {n}, {D})")
    if rows.dtype != torch.int64:
        raise ValueError("rows must be int64")
    rows = rows.contiguous()
    check(
        lib().ckv_scatter_rows(
            _ptr(K), _ptr(V), N * D, _ptr(k), k.stride(1), k.stride(2), _ptr(v), v.stride(1), v.stride(2),
            _ptr(rows), n, N, H, D, dtype_code(K.dtype), _ptr(err), _stream(K.device),
        ),
        "ckv_scatter_rows",
    )


def attention_active(
    q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    positions: torch.Tensor,
    scale: float | None = None,
    err: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    split: bool = True,
) -> torch.Tensor:
    """Attention of the active query rows over the cache, query i seeing positions <= positions[i]
    (the reference's boolean-mask SDPA with enable_gqa, torch_engine.py:157 and :68-72).

    q: (1, Hq, n, D) bf16 with contiguous rows; K/V: (1, Hkv, N, D) contiguous; positions: int64
    (n,). Returns (1, n, Hq, D) bf16, token-major (``.view(1, n, Hq * D)`` feeds o_proj).
    split: let launches too small to fill the chip split the cache range (a workspace is
    allocated for the partial results).
    """
    _dev(q, K, V, positions)
    _, Hq, n, D = q.shape
    _, Hkv, N, _ = K.shape
    if q.dtype != torch.bfloat16 or K.dtype != torch.bfloat16 or V.dtype != torch.bfloat16:
        raise TypeError("attention_active runs on bf16 q/K/V")
    if not (K.is_contiguous() and V.is_contiguous() and V.shape == K.shape) or K.shape[3] != D:
        raise ValueError("K/V must be contiguous (1, Hkv, N, D) and match q's head_dim")
    if q.stride(3) != 1:
        q = q.contiguous()
    if positions.dtype != torch.int64 or positions.numel() != n:
        raise ValueError("positions must be int64 (n,)")
    positions = positions.contiguous()
    if out is None:
        out = torch.empty((1, n, Hq, D), dtype=q.dtype, device=q.device)
    elif out.shape != (1, n, Hq, D) or not out.is_contiguous() or out.dtype != q.dtype:
        raise ValueError("out must be contiguous (1, n, Hq, D) bf16")
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    ws_bytes = lib().ckv_attention_workspace_bytes(n, N, Hq, D, None, None) if split else 0
    ws = torch.empty(ws_bytes // 4, dtype=torch.float32, device=q.device) if ws_bytes > 0 else None
    check(
        lib().ckv_attention_active(
            _ptr(out), _ptr(q), q.stride(1), q.stride(2), _ptr(K), _ptr(V), N * D, _ptr(positions), n, N, Hq, Hkv,
            D, dtype_code(q.dtype), scale, _ptr(ws), ws_bytes, _ptr(err), _stream(q.device),
        ),
        "ckv_attention_active",
    )
    return out


def _heads_view(t: torch.Tensor, n_heads: int, head_dim: int) -> tuple:
    """(pointer, head stride, token stride) of a (1, n, n_heads*D)-like token-major tensor or a
    (1, H, n, D) tensor with contiguous rows."""
    if t.dim() == 3:
        if t.stride(2) != 1 or t.shape[2] != n_heads * head_dim:
            raise ValueError("projection output must have contiguous rows of n_heads * head_dim")
        return _ptr(t), head_dim, t.stride(1)
    if t.dim() == 4 and t.shape[1] == n_heads and t.shape[3] == head_dim and t.stride(3) == 1:
        return _ptr(t), t.stride(1), t.stride(2)
    raise ValueError(f"unsupported layout {tuple(t.shape)} / {t.stride()}")


def rope_qkv(
    q_in: torch.Tensor | None,
    k_in: torch.Tensor,
    v_in: torch.Tensor | None,
    positions: torch.Tensor,
    n_q_heads: int,
    n_kv_heads: int,
    head_dim: int,
    theta: float,
    *,
    q_out: torch.Tensor | None = None,
    k_out: torch.Tensor | None = None,
    v_out: torch.Tensor | None = None,
    rows: torch.Tensor | None = None,
    table: torch.Tensor | None = None,
    err: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Fresh-token RoPE (torch_engine.py:61-66, :53-54, :46-51) of q and k, v copied alongside.

    n_q_heads = 0 (q_in ignored) rotates and writes k/v only. q_in/k_in/v_in: projection outputs, token-major (1, n, H*D) views or (1, H, n, D) tensors.
    Returns (q_out, k_out): q_out (1, n, Hq, D) token-major (the layout attention_active reads)
    unless given; k_out (1, Hkv, n, D) unless given. With rows (int64 (n,)), k/v land in rows
    rows[t] of k_out/v_out, e.g. the layer's cache (1, Hkv, N, D): the fresh-row scatter fused in.
    table: optional rope_table() covering every position (the same results). Without one (the
    default, and what HipEngine does) the kernel evaluates cos/sin from theta and the positions.
    """
    if table is not None:
        _dev(k_in, table)
        if table.dtype != torch.float32 or table.dim() != 3 or table.shape[1:] != (head_dim // 2, 2):
            raise ValueError("table must be a rope_table() output (n, D/2, 2) float32")
    _dev(k_in, positions)
    n = positions.numel()
    dev = k_in.device
    if n_q_heads == 0:  # k/v only
        q_in = k_in
    if positions.dtype != torch.int64:
        raise ValueError("positions must be int64")
    positions = positions.contiguous()
    if q_out is None and n_q_heads:
        q_out = torch.empty((1, n, n_q_heads, head_dim), dtype=q_in.dtype, device=dev)
    if k_out is None:
        if rows is not None:
            raise ValueError("rows needs k_out (the cache)")
        k_out = torch.empty((1, n_kv_heads, n, head_dim), dtype=q_in.dtype, device=dev)
    n_out = k_out.shape[2] if k_out.dim() == 4 else k_out.shape[1]
    if rows is not None:
        _dev(q_in, rows)
        if rows.dtype != torch.int64 or rows.numel() != n:
            raise ValueError("rows must be int64 (n,)")
        rows = rows.contiguous()
    if (v_in is None) != (v_out is None):
        raise ValueError("v_in and v_out go together")
    for t in (q_in, k_in, k_out) + ((q_out,) if n_q_heads else ()) + ((v_in, v_out) if v_in is not None else ()):
        if t.dtype != q_in.dtype:
            raise TypeError("q/k/v and outputs must share a dtype")
    if n_q_heads:
        if q_out.shape != (1, n, n_q_heads, head_dim) or not q_out.is_contiguous():
            raise ValueError("q_out must be contiguous (1, n, Hq, D), token-major")
        qo = _heads_view(q_out.view(1, n, n_q_heads * head_dim), n_q_heads, head_dim)
        qi = _heads_view(q_in, n_q_heads, head_dim)
    else:
        qo = qi = (None, 0, 0)
    ki = _heads_view(k_in, n_kv_heads, head_dim)
    ko = _heads_view(k_out, n_kv_heads, head_dim)
    vi = _heads_view(v_in, n_kv_heads, head_dim) if v_in is not None else (None, 0, 0)
    vo = _heads_view(v_out, n_kv_heads, head_dim) if v_out is not None else (None, 0, 0)
    check(
        lib().ckv_rope_qkv(
            qo[0], qo[1], qo[2], ko[0], ko[1], ko[2], vo[0], vo[1], vo[2], _ptr(rows), n_out, qi[0], qi[1], qi[2],
            ki[0], ki[1], ki[2], vi[0], vi[1], vi[2], _ptr(positions), _ptr(table),
            0 if table is None else table.shape[0], n, n_q_heads, n_kv_heads, head_dim,
            dtype_code(q_in.dtype), float(theta), _ptr(err), _stream(dev),
        ),
        "ckv_rope_qkv",
    )
    return q_out, k_out


def rope_table(n_positions: int, head_dim: int, theta: float, device) -> torch.Tensor:
    """(n_positions, head_dim/2, 2) float32: the correctly rounded (cos, sin) ckv_rope_qkv uses for
    each position (fp32 angle fl32(fl32(p) * inv_freq_i))."""
    out = torch.empty((n_positions, head_dim // 2, 2), dtype=torch.float32, device=device)
    _dev(out)
    check(lib().ckv_rope_table(_ptr(out), n_positions, head_dim, float(theta), _stream(out.device)), "ckv_rope_table")
    return out


def extract_chunks(
    k_slab: torch.Tensor, v_slab: torch.Tensor, spans: list, err: torch.Tensor | None = None
) -> list[torch.Tensor]:
    """Copies of token rows [start, end) of every layer's K and V for each (start, end) in spans,
    one launch for all of them (base.py:55-60 per layer and segment in the reference).

    k_slab/v_slab: (L, 1, H, N, D) contiguous. Returns one (2, L, 1, H, end - start, D) tensor per
    span (index 0 = keys, 1 = values), each its own allocation so a store can free it alone.
    """
    _dev(k_slab, v_slab)
    if not (k_slab.is_contiguous() and v_slab.is_contiguous() and k_slab.shape == v_slab.shape):
        raise ValueError("K/V slabs must be contiguous and of equal shape")
    L, _, H, N, D = k_slab.shape
    dev = k_slab.device
    bufs, meta = [], []
    for start, end in spans:
        start, end = int(start), int(end)
        if not 0 <= start <= end <= N:
            raise ValueError(f"span [{start}, {end}) outside the request of {N} tokens")
        b = torch.empty((2, L, 1, H, end - start, D), dtype=k_slab.dtype, device=dev)
        bufs.append(b)
        meta.append((b.data_ptr(), start, end - start))
    live = [(p, s, n) for p, s, n in meta if n > 0]
    if not live:
        return bufs
    # descriptors: [ptr lo, ptr hi] per span, then (start, len) pairs; pinned, one async copy
    # (torch's pinned allocator keeps the host block until the copy has run)
    pinned = torch.empty(len(live) * 4, dtype=torch.int32, pin_memory=True)
    host = pinned.numpy()
    host[: 2 * len(live)].view("<u8")[:] = [p for p, _, _ in live]
    host[2 * len(live) :] = [v for _, s, n in live for v in (s, n)]
    d = pinned.to(dev, non_blocking=True)
    check(
        lib().ckv_extract_chunks(
            _ptr(k_slab), _ptr(v_slab), H * N * D, N * D, _ptr(d), d.data_ptr() + 8 * len(live), len(live),
            max(n for _, _, n in live), L, H, N, D, dtype_code(k_slab.dtype), _ptr(err), _stream(dev),
        ),
        "ckv_extract_chunks",
    )
    return bufs


def _row_major(t: torch.Tensor, width: int, what: str) -> int:
    """Row stride (elements) of a (..., width) tensor whose rows are contiguous and evenly spaced."""
    if t.shape[-1] != width or t.stride(-1) != 1 or t.data_ptr() % 16 != 0:
        raise ValueError(f"{what} must have contiguous, 16-byte aligned rows of {width} elements")
    rows = t.reshape(-1, width) if t.dim() != 2 else t
    if rows.data_ptr() != t.data_ptr() or (rows.shape[0] > 1 and rows.stride(1) != 1):
        raise ValueError(f"{what} rows must be evenly spaced")
    return rows.stride(0) if rows.shape[0] > 1 else width


def add_rmsnorm(
    h: torch.Tensor,
    delta: torch.Tensor | None,
    weight: torch.Tensor,
    eps: float,
    *,
    h_out: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Residual add and RMSNorm: (h + delta, RMSNorm(h + delta)), or (h, RMSNorm(h)) with delta None.

    The Hugging Face Qwen2/Llama RMSNorm module's steps (fp32 math, the normalised row rounded to
    h.dtype before the weight multiplies it) after the decoder's residual add (torch_engine.py:71-72,
    :113, :75). h, delta: (..., hidden) contiguous; h_out defaults to a new tensor and may be h
    itself (in place).
    """
    _dev(h, weight, *(() if delta is None else (delta,)))
    hidden = h.shape[-1]
    if not h.is_contiguous() or (delta is not None and (not delta.is_contiguous() or delta.shape != h.shape)):
        raise ValueError("h and delta must be contiguous and of one shape")
    if weight.shape != (hidden,) or weight.dtype != h.dtype or (delta is not None and delta.dtype != h.dtype):
        raise ValueError("weight must be (hidden,) and every operand of h's dtype")
    if out is None:
        out = torch.empty_like(h)
    elif out.shape != h.shape or not out.is_contiguous() or out.dtype != h.dtype:
        raise ValueError("out must be contiguous, of h's shape and dtype")
    if delta is not None and h_out is None:
        h_out = torch.empty_like(h)
    elif h_out is not None and (h_out.shape != h.shape or not h_out.is_contiguous() or h_out.dtype != h.dtype):
        raise ValueError("h_out must be contiguous, of h's shape and dtype")
    n_rows = h.numel() // hidden if hidden else 0
    check(
        lib().ckv_add_rmsnorm(
            _ptr(h_out), _ptr(h), _ptr(delta), _ptr(out), _ptr(weight.contiguous()), n_rows, hidden, float(eps),
            dtype_code(h.dtype), _stream(h.device),
        ),
        "ckv_add_rmsnorm",
    )
    return (h if delta is None else h_out), out


def silu_mul(gate: torch.Tensor, up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """silu(gate) * up with the MLP's roundings (torch_engine.py:72 via the SiLU-gated Qwen2/Llama
    MLP). gate/up: (..., width) with evenly spaced contiguous rows (e.g. the halves of one
    stacked GEMM output); returns a contiguous (..., width) tensor."""
    _dev(gate, up)
    width = gate.shape[-1]
    if up.shape != gate.shape or up.dtype != gate.dtype:
        raise ValueError("gate and up must have one shape and dtype")
    gs, us = _row_major(gate, width, "gate"), _row_major(up, width, "up")
    if out is None:
        out = torch.empty(gate.shape, dtype=gate.dtype, device=gate.device)
    elif out.shape != gate.shape or not out.is_contiguous() or out.dtype != gate.dtype:
        raise ValueError("out must be contiguous, of gate's shape and dtype")
    n_rows = gate.numel() // width if width else 0
    check(
        lib().ckv_silu_mul(
            _ptr(out), width, _ptr(gate), gs, _ptr(up), us, n_rows, width, dtype_code(gate.dtype), _stream(gate.device),
        ),
        "ckv_silu_mul",
    )
    return out
