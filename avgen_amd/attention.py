"""Drop-in for ``avgen.models.attention`` backed by the gfx950 flash kernels.

Same public names and signatures as src/avgen/models/attention.py:
:func:`attention`, :func:`key_padding_mask`, :func:`device_arch`,
:func:`attention_backends`, :func:`sdpa_context`.  A caller swaps the module
(e.g. ``avgen.models.layers.attention = avgen_amd.attention.attention``) and
nothing else changes.

Semantics kept from the reference: zero-length query or key sequences
return ``zeros_like(query)`` (:261-262); the default scale is
``1/sqrt(head_dim)``; a boolean mask is ``True`` = attend.  Scope of the
kernel (anything else raises rather than silently running elsewhere):
bf16 tensors on a ROCm GPU (:func:`attention`, :func:`rotary_attention`,
:func:`windowed_attention`, :func:`temporal_neighbour_attention` and
:func:`varlen_attention` also take float32 tensors, computed in fp32 by
their own kernels, as the reference's SDPA computes in the caller's dtype),
head_dim 64 or 128,
``dropout_p == 0``,
``is_causal == False`` (video DiT attention is bidirectional), and masks
that are key-padding masks — boolean, broadcastable as ``(batch, 1, 1,
keys)`` — which is what :func:`key_padding_mask` and CrossAttention build
(src/avgen/models/layers.py:651-657).

Query-dependent masks are not taken as dense ``(queries, keys)`` tensors —
those are what makes the reference run out of memory — but as per-row key
windows ``[lo, hi)`` that the kernels skip tiles by:
:func:`temporal_neighbour_attention` for the audio-video fusion mask
(src/avgen/models/blocks.py:54-104, built at src/avgen/models/dit.py:931-942)
and :func:`varlen_attention` for packed sequences (the ``cu_seqlens`` of
src/avgen/data/packing.py:163-200); :func:`windowed_attention` takes the
windows directly.
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass
from contextlib import AbstractContextManager, nullcontext
from typing import Optional

import torch
from torch.nn.attention import SDPBackend, sdpa_kernel

from . import ops
from .rope import RotaryTables

__all__ = [
    "BACKEND",
    "attention",
    "attention_backends",
    "attention_fp8",
    "device_arch",
    "key_padding_mask",
    "rotary_attention",
    "sdpa_context",
    "packed_windows",
    "TemporalNeighbourhood",
    "temporal_neighbour_attention",
    "temporal_neighbourhood",
    "temporal_neighbour_windows",
    "varlen_attention",
    "windowed_attention",
]

#: Name of the kernel family behind every backend below: the hand-written
#: gfx950 kernels serve any backend list a caller pins.
BACKEND = "avattn_gfx950"

# Architecture family per CUDA-style compute capability (major * 10 + minor),
# read as "at least this capability", and the SDPA backend priority of each
# family, MATH last: the classification of
# src/avgen/models/attention.py:53-91, kept identical so that a caller's
# backend lists and contexts compose with this module exactly as with the
# reference's.  ROCm builds of PyTorch report gfx950 as capability (9, 5).
_CAPABILITY_FLOORS: tuple[tuple[int, str], ...] = (
    (100, "blackwell"),
    (90, "hopper"),
    (89, "ada"),
    (80, "ampere"),
    (0, "legacy"),
)


def _backend_table() -> dict[str, tuple[SDPBackend, ...]]:
    flash, eff, math_, cudnn = (
        SDPBackend.FLASH_ATTENTION,
        SDPBackend.EFFICIENT_ATTENTION,
        SDPBackend.MATH,
        SDPBackend.CUDNN_ATTENTION,
    )
    return {
        "blackwell": (cudnn, flash, eff, math_),
        "hopper": (cudnn, flash, eff, math_),
        "ada": (flash, eff, math_),
        "ampere": (flash, eff, math_),
        "legacy": (eff, math_),
        "cpu": (math_,),
    }


_BACKENDS = _backend_table()
_arch_by_index: dict[int, str] = {}


def device_arch(device: torch.device | str | None = None) -> str:
    """Architecture family of a device, as src/avgen/models/attention.py:98-130
    classifies it: ``"cpu"`` for anything but an available GPU, else the
    family of ``torch.cuda.get_device_capability`` (memoised per device
    index).  An MI355X reports capability (9, 5) under ROCm, i.e.
    ``"hopper"``, exactly what the reference returns on the same machine."""
    if device is None:
        resolved = torch.device("cuda" if torch.cuda.is_available() else "cpu")
    else:
        resolved = torch.device(device)
    if resolved.type != "cuda" or not torch.cuda.is_available():
        return "cpu"
    index = resolved.index if resolved.index is not None else torch.cuda.current_device()
    arch = _arch_by_index.get(index)
    if arch is None:
        major, minor = torch.cuda.get_device_capability(index)
        cap = 10 * major + minor
        arch = next(name for floor, name in _CAPABILITY_FLOORS if cap >= floor)
        _arch_by_index[index] = arch
    return arch


def attention_backends(
    device: torch.device | str | None = None, *, allow_flash: bool = True
) -> tuple[SDPBackend, ...]:
    """Backend priority list of a device (src/avgen/models/attention.py:133-153):
    the same ``SDPBackend`` tuple the reference returns, so callers can pass it
    on to :func:`attention` or :func:`sdpa_context`.  Every entry is served by
    the gfx950 kernels here (there is no dispatch between them)."""
    chosen = _BACKENDS[device_arch(device)]
    if not allow_flash:
        chosen = tuple(b for b in chosen if b is not SDPBackend.FLASH_ATTENTION)
    return chosen


def sdpa_context(
    device: torch.device | str | None = None, *, backends: Sequence[SDPBackend] | None = None
) -> AbstractContextManager[None]:
    """Context pinning PyTorch's SDPA backend priority, as
    src/avgen/models/attention.py:156-180 builds it: a no-op on CPU, else
    ``sdpa_kernel`` over ``backends`` (default :func:`attention_backends`).
    It governs PyTorch's own SDPA calls made inside it; the gfx950 kernels of
    this package run whatever it pins."""
    if device_arch(device) == "cpu":
        return nullcontext()
    chosen = tuple(backends) if backends is not None else attention_backends(device)
    return sdpa_kernel(list(chosen))


def key_padding_mask(mask: torch.Tensor | None, *, assume_dense: bool = False) -> torch.Tensor | None:
    """``(batch, keys)`` validity -> ``(batch, 1, 1, keys)`` or ``None`` when
    every key is valid (src/avgen/models/attention.py:183-224, including its
    one host-device synchronisation on the all-valid test).

    Raises:
        ValueError: mask not rank 2.
        TypeError: mask not bool.
    """
    if mask is None or assume_dense:
        return None
    if mask.ndim != 2:
        raise ValueError(f"key mask must have rank 2 (batch, keys); got {tuple(mask.shape)}")
    if mask.dtype is not torch.bool:
        raise TypeError(f"key mask must be bool; got {mask.dtype}")
    if mask.numel() == 0 or bool(mask.all()):
        return None
    return mask[:, None, None, :]


def _as_key_mask(attn_mask: Optional[torch.Tensor], batch: int, len_q: int, len_k: int) -> Optional[torch.Tensor]:
    """Reduce a broadcastable SDPA boolean mask to ``(batch|1, keys)``."""
    if attn_mask is None:
        return None
    if attn_mask.dtype is not torch.bool:
        raise NotImplementedError(
            "avgen_amd attention supports boolean key-padding masks only; got an additive "
            f"{attn_mask.dtype} mask"
        )
    m = attn_mask
    if m.ndim == 2:
        if m.shape[-1] != len_k or m.shape[0] not in (1, len_q):
            raise ValueError(f"mask {tuple(m.shape)} does not broadcast to (queries, keys)=({len_q}, {len_k})")
        if m.shape[0] != 1:
            raise NotImplementedError("avgen_amd attention supports key-padding masks only (no per-query rows)")
        return m
    if m.ndim != 4:
        raise ValueError(f"attention mask must be rank 2 or 4; got {tuple(m.shape)}")
    if m.shape[-1] != len_k or m.shape[0] not in (1, batch):
        raise ValueError(f"mask {tuple(m.shape)} does not broadcast to (batch, keys)=({batch}, {len_k})")
    if m.shape[1] != 1 or m.shape[2] != 1:
        raise NotImplementedError(
            f"avgen_amd attention supports key-padding masks (batch, 1, 1, keys) only; got {tuple(m.shape)}"
        )
    return m[:, 0, 0, :]


def _validate(query, key, value, dropout_p, is_causal, enable_gqa):
    if dropout_p != 0.0:
        raise NotImplementedError("avgen_amd attention has no dropout (video DiTs train without it)")
    if is_causal:
        raise NotImplementedError("avgen_amd attention is bidirectional; is_causal=True is not supported")
    if query.ndim != 4 or key.ndim != 4 or value.ndim != 4:
        raise ValueError("query/key/value must be (batch, heads, seq, head_dim)")
    if key.shape[1] != query.shape[1] and not enable_gqa:
        raise ValueError(
            f"query has {query.shape[1]} heads but key has {key.shape[1]}; pass enable_gqa=True for "
            "grouped-query attention"
        )


def attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    *,
    attn_mask: torch.Tensor | None = None,
    dropout_p: float = 0.0,
    is_causal: bool = False,
    enable_gqa: bool = False,
    backends: Sequence[object] | None = None,
) -> torch.Tensor:
    """Scaled dot-product attention on the gfx950 kernel
    (signature of src/avgen/models/attention.py:227-237).

    Args:
        query: ``(batch, heads, queries, head_dim)`` bf16 or float32 on a
            ROCm GPU (key and value in the same dtype).
        key/value: ``(batch, kv_heads, keys, head_dim)``.
        attn_mask: ``None`` or a boolean key-padding mask broadcastable as
            ``(batch, 1, 1, keys)``; True = attend.
        dropout_p, is_causal: must be 0 / False.
        enable_gqa: allow ``kv_heads`` dividing ``heads``.
        backends: SDPA backend priority for the call, pinned with
            :func:`sdpa_context` around it as the reference does (:264);
            the gfx950 kernel serves every list.

    Returns:
        ``(batch, heads, queries, head_dim)`` in query's dtype; differentiable.
    """
    if query.shape[-2] == 0 or key.shape[-2] == 0:
        return torch.zeros_like(query)
    _validate(query, key, value, dropout_p, is_causal, enable_gqa)
    mask = _as_key_mask(attn_mask, query.shape[0], query.shape[-2], key.shape[-2])
    with sdpa_context(query.device, backends=backends):
        out, _ = ops.flash_fwd(query, key, value, mask, None, None, ops.default_scale(query.shape[-1]))
    return out


def rotary_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    tables: RotaryTables,
    *,
    key_tables: RotaryTables | None = None,
    attn_mask: torch.Tensor | None = None,
    enable_gqa: bool = False,
) -> torch.Tensor:
    """``attention(apply_rotary(query, t), apply_rotary(key, t), value)`` with the
    query rotation fused into the kernel's Q load
    (src/avgen/models/layers.py:533-544).

    The key is rotated once by the standalone rotary kernel (every query tile
    re-reads K, so rotating per load would multiply its traffic).  The result
    equals the unfused composition bit for bit.  ``key_tables`` defaults to
    ``tables`` (self-attention); pass the key shard's tables for a KV chunk.
    """
    if query.shape[-2] == 0 or key.shape[-2] == 0:
        return torch.zeros_like(query)
    _validate(query, key, value, 0.0, False, enable_gqa)
    kt = tables if key_tables is None else key_tables
    k_rot = ops.rope_apply(key, kt.cos, kt.sin, False)
    mask = _as_key_mask(attn_mask, query.shape[0], query.shape[-2], key.shape[-2])
    out, _ = ops.flash_fwd(query, k_rot, value, mask, tables.cos, tables.sin, ops.default_scale(query.shape[-1]))
    return out


def attention_fp8(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    *,
    attn_mask: torch.Tensor | None = None,
    enable_gqa: bool = False,
    q_scale: torch.Tensor | None = None,
    k_scale: torch.Tensor | None = None,
) -> torch.Tensor:
    """:func:`attention` with q k^T on fp8 (OCP e4m3) operands: the
    sampling-time variant (forward only; no reference counterpart, whose
    attention is bf16 throughout).

    ``q_scale`` / ``k_scale`` are per-head dequantization scales, fp32
    ``(heads,)`` / ``(kv_heads,)`` on the GPU; each defaults to the head's
    absmax / 448 (:func:`avgen_amd.ops.fp8_absmax_scales`), computed on the
    GPU for this call.  Scores are ``(e4m3(q/q_scale) . e4m3(k/k_scale)) *
    q_scale * k_scale / sqrt(head_dim)``; P, V and the output accumulation
    are those of :func:`attention`.  Other arguments as for :func:`attention`.
    """
    if query.shape[-2] == 0 or key.shape[-2] == 0:
        return torch.zeros_like(query)
    _validate(query, key, value, 0.0, False, enable_gqa)
    mask = _as_key_mask(attn_mask, query.shape[0], query.shape[-2], key.shape[-2])
    if q_scale is None:
        q_scale = ops.fp8_absmax_scales(query)
    if k_scale is None:
        k_scale = ops.fp8_absmax_scales(key)
    out, _ = ops.flash_fwd_fp8(query, key, value, mask, q_scale, k_scale, ops.default_scale(query.shape[-1]))
    return out


# ---------------------------------------------------------------------------
# Per-row key windows
# ---------------------------------------------------------------------------


def windowed_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    window_lo: torch.Tensor,
    window_hi: torch.Tensor,
    *,
    attn_mask: torch.Tensor | None = None,
    enable_gqa: bool = False,
) -> torch.Tensor:
    """:func:`attention` where query row ``i`` attends only to keys
    ``window_lo[.., i] <= j < window_hi[.., i]`` (and the key-padding
    ``attn_mask``).

    ``window_lo``/``window_hi`` are int32 ``(batch, queries)`` or
    ``(queries,)`` on the query's device, shared by all heads.  A row whose
    window holds no attended key returns zeros.  The backward requires both
    bounds to be non-decreasing in the row (true of every window built here)
    and raises otherwise.
    """
    if query.shape[-2] == 0 or key.shape[-2] == 0:
        return torch.zeros_like(query)
    _validate(query, key, value, 0.0, False, enable_gqa)
    mask = _as_key_mask(attn_mask, query.shape[0], query.shape[-2], key.shape[-2])
    out, _ = ops.flash_fwd_windowed(
        query, key, value, window_lo, window_hi, mask, ops.default_scale(query.shape[-1])
    )
    return out


def _leading_count(pred, n: int, shape, device) -> torch.Tensor:
    """Per row, the number of leading ``j`` in ``0..n-1`` with ``pred(j)`` true,
    for a predicate that is true then false along ``j`` (binary lifting over
    the powers of two; ``pred`` takes an int64 index tensor of ``shape``)."""
    pos = torch.zeros(shape, dtype=torch.int64, device=device)
    if n == 0:
        return pos
    step = 1 << (n.bit_length() - 1)
    while step >= 1:
        cand = pos + step
        ok = cand <= n
        idx = torch.where(ok, cand - 1, torch.zeros_like(cand))
        pos = torch.where(ok & pred(idx), cand, pos)
        step >>= 1
    return pos


def temporal_neighbour_windows(
    query_seconds: torch.Tensor, key_seconds: torch.Tensor, *, window_seconds: float
) -> tuple[torch.Tensor, torch.Tensor]:
    """Key windows of the temporal neighbour mask (src/avgen/models/blocks.py
    :97-98): for ``key_seconds`` non-decreasing along each batch row, the
    keys with ``|tq - tk| <= window_seconds`` form one range ``[lo, hi)``.

    The bounds come from a binary search that evaluates the reference's own
    predicate (``tq - tk`` in the coordinates' dtype, compared with the
    Python float), so the windows select exactly the keys the dense mask
    does, ties and rounding included.  For non-decreasing ``query_seconds``
    both bounds are non-decreasing in the row.  Returns int32 ``(batch,
    queries)`` ``(lo, hi)`` on the coordinates' device.
    """
    if query_seconds.ndim != 2 or key_seconds.ndim != 2 or query_seconds.shape[0] != key_seconds.shape[0]:
        raise ValueError(
            f"query_seconds/key_seconds must be (batch, queries)/(batch, keys); got "
            f"{tuple(query_seconds.shape)} and {tuple(key_seconds.shape)}"
        )
    B, Lq = query_seconds.shape
    Lk = key_seconds.shape[1]
    tq = query_seconds

    def delta(j):
        return tq - torch.gather(key_seconds, 1, j)

    # (tq - tk) decreases along sorted keys: "delta > w" holds on a prefix (the
    # keys before the window), "-delta <= w" on a prefix too (up to its end).
    lo = _leading_count(lambda j: ~(delta(j) <= window_seconds), Lk, (B, Lq), tq.device)
    hi = _leading_count(lambda j: (-delta(j)) <= window_seconds, Lk, (B, Lq), tq.device)
    hi = torch.maximum(hi, lo)
    return lo.to(torch.int32), hi.to(torch.int32)


def _is_sorted_rows(t: torch.Tensor) -> torch.Tensor:
    return (t[:, 1:] >= t[:, :-1]).all() if t.shape[1] > 1 else torch.ones((), dtype=torch.bool, device=t.device)


@dataclass(frozen=True)
class TemporalNeighbourhood:
    """The temporal neighbour mask of src/avgen/models/blocks.py:54-104 as
    key windows, built once per forward (as the reference builds its dense
    mask once, src/avgen/models/dit.py:927-942) and reused by every fusion
    block without further host synchronisation.

    ``lo``/``hi`` are int32 ``(batch, queries)`` over the time-sorted key
    order; ``query_order``/``key_order`` (None when already sorted) permute
    tokens into time order and ``query_inverse`` back; ``key_mask`` is the
    key validity in sorted order; ``fallback`` lists, per batch row, the
    (sorted) query rows with no admissible key, which attend to every key;
    ``dense`` marks ``window_seconds <= 0`` (plain key-padding attention).
    """

    lo: torch.Tensor | None
    hi: torch.Tensor | None
    key_mask: torch.Tensor | None
    query_order: torch.Tensor | None
    query_inverse: torch.Tensor | None
    key_order: torch.Tensor | None
    fallback: tuple[tuple[int, torch.Tensor], ...]
    dense: bool
    len_q: int
    len_k: int


def temporal_neighbourhood(
    query_seconds: torch.Tensor,
    key_seconds: torch.Tensor,
    *,
    window_seconds: float,
    key_mask: torch.Tensor | None = None,
) -> TemporalNeighbourhood:
    """Build the :class:`TemporalNeighbourhood` of ``temporal_neighbour_mask(
    query_seconds, key_seconds, window_seconds=..., key_mask=...)``
    (src/avgen/models/blocks.py:54-104).  Two host synchronisations (the
    sortedness test and the fallback rows), here once instead of per block."""
    if query_seconds.ndim != 2 or key_seconds.ndim != 2 or query_seconds.shape[0] != key_seconds.shape[0]:
        raise ValueError(
            f"query_seconds/key_seconds must be (batch, queries)/(batch, keys); got "
            f"{tuple(query_seconds.shape)} and {tuple(key_seconds.shape)}"
        )
    B, Lq = query_seconds.shape
    Lk = key_seconds.shape[1]
    dev = query_seconds.device
    km = None if key_mask is None else key_mask.to(device=dev, dtype=torch.bool)
    if km is not None and tuple(km.shape) != (B, Lk):
        raise ValueError(f"key_mask must be (batch, keys)={(B, Lk)}; got {tuple(km.shape)}")
    if window_seconds <= 0.0 or Lq == 0 or Lk == 0:
        return TemporalNeighbourhood(None, None, km, None, None, None, (), True, Lq, Lk)
    tq = query_seconds
    tk = key_seconds.to(dev)
    sorted_q, sorted_k = (bool(x) for x in torch.stack([_is_sorted_rows(tq), _is_sorted_rows(tk)]).tolist())
    key_order = query_order = query_inverse = None
    if not sorted_k:
        key_order = torch.sort(tk, dim=1, stable=True).indices
        tk = torch.gather(tk, 1, key_order)
        km = None if km is None else torch.gather(km, 1, key_order)
    if not sorted_q:
        query_order = torch.sort(tq, dim=1, stable=True).indices
        query_inverse = torch.argsort(query_order, dim=1)
        tq = torch.gather(tq, 1, query_order)
    lo, hi = temporal_neighbour_windows(tq, tk, window_seconds=window_seconds)
    if km is None:
        empty = hi == lo
    else:
        pre = torch.nn.functional.pad(km.to(torch.int32).cumsum(1), (1, 0))
        empty = (torch.gather(pre, 1, hi.long()) - torch.gather(pre, 1, lo.long())) == 0
    rows = empty.nonzero()
    fallback = []
    if rows.shape[0] > 0:
        for b in rows[:, 0].unique().tolist():
            fallback.append((b, rows[rows[:, 0] == b, 1]))
    return TemporalNeighbourhood(lo, hi, km, query_order, query_inverse, key_order, tuple(fallback), False, Lq, Lk)


def _gather_rows(x: torch.Tensor, order: torch.Tensor) -> torch.Tensor:
    return torch.gather(x, 2, order[:, None, :, None].expand(-1, x.shape[1], -1, x.shape[3]))


def temporal_neighbour_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    query_seconds: torch.Tensor | None = None,
    key_seconds: torch.Tensor | None = None,
    *,
    window_seconds: float | None = None,
    key_mask: torch.Tensor | None = None,
    neighbourhood: TemporalNeighbourhood | None = None,
    enable_gqa: bool = False,
) -> torch.Tensor:
    """``attention(query, key, value, attn_mask=temporal_neighbour_mask(
    query_seconds, key_seconds, window_seconds=..., key_mask=key_mask))``
    without the dense ``(batch, 1, queries, keys)`` mask
    (src/avgen/models/blocks.py:54-104; the fusion call at
    src/avgen/models/dit.py:931-942).

    Same semantics as the reference composition: a query attends to the valid
    keys within ``window_seconds`` of it; ``window_seconds <= 0`` is plain
    key-padding attention; a query with no admissible key attends to every
    key, masked ones included (:101-103).  Pass either the coordinates
    (``(batch, tokens)`` seconds) with ``window_seconds``/``key_mask``, or a
    ``neighbourhood`` from :func:`temporal_neighbourhood` built once for
    several calls (then this call does no host synchronisation).  Tokens out
    of time order are permuted into it and back (attention is invariant
    under a permutation of the keys and equivariant under one of the
    queries).
    """
    if query.shape[-2] == 0 or key.shape[-2] == 0:
        return torch.zeros_like(query)
    _validate(query, key, value, 0.0, False, enable_gqa)
    B, Lq, Lk = query.shape[0], query.shape[-2], key.shape[-2]
    nb = neighbourhood
    if nb is None:
        if query_seconds is None or key_seconds is None or window_seconds is None:
            raise ValueError("pass query_seconds, key_seconds and window_seconds, or a neighbourhood")
        if tuple(query_seconds.shape) != (B, Lq) or tuple(key_seconds.shape) != (B, Lk):
            raise ValueError(
                f"query_seconds must be {(B, Lq)} and key_seconds {(B, Lk)}; got "
                f"{tuple(query_seconds.shape)} and {tuple(key_seconds.shape)}"
            )
        nb = temporal_neighbourhood(query_seconds.to(query.device), key_seconds.to(query.device),
                                    window_seconds=window_seconds, key_mask=key_mask)
    elif (nb.len_q, nb.len_k) != (Lq, Lk):
        raise ValueError(f"neighbourhood was built for {(nb.len_q, nb.len_k)} tokens; got {(Lq, Lk)}")
    scale = ops.default_scale(query.shape[-1])
    if nb.dense:
        return ops.flash_fwd(query, key, value, nb.key_mask, None, None, scale)[0]
    if nb.key_order is not None:
        key = _gather_rows(key, nb.key_order)
        value = _gather_rows(value, nb.key_order)
    if nb.query_order is not None:
        query = _gather_rows(query, nb.query_order)
    out, _ = ops.flash_fwd_windowed(query, key, value, nb.lo, nb.hi, nb.key_mask, scale, True)
    if nb.fallback:
        out = out.clone()
        for b, r in nb.fallback:
            qb = query[b:b + 1].index_select(2, r)
            ob, _ = ops.flash_fwd(qb, key[b:b + 1], value[b:b + 1], None, None, None, scale)
            out[b, :, r] = ob[0]
    if nb.query_inverse is not None:
        out = _gather_rows(out, nb.query_inverse)
    return out


def packed_windows(cu_seqlens: torch.Tensor, length: int, *, device=None) -> tuple[torch.Tensor, torch.Tensor]:
    """Key windows of a packed sequence's block-diagonal mask
    (src/avgen/data/packing.py:181-200): row ``i`` of segment ``s`` attends
    keys ``[cu[s], cu[s+1])``; rows past ``cu[-1]`` (padding) get the empty
    window ``[cu[-1], cu[-1])`` and no window reaches a padding key.  Returns
    int32 ``(length,)`` ``(lo, hi)``, both non-decreasing."""
    cu = cu_seqlens.to(device=device if device is not None else cu_seqlens.device, dtype=torch.int64)
    if cu.ndim != 1 or cu.numel() < 1:
        raise ValueError(f"cu_seqlens must be a non-empty 1-D tensor; got {tuple(cu_seqlens.shape)}")
    i = torch.arange(length, device=cu.device)
    seg = torch.searchsorted(cu[1:].contiguous(), i, right=True)
    ext = torch.cat([cu, cu[-1:]])
    return ext[seg].to(torch.int32), ext[seg + 1].to(torch.int32)


def varlen_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    cu_seqlens: torch.Tensor,
    *,
    enable_gqa: bool = False,
) -> torch.Tensor:
    """Attention over packed variable-length sequences: what
    ``attention(q, k, v, attn_mask=layout.attention_mask())`` computes
    (src/avgen/data/packing.py:181-200), from ``layout.cu_seqlens``
    (:163-179) instead of the ``(capacity, capacity)`` mask.

    ``query``/``key``/``value`` share the packed length; every batch row uses
    the same ``cu_seqlens`` (int32 ``(segments + 1,)``, on any device).
    Tokens attend within their own segment only; padding rows (past
    ``cu_seqlens[-1]``) attend to nothing and return zeros.
    """
    if query.shape[-2] != key.shape[-2]:
        raise ValueError("varlen_attention: query and key must share the packed length")
    if query.shape[-2] == 0:
        return torch.zeros_like(query)
    if int(cu_seqlens[-1]) > query.shape[-2]:
        raise ValueError(
            f"varlen_attention: cu_seqlens ends at {int(cu_seqlens[-1])}, past the packed length "
            f"{query.shape[-2]}"
        )
    _validate(query, key, value, 0.0, False, enable_gqa)
    lo, hi = packed_windows(cu_seqlens, query.shape[-2], device=query.device)
    out, _ = ops.flash_fwd_windowed(query, key, value, lo, hi, None, ops.default_scale(query.shape[-1]), True)
    return out
