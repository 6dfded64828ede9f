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
bf16 tensors on a ROCm GPU, head_dim 64 or 128, ``dropout_p == 0``,
``is_causal == False`` (video DiT attention is bidirectional), and masks
that are key-padding masks — boolean, broadcastable as ``(batch, 1, 1,
keys)`` — which is what :func:`key_padding_mask` and CrossAttention build
(src/avgen/models/layers.py:651-657).  Query-dependent dense masks
(src/avgen/models/blocks.py:54-104) are not supported by this kernel.
"""

from __future__ import annotations

from collections.abc import Sequence
from contextlib import AbstractContextManager, nullcontext
from typing import Optional

import torch

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
]

#: The single backend this package provides.
BACKEND = "avattn_gfx950"


def device_arch(device: torch.device | str | None = None) -> str:
    """Architecture family for a device: ``"cdna4"`` on a ROCm GPU, else ``"cpu"``
    (reference classification: src/avgen/models/attention.py:98-130)."""
    if device is None:
        resolved = torch.device("cuda" if torch.cuda.is_available() else "cpu")
    else:
        resolved = torch.device(device)
    if resolved.type != "cuda" or not torch.cuda.is_available():
        return "cpu"
    return "cdna4"


def attention_backends(
    device: torch.device | str | None = None, *, allow_flash: bool = True
) -> tuple[str, ...]:
    """Backend priority list (src/avgen/models/attention.py:133-153).  There is
    exactly one backend — the hand-written gfx950 kernel — and no fallback."""
    del device, allow_flash
    return (BACKEND,)


def sdpa_context(
    device: torch.device | str | None = None, *, backends: Sequence[object] | None = None
) -> AbstractContextManager[None]:
    """No-op context (src/avgen/models/attention.py:156-180): this package does
    not dispatch through PyTorch's SDPA backends."""
    del device, backends
    return nullcontext()


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
        query: ``(batch, heads, queries, head_dim)`` bf16 on a ROCm GPU.
        key/value: ``(batch, kv_heads, keys, head_dim)``.
        attn_mask: ``None`` or a boolean key-padding mask broadcastable as
            ``(batch, 1, 1, keys)``; True = attend.
        dropout_p, is_causal: must be 0 / False.
        enable_gqa: allow ``kv_heads`` dividing ``heads``.
        backends: accepted for signature compatibility; ignored.

    Returns:
        ``(batch, heads, queries, head_dim)`` in query's dtype; differentiable.
    """
    del backends
    if query.shape[-2] == 0 or key.shape[-2] == 0:
        return torch.zeros_like(query)
    _validate(query, key, value, dropout_p, is_causal, enable_gqa)
    mask = _as_key_mask(attn_mask, query.shape[0], query.shape[-2], key.shape[-2])
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
