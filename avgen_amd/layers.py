"""The attention section of ``SelfAttention.forward`` on the gfx950 kernels
(src/avgen/models/layers.py:530-545): everything between the q/k/v
projections and ``out_proj``.

The reference splits heads with ``unflatten(-1, (-1, head_dim)).transpose(1,
2)`` (:496-504), normalises q and k (``q_norm``/``k_norm``, RMSNorm with a
bf16 gain, :106-118), rotates them (``apply_rotary``, :535-536), runs
attention, and flattens ``out.transpose(1, 2)`` for ``out_proj`` (:545) —
a copy, since SDPA's output is ``(batch, heads, seq, dim)``.

Here the head split stays a strided view of the projection output
``(batch, seq, heads*dim)``, the norm and rotation are one HBM pass
(:func:`avgen_amd.ops.qk_norm_rope`) whose output keeps that
``(batch, seq, heads, dim)`` layout, and the attention kernel, which takes
and produces any such layout, writes its output in it too, so the final
``transpose(1, 2).flatten(2)`` is a view: no copy on either side of the
kernel, forward or backward.
"""

from __future__ import annotations

import torch

from . import attention as _attention
from . import ops
from .rope import RotaryTables

__all__ = ["qk_norm_rope", "self_attention_core", "split_heads"]


def split_heads(projected: torch.Tensor, head_dim: int) -> torch.Tensor:
    """``(batch, seq, heads*head_dim)`` -> ``(batch, heads, seq, head_dim)``
    view (src/avgen/models/layers.py:496-504), no copy."""
    return projected.unflatten(-1, (-1, head_dim)).transpose(1, 2)


def qk_norm_rope(
    x: torch.Tensor, weight: torch.Tensor | None, *, eps: float = 1e-6, tables: RotaryTables | None = None
) -> torch.Tensor:
    """``apply_rotary(rms_norm(x) * weight, tables)`` in one pass
    (src/avgen/models/layers.py:530-536); ``weight`` None: no gain (the
    rotation alone when ``tables`` is also None is :func:`avgen_amd.rope.apply_rotary`).
    Differentiable in ``x`` and ``weight``; the output keeps ``x``'s layout."""
    cos = sin = None
    if tables is not None:
        cos, sin = tables.cos, tables.sin
    return ops.qk_norm_rope(x, weight, float(eps), cos, sin)


def _prepare(x: torch.Tensor, weight, eps, tables):
    if weight is None and tables is None:
        return x
    if weight is None:
        return ops.rope_apply(x, tables.cos, tables.sin, False)
    return qk_norm_rope(x, weight, eps=eps, tables=tables)


def self_attention_core(
    q_proj: torch.Tensor,
    k_proj: torch.Tensor,
    v_proj: torch.Tensor,
    *,
    head_dim: int,
    q_norm_weight: torch.Tensor | None = None,
    k_norm_weight: torch.Tensor | None = None,
    eps: float = 1e-6,
    rope: RotaryTables | None = None,
    key_mask: torch.Tensor | None = None,
) -> torch.Tensor:
    """src/avgen/models/layers.py:530-545 between the projections and
    ``out_proj``: split heads, RMSNorm q and k (gains ``q_norm_weight`` /
    ``k_norm_weight``; None = the reference's ``qk_norm=False`` identity),
    rotate both with ``rope``, attend (``key_mask`` as built by
    :func:`avgen_amd.attention.key_padding_mask`; grouped-query when k has
    fewer heads), and flatten the heads back.

    Args:
        q_proj: ``(batch, seq, heads*head_dim)`` bf16 output of ``q_proj``.
        k_proj, v_proj: ``(batch, seq, kv_heads*head_dim)``.

    Returns:
        ``(batch, seq, heads*head_dim)``, ready for ``out_proj`` — a view of
        the attention kernel's output, which is written in that layout.
    """
    q = _prepare(split_heads(q_proj, head_dim), q_norm_weight, eps, rope)
    k = _prepare(split_heads(k_proj, head_dim), k_norm_weight, eps, rope)
    v = split_heads(v_proj, head_dim)
    out = _attention.attention(q, k, v, attn_mask=key_mask, enable_gqa=q.shape[1] != k.shape[1])
    return out.transpose(1, 2).flatten(2)
