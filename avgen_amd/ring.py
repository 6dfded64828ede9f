"""Ring-attention local step, LSE merge and a one-GPU emulated ring.

The callables here keep the shapes of what PyTorch's context-parallel ring
calls for each KV chunk, so they drop into that loop
(torch/distributed/tensor/experimental/_context_parallel/_attention.py):

* :func:`flash_attention_op` — the ``op(q, k, v, is_causal=..., **kwargs)``
  of :309-478 (aten::_scaled_dot_product_flash_attention's 9-tuple);
* :func:`flash_attention_backward_op` — the backward ``op(grad_out=...,
  query=..., key=..., value=..., out=..., logsumexp=..., ...)`` of :567-575;
* :class:`SDPAMerger` — ``_SDPAMerger`` (:138-223): ``step(out, lse,
  partial)`` / ``results()``, fp32 accumulation, merge in a HIP kernel.

:func:`ring_attention_forward` / :func:`ring_attention_backward` replay the
non-causal ring (:422-478 and :514-646) on one GPU by looping over the KV
chunks in order, with no collectives; :func:`ring_attention` wraps both as a
differentiable function over contiguous shards
(src/avgen/parallel/context.py:58-80).
"""

from __future__ import annotations

from collections.abc import Sequence
from typing import Any, Optional

import torch

from . import ops
from .context import shard_bounds
from .rope import RotaryTables

__all__ = [
    "SDPAMerger",
    "flash_attention_backward_op",
    "flash_attention_op",
    "ring_attention",
    "ring_attention_backward",
    "ring_attention_forward",
]


def _key_mask(attn_mask: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    if attn_mask is None:
        return None
    if attn_mask.ndim == 4:
        if attn_mask.shape[1] != 1 or attn_mask.shape[2] != 1:
            raise NotImplementedError("only key-padding masks (batch, 1, 1, keys) are supported")
        return attn_mask[:, 0, 0, :]
    return attn_mask


def flash_attention_op(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    dropout_p: float = 0.0,
    is_causal: bool = False,
    return_debug_mask: bool = False,
    *,
    scale: Optional[float] = None,
    attn_mask: Optional[torch.Tensor] = None,
) -> tuple[Any, ...]:
    """One ring step: attention of the local query shard against one KV chunk.

    Returns aten::_scaled_dot_product_flash_attention's 9-tuple ``(output,
    logsumexp, cum_seq_q, cum_seq_k, max_q, max_k, rng_state, unused,
    debug_attn_mask)``; only the first two carry data.  ``logsumexp`` is
    ``(batch, heads, queries)`` float32, natural log, -inf for rows with no
    valid key.  ``attn_mask`` (an extension) is a key-padding mask.
    """
    if dropout_p != 0.0:
        raise NotImplementedError("dropout is not supported")
    if is_causal:
        raise NotImplementedError("the video DiT ring step is non-causal")
    if return_debug_mask:
        raise NotImplementedError("return_debug_mask is not supported")
    s = ops.default_scale(query.shape[-1]) if scale is None else float(scale)
    out, lse = ops.flash_fwd(query, key, value, _key_mask(attn_mask), None, None, s)
    empty = query.new_empty(0)
    return out, lse, None, None, query.shape[-2], key.shape[-2], empty, empty, empty


def flash_attention_backward_op(
    grad_out: torch.Tensor,
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    out: torch.Tensor,
    logsumexp: torch.Tensor,
    cum_seq_q: Any = None,
    cum_seq_k: Any = None,
    max_q: int = 0,
    max_k: int = 0,
    dropout_p: float = 0.0,
    is_causal: bool = False,
    philox_seed: Any = None,
    philox_offset: Any = None,
    *,
    scale: Optional[float] = None,
    attn_mask: Optional[torch.Tensor] = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Backward of one ring step given the *merged* ``out``/``logsumexp``
    (torch/.../_attention.py:567-575).  Returns this chunk's ``(dq, dk, dv)``
    in the input dtype."""
    del cum_seq_q, cum_seq_k, max_q, max_k, philox_seed, philox_offset
    if dropout_p != 0.0 or is_causal:
        raise NotImplementedError("only non-causal, dropout-free attention is supported")
    s = ops.default_scale(query.shape[-1]) if scale is None else float(scale)
    return ops.flash_bwd(grad_out, query, key, value, out, logsumexp, _key_mask(attn_mask), s)


class SDPAMerger:
    """Running merge of per-chunk ``(out, lse)`` (torch/.../_attention.py:138-223).

    ``convert_to_f32`` must be True (the accumulator is fp32, as torch's
    default ``_cp_options.convert_to_f32``); ``partial`` (round-robin
    load balancing, causal only) is not supported.
    """

    def __init__(self, convert_to_f32: bool = True, seq_dim: int = 2) -> None:
        if not convert_to_f32:
            raise NotImplementedError("the merge accumulates in float32")
        if seq_dim != 2:
            raise NotImplementedError("sequence dim must be 2 for (batch, heads, seq, dim)")
        self._out: Optional[torch.Tensor] = None
        self._lse: Optional[torch.Tensor] = None
        self._out_dtype = torch.float32
        self._lse_dtype = torch.float32

    def step(self, out: torch.Tensor, lse: torch.Tensor, partial: bool = False) -> None:
        """Merge one chunk's output (bf16 or fp32) and LSE (fp32)."""
        if partial:
            raise NotImplementedError("partial (causal load-balanced) merges are not supported")
        self._out_dtype = out.dtype
        self._lse_dtype = lse.dtype
        if self._out is None:
            # One copy (a dtype change alone already copies; copy=True covers
            # inputs that are fp32 and contiguous already).
            self._out = out.to(torch.float32, memory_format=torch.contiguous_format, copy=True)
            self._lse = lse.to(torch.float32, memory_format=torch.contiguous_format, copy=True)
            return
        ops.lse_merge_(self._out, self._lse, out, lse.to(torch.float32))

    def results(self) -> tuple[torch.Tensor, torch.Tensor]:
        """``(out, lse)`` cast back to the dtypes of the last step."""
        assert self._out is not None and self._lse is not None
        return self._out.to(self._out_dtype), self._lse.to(self._lse_dtype)


def _chunk_masks(key_masks, n):
    if key_masks is None:
        return [None] * n
    if len(key_masks) != n:
        raise ValueError(f"{len(key_masks)} key masks for {n} chunks")
    return list(key_masks)


def ring_attention_forward(
    query: torch.Tensor,
    keys: Sequence[torch.Tensor],
    values: Sequence[torch.Tensor],
    *,
    key_masks: Optional[Sequence[Optional[torch.Tensor]]] = None,
    scale: Optional[float] = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Non-causal ring forward over KV chunks in ring order
    (torch/.../_attention.py:422-478): per chunk ``flash_attention_op`` then
    ``SDPAMerger.step``.  Returns ``(out, lse)``."""
    if len(keys) != len(values) or not keys:
        raise ValueError("need the same, non-zero number of key and value chunks")
    masks = _chunk_masks(key_masks, len(keys))
    merger = SDPAMerger(True, 2)
    for k, v, m in zip(keys, values, masks):
        out, lse, *_ = flash_attention_op(query, k, v, scale=scale, attn_mask=m)
        merger.step(out, lse, False)
    return merger.results()


def ring_attention_backward(
    grad_out: torch.Tensor,
    query: torch.Tensor,
    keys: Sequence[torch.Tensor],
    values: Sequence[torch.Tensor],
    out: torch.Tensor,
    lse: torch.Tensor,
    *,
    key_masks: Optional[Sequence[Optional[torch.Tensor]]] = None,
    scale: Optional[float] = None,
) -> tuple[torch.Tensor, list[torch.Tensor], list[torch.Tensor]]:
    """Non-causal ring backward (torch/.../_attention.py:514-646): each chunk's
    backward uses the merged ``out``/``lse``; dq accumulates in fp32 and is
    cast once; each chunk's dk/dv is that chunk's gradient (on a real ring it
    travels back to the chunk's owner)."""
    masks = _chunk_masks(key_masks, len(keys))
    dq_acc = None
    dks, dvs = [], []
    for k, v, m in zip(keys, values, masks):
        dq_i, dk_i, dv_i = flash_attention_backward_op(
            grad_out, query, k, v, out, lse, scale=scale, attn_mask=m
        )
        dq_acc = dq_i.float() if dq_acc is None else dq_acc.add_(dq_i)
        dks.append(dk_i)
        dvs.append(dv_i)
    return dq_acc.to(query.dtype), dks, dvs


def _ring_workspace(B, Hq, Hkv, Lq, D, bounds, device):
    """One backward workspace for every chunk of the ring: that of the longest
    chunk (chunks of a contiguous split differ by at most one key)."""
    longest = max(b - a for a, b in bounds)
    return ops._alloc_bwd_workspace(B, Hq, Hkv, Lq, longest, D, device)


def _ring_backward_into(grad_out, query, key, value, out, lse, key_mask, cp, scale, overlap=False):
    """The emulated ring's backward.  Each chunk's dk/dv goes straight into its
    slice of the full-sequence gradients (one chunk, one contribution, so no
    accumulation or concatenation is needed); dq accumulates in fp32 as in
    the torch ring (torch/.../_attention.py:505-506, 623, 636), inside the
    kernel; the query-side preparation (copies of q and dout, softmax
    statistics) is made once per workspace and reused for the other chunks.

    With ``overlap`` chunk r's dq (a memory-bound product of the staged dS
    with k) runs on a side stream while chunk r+1's dk/dv (compute-bound) run
    on the current one; two workspaces alternate, each reused only once its
    dq has finished.  Off by default: on one MI355X at the c3 ring shape the
    concurrent kernels slowed each other (both power- and HBM-limited) and
    the step took 3% longer than running them in turn."""
    L = key.shape[2]
    D = query.shape[-1]
    scale = ops.default_scale(D) if scale is None else float(scale)
    dk = torch.empty(key.shape, dtype=key.dtype, device=key.device)
    dv = torch.empty(value.shape, dtype=value.dtype, device=value.device)
    dq_acc = torch.zeros(query.shape, dtype=torch.float32, device=query.device)
    from . import _lib

    lib = _lib.load()
    B, Hq, Lq, _ = query.shape
    Hkv = key.shape[1]
    bounds = [shard_bounds(L, cp, r) for r in range(cp)]
    masks = [None if key_mask is None else key_mask[:, a:b] for a, b in bounds]
    full = max(lib.avattn_bwd_staged_workspace_size(B, Hq, Hkv, Lq, b - a, D, B * Hkv) for a, b in bounds)
    if overlap and not (cp > 1 and full > 0):
        overlap = False
    if overlap:
        dev = query.device
        ws = [ops._workspace(full, dev) for _ in range(2)]
        main = torch.cuda.current_stream(dev)
        side = torch.cuda.Stream(dev)
        done = [None, None]
        for r, (a, b) in enumerate(bounds):
            w = r % 2
            if done[w] is not None:
                main.wait_event(done[w])  # chunk r-2's dq has read this workspace
            ops._bwd_impl(grad_out, query, key[:, :, a:b], value[:, :, a:b], out, lse, masks[r], scale,
                          dk=dk[:, :, a:b], dv=dv[:, :, a:b], workspace=ws[w], reuse_query_side=r >= 2,
                          stage_ds=True, defer_dq=True)
            ready = torch.cuda.Event()
            ready.record(main)
            side.wait_event(ready)
            with torch.cuda.stream(side):
                ops._bwd_dq_staged_impl(query, Hkv, b - a, scale, ws[w], dq_accumulate=dq_acc)
                done[w] = torch.cuda.Event()
                done[w].record(side)
        main.wait_stream(side)
    else:
        ws = _ring_workspace(B, Hq, Hkv, Lq, D, bounds, query.device)
        for r, (a, b) in enumerate(bounds):
            ops._bwd_impl(grad_out, query, key[:, :, a:b], value[:, :, a:b], out, lse, masks[r], scale,
                          dk=dk[:, :, a:b], dv=dv[:, :, a:b], workspace=ws, reuse_query_side=r > 0,
                          dq_accumulate=dq_acc)
    return dq_acc.to(query.dtype), dk, dv


def _chunk_tables(tables, a, b):
    return None if tables is None else tables.slice(a, b)


def _ring_forward_fused(query, key, value, key_mask, cp, scale, tables_q, tables_k):
    """The emulated ring forward with RoPE and the merge fused into each
    chunk's launch (``ops.ring_fwd_step_``): q and k are unrotated, each
    chunk rotates its keys in its operand copy and the query shard on load,
    and merges into one fp32 accumulator; the last chunk writes the bf16
    output.  Same bits as apply_rotary + :func:`ring_attention_forward`."""
    B, Hq, Lq, D = query.shape
    L = key.shape[2]
    if L == 0 or Lq == 0:
        # No keys: zeros (src/avgen/models/attention.py:261-262), lse -inf.
        return torch.zeros_like(query), torch.full((B, Hq, Lq), float("-inf"), device=query.device)
    bounds = [shard_bounds(L, cp, r) for r in range(cp)]
    acc = torch.empty(query.shape, dtype=torch.float32, device=query.device)
    lse = torch.empty((B, Hq, Lq), dtype=torch.float32, device=query.device)
    out = ops._kernel_ready(torch.empty_like(query, memory_format=torch.preserve_format))
    for r, (a, b) in enumerate(bounds):
        ops.ring_fwd_step_(query, key[:, :, a:b], value[:, :, a:b],
                           None if key_mask is None else key_mask[:, a:b], tables_q,
                           _chunk_tables(tables_k, a, b), scale, acc, lse, out,
                           first=r == 0, last=r == cp - 1)
    return out, lse


def _ring_backward_fused(grad_out, query, key, value, out, lse, key_mask, cp, scale, tables_q, tables_k):
    """The emulated ring backward with RoPE fused in (``ops.ring_bwd_step``):
    each chunk's dk/dv land in their slice of the full-sequence gradients
    (dk already of the unrotated keys), dq (of the rotated query) sums in fp32
    across chunks and ``ops.ring_dq_finish`` casts and un-rotates it once.
    Same bits as :func:`_ring_backward_into` followed by apply_rotary's
    backward on dq and dk."""
    L = key.shape[2]
    B, Hq, Lq, D = query.shape
    Hkv = key.shape[1]
    dk = torch.empty(key.shape, dtype=key.dtype, device=key.device)
    dv = torch.empty(value.shape, dtype=value.dtype, device=value.device)
    dq = ops._kernel_ready(torch.empty_like(query, memory_format=torch.preserve_format))
    if L == 0 or Lq == 0:
        return dq.zero_(), dk.zero_(), dv.zero_()
    dq_acc = torch.zeros(query.shape, dtype=torch.float32, device=query.device)
    bounds = [shard_bounds(L, cp, r) for r in range(cp)]
    ws = _ring_workspace(B, Hq, Hkv, Lq, D, bounds, query.device)
    for r, (a, b) in enumerate(bounds):
        ops.ring_bwd_step(grad_out, query, key[:, :, a:b], value[:, :, a:b], out, lse,
                          None if key_mask is None else key_mask[:, a:b], tables_q, _chunk_tables(tables_k, a, b),
                          scale, dq_acc, dk[:, :, a:b], dv[:, :, a:b], workspace=ws, reuse_query_side=r > 0)
    ops.ring_dq_finish(dq_acc, tables_q, dq)
    return dq, dk, dv


# The RoPE-fused emulated ring as one op pair with registered autograd: a
# compiled region (torch.compile per block, src/avgen/parallel/apply.py
# :216-221) sees two opaque ops, whose implementations run the per-chunk
# step ops above in ring order.


@torch.library.custom_op("avgen_amd::ring_attention_rope", mutates_args=())
def _ring_attention_rope_op(
    query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, key_mask: Optional[torch.Tensor],
    cos_q: torch.Tensor, sin_q: torch.Tensor, cos_k: torch.Tensor, sin_k: torch.Tensor, cp: int, scale: float,
) -> tuple[torch.Tensor, torch.Tensor]:
    return _ring_forward_fused(query, key, value, key_mask, cp, scale, RotaryTables(cos_q, sin_q),
                               RotaryTables(cos_k, sin_k))


@_ring_attention_rope_op.register_fake
def _(query, key, value, key_mask, cos_q, sin_q, cos_k, sin_k, cp, scale):
    B, H, Lq, _ = query.shape
    return torch.empty_like(query), query.new_empty((B, H, Lq), dtype=torch.float32)


@torch.library.custom_op("avgen_amd::ring_attention_rope_bwd", mutates_args=())
def _ring_attention_rope_bwd_op(
    grad_out: torch.Tensor, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, out: torch.Tensor,
    lse: torch.Tensor, key_mask: Optional[torch.Tensor], cos_q: torch.Tensor, sin_q: torch.Tensor,
    cos_k: torch.Tensor, sin_k: torch.Tensor, cp: int, scale: float,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return _ring_backward_fused(grad_out.contiguous(), query, key, value, out, lse, key_mask, cp, scale,
                                RotaryTables(cos_q, sin_q), RotaryTables(cos_k, sin_k))


@_ring_attention_rope_bwd_op.register_fake
def _(grad_out, query, key, value, out, lse, key_mask, cos_q, sin_q, cos_k, sin_k, cp, scale):
    return torch.empty_like(query), key.new_empty(key.shape), value.new_empty(value.shape)


def _ring_rope_setup(ctx, inputs, output):
    query, key, value, key_mask, cos_q, sin_q, cos_k, sin_k, cp, scale = inputs
    out, lse = output
    ctx.cp = cp
    ctx.scale = scale
    ctx.save_for_backward(query, key, value, out, lse, key_mask, cos_q, sin_q, cos_k, sin_k)
    ctx.mark_non_differentiable(lse)


def _ring_rope_backward(ctx, grad_out, _grad_lse):
    query, key, value, out, lse, key_mask, cos_q, sin_q, cos_k, sin_k = ctx.saved_tensors
    dq, dk, dv = _ring_attention_rope_bwd_op(grad_out, query, key, value, out, lse, key_mask, cos_q, sin_q, cos_k,
                                             sin_k, ctx.cp, ctx.scale)
    return dq, dk, dv, None, None, None, None, None, None, None


torch.library.register_autograd("avgen_amd::ring_attention_rope", _ring_rope_backward,
                                setup_context=_ring_rope_setup)


class _RingAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, query, key, value, key_mask, cp, scale):
        L = key.shape[2]
        bounds = [shard_bounds(L, cp, r) for r in range(cp)]
        keys = [key[:, :, a:b] for a, b in bounds]
        values = [value[:, :, a:b] for a, b in bounds]
        masks = None if key_mask is None else [key_mask[:, a:b] for a, b in bounds]
        out, lse = ring_attention_forward(query, keys, values, key_masks=masks, scale=scale)
        ctx.save_for_backward(query, key, value, out, lse, key_mask)
        ctx.cp = cp
        ctx.scale = scale
        ctx.mark_non_differentiable(lse)
        return out, lse

    @staticmethod
    def backward(ctx, grad_out, _grad_lse):
        query, key, value, out, lse, key_mask = ctx.saved_tensors
        if query.dtype is torch.float32:
            # float32: the per-chunk backward op (its fp32 kernels) in ring
            # order; the workspace-sharing ring steps are bf16 kernels.
            bounds = [shard_bounds(key.shape[2], ctx.cp, r) for r in range(ctx.cp)]
            masks = None if key_mask is None else [key_mask[:, a:b] for a, b in bounds]
            dq, dks, dvs = ring_attention_backward(grad_out.contiguous(), query,
                                                   [key[:, :, a:b] for a, b in bounds],
                                                   [value[:, :, a:b] for a, b in bounds], out, lse,
                                                   key_masks=masks, scale=ctx.scale)
            return dq, torch.cat(dks, 2), torch.cat(dvs, 2), None, None, None
        dq, dk, dv = _ring_backward_into(grad_out.contiguous(), query, key, value, out, lse, key_mask, ctx.cp,
                                         ctx.scale)
        return dq, dk, dv, None, None, None


def ring_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    *,
    cp: int,
    key_mask: Optional[torch.Tensor] = None,
    scale: Optional[float] = None,
    tables_q=None,
    tables_k=None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Differentiable emulated ring: ``key``/``value`` (full sequence) are split
    into ``cp`` contiguous chunks (ragged lengths raise, as
    src/avgen/parallel/context.py:74-79), the local ``query`` shard attends to
    each in ring order, and results merge online.  Returns ``(out, lse)``.

    With ``tables_q`` / ``tables_k`` (RotaryTables of the query shard's and
    of the full key sequence's positions), ``query`` and ``key`` are the
    UNROTATED tensors and the 3D RoPE of src/avgen/models/rope.py:297-338
    (called at src/avgen/models/layers.py:535-536) is fused into the
    kernels: no separate rotation or merge launches, the same bits as
    ``ring_attention(apply_rotary(q, tables_q), apply_rotary(k, tables_k), v)``
    and the same gradients with respect to the unrotated inputs."""
    if (tables_q is None) != (tables_k is None):
        raise ValueError("pass both tables_q and tables_k, or neither")
    if tables_q is not None:
        shard_bounds(key.shape[2], cp, 0)  # ragged lengths raise before any launch
        if query.dtype is torch.float32:
            # The fused ring steps are bf16 kernels; float32 rotates first (the
            # reference's own order: apply_rotary, then attention) and runs
            # the ring on its fp32 kernels.
            from .rope import apply_rotary

            return _RingAttention.apply(apply_rotary(query, tables_q), apply_rotary(key, tables_k), value, key_mask,
                                        cp, scale)
        s = ops.default_scale(query.shape[-1]) if scale is None else float(scale)
        return _ring_attention_rope_op(query, key, value, key_mask, tables_q.cos, tables_q.sin, tables_k.cos,
                                       tables_k.sin, int(cp), s)
    return _RingAttention.apply(query, key, value, key_mask, cp, scale)
