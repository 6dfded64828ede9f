"""The reference hot path written in PyTorch CPU ops — test oracle and timed
CPU baseline only.

The reference is PyTorch code, so restating it in the same PyTorch
operations on the CPU reproduces its algorithm: RoPE tables and rotation as
src/avgen/models/rope.py:264-294,332-338, attention through PyTorch's CPU
flash-attention kernel (what F.scaled_dot_product_attention at
src/avgen/models/attention.py:265-273 dispatches to on the CPU, here called
directly so the LSE is available), the ring loop and merge of
torch/.../_context_parallel/_attention.py:422-478 with the formula at
:182-183, and the ring backward of :514-646.
"""

from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn.functional as F

_flash_cpu = torch.ops.aten._scaled_dot_product_flash_attention_for_cpu
_flash_cpu_bwd = torch.ops.aten._scaled_dot_product_flash_attention_for_cpu_backward


def rope_axis_pairs(head_dim: int) -> tuple[int, int, int]:
    """src/avgen/models/rope.py:150-157."""
    pairs = head_dim // 2
    spatial = pairs // 3
    return (pairs - 2 * spatial, spatial, spatial)


def rotary_tables(coords: torch.Tensor, head_dim: int, theta: float = 10000.0, time_scale: float = 1.0,
                  scaling: tuple[str, float, float] = ("none", 1.0, 1.0)) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin ``(B, 1, L, pairs)`` with the reference's float32 op sequence
    (src/avgen/models/rope.py:264-294)."""
    mode, tf, sf = scaling
    angles = []
    for axis, (pairs, factor) in enumerate(zip(rope_axis_pairs(head_dim), (tf, sf, sf))):
        axis_theta = theta
        position = coords[..., axis]
        if axis == 0 and time_scale != 1.0:
            position = position * time_scale
        if mode == "linear" and factor != 1.0:
            position = position / factor
        elif mode == "ntk" and factor != 1.0:
            dim = 2 * pairs
            if dim > 2:
                axis_theta = theta * factor ** (dim / (dim - 2))
        exponent = torch.arange(pairs, dtype=torch.float32) / pairs
        inv = torch.pow(torch.tensor(axis_theta, dtype=torch.float32), -exponent)
        angles.append(position[..., None] * inv)
    phase = torch.cat(angles, dim=-1)[:, None]
    return torch.cos(phase), torch.sin(phase)


def apply_rotary(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """src/avgen/models/rope.py:332-338 (differentiable)."""
    pairs = x.float().unflatten(-1, (cos.shape[-1], 2))
    even = pairs[..., 0]
    odd = pairs[..., 1]
    rotated = torch.stack((even * cos - odd * sin, even * sin + odd * cos), dim=-1)
    return rotated.flatten(-2).to(x.dtype)


def _bias(key_mask: Optional[torch.Tensor], dtype: torch.dtype) -> Optional[torch.Tensor]:
    if key_mask is None:
        return None
    zero = torch.zeros((), dtype=dtype)
    return torch.where(key_mask, zero, torch.tensor(float("-inf"), dtype=dtype))[:, None, None, :]


def sdpa(q, k, v, key_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
    """F.scaled_dot_product_attention with a boolean key mask (True = attend),
    src/avgen/models/attention.py:265-273."""
    m = None if key_mask is None else key_mask[:, None, None, :]
    return F.scaled_dot_product_attention(q, k, v, attn_mask=m)


def chunk_fwd(q, k, v, key_mask=None, scale=None):
    """One ring step on the CPU: ``(out, lse)``.  A fully masked row has
    out 0 and lse -inf here (PyTorch's CPU kernel reports 0; the merge's
    identity element is -inf)."""
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    bias = _bias(key_mask, q.dtype)
    if bias is not None:
        bias = bias.expand(q.shape[0], q.shape[1], q.shape[2], k.shape[2])
    out, lse = _flash_cpu(q, k, v, 0.0, False, attn_mask=bias, scale=scale)
    if key_mask is not None:
        empty = ~key_mask.any(dim=-1)
        lse = torch.where(empty[:, None, None], torch.tensor(float("-inf")), lse)
    return out, lse


def chunk_bwd(dout, q, k, v, out, lse, key_mask=None, scale=None):
    """One ring backward step on the CPU with merged out/lse."""
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    bias = _bias(key_mask, q.dtype)
    if bias is not None:
        bias = bias.expand(q.shape[0], q.shape[1], q.shape[2], k.shape[2])
    lse = torch.where(torch.isneginf(lse), torch.tensor(float("inf")), lse)
    return _flash_cpu_bwd(dout, q, k, v, out, lse, 0.0, False, attn_mask=bias, scale=scale)


def merge(out, lse, out_b, lse_b):
    """``_SDPAMerger._merge_one`` (torch/.../_attention.py:182-183) in fp32 on
    (B,H,L,1)-shaped LSEs, with -inf as the identity element."""
    lse4, lse_b4 = lse[..., None], lse_b[..., None]
    new_out = out - torch.sigmoid(lse_b4 - lse4) * (out - out_b)
    new_lse = lse4 - F.logsigmoid(lse4 - lse_b4)
    b_empty = torch.isneginf(lse_b4)
    a_empty = torch.isneginf(lse4) & ~b_empty
    new_out = torch.where(b_empty, out, torch.where(a_empty, out_b, new_out))
    new_lse = torch.where(b_empty, lse4, torch.where(a_empty, lse_b4, new_lse))
    return new_out, new_lse[..., 0]


def ring_forward(q, keys, values, masks=None, scale=None):
    """torch/.../_attention.py:422-478 (non-causal): fp32 merge, cast back."""
    masks = masks if masks is not None else [None] * len(keys)
    acc_out = acc_lse = None
    for k, v, m in zip(keys, values, masks):
        out, lse = chunk_fwd(q, k, v, m, scale)
        out, lse = out.float(), lse.float()
        if acc_out is None:
            acc_out, acc_lse = out, lse
        else:
            acc_out, acc_lse = merge(acc_out, acc_lse, out, lse)
    return acc_out.to(q.dtype), acc_lse


def ring_backward(dout, q, keys, values, out, lse, masks=None, scale=None):
    """torch/.../_attention.py:514-646 (non-causal): dq accumulated in fp32."""
    masks = masks if masks is not None else [None] * len(keys)
    dq = torch.zeros(q.shape, dtype=torch.float32)
    dks, dvs = [], []
    for k, v, m in zip(keys, values, masks):
        a, b, c = chunk_bwd(dout, q, k, v, out, lse, m, scale)
        dq += a
        dks.append(b)
        dvs.append(c)
    return dq.to(q.dtype), dks, dvs


def reference_step(q, k, v, cos_q, sin_q, cos_k, sin_k, dout, cp: int, key_mask=None):
    """One fwd+bwd of the ring local step with RoPE, as the reference would
    run it on the CPU: rotate q (local shard) and k (all chunks), ring forward
    over ``cp`` contiguous KV chunks with the merge, ring backward with the
    merged out/lse, then the rotation's autograd for dq/dk.

    Returns ``(out, lse, dq, dk, dv)``.
    """
    qg = q.detach().requires_grad_(True)
    kg = k.detach().requires_grad_(True)
    q_rot = apply_rotary(qg, cos_q, sin_q)
    k_rot = apply_rotary(kg, cos_k, sin_k)
    L = k.shape[2]
    n = L // cp
    keys = [k_rot.detach()[:, :, i * n:(i + 1) * n] for i in range(cp)]
    values = [v[:, :, i * n:(i + 1) * n] for i in range(cp)]
    masks = None if key_mask is None else [key_mask[:, i * n:(i + 1) * n] for i in range(cp)]
    out, lse = ring_forward(q_rot.detach(), keys, values, masks)
    dq_rot, dks, dvs = ring_backward(dout, q_rot.detach(), keys, values, out, lse, masks)
    torch.autograd.backward([q_rot, k_rot], [dq_rot, torch.cat(dks, dim=2)])
    return out, lse, qg.grad, kg.grad, torch.cat(dvs, dim=2)
