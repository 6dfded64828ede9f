"""Tensor-level wrappers over the C ABI, registered as ``torch.library`` ops.

Every function here validates shapes/dtypes/devices, allocates outputs with
PyTorch's caching allocator, and launches through ``libavattn.so`` on the
current HIP stream.  There is no fallback: a CPU tensor or a missing library
is an error.

Ops (namespace ``avgen_amd``):

* ``flash_fwd(q, k, v, key_mask, rope_cos, rope_sin, scale) -> (out, lse)`` —
  the ring local step (torch/.../_context_parallel/_attention.py:468-474);
  differentiable in q/k/v (``lse`` is a non-differentiable output).
* ``flash_bwd(dout, q, k, v, out, lse, key_mask, scale) -> (dq, dk, dv)`` —
  the ring backward step (torch/.../_context_parallel/_attention.py:567-575).
* ``rope_apply(x, cos, sin, inverse) -> x_rot`` — src/avgen/models/rope.py
  :297-338, differentiable.

``flash_fwd``, ``flash_bwd``, ``flash_fwd_windowed``, ``flash_bwd_windowed``,
``qk_norm_rope(_bwd)`` and ``rope_apply`` take float32 tensors too (all of q, k, v and dout/out, or
x), computed in fp32 by the library's fp32 kernels (the reference's
attention runs in the caller's dtype); every other op is bf16 only.
* ``flash_fwd_fp8(q, k, v, key_mask, q_scale, k_scale, scale) -> (out, lse)``
  — forward with q k^T on e4m3 operands and per-head scales (no reference
  counterpart; the sampling-time fp8 variant of ``flash_fwd``), forward only.
* ``flash_fwd_windowed(q, k, v, window_lo, window_hi, key_mask, scale)`` /
  ``flash_bwd_windowed(...)`` — every query row i attends only keys
  [window_lo[i], window_hi[i]) (int32, per batch or shared): the temporal
  neighbour mask (src/avgen/models/blocks.py:54-104) and the block-diagonal
  mask of packed variable-length sequences (src/avgen/data/packing.py:185-200)
  as row ranges instead of an (L, L) boolean tensor; differentiable.
* ``qk_norm_rope(x, weight, eps, cos, sin)`` — per-head RMSNorm of q or k
  with a bf16 gain, then the rotation (tables None: norm only), in one pass:
  src/avgen/models/layers.py:530-536; differentiable in ``x`` and ``weight``.
"""

from __future__ import annotations

import ctypes
import math
import os
from typing import Optional

import torch

from . import _lib

__all__ = [
    "flash_fwd",
    "flash_bwd",
    "flash_fwd_fp8",
    "flash_fwd_windowed",
    "flash_bwd_windowed",
    "fp8_absmax_scales",
    "lse_merge_",
    "rope_apply",
    "rope_tables",
    "qk_norm_rope",
    "qk_norm_rope_bwd",
    "default_scale",
    "ring_fwd_step_",
    "ring_bwd_step",
    "ring_dq_finish",
    "set_ds_budget",
]

SUPPORTED_HEAD_DIMS = (64, 128)


def default_scale(head_dim: int) -> float:
    """``1/sqrt(head_dim)``, SDPA's default (src/avgen/models/attention.py:265-273)."""
    return 1.0 / math.sqrt(head_dim)


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _strides3(t: torch.Tensor) -> ctypes.Array:
    return _lib.i64_array(t.stride()[:3])


def _workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """Caller-owned scratch for one C-ABI call (torch's caching allocator; the
    library itself never allocates).  Never empty, so its pointer is valid."""
    return torch.empty(max(int(nbytes), 256), device=device, dtype=torch.uint8)


def _require_gpu(name: str, *tensors: Optional[torch.Tensor]) -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError(
                f"{name}: avgen_amd runs only on a ROCm GPU (got a tensor on {t.device}); "
                "there is no CPU path"
            )


def _check_qkv(name: str, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, allow_f32: bool = False) -> None:
    """Shapes and dtypes: bf16, or (``allow_f32``: the plain forward and
    backward) float32 for all three."""
    for label, t in (("query", q), ("key", k), ("value", v)):
        if t.ndim != 4:
            raise ValueError(f"{name}: {label} must be (batch, heads, seq, head_dim); got {tuple(t.shape)}")
    f32 = allow_f32 and q.dtype is torch.float32
    want = torch.float32 if f32 else torch.bfloat16
    for label, t in (("query", q), ("key", k), ("value", v)):
        if t.dtype is not want:
            if allow_f32:
                raise TypeError(f"{name}: {label} must be bfloat16 or float32 like the query; got {t.dtype} "
                                f"(query {q.dtype})")
            raise TypeError(f"{name}: {label} must be bfloat16; got {t.dtype}")
    if k.shape != v.shape:
        raise ValueError(f"{name}: key {tuple(k.shape)} and value {tuple(v.shape)} shapes differ")
    if q.shape[0] != k.shape[0]:
        raise ValueError(f"{name}: batch mismatch between query {tuple(q.shape)} and key {tuple(k.shape)}")
    if q.shape[-1] != k.shape[-1]:
        raise ValueError(f"{name}: head_dim mismatch between query and key")
    if q.shape[-1] not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"{name}: head_dim {q.shape[-1]} not supported (supported: {SUPPORTED_HEAD_DIMS})")
    if k.shape[1] == 0 or q.shape[1] % k.shape[1] != 0:
        raise ValueError(f"{name}: query heads {q.shape[1]} must be a multiple of key heads {k.shape[1]}")


def _kernel_ready(t: torch.Tensor) -> torch.Tensor:
    """Make the last dim contiguous and row starts 16-byte aligned."""
    ok = t.stride(-1) == 1 and t.data_ptr() % 16 == 0
    ok = ok and all(s % 8 == 0 or n == 1 for s, n in zip(t.stride()[:3], t.shape[:3]))
    return t if ok else t.contiguous()


def _normalise_mask(name: str, key_mask: Optional[torch.Tensor], batch: int, len_k: int):
    """(B|1, Lk) bool/uint8 -> (uint8 tensor, batch stride) or (None, 0)."""
    if key_mask is None:
        return None, 0
    if key_mask.ndim != 2 or key_mask.shape[-1] != len_k or key_mask.shape[0] not in (1, batch):
        raise ValueError(f"{name}: key mask must be (batch, keys) = ({batch}, {len_k}); got {tuple(key_mask.shape)}")
    if key_mask.dtype not in (torch.bool, torch.uint8):
        raise TypeError(f"{name}: key mask must be bool; got {key_mask.dtype}")
    m = key_mask if key_mask.stride(-1) == 1 else key_mask.contiguous()
    if m.dtype is torch.bool:
        m = m.view(torch.uint8)
    stride_b = 0 if m.shape[0] == 1 else m.stride(0)
    return m, stride_b


def _check_tables(name: str, cos: torch.Tensor, sin: torch.Tensor, batch: int, length: int, head_dim: int):
    if cos.ndim != 4 or cos.shape != sin.shape:
        raise ValueError(f"{name}: rotary tables must be (batch, 1, length, pairs) and agree")
    if cos.dtype is not torch.float32 or sin.dtype is not torch.float32:
        raise TypeError(f"{name}: rotary tables must be float32")
    if cos.shape[-1] * 2 != head_dim:
        raise ValueError(
            f"{name}: head_dim {head_dim} does not match rotary tables built for head_dim {2 * cos.shape[-1]}"
        )
    if cos.shape[-2] != length:
        raise ValueError(
            f"{name}: sequence length {length} does not match rotary tables built for length {cos.shape[-2]}"
        )
    if cos.shape[0] not in (1, batch) or cos.shape[1] != 1:
        raise ValueError(f"{name}: rotary tables batch {cos.shape[0]} does not broadcast to {batch}")
    cos = cos if cos.is_contiguous() else cos.contiguous()
    sin = sin if sin.is_contiguous() else sin.contiguous()
    stride_b = 0 if cos.shape[0] == 1 else cos.stride(0)
    return cos, sin, stride_b


# ---------------------------------------------------------------------------
# Eager implementations (called by the custom ops)
# ---------------------------------------------------------------------------


def _fwd_impl(q, k, v, key_mask, rope_cos, rope_sin, scale):
    name = "avgen_amd.flash_fwd"
    _check_qkv(name, q, k, v, allow_f32=True)
    _require_gpu(name, q, k, v, key_mask, rope_cos, rope_sin)
    if q.dtype is torch.float32:
        return _fwd_f32_impl(name, q, k, v, key_mask, rope_cos, rope_sin, scale)
    B, Hq, Lq, D = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    q, k, v = _kernel_ready(q), _kernel_ready(k), _kernel_ready(v)
    mask, msb = _normalise_mask(name, key_mask, B, Lk)
    rsb = 0
    if (rope_cos is None) != (rope_sin is None):
        raise ValueError(f"{name}: pass both rotary tables or neither")
    if rope_cos is not None:
        rope_cos, rope_sin, rsb = _check_tables(name, rope_cos, rope_sin, B, Lq, D)
    out = torch.empty_like(q, memory_format=torch.preserve_format)
    out = _kernel_ready(out)
    lse = torch.empty((B, Hq, Lq), device=q.device, dtype=torch.float32)
    lib = _lib.load()
    ws = _workspace(lib.avattn_fwd_workspace_size(B, Hkv, Lk, D), q.device)
    st = lib.avattn_fwd(
        _ptr(q), _ptr(k), _ptr(v), _strides3(q), _strides3(k), _strides3(v),
        B, Hq, Hkv, Lq, Lk, D,
        _ptr(mask), msb,
        _ptr(rope_cos), _ptr(rope_sin), rsb,
        float(scale),
        _ptr(out), _strides3(out), _ptr(lse),
        _ptr(ws), ws.numel(),
        _stream(q.device),
    )
    _lib.check(st, name)
    return out, lse


def _f32_ready(t: torch.Tensor) -> torch.Tensor:
    """float32 rows for the fp32 kernels: head_dim contiguous, 16-byte aligned
    row starts (strides a multiple of 4 elements)."""
    ok = t.stride(-1) == 1 and t.data_ptr() % 16 == 0
    ok = ok and all(s % 4 == 0 or n == 1 for s, n in zip(t.stride()[:3], t.shape[:3]))
    return t if ok else t.contiguous()


def _fwd_f32_impl(name, q, k, v, key_mask, rope_cos, rope_sin, scale):
    """The float32 forward (``avattn_fwd_f32``); rotary tables rotate q first
    (``avattn_rope_apply_f32``), the same result as rotating it before the
    call."""
    B, Hq, Lq, D = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    if (rope_cos is None) != (rope_sin is None):
        raise ValueError(f"{name}: pass both rotary tables or neither")
    if rope_cos is not None:
        q = _rope_apply_impl(q, rope_cos, rope_sin, False)
    q, k, v = _f32_ready(q), _f32_ready(k), _f32_ready(v)
    mask, msb = _normalise_mask(name, key_mask, B, Lk)
    out = _f32_ready(torch.empty_like(q, memory_format=torch.preserve_format))
    lse = torch.empty((B, Hq, Lq), device=q.device, dtype=torch.float32)
    st = _lib.load().avattn_fwd_f32(
        _ptr(q), _ptr(k), _ptr(v), _strides3(q), _strides3(k), _strides3(v),
        B, Hq, Hkv, Lq, Lk, D,
        _ptr(mask), msb,
        float(scale),
        _ptr(out), _strides3(out), _ptr(lse),
        _stream(q.device),
    )
    _lib.check(st, name)
    return out, lse


def _fwd_windowed_f32_impl(name, q, k, v, lo, hi, wsb, key_mask, scale):
    """The float32 forward with per-row key windows
    (``avattn_fwd_windowed_f32``); ``lo``/``hi``/``wsb`` as checked by
    ``_check_windows``."""
    B, Hq, Lq, D = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    q, k, v = _f32_ready(q), _f32_ready(k), _f32_ready(v)
    mask, msb = _normalise_mask(name, key_mask, B, Lk)
    out = _f32_ready(torch.empty_like(q, memory_format=torch.preserve_format))
    lse = torch.empty((B, Hq, Lq), device=q.device, dtype=torch.float32)
    st = _lib.load().avattn_fwd_windowed_f32(
        _ptr(q), _ptr(k), _ptr(v), _strides3(q), _strides3(k), _strides3(v),
        B, Hq, Hkv, Lq, Lk, D,
        _ptr(mask), msb,
        _ptr(lo), _ptr(hi), wsb,
        float(scale),
        _ptr(out), _strides3(out), _ptr(lse),
        _stream(q.device),
    )
    _lib.check(st, name)
    return out, lse


def _bwd_f32_impl(name, dout, q, k, v, out, lse, key_mask, scale, windows=None):
    """The float32 backward (``avattn_bwd_f32``; with ``windows`` = (lo, hi,
    batch stride), non-decreasing along the queries,
    ``avattn_bwd_windowed_f32``): new dq, dk, dv."""
    B, Hq, Lq, D = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    for label, t in (("grad_out", dout), ("out", out)):
        if t.shape != q.shape:
            raise ValueError(f"{name}: {label} must have the query's shape {tuple(q.shape)}")
        if t.dtype is not torch.float32:
            raise TypeError(f"{name}: {label} must be float32 like the query; got {t.dtype}")
    if lse.shape != (B, Hq, Lq) or lse.dtype is not torch.float32:
        raise ValueError(f"{name}: logsumexp must be float32 (batch, heads, queries)")
    dout, q, k, v, out = (_f32_ready(t) for t in (dout, q, k, v, out))
    lse = lse.contiguous()
    mask, msb = _normalise_mask(name, key_mask, B, Lk)
    dq = _f32_ready(torch.empty_like(q))
    dk = _f32_ready(torch.empty_like(k))
    dv = _f32_ready(torch.empty_like(v))
    lib = _lib.load()
    ws = _alloc_bwd_f32_workspace(B, Hq, Hkv, Lq, Lk, q.device)
    head = (
        _ptr(dout), _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(lse),
        _strides3(dout), _strides3(q), _strides3(k), _strides3(v), _strides3(out),
        B, Hq, Hkv, Lq, Lk, D,
        _ptr(mask), msb,
    )
    if windows is not None:
        lo, hi, wsb = windows
        entry, head = lib.avattn_bwd_windowed_f32, head + (_ptr(lo), _ptr(hi), wsb)
    else:
        entry = lib.avattn_bwd_f32
    st = entry(
        *head,
        float(scale),
        _ptr(dq), _strides3(dq), _ptr(dk), _strides3(dk), _ptr(dv), _strides3(dv),
        _ptr(ws), ws.numel(),
        _stream(q.device),
    )
    _lib.check(st, name)
    return dq, dk, dv


def f32_ds_bytes_per_pair(group, Lq, Lk):
    """Bytes of staged fp32 dS per (batch, kv head) pair: float32 per (query
    head of the group, query row padded to 32, key padded to 128)."""
    return 4 * group * ((Lq + 31) // 32 * 32) * ((Lk + 127) // 128 * 128)


def _alloc_bwd_f32_workspace(B, Hq, Hkv, Lq, Lk, device) -> torch.Tensor:
    """The float32 backward's workspace: with the staged-dS budget (the one
    the bf16 backward uses) holding at least one (batch, kv head) pair's fp32
    dS, the staged size for as many pairs per pass as fit in equal passes
    (halving while the allocator cannot provide it), else the statistics
    alone (dq recomputes S and dP)."""
    lib = _lib.load()
    pairs = 0
    if B * Hkv > 0 and Lq > 0 and Lk > 0:
        pairs = min(B * Hkv, _ds_budget(device) // f32_ds_bytes_per_pair(Hq // Hkv, Lq, Lk))
    if pairs > 0:
        npass = -(-(B * Hkv) // pairs)
        pairs = -(-(B * Hkv) // npass)
    while pairs > 0:
        try:
            return _workspace(lib.avattn_bwd_f32_staged_workspace_size(B, Hq, Hkv, Lq, Lk, int(pairs)), device)
        except torch.OutOfMemoryError:
            pairs = 0 if pairs == 1 else (pairs + 1) // 2
    return _workspace(lib.avattn_bwd_f32_workspace_size(B, Hq, Lq), device)


def _check_windows(name, lo, hi, B, Lq):
    """Key windows: int32 (B, Lq) or (Lq,) device tensors -> (lo, hi, batch stride)."""
    if lo is None or hi is None:
        raise ValueError(f"{name}: pass both window_lo and window_hi")
    for label, t in (("window_lo", lo), ("window_hi", hi)):
        if t.dtype is not torch.int32:
            raise TypeError(f"{name}: {label} must be int32; got {t.dtype}")
        if t.shape not in ((B, Lq), (Lq,), (1, Lq)):
            raise ValueError(f"{name}: {label} must be (batch, queries) or (queries,); got {tuple(t.shape)}")
    if lo.shape != hi.shape:
        raise ValueError(f"{name}: window_lo and window_hi shapes differ")
    lo, hi = lo.contiguous(), hi.contiguous()
    wsb = Lq if lo.ndim == 2 and lo.shape[0] == B and B > 1 else 0
    return lo, hi, wsb


def _fwd_windowed_impl(q, k, v, window_lo, window_hi, key_mask, scale):
    name = "avgen_amd.flash_fwd_windowed"
    _check_qkv(name, q, k, v, allow_f32=True)
    _require_gpu(name, q, k, v, key_mask, window_lo, window_hi)
    B, Hq, Lq, D = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    lo, hi, wsb = _check_windows(name, window_lo, window_hi, B, Lq)
    if q.dtype is torch.float32:
        return _fwd_windowed_f32_impl(name, q, k, v, lo, hi, wsb, key_mask, scale)
    q, k, v = _kernel_ready(q), _kernel_ready(k), _kernel_ready(v)
    mask, msb = _normalise_mask(name, key_mask, B, Lk)
    out = _kernel_ready(torch.empty_like(q, memory_format=torch.preserve_format))
    lse = torch.empty((B, Hq, Lq), device=q.device, dtype=torch.float32)
    lib = _lib.load()
    ws = _workspace(lib.avattn_fwd_workspace_size(B, Hkv, Lk, D), q.device)
    st = lib.avattn_fwd_windowed(
        _ptr(q), _ptr(k), _ptr(v), _strides3(q), _strides3(k), _strides3(v),
        B, Hq, Hkv, Lq, Lk, D,
        _ptr(mask), msb,
        _ptr(lo), _ptr(hi), wsb,
        float(scale),
        _ptr(out), _strides3(out), _ptr(lse),
        _ptr(ws), ws.numel(),
        _stream(q.device),
    )
    _lib.check(st, name)
    return out, lse


def _bwd_windowed_impl(dout, q, k, v, out, lse, window_lo, window_hi, key_mask, scale, check_monotone=True,
                       compact=True):
    """Backward of _fwd_windowed_impl (windows non-decreasing in the row,
    verified with one host synchronisation unless ``check_monotone`` is
    False; always with staged dS, in passes if one pass does not fit the
    budget).  ``compact``: stage only the key blocks each query tile's
    windows admit (:func:`compact_ds_table`, one more host synchronisation
    for its size); False: the dense layout, the same results."""
    name = "avgen_amd.flash_bwd_windowed"
    _check_qkv(name, q, k, v, allow_f32=True)
    _require_gpu(name, dout, q, k, v, out, lse, key_mask, window_lo, window_hi)
    B, Hq, Lq, D = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    lo, hi, wsb = _check_windows(name, window_lo, window_hi, B, Lq)
    if check_monotone and Lq > 1 and bool(((lo[..., 1:] < lo[..., :-1]) | (hi[..., 1:] < hi[..., :-1])).any()):
        raise ValueError(f"{name}: the backward needs window_lo and window_hi non-decreasing along the queries")
    if q.dtype is torch.float32:
        return _bwd_f32_impl(name, dout, q, k, v, out, lse, key_mask, scale, windows=(lo, hi, wsb))
    dout, q, k, v, out = (_kernel_ready(t) for t in (dout, q, k, v, out))
    lse = lse.contiguous()
    mask, msb = _normalise_mask(name, key_mask, B, Lk)
    dq = _out_or_new(None, q, name, "dq")
    dk = _out_or_new(None, k, name, "dk")
    dv = _out_or_new(None, v, name, "dv")
    lib = _lib.load()
    common_head = (
        _ptr(dout), _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(lse),
        _strides3(dout), _strides3(q), _strides3(k), _strides3(v), _strides3(out),
        B, Hq, Hkv, Lq, Lk, D,
        _ptr(mask), msb,
        _ptr(lo), _ptr(hi), wsb,
    )
    if compact:
        table, units = compact_ds_table(lo, hi, Lq, Lk)
        tsb = 0 if table.shape[0] == 1 else table.shape[1]
        ws = _alloc_bwd_workspace(B, Hq, Hkv, Lq, Lk, D, q.device, stage_ds=True, ds_units=units)
        st = lib.avattn_bwd_windowed_compact(
            *common_head, _ptr(table), tsb, units,
            float(scale),
            _ptr(dq), _strides3(dq), _ptr(dk), _strides3(dk), _ptr(dv), _strides3(dv),
            _ptr(ws), ws.numel(),
            _lib.BWD_STAGE_DS,
            _stream(q.device),
        )
    else:
        ws = _alloc_bwd_workspace(B, Hq, Hkv, Lq, Lk, D, q.device, stage_ds=True)
        st = lib.avattn_bwd_windowed(
            *common_head,
            float(scale),
            _ptr(dq), _strides3(dq), _ptr(dk), _strides3(dk), _ptr(dv), _strides3(dv),
            _ptr(ws), ws.numel(),
            _lib.BWD_STAGE_DS,
            _stream(q.device),
        )
    _lib.check(st, name)
    return dq, dk, dv


def _fwd_fp8_impl(q, k, v, key_mask, q_scale, k_scale, scale):
    name = "avgen_amd.flash_fwd_fp8"
    _check_qkv(name, q, k, v)
    _require_gpu(name, q, k, v, key_mask, q_scale, k_scale)
    B, Hq, Lq, D = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    for label, t, n in (("q_scale", q_scale, Hq), ("k_scale", k_scale, Hkv)):
        if t.dtype is not torch.float32:
            raise TypeError(f"{name}: {label} must be float32; got {t.dtype}")
        if t.shape != (n,):
            raise ValueError(f"{name}: {label} must have one entry per head ({n},); got {tuple(t.shape)}")
    q_scale, k_scale = q_scale.contiguous(), k_scale.contiguous()
    q, k, v = _kernel_ready(q), _kernel_ready(k), _kernel_ready(v)
    mask, msb = _normalise_mask(name, key_mask, B, Lk)
    out = _kernel_ready(torch.empty_like(q, memory_format=torch.preserve_format))
    lse = torch.empty((B, Hq, Lq), device=q.device, dtype=torch.float32)
    lib = _lib.load()
    ws = _workspace(lib.avattn_fwd_fp8_workspace_size(B, Hkv, Lk, D), q.device)
    st = lib.avattn_fwd_fp8(
        _ptr(q), _ptr(k), _ptr(v), _strides3(q), _strides3(k), _strides3(v),
        B, Hq, Hkv, Lq, Lk, D,
        _ptr(mask), msb,
        _ptr(q_scale), _ptr(k_scale),
        float(scale),
        _ptr(out), _strides3(out), _ptr(lse),
        _ptr(ws), ws.numel(),
        _stream(q.device),
    )
    _lib.check(st, name)
    return out, lse


def _out_or_new(t: Optional[torch.Tensor], like: torch.Tensor, name: str, label: str) -> torch.Tensor:
    """A caller-provided output (any kernel-ready strides, e.g. a slice of a
    larger tensor) or a new one shaped like ``like``."""
    if t is None:
        return _kernel_ready(torch.empty_like(like))
    if t.shape != like.shape or t.dtype is not torch.bfloat16 or t.device != like.device:
        raise ValueError(f"{name}: {label} must be bf16 {tuple(like.shape)} on {like.device}")
    if _kernel_ready(t) is not t:
        raise ValueError(f"{name}: {label} needs a contiguous head_dim and 16-byte aligned rows")
    return t


# Staged dS (the dK/dV kernel stores dS and dQ is one product with k): the
# device memory it may take.  Fixed per device (never read from the
# allocator's current state, so the pass count of a given shape does not
# change from call to call): set_ds_budget(), else AVGEN_AMD_DS_BUDGET_GB
# (0 turns staging off), else the default below, capped at a third of the
# device.  64 GiB holds a c3 ring chunk's 40 (batch, head) pairs in one pass
# (26.7 GiB) and a c2 block's 40 pairs (20 GiB); 76k-token pairs (10.8 GiB)
# go five per pass, and the compact dS of the temporal-window and varlen
# workloads (2.4 / 3.0 GiB per pair) twenty per pass.  Fewer, larger passes
# keep the dK/dV and dQ grids many rounds deep: against 32 GiB, c4 ran 2.4%
# and varlen 2.3% faster (window and c3 unchanged).  When the allocator
# cannot provide a planned workspace the call retries with fewer pairs per
# pass, then (where staging is optional) without staging.
_DS_BUDGET_DEFAULT = 64 << 30
_ds_budgets: dict[int, int] = {}


def set_ds_budget(nbytes: Optional[int], device: Optional[torch.device] = None) -> None:
    """Cap the staged-dS workspace of backward calls on ``device`` (default:
    the current device) at ``nbytes`` (0: never stage; None: back to the
    default)."""
    idx = torch.device(device).index if device is not None else torch.cuda.current_device()
    idx = torch.cuda.current_device() if idx is None else idx
    if nbytes is None:
        _ds_budgets.pop(idx, None)
    else:
        _ds_budgets[idx] = max(0, int(nbytes))


def _ds_budget(device: torch.device) -> int:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _ds_budgets:
        env = os.environ.get("AVGEN_AMD_DS_BUDGET_GB")
        if env is not None:
            _ds_budgets[idx] = int(float(env) * (1 << 30))
        else:
            total = torch.cuda.get_device_properties(idx).total_memory
            _ds_budgets[idx] = min(_DS_BUDGET_DEFAULT, total // 3)
    return _ds_budgets[idx]


def ds_bytes_per_pair(group, Lq, Lk, ds_units=0):
    """Bytes of staged dS per (batch, kv head) pair: bf16 per (query head of
    the group, query row padded to 64, key padded to 128); with ``ds_units``
    (the compact layout of key windows, :func:`compact_ds_table`) 8 KB per
    unit of each query head."""
    if ds_units:
        return group * ds_units * 8192
    return group * ((Lq + 63) // 64 * 64) * ((Lk + 127) // 128 * 128) * 2


def compact_ds_table(window_lo: torch.Tensor, window_hi: torch.Tensor, len_q: int, len_k: int):
    """The compact staged-dS layout of a windowed backward
    (``avattn_bwd_windowed_compact``): per 64-row query tile, the 128-key
    blocks its rows' windows admit, as the dK/dV kernel visits them.

    ``window_lo``/``window_hi``: int32 ``(rows, len_q)`` or ``(len_q,)``, one
    window array per batch row (or one shared), non-decreasing along the
    queries.  Returns ``(table, units)``: int32 ``(rows, tiles, 4)`` on the
    windows' device holding ``[kb_lo, nblk, gbase, 0]`` per tile, and the
    units one query head needs (the largest over the batch rows; at least 1)
    -- read back to the host, one synchronisation."""
    lo = window_lo.reshape(-1, len_q).to(torch.int64)
    hi = window_hi.reshape(-1, len_q).to(torch.int64)
    tiles = (len_q + 63) // 64
    first = torch.arange(tiles, device=lo.device) * 64
    last = torch.clamp(first + 63, max=len_q - 1)
    lo0 = lo[:, first].clamp(0, len_k)
    lo1 = lo[:, last].clamp(0, len_k)
    hi1 = torch.maximum(hi[:, last], lo1).clamp(max=len_k)
    kb_lo = lo0 // 128
    kb_hi = (hi1 + 127) // 128
    nblk = torch.where(lo0 < len_k, (kb_hi - kb_lo).clamp(min=0), torch.zeros_like(kb_lo))
    two = 2 * nblk
    gbase = torch.cumsum(two, 1) - two
    table = torch.stack([kb_lo, nblk, gbase, torch.zeros_like(kb_lo)], -1).to(torch.int32).contiguous()
    units = int(two.sum(1).max().item()) if tiles else 0
    return table, max(units, 1)


def _staged_pairs(B, Hq, Hkv, Lq, Lk, D, device, stage_ds=None, ds_units=0) -> int:
    """(batch, kv head) pairs per pass that a backward call stages dS for (0:
    no staging): as many as the budget holds (``stage_ds`` None), at least one
    (True), none (False); equal passes, as the library splits them."""
    lib = _lib.load()
    if stage_ds is False or lib.avattn_bwd_workspace_size(B, Hq, Hkv, Lq, Lk, D) == 0:
        return 0
    per = ds_bytes_per_pair(Hq // Hkv, Lq, Lk, ds_units)
    pairs = min(B * Hkv, _ds_budget(device) // max(per, 1))
    if pairs == 0:
        if not stage_ds:
            return 0
        pairs = 1
    npass = -(-(B * Hkv) // pairs)
    return -(-(B * Hkv) // npass)


def bwd_workspace_plan(B, Hq, Hkv, Lq, Lk, D, device, stage_ds=None):
    """(bytes, staged) for one backward call: the workspace to allocate and
    whether dS is staged (``stage_ds`` None: when the staged dS of at least
    one (batch, kv head) pair fits the budget; True: at least one pair
    whatever the budget; False: never)."""
    lib = _lib.load()
    pairs = _staged_pairs(B, Hq, Hkv, Lq, Lk, D, device, stage_ds)
    if pairs == 0:
        return lib.avattn_bwd_workspace_size(B, Hq, Hkv, Lq, Lk, D), False
    return lib.avattn_bwd_staged_workspace_size(B, Hq, Hkv, Lq, Lk, D, int(pairs)), True


def _alloc_bwd_workspace(B, Hq, Hkv, Lq, Lk, D, device, stage_ds=None, ds_units=0) -> torch.Tensor:
    """The workspace of :func:`bwd_workspace_plan`, allocated; if the caching
    allocator cannot provide it (memory held by activations, say), the
    staged pairs per pass halve until it can (more passes, the same
    results), and with staging optional (``stage_ds`` not True) a last
    attempt goes without staging (the recomputing dQ kernel).  ``ds_units``:
    the compact layout of key windows (units per query head)."""
    lib = _lib.load()
    pairs = _staged_pairs(B, Hq, Hkv, Lq, Lk, D, device, stage_ds, ds_units)

    def staged_size(p):
        if ds_units:
            return lib.avattn_bwd_compact_workspace_size(B, Hq, Hkv, Lq, Lk, D, int(p), int(ds_units))
        return lib.avattn_bwd_staged_workspace_size(B, Hq, Hkv, Lq, Lk, D, int(p))

    while pairs > 0:
        try:
            return _workspace(staged_size(pairs), device)
        except torch.OutOfMemoryError:
            if pairs == 1:
                if stage_ds:
                    raise
                break
            pairs = (pairs + 1) // 2
    return _workspace(lib.avattn_bwd_workspace_size(B, Hq, Hkv, Lq, Lk, D), device)


def _bwd_impl(dout, q, k, v, out, lse, key_mask, scale, dq=None, dk=None, dv=None, *,
              workspace=None, reuse_query_side=False, dq_accumulate=None, stage_ds=None, defer_dq=False):
    """Backward launch; ``dq``/``dk``/``dv`` may be preallocated outputs
    (written in place, e.g. slices of a full-sequence gradient).

    Ring-step options (one query shard against consecutive KV chunks):
    ``workspace`` is a caller-kept workspace of at least the size this call
    needs; ``reuse_query_side`` asserts that it already holds the query-side
    preparation of a previous call with the same dout/q/out/lse/scale;
    ``dq_accumulate`` is an fp32 tensor shaped like q that this chunk's dq is
    added to (returned in dq's place).  ``stage_ds``: see bwd_workspace_plan;
    with a caller workspace, dS is staged when it is large enough for one
    (batch, kv head) pair (and ``stage_ds`` is not False).  ``defer_dq``: stage
    every pair's dS in the caller's workspace and compute dk/dv only (dq is
    returned as None); _bwd_dq_staged_impl on that workspace computes dq.
    """
    name = "avgen_amd.flash_bwd"
    _check_qkv(name, q, k, v, allow_f32=True)
    _require_gpu(name, dout, q, k, v, out, lse, key_mask)
    if q.dtype is torch.float32:
        if (dq is not None or dk is not None or dv is not None or workspace is not None or reuse_query_side
                or dq_accumulate is not None or defer_dq):
            raise TypeError(f"{name}: the ring-step options take bfloat16 tensors only")
        return _bwd_f32_impl(name, dout, q, k, v, out, lse, key_mask, scale)
    B, Hq, Lq, D = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    if dout.shape != q.shape or out.shape != q.shape:
        raise ValueError(f"{name}: grad_out/out must have the query's shape {tuple(q.shape)}")
    if dout.dtype is not torch.bfloat16 or out.dtype is not torch.bfloat16:
        raise TypeError(f"{name}: grad_out and out must be bfloat16")
    if lse.shape != (B, Hq, Lq) or lse.dtype is not torch.float32:
        raise ValueError(f"{name}: logsumexp must be float32 (batch, heads, queries)")
    dout, q, k, v, out = (_kernel_ready(t) for t in (dout, q, k, v, out))
    lse = lse.contiguous()
    mask, msb = _normalise_mask(name, key_mask, B, Lk)
    flags = 0
    if defer_dq:
        if workspace is None or stage_ds is False:
            raise ValueError(f"{name}: a deferred dq needs staged dS in the caller's workspace")
        flags |= _lib.BWD_DEFER_DQ
        dq = None
    elif dq_accumulate is not None:
        if dq_accumulate.shape != q.shape or dq_accumulate.dtype is not torch.float32:
            raise ValueError(f"{name}: dq accumulator must be float32 {tuple(q.shape)}")
        if dq_accumulate.stride(-1) != 1 or dq_accumulate.data_ptr() % 16 or any(
                st % 4 for st in dq_accumulate.stride()[:3]):
            raise ValueError(f"{name}: dq accumulator needs a contiguous head_dim and 16-byte aligned rows")
        dq = dq_accumulate
        flags |= _lib.BWD_DQ_ACCUMULATE_F32
    else:
        dq = _out_or_new(dq, q, name, "dq")
    dk = _out_or_new(dk, k, name, "dk")
    dv = _out_or_new(dv, v, name, "dv")
    lib = _lib.load()
    need = lib.avattn_bwd_workspace_size(B, Hq, Hkv, Lq, Lk, D)
    if workspace is None:
        if reuse_query_side:
            raise ValueError(f"{name}: reuse_query_side needs the caller's workspace")
        ws = _alloc_bwd_workspace(B, Hq, Hkv, Lq, Lk, D, q.device, stage_ds)
        one = lib.avattn_bwd_staged_workspace_size(B, Hq, Hkv, Lq, Lk, D, 1)
        staged = stage_ds is not False and one > 0 and ws.numel() >= one
    else:
        if workspace.dtype is not torch.uint8 or workspace.numel() < need or workspace.device != q.device:
            raise ValueError(f"{name}: workspace must be uint8 with at least {need} bytes on {q.device}")
        ws = workspace
        one = lib.avattn_bwd_staged_workspace_size(B, Hq, Hkv, Lq, Lk, D, 1)
        staged = stage_ds is not False and one > 0 and ws.numel() >= one
        if stage_ds and not staged:
            raise ValueError(f"{name}: staging dS needs a workspace of at least {one} bytes")
    if staged:
        flags |= _lib.BWD_STAGE_DS
    if reuse_query_side:
        flags |= _lib.BWD_REUSE_QUERY_SIDE
    st = lib.avattn_bwd(
        _ptr(dout), _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(lse),
        _strides3(dout), _strides3(q), _strides3(k), _strides3(v), _strides3(out),
        B, Hq, Hkv, Lq, Lk, D,
        _ptr(mask), msb,
        float(scale),
        _ptr(dq), _strides3(dq if dq is not None else q), _ptr(dk), _strides3(dk), _ptr(dv), _strides3(dv),
        _ptr(ws), ws.numel(),
        flags,
        _stream(q.device),
    )
    _lib.check(st, name)
    return dq, dk, dv


def _bwd_dq_staged_impl(q, Hkv, Lk, scale, workspace, dq=None, dq_accumulate=None):
    """dq of a backward run with ``defer_dq`` on ``workspace`` (same q shape,
    kv heads and key length), on the current stream: written to ``dq`` (new
    if None) or added in fp32 to ``dq_accumulate`` (returned)."""
    name = "avgen_amd.flash_bwd"
    B, Hq, Lq, D = q.shape
    flags = 0
    if dq_accumulate is not None:
        if dq_accumulate.shape != q.shape or dq_accumulate.dtype is not torch.float32:
            raise ValueError(f"{name}: dq accumulator must be float32 {tuple(q.shape)}")
        dq = dq_accumulate
        flags |= _lib.BWD_DQ_ACCUMULATE_F32
    else:
        dq = _out_or_new(dq, q, name, "dq")
    _require_gpu(name, dq, workspace)
    st = _lib.load().avattn_bwd_dq_staged(
        B, Hq, Hkv, Lq, Lk, D, float(scale), _ptr(dq), _strides3(dq), _ptr(workspace), workspace.numel(), flags,
        _stream(q.device))
    _lib.check(st, name)
    return dq


def _ring_tables(name, cos, sin, batch, length, head_dim):
    """(cos, sin, batch stride) of one rotation table pair (or (None, None, 0)
    without tables): shape (B|1, 1, length, head_dim/2) float32 with
    contiguous rows of pairs, e.g. a slice of full-sequence tables along the
    sequence (no copy is made)."""
    if cos is None and sin is None:
        return None, None, 0
    if cos is None or sin is None:
        raise ValueError(f"{name}: pass both rotation tables or neither")
    if cos.ndim != 4 or cos.shape != sin.shape:
        raise ValueError(f"{name}: rotary tables must be (batch, 1, length, pairs) and agree")
    if cos.dtype is not torch.float32 or sin.dtype is not torch.float32:
        raise TypeError(f"{name}: rotary tables must be float32")
    if cos.shape[-1] * 2 != head_dim:
        raise ValueError(f"{name}: head_dim {head_dim} does not match rotary tables built for head_dim "
                         f"{2 * cos.shape[-1]}")
    if cos.shape[-2] != length:
        raise ValueError(f"{name}: sequence length {length} does not match rotary tables built for length "
                         f"{cos.shape[-2]}")
    if cos.shape[0] not in (1, batch) or cos.shape[1] != 1:
        raise ValueError(f"{name}: rotary tables batch {cos.shape[0]} does not broadcast to {batch}")
    pairs = cos.shape[-1]
    out = []
    for t in (cos, sin):
        ok = t.stride(-1) == 1 and (t.shape[-2] <= 1 or t.stride(-2) == pairs) and t.data_ptr() % 16 == 0
        ok = ok and (t.shape[0] == 1 or t.stride(0) % 4 == 0)
        out.append(t if ok else t.contiguous())
    cos, sin = out
    if cos.stride(0) != sin.stride(0):
        sin = sin.contiguous()
        cos = cos.contiguous()
    stride_b = 0 if cos.shape[0] == 1 else cos.stride(0)
    _require_gpu(name, cos, sin)
    return cos, sin, stride_b


def _table_pair(tables):
    return (None, None) if tables is None else (tables.cos, tables.sin)


def _ring_fwd_step_impl(q, k, v, key_mask, cos_q, sin_q, cos_k, sin_k, scale, out_acc, lse_acc, out, first, last):
    name = "avgen_amd.ring_fwd_step"
    _check_qkv(name, q, k, v)
    _require_gpu(name, q, k, v, key_mask, out_acc, lse_acc, out)
    B, Hq, Lq, D = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    if out_acc.shape != q.shape or out_acc.dtype is not torch.float32 or not out_acc.is_contiguous():
        raise ValueError(f"{name}: out_acc must be contiguous float32 {tuple(q.shape)}")
    if lse_acc.shape != (B, Hq, Lq) or lse_acc.dtype is not torch.float32 or not lse_acc.is_contiguous():
        raise ValueError(f"{name}: lse_acc must be contiguous float32 {(B, Hq, Lq)}")
    if last and (out is None or out.shape != q.shape or out.dtype is not torch.bfloat16
                 or _kernel_ready(out) is not out):
        raise ValueError(f"{name}: the last step needs a kernel-ready bf16 output shaped like the query")
    q, k, v = _kernel_ready(q), _kernel_ready(k), _kernel_ready(v)
    mask, msb = _normalise_mask(name, key_mask, B, Lk)
    cq, sq, rqsb = _ring_tables(name, cos_q, sin_q, B, Lq, D)
    ck, sk, rksb = _ring_tables(name, cos_k, sin_k, B, Lk, D)
    flags = (_lib.RING_FIRST if first else 0) | (_lib.RING_LAST if last else 0)
    lib = _lib.load()
    ws = _workspace(lib.avattn_fwd_workspace_size(B, Hkv, Lk, D), q.device)
    st = lib.avattn_ring_fwd_step(
        _ptr(q), _ptr(k), _ptr(v), _strides3(q), _strides3(k), _strides3(v),
        B, Hq, Hkv, Lq, Lk, D,
        _ptr(mask), msb,
        _ptr(cq), _ptr(sq), rqsb, _ptr(ck), _ptr(sk), rksb,
        float(scale),
        _ptr(out_acc), _ptr(lse_acc),
        _ptr(out) if last else None, _strides3(out) if last else None,
        flags,
        _ptr(ws), ws.numel(),
        _stream(q.device),
    )
    _lib.check(st, name)


def _ring_bwd_step_impl(dout, q, k, v, out, lse, key_mask, cos_q, sin_q, cos_k, sin_k, scale, dq_acc, dk, dv,
                        workspace, reuse_query_side):
    name = "avgen_amd.ring_bwd_step"
    _check_qkv(name, q, k, v)
    _require_gpu(name, dout, q, k, v, out, lse, key_mask, dq_acc, dk, dv, workspace)
    B, Hq, Lq, D = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    if dq_acc.shape != q.shape or dq_acc.dtype is not torch.float32:
        raise ValueError(f"{name}: dq accumulator must be float32 {tuple(q.shape)}")
    if workspace.dtype is not torch.uint8 or workspace.ndim != 1:
        raise ValueError(f"{name}: workspace must be a 1-D uint8 tensor")
    dout, q, k, v, out = (_kernel_ready(t) for t in (dout, q, k, v, out))
    lse = lse.contiguous()
    mask, msb = _normalise_mask(name, key_mask, B, Lk)
    cq, sq, rqsb = _ring_tables(name, cos_q, sin_q, B, Lq, D)
    ck, sk, rksb = _ring_tables(name, cos_k, sin_k, B, Lk, D)
    lib = _lib.load()
    one = lib.avattn_bwd_staged_workspace_size(B, Hq, Hkv, Lq, Lk, D, 1)
    flags = _lib.BWD_STAGE_DS if (one > 0 and workspace.numel() >= one) else 0
    if reuse_query_side:
        flags |= _lib.BWD_REUSE_QUERY_SIDE
    st = lib.avattn_ring_bwd_step(
        _ptr(dout), _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(lse),
        _strides3(dout), _strides3(q), _strides3(k), _strides3(v), _strides3(out),
        B, Hq, Hkv, Lq, Lk, D,
        _ptr(mask), msb,
        _ptr(cq), _ptr(sq), rqsb, _ptr(ck), _ptr(sk), rksb,
        float(scale),
        _ptr(dq_acc), _strides3(dq_acc), _ptr(dk), _strides3(dk), _ptr(dv), _strides3(dv),
        _ptr(workspace), workspace.numel(),
        flags,
        _stream(q.device),
    )
    _lib.check(st, name)


def _ring_dq_finish_impl(dq_acc, cos_q, sin_q, dq):
    name = "avgen_amd.ring_dq_finish"
    _require_gpu(name, dq_acc, dq)
    B, H, L, D = dq_acc.shape
    if dq_acc.dtype is not torch.float32 or dq.dtype is not torch.bfloat16 or dq.shape != dq_acc.shape:
        raise ValueError(f"{name}: dq_acc must be float32 and dq bfloat16 of the same shape")
    cq, sq, rqsb = _ring_tables(name, cos_q, sin_q, B, L, D)
    st = _lib.load().avattn_ring_dq_finish(
        _ptr(dq_acc), _strides3(dq_acc), B, H, L, D, _ptr(cq), _ptr(sq), rqsb, _ptr(dq), _strides3(dq),
        _stream(dq.device))
    _lib.check(st, name)


def _lse_merge_impl(out_acc, lse_acc, out_blk, lse_blk):
    name = "avgen_amd.lse_merge_"
    _require_gpu(name, out_acc, lse_acc, out_blk, lse_blk)
    if out_acc.dtype is not torch.float32 or lse_acc.dtype is not torch.float32 or lse_blk.dtype is not torch.float32:
        raise TypeError(f"{name}: accumulators and block LSE must be float32")
    if out_blk.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"{name}: block output must be bfloat16 or float32")
    if out_blk.shape != out_acc.shape or lse_acc.shape != lse_blk.shape or out_acc.shape[:-1] != lse_acc.shape:
        raise ValueError(f"{name}: shapes disagree")
    if not (out_acc.is_contiguous() and lse_acc.is_contiguous()):
        raise ValueError(f"{name}: accumulators must be contiguous (they are updated in place)")
    out_blk = out_blk.contiguous()
    lse_blk = lse_blk.contiguous()
    D = out_acc.shape[-1]
    rows = lse_acc.numel()
    st = _lib.load().avattn_lse_merge(
        _ptr(out_acc), _ptr(lse_acc), _ptr(out_blk), _ptr(lse_blk), rows, D,
        1 if out_blk.dtype is torch.bfloat16 else 0, _stream(out_acc.device),
    )
    _lib.check(st, name)


# The ring's per-chunk steps as ops that update their accumulators in place
# (schema: Tensor(a!)), so a compiled region that calls them keeps them as
# opaque, correctly ordered mutations.


@torch.library.custom_op("avgen_amd::ring_fwd_step", mutates_args=("out_acc", "lse_acc", "out"))
def _ring_fwd_step_op(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, key_mask: Optional[torch.Tensor],
    cos_q: Optional[torch.Tensor], sin_q: Optional[torch.Tensor], cos_k: Optional[torch.Tensor],
    sin_k: Optional[torch.Tensor], scale: float, out_acc: torch.Tensor, lse_acc: torch.Tensor,
    out: Optional[torch.Tensor], first: bool, last: bool,
) -> None:
    _ring_fwd_step_impl(q, k, v, key_mask, cos_q, sin_q, cos_k, sin_k, scale, out_acc, lse_acc, out, first, last)


@_ring_fwd_step_op.register_fake
def _(q, k, v, key_mask, cos_q, sin_q, cos_k, sin_k, scale, out_acc, lse_acc, out, first, last):
    return None


@torch.library.custom_op("avgen_amd::ring_bwd_step", mutates_args=("dq_acc", "dk", "dv", "workspace"))
def _ring_bwd_step_op(
    dout: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor, lse: torch.Tensor,
    key_mask: Optional[torch.Tensor], cos_q: Optional[torch.Tensor], sin_q: Optional[torch.Tensor],
    cos_k: Optional[torch.Tensor], sin_k: Optional[torch.Tensor], scale: float, dq_acc: torch.Tensor,
    dk: torch.Tensor, dv: torch.Tensor, workspace: torch.Tensor, reuse_query_side: bool,
) -> None:
    _ring_bwd_step_impl(dout, q, k, v, out, lse, key_mask, cos_q, sin_q, cos_k, sin_k, scale, dq_acc, dk, dv,
                        workspace, reuse_query_side)


@_ring_bwd_step_op.register_fake
def _(dout, q, k, v, out, lse, key_mask, cos_q, sin_q, cos_k, sin_k, scale, dq_acc, dk, dv, workspace,
      reuse_query_side):
    return None


@torch.library.custom_op("avgen_amd::ring_dq_finish", mutates_args=("dq",))
def _ring_dq_finish_op(dq_acc: torch.Tensor, cos_q: Optional[torch.Tensor], sin_q: Optional[torch.Tensor],
                       dq: torch.Tensor) -> None:
    _ring_dq_finish_impl(dq_acc, cos_q, sin_q, dq)


@_ring_dq_finish_op.register_fake
def _(dq_acc, cos_q, sin_q, dq):
    return None


@torch.library.custom_op("avgen_amd::lse_merge", mutates_args=("out_acc", "lse_acc"))
def _lse_merge_op(out_acc: torch.Tensor, lse_acc: torch.Tensor, out_blk: torch.Tensor, lse_blk: torch.Tensor) -> None:
    _lse_merge_impl(out_acc, lse_acc, out_blk, lse_blk)


@_lse_merge_op.register_fake
def _(out_acc, lse_acc, out_blk, lse_blk):
    return None


def ring_fwd_step_(q, k, v, key_mask, tables_q, tables_k, scale, out_acc, lse_acc, out, *, first: bool,
                   last: bool) -> None:
    """One fused ring forward step (op ``avgen_amd::ring_fwd_step`` over
    ``avattn_ring_fwd_step``): attention of the UNROTATED query shard ``q``
    against one UNROTATED KV chunk, rotated on the fly with ``tables_q`` /
    ``tables_k`` (RotaryTables or None), merged into the running fp32
    ``out_acc`` / ``lse_acc`` (``first``: they take this chunk's result);
    with ``last`` the merged output is also written to ``out`` (bf16, q's
    shape).  Replaces apply_rotary + the ring's local op +
    ``_SDPAMerger.step`` (torch/.../_context_parallel/_attention.py:182-183)."""
    cq, sq = _table_pair(tables_q)
    ck, sk = _table_pair(tables_k)
    _ring_fwd_step_op(q, k, v, key_mask, cq, sq, ck, sk, float(scale), out_acc, lse_acc, out, bool(first),
                      bool(last))


def ring_bwd_step(dout, q, k, v, out, lse, key_mask, tables_q, tables_k, scale, dq_acc, dk, dv, *, workspace,
                  reuse_query_side: bool) -> None:
    """One fused ring backward step (op ``avgen_amd::ring_bwd_step`` over
    ``avattn_ring_bwd_step``): adds this chunk's gradient of the rotated query
    to the fp32 ``dq_acc`` and writes the chunk's ``dk`` (of the unrotated
    keys) and ``dv`` in place.  ``workspace`` is a uint8 device tensor of at
    least the plain backward's size; dS is staged when it holds at least one
    (batch, kv head) pair's dS (torch/.../_attention.py:567-575)."""
    cq, sq = _table_pair(tables_q)
    ck, sk = _table_pair(tables_k)
    _ring_bwd_step_op(dout, q, k, v, out, lse, key_mask, cq, sq, ck, sk, float(scale), dq_acc, dk, dv, workspace,
                      bool(reuse_query_side))


def ring_dq_finish(dq_acc, tables_q, dq) -> None:
    """``dq`` (bf16) = transposed rotation of ``bf16(dq_acc)`` (op
    ``avgen_amd::ring_dq_finish`` over ``avattn_ring_dq_finish``); a plain cast
    without tables."""
    cq, sq = _table_pair(tables_q)
    _ring_dq_finish_op(dq_acc, cq, sq, dq)


def _rope_apply_impl(x, cos, sin, inverse):
    name = "avgen_amd.rope_apply"
    if x.ndim != 4:
        raise ValueError(f"rotary input must be (batch, heads, length, head_dim); got {tuple(x.shape)}")
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"{name}: input must be bfloat16 or float32; got {x.dtype}")
    B, H, L, D = x.shape
    cos, sin, tsb = _check_tables(name, cos, sin, B, L, D)
    _require_gpu(name, x, cos, sin)
    if x.dtype is torch.float32:
        x = _f32_ready(x)
        out = _f32_ready(torch.empty_like(x, memory_format=torch.preserve_format))
        st = _lib.load().avattn_rope_apply_f32(
            _ptr(x), _strides3(x), B, H, L, D, _ptr(cos), _ptr(sin), tsb, 1 if inverse else 0,
            _ptr(out), _strides3(out), _stream(x.device),
        )
        _lib.check(st, name)
        return out
    x = _kernel_ready(x)
    out = _kernel_ready(torch.empty_like(x, memory_format=torch.preserve_format))
    st = _lib.load().avattn_rope_apply(
        _ptr(x), _strides3(x), B, H, L, D, _ptr(cos), _ptr(sin), tsb, 1 if inverse else 0,
        _ptr(out), _strides3(out), _stream(x.device),
    )
    _lib.check(st, name)
    return out


def _qk_norm_common(name, x, weight, eps, cos, sin):
    if x.ndim != 4:
        raise ValueError(f"{name}: input must be (batch, heads, length, head_dim); got {tuple(x.shape)}")
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"{name}: input must be bfloat16 or float32; got {x.dtype}")
    B, H, L, D = x.shape
    if D not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"{name}: head_dim {D} not supported (supported: {SUPPORTED_HEAD_DIMS})")
    if weight is not None:
        if weight.shape != (D,):
            raise ValueError(f"{name}: weight must be ({D},); got {tuple(weight.shape)}")
        # the gain in the activation's dtype (src/avgen/models/layers.py:114-116)
        weight = weight.to(x.dtype).contiguous()
    tsb = 0
    if cos is not None or sin is not None:
        if cos is None or sin is None:
            raise ValueError(f"{name}: pass both rotation tables or neither")
        cos, sin, tsb = _check_tables(name, cos, sin, B, L, D)
    if not (eps >= 0.0 and math.isfinite(eps)):
        raise ValueError(f"{name}: eps must be finite and >= 0; got {eps}")
    _require_gpu(name, x, weight, cos, sin)
    return (_f32_ready(x) if x.dtype is torch.float32 else _kernel_ready(x)), weight, cos, sin, tsb


def _qk_norm_rope_impl(x, weight, eps, cos, sin):
    name = "avgen_amd.qk_norm_rope"
    x, w, cos, sin, tsb = _qk_norm_common(name, x, weight, eps, cos, sin)
    B, H, L, D = x.shape
    f32 = x.dtype is torch.float32
    out = torch.empty_like(x, memory_format=torch.preserve_format)
    out = _f32_ready(out) if f32 else _kernel_ready(out)
    lib = _lib.load()
    st = (lib.avattn_qk_norm_rope_f32 if f32 else lib.avattn_qk_norm_rope)(
        _ptr(x), _strides3(x), B, H, L, D, _ptr(w), float(eps), _ptr(cos), _ptr(sin), tsb,
        _ptr(out), _strides3(out), _stream(x.device))
    _lib.check(st, name)
    return out


def _qk_norm_rope_bwd_impl(dy, x, weight, eps, cos, sin):
    name = "avgen_amd.qk_norm_rope_bwd"
    x, w, cos, sin, tsb = _qk_norm_common(name, x, weight, eps, cos, sin)
    B, H, L, D = x.shape
    f32 = x.dtype is torch.float32
    if dy.shape != x.shape or dy.dtype is not x.dtype:
        raise ValueError(f"{name}: dy must be {x.dtype} {tuple(x.shape)}")
    _require_gpu(name, dy)
    ready = _f32_ready if f32 else _kernel_ready
    dy = ready(dy)
    dx = ready(torch.empty_like(x, memory_format=torch.preserve_format))
    lib = _lib.load()
    dw = ws = None
    if w is not None:
        dw = torch.empty(D, device=x.device, dtype=torch.float32)
        ws = _workspace(lib.avattn_qk_norm_rope_bwd_workspace_size(D), x.device)
    st = (lib.avattn_qk_norm_rope_bwd_f32 if f32 else lib.avattn_qk_norm_rope_bwd)(
        _ptr(x), _strides3(x), _ptr(dy), _strides3(dy), B, H, L, D, _ptr(w), float(eps),
        _ptr(cos), _ptr(sin), tsb, _ptr(dx), _strides3(dx), _ptr(dw), _ptr(ws), 0 if ws is None else ws.numel(),
        _stream(x.device))
    _lib.check(st, name)
    return dx, dw


# ---------------------------------------------------------------------------
# torch.library registration
# ---------------------------------------------------------------------------


@torch.library.custom_op("avgen_amd::flash_fwd", mutates_args=())
def flash_fwd(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    key_mask: Optional[torch.Tensor],
    rope_cos: Optional[torch.Tensor],
    rope_sin: Optional[torch.Tensor],
    scale: float,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Attention forward over one KV chunk: ``(out, lse)``; see module docstring."""
    return _fwd_impl(q, k, v, key_mask, rope_cos, rope_sin, scale)


@flash_fwd.register_fake
def _(q, k, v, key_mask, rope_cos, rope_sin, scale):
    return torch.empty_like(q), q.new_empty((q.shape[0], q.shape[1], q.shape[2]), dtype=torch.float32)


@torch.library.custom_op("avgen_amd::flash_bwd", mutates_args=())
def flash_bwd(
    dout: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    out: torch.Tensor,
    lse: torch.Tensor,
    key_mask: Optional[torch.Tensor],
    scale: float,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Attention backward over one KV chunk given the (possibly merged) out/lse."""
    return _bwd_impl(dout, q, k, v, out, lse, key_mask, scale)


@flash_bwd.register_fake
def _(dout, q, k, v, out, lse, key_mask, scale):
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)


@torch.library.custom_op("avgen_amd::rope_apply", mutates_args=())
def rope_apply(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, inverse: bool) -> torch.Tensor:
    """Interleaved-pair rotation (or its transpose) of ``x``."""
    return _rope_apply_impl(x, cos, sin, inverse)


@rope_apply.register_fake
def _(x, cos, sin, inverse):
    return x.new_empty(x.shape)


@torch.library.custom_op("avgen_amd::flash_fwd_fp8", mutates_args=())
def flash_fwd_fp8(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    key_mask: Optional[torch.Tensor],
    q_scale: torch.Tensor,
    k_scale: torch.Tensor,
    scale: float,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Forward with e4m3 q k^T: ``(out, lse)``; not differentiable."""
    return _fwd_fp8_impl(q, k, v, key_mask, q_scale, k_scale, scale)


@flash_fwd_fp8.register_fake
def _(q, k, v, key_mask, q_scale, k_scale, scale):
    return torch.empty_like(q), q.new_empty((q.shape[0], q.shape[1], q.shape[2]), dtype=torch.float32)


@torch.library.custom_op("avgen_amd::flash_fwd_windowed", mutates_args=())
def flash_fwd_windowed(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    window_lo: torch.Tensor,
    window_hi: torch.Tensor,
    key_mask: Optional[torch.Tensor],
    scale: float,
    monotone: bool = False,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Forward where query row i attends keys [window_lo[i], window_hi[i]) only.
    ``monotone``: the caller guarantees both bounds non-decreasing in the row
    (its backward then skips the check and its host synchronisation)."""
    return _fwd_windowed_impl(q, k, v, window_lo, window_hi, key_mask, scale)


@flash_fwd_windowed.register_fake
def _(q, k, v, window_lo, window_hi, key_mask, scale, monotone=False):
    return torch.empty_like(q), q.new_empty((q.shape[0], q.shape[1], q.shape[2]), dtype=torch.float32)


@torch.library.custom_op("avgen_amd::flash_bwd_windowed", mutates_args=())
def flash_bwd_windowed(
    dout: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    out: torch.Tensor,
    lse: torch.Tensor,
    window_lo: torch.Tensor,
    window_hi: torch.Tensor,
    key_mask: Optional[torch.Tensor],
    scale: float,
    monotone: bool = False,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Backward of ``flash_fwd_windowed`` (windows non-decreasing in the row;
    checked unless ``monotone``)."""
    return _bwd_windowed_impl(dout, q, k, v, out, lse, window_lo, window_hi, key_mask, scale,
                              check_monotone=not monotone)


@flash_bwd_windowed.register_fake
def _(dout, q, k, v, out, lse, window_lo, window_hi, key_mask, scale, monotone=False):
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)


def _fwd_windowed_setup(ctx, inputs, output):
    q, k, v, window_lo, window_hi, key_mask, scale, monotone = inputs
    out, lse = output
    ctx.scale = scale
    ctx.monotone = monotone
    ctx.save_for_backward(q, k, v, out, lse, window_lo, window_hi, key_mask)
    ctx.mark_non_differentiable(lse)


def _fwd_windowed_backward(ctx, dout, _dlse):
    q, k, v, out, lse, window_lo, window_hi, key_mask = ctx.saved_tensors
    dq, dk, dv = flash_bwd_windowed(dout, q, k, v, out, lse, window_lo, window_hi, key_mask, ctx.scale,
                                    ctx.monotone)
    return dq, dk, dv, None, None, None, None, None


torch.library.register_autograd(
    "avgen_amd::flash_fwd_windowed", _fwd_windowed_backward, setup_context=_fwd_windowed_setup
)


@torch.library.custom_op("avgen_amd::qk_norm_rope", mutates_args=())
def qk_norm_rope(
    x: torch.Tensor, weight: Optional[torch.Tensor], eps: float, cos: Optional[torch.Tensor],
    sin: Optional[torch.Tensor],
) -> torch.Tensor:
    """Per-head RMSNorm (gain ``weight`` cast to the input's dtype, bf16 or
    float32) then the rotation; see module docstring."""
    return _qk_norm_rope_impl(x, weight, eps, cos, sin)


@qk_norm_rope.register_fake
def _(x, weight, eps, cos, sin):
    return torch.empty_like(x)


@torch.library.custom_op("avgen_amd::qk_norm_rope_bwd", mutates_args=())
def qk_norm_rope_bwd(
    dy: torch.Tensor, x: torch.Tensor, weight: Optional[torch.Tensor], eps: float, cos: Optional[torch.Tensor],
    sin: Optional[torch.Tensor],
) -> tuple[torch.Tensor, torch.Tensor]:
    """``(dx, dweight)`` of ``qk_norm_rope`` (``dweight`` fp32; zeros(0) without a gain)."""
    dx, dw = _qk_norm_rope_bwd_impl(dy, x, weight, eps, cos, sin)
    return dx, (dw if dw is not None else x.new_zeros(0, dtype=torch.float32))


@qk_norm_rope_bwd.register_fake
def _(dy, x, weight, eps, cos, sin):
    return torch.empty_like(x), x.new_empty(0 if weight is None else x.shape[-1], dtype=torch.float32)


def _qk_norm_setup(ctx, inputs, output):
    x, weight, eps, cos, sin = inputs
    ctx.eps = eps
    ctx.has_weight = weight is not None
    ctx.weight_dtype = None if weight is None else weight.dtype
    ctx.save_for_backward(x, weight, cos, sin)


def _qk_norm_backward(ctx, dy):
    x, weight, cos, sin = ctx.saved_tensors
    dx, dw = qk_norm_rope_bwd(dy, x, weight, ctx.eps, cos, sin)
    return dx, (dw.to(ctx.weight_dtype) if ctx.has_weight else None), None, None, None


torch.library.register_autograd("avgen_amd::qk_norm_rope", _qk_norm_backward, setup_context=_qk_norm_setup)


def _fwd_setup(ctx, inputs, output):
    q, k, v, key_mask, rope_cos, rope_sin, scale = inputs
    out, lse = output
    ctx.scale = scale
    ctx.save_for_backward(q, k, v, out, lse, key_mask, rope_cos, rope_sin)
    ctx.mark_non_differentiable(lse)


def _fwd_backward(ctx, dout, _dlse):
    q, k, v, out, lse, key_mask, rope_cos, rope_sin = ctx.saved_tensors
    if rope_cos is not None:
        q_rot = rope_apply(q, rope_cos, rope_sin, False)
        dq_rot, dk, dv = flash_bwd(dout, q_rot, k, v, out, lse, key_mask, ctx.scale)
        dq = rope_apply(dq_rot, rope_cos, rope_sin, True)
    else:
        dq, dk, dv = flash_bwd(dout, q, k, v, out, lse, key_mask, ctx.scale)
    return dq, dk, dv, None, None, None, None


torch.library.register_autograd("avgen_amd::flash_fwd", _fwd_backward, setup_context=_fwd_setup)


def _rope_setup(ctx, inputs, output):
    _x, cos, sin, inverse = inputs
    ctx.inverse = inverse
    ctx.save_for_backward(cos, sin)


def _rope_backward(ctx, grad):
    cos, sin = ctx.saved_tensors
    return rope_apply(grad, cos, sin, not ctx.inverse), None, None, None


torch.library.register_autograd("avgen_amd::rope_apply", _rope_backward, setup_context=_rope_setup)


# ---------------------------------------------------------------------------
# Non-differentiable helpers
# ---------------------------------------------------------------------------


def fp8_absmax_scales(x: torch.Tensor) -> torch.Tensor:
    """Per-head e4m3 scales of ``x (batch, heads, seq, head_dim)`` bf16:
    ``max|x[:, h]| / 448`` in fp32 (1 for an all-zero head), shape ``(heads,)``."""
    name = "avgen_amd.fp8_absmax_scales"
    if x.ndim != 4:
        raise ValueError(f"{name}: input must be (batch, heads, seq, head_dim); got {tuple(x.shape)}")
    if x.dtype is not torch.bfloat16:
        raise TypeError(f"{name}: input must be bfloat16; got {x.dtype}")
    if x.shape[-1] not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"{name}: head_dim {x.shape[-1]} not supported (supported: {SUPPORTED_HEAD_DIMS})")
    _require_gpu(name, x)
    B, H, L, D = x.shape
    x = _kernel_ready(x)
    out = torch.empty((H,), device=x.device, dtype=torch.float32)
    st = _lib.load().avattn_fp8_absmax_scales(_ptr(x), _strides3(x), B, H, L, D, _ptr(out), _stream(x.device))
    _lib.check(st, name)
    return out


def lse_merge_(out_acc: torch.Tensor, lse_acc: torch.Tensor, out_blk: torch.Tensor, lse_blk: torch.Tensor) -> None:
    """In-place fp32 online-softmax merge (op ``avgen_amd::lse_merge``;
    torch/.../_attention.py:182-183).

    ``out_acc``: fp32 contiguous (..., D); ``lse_acc``: fp32 contiguous (...);
    ``out_blk``: bf16 or fp32 with out_acc's shape; ``lse_blk``: lse_acc's shape.
    """
    _lse_merge_op(out_acc, lse_acc, out_blk, lse_blk)


def rope_tables(
    coords: torch.Tensor,
    inv_freq: list[float],
    axis_of_pair: list[int],
    pos_mul: tuple[Optional[float], Optional[float], Optional[float]],
    pos_div: tuple[Optional[float], Optional[float], Optional[float]],
) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin tables ``(B, 1, L, pairs)`` from ``coords (B, L, 3)`` on the GPU.

    ``pos_mul[a]`` / ``pos_div[a]`` are ``None`` when that step is skipped for
    axis ``a`` (src/avgen/models/rope.py:270-277).
    """
    name = "avgen_amd.rope_tables"
    _require_gpu(name, coords)
    if coords.dtype is not torch.float32:
        raise TypeError(f"{name}: coords must be float32; got {coords.dtype}")
    if coords.stride(-1) != 1:
        coords = coords.contiguous()
    B, L, _ = coords.shape
    P = len(inv_freq)
    cos = torch.empty((B, 1, L, P), device=coords.device, dtype=torch.float32)
    sin = torch.empty_like(cos)
    f32 = ctypes.c_float
    i32 = ctypes.c_int32
    inv = (f32 * P)(*inv_freq)
    axes = (i32 * P)(*axis_of_pair)
    am = (i32 * 3)(*[0 if m is None else 1 for m in pos_mul])
    pm = (f32 * 3)(*[1.0 if m is None else m for m in pos_mul])
    ad = (i32 * 3)(*[0 if d is None else 1 for d in pos_div])
    pd = (f32 * 3)(*[1.0 if d is None else d for d in pos_div])
    st = _lib.load().avattn_rope_tables(
        _ptr(coords), coords.stride(0), coords.stride(1), B, L, P,
        ctypes.cast(inv, ctypes.c_void_p), ctypes.cast(axes, ctypes.c_void_p),
        ctypes.cast(am, ctypes.c_void_p), ctypes.cast(pm, ctypes.c_void_p),
        ctypes.cast(ad, ctypes.c_void_p), ctypes.cast(pd, ctypes.c_void_p),
        _ptr(cos), _ptr(sin), _stream(coords.device),
    )
    _lib.check(st, name)
    return cos, sin
