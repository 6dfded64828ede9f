"""numpy restatement of the reference's attention hot path (test oracle only).

Conventions: tensors are numpy arrays shaped like the reference's torch
tensors; ``q, k, v`` are ``(B, H, L, D)``; LSE is ``(B, H, Lq)`` natural log.
bf16 values are carried as float32 arrays holding exactly-representable
bf16 numbers (see :func:`bf16_round`).
"""

from __future__ import annotations

import math
from collections.abc import Sequence

import numpy as np

# ---------------------------------------------------------------------------
# bf16 helpers
# ---------------------------------------------------------------------------


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bf16 (ties to even), returned as float32.

    Same rounding as torch's float32 -> bfloat16 cast (round-to-nearest-even);
    NaN stays NaN.
    """
    f = np.asarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32)
    r = np.where(np.isnan(f), np.uint32(0x7FC0), r)
    return (r.astype(np.uint32) << 16).view(np.float32)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """uint16 bit patterns of float32 values that are exactly bf16."""
    return (np.asarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


# ---------------------------------------------------------------------------
# 3D RoPE  (src/avgen/models/rope.py)
# ---------------------------------------------------------------------------


def rope_axis_pairs(head_dim: int) -> tuple[int, int, int]:
    """src/avgen/models/rope.py:128-157 — time takes the remainder."""
    if head_dim < 6 or head_dim % 2 != 0:
        raise ValueError(f"head_dim must be an even integer of at least 6; got {head_dim!r}")
    pairs = head_dim // 2
    spatial = pairs // 3
    return (pairs - 2 * spatial, spatial, spatial)


def axis_plan(
    head_dim: int, theta: float, scaling: tuple[str, float, float] = ("none", 1.0, 1.0)
) -> list[tuple[int, float, float | None]]:
    """Per axis ``(pairs, axis_theta, linear_factor_or_None)``
    (src/avgen/models/rope.py:259-285).  ``scaling`` = (mode, time, spatial)."""
    mode, tf, sf = scaling
    plan = []
    for axis, (pairs, factor) in enumerate(zip(rope_axis_pairs(head_dim), (tf, sf, sf))):
        axis_theta = theta
        div = None
        if mode == "linear" and factor != 1.0:
            div = factor
        elif mode == "ntk" and factor != 1.0:
            dim = 2 * pairs
            if dim > 2:
                axis_theta = theta * factor ** (dim / (dim - 2))
        plan.append((pairs, axis_theta, div))
    return plan


def rotary_tables_f64(
    coords: np.ndarray,
    head_dim: int,
    theta: float = 10000.0,
    time_scale: float = 1.0,
    scaling: tuple[str, float, float] = ("none", 1.0, 1.0),
) -> tuple[np.ndarray, np.ndarray]:
    """Exact (float64) cos/sin tables ``(B, 1, L, pairs)``
    (src/avgen/models/rope.py:264-294): per axis ``angle = pos * theta_a^(-k/pairs_a)``
    with ``pos`` multiplied by time_scale on axis 0 and divided by the linear
    factor; axes concatenated t | h | w."""
    coords = np.asarray(coords, dtype=np.float64)
    angles = []
    for axis, (pairs, axis_theta, div) in enumerate(axis_plan(head_dim, theta, scaling)):
        pos = coords[..., axis]
        if axis == 0 and time_scale != 1.0:
            pos = pos * time_scale
        if div is not None:
            pos = pos / div
        inv = axis_theta ** (-(np.arange(pairs, dtype=np.float64) / pairs))
        angles.append(pos[..., None] * inv)
    phase = np.concatenate(angles, axis=-1)[:, None]
    return np.cos(phase), np.sin(phase)


def apply_rotary_bf16(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, inverse: bool = False) -> np.ndarray:
    """Interleaved-pair rotation exactly as src/avgen/models/rope.py:332-338
    evaluates it: float32 math, ``even*cos - odd*sin`` and ``even*sin +
    odd*cos`` with every product and sum rounded to float32 separately, then
    one round to bf16.  ``inverse`` gives the transpose ``(e*c + o*s, o*c -
    e*s)``, which is what torch autograd computes for the gradient of the
    forward rotation (each product rounded, then one add).

    x: ``(B, H, L, D)`` float32 holding bf16 values; tables float32 ``(B|1, 1, L, D/2)``.
    """
    x = np.asarray(x, dtype=np.float32)
    c = np.asarray(cos, dtype=np.float32)
    s = np.asarray(sin, dtype=np.float32)
    e = x[..., 0::2]
    o = x[..., 1::2]
    with np.errstate(over="ignore", invalid="ignore"):
        if not inverse:
            a = (e * c).astype(np.float32) - (o * s).astype(np.float32)
            b = (e * s).astype(np.float32) + (o * c).astype(np.float32)
        else:
            a = (e * c).astype(np.float32) + (o * s).astype(np.float32)
            b = (o * c).astype(np.float32) - (e * s).astype(np.float32)
    out = np.empty_like(x)
    out[..., 0::2] = a
    out[..., 1::2] = b
    return bf16_round(out)


# ---------------------------------------------------------------------------
# QK RMSNorm  (src/avgen/models/layers.py:70-118, 153-174, 530-531)
# ---------------------------------------------------------------------------


def rms_norm_bf16(x: np.ndarray, weight: np.ndarray | None, eps: float = 1e-6) -> np.ndarray:
    """F.rms_norm over the last axis as FusedRMSNorm calls it on bf16
    activations (src/avgen/models/layers.py:106-118: the gain cast to bf16):
    float32 ``rstd = 1/sqrt(mean(x^2) + eps)``, ``(x * rstd) * w`` in float32,
    rounded once to bf16.  ``x`` holds bf16 values as float32."""
    x = np.asarray(x, np.float32)
    D = x.shape[-1]
    ms = (np.square(x, dtype=np.float32).sum(axis=-1, keepdims=True, dtype=np.float32) / np.float32(D)).astype(np.float32)
    rstd = (np.float32(1.0) / np.sqrt(ms + np.float32(eps), dtype=np.float32)).astype(np.float32)
    t = (x * rstd).astype(np.float32)
    if weight is not None:
        t = (t * bf16_round(np.asarray(weight, np.float32))).astype(np.float32)
    return bf16_round(t)


def rms_norm_f64(x: np.ndarray, weight: np.ndarray | None, eps: float = 1e-6) -> np.ndarray:
    """F.rms_norm over the last axis in float64 with the gain as given: a
    float32 model's FusedRMSNorm outside autocast
    (src/avgen/models/layers.py:106-118, the gain kept in fp32)."""
    x = np.asarray(x, np.float64)
    y = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return y if weight is None else y * np.asarray(weight, np.float64)


def rms_norm_bwd_f64(
    x: np.ndarray, weight: np.ndarray | None, g: np.ndarray, eps: float = 1e-6, round_gain: bool = True
) -> tuple[np.ndarray, np.ndarray | None]:
    """Gradients of ``y = x * rstd(x) * w`` over the last axis in float64:
    ``dx = rstd * (w*g - xh * mean(w*g*xh))``, ``xh = x*rstd``, and
    ``dw = sum(g * xh)`` over every other axis (None without a gain).  The
    gain is rounded to bf16 first (bf16 activations), unless ``round_gain``
    is False (float32 activations keep it in fp32)."""
    x = np.asarray(x, np.float64)
    g = np.asarray(g, np.float64)
    if weight is None:
        w = np.ones(x.shape[-1])
    elif round_gain:
        w = bf16_round(np.asarray(weight, np.float32)).astype(np.float64)
    else:
        w = np.asarray(weight, np.float64)
    rstd = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    xh = x * rstd
    wg = w * g
    dx = rstd * (wg - xh * np.mean(wg * xh, axis=-1, keepdims=True))
    dw = None if weight is None else (g * xh).reshape(-1, x.shape[-1]).sum(0)
    return dx, dw


def video_coords(frames: int, height: int, width: int, fps: float = 8.0,
                 patch: tuple[int, int] = (2, 2), batch: int = 1) -> np.ndarray:
    """``(B, F*H*W, 3)`` float32 ``(seconds, row*patch_h, col*patch_w)``, token
    order time -> row -> column (src/avgen/core/patchify.py:45-105 with
    temporal patch 1; 8 fps is the synthetic default, src/avgen/data/
    synthetic.py:160-161)."""
    t = (np.arange(frames, dtype=np.float32) / np.float32(fps)).astype(np.float32)
    r = np.arange(height, dtype=np.float32) * np.float32(patch[0])
    c = np.arange(width, dtype=np.float32) * np.float32(patch[1])
    tg, rg, cg = np.meshgrid(t, r, c, indexing="ij")
    xyz = np.stack([tg.reshape(-1), rg.reshape(-1), cg.reshape(-1)], axis=-1).astype(np.float32)
    return np.broadcast_to(xyz, (batch,) + xyz.shape).copy()


def temporal_coords(positions: np.ndarray, frames: int, height: int, width: int,
                    patch: tuple[int, int, int] = (1, 2, 2), normalize_space: bool = False) -> np.ndarray:
    """src/avgen/core/patchify.py:45-105 (build_temporal_coords) with an
    explicit loop over tokens: token ``(f, r, c)`` of the post-patch grid
    gets ``(mean of positions[b, f*pf:(f+1)*pf], r*ph, c*pw)`` (or ``r/(gh-1)``,
    ``c/(gw-1)`` with ``normalize_space``), in float32, time -> row -> column
    order.  ``positions`` is ``(B, frames)`` seconds before temporal patching."""
    pos = np.asarray(positions, np.float32)
    pf, ph, pw = patch
    gf, gh, gw = frames // pf, height // ph, width // pw
    out = np.empty((pos.shape[0], gf * gh * gw, 3), np.float32)
    for b in range(pos.shape[0]):
        i = 0
        for f in range(gf):
            t = np.float32(pos[b, f * pf:(f + 1) * pf].astype(np.float64).mean())
            for r in range(gh):
                for c in range(gw):
                    if normalize_space:
                        y = np.float32(r) / np.float32(max(gh - 1, 1))
                        x = np.float32(c) / np.float32(max(gw - 1, 1))
                    else:
                        y, x = np.float32(r * ph), np.float32(c * pw)
                    out[b, i] = (t, y, x)
                    i += 1
    return out


# ---------------------------------------------------------------------------
# Attention with key-padding mask and LSE  (src/avgen/models/attention.py)
# ---------------------------------------------------------------------------


def key_padding_mask(mask: np.ndarray | None, assume_dense: bool = False) -> np.ndarray | None:
    """src/avgen/models/attention.py:183-224: None when absent, assumed dense
    or all valid; else ``mask[:, None, None, :]``."""
    if mask is None or assume_dense:
        return None
    mask = np.asarray(mask)
    if mask.ndim != 2:
        raise ValueError("key mask must have rank 2 (batch, keys)")
    if mask.dtype != np.bool_:
        raise TypeError("key mask must be bool")
    if mask.size == 0 or bool(mask.all()):
        return None
    return mask[:, None, None, :]


def _expand_kv(k: np.ndarray, hq: int) -> np.ndarray:
    hk = k.shape[1]
    return np.repeat(k, hq // hk, axis=1) if hk != hq else k


def _dense_mask(key_mask, attn_mask):
    """Combined ``(B|1, 1, Lq|1, Lk)`` bool mask (True = attend), or None."""
    m = None
    if key_mask is not None:
        m = np.asarray(key_mask, bool)[:, None, None, :]
    if attn_mask is not None:
        a = np.asarray(attn_mask, bool)
        a = a[:, None] if a.ndim == 3 else a
        m = a if m is None else (m & a)
    return m


def attention_f64(
    q: np.ndarray, k: np.ndarray, v: np.ndarray, key_mask: np.ndarray | None = None,
    scale: float | None = None, attn_mask: np.ndarray | None = None,
) -> tuple[np.ndarray, np.ndarray]:
    """Softmax attention in float64 (the math of F.scaled_dot_product_attention
    called at src/avgen/models/attention.py:265-273, default scale 1/sqrt(D)).

    key_mask: ``(B|1, Lk)`` bool, True = attend; attn_mask: a dense
    ``(B|1, [1,] Lq, Lk)`` bool mask (the query-dependent masks of
    :func:`temporal_neighbour_mask` and :func:`packed_attention_mask`), and-ed
    with key_mask.  Returns ``(out, lse)``:
    ``out (B, H, Lq, D)``, ``lse (B, H, Lq)`` natural log.  A row with no
    valid key gives out = 0 (what F.scaled_dot_product_attention returns) and
    lse = -inf.  Zero-length keys give zeros (src/avgen/models/attention.py
    :261-262).

    Non-finite inputs follow the math of SDPA's masked softmax: a mask is an
    additive 0 / -inf bias (so a NaN score stays NaN even at a masked key,
    as torch's math path computes it), and a row holding a NaN or a +inf
    score gets out = NaN and lse = NaN (softmax(+inf, ...) is inf/inf).
    Only a row whose every score is -inf counts as "no valid key".
    """
    q = np.asarray(q, np.float64)
    k = _expand_kv(np.asarray(k, np.float64), q.shape[1])
    v = _expand_kv(np.asarray(v, np.float64), q.shape[1])
    B, H, Lq, D = q.shape
    if Lq == 0 or k.shape[2] == 0:
        return np.zeros_like(q), np.full((B, H, Lq), -np.inf)
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    with np.errstate(invalid="ignore", over="ignore"):
        s = np.einsum("bhqd,bhkd->bhqk", q, k) * scale
        m = _dense_mask(key_mask, attn_mask)
        if m is not None:
            s = s + np.where(m, 0.0, -np.inf)
    bad = (np.isnan(s) | np.isposinf(s)).any(axis=-1)  # (B, H, Lq)
    s = np.where(bad[..., None], -np.inf, s)
    mx = s.max(axis=-1, keepdims=True)
    safe = np.where(np.isfinite(mx), mx, 0.0)
    p = np.exp(s - safe)
    l = p.sum(axis=-1, keepdims=True)
    with np.errstate(divide="ignore", invalid="ignore"):
        out = np.where(l > 0, np.einsum("bhqk,bhkd->bhqd", p, v) / np.where(l > 0, l, 1.0), 0.0)
        lse = np.where(l[..., 0] > 0, np.log(np.where(l[..., 0] > 0, l[..., 0], 1.0)) + safe[..., 0], -np.inf)
    out = np.where(bad[..., None], np.nan, out)
    lse = np.where(bad, np.nan, lse)
    return out, lse


# ---------------------------------------------------------------------------
# Query-dependent masks: temporal neighbourhoods (src/avgen/models/blocks.py)
# and packed variable-length sequences (src/avgen/data/packing.py)
# ---------------------------------------------------------------------------


def temporal_neighbour_mask(
    query_seconds: np.ndarray, key_seconds: np.ndarray, window_seconds: float,
    key_mask: np.ndarray | None = None,
) -> np.ndarray | None:
    """src/avgen/models/blocks.py:54-104: ``(B, 1, Lq, Lk)`` bool, True where
    ``|tq - tk| <= window_seconds`` and the key is valid; a query row with no
    admissible key attends to every key (the key mask included, :101-103).
    ``window_seconds <= 0``: None when every key is valid (or no mask), else
    the key mask as ``(B, 1, 1, Lk)`` (:92-95)."""
    if window_seconds <= 0.0:
        if key_mask is None or bool(np.asarray(key_mask, bool).all()):
            return None
        return np.asarray(key_mask, bool)[:, None, None, :]
    tq = np.asarray(query_seconds)
    tk = np.asarray(key_seconds)
    m = np.abs(tq[:, :, None] - tk[:, None, :]) <= window_seconds
    if key_mask is not None:
        m = m & np.asarray(key_mask, bool)[:, None, :]
    m = m | ~m.any(axis=-1, keepdims=True)
    return m[:, None]


PADDING_SEGMENT = -1


def packed_segment_ids(lengths: Sequence[int], capacity: int) -> np.ndarray:
    """src/avgen/data/packing.py:136-158: ``(capacity,)`` int32 segment index of
    each position, PADDING_SEGMENT past the last segment."""
    ids = np.full(capacity, PADDING_SEGMENT, np.int32)
    start = 0
    for seg, n in enumerate(lengths):
        ids[start:start + n] = seg
        start += n
    return ids


def packed_cu_seqlens(lengths: Sequence[int]) -> np.ndarray:
    """src/avgen/data/packing.py:163-179: ``(segments + 1,)`` int32 bounds."""
    return np.concatenate([[0], np.cumsum(np.asarray(lengths, np.int64))]).astype(np.int32)


def packed_attention_mask(lengths: Sequence[int], capacity: int) -> np.ndarray:
    """src/avgen/data/packing.py:181-200: ``(capacity, capacity)`` bool,
    True where row and column lie in the same segment; padding positions
    attend to nothing and are attended to by nothing."""
    ids = packed_segment_ids(lengths, capacity)
    valid = ids != PADDING_SEGMENT
    return (ids[:, None] == ids[None, :]) & valid[:, None] & valid[None, :]


# ---------------------------------------------------------------------------
# fp8 (e4m3) q k^T variant.  The reference has no fp8 path (its attention is
# bf16 SDPA, src/avgen/models/attention.py:265-273); this is the sampling-time
# configuration's definition: per-head absmax scales, OCP e4m3 operands (k
# quantized with its scale, q against the softmax constant and k's scale
# with a power-of-two block exponent), everything else as attention_f64.
# ---------------------------------------------------------------------------

E4M3_MAX = 448.0


def e4m3_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest OCP FP8 E4M3 value (ties to even),
    returned as float32.

    E4M3: exponent bias 7, 3 mantissa bits, normal values down to 2**-6,
    subnormals in steps of 2**-9, largest finite 448, no infinities (a value
    that rounds above 448 — |x| > 464 — is NaN, as is NaN).  Signed zeros
    keep their sign.
    """
    f = np.asarray(x, dtype=np.float32).astype(np.float64)
    a = np.abs(f)
    _, ex = np.frexp(a)  # a = m * 2**ex, 0.5 <= m < 1
    e = np.maximum(ex - 1, -6)  # exponent of the binade, clamped at the subnormal range
    step = np.ldexp(1.0, e - 3)  # spacing of 3-bit mantissas in that binade
    with np.errstate(invalid="ignore"):
        r = np.round(a / step) * step  # np.round: half to even
        r = np.where((r > E4M3_MAX) | np.isnan(f), np.nan, r)
    return np.copysign(r, f).astype(np.float32)


def fp8_absmax_scale(x: np.ndarray) -> np.ndarray:
    """Per-head scales of ``x (B, H, L, D)``: float32(max |x[:, h]|) / 448 in
    float32 (correctly rounded), 1 for an all-zero head."""
    m = np.abs(np.asarray(x, np.float32)).max(axis=(0, 2, 3)) if x.size else np.zeros(x.shape[1], np.float32)
    m = m.astype(np.float32)
    return np.where(m > 0, m / np.float32(E4M3_MAX), np.float32(1.0)).astype(np.float32)


def fp8_quantize(x: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """e4m3(x * (1/scale[h])) per head, the product and reciprocal in float32
    (each correctly rounded); returns the e4m3 values as float32."""
    inv = (np.float32(1.0) / np.asarray(scale, np.float32)).astype(np.float32)
    return e4m3_round(np.asarray(x, np.float32) * inv[None, :, None, None])


LOG2E_F32 = np.float32(1.4426950408889634)


def ceil_log2_clamped(t: np.ndarray) -> np.ndarray:
    """The smallest integer e with 2**e >= |t| for float32 t, clamped to
    [-126, 127]: zero and subnormal t give -126, infinite or NaN t 127."""
    a = np.abs(np.asarray(t, np.float32)).astype(np.float64)
    with np.errstate(invalid="ignore", divide="ignore"):
        f, ex = np.frexp(a)  # a = f * 2**ex, 0.5 <= f < 1
    e = np.where(f == 0.5, ex - 1, ex).astype(np.int64)
    e = np.where(a < 2.0**-126, -126, e)
    e = np.where(~np.isfinite(a), 127, e)
    return np.clip(e, -126, 127)


def fp8_q_operand(q: np.ndarray, q_scale: np.ndarray, k_scale: np.ndarray, scale: float):
    """The fp8 forward's q operand and its block exponent, per head h with
    kv head hk = h // (Hq // Hkv): g = f32(f32(scale * log2 e) * k_scale[hk]),
    eq = ceil_log2_clamped(f32(g * q_scale[h])) (so 2**eq >= g * q_scale[h]),
    q8 = e4m3(f32(q * f32(g * 2**-eq))).  The scores the kernel forms are
    ``2**eq * (q8 . k8)`` in log2 units (k8 = fp8_quantize(k, k_scale)).
    Returns ``(q8, eq)``: q8 float32 e4m3 values, eq int64 (Hq,)."""
    q = np.asarray(q, np.float32)
    hq, hkv = q.shape[1], np.asarray(k_scale).shape[0]
    ks = np.asarray(k_scale, np.float32)[np.arange(hq) // (hq // hkv)]
    sl2 = np.float32(np.float32(scale) * LOG2E_F32)
    g = (sl2 * ks).astype(np.float32)
    eq = ceil_log2_clamped((g * np.asarray(q_scale, np.float32)).astype(np.float32))
    mult = np.ldexp(g, -eq).astype(np.float32)
    return e4m3_round((q * mult[None, :, None, None]).astype(np.float32)), eq


def attention_fp8_f64(
    q: np.ndarray, k: np.ndarray, v: np.ndarray, q_scale: np.ndarray, k_scale: np.ndarray,
    key_mask: np.ndarray | None = None, scale: float | None = None,
) -> tuple[np.ndarray, np.ndarray]:
    """attention_f64 on the fp8 forward's scores: ``2**eq[h] * (q8 . k8)``
    log2-unit scores (fp8_q_operand, fp8_quantize), i.e. natural-log scores
    ``ln 2 * 2**eq[h] * (q8 . k8)``, which approximate ``scale * (q . k)``.

    q8, k8 and the power of two are exact in float64, so this is
    attention_f64 on ``q8 * 2**eq * ln 2`` and ``k8`` with unit scale.
    """
    D = np.asarray(q).shape[-1]
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    q8, eq = fp8_q_operand(q, q_scale, k_scale, scale)
    qd = q8.astype(np.float64) * np.ldexp(1.0, eq)[None, :, None, None] * math.log(2.0)
    kd = fp8_quantize(k, k_scale).astype(np.float64)
    return attention_f64(qd, kd, v, key_mask, 1.0)


def attention_bwd_f64(
    dout: np.ndarray, q: np.ndarray, k: np.ndarray, v: np.ndarray, out: np.ndarray, lse: np.ndarray,
    key_mask: np.ndarray | None = None, scale: float | None = None, attn_mask: np.ndarray | None = None,
) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Flash-attention backward in float64 given (possibly merged) ``out``/``lse``
    (what the ring backward hands the op, torch/.../_attention.py:567-575):
    ``P = exp(s*QK^T - lse)``, ``dV = P^T dO``, ``dP = dO V^T``,
    ``Dr = rowsum(dO * O)``, ``dS = P * (dP - Dr)``, ``dQ = s dS K``,
    ``dK = s dS^T Q``.  With grouped KV heads, dK/dV sum over each group."""
    q = np.asarray(q, np.float64)
    hq, hk = q.shape[1], np.asarray(k).shape[1]
    kk = _expand_kv(np.asarray(k, np.float64), hq)
    vv = _expand_kv(np.asarray(v, np.float64), hq)
    do = np.asarray(dout, np.float64)
    o = np.asarray(out, np.float64)
    lse = np.asarray(lse, np.float64)
    D = q.shape[-1]
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    s = np.einsum("bhqd,bhkd->bhqk", q, kk) * scale
    lse_b = np.where(np.isfinite(lse), lse, np.inf)[..., None]
    p = np.exp(s - lse_b)
    m = _dense_mask(key_mask, attn_mask)
    if m is not None:
        p = np.where(m, p, 0.0)
    dv = np.einsum("bhqk,bhqd->bhkd", p, do)
    dp = np.einsum("bhqd,bhkd->bhqk", do, vv)
    dr = (do * o).sum(-1, keepdims=True)
    ds = p * (dp - dr)
    dq = np.einsum("bhqk,bhkd->bhqd", ds, kk) * scale
    dk = np.einsum("bhqk,bhqd->bhkd", ds, q) * scale
    if hk != hq:
        g = hq // hk
        dk = dk.reshape(dk.shape[0], hk, g, *dk.shape[2:]).sum(2)
        dv = dv.reshape(dv.shape[0], hk, g, *dv.shape[2:]).sum(2)
    return dq, dk, dv


def attention_bwd_magnitudes_f64(
    dout: np.ndarray, q: np.ndarray, k: np.ndarray, v: np.ndarray, out: np.ndarray, lse: np.ndarray,
    key_mask: np.ndarray | None = None, scale: float | None = None, attn_mask: np.ndarray | None = None,
) -> tuple[np.ndarray, np.ndarray]:
    """The size of the terms dq and dk are computed from, for error floors:
    ``s (P * (|dP| + |Dr|)) |K|`` and ``s (P * (|dP| + |Dr|))^T |Q|``, the
    formulas of :func:`attention_bwd_f64` with every factor of ``dS = P *
    (dP - Dr)`` taken in absolute value (dK summed over a GQA group).
    ``dP - Dr`` cancels where one key carries the row's weight (one key:
    ``dP == Dr`` exactly, so dq = dk = 0), and any finite-precision
    evaluation of it carries a rounding error proportional to ``|dP| +
    |Dr|``, not to the result; these are the scales of that error."""
    q = np.asarray(q, np.float64)
    hq, hk = q.shape[1], np.asarray(k).shape[1]
    kk = _expand_kv(np.asarray(k, np.float64), hq)
    vv = _expand_kv(np.asarray(v, np.float64), hq)
    do = np.asarray(dout, np.float64)
    o = np.asarray(out, np.float64)
    lse = np.asarray(lse, np.float64)
    D = q.shape[-1]
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    s = np.einsum("bhqd,bhkd->bhqk", q, kk) * scale
    lse_b = np.where(np.isfinite(lse), lse, np.inf)[..., None]
    p = np.exp(s - lse_b)
    m = _dense_mask(key_mask, attn_mask)
    if m is not None:
        p = np.where(m, p, 0.0)
    dp = np.einsum("bhqd,bhkd->bhqk", do, vv)
    dr = (do * o).sum(-1, keepdims=True)
    w = p * (np.abs(dp) + np.abs(dr))
    mq = np.einsum("bhqk,bhkd->bhqd", w, np.abs(kk)) * scale
    mk = np.einsum("bhqk,bhqd->bhkd", w, np.abs(q)) * scale
    if hk != hq:
        mk = mk.reshape(mk.shape[0], hk, hq // hk, *mk.shape[2:]).sum(2)
    return mq, mk


# ---------------------------------------------------------------------------
# Ring merge and ring loops  (torch/.../_context_parallel/_attention.py)
# ---------------------------------------------------------------------------


def _sigmoid_f32(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        return (np.float32(1) / (np.float32(1) + np.exp(-x))).astype(np.float32)


def _logsigmoid_f32(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        return (np.minimum(x, np.float32(0)) - np.log1p(np.exp(-np.abs(x)))).astype(np.float32)


def lse_merge_f32(out: np.ndarray, lse: np.ndarray, out_b: np.ndarray, lse_b: np.ndarray):
    """One ``_SDPAMerger._merge_one`` step (torch/.../_attention.py:182-183) in
    float32: ``out - sigmoid(lse_b - lse) * (out - out_b)`` and ``lse -
    logsigmoid(lse - lse_b)``.  A -inf LSE is the identity element (a block of
    fully masked rows changes nothing; an empty accumulator takes the block),
    where torch's formula would give NaN.  lse shapes are ``(..., )`` without
    the trailing singleton."""
    out = np.asarray(out, np.float32)
    out_b = np.asarray(out_b, np.float32)
    lse = np.asarray(lse, np.float32)
    lse_b = np.asarray(lse_b, np.float32)
    with np.errstate(invalid="ignore"):
        w = _sigmoid_f32((lse_b - lse).astype(np.float32))[..., None]
        merged = (out - (w * (out - out_b)).astype(np.float32)).astype(np.float32)
        mlse = (lse - _logsigmoid_f32((lse - lse_b).astype(np.float32))).astype(np.float32)
    b_empty = np.isneginf(lse_b)
    a_empty = np.isneginf(lse) & ~b_empty
    merged = np.where(b_empty[..., None], out, np.where(a_empty[..., None], out_b, merged))
    mlse = np.where(b_empty, lse, np.where(a_empty, lse_b, mlse))
    return merged.astype(np.float32), mlse.astype(np.float32)


def lse_merge_f64(out: np.ndarray, lse: np.ndarray, out_b: np.ndarray, lse_b: np.ndarray):
    """Exact (float64) combination of two partial softmax results: weights
    ``exp(lse - L)`` and ``exp(lse_b - L)`` with ``L = logaddexp(lse, lse_b)``."""
    lse = np.asarray(lse, np.float64)
    lse_b = np.asarray(lse_b, np.float64)
    with np.errstate(invalid="ignore"):
        L = np.logaddexp(lse, lse_b)  # NaN in either stays NaN
        wa = np.where(np.isneginf(lse), 0.0, np.exp(lse - np.where(np.isneginf(L), 0.0, L)))
        wb = np.where(np.isneginf(lse_b), 0.0, np.exp(lse_b - np.where(np.isneginf(L), 0.0, L)))
    return wa[..., None] * np.asarray(out, np.float64) + wb[..., None] * np.asarray(out_b, np.float64), L


def ring_forward_f64(q, keys: Sequence, values: Sequence, masks: Sequence | None = None, scale=None):
    """Non-causal ring forward (torch/.../_attention.py:422-478): per chunk
    attention, then merge in ring order.  Float64 throughout."""
    masks = masks if masks is not None else [None] * len(keys)
    out, lse = attention_f64(q, keys[0], values[0], masks[0], scale)
    for k, v, m in zip(keys[1:], values[1:], masks[1:]):
        ob, lb = attention_f64(q, k, v, m, scale)
        out, lse = lse_merge_f64(out, lse, ob, lb)
    return out, lse


def ring_backward_f64(dout, q, keys, values, out, lse, masks=None, scale=None):
    """Non-causal ring backward (torch/.../_attention.py:514-646): each
    chunk's backward with the merged out/lse; dq summed over chunks."""
    masks = masks if masks is not None else [None] * len(keys)
    dq = np.zeros(np.shape(q))
    dks, dvs = [], []
    for k, v, m in zip(keys, values, masks):
        a, b, c = attention_bwd_f64(dout, q, k, v, out, lse, m, scale)
        dq = dq + a
        dks.append(b)
        dvs.append(c)
    return dq, dks, dvs


# ---------------------------------------------------------------------------
# Context-parallel shard rules  (src/avgen/parallel/context.py)
# ---------------------------------------------------------------------------


def sharded_length(total: int, shards: int) -> int:
    """src/avgen/parallel/context.py:58-80."""
    if total % shards != 0:
        raise ValueError(f"sequence length {total} is not divisible by context-parallel degree {shards}")
    return total // shards


def shard_bounds(total: int, shards: int, index: int) -> tuple[int, int]:
    """src/avgen/parallel/context.py:159-163."""
    local = sharded_length(total, shards)
    return index * local, (index + 1) * local


def pad_to_multiple(tokens: np.ndarray, coords: np.ndarray, mask: np.ndarray, multiple: int):
    """src/avgen/parallel/context.py:83-139: zero tokens/coords, False mask."""
    if multiple < 1:
        raise ValueError("multiple must be positive")
    L = tokens.shape[1]
    pad = (-L) % multiple
    if pad == 0:
        return tokens, coords, mask

    def _pad(t):
        shape = list(t.shape)
        shape[1] = pad
        return np.concatenate([t, np.zeros(shape, dtype=t.dtype)], axis=1)

    return _pad(tokens), _pad(coords), _pad(mask)


# ---------------------------------------------------------------------------
# FLOP convention  (src/avgen/simulate/compute.py:126,142)
# ---------------------------------------------------------------------------


def attention_flops(batch: int, heads: int, len_q: int, len_k: int, head_dim: int, backward: bool = True) -> float:
    """Algorithmic attention FLOPs: ``2*2*Lq*Lk*D`` per (batch, head) forward
    (scores + value-weighted sum, src/avgen/simulate/compute.py:126), times 3
    with the backward (:142).  The backward's recompute of QK^T is not counted."""
    fwd = 4.0 * batch * heads * len_q * len_k * head_dim
    return fwd * (3.0 if backward else 1.0)
