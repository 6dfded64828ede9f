"""Write the small golden fixtures in tests/golden/ from the pinned CPU oracle.

The reference ships no golden vectors for this path, so these are produced by
``oracle/reference.py`` (itself pinned by tests/test_oracle.py) and committed
as data: inputs (bf16 values stored as uint16 bit patterns, fp32 coords) and
expected outputs (float64/float32).  Re-running this script must reproduce
the committed files bit for bit (checked by tests/test_golden.py).

Usage: python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import reference as R  # noqa: E402


def _bf16(rng: np.random.Generator, shape, scale=1.0) -> np.ndarray:
    return R.bf16_round((rng.standard_normal(shape) * scale).astype(np.float32))


def build() -> dict[str, dict[str, np.ndarray]]:
    out: dict[str, dict[str, np.ndarray]] = {}

    # RoPE tables for a 2x3x4 grid (2 frames at 8 fps, 2x2 patches).
    coords = R.video_coords(2, 3, 4, fps=8.0, patch=(2, 2))
    for d in (12, 128):
        cos, sin = R.rotary_tables_f64(coords, d)
        out[f"rope_tables_d{d}"] = {"coords": coords, "cos": cos, "sin": sin}
    cos, sin = R.rotary_tables_f64(coords, 128, time_scale=1.5, scaling=("ntk", 2.0, 1.5))
    out["rope_tables_d128_ntk"] = {"coords": coords, "cos": cos, "sin": sin,
                                   "time_scale": np.float64(1.5), "factors": np.array([2.0, 1.5])}

    # RoPE rotation (bit-exact fixture) at d=64 on the same grid.
    rng = np.random.default_rng(20261201)
    c64, s64 = R.rotary_tables_f64(coords, 64)
    c32, s32 = c64.astype(np.float32), s64.astype(np.float32)
    x = _bf16(rng, (1, 2, coords.shape[1], 64), 2.0)
    out["rope_apply_d64"] = {
        "x_bits": R.bf16_bits(x), "cos": c32, "sin": s32,
        "out_bits": R.bf16_bits(R.apply_rotary_bf16(x, c32, s32)),
        "inv_bits": R.bf16_bits(R.apply_rotary_bf16(x, c32, s32, inverse=True)),
    }

    # Attention forward + backward with a key-padding mask (one fully masked
    # batch row), GQA, d=64 and d=128.
    for d, (B, H, Hk, Lq, Lk) in ((64, (2, 4, 2, 40, 56)), (128, (2, 2, 2, 33, 70))):
        q = _bf16(rng, (B, H, Lq, d))
        k = _bf16(rng, (B, Hk, Lk, d))
        v = _bf16(rng, (B, Hk, Lk, d))
        do = _bf16(rng, (B, H, Lq, d))
        mask = np.ones((B, Lk), bool)
        mask[0, Lk - 9:] = False
        mask[1, :] = False
        o, lse = R.attention_f64(q, k, v, mask)
        dq, dk, dv = R.attention_bwd_f64(do, q, k, v, o, lse, mask)
        out[f"attn_d{d}"] = {
            "q_bits": R.bf16_bits(q), "k_bits": R.bf16_bits(k), "v_bits": R.bf16_bits(v),
            "do_bits": R.bf16_bits(do), "mask": mask,
            "out": o.astype(np.float32), "lse": lse, "dq": dq.astype(np.float32),
            "dk": dk.astype(np.float32), "dv": dv.astype(np.float32),
        }

    # Ring: one query shard, 3 KV chunks, merged; the float32 merge step too.
    q = _bf16(rng, (1, 2, 24, 64))
    k = _bf16(rng, (1, 2, 60, 64))
    v = _bf16(rng, (1, 2, 60, 64))
    keys = [k[:, :, i:i + 20] for i in (0, 20, 40)]
    vals = [v[:, :, i:i + 20] for i in (0, 20, 40)]
    o, lse = R.ring_forward_f64(q, keys, vals)
    o1, l1 = R.attention_f64(q, keys[0], vals[0])
    o2, l2 = R.attention_f64(q, keys[1], vals[1])
    mo, ml = R.lse_merge_f32(o1.astype(np.float32), l1.astype(np.float32),
                             o2.astype(np.float32), l2.astype(np.float32))
    out["ring_3chunks"] = {
        "q_bits": R.bf16_bits(q), "k_bits": R.bf16_bits(k), "v_bits": R.bf16_bits(v),
        "out": o.astype(np.float32), "lse": lse, "merge01_out": mo, "merge01_lse": ml,
    }
    # Packed variable-length sequences (segments 3/4/2 in 12, the reference's
    # own test layout): block-diagonal mask and attention over it.
    lengths, cap = [3, 4, 2], 12
    pm = R.packed_attention_mask(lengths, cap)
    q = _bf16(rng, (1, 2, cap, 64))
    k = _bf16(rng, (1, 2, cap, 64))
    v = _bf16(rng, (1, 2, cap, 64))
    do = _bf16(rng, (1, 2, cap, 64))
    o, lse = R.attention_f64(q, k, v, attn_mask=pm[None])
    dq, dk, dv = R.attention_bwd_f64(do, q, k, v, o, lse, attn_mask=pm[None])
    out["packed_attention"] = {
        "lengths": np.array(lengths, np.int32), "capacity": np.int32(cap),
        "segment_ids": R.packed_segment_ids(lengths, cap), "cu_seqlens": R.packed_cu_seqlens(lengths), "mask": pm,
        "q_bits": R.bf16_bits(q), "k_bits": R.bf16_bits(k), "v_bits": R.bf16_bits(v), "do_bits": R.bf16_bits(do),
        "out": o.astype(np.float32), "lse": lse, "dq": dq.astype(np.float32), "dk": dk.astype(np.float32),
        "dv": dv.astype(np.float32),
    }

    # Temporal neighbour mask: video frames at 8 fps against audio tokens at
    # 20 per second, window 0.1 s, a key mask, and queries past the audio
    # (rows that fall back to every key).
    tq = np.stack([np.repeat(np.arange(8, dtype=np.float32) / np.float32(8.0), 3)] * 2)
    tk = np.stack([np.arange(12, dtype=np.float32) / np.float32(20.0)] * 2)
    tk[1] += np.float32(0.05)
    km = np.ones((2, 12), bool)
    km[1, ::3] = False
    tm = R.temporal_neighbour_mask(tq, tk, 0.1, km)
    q = _bf16(rng, (2, 4, 24, 128))
    k = _bf16(rng, (2, 2, 12, 128))
    v = _bf16(rng, (2, 2, 12, 128))
    o, lse = R.attention_f64(q, k, v, attn_mask=tm)
    out["temporal_attention"] = {
        "query_seconds": tq, "key_seconds": tk, "window_seconds": np.float64(0.1), "key_mask": km, "mask": tm,
        "q_bits": R.bf16_bits(q), "k_bits": R.bf16_bits(k), "v_bits": R.bf16_bits(v),
        "out": o.astype(np.float32), "lse": lse,
    }

    # QK RMSNorm + rotation on a (batch, seq, heads, dim) projection output.
    c128, s128 = R.rotary_tables_f64(coords, 128)
    c32, s32 = c128.astype(np.float32), s128.astype(np.float32)
    L = coords.shape[1]
    xp = _bf16(rng, (1, L, 3, 128), 3.0)
    x = xp.transpose(0, 2, 1, 3)
    w = R.bf16_round((rng.uniform(0.5, 1.5, 128)).astype(np.float32))
    n = R.rms_norm_bf16(x, w, 1e-6)
    y = R.apply_rotary_bf16(n, c32, s32)
    dy = _bf16(rng, x.shape)
    g = R.apply_rotary_bf16(dy, c32, s32, inverse=True)
    dx, dw = R.rms_norm_bwd_f64(x, w, g, 1e-6)
    out["qk_norm_rope_d128"] = {
        "x_bits": R.bf16_bits(xp), "w_bits": R.bf16_bits(w), "cos": c32, "sin": s32, "eps": np.float64(1e-6),
        "norm_bits": R.bf16_bits(n), "out_bits": R.bf16_bits(y), "dy_bits": R.bf16_bits(dy),
        "dx": dx.astype(np.float32), "dw": dw,
    }

    # fp8 (e4m3) q k^T forward: per-head absmax scales, GQA, a key mask with
    # one fully masked batch row; the quantized operands and the block
    # exponent are stored with the expected output.
    B, H, Hk, Lq, Lk, d = 2, 4, 2, 48, 80, 128
    q = _bf16(rng, (B, H, Lq, d), 2.0)
    k = _bf16(rng, (B, Hk, Lk, d))
    v = _bf16(rng, (B, Hk, Lk, d))
    mask = np.ones((B, Lk), bool)
    mask[0, 61:] = False
    mask[1, :] = False
    qs, ks = R.fp8_absmax_scale(q), R.fp8_absmax_scale(k)
    sc = np.float32(d ** -0.5)
    q8, eq = R.fp8_q_operand(q, qs, ks, float(sc))
    o, lse = R.attention_fp8_f64(q, k, v, qs, ks, mask, float(sc))
    out["attn_fp8_d128"] = {
        "q_bits": R.bf16_bits(q), "k_bits": R.bf16_bits(k), "v_bits": R.bf16_bits(v), "mask": mask,
        "q_scale": qs, "k_scale": ks, "scale": sc, "q8": q8, "eq": eq, "k8": R.fp8_quantize(k, ks),
        "out": o.astype(np.float32), "lse": lse,
    }
    return out


def main() -> None:
    for name, arrays in build().items():
        np.savez_compressed(HERE / f"{name}.npz", **arrays)
        print("wrote", name)


if __name__ == "__main__":
    main()
