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
    return out


def main() -> None:
    for name, arrays in build().items():
        np.savez_compressed(HERE / f"{name}.npz", **arrays)
        print("wrote", name)


if __name__ == "__main__":
    main()
