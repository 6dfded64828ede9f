"""Pins the CPU oracle (oracle/) before it is trusted as the parity checker.

Each oracle function is checked against something other than its own
formula: closed forms and textbook special cases, an independent
implementation (PyTorch's CPU SDPA kernels and autograd), finite
differences, or invariants chosen so that a plausible slip (wrong pairing,
wrong sign, wrong exponent denominator, transposed operand, dropped term)
fails.  The reference ships no golden vectors for this path.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import reference as R
from oracle import torch_path as T


# ---------------------------------------------------------------------------
# bf16 rounding
# ---------------------------------------------------------------------------


def test_bf16_round_matches_torch_cast(rng):
    x = rng.standard_normal(20000).astype(np.float32) * 10.0
    edge = np.array(
        [0.0, -0.0, 1.0, 1.00390625, 1.005859375, 1.001953125, 3.0e38, -3.0e38, 1e-40, -1e-40, np.inf, -np.inf],
        dtype=np.float32,
    )
    # ties: bf16(1 + 2^-8) is a tie between 1 and 1+2^-7
    x = np.concatenate([x, edge, np.nextafter(edge, np.float32(np.inf)).astype(np.float32)])
    ours = R.bf16_round(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(ours.view(np.uint32), theirs.view(np.uint32))


def test_bf16_round_keeps_nan():
    assert np.isnan(R.bf16_round(np.array([np.nan], np.float32)))[0]


# ---------------------------------------------------------------------------
# rope_axis_pairs / tables (src/avgen/models/rope.py:128-294)
# ---------------------------------------------------------------------------


def test_rope_axis_pairs_closed_form():
    # values stated in the reference's own docstring and in the BASELINE configs
    assert R.rope_axis_pairs(64) == (12, 10, 10)
    assert R.rope_axis_pairs(128) == (22, 21, 21)
    assert R.rope_axis_pairs(6) == (1, 1, 1)
    assert R.rope_axis_pairs(8) == (2, 1, 1)
    for d in range(6, 258, 2):
        t, h, w = R.rope_axis_pairs(d)
        assert t + h + w == d // 2 and h == w and t >= h and t - h <= 2
    for bad in (0, 4, 5, 7, 127, -6):
        with pytest.raises(ValueError):
            R.rope_axis_pairs(bad)


def test_tables_zero_coords_are_identity():
    cos, sin = R.rotary_tables_f64(np.zeros((2, 5, 3), np.float32), 128)
    assert cos.shape == (2, 1, 5, 64)
    assert np.all(cos == 1.0) and np.all(sin == 0.0)


def test_tables_per_axis_denominator_known_values():
    # d=12 -> 2 pairs per axis; axis frequencies 1 and theta^(-1/2) = 0.01.
    # (A denominator of head_dim/2 instead of the axis's pair count would give
    # theta^(-1/6).)
    coords = np.array([[[1.0, 0.0, 0.0], [0.0, 1.0, 0.0], [0.0, 0.0, 3.0]]], np.float32)
    cos, sin = R.rotary_tables_f64(coords, 12, theta=10000.0)
    ang = np.arccos(np.clip(cos[0, 0], -1, 1)) * np.sign(sin[0, 0] + 1e-300)
    expected = np.array(
        [[1.0, 0.01, 0, 0, 0, 0], [0, 0, 1.0, 0.01, 0, 0], [0, 0, 0, 0, 3.0, 0.03]]
    )
    assert np.allclose(ang, expected, atol=1e-12)


def test_tables_time_scale_linear_and_ntk():
    coords = np.array([[[2.0, 4.0, 6.0]]], np.float32)
    base_c, base_s = R.rotary_tables_f64(coords, 12)
    c, s = R.rotary_tables_f64(coords, 12, time_scale=0.5)
    # time_scale 0.5 on t=2 equals t=1 unscaled
    c1, s1 = R.rotary_tables_f64(np.array([[[1.0, 4.0, 6.0]]], np.float32), 12)
    assert np.allclose(c, c1) and np.allclose(s, s1)
    # linear: positions divided by the factor (time factor 2, spatial 2)
    cl, sl = R.rotary_tables_f64(coords, 12, scaling=("linear", 2.0, 2.0))
    ch, sh = R.rotary_tables_f64(coords / 2, 12)
    assert np.allclose(cl, ch) and np.allclose(sl, sh)
    # ntk: dim = 4 per axis -> theta * f^(4/2); pair 1 frequency = (theta f^2)^(-1/2)
    cn, sn = R.rotary_tables_f64(np.array([[[1.0, 0.0, 0.0]]], np.float32), 12, scaling=("ntk", 3.0, 1.0))
    assert math.isclose(math.atan2(sn[0, 0, 0, 1], cn[0, 0, 0, 1]), 1.0 / (100.0 * 3.0), rel_tol=1e-12)
    assert base_c.shape == (1, 1, 1, 6)


@pytest.mark.parametrize("head_dim", [12, 64, 128])
def test_tables_f64_agree_with_torch_restatement(head_dim):
    coords = torch.from_numpy(R.video_coords(3, 4, 5))
    ct, st = T.rotary_tables(coords, head_dim, time_scale=1.7, scaling=("ntk", 2.0, 1.5))
    c, s = R.rotary_tables_f64(coords.numpy(), head_dim, time_scale=1.7, scaling=("ntk", 2.0, 1.5))
    # fp32 angle rounding bounds the difference: |angle| * 2^-23 + a few ulp
    tol = 2e-6 + 3e-7 * 12.0
    assert np.abs(ct.numpy() - c).max() < tol and np.abs(st.numpy() - s).max() < tol


# ---------------------------------------------------------------------------
# apply_rotary (src/avgen/models/rope.py:297-338)
# ---------------------------------------------------------------------------


def _rand_bf16(rng, shape, scale=1.0):
    return R.bf16_round((rng.standard_normal(shape) * scale).astype(np.float32))


def test_rotation_is_interleaved_with_standard_sign():
    # x = e_0 rotates to (cos, sin) in channels (0, 1); x = e_1 to (-sin, cos).
    theta0 = 0.7
    cos = np.full((1, 1, 1, 3), 1.0, np.float32)
    sin = np.zeros((1, 1, 1, 3), np.float32)
    cos[..., 0] = np.float32(math.cos(theta0))
    sin[..., 0] = np.float32(math.sin(theta0))
    e0 = np.zeros((1, 1, 1, 6), np.float32)
    e0[..., 0] = 1.0
    e1 = np.zeros((1, 1, 1, 6), np.float32)
    e1[..., 1] = 1.0
    r0 = R.apply_rotary_bf16(e0, cos, sin)[0, 0, 0]
    r1 = R.apply_rotary_bf16(e1, cos, sin)[0, 0, 0]
    assert np.array_equal(r0, R.bf16_round(np.array([cos[0, 0, 0, 0], sin[0, 0, 0, 0], 0, 0, 0, 0], np.float32)))
    assert np.array_equal(r1, R.bf16_round(np.array([-sin[0, 0, 0, 0], cos[0, 0, 0, 0], 0, 0, 0, 0], np.float32)))


def test_rotation_identity_at_zero_coords(rng):
    x = _rand_bf16(rng, (2, 3, 7, 12))
    cos, sin = R.rotary_tables_f64(np.zeros((2, 7, 3), np.float32), 12)
    out = R.apply_rotary_bf16(x, cos.astype(np.float32), sin.astype(np.float32))
    assert np.array_equal(out.view(np.uint32), x.view(np.uint32))


def test_rotation_matches_torch_restatement_bitwise(rng):
    coords = R.video_coords(3, 4, 5, batch=2)
    cos, sin = T.rotary_tables(torch.from_numpy(coords), 64)
    x = torch.randn(2, 3, coords.shape[1], 64).to(torch.bfloat16)
    ref = T.apply_rotary(x, cos, sin).float().numpy()
    ours = R.apply_rotary_bf16(x.float().numpy(), cos.numpy(), sin.numpy())
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))


def test_inverse_rotation_is_torch_autograd_gradient(rng):
    coords = R.video_coords(2, 3, 4)
    cos, sin = T.rotary_tables(torch.from_numpy(coords), 64)
    x = torch.randn(1, 2, coords.shape[1], 64).to(torch.bfloat16).requires_grad_(True)
    g = torch.randn(1, 2, coords.shape[1], 64).to(torch.bfloat16)
    T.apply_rotary(x, cos, sin).backward(g)
    ours = R.apply_rotary_bf16(g.float().numpy(), cos.numpy(), sin.numpy(), inverse=True)
    assert np.array_equal(ours.view(np.uint32), x.grad.float().numpy().view(np.uint32))


def test_rotation_norm_and_relative_position(rng):
    # Rotation is orthogonal per pair: norms preserved (up to the bf16 round),
    # and <R(p) q, R(p') k> depends only on p - p'.
    q = _rand_bf16(rng, (1, 1, 1, 12))
    k = _rand_bf16(rng, (1, 1, 1, 12))

    def rot(x, pos):
        c, s = R.rotary_tables_f64(np.array([[pos]], np.float32), 12)
        return R.apply_rotary_bf16(x, c.astype(np.float32), s.astype(np.float32)).astype(np.float64)

    for pos in ([0.5, 3.0, 7.0], [2.0, 0.0, 11.0]):
        r = rot(q, pos)
        pr = r.reshape(-1, 2)
        p0 = q.astype(np.float64).reshape(-1, 2)
        assert np.allclose(np.linalg.norm(pr, axis=1), np.linalg.norm(p0, axis=1), rtol=2 ** -7)
    d1 = float((rot(q, [1.0, 2.0, 3.0]) * rot(k, [0.5, 1.0, 1.0])).sum())
    d2 = float((rot(q, [2.5, 5.0, 10.0]) * rot(k, [2.0, 4.0, 8.0])).sum())
    assert abs(d1 - d2) < 0.05 * (1 + abs(d1))


# ---------------------------------------------------------------------------
# Attention + LSE (src/avgen/models/attention.py:227-273 -> SDPA)
# ---------------------------------------------------------------------------


def _qkv(rng, B=2, H=3, Hk=None, Lq=9, Lk=13, D=16):
    Hk = H if Hk is None else Hk
    return (rng.standard_normal((B, H, Lq, D)), rng.standard_normal((B, Hk, Lk, D)),
            rng.standard_normal((B, Hk, Lk, D)))


def test_attention_matches_torch_sdpa_float64(rng):
    q, k, v = _qkv(rng)
    mask = rng.random((2, 13)) > 0.3
    mask[:, 0] = True
    out, lse = R.attention_f64(q, k, v, mask)
    ref = F.scaled_dot_product_attention(
        torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v),
        attn_mask=torch.from_numpy(mask)[:, None, None, :],
    ).numpy()
    assert np.abs(out - ref).max() < 1e-12
    # LSE against PyTorch's CPU flash kernel (float32 inputs)
    _, lse_t = T.chunk_fwd(torch.from_numpy(q).float(), torch.from_numpy(k).float(),
                           torch.from_numpy(v).float(), torch.from_numpy(mask))
    assert np.abs(lse - lse_t.numpy()).max() < 1e-5


def test_attention_special_cases(rng):
    q, k, v = _qkv(rng, B=1, H=1, Lq=4, Lk=6, D=8)
    # identical keys -> uniform weights: out = mean(v), lse = s + log(Lk)
    k_same = np.repeat(k[:, :, :1], 6, axis=2)
    out, lse = R.attention_f64(q, k_same, v)
    s = (q @ k_same[0, 0, 0]) / math.sqrt(8)
    assert np.allclose(out, v.mean(axis=2, keepdims=True).repeat(4, axis=2))
    assert np.allclose(lse, s + math.log(6))
    # one key -> out = v, lse = score
    out1, lse1 = R.attention_f64(q, k[:, :, :1], v[:, :, :1])
    assert np.allclose(out1, np.repeat(v[:, :, :1], 4, axis=2))
    assert np.allclose(lse1, (q @ k[0, 0, 0]) / math.sqrt(8))
    # empty keys -> zeros (src/avgen/models/attention.py:261-262)
    out0, lse0 = R.attention_f64(q, k[:, :, :0], v[:, :, :0])
    assert np.all(out0 == 0) and np.all(np.isneginf(lse0))


def test_masked_keys_equal_deleted_keys(rng):
    q, k, v = _qkv(rng, B=1, H=2, Lq=5, Lk=10, D=8)
    mask = np.array([[True, False, True, True, False, False, True, True, False, True]])
    out, lse = R.attention_f64(q, k, v, mask)
    keep = mask[0]
    out2, lse2 = R.attention_f64(q, k[:, :, keep], v[:, :, keep])
    assert np.allclose(out, out2, atol=1e-13) and np.allclose(lse, lse2, atol=1e-13)


def test_fully_masked_rows_give_zero_and_neg_inf(rng):
    q, k, v = _qkv(rng, B=2, H=1, Lq=3, Lk=4, D=8)
    mask = np.array([[False] * 4, [True, False, True, False]])
    out, lse = R.attention_f64(q, k, v, mask)
    assert np.all(out[0] == 0) and np.all(np.isneginf(lse[0]))
    assert np.all(np.isfinite(lse[1]))
    # PyTorch's SDPA also returns zeros for such rows (the reference's backend)
    ref = F.scaled_dot_product_attention(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v),
                                         attn_mask=torch.from_numpy(mask)[:, None, None, :])
    assert np.allclose(out, ref.numpy(), atol=1e-12)


def test_gqa_equals_repeated_heads(rng):
    q, k, v = _qkv(rng, B=1, H=4, Hk=2, Lq=5, Lk=7, D=8)
    out, lse = R.attention_f64(q, k, v)
    out2, lse2 = R.attention_f64(q, np.repeat(k, 2, axis=1), np.repeat(v, 2, axis=1))
    assert np.array_equal(out, out2) and np.array_equal(lse, lse2)


# ---------------------------------------------------------------------------
# Backward (flash backward with recompute; torch/.../_attention.py:567-575)
# ---------------------------------------------------------------------------


def _torch_grads(q, k, v, do, mask=None, gqa=False):
    tq, tk, tv = (torch.from_numpy(x).requires_grad_(True) for x in (q, k, v))
    m = None if mask is None else torch.from_numpy(mask)[:, None, None, :]
    o = F.scaled_dot_product_attention(tq, tk, tv, attn_mask=m, enable_gqa=gqa)
    o.backward(torch.from_numpy(do))
    return tq.grad.numpy(), tk.grad.numpy(), tv.grad.numpy()


def test_backward_matches_torch_autograd_float64(rng):
    q, k, v = _qkv(rng)
    mask = rng.random((2, 13)) > 0.4
    mask[:, 3] = True
    do = rng.standard_normal(q.shape)
    out, lse = R.attention_f64(q, k, v, mask)
    dq, dk, dv = R.attention_bwd_f64(do, q, k, v, out, lse, mask)
    rq, rk, rv = _torch_grads(q, k, v, do, mask)
    for a, b in ((dq, rq), (dk, rk), (dv, rv)):
        assert np.abs(a - b).max() < 1e-11
    # masked keys get exactly zero gradient
    assert np.all(dk[:, :, :][~np.broadcast_to(mask[:, None, :], dk.shape[:3])] == 0)


def test_backward_gqa_matches_torch_autograd(rng):
    q, k, v = _qkv(rng, B=1, H=4, Hk=2, Lq=6, Lk=5, D=8)
    do = rng.standard_normal(q.shape)
    out, lse = R.attention_f64(q, k, v)
    dq, dk, dv = R.attention_bwd_f64(do, q, k, v, out, lse)
    rq, rk, rv = _torch_grads(q, k, v, do, gqa=True)
    assert np.abs(dq - rq).max() < 1e-11 and np.abs(dk - rk).max() < 1e-11 and np.abs(dv - rv).max() < 1e-11


def test_backward_finite_differences(rng):
    q, k, v = _qkv(rng, B=1, H=1, Lq=3, Lk=4, D=4)
    do = rng.standard_normal(q.shape)
    out, lse = R.attention_f64(q, k, v)
    dq, dk, dv = R.attention_bwd_f64(do, q, k, v, out, lse)
    eps = 1e-6

    def loss(q_, k_, v_):
        return float((R.attention_f64(q_, k_, v_)[0] * do).sum())

    for arr, grad, idx in ((q, dq, (0, 0, 1, 2)), (k, dk, (0, 0, 3, 0)), (v, dv, (0, 0, 2, 3))):
        plus, minus = arr.copy(), arr.copy()
        plus[idx] += eps
        minus[idx] -= eps
        args_p = [plus if a is arr else a for a in (q, k, v)]
        args_m = [minus if a is arr else a for a in (q, k, v)]
        fd = (loss(*args_p) - loss(*args_m)) / (2 * eps)
        assert abs(fd - grad[idx]) < 1e-6


# ---------------------------------------------------------------------------
# Ring merge and loops (torch/.../_attention.py:138-223, 422-478, 514-646)
# ---------------------------------------------------------------------------


def test_chunked_merged_equals_unchunked(rng):
    q, k, v = _qkv(rng, B=1, H=2, Lq=6, Lk=20, D=8)
    mask = rng.random((1, 20)) > 0.3
    mask[0, :5] = False  # first chunk fully masked for every row
    mask[0, 7] = True
    keys = [k[:, :, i:i + 5] for i in range(0, 20, 5)]
    vals = [v[:, :, i:i + 5] for i in range(0, 20, 5)]
    masks = [mask[:, i:i + 5] for i in range(0, 20, 5)]
    out, lse = R.ring_forward_f64(q, keys, vals, masks)
    ref_out, ref_lse = R.attention_f64(q, k, v, mask)
    assert np.abs(out - ref_out).max() < 1e-13 and np.abs(lse - ref_lse).max() < 1e-13
    do = rng.standard_normal(q.shape)
    dq, dks, dvs = R.ring_backward_f64(do, q, keys, vals, out, lse, masks)
    rq, rk, rv = R.attention_bwd_f64(do, q, k, v, ref_out, ref_lse, mask)
    assert np.abs(dq - rq).max() < 1e-12
    assert np.abs(np.concatenate(dks, 2) - rk).max() < 1e-12
    assert np.abs(np.concatenate(dvs, 2) - rv).max() < 1e-12


def test_merge_f32_matches_torch_formula_and_exact_merge(rng):
    out = rng.standard_normal((2, 3, 4, 8)).astype(np.float32)
    out_b = rng.standard_normal((2, 3, 4, 8)).astype(np.float32)
    lse = (rng.standard_normal((2, 3, 4)) * 5).astype(np.float32)
    lse_b = (rng.standard_normal((2, 3, 4)) * 5).astype(np.float32)
    mo, ml = R.lse_merge_f32(out, lse, out_b, lse_b)
    to, tl = T.merge(torch.from_numpy(out), torch.from_numpy(lse), torch.from_numpy(out_b), torch.from_numpy(lse_b))
    assert np.allclose(mo, to.numpy(), atol=2e-6) and np.allclose(ml, tl.numpy(), atol=2e-6)
    eo, el = R.lse_merge_f64(out, lse, out_b, lse_b)
    assert np.allclose(mo, eo, atol=1e-5) and np.allclose(ml, el, atol=1e-5)


def test_merge_neg_inf_is_identity(rng):
    out = rng.standard_normal((3, 8)).astype(np.float32)
    out_b = rng.standard_normal((3, 8)).astype(np.float32)
    lse = np.array([-np.inf, 1.0, -np.inf], np.float32)
    lse_b = np.array([2.0, -np.inf, -np.inf], np.float32)
    mo, ml = R.lse_merge_f32(out, lse, out_b, lse_b)
    assert np.array_equal(mo[0], out_b[0]) and ml[0] == 2.0
    assert np.array_equal(mo[1], out[1]) and ml[1] == 1.0
    assert np.array_equal(mo[2], out[2]) and np.isneginf(ml[2])
    to, tl = T.merge(torch.from_numpy(out), torch.from_numpy(lse), torch.from_numpy(out_b), torch.from_numpy(lse_b))
    assert np.array_equal(to.numpy(), mo) and np.array_equal(tl.numpy(), ml)


def _sdpa_math(q, k, v, mask=None):
    from torch.nn.attention import SDPBackend, sdpa_kernel

    with sdpa_kernel([SDPBackend.MATH]):
        return F.scaled_dot_product_attention(q, k, v, attn_mask=mask)


def test_non_finite_scores_propagate_like_sdpa(rng):
    """A NaN (or +inf) score makes its row NaN in out and lse, as torch's math
    SDPA (out) and its CPU flash op (lse) give; a -inf score only drops its key;
    a NaN at a masked key still poisons the row (the mask is an additive bias)."""
    q, k, v = _qkv(rng, B=1, H=2, Lq=6, Lk=7, D=8)
    cases = []
    kn = k.copy()
    kn[0, 1, 3, 2] = np.nan  # every row of head 1 sees a NaN score
    cases.append(("nan key", q, kn, None))
    ki = k.copy()
    ki[0, 0, 4, 5] = np.inf  # +inf where q[.., 5] > 0, -inf (key dropped) where < 0
    cases.append(("inf key", q, ki, None))
    qn = q.copy()
    qn[0, 0, 2, 0] = np.nan  # one query row
    cases.append(("nan query row", qn, k, None))
    mask = np.ones((1, 7), bool)
    mask[0, 3] = False
    cases.append(("nan at a masked key", q, kn, mask))
    for name, qq, kk, m in cases:
        out, lse = R.attention_f64(qq, kk, v, m)
        tq, tk, tv = (torch.from_numpy(x) for x in (qq, kk, v))
        tm = None if m is None else torch.from_numpy(m)[:, None, None, :]
        ref = _sdpa_math(tq, tk, tv, tm).numpy()
        assert np.array_equal(np.isnan(out), np.isnan(ref)), name
        fin = ~np.isnan(ref)
        assert np.abs(out[fin] - ref[fin]).max() < 1e-12, name
        assert np.array_equal(np.isnan(lse), np.isnan(out).any(-1)), name
        if name in ("nan key", "inf key"):
            # torch's CPU flash op agrees on which rows have a NaN LSE and on
            # the finite ones (its all-NaN-row case returns 0s, so it is not
            # used for the query-row case).
            _, tl = torch.ops.aten._scaled_dot_product_flash_attention_for_cpu(tq.float(), tk.float(), tv.float())[:2]
            tl = tl.numpy()
            assert np.array_equal(np.isnan(lse), np.isnan(tl)), name
            assert np.abs(lse[~np.isnan(lse)] - tl[~np.isnan(tl)]).max() < 1e-5, name
    out, lse = R.attention_f64(q, ki, v)
    neg = q[0, 0, :, 5] < 0
    assert neg.any() and (~neg).any()
    assert np.isfinite(out[0, 0, neg]).all() and np.isnan(out[0, 0, ~neg]).all()
    # a dropped (-inf) key equals deleting it
    keep = [j for j in range(7) if j != 4]
    ro, rl = R.attention_f64(q[:, :, neg], k[:, :, keep], v[:, :, keep])
    assert np.abs(out[:, 0:1, neg] - ro[:, 0:1]).max() < 1e-12
    # a row with no valid key is still zeros / -inf, not NaN
    none = np.zeros((1, 7), bool)
    out, lse = R.attention_f64(q, k, v, none)
    assert (out == 0).all() and np.isneginf(lse).all()


def test_merge_propagates_nan_but_not_neg_inf(rng):
    """The merge treats only -inf as the identity: a NaN chunk LSE (or
    accumulator) stays NaN, as the torch formula (:182-183) computes it, so a
    ring cannot drop a chunk whose scores held a NaN."""
    out = rng.standard_normal((3, 8)).astype(np.float32)
    out_b = rng.standard_normal((3, 8)).astype(np.float32)
    lse = np.array([1.0, np.nan, np.nan], np.float32)
    lse_b = np.array([np.nan, 2.0, -np.inf], np.float32)
    out_b[0] = np.nan
    mo, ml = R.lse_merge_f32(out, lse, out_b, lse_b)
    assert np.isnan(ml).all()
    assert np.isnan(mo[0]).all() and np.isnan(mo[1]).all()
    assert np.array_equal(mo[2], out[2])  # a -inf block keeps the (NaN-LSE) accumulator's values
    to, tl = T.merge(torch.from_numpy(out), torch.from_numpy(lse), torch.from_numpy(out_b), torch.from_numpy(lse_b))
    assert np.array_equal(np.isnan(to.numpy()), np.isnan(mo)) and np.isnan(tl.numpy()).all()
    # a 4-chunk ring with a NaN in one key row of chunk 2 returns NaN rows,
    # where dropping the chunk would have given a finite answer
    q, k, v = _qkv(rng, B=1, H=1, Lq=5, Lk=16, D=8)
    k[0, 0, 9] = np.nan
    keys = [k[:, :, 4 * i:4 * i + 4] for i in range(4)]
    values = [v[:, :, 4 * i:4 * i + 4] for i in range(4)]
    ro, rl = R.ring_forward_f64(q, keys, values)
    assert np.isnan(ro).all() and np.isnan(rl).all()
    uo, _ = R.attention_f64(q, k, v)
    assert np.isnan(uo).all()
    to, tl = T.ring_forward(*(torch.from_numpy(x) for x in (q,)), [torch.from_numpy(x) for x in keys],
                            [torch.from_numpy(x) for x in values])
    assert torch.isnan(to).all() and torch.isnan(tl).all()


def test_merge_is_associative_and_commutative(rng):
    parts = [(rng.standard_normal((4, 8)), rng.standard_normal(4) * 3) for _ in range(3)]
    (a, la), (b, lb), (c, lc) = parts
    ab, lab = R.lse_merge_f64(a, la, b, lb)
    left, lleft = R.lse_merge_f64(ab, lab, c, lc)
    bc, lbc = R.lse_merge_f64(b, lb, c, lc)
    right, lright = R.lse_merge_f64(a, la, bc, lbc)
    assert np.allclose(left, right) and np.allclose(lleft, lright)
    ba, lba = R.lse_merge_f64(b, lb, a, la)
    assert np.allclose(ab, ba) and np.allclose(lab, lba)


def test_torch_ring_restatement_matches_oracle(rng):
    q = torch.randn(1, 2, 8, 16)
    k = torch.randn(1, 2, 24, 16)
    v = torch.randn(1, 2, 24, 16)
    mask = torch.rand(1, 24) > 0.3
    mask[0, 0] = True
    keys = list(k.split(6, dim=2))
    vals = list(v.split(6, dim=2))
    masks = list(mask.split(6, dim=1))
    out, lse = T.ring_forward(q, keys, vals, masks)
    ref_out, ref_lse = R.attention_f64(q.numpy(), k.numpy(), v.numpy(), mask.numpy())
    assert np.abs(out.numpy() - ref_out).max() < 1e-5 and np.abs(lse.numpy() - ref_lse).max() < 1e-5
    do = torch.randn_like(q)
    dq, dks, dvs = T.ring_backward(do, q, keys, vals, out, lse, masks)
    rq, rk, rv = R.attention_bwd_f64(do.numpy(), q.numpy(), k.numpy(), v.numpy(), ref_out, ref_lse, mask.numpy())
    assert np.abs(dq.numpy() - rq).max() < 1e-4
    assert np.abs(torch.cat(dks, 2).numpy() - rk).max() < 1e-4
    assert np.abs(torch.cat(dvs, 2).numpy() - rv).max() < 1e-4


# ---------------------------------------------------------------------------
# Shard rules (src/avgen/parallel/context.py) and FLOP convention
# ---------------------------------------------------------------------------


def test_shard_rules_follow_reference_tests():
    # tests/test_parallel.py:122-148 of the reference
    assert R.sharded_length(64, 8) == 8
    with pytest.raises(ValueError, match="not divisible"):
        R.sharded_length(65, 8)
    toks = np.arange(16, dtype=np.float32).reshape(1, 16, 1)
    seen = [toks[0, slice(*R.shard_bounds(16, 4, r)), 0].tolist() for r in range(4)]
    assert seen[0] == [0.0, 1.0, 2.0, 3.0] and seen[3] == [12.0, 13.0, 14.0, 15.0]
    t, c, m = R.pad_to_multiple(np.ones((1, 10, 2)), np.ones((1, 10, 3), np.float32), np.ones((1, 10), bool), 4)
    assert t.shape[1] == 12 and m[0, 10:].tolist() == [False, False] and m[0, :10].all()
    assert np.all(c[0, 10:] == 0) and np.all(t[0, 10:] == 0)
    # c3 shard boundary falls mid-frame: 75,600 / 4 = 18,900 = 5.25 frames of 3,600
    assert R.sharded_length(21 * 45 * 80, 4) == 18900


def test_flop_convention_matches_baseline_table():
    assert R.attention_flops(1, 4, 1024, 1024, 64, backward=False) == pytest.approx(1.07e9, rel=5e-3)
    assert R.attention_flops(2, 20, 16384, 16384, 128) == pytest.approx(1.65e13, rel=5e-3)
    assert R.attention_flops(1, 40, 18900, 75600, 128) == pytest.approx(8.78e13, rel=5e-3)
    assert R.attention_flops(2, 40, 75600, 75600, 128, backward=False) == pytest.approx(2.34e14, rel=5e-3)


def test_key_padding_mask_semantics():
    # tests/test_gpu_distributed.py:135-145 of the reference, on the CPU
    full = np.ones((2, 128), bool)
    assert R.key_padding_mask(full) is None
    ragged = full.copy()
    ragged[0, -1] = False
    m = R.key_padding_mask(ragged)
    assert m is not None and m.shape == (2, 1, 1, 128)
    assert R.key_padding_mask(ragged, assume_dense=True) is None
    with pytest.raises(ValueError):
        R.key_padding_mask(np.ones((2, 1, 128), bool))
    with pytest.raises(TypeError):
        R.key_padding_mask(np.ones((2, 128), np.int32))


# ---------------------------------------------------------------------------
# fp8 (e4m3) q k^T variant
# ---------------------------------------------------------------------------


def _e4m3_finite_values() -> torch.Tensor:
    vals = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float()
    return torch.sort(vals[torch.isfinite(vals)].unique()).values


def test_e4m3_round_matches_torch_cast(rng):
    """Bit for bit against torch's float8_e4m3fn cast: every finite value, every
    midpoint (ties), points just off the midpoints, subnormals, random values
    over many binades, the overflow edge."""
    fin = _e4m3_finite_values()
    assert fin.numel() == 253  # 254 finite codes, +0 and -0 equal
    mids = (fin[1:] + fin[:-1]) / 2
    off = (mids[:, None] * torch.tensor([1 - 2**-20, 1 + 2**-20])).flatten()
    rand = torch.from_numpy(rng.standard_normal(20000).astype(np.float32)) * torch.from_numpy(
        np.exp2(rng.integers(-14, 9, 20000)).astype(np.float32))
    edge = torch.tensor([448.0, 463.99, 464.0, 464.01, 465.0, 1e30, float("inf"), -0.0, 0.0, 2.0**-10,
                         3 * 2.0**-10, 2.0**-9 * 0.5000001, float("nan")])
    x = torch.cat([fin, -fin, mids, -mids, off, rand, edge])
    ref = x.to(torch.float8_e4m3fn).float().numpy()
    got = R.e4m3_round(x.numpy())
    same = (got == ref) | (np.isnan(got) & np.isnan(ref))
    assert same.all(), x.numpy()[~same][:10]
    assert np.array_equal(np.signbit(got[~np.isnan(got)]), np.signbit(ref[~np.isnan(ref)]))


def test_e4m3_round_closed_forms():
    """Values fixed by the format definition (bias 7, 3 mantissa bits)."""
    r = lambda v: float(R.e4m3_round(np.array([v], np.float32))[0])
    assert r(448.0) == 448.0 and r(-448.0) == -448.0
    assert r(2.0**-9) == 2.0**-9  # smallest subnormal
    assert r(2.0**-6) == 2.0**-6  # smallest normal
    assert r(2.0**-10) == 0.0  # tie between 0 and 2**-9 -> even (0)
    assert r(3 * 2.0**-10) == 2.0**-8  # tie between 1 and 2 steps -> even (2)
    assert r(1.0625) == 1.0 and r(1.1875) == 1.25  # ties in [1, 2): steps of 1/8
    assert r(240.0) == 240.0 and r(232.0) == 224.0  # [128, 256): steps of 16, tie -> even
    assert math.isnan(r(465.0)) and r(464.0) == 448.0
    # every representable value is a fixed point
    fin = _e4m3_finite_values().numpy()
    assert np.array_equal(R.e4m3_round(fin), fin)


def test_fp8_absmax_scale_and_quantize(rng):
    x = rng.standard_normal((2, 3, 17, 8)).astype(np.float32)
    x[:, 1] = 0.0  # all-zero head -> scale 1
    x[1, 2, 5, 3] = -7.5  # head 2's absmax, negative, in batch 1
    x[:, 2] = np.clip(x[:, 2], -7.0, 7.0)
    x[1, 2, 5, 3] = -7.5
    s = R.fp8_absmax_scale(x)
    assert s.dtype == np.float32 and s.shape == (3,)
    assert s[1] == np.float32(1.0)
    assert s[2] == np.float32(7.5) / np.float32(448.0)
    assert s[0] == np.float32(np.abs(x[:, 0]).max()) / np.float32(448.0)
    q8 = R.fp8_quantize(x, s)
    # the absmax element lands exactly on -448; everything stays finite and in range
    assert q8[1, 2, 5, 3] == -448.0
    assert np.isfinite(q8).all() and np.abs(q8).max() <= 448.0
    # quantized values are e4m3 values within half a step of x / scale
    y = x * (np.float32(1) / s)[None, :, None, None]
    assert np.array_equal(R.e4m3_round(q8), q8)
    assert (np.abs(q8 - y) <= np.maximum(np.abs(y) * 2.0**-4, 2.0**-10) + 1e-12).all()


def _pow2_scale(e):
    """A float32 softmax scale whose float32 product with log2(e) is 2**e."""
    s = np.float32(2.0**e / np.log2(np.e))
    assert np.float32(s * R.LOG2E_F32) == np.float32(2.0**e)
    return float(s)


def test_fp8_q_operand_closed_forms(rng):
    """q's operand: its block exponent is the smallest power of two covering
    g * q_scale (so the absmax element lands in (224, 448]), and q8 * 2**eq / g
    is q to within half an e4m3 step; GQA picks each q head's kv scale."""
    q = rng.standard_normal((2, 4, 33, 16)).astype(np.float32) * 3
    qs = R.fp8_absmax_scale(q)
    ks = np.array([0.37, 5.1], np.float32)  # kv heads: q heads 0,1 -> 0; 2,3 -> 1
    scale = 0.125
    q8, eq = R.fp8_q_operand(q, qs, ks, scale)
    g = (np.float32(np.float32(scale) * R.LOG2E_F32) * ks[[0, 0, 1, 1]]).astype(np.float32)
    t = (g * qs).astype(np.float32).astype(np.float64)
    assert np.all(np.ldexp(1.0, eq) >= t) and np.all(np.ldexp(1.0, eq - 1) < t)
    amax = np.abs(q8).max(axis=(0, 2, 3))
    assert np.all(amax <= 448.0) and np.all(amax > 224.0)
    assert np.array_equal(R.e4m3_round(q8), q8)
    y = q.astype(np.float64) * (g.astype(np.float64) * np.ldexp(1.0, -eq))[None, :, None, None]
    assert (np.abs(q8 - y) <= np.maximum(np.abs(y) * 2.0**-4, 2.0**-10) * (1 + 1e-6)).all()


def test_attention_fp8_reduces_to_bf16_attention(rng):
    """With e4m3-representable q, k, unit scales and a softmax scale whose
    log2(e) product is a power of two, the fp8 operands are q and k
    themselves and the fp8 variant is plain attention; scaling q (or k) and
    its scale by the same power of two gives plain attention of the scaled
    operands (quantization commutes with powers of two in range)."""
    fin = _e4m3_finite_values().numpy()
    small = fin[(np.abs(fin) <= 2.0) & (np.abs(fin) >= 2.0**-3)]
    q = rng.choice(small, size=(1, 2, 9, 16)).astype(np.float32)
    k = rng.choice(small, size=(1, 1, 11, 16)).astype(np.float32)
    v = rng.standard_normal((1, 1, 11, 16)).astype(np.float32)
    mask = np.ones((1, 11), bool)
    mask[0, 3] = False
    one_q, one_k = np.ones(2, np.float32), np.ones(1, np.float32)
    sc = _pow2_scale(-3)
    q8, eq = R.fp8_q_operand(q, one_q, one_k, sc)
    assert np.array_equal(q8, q) and np.array_equal(eq, [-3, -3])
    o8, l8 = R.attention_fp8_f64(q, k, v, one_q, one_k, mask, scale=sc)
    o, l = R.attention_f64(q, k, v, mask, scale=sc)
    np.testing.assert_allclose(o8, o, rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(l8, l, rtol=1e-6, atol=1e-9)
    # q * 8 with scale 8, k / 4 with scale 1/4: the same e4m3 operands, and
    # plain attention of the scaled operands
    o8b, l8b = R.attention_fp8_f64(q * 8, k / 4, v, one_q * 8, one_k / 4, mask, scale=sc)
    ob, lb = R.attention_f64(q * 8, k / 4, v, mask, scale=sc)
    np.testing.assert_allclose(o8b, ob, rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(l8b, lb, rtol=1e-6, atol=1e-9)
    # a softmax scale that is no power of two rounds q: off plain attention
    o8c, _ = R.attention_fp8_f64(q, k, v, one_q, one_k, mask, scale=sc * 1.03)
    oc, _ = R.attention_f64(q, k, v, mask, scale=sc * 1.03)
    assert not np.allclose(o8c, oc, rtol=0, atol=1e-9)
    # and an unquantized q is rounded the same way
    o8d, _ = R.attention_fp8_f64(q * 1.03, k, v, one_q, one_k, mask, scale=sc)
    od, _ = R.attention_f64(q * 1.03, k, v, mask, scale=sc)
    assert not np.allclose(o8d, od, rtol=0, atol=1e-9)

def test_backward_magnitudes_bound_the_gradients():
    """attention_bwd_magnitudes_f64 is the dq/dk formula with every factor of
    dS in absolute value: by the triangle inequality it bounds |dq| and |dk|
    elementwise (GQA included); with a single key dS cancels (dP == Dr),
    the gradients vanish to float64 rounding while the magnitudes do not."""
    rng = np.random.default_rng(11)
    q, do = rng.standard_normal((2, 4, 9, 16)), rng.standard_normal((2, 4, 9, 16))
    k, v = rng.standard_normal((2, 2, 13, 16)), rng.standard_normal((2, 2, 13, 16))
    mask = rng.random((2, 13)) < 0.7
    o, l = R.attention_f64(q, k, v, mask)
    dq, dk, _ = R.attention_bwd_f64(do, q, k, v, o, l, mask)
    mq, mk = R.attention_bwd_magnitudes_f64(do, q, k, v, o, l, mask)
    assert mq.shape == dq.shape and mk.shape == dk.shape
    assert np.all(np.abs(dq) <= mq * (1 + 1e-12)) and np.all(np.abs(dk) <= mk * (1 + 1e-12))
    assert mq.max() > 0 and mk.max() > 0
    k1, v1 = k[:, :, :1] * 4, v[:, :, :1] * 4
    o, l = R.attention_f64(q * 4, k1, v1)
    dq, dk, _ = R.attention_bwd_f64(do, q * 4, k1, v1, o, l)
    mq, mk = R.attention_bwd_magnitudes_f64(do, q * 4, k1, v1, o, l)
    assert np.abs(dq).max() <= 1e-12 * mq.max() and np.abs(dk).max() <= 1e-12 * mk.max()
    assert mq.max() > 1.0
