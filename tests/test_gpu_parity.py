"""GPU parity of the HIP kernels (through the C ABI) against the CPU oracle.

Tolerances: output max-abs <= 2e-2 and LSE <= 1e-3 for
bf16 inputs against a float64 evaluation of the same bf16 values; masks and
padding bit-exact (masked keys contribute exactly nothing: identical output
bits when masked K/V change, exactly zero dK/dV).  The RoPE rotation is
bit-exact against the reference's float32 chain.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reference as R
from oracle import torch_path as T

pytestmark = pytest.mark.gpu

OUT_TOL = 2e-2
LSE_TOL = 1e-3
# Gradients: max-abs error relative to the largest reference magnitude.
GRAD_REL_TOL = 2e-2


@pytest.fixture(scope="module")
def amd():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    import avgen_amd

    avgen_amd.ops  # noqa: B018 — loads the library lazily on first call
    return avgen_amd


def _gen(seed):
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def _randn(shape, seed, scale=1.0):
    return (torch.randn(shape, generator=_gen(seed)) * scale).to(torch.bfloat16)


def _f64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _key_mask(B, Lk, seed, full_rows=(), empty_rows=()):
    g = _gen(seed)
    lengths = torch.randint(1, Lk + 1, (B,), generator=g)
    m = torch.arange(Lk)[None, :] < lengths[:, None]
    for b in full_rows:
        m[b] = True
    for b in empty_rows:
        m[b] = False
    return m


FWD_CASES = [
    # B, Hq, Hkv, Lq, Lk, D
    (1, 2, 2, 128, 128, 128),
    (2, 3, 3, 200, 333, 128),
    (1, 4, 4, 1024, 1024, 64),
    (1, 4, 2, 130, 257, 128),
    (2, 2, 1, 65, 64, 64),
    (1, 1, 1, 1, 1, 128),
    (1, 2, 2, 300, 5, 128),
]


@pytest.mark.parametrize("B,Hq,Hkv,Lq,Lk,D", FWD_CASES)
@pytest.mark.parametrize("masked", [False, True])
def test_forward_matches_oracle(amd, B, Hq, Hkv, Lq, Lk, D, masked):
    q = _randn((B, Hq, Lq, D), 0)
    k = _randn((B, Hkv, Lk, D), 1)
    v = _randn((B, Hkv, Lk, D), 2)
    mask = _key_mask(B, Lk, 4, empty_rows=(0,) if (masked and B > 1) else ()) if masked else None
    print(f"fwd case B={B} Hq={Hq} Hkv={Hkv} Lq={Lq} Lk={Lk} D={D} masked={masked}", flush=True)
    out, lse = amd.ops.flash_fwd(q.cuda(), k.cuda(), v.cuda(), None if mask is None else mask.cuda(), None, None,
                                 D ** -0.5)
    ro, rl = R.attention_f64(_f64(q), _f64(k), _f64(v), None if mask is None else mask.numpy())
    o = _f64(out)
    l = lse.cpu().numpy().astype(np.float64)
    assert np.isfinite(o).all()
    assert np.abs(o - ro).max() <= OUT_TOL
    fin = np.isfinite(rl)
    assert np.array_equal(np.isneginf(l), ~fin)
    assert np.abs(l[fin] - rl[fin]).max(initial=0.0) <= LSE_TOL
    if masked and B > 1:
        assert np.all(o[0] == 0)


def test_forward_score_bound_paths(amd):
    """The forward stops tracking row maxima once |q_row| * max|k| certifies
    that no later score can grow a probability past 2^32; rows whose bound is
    loose (large-norm queries nearly orthogonal to every key) keep the exact
    path, and a late dominant key must still move the reference max.  Both
    regimes in one launch match float64."""
    B, H, Lq, Lk, D = 1, 2, 300, 700, 128
    q = _randn((B, H, Lq, D), 80).float()
    k = _randn((B, H, Lk, D), 81).float()
    v = _randn((B, H, Lk, D), 82)
    q[:, :, 40:72] = 0.0
    q[:, :, 40:72, 0] = 60.0  # huge norm, scores ~ 60 * k[..., 0]: loose bound
    k[:, :, :, 0] *= 0.05
    k[:, :, 650] *= 6.0  # a late key that dominates its rows
    q, k = q.to(torch.bfloat16), k.to(torch.bfloat16)
    out, lse = amd.ops.flash_fwd(q.cuda(), k.cuda(), v.cuda(), None, None, None, D ** -0.5)
    ro, rl = R.attention_f64(_f64(q), _f64(k), _f64(v))
    assert np.abs(_f64(out) - ro).max() <= OUT_TOL
    assert np.abs(lse.cpu().numpy() - rl).max() <= LSE_TOL


def test_max_raised_by_the_second_half_of_a_tile(amd):
    """The forward processes a 64-key tile as two 32-key halves; when the
    second half holds a key that raises a row's maximum far (here by tens of
    log2 units) above the first half's, both halves' probabilities must still
    enter P V against the same reference: in the first tile and in a later
    one, on the plain, windowed and fp8 forwards."""
    B, H, Lq, Lk, D = 1, 2, 96, 700, 128
    q = _randn((B, H, Lq, D), 90, 0.7).float()
    k = _randn((B, H, Lk, D), 91, 0.7).float()
    v = _randn((B, H, Lk, D), 92)
    k[:, :, 40] = q[:, :, 0] * 4.0     # tile 0, second half: dominates row 0
    k[:, :, 370] = q[:, :, 40] * 4.0   # tile 5, second half: dominates row 40
    k[:, :, 690] = q[:, :, 70] * 2.0   # tile 10, second half
    q, k = q.to(torch.bfloat16), k.to(torch.bfloat16)
    qc, kc, vc = q.cuda(), k.cuda(), v.cuda()
    ro, rl = R.attention_f64(_f64(q), _f64(k), _f64(v))
    outs = {"plain": amd.ops.flash_fwd(qc, kc, vc, None, None, None, D ** -0.5)}
    lo = torch.zeros(Lq, dtype=torch.int32, device="cuda")
    hi = torch.full((Lq,), Lk, dtype=torch.int32, device="cuda")
    outs["windowed"] = amd.ops.flash_fwd_windowed(qc, kc, vc, lo, hi, None, D ** -0.5)
    for name, (out, lse) in outs.items():
        print(f"second-half max {name}", flush=True)
        assert np.abs(_f64(out) - ro).max() <= OUT_TOL, name
        assert np.abs(lse.cpu().numpy() - rl).max() <= LSE_TOL, name
    qs, ks = R.fp8_absmax_scale(_f64(q)), R.fp8_absmax_scale(_f64(k))
    out8, lse8 = amd.ops.flash_fwd_fp8(qc, kc, vc, None, torch.from_numpy(qs).cuda(), torch.from_numpy(ks).cuda(),
                                       D ** -0.5)
    r8, l8 = R.attention_fp8_f64(_f64(q), _f64(k), _f64(v), qs, ks)
    assert np.abs(_f64(out8) - r8).max() <= OUT_TOL
    assert (np.abs(lse8.cpu().numpy() - l8) <= LSE_TOL + 2.0 ** -14 * np.abs(l8)).all()


def test_attention_dropin_matches_torch_restatement(amd):
    q, k, v = _randn((1, 4, 256, 128), 10), _randn((1, 4, 384, 128), 11), _randn((1, 4, 384, 128), 12)
    out = amd.attention.attention(q.cuda(), k.cuda(), v.cuda())
    ref = T.sdpa(q.float(), k.float(), v.float()).numpy()
    assert np.abs(_f64(out) - ref).max() <= OUT_TOL
    # key-padding mask path with key_padding_mask's (B,1,1,Lk) form
    m = _key_mask(1, 384, 3)
    km = amd.attention.key_padding_mask(m.cuda())
    out_m = amd.attention.attention(q.cuda(), k.cuda(), v.cuda(), attn_mask=km)
    ref_m = T.sdpa(q.float(), k.float(), v.float(), m).numpy()
    assert np.abs(_f64(out_m) - ref_m).max() <= OUT_TOL


def test_strided_blhd_inputs(amd):
    # (B, L, H, D) storage viewed as (B, H, L, D), as SelfAttention._heads does
    # (src/avgen/models/layers.py:496-504).
    base = _randn((2, 200, 3, 128), 20).cuda()
    kb = _randn((2, 150, 3, 128), 21).cuda()
    vb = _randn((2, 150, 3, 128), 22).cuda()
    q, k, v = base.transpose(1, 2), kb.transpose(1, 2), vb.transpose(1, 2)
    out, lse = amd.ops.flash_fwd(q, k, v, None, None, None, 128 ** -0.5)
    out_c, lse_c = amd.ops.flash_fwd(q.contiguous(), k.contiguous(), v.contiguous(), None, None, None, 128 ** -0.5)
    assert torch.equal(out.contiguous(), out_c) and torch.equal(lse, lse_c)


def test_zero_length_sequences(amd):
    q = _randn((1, 2, 16, 128), 1).cuda()
    k = _randn((1, 2, 0, 128), 2).cuda()
    out = amd.attention.attention(q, k, k)
    assert out.shape == q.shape and torch.all(out == 0)
    out2, lse2 = amd.ops.flash_fwd(q, k, k, None, None, None, 0.1)
    assert torch.all(out2 == 0) and torch.all(torch.isneginf(lse2))
    q0 = _randn((1, 2, 0, 128), 3).cuda()
    assert amd.attention.attention(q0, q, q).shape == q0.shape


def test_masked_keys_are_bit_exact(amd):
    B, H, Lq, Lk, D = 2, 2, 96, 200, 128
    q, k, v = _randn((B, H, Lq, D), 30), _randn((B, H, Lk, D), 31), _randn((B, H, Lk, D), 32)
    m = _key_mask(B, Lk, 5)
    m[1, 150:] = False
    out, lse = amd.ops.flash_fwd(q.cuda(), k.cuda(), v.cuda(), m.cuda(), None, None, D ** -0.5)
    k2, v2 = k.clone(), v.clone()
    garbage = _randn((B, H, Lk, D), 33, scale=50.0)
    sel = (~m)[:, None, :, None].expand_as(k2)
    k2[sel] = garbage[sel]
    v2[sel] = garbage[sel]
    out2, lse2 = amd.ops.flash_fwd(q.cuda(), k2.cuda(), v2.cuda(), m.cuda(), None, None, D ** -0.5)
    assert torch.equal(out, out2) and torch.equal(lse, lse2)
    do = _randn((B, H, Lq, D), 34).cuda()
    dq, dk, dv = amd.ops.flash_bwd(do, q.cuda(), k.cuda(), v.cuda(), out, lse, m.cuda(), D ** -0.5)
    dq2, dk2, dv2 = amd.ops.flash_bwd(do, q.cuda(), k2.cuda(), v2.cuda(), out2, lse2, m.cuda(), D ** -0.5)
    msk = (~m.cuda())[:, None, :, None].expand_as(dk)
    assert torch.all(dk[msk] == 0) and torch.all(dv[msk] == 0)
    assert torch.equal(dq, dq2) and torch.equal(dk[~msk], dk2[~msk]) and torch.equal(dv[~msk], dv2[~msk])


BWD_CASES = [
    (1, 2, 2, 128, 128, 128, False),
    (2, 3, 3, 200, 333, 128, True),
    (1, 4, 2, 130, 257, 128, False),
    (1, 4, 4, 512, 512, 64, False),
    (2, 2, 1, 65, 97, 64, True),
    # 2 x 141 = 282 key blocks of 128: on a 256-CU device the last 26 (the
    # ragged last block among them) are split over 8 workgroups each
    (1, 4, 2, 640, 17965, 128, True),
    # 8 x 34 = 272 dQ workgroups of 256 query rows (a partial last round)
    (1, 8, 4, 8465, 300, 64, True),
]


@pytest.mark.parametrize("B,Hq,Hkv,Lq,Lk,D,masked", BWD_CASES)
@pytest.mark.parametrize("staged", [True, False])
def test_backward_matches_oracle(amd, B, Hq, Hkv, Lq, Lk, D, masked, staged):
    """Both dQ paths: staged dS (dK/dV kernel stores dS, dQ = dS K) and the
    kernel that recomputes S and dP."""
    q, k, v = _randn((B, Hq, Lq, D), 40), _randn((B, Hkv, Lk, D), 41), _randn((B, Hkv, Lk, D), 42)
    do = _randn((B, Hq, Lq, D), 43)
    m = _key_mask(B, Lk, 6, empty_rows=(1,) if B > 1 else ()) if masked else None
    print(f"bwd case B={B} Hq={Hq} Hkv={Hkv} Lq={Lq} Lk={Lk} D={D} masked={masked} staged={staged}", flush=True)
    mc = None if m is None else m.cuda()
    out, lse = amd.ops.flash_fwd(q.cuda(), k.cuda(), v.cuda(), mc, None, None, D ** -0.5)
    dq, dk, dv = amd.ops._bwd_impl(do.cuda(), q.cuda(), k.cuda(), v.cuda(), out, lse, mc, D ** -0.5,
                                   stage_ds=staged)
    mn = None if m is None else m.numpy()
    ro, rl = R.attention_f64(_f64(q), _f64(k), _f64(v), mn)
    rq, rk, rv = R.attention_bwd_f64(_f64(do), _f64(q), _f64(k), _f64(v), ro, rl, mn)
    for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        g = _f64(got)
        assert np.isfinite(g).all(), name
        err = np.abs(g - ref).max()
        scale = max(np.abs(ref).max(), 1e-3)
        print(f"  {name}: max err {err:.3e} (ref max {scale:.3e})", flush=True)
        assert err <= GRAD_REL_TOL * scale, name


@pytest.mark.parametrize("ntiles", [1, 2, 3, 4, 5, 6, 7])
@pytest.mark.parametrize("staged", [True, False])
@pytest.mark.parametrize("D", [128, 64])
def test_backward_query_tile_counts(amd, ntiles, staged, D):
    """dK/dV's tile loop (unrolled by three, the dS waves one tile behind and
    one iteration longer) ending at every position: 1..7 query tiles of 64
    rows, the last one ragged, at both head dims (their phases have 16 and 8
    MFMA slots)."""
    Lq, Lk = 64 * ntiles - 5, 256
    q, k, v = _randn((1, 2, Lq, D), 60), _randn((1, 2, Lk, D), 61), _randn((1, 2, Lk, D), 62)
    do = _randn((1, 2, Lq, D), 63)
    print(f"tile-count case Lq={Lq} D={D} staged={staged}", flush=True)
    out, lse = amd.ops.flash_fwd(q.cuda(), k.cuda(), v.cuda(), None, None, None, D ** -0.5)
    dq, dk, dv = amd.ops._bwd_impl(do.cuda(), q.cuda(), k.cuda(), v.cuda(), out, lse, None, D ** -0.5,
                                   stage_ds=staged)
    ro, rl = R.attention_f64(_f64(q), _f64(k), _f64(v))
    rq, rk, rv = R.attention_bwd_f64(_f64(do), _f64(q), _f64(k), _f64(v), ro, rl)
    for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        err = np.abs(_f64(got) - ref).max()
        assert err <= GRAD_REL_TOL * max(np.abs(ref).max(), 1e-3), name


@pytest.mark.parametrize("Lq", [60, 100, 250])
@pytest.mark.parametrize("staged", [True, False])
def test_backward_gqa_group_of_three(amd, Lq, staged):
    """Three query heads per KV head: dK/dV's tile loop runs over the tiles of
    every head of the group, so the head changes at different positions of
    the three-slot rotation (1, 2 and 4 tiles per head)."""
    Hq, Hkv, Lk, D = 6, 2, 200, 128
    q, k, v = _randn((1, Hq, Lq, D), 70), _randn((1, Hkv, Lk, D), 71), _randn((1, Hkv, Lk, D), 72)
    do = _randn((1, Hq, Lq, D), 73)
    print(f"gqa-3 case Lq={Lq} staged={staged}", flush=True)
    out, lse = amd.ops.flash_fwd(q.cuda(), k.cuda(), v.cuda(), None, None, None, D ** -0.5)
    dq, dk, dv = amd.ops._bwd_impl(do.cuda(), q.cuda(), k.cuda(), v.cuda(), out, lse, None, D ** -0.5,
                                   stage_ds=staged)
    ro, rl = R.attention_f64(_f64(q), _f64(k), _f64(v))
    rq, rk, rv = R.attention_bwd_f64(_f64(do), _f64(q), _f64(k), _f64(v), ro, rl)
    for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        err = np.abs(_f64(got) - ref).max()
        assert err <= GRAD_REL_TOL * max(np.abs(ref).max(), 1e-3), name


def test_autograd_through_dropin(amd):
    q = _randn((1, 2, 96, 128), 50).cuda().requires_grad_(True)
    k = _randn((1, 2, 80, 128), 51).cuda().requires_grad_(True)
    v = _randn((1, 2, 80, 128), 52).cuda().requires_grad_(True)
    do = _randn((1, 2, 96, 128), 53).cuda()
    amd.attention.attention(q, k, v).backward(do)
    ro, rl = R.attention_f64(_f64(q), _f64(k), _f64(v))
    rq, rk, rv = R.attention_bwd_f64(_f64(do), _f64(q), _f64(k), _f64(v), ro, rl)
    for got, ref in ((q.grad, rq), (k.grad, rk), (v.grad, rv)):
        assert np.abs(_f64(got) - ref).max() <= GRAD_REL_TOL * np.abs(ref).max()


# ---------------------------------------------------------------------------
# RoPE
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("head_dim", [64, 128])
def test_rope_tables_match_oracle(amd, head_dim):
    coords = torch.from_numpy(R.video_coords(4, 6, 8, batch=2))
    tabs = amd.rope.build_rotary_tables(coords.cuda(), head_dim=head_dim, time_scale=1.5,
                                        scaling=amd.rope.RoPEScaling("ntk", 2.0, 1.5))
    c64, s64 = R.rotary_tables_f64(coords.numpy(), head_dim, time_scale=1.5, scaling=("ntk", 2.0, 1.5))
    ct, st = T.rotary_tables(coords, head_dim, time_scale=1.5, scaling=("ntk", 2.0, 1.5))
    c, s = tabs.cos.cpu().numpy(), tabs.sin.cpu().numpy()
    assert np.abs(c - c64).max() < 1e-5 and np.abs(s - s64).max() < 1e-5
    # same fp32 angles as the torch restatement; only cos/sin rounding differs
    assert np.abs(c - ct.numpy()).max() < 5e-7 and np.abs(s - st.numpy()).max() < 5e-7
    zero = amd.rope.build_rotary_tables(torch.zeros(1, 5, 3).cuda(), head_dim=head_dim)
    assert torch.all(zero.cos == 1) and torch.all(zero.sin == 0)


def test_rope_linear_scaling_tables(amd):
    coords = torch.from_numpy(R.video_coords(3, 4, 5))
    tabs = amd.rope.build_rotary_tables(coords.cuda(), head_dim=128, scaling=amd.rope.RoPEScaling("linear", 2.0, 3.0))
    ct, st = T.rotary_tables(coords, 128, scaling=("linear", 2.0, 3.0))
    assert np.abs(tabs.cos.cpu().numpy() - ct.numpy()).max() < 5e-7


@pytest.mark.parametrize("head_dim", [64, 128])
def test_rope_apply_bit_exact(amd, head_dim):
    coords = torch.from_numpy(R.video_coords(5, 6, 7, batch=2))
    cos, sin = T.rotary_tables(coords, head_dim)
    x = _randn((2, 3, coords.shape[1], head_dim), 60, scale=3.0)
    tabs = amd.rope.RotaryTables(cos.cuda(), sin.cuda())
    got = amd.rope.apply_rotary(x.cuda(), tabs).cpu()
    ref = T.apply_rotary(x, cos, sin)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    inv = amd.ops.rope_apply(x.cuda(), tabs.cos, tabs.sin, True).cpu().float().numpy()
    ref_inv = R.apply_rotary_bf16(x.float().numpy(), cos.numpy(), sin.numpy(), inverse=True)
    assert np.array_equal(inv.view(np.uint32), ref_inv.view(np.uint32))


def test_rope_autograd_bit_exact(amd):
    coords = torch.from_numpy(R.video_coords(2, 4, 4))
    cos, sin = T.rotary_tables(coords, 128)
    x = _randn((1, 2, 32, 128), 61)
    g = _randn((1, 2, 32, 128), 62)
    xg = x.cuda().requires_grad_(True)
    amd.rope.apply_rotary(xg, amd.rope.RotaryTables(cos.cuda(), sin.cuda())).backward(g.cuda())
    xr = x.clone().requires_grad_(True)
    T.apply_rotary(xr, cos, sin).backward(g)
    assert torch.equal(xg.grad.cpu().view(torch.int16), xr.grad.view(torch.int16))


def test_fused_rope_forward_equals_unfused(amd):
    B, H, L, D = 1, 2, 300, 128
    coords = torch.from_numpy(R.video_coords(3, 10, 10, batch=B))
    cos, sin = T.rotary_tables(coords, D)
    tabs = amd.rope.RotaryTables(cos.cuda(), sin.cuda())
    q, k, v = _randn((B, H, L, D), 70).cuda(), _randn((B, H, L, D), 71).cuda(), _randn((B, H, L, D), 72).cuda()
    fused = amd.attention.rotary_attention(q, k, v, tabs)
    qr = amd.rope.apply_rotary(q, tabs)
    kr = amd.rope.apply_rotary(k, tabs)
    unfused = amd.attention.attention(qr, kr, v)
    assert torch.equal(fused, unfused)
    # and gradients agree with the unfused composition through autograd
    qa, ka, va = (t.clone().requires_grad_(True) for t in (q, k, v))
    qb, kb, vb = (t.clone().requires_grad_(True) for t in (q, k, v))
    do = _randn((B, H, L, D), 73).cuda()
    amd.attention.rotary_attention(qa, ka, va, tabs).backward(do)
    amd.attention.attention(amd.rope.apply_rotary(qb, tabs), amd.rope.apply_rotary(kb, tabs), vb).backward(do)
    assert torch.equal(qa.grad, qb.grad) and torch.equal(ka.grad, kb.grad) and torch.equal(va.grad, vb.grad)


# ---------------------------------------------------------------------------
# Merge and emulated ring
# ---------------------------------------------------------------------------


def test_lse_merge_kernel_matches_oracle(amd):
    g = _gen(80)
    out = torch.randn(2, 3, 50, 128, generator=g)
    lse = torch.randn(2, 3, 50, generator=g) * 4
    out_b = torch.randn(2, 3, 50, 128, generator=g).to(torch.bfloat16)
    lse_b = torch.randn(2, 3, 50, generator=g) * 4
    lse[0, 0, :5] = float("-inf")
    lse_b[0, 1, :5] = float("-inf")
    lse[1, 2, :3] = float("-inf")
    lse_b[1, 2, :3] = float("-inf")
    oa, la = out.cuda(), lse.cuda()
    amd.ops.lse_merge_(oa, la, out_b.cuda(), lse_b.cuda())
    ro, rl = R.lse_merge_f32(out.numpy(), lse.numpy(), out_b.float().numpy(), lse_b.numpy())
    assert np.allclose(oa.cpu().numpy(), ro, atol=2e-6, rtol=0)
    lg = la.cpu().numpy()
    assert np.array_equal(np.isneginf(lg), np.isneginf(rl))
    fin = np.isfinite(rl)
    assert np.allclose(lg[fin], rl[fin], atol=2e-6, rtol=0)


@pytest.mark.parametrize("masked,Hkv", [(False, 3), (True, 3), (False, 1)])
def test_emulated_ring_matches_unchunked(amd, masked, Hkv):
    B, H, Lq, L, D, cp = 1, 3, 256, 1024, 128, 4
    q, k, v = _randn((B, H, Lq, D), 90), _randn((B, Hkv, L, D), 91), _randn((B, Hkv, L, D), 92)
    do = _randn((B, H, Lq, D), 93)
    m = None
    if masked:
        m = torch.ones(B, L, dtype=torch.bool)
        m[:, 700:] = False  # last chunk fully masked, third partly
    mc = None if m is None else m.cuda()
    qg, kg, vg = (t.cuda().requires_grad_(True) for t in (q, k, v))
    out, lse = amd.ring.ring_attention(qg, kg, vg, cp=cp, key_mask=mc)
    out.backward(do.cuda())
    mn = None if m is None else m.numpy()
    ro, rl = R.attention_f64(_f64(q), _f64(k), _f64(v), mn)
    assert np.abs(_f64(out) - ro).max() <= OUT_TOL
    assert np.abs(lse.cpu().numpy() - rl).max() <= LSE_TOL
    rq, rk, rv = R.attention_bwd_f64(_f64(do), _f64(q), _f64(k), _f64(v), ro, rl, mn)
    for got, ref in ((qg.grad, rq), (kg.grad, rk), (vg.grad, rv)):
        assert np.abs(_f64(got) - ref).max() <= GRAD_REL_TOL * np.abs(ref).max()


@pytest.mark.parametrize("staged", [False, True])
def test_bwd_query_side_reuse_and_dq_accumulation(amd, staged):
    """avattn_bwd flags: the query-side preparation kept in the workspace gives
    bit-identical dk/dv, and the fp32 dq accumulator equals the sum of the
    per-chunk dq up to their bf16 rounding (it adds unrounded values); with
    and without staged dS."""
    B, H, Lq, Lc, D = 1, 2, 200, 150, 128
    q, do = _randn((B, H, Lq, D), 70).cuda(), _randn((B, H, Lq, D), 71).cuda()
    ks = [_randn((B, H, Lc, D), 72 + i).cuda() for i in range(2)]
    vs = [_randn((B, H, Lc, D), 74 + i).cuda() for i in range(2)]
    kf, vf = torch.cat(ks, 2), torch.cat(vs, 2)
    out, lse = amd.ops.flash_fwd(q, kf, vf, None, None, None, D ** -0.5)
    ref = [amd.ops.flash_bwd(do, q, k, v, out, lse, None, D ** -0.5) for k, v in zip(ks, vs)]
    lib = amd._lib.load()
    size = (lib.avattn_bwd_staged_workspace_size(B, H, H, Lq, Lc, D, B * H) if staged
            else lib.avattn_bwd_workspace_size(B, H, H, Lq, Lc, D))
    ws = amd.ops._workspace(size, q.device)
    acc = torch.zeros(q.shape, dtype=torch.float32, device=q.device)
    for i, (k, v) in enumerate(zip(ks, vs)):
        _, dk, dv = amd.ops._bwd_impl(do, q, k, v, out, lse, None, D ** -0.5, workspace=ws,
                                      reuse_query_side=i > 0, dq_accumulate=acc, stage_ds=staged)
        assert torch.equal(dk, ref[i][1]) and torch.equal(dv, ref[i][2])
    summed = ref[0][0].float() + ref[1][0].float()
    assert (acc - summed).abs().max().item() <= 8e-3 * summed.abs().max().item()
    rq, _, _ = R.attention_bwd_f64(_f64(do), _f64(q), _f64(kf), _f64(vf), _f64(out),
                                   lse.cpu().numpy().astype(np.float64))
    assert np.abs(acc.cpu().numpy() - rq).max() <= GRAD_REL_TOL * np.abs(rq).max()


def test_staged_ds_in_passes_matches_recompute(amd, monkeypatch):
    """A dS budget of two (batch, kv head) pairs: the backward runs in three
    passes; dk/dv are bit-identical to the recomputing path (same dK/dV
    kernel arithmetic) and dq agrees to rounding; masked keys stay exact."""
    B, Hq, Hkv, Lq, Lk, D = 2, 6, 3, 200, 333, 128
    q, k, v = _randn((B, Hq, Lq, D), 80).cuda(), _randn((B, Hkv, Lk, D), 81).cuda(), _randn((B, Hkv, Lk, D), 82).cuda()
    do = _randn((B, Hq, Lq, D), 83).cuda()
    m = _key_mask(B, Lk, 7).cuda()
    per = amd.ops.ds_bytes_per_pair(Hq // Hkv, Lq, Lk)
    out, lse = amd.ops.flash_fwd(q, k, v, m, None, None, D ** -0.5)
    ref = amd.ops._bwd_impl(do, q, k, v, out, lse, m, D ** -0.5, stage_ds=False)
    amd.ops.set_ds_budget(int(2.5 * per), q.device)
    try:
        nbytes, staged = amd.ops.bwd_workspace_plan(B, Hq, Hkv, Lq, Lk, D, q.device)
        lib = amd._lib.load()
        assert staged and nbytes == lib.avattn_bwd_staged_workspace_size(B, Hq, Hkv, Lq, Lk, D, 2)
        print(f"staged passes: {per} bytes per pair, workspace {nbytes}", flush=True)
        got = amd.ops._bwd_impl(do, q, k, v, out, lse, m, D ** -0.5)
    finally:
        amd.ops.set_ds_budget(None, q.device)
    assert torch.equal(got[1], ref[1]) and torch.equal(got[2], ref[2])
    err = (got[0].float() - ref[0].float()).abs().max().item()
    assert err <= 1e-2 * ref[0].float().abs().max().item(), err
    rq, _, _ = R.attention_bwd_f64(_f64(do), _f64(q), _f64(k), _f64(v), _f64(out),
                                   lse.cpu().numpy().astype(np.float64), m.cpu().numpy())
    assert np.abs(_f64(got[0]) - rq).max() <= GRAD_REL_TOL * np.abs(rq).max()


def test_tail_split_changes_only_the_split_blocks(amd):
    """dk/dv bits depend on the dK/dV grid's tail split, i.e. on the device's
    CU count and on how the (batch, kv head) pairs are split into passes: a
    pass whose 128-key blocks exceed one round of CUs gives its last
    ``total % cus`` blocks to several workgroups, whose fp32 partial sums add
    in another order.  Here 3 pairs x 100 blocks: one pass (300 blocks, split
    tail) against three passes of 100 blocks (no split).  Keys outside the
    split blocks are bit-identical; the split blocks agree to fp32
    reassociation (then one bf16 rounding)."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    B, H, Lq, D = 1, 3, 512, 128
    nkt = 100
    Lk = 128 * nkt
    if H * nkt <= cus:
        pytest.skip(f"{cus} CUs: 300 blocks fit one round, no tail split")
    q, k, v = _randn((B, H, Lq, D), 84).cuda(), _randn((B, H, Lk, D), 85).cuda(), _randn((B, H, Lk, D), 86).cuda()
    do = _randn((B, H, Lq, D), 87).cuda()
    out, lse = amd.ops.flash_fwd(q, k, v, None, None, None, D ** -0.5)
    per = amd.ops.ds_bytes_per_pair(1, Lq, Lk)
    results = []
    for budget in (H * per, per):  # one pass of 300 blocks; three of 100
        amd.ops.set_ds_budget(budget, q.device)
        try:
            results.append(amd.ops._bwd_impl(do, q, k, v, out, lse, None, D ** -0.5))
        finally:
            amd.ops.set_ds_budget(None, q.device)
    torch.cuda.synchronize()
    (dq1, dk1, dv1), (dq3, dk3, dv3) = results
    total = H * nkt
    first_split = total - total % cus  # flat (pair, block) index of the first split block
    split_keys = torch.zeros(B, H, Lk, dtype=torch.bool, device="cuda")
    for flat in range(first_split, total):
        split_keys[0, flat // nkt, 128 * (flat % nkt):128 * (flat % nkt + 1)] = True
    for a_, b_ in ((dk1, dk3), (dv1, dv3)):
        differs = (a_ != b_).any(-1)
        assert not (differs & ~split_keys).any()
        rel = ((a_.float() - b_.float()).abs().max() / b_.float().abs().max()).item()
        assert rel <= 4e-3, rel
    print(f"{cus} CUs: {int(split_keys.sum())} keys in split blocks, "
          f"{int((dk1 != dk3).any(-1).sum())} dk rows differ", flush=True)
    assert torch.equal(dq1, dq3)  # dq does not depend on the split


@pytest.mark.parametrize("masked", [False, True])
def test_ring_backward_overlapped_dq_is_identical(amd, masked):
    """The ring backward with each chunk's dq on a side stream (two
    alternating workspaces, deferred dq) gives the same bits as the
    sequential staged backward."""
    B, Hq, Hkv, Lq, L, D, cp = 2, 4, 2, 200, 700, 128, 4
    q = _randn((B, Hq, Lq, D), 90).cuda()
    k, v = _randn((B, Hkv, L, D), 91).cuda(), _randn((B, Hkv, L, D), 92).cuda()
    do = _randn((B, Hq, Lq, D), 93).cuda()
    m = _key_mask(B, L, 8).cuda() if masked else None
    out, lse = amd.ring.ring_attention(q, k, v, cp=cp, key_mask=m)
    seq = amd.ring._ring_backward_into(do, q, k, v, out, lse, m, cp, None, overlap=False)
    ovl = amd.ring._ring_backward_into(do, q, k, v, out, lse, m, cp, None, overlap=True)
    torch.cuda.synchronize()
    for a_, b_ in zip(seq, ovl):
        assert torch.equal(a_, b_)
    rq, rk, rv = R.attention_bwd_f64(_f64(do), _f64(q), _f64(k), _f64(v), _f64(out),
                                     lse.cpu().numpy().astype(np.float64), None if m is None else m.cpu().numpy())
    for got, ref in zip(ovl, (rq, rk, rv)):
        assert np.abs(_f64(got) - ref).max() <= GRAD_REL_TOL * np.abs(ref).max()


def test_ring_step_signatures_drop_into_torch_loop(amd):
    # Call the local-step ops exactly as torch's ring does
    # (torch/.../_attention.py:468-475 and 567-575).
    q, k, v = _randn((1, 2, 128, 128), 100).cuda(), _randn((1, 2, 256, 128), 101).cuda(), _randn(
        (1, 2, 256, 128), 102).cuda()
    merger = amd.ring.SDPAMerger(True, seq_dim=2)
    for kk, vv in zip(k.chunk(2, dim=2), v.chunk(2, dim=2)):
        out, logsumexp, *rest = amd.ring.flash_attention_op(q, kk, vv, is_causal=False, dropout_p=0.0, scale=None)
        assert len(rest) == 7
        merger.step(out, logsumexp, False)
    out, lse = merger.results()
    full, full_lse = amd.ops.flash_fwd(q, k, v, None, None, None, 128 ** -0.5)
    assert (out.float() - full.float()).abs().max().item() <= 2e-2
    assert (lse - full_lse).abs().max().item() <= 1e-3
    do = _randn((1, 2, 128, 128), 103).cuda()
    dq, dk, dv, *rest = amd.ring.flash_attention_backward_op(
        grad_out=do, query=q, key=k, value=v, out=out, logsumexp=lse, is_causal=False, dropout_p=0.0,
        cum_seq_q=None, cum_seq_k=None, max_q=128, max_k=256, philox_seed=None, philox_offset=None, scale=None)
    assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == v.shape


# ---------------------------------------------------------------------------
# Errors surface like the reference's
# ---------------------------------------------------------------------------


def test_error_types(amd):
    q = _randn((1, 2, 16, 128), 1).cuda()
    with pytest.raises(TypeError):
        amd.ops.flash_fwd(q.float(), q, q, None, None, None, 0.1)
    with pytest.raises(ValueError):
        amd.ops.flash_fwd(q[..., :96].contiguous(), q[..., :96].contiguous(), q[..., :96].contiguous(), None, None,
                          None, 0.1)
    with pytest.raises(NotImplementedError):
        amd.attention.attention(q, q, q, is_causal=True)
    with pytest.raises(NotImplementedError):
        amd.attention.attention(q, q, q, dropout_p=0.1)
    with pytest.raises(RuntimeError):
        amd.ops.flash_fwd(q.cpu(), q.cpu(), q.cpu(), None, None, None, 0.1)
