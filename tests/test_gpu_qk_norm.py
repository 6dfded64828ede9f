"""GPU parity of the fused q/k RMSNorm + rotation kernels and of the
attention section of SelfAttention.forward built on them
(src/avgen/models/layers.py:530-545) against the CPU oracle.

Tolerances: the forward output within one bf16 ulp of the oracle's float32
chain (norm rounded to bf16, then the bit-exact rotation) — the row's sum of
squares is added in another order, so rstd may differ in its last bit — and
at most 0.1% of the values off at all; dX within 2e-2 of the largest float64
reference magnitude (bf16 output), dW within 1e-3 (float32 sums of the same
bf16 gradients); attention output as for the kernels (2e-2).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reference as R

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def amd():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    import avgen_amd

    return avgen_amd


def _bf16(shape, seed, scale=1.0):
    g = torch.Generator()
    g.manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


def _f(t):
    return t.detach().float().cpu().numpy()


def _tables(amd, B, grid, D):
    F, Hh, W = grid
    coords = torch.from_numpy(R.video_coords(F, Hh, W, batch=B)).cuda()
    return amd.rope.build_rotary_tables(coords, head_dim=D)


def _oracle_fwd(x, w, eps, tables):
    n = R.rms_norm_bf16(x, w, eps)
    if tables is None:
        return n
    return R.apply_rotary_bf16(n, _f(tables.cos), _f(tables.sin))


def _assert_within_ulp(got, ref):
    diff = np.abs(got - ref)
    assert (diff <= np.abs(ref) * 2.0 ** -7 + 1e-6).all(), float(diff.max())
    assert (diff > 0).mean() < 1e-3


CASES = [
    # B, H, grid, D, layout ("bhld" contiguous or "blhd" projection view), gain, rope
    (1, 4, (3, 8, 10), 128, "blhd", True, True),
    (2, 3, (2, 5, 7), 64, "bhld", True, True),
    (1, 2, (4, 6, 6), 128, "bhld", False, True),
    (2, 5, (1, 3, 9), 128, "blhd", True, False),
]


def _make_x(B, H, L, D, layout, seed):
    if layout == "blhd":
        return _bf16((B, L, H * D), seed).cuda().unflatten(-1, (H, D)).transpose(1, 2)
    return _bf16((B, H, L, D), seed).cuda()


@pytest.mark.parametrize("B,H,grid,D,layout,gain,rope", CASES)
def test_qk_norm_rope_matches_oracle(amd, B, H, grid, D, layout, gain, rope):
    L = grid[0] * grid[1] * grid[2]
    print(f"qk_norm case B={B} H={H} L={L} D={D} layout={layout} gain={gain} rope={rope}", flush=True)
    x = _make_x(B, H, L, D, layout, 1).requires_grad_(True)
    w = (torch.rand(D, generator=torch.Generator().manual_seed(2)) + 0.5).cuda().requires_grad_(True) if gain else None
    tables = _tables(amd, B, grid, D) if rope else None
    y = amd.layers.qk_norm_rope(x, w, eps=1e-6, tables=tables)
    assert y.stride() == x.stride(), "output keeps the input's layout"
    wn = None if w is None else _f(w)
    _assert_within_ulp(_f(y), _oracle_fwd(_f(x), wn, 1e-6, tables))
    dy = _bf16((B, H, L, D), 3).cuda()
    y.backward(dy)
    g = _f(dy) if tables is None else R.apply_rotary_bf16(_f(dy), _f(tables.cos), _f(tables.sin), inverse=True)
    rdx, rdw = R.rms_norm_bwd_f64(_f(x), wn, g, 1e-6)
    err = np.abs(_f(x.grad) - rdx).max()
    print(f"  dx err {err:.3e} (ref max {np.abs(rdx).max():.3e})", flush=True)
    assert err <= 2e-2 * np.abs(rdx).max()
    if gain:
        assert w.grad.dtype is torch.float32
        derr = np.abs(_f(w.grad) - rdw).max()
        print(f"  dw err {derr:.3e} (ref max {np.abs(rdw).max():.3e})", flush=True)
        assert derr <= 1e-3 * np.abs(rdw).max()


def test_qk_norm_dw_is_deterministic(amd):
    x = _bf16((1, 8, 3000, 128), 5).cuda()
    w = torch.ones(128, device="cuda", dtype=torch.bfloat16)
    dy = _bf16((1, 8, 3000, 128), 6).cuda()
    a = amd.ops.qk_norm_rope_bwd(dy, x, w, 1e-6, None, None)
    b = amd.ops.qk_norm_rope_bwd(dy, x, w, 1e-6, None, None)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


@pytest.mark.parametrize("Hq,Hkv,masked", [(4, 4, False), (4, 2, True)])
def test_self_attention_core_matches_oracle(amd, Hq, Hkv, masked):
    """Projection outputs in, (batch, seq, heads*dim) out, the output a view of
    the kernel's (no transpose copy); values against the oracle composition."""
    B, D, grid = 2, 128, (3, 8, 12)
    L = grid[0] * grid[1] * grid[2]
    qp = _bf16((B, L, Hq * D), 11).cuda().requires_grad_(True)
    kp = _bf16((B, L, Hkv * D), 12).cuda().requires_grad_(True)
    vp = _bf16((B, L, Hkv * D), 13).cuda().requires_grad_(True)
    wq = (torch.rand(D, generator=torch.Generator().manual_seed(14)) + 0.5).cuda().requires_grad_(True)
    wk = (torch.rand(D, generator=torch.Generator().manual_seed(15)) + 0.5).cuda().requires_grad_(True)
    tables = _tables(amd, B, grid, D)
    km = None
    if masked:
        km = torch.ones(B, L, dtype=torch.bool)
        km[1, L - 50:] = False
    mask = amd.attention.key_padding_mask(None if km is None else km.cuda())
    out = amd.layers.self_attention_core(qp, kp, vp, head_dim=D, q_norm_weight=wq, k_norm_weight=wk,
                                         rope=tables, key_mask=mask)
    assert out.shape == (B, L, Hq * D)
    assert out.is_contiguous(), "the kernel writes the (batch, seq, heads, dim) layout directly"
    qn = _oracle_fwd(_f(qp).reshape(B, L, Hq, D).transpose(0, 2, 1, 3), _f(wq), 1e-6, tables)
    kn = _oracle_fwd(_f(kp).reshape(B, L, Hkv, D).transpose(0, 2, 1, 3), _f(wk), 1e-6, tables)
    vv = _f(vp).reshape(B, L, Hkv, D).transpose(0, 2, 1, 3)
    ro, _ = R.attention_f64(qn, kn, vv, None if km is None else km.numpy())
    ro = ro.transpose(0, 2, 1, 3).reshape(B, L, Hq * D)
    assert np.abs(_f(out) - ro).max() <= 2e-2
    out.backward(_bf16((B, L, Hq * D), 16).cuda())
    for t in (qp, kp, vp, wq, wk):
        assert t.grad is not None and torch.isfinite(t.grad).all()


@pytest.mark.parametrize("norm,rope", [(False, True), (False, False), (True, False)])
def test_self_attention_core_variants(amd, norm, rope):
    """qk_norm=False (no gains) and/or no rotary tables: the same composition
    with those steps left out."""
    B, H, D, grid = 1, 2, 64, (2, 4, 8)
    L = grid[0] * grid[1] * grid[2]
    qp, kp, vp = (_bf16((B, L, H * D), s).cuda() for s in (31, 32, 33))
    w = (torch.rand(D, generator=torch.Generator().manual_seed(34)) + 0.5).cuda() if norm else None
    tables = _tables(amd, B, grid, D) if rope else None
    out = amd.layers.self_attention_core(qp, kp, vp, head_dim=D, q_norm_weight=w, k_norm_weight=w, rope=tables)

    def prep(t):
        x = _f(t).reshape(B, L, H, D).transpose(0, 2, 1, 3)
        if norm:
            x = R.rms_norm_bf16(x, _f(w), 1e-6)
        if rope:
            x = R.apply_rotary_bf16(x, _f(tables.cos), _f(tables.sin))
        return x

    ro, _ = R.attention_f64(prep(qp), prep(kp), _f(vp).reshape(B, L, H, D).transpose(0, 2, 1, 3))
    ro = ro.transpose(0, 2, 1, 3).reshape(B, L, H * D)
    assert np.abs(_f(out) - ro).max() <= 2e-2


# ---------------------------------------------------------------------------
# float32 rows (avattn_qk_norm_rope_f32 / _bwd_f32): a float32 model outside
# autocast keeps the gain in fp32 (src/avgen/models/layers.py:106-118).
# References in float64: the norm from the pinned oracle, the rotation as a
# complex multiplication by cos + i*sin (its transpose: by the conjugate).
# ---------------------------------------------------------------------------


def _f32(shape, seed, scale=1.0):
    g = torch.Generator()
    g.manual_seed(seed)
    return torch.randn(shape, generator=g) * scale


def _rot64(x, cos, sin, inverse=False):
    z = x[..., 0::2].astype(np.float64) + 1j * x[..., 1::2].astype(np.float64)
    r = np.asarray(cos, np.float64) + 1j * np.asarray(sin, np.float64)
    z = z * (np.conj(r) if inverse else r)
    out = np.empty(x.shape, np.float64)
    out[..., 0::2], out[..., 1::2] = z.real, z.imag
    return out


@pytest.mark.parametrize("B,H,grid,D,layout,gain,rope", CASES)
def test_f32_qk_norm_rope_matches_oracle(amd, B, H, grid, D, layout, gain, rope):
    L = grid[0] * grid[1] * grid[2]
    print(f"f32 qk_norm case B={B} H={H} L={L} D={D} layout={layout} gain={gain} rope={rope}", flush=True)
    if layout == "blhd":
        x = _f32((B, L, H * D), 41).cuda().unflatten(-1, (H, D)).transpose(1, 2)
    else:
        x = _f32((B, H, L, D), 41).cuda()
    x.requires_grad_(True)
    w = ((torch.rand(D, generator=torch.Generator().manual_seed(42)) + 0.5 + 1e-4).cuda().requires_grad_(True)
         if gain else None)
    tables = _tables(amd, B, grid, D) if rope else None
    y = amd.layers.qk_norm_rope(x, w, eps=1e-6, tables=tables)
    assert y.dtype is torch.float32 and y.stride() == x.stride()
    wn = None if w is None else _f(w)
    ref = R.rms_norm_f64(_f(x), wn, 1e-6)
    if tables is not None:
        ref = _rot64(ref, _f(tables.cos), _f(tables.sin))
    err = np.abs(_f(y) - ref).max()
    print(f"  y err {err:.3e} (ref max {np.abs(ref).max():.3e})", flush=True)
    assert err <= 1e-6 * max(1.0, np.abs(ref).max())
    dy = _f32((B, H, L, D), 43).cuda()
    y.backward(dy)
    g = _f(dy) if tables is None else _rot64(_f(dy), _f(tables.cos), _f(tables.sin), inverse=True)
    rdx, rdw = R.rms_norm_bwd_f64(_f(x), wn, g, 1e-6, round_gain=False)
    err = np.abs(_f(x.grad) - rdx).max()
    print(f"  dx err {err:.3e} (ref max {np.abs(rdx).max():.3e})", flush=True)
    assert x.grad.dtype is torch.float32 and err <= 2e-5 * np.abs(rdx).max()
    if gain:
        derr = np.abs(_f(w.grad) - rdw).max()
        print(f"  dw err {derr:.3e} (ref max {np.abs(rdw).max():.3e})", flush=True)
        assert w.grad.dtype is torch.float32 and derr <= 1e-4 * np.abs(rdw).max()


def test_f32_qk_norm_dw_is_deterministic(amd):
    x = _f32((1, 8, 3000, 128), 45).cuda()
    w = torch.rand(128, device="cuda") + 0.5
    dy = _f32((1, 8, 3000, 128), 46).cuda()
    a = amd.ops.qk_norm_rope_bwd(dy, x, w, 1e-6, None, None)
    b = amd.ops.qk_norm_rope_bwd(dy, x, w, 1e-6, None, None)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_f32_self_attention_core_matches_oracle(amd):
    """The attention section of SelfAttention on float32 projections: fp32
    norm with fp32 gains, fp32 rotation and fp32 attention against the
    float64 composition; gradients reach every input."""
    B, Hq, Hkv, D, grid = 2, 4, 2, 128, (3, 8, 12)
    L = grid[0] * grid[1] * grid[2]
    qp = _f32((B, L, Hq * D), 51).cuda().requires_grad_(True)
    kp = _f32((B, L, Hkv * D), 52).cuda().requires_grad_(True)
    vp = _f32((B, L, Hkv * D), 53).cuda().requires_grad_(True)
    wq = (torch.rand(D, generator=torch.Generator().manual_seed(54)) + 0.5).cuda().requires_grad_(True)
    wk = (torch.rand(D, generator=torch.Generator().manual_seed(55)) + 0.5).cuda().requires_grad_(True)
    tables = _tables(amd, B, grid, D)
    km = torch.ones(B, L, dtype=torch.bool)
    km[1, L - 50:] = False
    mask = amd.attention.key_padding_mask(km.cuda())
    out = amd.layers.self_attention_core(qp, kp, vp, head_dim=D, q_norm_weight=wq, k_norm_weight=wk,
                                         rope=tables, key_mask=mask)
    assert out.dtype is torch.float32 and out.shape == (B, L, Hq * D)

    def prep(t, w, H):
        x = R.rms_norm_f64(_f(t).reshape(B, L, H, D).transpose(0, 2, 1, 3), _f(w), 1e-6)
        return _rot64(x, _f(tables.cos), _f(tables.sin))

    ro, _ = R.attention_f64(prep(qp, wq, Hq), prep(kp, wk, Hkv), _f(vp).reshape(B, L, Hkv, D).transpose(0, 2, 1, 3),
                            km.numpy())
    ro = ro.transpose(0, 2, 1, 3).reshape(B, L, Hq * D)
    err = np.abs(_f(out) - ro).max()
    print(f"  f32 self-attention out err {err:.3e}", flush=True)
    assert err <= 2e-5 * max(1.0, np.abs(ro).max())
    out.backward(_f32((B, L, Hq * D), 56).cuda())
    for t in (qp, kp, vp, wq, wk):
        assert t.grad is not None and t.grad.dtype is torch.float32 and torch.isfinite(t.grad).all()
