"""GPU parity of the float32 path (avattn_fwd_f32 / avattn_bwd_f32 with
staged or recomputed dq, avattn_fwd_windowed_f32 / avattn_bwd_windowed_f32,
avattn_rope_apply_f32, through the C ABI) against the float64 oracle.

The reference's attention runs in the caller's dtype
(src/avgen/models/attention.py:227-273 -> F.scaled_dot_product_attention),
so float32 tensors are computed with float32 operands and products.  The bar
is float32's, about 500x tighter than the bf16 one: output 2e-5 of max(1,
|out|), LSE 2e-5 of max(1, |lse|), gradients 1e-4 of their largest
magnitude; masks and the row states (no valid key: out 0, LSE -inf) exact;
the rotation equal bit for bit to torch's float32 ops on the reference's
formula (src/avgen/models/rope.py:332-338).  BASELINE config c1 (float32,
1x4x1024x64 with its 3D RoPE) runs here without a bf16 cast.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reference as R

pytestmark = pytest.mark.gpu

OUT_TOL, LSE_TOL, GRAD_REL_TOL = 2e-5, 2e-5, 1e-4


@pytest.fixture(scope="module")
def amd():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    import avgen_amd

    return avgen_amd


def _randn(shape, seed, scale=1.0):
    g = torch.Generator()
    g.manual_seed(seed)
    return torch.randn(shape, generator=g) * scale


def _f64(t):
    return t.detach().cpu().numpy().astype(np.float64)


def _check_fwd(o, l, ro, rl):
    assert np.array_equal(np.isnan(o), np.isnan(ro))
    fin = np.isfinite(rl)
    assert np.array_equal(np.isneginf(l), np.isneginf(rl))
    ok = ~np.isnan(ro)
    assert np.abs(o[ok] - ro[ok]).max(initial=0.0) <= OUT_TOL * max(1.0, np.abs(ro[ok]).max(initial=0.0))
    assert (np.abs(l[fin] - rl[fin]) <= LSE_TOL * np.maximum(1.0, np.abs(rl[fin]))).all()


CASES = [
    # B, Hq, Hkv, Lq, Lk, D, masked
    (1, 2, 2, 128, 128, 128, False),
    (2, 4, 2, 200, 333, 128, True),
    (1, 3, 1, 77, 1000, 64, True),
    (2, 2, 2, 1, 5, 64, False),
    (1, 2, 1, 513, 31, 128, True),
]


@pytest.mark.parametrize("staged", [True, False], ids=["staged_ds", "recompute"])
@pytest.mark.parametrize("B,Hq,Hkv,Lq,Lk,D,masked", CASES)
def test_f32_forward_backward_match_oracle(amd, B, Hq, Hkv, Lq, Lk, D, masked, staged):
    print(f"f32 case B={B} Hq={Hq} Hkv={Hkv} Lq={Lq} Lk={Lk} D={D} masked={masked} staged={staged}", flush=True)
    q, k, v, do = _randn((B, Hq, Lq, D), 1), _randn((B, Hkv, Lk, D), 2), _randn((B, Hkv, Lk, D), 3), _randn(
        (B, Hq, Lq, D), 4)
    mask = None
    if masked:
        g = torch.Generator()
        g.manual_seed(5)
        mask = torch.rand((B, Lk), generator=g) < 0.7
        mask[0, 0] = True
        if B > 1:
            mask[-1] = False  # a batch row without valid keys
    mk = None if mask is None else mask.cuda()
    out, lse = amd.ops.flash_fwd(q.cuda(), k.cuda(), v.cuda(), mk, None, None, D ** -0.5)
    assert out.dtype is torch.float32
    km = None if mask is None else mask.numpy()
    ro, rl = R.attention_f64(_f64(q), _f64(k), _f64(v), km)
    o, l = _f64(out), _f64(lse)
    _check_fwd(o, l, ro, rl)
    if masked and B > 1:
        assert np.all(o[-1] == 0) and np.all(np.isneginf(l[-1]))
    dev = torch.device("cuda", 0)
    amd.ops.set_ds_budget(None if staged else 0, dev)
    try:
        dq, dk, dv = amd.ops.flash_bwd(do.cuda(), q.cuda(), k.cuda(), v.cuda(), out, lse, mk, D ** -0.5)
    finally:
        amd.ops.set_ds_budget(None, dev)
    ref = R.attention_bwd_f64(_f64(do), _f64(q), _f64(k), _f64(v), o, l, km)
    for name, got, r in zip(("dq", "dk", "dv"), (dq, dk, dv), ref):
        assert got.dtype is torch.float32
        err = np.abs(_f64(got) - r).max()
        print(f"  {name}: max err {err:.3e} (ref max {np.abs(r).max():.3e})", flush=True)
        assert err <= GRAD_REL_TOL * max(np.abs(r).max(), 1e-6), name
    if mask is not None:
        gone = np.broadcast_to(~mask.numpy()[:, None, :, None], dk.shape)
        assert np.all(_f64(dk)[gone] == 0) and np.all(_f64(dv)[gone] == 0)


@pytest.mark.parametrize("B,Hq,Hkv,Lq,Lk,D", [(3, 4, 2, 300, 700, 128), (2, 3, 1, 129, 250, 64)])
def test_f32_staged_ds_passes_and_recompute(amd, B, Hq, Hkv, Lq, Lk, D):
    """The staged-dS backward in passes of 1, some and all (batch, kv head)
    pairs, and the recomputing one: dk and dv are the same bits every way
    (the dK/dV kernel's arithmetic does not change when it also stores dS),
    dq from the staged dS the same bits for every pass size (pairs are
    independent) and within fp32 rounding of the recomputed dq."""
    print(f"f32 staged passes B={B} Hq={Hq} Hkv={Hkv} Lq={Lq} Lk={Lk} D={D}", flush=True)
    dev = torch.device("cuda", 0)
    q, k, v, do = (_randn(s, 10 + i).cuda() for i, s in enumerate(
        ((B, Hq, Lq, D), (B, Hkv, Lk, D), (B, Hkv, Lk, D), (B, Hq, Lq, D))))
    g = torch.Generator()
    g.manual_seed(11)
    mask = (torch.rand((B, Lk), generator=g) < 0.8).cuda()
    out, lse = amd.ops.flash_fwd(q, k, v, mask, None, None, D ** -0.5)
    per = amd.ops.f32_ds_bytes_per_pair(Hq // Hkv, Lq, Lk)
    runs = {}
    for label, budget in (("recompute", 0), ("one pair", per), ("passes", 2 * per + 1), ("one pass", None)):
        amd.ops.set_ds_budget(budget, dev)
        try:
            runs[label] = amd.ops.flash_bwd(do, q, k, v, out, lse, mask, D ** -0.5)
        finally:
            amd.ops.set_ds_budget(None, dev)
    torch.cuda.synchronize()
    base = runs["one pass"]
    for label, got in runs.items():
        assert torch.equal(got[1], base[1]) and torch.equal(got[2], base[2]), label
        if label != "recompute":
            assert torch.equal(got[0], base[0]), label
    diff = (runs["recompute"][0] - base[0]).abs().max().item()
    top = base[0].abs().max().item()
    print(f"  dq staged vs recomputed: {diff:.3e} of {top:.3e}", flush=True)
    assert diff <= 1e-5 * top


def test_f32_rotation_bit_exact(amd):
    """rope_apply on float32 equals torch's float32 ops on the reference's
    formula bit for bit, forward and transpose; its autograd is the
    transpose."""
    B, H, L, D = 2, 3, 257, 128
    coords = torch.stack(torch.meshgrid(torch.arange(1.0) / 8, torch.arange(257.0) * 2, torch.arange(1.0),
                                        indexing="ij"), -1).reshape(1, L, 3).expand(B, -1, -1).contiguous()
    tables = amd.rope.build_rotary_tables(coords.cuda(), head_dim=D)
    x = _randn((B, H, L, D), 7, 3.0).cuda()
    c, s = tables.cos, tables.sin
    e, o = x[..., 0::2], x[..., 1::2]
    ref = torch.stack((e * c - o * s, e * s + o * c), -1).flatten(-2)
    ref_t = torch.stack((e * c + o * s, o * c - e * s), -1).flatten(-2)
    got = amd.rope.apply_rotary(x, tables)
    assert got.dtype is torch.float32
    assert torch.equal(got, ref)
    assert torch.equal(amd.ops.rope_apply(x, c, s, True), ref_t)
    xg = x.clone().requires_grad_(True)
    amd.rope.apply_rotary(xg, tables).backward(x)
    assert torch.equal(xg.grad, ref_t)


def _coords(frames, height, width, batch):
    t = torch.arange(frames, dtype=torch.float32) / 8.0
    r = torch.arange(height, dtype=torch.float32) * 2.0
    c = torch.arange(width, dtype=torch.float32) * 2.0
    g = torch.stack(torch.meshgrid(t, r, c, indexing="ij"), -1).reshape(1, -1, 3)
    return g.expand(batch, -1, -1).contiguous()


def test_c1_config_in_float32(amd):
    """BASELINE config c1 as stated: float32 q/k/v (B=1, 4 heads, head_dim 64,
    a 4x16x16 latent = 1,024 tokens, N(0,1)), the 3D RoPE with theta 1e4 and
    the head_dim-64 split (12, 10, 10), no mask, forward out + LSE, against
    float64 attention on the float64 rotation of the same float32 inputs."""
    B, H, D, grid = 1, 4, 64, (4, 16, 16)
    L = grid[0] * grid[1] * grid[2]
    g = torch.Generator()
    g.manual_seed(0)
    q32, k32, v32 = (torch.randn((B, H, L, D), generator=g) for _ in range(3))
    coords = _coords(*grid, B)
    tables = amd.rope.build_rotary_tables(coords.cuda(), head_dim=D)
    out, lse = amd.ops.flash_fwd(q32.cuda(), amd.rope.apply_rotary(k32.cuda(), tables), v32.cuda(), None,
                                 tables.cos, tables.sin, D ** -0.5)
    c64, s64 = R.rotary_tables_f64(coords.numpy(), D)

    def rot64(x):
        x = x.numpy().astype(np.float64)
        e, od = x[..., 0::2], x[..., 1::2]
        y = np.empty_like(x)
        y[..., 0::2] = e * c64 - od * s64
        y[..., 1::2] = e * s64 + od * c64
        return y

    fo, fl = R.attention_f64(rot64(q32), rot64(k32), v32.numpy().astype(np.float64))
    o, l = _f64(out), _f64(lse)
    print(f"c1 float32: out err {np.abs(o - fo).max():.2e}, lse err {np.abs(l - fl).max():.2e}", flush=True)
    _check_fwd(o, l, fo, fl)


def test_f32_attention_dropin_autograd(amd):
    """attention() and rotary_attention() with float32 tensors through
    autograd, against float64 gradients."""
    B, H, L, D = 1, 2, 300, 128
    q, k, v, do = (_randn((B, H, L, D), s) for s in (11, 12, 13, 14))
    mask = torch.ones(B, L, dtype=torch.bool)
    mask[:, 250:] = False
    qg, kg, vg = (t.cuda().requires_grad_(True) for t in (q, k, v))
    out = amd.attention.attention(qg, kg, vg, attn_mask=amd.attention.key_padding_mask(mask.cuda()))
    out.backward(do.cuda())
    ro, rl = R.attention_f64(_f64(q), _f64(k), _f64(v), mask.numpy())
    assert np.abs(_f64(out) - ro).max() <= OUT_TOL * max(1.0, np.abs(ro).max())
    ref = R.attention_bwd_f64(_f64(do), _f64(q), _f64(k), _f64(v), ro, rl, mask.numpy())
    for got, r in zip((qg.grad, kg.grad, vg.grad), ref):
        assert np.abs(_f64(got) - r).max() <= GRAD_REL_TOL * np.abs(r).max()
    # the rotary drop-in: same as rotating first (fp32 rotation is exact torch ops)
    coords = _coords(3, 10, 10, B)
    tables = amd.rope.build_rotary_tables(coords.cuda(), head_dim=D)
    qa, ka, va = (t.cuda().requires_grad_(True) for t in (q, k, v))
    oa = amd.attention.rotary_attention(qa, ka, va, tables)
    oa.backward(do.cuda())
    qb, kb, vb = (t.cuda().requires_grad_(True) for t in (q, k, v))
    ob = amd.attention.attention(amd.rope.apply_rotary(qb, tables), amd.rope.apply_rotary(kb, tables), vb)
    ob.backward(do.cuda())
    assert torch.equal(oa, ob)
    for a_, b_ in ((qa.grad, qb.grad), (ka.grad, kb.grad), (va.grad, vb.grad)):
        assert torch.equal(a_, b_)


def test_f32_edges(amd):
    """Zero-length sequences, a NaN key reaching every row of its head (as
    the float64 math gives), and run-to-run bits."""
    q = _randn((1, 2, 40, 64), 20).cuda()
    k0 = torch.empty((1, 2, 0, 64), device="cuda")
    out, lse = amd.ops.flash_fwd(q, k0, k0, None, None, None, 0.125)
    assert torch.all(out == 0) and torch.all(torch.isneginf(lse))
    assert torch.all(amd.attention.attention(q, k0, k0) == 0)
    dq, dk, dv = amd.ops.flash_bwd(q, q, k0, k0, out, lse, None, 0.125)
    assert torch.all(dq == 0) and dk.numel() == 0
    k = _randn((1, 2, 70, 64), 21).cuda()
    k[0, 1, 33, 5] = float("nan")
    out, lse = amd.ops.flash_fwd(q, k, k, None, None, None, 0.125)
    ro, rl = R.attention_f64(_f64(q), _f64(k), _f64(k), None, 0.125)
    _check_fwd(_f64(out), _f64(lse), ro, rl)
    assert torch.isnan(out[0, 1]).all() and not torch.isnan(out[0, 0]).any()
    k = _randn((2, 1, 700, 128), 22).cuda()
    q = _randn((2, 4, 300, 128), 23).cuda()
    do = _randn((2, 4, 300, 128), 24).cuda()
    m = torch.rand((2, 700), device="cuda") < 0.9

    def run():
        o, l = amd.ops.flash_fwd(q, k, k, m, None, None, 0.09)
        return (o, l, *amd.ops.flash_bwd(do, q, k, k, o, l, m, 0.09))

    first = run()
    torch.randn(1 << 20, device="cuda").sum().item()
    for a_, b_ in zip(first, run()):
        assert torch.equal(a_, b_)


def test_f32_ring_matches_oracle(amd):
    """ring_attention on float32 tensors: the ring forward and backward over
    cp chunks against float64 (the unchunked attention), and with tables the
    same bits as rotating first."""
    B, H, D, cp = 2, 2, 64, 3
    L = 3 * 96
    q, k, v, do = (_randn((B, H, L if i else 96, D), 30 + i) for i in (0, 1, 2, 3))
    q, do = q[:, :, :96].contiguous(), do[:, :, :96].contiguous()
    mask = torch.ones(B, L, dtype=torch.bool)
    mask[1, 100:250] = False
    qg, kg, vg = (t.cuda().requires_grad_(True) for t in (q, k, v))
    out, lse = amd.ring.ring_attention(qg, kg, vg, cp=cp, key_mask=mask.cuda())
    out.backward(do.cuda())
    assert out.dtype is torch.float32
    ro, rl = R.attention_f64(_f64(q), _f64(k), _f64(v), mask.numpy())
    _check_fwd(_f64(out), _f64(lse), ro, rl)
    ref = R.attention_bwd_f64(_f64(do), _f64(q), _f64(k), _f64(v), ro, rl, mask.numpy())
    for got, r in zip((qg.grad, kg.grad, vg.grad), ref):
        assert np.abs(_f64(got) - r).max() <= GRAD_REL_TOL * np.abs(r).max()
    coords = _coords(3, 12, 8, B)
    tables = amd.rope.build_rotary_tables(coords.cuda(), head_dim=D)
    tq = tables.slice(0, 96)
    qa, ka, va = (t.cuda().requires_grad_(True) for t in (q, k, v))
    oa, la = amd.ring.ring_attention(qa, ka, va, cp=cp, tables_q=tq, tables_k=tables)
    oa.backward(do.cuda())
    qb, kb, vb = (t.cuda().requires_grad_(True) for t in (q, k, v))
    ob, lb = amd.ring.ring_attention(amd.rope.apply_rotary(qb, tq), amd.rope.apply_rotary(kb, tables), vb, cp=cp)
    ob.backward(do.cuda())
    for a_, b_ in ((oa, ob), (la, lb), (qa.grad, qb.grad), (ka.grad, kb.grad), (va.grad, vb.grad)):
        assert torch.equal(a_, b_)


def test_f32_compiles_to_the_eager_bits(amd):
    """torch.compile(fullgraph=True) over float32 attention with rotation and
    its backward: the same bits as eager (the ops' fake kernels give float32
    outputs)."""
    B, H, L, D = 1, 2, 200, 64
    q, k, v, do = (_randn((B, H, L, D), s).cuda() for s in (40, 41, 42, 43))
    tables = amd.rope.build_rotary_tables(_coords(2, 10, 10, B).cuda(), head_dim=D)

    def f(q, k, v):
        return amd.attention.rotary_attention(q, k, v, tables)

    def run(fn):
        qg, kg, vg = (t.clone().requires_grad_(True) for t in (q, k, v))
        out = fn(qg, kg, vg)
        out.backward(do)
        return out.detach(), qg.grad, kg.grad, vg.grad

    eager = run(f)
    compiled = run(torch.compile(f, fullgraph=True))
    for a_, b_ in zip(eager, compiled):
        assert a_.dtype is torch.float32 and torch.equal(a_, b_)


# ---------------------------------------------------------------------------
# float32 with per-row key windows (avattn_fwd_windowed_f32 /
# avattn_bwd_windowed_f32): the reference's temporal neighbour mask
# (src/avgen/models/blocks.py:54-104) and packed block-diagonal mask
# (src/avgen/data/packing.py:181-200) in the caller's dtype.
# ---------------------------------------------------------------------------


def _window_mask(lo, hi, Lk):
    j = np.arange(Lk)
    return (j >= np.asarray(lo)[..., None]) & (j < np.asarray(hi)[..., None])


def _monotone_windows(B, Lq, Lk, seed, max_width, empty_tail=0):
    """Non-decreasing (lo, hi) with widths up to max_width and some empty
    rows; the last empty_tail rows get the empty window [Lk, Lk)."""
    rng = np.random.default_rng(seed)
    lo = np.sort(rng.integers(0, Lk + 1, (B, Lq)), axis=1)
    hi = np.maximum.accumulate(np.minimum(lo + rng.integers(0, max_width + 1, (B, Lq)), Lk), axis=1)
    if empty_tail:
        lo[:, Lq - empty_tail:] = Lk
        hi[:, Lq - empty_tail:] = Lk
    return lo.astype(np.int32), hi.astype(np.int32)


F32_WIN_CASES = [
    # B, Hq, Hkv, Lq, Lk, D, width, empty tail, per-batch windows
    (1, 2, 2, 300, 500, 128, 120, 0, False),
    (2, 4, 2, 257, 700, 64, 300, 17, True),
    (2, 2, 1, 1000, 333, 128, 60, 5, True),
]


@pytest.mark.parametrize("staged", [True, False], ids=["staged_ds", "recompute"])
@pytest.mark.parametrize("B,Hq,Hkv,Lq,Lk,D,width,tail,per_batch", F32_WIN_CASES)
def test_f32_windowed_forward_backward_match_oracle(amd, B, Hq, Hkv, Lq, Lk, D, width, tail, per_batch, staged):
    print(f"f32 windowed B={B} Hq={Hq} Hkv={Hkv} Lq={Lq} Lk={Lk} D={D} width={width} tail={tail} "
          f"per_batch={per_batch} staged={staged}", flush=True)
    q, k, v, do = (_randn(s, 60 + i) for i, s in enumerate(
        ((B, Hq, Lq, D), (B, Hkv, Lk, D), (B, Hkv, Lk, D), (B, Hq, Lq, D))))
    lo, hi = _monotone_windows(B if per_batch else 1, Lq, Lk, 65, width, tail)
    km = np.random.default_rng(66).random((B, Lk)) < 0.8
    lo_t, hi_t = torch.from_numpy(lo).cuda(), torch.from_numpy(hi).cuda()
    if not per_batch:
        lo_t, hi_t = lo_t[0], hi_t[0]
    kmc = torch.from_numpy(km).cuda()
    scale = D ** -0.5
    out, lse = amd.ops.flash_fwd_windowed(q.cuda(), k.cuda(), v.cuda(), lo_t, hi_t, kmc, scale)
    assert out.dtype is torch.float32
    dense = _window_mask(lo, hi, Lk)  # (B|1, Lq, Lk)
    ro, rl = R.attention_f64(_f64(q), _f64(k), _f64(v), km, attn_mask=dense)
    o, l = _f64(out), _f64(lse)
    _check_fwd(o, l, ro, rl)
    dev = torch.device("cuda", 0)
    amd.ops.set_ds_budget(None if staged else 0, dev)
    try:
        grads = amd.ops.flash_bwd_windowed(do.cuda(), q.cuda(), k.cuda(), v.cuda(), out, lse, lo_t, hi_t, kmc, scale)
    finally:
        amd.ops.set_ds_budget(None, dev)
    ref = R.attention_bwd_f64(_f64(do), _f64(q), _f64(k), _f64(v), o, l, km, attn_mask=dense)
    for name, got, r in zip(("dq", "dk", "dv"), grads, ref):
        assert got.dtype is torch.float32
        err = np.abs(_f64(got) - r).max()
        print(f"  {name}: max err {err:.3e} (ref max {np.abs(r).max():.3e})", flush=True)
        assert err <= GRAD_REL_TOL * max(np.abs(r).max(), 1e-6), name
    # keys no row reaches (window or key mask): exactly zero dK/dV
    reached = np.broadcast_to(dense.any(axis=-2), (B, Lk)) & km
    for g in grads[1:]:
        gz = _f64(g)
        for b in range(B):
            assert (gz[b][:, ~reached[b]] == 0).all()


@pytest.mark.parametrize("D", [64, 128])
def test_f32_full_windows_equal_the_unwindowed_kernels(amd, D):
    """Windows [0, Lk) for every row: the windowed kernels visit the same
    tiles and compute the same values, so forward and backward (staged and
    recomputing) give the unwindowed kernels' bits.  (A tile loop whose
    bounds the compiler could not prove wave-uniform once ran as a divergent
    loop around its barriers and gave garbage at head_dim 64.)"""
    B, Hq, Hkv, Lq, Lk = 2, 4, 2, 200, 300
    q, k, v, do = (_randn(s, 70 + i).cuda() for i, s in enumerate(
        ((B, Hq, Lq, D), (B, Hkv, Lk, D), (B, Hkv, Lk, D), (B, Hq, Lq, D))))
    lo = torch.zeros(Lq, dtype=torch.int32, device="cuda")
    hi = torch.full((Lq,), Lk, dtype=torch.int32, device="cuda")
    out, lse = amd.ops.flash_fwd(q, k, v, None, None, None, D ** -0.5)
    wout, wlse = amd.ops.flash_fwd_windowed(q, k, v, lo, hi, None, D ** -0.5)
    assert torch.equal(out, wout) and torch.equal(lse, wlse)
    dev = torch.device("cuda", 0)
    for budget in (None, 0):
        amd.ops.set_ds_budget(budget, dev)
        try:
            g = amd.ops.flash_bwd(do, q, k, v, out, lse, None, D ** -0.5)
            wg = amd.ops.flash_bwd_windowed(do, q, k, v, out, lse, lo, hi, None, D ** -0.5)
        finally:
            amd.ops.set_ds_budget(None, dev)
        for name, x, y in zip(("dq", "dk", "dv"), g, wg):
            assert torch.equal(x, y), (budget, name)


def test_f32_varlen_attention_matches_the_packed_mask(amd):
    lengths, capacity, H, D = [700, 129, 64, 1000], 2048, 2, 128
    q, k, v = (_randn((1, H, capacity, D), s).cuda().requires_grad_(True) for s in (81, 82, 83))
    do = _randn((1, H, capacity, D), 84)
    cu = torch.tensor(R.packed_cu_seqlens(lengths))
    out = amd.attention.varlen_attention(q, k, v, cu)
    assert out.dtype is torch.float32
    dense = R.packed_attention_mask(lengths, capacity)[None]
    ro, rl = R.attention_f64(_f64(q), _f64(k), _f64(v), attn_mask=dense)
    o = _f64(out)
    assert np.abs(o - ro).max() <= OUT_TOL * max(1.0, np.abs(ro).max())
    assert (o[:, :, sum(lengths):] == 0).all()
    out.backward(do.cuda())
    ref = R.attention_bwd_f64(_f64(do), _f64(q), _f64(k), _f64(v), ro, rl, attn_mask=dense)
    for name, got, r in zip(("dq", "dk", "dv"), (q.grad, k.grad, v.grad), ref):
        assert np.abs(_f64(got) - r).max() <= GRAD_REL_TOL * max(np.abs(r).max(), 1e-6), name


def test_f32_temporal_neighbour_attention_matches_the_dense_mask(amd):
    """Video queries (frames of 48 tokens at 24 fps) against audio keys, a
    0.1 s window, shuffled token order and masked keys, in float32; the last
    frames have no key in range and fall back to every key."""
    B, Hq, Hkv, D = 2, 4, 2, 64
    tq = np.stack([(np.arange(960) // 48) / 24.0, 0.05 + (np.arange(960) // 48) / 24.0]).astype(np.float32)
    tk = np.stack([np.arange(260) / 43.0, 0.2 + np.arange(260) / 43.0]).astype(np.float32)
    Lq, Lk = tq.shape[1], tk.shape[1]
    rng = np.random.default_rng(91)
    km = rng.random((B, Lk)) < 0.7
    pq, pk = rng.permutation(Lq), rng.permutation(Lk)
    tq, tk = tq[:, pq], tk[:, pk]
    q = _randn((B, Hq, Lq, D), 92).cuda().requires_grad_(True)
    k = _randn((B, Hkv, Lk, D), 93).cuda().requires_grad_(True)
    v = _randn((B, Hkv, Lk, D), 94).cuda().requires_grad_(True)
    do = _randn((B, Hq, Lq, D), 95)
    out = amd.attention.temporal_neighbour_attention(
        q, k, v, torch.from_numpy(tq).cuda(), torch.from_numpy(tk).cuda(), window_seconds=0.1,
        key_mask=torch.from_numpy(km).cuda(), enable_gqa=True)
    assert out.dtype is torch.float32
    dense = R.temporal_neighbour_mask(tq, tk, 0.1, km)
    ro, rl = R.attention_f64(_f64(q), _f64(k), _f64(v), attn_mask=dense)
    assert np.abs(_f64(out) - ro).max() <= OUT_TOL * max(1.0, np.abs(ro).max())
    out.backward(do.cuda())
    ref = R.attention_bwd_f64(_f64(do), _f64(q), _f64(k), _f64(v), ro, rl, attn_mask=dense)
    for name, got, r in zip(("dq", "dk", "dv"), (q.grad, k.grad, v.grad), ref):
        assert np.abs(_f64(got) - r).max() <= GRAD_REL_TOL * max(np.abs(r).max(), 1e-6), name


@pytest.mark.parametrize("staged", [True, False], ids=["staged_ds", "recompute"])
@pytest.mark.parametrize("windowed", [False, True], ids=["plain", "windowed"])
def test_f32_large_query_group(amd, staged, windowed):
    """Five query heads per kv head (the dK/dV kernel's loop over the group),
    plain and with per-batch windows, against float64."""
    B, Hq, Hkv, Lq, Lk, D = 2, 10, 2, 300, 260, 64
    print(f"f32 group-5 staged={staged} windowed={windowed}", flush=True)
    q, k, v, do = (_randn(s, 100 + i) for i, s in enumerate(
        ((B, Hq, Lq, D), (B, Hkv, Lk, D), (B, Hkv, Lk, D), (B, Hq, Lq, D))))
    km = np.random.default_rng(105).random((B, Lk)) < 0.85
    kmc = torch.from_numpy(km).cuda()
    dev = torch.device("cuda", 0)
    dense = None
    if windowed:
        lo, hi = _monotone_windows(B, Lq, Lk, 106, 90, 7)
        lo_t, hi_t = torch.from_numpy(lo).cuda(), torch.from_numpy(hi).cuda()
        dense = _window_mask(lo, hi, Lk)
        out, lse = amd.ops.flash_fwd_windowed(q.cuda(), k.cuda(), v.cuda(), lo_t, hi_t, kmc, D ** -0.5)
    else:
        out, lse = amd.ops.flash_fwd(q.cuda(), k.cuda(), v.cuda(), kmc, None, None, D ** -0.5)
    ro, rl = R.attention_f64(_f64(q), _f64(k), _f64(v), km, attn_mask=dense)
    o, l = _f64(out), _f64(lse)
    _check_fwd(o, l, ro, rl)
    amd.ops.set_ds_budget(None if staged else 0, dev)
    try:
        if windowed:
            grads = amd.ops.flash_bwd_windowed(do.cuda(), q.cuda(), k.cuda(), v.cuda(), out, lse, lo_t, hi_t, kmc,
                                               D ** -0.5)
        else:
            grads = amd.ops.flash_bwd(do.cuda(), q.cuda(), k.cuda(), v.cuda(), out, lse, kmc, D ** -0.5)
    finally:
        amd.ops.set_ds_budget(None, dev)
    ref = R.attention_bwd_f64(_f64(do), _f64(q), _f64(k), _f64(v), o, l, km, attn_mask=dense)
    for name, got, r in zip(("dq", "dk", "dv"), grads, ref):
        err = np.abs(_f64(got) - r).max()
        print(f"  {name}: max err {err:.3e} (ref max {np.abs(r).max():.3e})", flush=True)
        assert err <= GRAD_REL_TOL * max(np.abs(r).max(), 1e-6), name
