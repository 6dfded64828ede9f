"""Seeded sweeps of random shapes through the windowed, fp8 and ring entry
points against the float64 oracle (the plain forward/backward has its own
sweep).  Each case draws batch 1-3, 1-3 KV heads with 1-2 query heads each,
lengths 1-700 (every padding remainder of the 64-row tiles and 128-key
blocks), head dims 64 and 128, input scales 0.1-4 and key-padding masks
with holes and fully masked batch rows.

- windowed: random non-decreasing windows (shared or per batch row, widths
  1-400, empty windows, a tail of rows with none), compact or dense staged
  dS, one pass or one (batch, kv head) pair per pass;
- fp8: per-head absmax scales, quantized exactly as the kernels do;
- ring: cp 1-4 equal chunks of the key sequence, with and without the fused
  3D RoPE (whose results must equal the unfused composition bit for bit);
- float32: the fp32 forward and backward at float32's bar, and with random
  key windows (shuffled for a forward check; staged or recomputed dq).

The bars are the kernels' usual ones, scaled with the data: output 2e-2 of
max(1, its largest magnitude), LSE 1e-3 (fp8: plus 2^-14 of |lse|, the e4m3
MFMA's fixed-point accumulation), gradients 2e-2 of their largest magnitude
(float32: 1e-4), plus for dq and dk 2^-20 of the size of the terms dS = P
(dP - Dr) cancels (a single key makes the true dq and dk exactly 0); keys
no window or mask admits get exactly zero dK/dV."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reference as R

pytestmark = pytest.mark.gpu

OUT_TOL, LSE_TOL, GRAD_REL_TOL = 2e-2, 1e-3, 2e-2


@pytest.fixture(scope="module")
def amd():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    import avgen_amd

    return avgen_amd


def _f64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _shape(rng, max_len=700):
    hkv = int(rng.integers(1, 4))
    return dict(B=int(rng.integers(1, 4)), Hq=hkv * int(rng.integers(1, 3)), Hkv=hkv,
                Lq=int(rng.integers(1, max_len + 1)), Lk=int(rng.integers(1, max_len + 1)),
                D=int(rng.choice([64, 128])), scale=float(rng.choice([0.1, 0.7, 2.0, 4.0])),
                masked=bool(rng.integers(0, 2)))


def _tensors(c, seed, Lk=None):
    g = torch.Generator()
    g.manual_seed(seed)
    B, Hq, Hkv, Lq, D = c["B"], c["Hq"], c["Hkv"], c["Lq"], c["D"]
    Lk = c["Lk"] if Lk is None else Lk
    q, k, v, do = ((torch.randn(s, generator=g) * c["scale"]).to(torch.bfloat16)
                   for s in ((B, Hq, Lq, D), (B, Hkv, Lk, D), (B, Hkv, Lk, D), (B, Hq, Lq, D)))
    mask = None
    if c["masked"]:
        mask = torch.rand((B, Lk), generator=g) < 0.8
        mask[0, : max(1, Lk // 3)] = True
        if B > 1:
            mask[-1] = False  # a fully masked batch row
    return q, k, v, do, mask


def _check_out(o, l, ro, rl, lse_rel=0.0):
    assert np.isfinite(o).all()
    assert np.abs(o - ro).max() <= OUT_TOL * max(1.0, np.abs(ro).max())
    fin = np.isfinite(rl)
    assert np.array_equal(np.isneginf(l), ~fin)
    assert (o[~fin] == 0).all()
    assert (np.abs(l[fin] - rl[fin]) <= LSE_TOL + lse_rel * np.abs(rl[fin])).all()


def _check_grads(got, ref, mags=(None, None), rel=GRAD_REL_TOL, floor=1e-3):
    """Gradients against float64: rel of their largest magnitude (at least
    ``floor``), plus for dq and dk 2^-20 of the size of the terms that dS =
    P (dP - Dr) cancels (``mags``: attention_bwd_magnitudes_f64), the scale
    of its rounding where one key carries a row."""
    for name, g, r, m in zip(("dq", "dk", "dv"), got, ref, (*mags, None)):
        g = _f64(g)
        assert np.isfinite(g).all(), name
        err = np.abs(g - r).max()
        extra = 0.0 if m is None else 2.0**-20 * m.max(initial=0.0)
        assert err <= rel * max(np.abs(r).max(), floor) + extra, (name, err)


def _windows(rng, rows, Lq, Lk):
    width = int(rng.integers(1, 401))
    lo = np.sort(rng.integers(0, Lk + 1, (rows, Lq)), axis=1)
    hi = np.maximum.accumulate(np.minimum(lo + rng.integers(0, width + 1, (rows, Lq)), Lk), axis=1)
    tail = int(rng.integers(0, 2)) * int(rng.integers(1, Lq + 1))
    if tail:
        lo[:, Lq - tail:] = Lk
        hi[:, Lq - tail:] = Lk
    return lo.astype(np.int32), hi.astype(np.int32)


@pytest.mark.parametrize("seed", range(16))
def test_windowed_random_shapes_match_oracle(amd, seed):
    rng = np.random.default_rng(2000 + seed)
    c = _shape(rng)
    per_batch, compact, one_pair = (bool(rng.integers(0, 2)) for _ in range(3))
    B, Lq, Lk, D = c["B"], c["Lq"], c["Lk"], c["D"]
    lo, hi = _windows(rng, B if per_batch else 1, Lq, Lk)
    q, k, v, do, mask = _tensors(c, seed)
    print(f"windowed sweep seed={seed} {c} per_batch={per_batch} compact={compact} one_pair={one_pair}",
          flush=True)
    dev = torch.device("cuda", 0)
    lo_t, hi_t = torch.from_numpy(lo).cuda(), torch.from_numpy(hi).cuda()
    if not per_batch:
        lo_t, hi_t = lo_t[0], hi_t[0]
    mk = None if mask is None else mask.cuda()
    ops = amd.ops
    out, lse = ops.flash_fwd_windowed(q.cuda(), k.cuda(), v.cuda(), lo_t, hi_t, mk, D ** -0.5)
    ops.set_ds_budget(1 if one_pair else None, dev)  # 1 byte: one (batch, kv head) pair per pass
    try:
        grads = ops._bwd_windowed_impl(do.cuda(), q.cuda(), k.cuda(), v.cuda(), out, lse, lo_t, hi_t, mk,
                                       D ** -0.5, compact=compact)
    finally:
        ops.set_ds_budget(None, dev)
    km = None if mask is None else mask.numpy()
    j = np.arange(Lk)
    dense = (j >= lo[..., None]) & (j < hi[..., None])
    ro, rl = R.attention_f64(_f64(q), _f64(k), _f64(v), km, attn_mask=dense)
    o, l = _f64(out), lse.cpu().numpy().astype(np.float64)
    _check_out(o, l, ro, rl)
    ref = R.attention_bwd_f64(_f64(do), _f64(q), _f64(k), _f64(v), o, l, km, attn_mask=dense)
    _check_grads(grads, ref, R.attention_bwd_magnitudes_f64(_f64(do), _f64(q), _f64(k), _f64(v), o, l, km,
                                                           attn_mask=dense))
    reached = dense.any(axis=1)  # (rows, Lk): keys some query's window holds
    if km is not None:
        reached = reached & km
    gone = np.broadcast_to(~reached[:, None, :, None], grads[1].shape)
    assert np.all(_f64(grads[1])[gone] == 0) and np.all(_f64(grads[2])[gone] == 0)


@pytest.mark.parametrize("seed", range(12))
def test_fp8_random_shapes_match_oracle(amd, seed):
    rng = np.random.default_rng(3000 + seed)
    c = _shape(rng)
    q, k, v, _, mask = _tensors(c, seed)
    print(f"fp8 sweep seed={seed} {c}", flush=True)
    qs, ks = R.fp8_absmax_scale(q.float().numpy()), R.fp8_absmax_scale(k.float().numpy())
    out, lse = amd.ops.flash_fwd_fp8(q.cuda(), k.cuda(), v.cuda(), None if mask is None else mask.cuda(),
                                     torch.from_numpy(qs).cuda(), torch.from_numpy(ks).cuda(), c["D"] ** -0.5)
    ro, rl = R.attention_fp8_f64(q.float().numpy(), k.float().numpy(), v.float().numpy(), qs, ks,
                                 None if mask is None else mask.numpy())
    _check_out(_f64(out), lse.cpu().numpy().astype(np.float64), ro, rl, lse_rel=2.0**-14)


def _coords(frames, height, width, batch):
    t = torch.arange(frames, dtype=torch.float32) / 8.0
    r = torch.arange(height, dtype=torch.float32) * 2.0
    c = torch.arange(width, dtype=torch.float32) * 2.0
    g = torch.stack(torch.meshgrid(t, r, c, indexing="ij"), -1).reshape(1, -1, 3)
    return g.expand(batch, -1, -1).contiguous()


def _ring_run(amd, q, k, v, do, cp, mask, tq=None, tk=None, fused=False):
    qg, kg, vg = (t.clone().requires_grad_(True) for t in (q, k, v))
    if tq is None:
        out, lse = amd.ring.ring_attention(qg, kg, vg, cp=cp, key_mask=mask)
    elif fused:
        out, lse = amd.ring.ring_attention(qg, kg, vg, cp=cp, key_mask=mask, tables_q=tq, tables_k=tk)
    else:
        out, lse = amd.ring.ring_attention(amd.rope.apply_rotary(qg, tq), amd.rope.apply_rotary(kg, tk), vg,
                                           cp=cp, key_mask=mask)
    out.backward(do)
    torch.cuda.synchronize()
    return out.detach(), lse.detach(), qg.grad, kg.grad, vg.grad


@pytest.mark.parametrize("seed", range(12))
def test_ring_random_shapes_match_oracle(amd, seed):
    rng = np.random.default_rng(4000 + seed)
    c = _shape(rng)
    cp = int(rng.integers(1, 5))
    # key grid (frames, rows, cols) whose length splits into cp equal chunks
    F, H, W = int(rng.integers(1, 5)), int(rng.integers(1, 9)), int(rng.integers(1, 21))
    Lk = cp * F * H * W
    c["Lq"] = min(c["Lq"], Lk)  # the query shard is a prefix of the key positions
    rope = bool(rng.integers(0, 2))
    q, k, v, do, mask = _tensors(c, seed, Lk=Lk)
    print(f"ring sweep seed={seed} {c} cp={cp} grid={(cp * F, H, W)} Lk={Lk} rope={rope}", flush=True)
    B, Lq, D = c["B"], c["Lq"], c["D"]
    qc, kc, vc, dc = q.cuda(), k.cuda(), v.cuda(), do.cuda()
    mk = None if mask is None else mask.cuda()
    if rope:
        tables = amd.rope.build_rotary_tables(_coords(cp * F, H, W, B).cuda(), head_dim=D)
        tq = tables.slice(0, Lq)
        fu = _ring_run(amd, qc, kc, vc, dc, cp, mk, tq, tables, fused=True)
        un = _ring_run(amd, qc, kc, vc, dc, cp, mk, tq, tables, fused=False)
        for name, a, b in zip(("out", "lse", "dq", "dk", "dv"), fu, un):
            assert torch.equal(a, b), name
        qn = R.apply_rotary_bf16(q.float().numpy(), tq.cos.cpu().numpy(), tq.sin.cpu().numpy())
        kn = R.apply_rotary_bf16(k.float().numpy(), tables.cos.cpu().numpy(), tables.sin.cpu().numpy())
    else:
        fu = _ring_run(amd, qc, kc, vc, dc, cp, mk)
        qn, kn = q.float().numpy(), k.float().numpy()
    vn = v.float().numpy()
    km = None if mask is None else mask.numpy()
    bounds = [R.shard_bounds(Lk, cp, r) for r in range(cp)]
    ro, rl = R.ring_forward_f64(qn, [kn[:, :, a:b] for a, b in bounds], [vn[:, :, a:b] for a, b in bounds],
                                None if km is None else [km[:, a:b] for a, b in bounds])
    o, l = _f64(fu[0]), fu[1].cpu().numpy().astype(np.float64)
    _check_out(o, l, ro, rl)
    if not rope:
        # without rotation the ring's gradients are plain attention's over the whole key sequence
        args = (_f64(do), qn.astype(np.float64), kn.astype(np.float64), vn.astype(np.float64), o, l, km)
        _check_grads(fu[2:], R.attention_bwd_f64(*args), R.attention_bwd_magnitudes_f64(*args))


@pytest.mark.parametrize("seed", range(10))
def test_f32_random_shapes_match_oracle(amd, seed):
    """The float32 path on random shapes at float32's bar: output 2e-5 of
    max(1, |out|), LSE 2e-5 of max(1, |lse|), gradients 1e-4 of their
    largest magnitude."""
    rng = np.random.default_rng(5000 + seed)
    c = _shape(rng)
    g = torch.Generator()
    g.manual_seed(seed)
    B, Hq, Hkv, Lq, Lk, D = c["B"], c["Hq"], c["Hkv"], c["Lq"], c["Lk"], c["D"]
    q, k, v, do = (torch.randn(s, generator=g) * c["scale"]
                   for s in ((B, Hq, Lq, D), (B, Hkv, Lk, D), (B, Hkv, Lk, D), (B, Hq, Lq, D)))
    mask = None
    if c["masked"]:
        mask = torch.rand((B, Lk), generator=g) < 0.8
        mask[0, : max(1, Lk // 3)] = True
        if B > 1:
            mask[-1] = False
    print(f"f32 sweep seed={seed} {c}", flush=True)
    mk = None if mask is None else mask.cuda()
    out, lse = amd.ops.flash_fwd(q.cuda(), k.cuda(), v.cuda(), mk, None, None, D ** -0.5)
    dq, dk, dv = amd.ops.flash_bwd(do.cuda(), q.cuda(), k.cuda(), v.cuda(), out, lse, mk, D ** -0.5)
    km = None if mask is None else mask.numpy()
    ro, rl = R.attention_f64(_f64(q), _f64(k), _f64(v), km)
    o, l = _f64(out), lse.cpu().numpy().astype(np.float64)
    assert np.abs(o - ro).max() <= 2e-5 * max(1.0, np.abs(ro).max())
    fin = np.isfinite(rl)
    assert np.array_equal(np.isneginf(l), ~fin)
    assert (np.abs(l[fin] - rl[fin]) <= 2e-5 * np.maximum(1.0, np.abs(rl[fin]))).all()
    args = (_f64(do), _f64(q), _f64(k), _f64(v), o, l, km)
    _check_grads((dq, dk, dv), R.attention_bwd_f64(*args), R.attention_bwd_magnitudes_f64(*args), rel=1e-4,
                 floor=1e-6)


@pytest.mark.parametrize("seed", range(10))
def test_f32_windowed_random_shapes_match_oracle(amd, seed):
    """float32 with random per-row key windows at float32's bar: the
    backward (staged dS or recomputed dq) on non-decreasing windows, the
    forward also on the same windows shuffled across rows (it takes any)."""
    rng = np.random.default_rng(6000 + seed)
    c = _shape(rng)
    per_batch, staged = bool(rng.integers(0, 2)), bool(rng.integers(0, 2))
    B, Hq, Hkv, Lq, Lk, D = c["B"], c["Hq"], c["Hkv"], c["Lq"], c["Lk"], c["D"]
    lo, hi = _windows(rng, B if per_batch else 1, Lq, Lk)
    g = torch.Generator()
    g.manual_seed(seed)
    q, k, v, do = (torch.randn(s, generator=g) * c["scale"]
                   for s in ((B, Hq, Lq, D), (B, Hkv, Lk, D), (B, Hkv, Lk, D), (B, Hq, Lq, D)))
    mask = (torch.rand((B, Lk), generator=g) < 0.8) if c["masked"] else None
    print(f"f32 windowed sweep seed={seed} {c} per_batch={per_batch} staged={staged}", flush=True)
    dev = torch.device("cuda", 0)
    mk = None if mask is None else mask.cuda()
    km = None if mask is None else mask.numpy()
    j = np.arange(Lk)

    def run_fwd(lo_np, hi_np):
        lo_t, hi_t = torch.from_numpy(lo_np).cuda(), torch.from_numpy(hi_np).cuda()
        if not per_batch:
            lo_t, hi_t = lo_t[0], hi_t[0]
        out, lse = amd.ops.flash_fwd_windowed(q.cuda(), k.cuda(), v.cuda(), lo_t, hi_t, mk, D ** -0.5)
        dense = (j >= lo_np[..., None]) & (j < hi_np[..., None])
        ro, rl = R.attention_f64(_f64(q), _f64(k), _f64(v), km, attn_mask=dense)
        o, l = _f64(out), lse.cpu().numpy().astype(np.float64)
        assert np.abs(o - ro).max() <= 2e-5 * max(1.0, np.abs(ro).max())
        fin = np.isfinite(rl)
        assert np.array_equal(np.isneginf(l), ~fin)
        assert (np.abs(l[fin] - rl[fin]) <= 2e-5 * np.maximum(1.0, np.abs(rl[fin]))).all()
        return out, lse, lo_t, hi_t, dense, o, l

    perm = rng.permutation(Lq)
    run_fwd(np.ascontiguousarray(lo[:, perm]), np.ascontiguousarray(hi[:, perm]))
    out, lse, lo_t, hi_t, dense, o, l = run_fwd(lo, hi)
    amd.ops.set_ds_budget(None if staged else 0, dev)
    try:
        grads = amd.ops.flash_bwd_windowed(do.cuda(), q.cuda(), k.cuda(), v.cuda(), out, lse, lo_t, hi_t, mk,
                                           D ** -0.5)
    finally:
        amd.ops.set_ds_budget(None, dev)
    args = (_f64(do), _f64(q), _f64(k), _f64(v), o, l, km)
    _check_grads(grads, R.attention_bwd_f64(*args, attn_mask=dense),
                 R.attention_bwd_magnitudes_f64(*args, attn_mask=dense), rel=1e-4, floor=1e-6)
    reached = dense.any(axis=1)
    if km is not None:
        reached = reached & km
    gone = np.broadcast_to(~reached[:, None, :, None], grads[1].shape)
    assert np.all(_f64(grads[1])[gone] == 0) and np.all(_f64(grads[2])[gone] == 0)
