"""GPU parity of the per-row key-window kernels (forward, dK/dV with staged
dS, dQ from dS) against the float64 oracle with the equivalent dense mask,
and of the attention-level entry points built on them: packed
variable-length sequences (src/avgen/data/packing.py:181-200) and the
temporal neighbour mask (src/avgen/models/blocks.py:54-104).

Tolerances as for the unwindowed kernels: output max-abs <= 2e-2, LSE <=
1e-3, gradients 2e-2 of the largest reference magnitude; keys outside every
window get exactly zero dK/dV; rows with no admissible key give exactly zero
output and LSE -inf.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reference as R

pytestmark = pytest.mark.gpu

OUT_TOL = 2e-2
LSE_TOL = 1e-3
GRAD_REL_TOL = 2e-2


@pytest.fixture(scope="module")
def amd():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    import avgen_amd

    return avgen_amd


def _randn(shape, seed):
    g = torch.Generator()
    g.manual_seed(seed)
    return torch.randn(shape, generator=g).to(torch.bfloat16)


def _f64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


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


def _check_fwd(out, lse, ro, rl):
    o, l = _f64(out), lse.detach().cpu().numpy().astype(np.float64)
    assert np.isfinite(o).all()
    err = np.abs(o - ro).max()
    fin = np.isfinite(rl)
    assert (np.isneginf(l) == ~fin).all(), "rows without keys must give lse = -inf"
    assert (o[~fin] == 0).all(), "rows without keys must give zeros"
    lerr = np.abs(l[fin] - rl[fin]).max() if fin.any() else 0.0
    print(f"  out err {err:.3e}  lse err {lerr:.3e}", flush=True)
    assert err <= OUT_TOL and lerr <= LSE_TOL


def _check_grads(got, ref):
    for name, g, r in zip(("dq", "dk", "dv"), got, ref):
        g = _f64(g)
        assert np.isfinite(g).all(), name
        err = np.abs(g - r).max()
        scale = max(np.abs(r).max(), 1e-3)
        print(f"  {name}: max err {err:.3e} (ref max {scale:.3e})", flush=True)
        assert err <= GRAD_REL_TOL * scale, name


WIN_CASES = [
    # B, Hq, Hkv, Lq, Lk, D, max_width, empty_tail, per_batch
    (1, 2, 2, 256, 256, 128, 64, 0, False),
    (2, 4, 2, 300, 333, 128, 100, 37, True),
    (1, 2, 1, 517, 1100, 64, 300, 0, False),
    (2, 2, 2, 130, 70, 128, 5, 3, True),
    (1, 2, 2, 640, 640, 128, 1, 0, False),
]


@pytest.mark.parametrize("B,Hq,Hkv,Lq,Lk,D,width,tail,per_batch", WIN_CASES)
@pytest.mark.parametrize("masked", [False, True])
def test_windowed_forward_backward_match_oracle(amd, B, Hq, Hkv, Lq, Lk, D, width, tail, per_batch, masked):
    print(f"windowed case B={B} Hq={Hq} Hkv={Hkv} Lq={Lq} Lk={Lk} D={D} width={width} tail={tail} "
          f"per_batch={per_batch} masked={masked}", flush=True)
    q, k, v = _randn((B, Hq, Lq, D), 1), _randn((B, Hkv, Lk, D), 2), _randn((B, Hkv, Lk, D), 3)
    do = _randn((B, Hq, Lq, D), 4)
    lo, hi = _monotone_windows(B if per_batch else 1, Lq, Lk, 5, width, tail)
    km = None
    if masked:
        rng = np.random.default_rng(6)
        km = rng.random((B, Lk)) < 0.8
    lo_t, hi_t = torch.from_numpy(lo).cuda(), torch.from_numpy(hi).cuda()
    if not per_batch:
        lo_t, hi_t = lo_t[0], hi_t[0]
    kmc = None if km is None else torch.from_numpy(km).cuda()
    scale = D ** -0.5
    out, lse = amd.ops.flash_fwd_windowed(q.cuda(), k.cuda(), v.cuda(), lo_t, hi_t, kmc, scale)
    dense = _window_mask(lo, hi, Lk)  # (B|1, Lq, Lk)
    ro, rl = R.attention_f64(_f64(q), _f64(k), _f64(v), km, attn_mask=dense)
    _check_fwd(out, lse, ro, rl)
    grads = amd.ops.flash_bwd_windowed(do.cuda(), q.cuda(), k.cuda(), v.cuda(), out, lse, lo_t, hi_t, kmc, scale)
    rq, rk, rv = R.attention_bwd_f64(_f64(do), _f64(q), _f64(k), _f64(v), ro, rl, km, attn_mask=dense)
    _check_grads(grads, (rq, rk, rv))
    # keys no window reaches: exactly zero dK/dV
    reached = dense.any(axis=-2)  # (B|1, Lk)
    reached = np.broadcast_to(reached, (B, Lk))
    for g in grads[1:]:
        gz = g.float().cpu().numpy()
        for b in range(B):
            assert (gz[b][:, ~reached[b]] == 0).all()


def test_windowed_forward_accepts_any_windows(amd):
    """The forward takes windows in any order (the backward needs them
    non-decreasing and says so)."""
    B, H, Lq, Lk, D = 1, 2, 400, 700, 128
    q, k, v = _randn((B, H, Lq, D), 11), _randn((B, H, Lk, D), 12), _randn((B, H, Lk, D), 13)
    rng = np.random.default_rng(14)
    a, b = rng.integers(0, Lk + 1, (2, Lq))
    lo, hi = np.minimum(a, b).astype(np.int32), np.maximum(a, b).astype(np.int32)
    lo_t, hi_t = torch.from_numpy(lo).cuda(), torch.from_numpy(hi).cuda()
    out, lse = amd.ops.flash_fwd_windowed(q.cuda(), k.cuda(), v.cuda(), lo_t, hi_t, None, D ** -0.5)
    ro, rl = R.attention_f64(_f64(q), _f64(k), _f64(v), attn_mask=_window_mask(lo, hi, Lk)[None])
    _check_fwd(out, lse, ro, rl)
    with pytest.raises(ValueError, match="non-decreasing"):
        amd.ops.flash_bwd_windowed(q.cuda(), q.cuda(), k.cuda(), v.cuda(), out, lse, lo_t, hi_t, None, D ** -0.5)


def test_nan_key_reaches_only_workgroups_that_visit_its_tile(amd):
    """The documented deviation from the dense-mask reference, whose additive
    -inf mask turns a NaN score into NaN on every row: the windowed forward
    visits, per 256-row workgroup, only the 64-key tiles its rows' windows
    meet, so a NaN key row reaches the output rows of the workgroups that
    visit its tile (through a window holding the key, or 0 x NaN in P V for
    rows whose window excludes it) and the LSE of the rows whose window holds
    it, and nothing else, which equals the run with that key zeroed."""
    B, H, Lq, Lk, D = 1, 2, 1300, 2000, 128
    q, k, v = _randn((B, H, Lq, D), 31), _randn((B, H, Lk, D), 32), _randn((B, H, Lk, D), 33)
    rows = np.arange(Lq)
    lo = np.minimum(rows * Lk // Lq, Lk).astype(np.int32)
    hi = np.minimum(lo + 150, Lk).astype(np.int32)
    j = 1033
    kz, vz = k.clone(), v.clone()
    kz[:, :, j], vz[:, :, j] = 0, 0
    kn, vn = kz.clone(), vz.clone()
    kn[:, :, j], vn[:, :, j] = float("nan"), float("nan")
    lo_t, hi_t = torch.from_numpy(lo).cuda(), torch.from_numpy(hi).cuda()
    print("window NaN key", flush=True)
    o_n, l_n = amd.ops.flash_fwd_windowed(q.cuda(), kn.cuda(), vn.cuda(), lo_t, hi_t, None, D ** -0.5)
    o_z, l_z = amd.ops.flash_fwd_windowed(q.cuda(), kz.cuda(), vz.cuda(), lo_t, hi_t, None, D ** -0.5)
    # workgroups of 256 rows: tiles [lo(first) // 64, ceil(hi(last) / 64))
    reach = np.zeros(Lq, dtype=bool)
    for r0 in range(0, Lq, 256):
        r1 = min(r0 + 256, Lq)
        if lo[r0] // 64 <= j // 64 < (hi[r1 - 1] + 63) // 64:
            reach[r0:r1] = True
    assert reach.any() and (~reach).any()
    reach_t = torch.from_numpy(reach).cuda()
    holds = torch.from_numpy((lo <= j) & (j < hi)).cuda()
    assert torch.isnan(o_n[:, :, reach_t]).all()
    # the LSE (no P V product) is NaN exactly on the rows whose window holds the key
    assert torch.equal(torch.isnan(l_n[0]), holds[None].expand(H, Lq))
    assert torch.equal(l_n[:, :, ~holds], l_z[:, :, ~holds])
    assert torch.equal(o_n[:, :, ~reach_t], o_z[:, :, ~reach_t])


def test_full_windows_equal_the_unwindowed_kernel(amd):
    """Windows [0, Lk) on every row: the windowed forward is the plain one."""
    B, Hq, Hkv, Lq, Lk, D = 1, 8, 8, 4096, 4096, 128
    q, k, v = _randn((B, Hq, Lq, D), 21).cuda(), _randn((B, Hkv, Lk, D), 22).cuda(), _randn((B, Hkv, Lk, D), 23).cuda()
    lo = torch.zeros(Lq, dtype=torch.int32, device="cuda")
    hi = torch.full((Lq,), Lk, dtype=torch.int32, device="cuda")
    o1, l1 = amd.ops.flash_fwd_windowed(q, k, v, lo, hi, None, D ** -0.5)
    o0, l0 = amd.ops.flash_fwd(q, k, v, None, None, None, D ** -0.5)
    assert (o1.float() - o0.float()).abs().max().item() <= 1e-2
    assert (l1 - l0).abs().max().item() <= 1e-4


@pytest.mark.parametrize("lengths,capacity,H,D", [([3, 4, 2], 12, 2, 128), ([700, 129, 64, 1000], 2048, 4, 128),
                                                  ([333, 333], 700, 2, 64)])
def test_varlen_attention_matches_the_packed_mask(amd, lengths, capacity, H, D):
    print(f"varlen case lengths={lengths} capacity={capacity}", flush=True)
    q, k, v = (_randn((1, H, capacity, D), s).cuda().requires_grad_(True) for s in (31, 32, 33))
    do = _randn((1, H, capacity, D), 34)
    cu = torch.tensor(R.packed_cu_seqlens(lengths))
    out = amd.attention.varlen_attention(q, k, v, cu)
    dense = R.packed_attention_mask(lengths, capacity)[None]
    ro, rl = R.attention_f64(_f64(q), _f64(k), _f64(v), attn_mask=dense)
    o = _f64(out)
    assert np.abs(o - ro).max() <= OUT_TOL
    pad = np.arange(capacity) >= sum(lengths)
    assert (o[:, :, pad] == 0).all()
    out.backward(do.cuda())
    rq, rk, rv = R.attention_bwd_f64(_f64(do), _f64(q), _f64(k), _f64(v), ro, rl, attn_mask=dense)
    _check_grads((q.grad, k.grad, v.grad), (rq, rk, rv))
    for g in (k.grad, v.grad):
        assert (g[:, :, torch.from_numpy(pad).cuda()] == 0).all()


def _times(n, rate, per_step, start=0.0):
    return (start + (np.arange(n) // per_step) / rate).astype(np.float32)


@pytest.mark.parametrize("order", ["sorted", "shuffled"])
@pytest.mark.parametrize("masked", [False, True])
def test_temporal_neighbour_attention_matches_the_dense_mask(amd, order, masked):
    """Video queries (frames of 48 tokens at 24 fps) against audio keys (43
    tokens per second), a window of 0.1 s; the video runs past the audio so
    the last frames have no key in range and fall back to every key."""
    B, Hq, Hkv, D = 2, 4, 2, 128
    tq = np.stack([_times(960, 24.0, 48), _times(960, 24.0, 48, 0.05)])
    tk = np.stack([_times(300, 43.0, 1), _times(300, 43.0, 1, 0.2)])[:, :260]
    Lq, Lk = tq.shape[1], tk.shape[1]
    rng = np.random.default_rng(41)
    km = (rng.random((B, Lk)) < 0.7) if masked else None
    if order == "shuffled":
        pq, pk = rng.permutation(Lq), rng.permutation(Lk)
        tq, tk = tq[:, pq], tk[:, pk]
    print(f"temporal case order={order} masked={masked}", flush=True)
    q = _randn((B, Hq, Lq, D), 42).cuda().requires_grad_(True)
    k = _randn((B, Hkv, Lk, D), 43).cuda().requires_grad_(True)
    v = _randn((B, Hkv, Lk, D), 44).cuda().requires_grad_(True)
    do = _randn((B, Hq, Lq, D), 45)
    out = amd.attention.temporal_neighbour_attention(
        q, k, v, torch.from_numpy(tq).cuda(), torch.from_numpy(tk).cuda(), window_seconds=0.1,
        key_mask=None if km is None else torch.from_numpy(km).cuda(), enable_gqa=True)
    dense = R.temporal_neighbour_mask(tq, tk, 0.1, km)
    fallback = dense[:, 0].all(axis=-1) & ~(np.abs(tq[:, :, None] - tk[:, None, :]) <= 0.1).all(axis=-1)
    assert fallback.any(), "the case must exercise the fallback rows"
    ro, rl = R.attention_f64(_f64(q), _f64(k), _f64(v), attn_mask=dense)
    assert np.abs(_f64(out) - ro).max() <= OUT_TOL
    out.backward(do.cuda())
    rq, rk, rv = R.attention_bwd_f64(_f64(do), _f64(q), _f64(k), _f64(v), ro, rl, attn_mask=dense)
    _check_grads((q.grad, k.grad, v.grad), (rq, rk, rv))


@pytest.mark.parametrize("order", ["sorted", "shuffled"])
def test_neighbourhood_built_once_matches_per_call(amd, order):
    """A TemporalNeighbourhood built once and reused (the reference builds its
    fusion masks once per forward) gives the same bits as building it per
    call, on two different q/k/v."""
    B, H, D = 2, 2, 128
    tq = np.stack([_times(480, 24.0, 48), _times(480, 24.0, 48, 0.05)])
    tk = np.stack([_times(120, 43.0, 1), _times(120, 43.0, 1, 0.2)])
    rng = np.random.default_rng(51)
    km = rng.random((B, 120)) < 0.8
    if order == "shuffled":
        tq, tk = tq[:, rng.permutation(480)], tk[:, rng.permutation(120)]
    tqc, tkc, kmc = (torch.from_numpy(a).cuda() for a in (tq, tk, km))
    nb = amd.attention.temporal_neighbourhood(tqc, tkc, window_seconds=0.1, key_mask=kmc)
    for seed in (1, 2):
        q, k, v = _randn((B, H, 480, D), 10 * seed), _randn((B, H, 120, D), 10 * seed + 1), \
            _randn((B, H, 120, D), 10 * seed + 2)
        q, k, v = q.cuda(), k.cuda(), v.cuda()
        a = amd.attention.temporal_neighbour_attention(q, k, v, neighbourhood=nb)
        b = amd.attention.temporal_neighbour_attention(q, k, v, tqc, tkc, window_seconds=0.1, key_mask=kmc)
        assert torch.equal(a, b)
    ref, _ = R.attention_f64(_f64(q), _f64(k), _f64(v), attn_mask=R.temporal_neighbour_mask(tq, tk, 0.1, km))
    assert np.abs(_f64(a) - ref).max() <= OUT_TOL


def test_varlen_batch_of_packed_sequences(amd):
    """Two packed rows sharing one layout (cu_seqlens applies to every batch
    row), GQA, D=64."""
    B, Hq, Hkv, D, cap = 2, 4, 2, 64, 300
    lengths = [100, 57, 120]
    q = _randn((B, Hq, cap, D), 81).cuda().requires_grad_(True)
    k = _randn((B, Hkv, cap, D), 82).cuda().requires_grad_(True)
    v = _randn((B, Hkv, cap, D), 83).cuda().requires_grad_(True)
    do = _randn((B, Hq, cap, D), 84)
    out = amd.attention.varlen_attention(q, k, v, torch.tensor(R.packed_cu_seqlens(lengths)), enable_gqa=True)
    dense = R.packed_attention_mask(lengths, cap)[None]
    ro, rl = R.attention_f64(_f64(q), _f64(k), _f64(v), attn_mask=dense)
    assert np.abs(_f64(out) - ro).max() <= OUT_TOL
    out.backward(do.cuda())
    rq, rk, rv = R.attention_bwd_f64(_f64(do), _f64(q), _f64(k), _f64(v), ro, rl, attn_mask=dense)
    _check_grads((q.grad, k.grad, v.grad), (rq, rk, rv))


@pytest.mark.parametrize("B,Hq,Hkv,Lq,Lk,D,width,per_batch,masked,budget_pairs", [
    (2, 4, 2, 700, 900, 128, 300, True, True, 0),    # per-batch windows, GQA, masked
    (1, 3, 3, 1000, 1000, 64, 200, False, False, 1),  # shared windows, three passes of one pair
    (2, 2, 2, 333, 300, 128, 120, True, False, 0),   # neither length a multiple of 64 / 128
])
def test_compact_staged_ds_gives_the_dense_layouts_bits(amd, B, Hq, Hkv, Lq, Lk, D, width, per_batch, masked,
                                                        budget_pairs):
    """The windowed backward staging dS compactly (only the key blocks each
    query tile's windows admit) gives the bits of the dense layout: the same
    kernels and arithmetic, only dS lives elsewhere.  Also in passes (a
    budget of one pair) and with a key mask."""
    print(f"compact dS: B={B} Hq={Hq} Hkv={Hkv} Lq={Lq} Lk={Lk} D={D} per_batch={per_batch} masked={masked}",
          flush=True)
    lo2, hi2 = _monotone_windows(B if per_batch else 1, Lq, Lk, seed=Lq + Lk, max_width=width, empty_tail=5)
    lo, hi = (lo2, hi2) if per_batch else (lo2[0], hi2[0])
    q = _randn((B, Hq, Lq, D), 1).cuda()
    k, v = _randn((B, Hkv, Lk, D), 2).cuda(), _randn((B, Hkv, Lk, D), 3).cuda()
    do = _randn((B, Hq, Lq, D), 4).cuda()
    lo_t, hi_t = torch.from_numpy(lo).cuda(), torch.from_numpy(hi).cuda()
    mask = None
    if masked:
        g = torch.Generator().manual_seed(5)
        mask = (torch.rand((B, Lk), generator=g) > 0.1).cuda()
    scale = D ** -0.5
    out, lse = amd.ops.flash_fwd_windowed(q, k, v, lo_t, hi_t, mask, scale)
    table, units = amd.ops.compact_ds_table(lo_t, hi_t, Lq, Lk)
    dense_units = (Lq + 63) // 64 * 2 * ((Lk + 127) // 128)
    print(f"  units per head: compact {units}, dense {dense_units}", flush=True)
    assert units <= dense_units
    if budget_pairs:
        amd.ops.set_ds_budget(budget_pairs * amd.ops.ds_bytes_per_pair(Hq // Hkv, Lq, Lk, units), q.device)
    try:
        got = amd.ops._bwd_windowed_impl(do, q, k, v, out, lse, lo_t, hi_t, mask, scale, compact=True)
        ref = amd.ops._bwd_windowed_impl(do, q, k, v, out, lse, lo_t, hi_t, mask, scale, compact=False)
        torch.cuda.synchronize()
    finally:
        amd.ops.set_ds_budget(None, q.device)
    for name, a_, b_ in zip(("dq", "dk", "dv"), got, ref):
        assert torch.equal(a_, b_), name
    # and both against the oracle with the equivalent dense mask
    km = None if mask is None else mask.cpu().numpy()
    rq, rk, rv = R.attention_bwd_f64(_f64(do), _f64(q), _f64(k), _f64(v), _f64(out),
                                     lse.cpu().numpy().astype(np.float64), km,
                                     attn_mask=_window_mask(lo2, hi2, Lk))
    _check_grads(got, (rq, rk, rv))
