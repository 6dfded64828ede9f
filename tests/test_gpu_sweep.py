"""A seeded sweep of random shapes through the C ABI against the float64
oracle, forward and backward, on both dQ paths (staged dS and recompute):
batch 1-3, query heads 1-6 over 1-3 KV heads (GQA), query and key lengths
1-700 (every padding remainder of the 64-row tiles and 128-key blocks
occurs), head dims 64 and 128, input scales 0.1-4, key-padding masks with
holes and fully masked batch rows.  The bar is the kernels' usual one,
scaled with the data: output 2e-2 of max(1, its largest magnitude) (bf16
outputs of magnitude 10 carry rounding of 0.03 on their own), LSE 1e-3,
gradients 2e-2 of their largest magnitude, plus for dq and dk 2^-20 of
the size of the terms dS = P (dP - Dr) cancels (a single key makes the
true dq and dk exactly 0); masked keys get exactly zero dK/dV."""

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


def _case(seed):
    rng = np.random.default_rng(seed)
    hkv = int(rng.integers(1, 4))
    return dict(B=int(rng.integers(1, 4)), Hq=hkv * int(rng.integers(1, 3)), Hkv=hkv,
                Lq=int(rng.integers(1, 701)), Lk=int(rng.integers(1, 701)), D=int(rng.choice([64, 128])),
                scale=float(rng.choice([0.1, 0.7, 2.0, 4.0])), masked=bool(rng.integers(0, 2)),
                stage=bool(rng.integers(0, 2)))


@pytest.mark.parametrize("seed", range(24))
def test_random_shapes_match_oracle(amd, seed):
    c = _case(1000 + seed)
    B, Hq, Hkv, Lq, Lk, D = c["B"], c["Hq"], c["Hkv"], c["Lq"], c["Lk"], c["D"]
    g = torch.Generator()
    g.manual_seed(seed)
    q, k, v, do = (
        (torch.randn(shape, generator=g) * c["scale"]).to(torch.bfloat16)
        for shape in ((B, Hq, Lq, D), (B, Hkv, Lk, D), (B, Hkv, Lk, D), (B, Hq, Lq, D)))
    mask = None
    if c["masked"]:
        mask = torch.rand((B, Lk), generator=g) < 0.8
        mask[0, : max(1, Lk // 3)] = True
        if B > 1:
            mask[-1] = False  # a fully masked batch row
    print(f"sweep seed={seed} {c}", flush=True)
    ops = amd.ops
    ops.set_ds_budget(None if c["stage"] else 0, torch.device("cuda", 0))
    try:
        mk = None if mask is None else mask.cuda()
        out, lse = ops.flash_fwd(q.cuda(), k.cuda(), v.cuda(), mk, None, None, D ** -0.5)
        dq, dk, dv = ops.flash_bwd(do.cuda(), q.cuda(), k.cuda(), v.cuda(), out, lse, mk, D ** -0.5)
    finally:
        ops.set_ds_budget(None, torch.device("cuda", 0))
    f64 = lambda t: t.float().cpu().numpy().astype(np.float64)  # noqa: E731
    km = None if mask is None else mask.numpy()
    ro, rl = R.attention_f64(f64(q), f64(k), f64(v), km)
    o, l = f64(out), lse.cpu().numpy().astype(np.float64)
    assert np.abs(o - ro).max() <= OUT_TOL * max(1.0, np.abs(ro).max())
    fin = np.isfinite(rl)
    assert np.array_equal(np.isneginf(l), ~fin)
    assert np.abs(l[fin] - rl[fin]).max(initial=0.0) <= LSE_TOL
    grads = R.attention_bwd_f64(f64(do), f64(q), f64(k), f64(v), o, l, km)
    mags = (*R.attention_bwd_magnitudes_f64(f64(do), f64(q), f64(k), f64(v), o, l, km), None)
    for got, ref, mag, name in zip((dq, dk, dv), grads, mags, ("dq", "dk", "dv")):
        err = np.abs(f64(got) - ref).max()
        # dq and dk come from dS = P (dP - Dr), which cancels where one key
        # carries the row (one key: exactly 0); its rounding scales with the
        # cancelling terms: 2^-20 of their size (16 float32 ulps)
        floor = 0.0 if mag is None else 2.0**-20 * mag.max(initial=0.0)
        assert err <= GRAD_REL_TOL * max(np.abs(ref).max(), 1e-3) + floor, (name, err)
    if mask is not None:
        gone = ~mask.numpy()[:, None, :, None]
        assert np.all(f64(dk)[np.broadcast_to(gone, dk.shape)] == 0)
        assert np.all(f64(dv)[np.broadcast_to(gone, dv.shape)] == 0)
