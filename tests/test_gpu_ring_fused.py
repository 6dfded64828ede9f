"""GPU tests of the fused ring step (RoPE + forward + merge in one launch per
chunk, RoPE folded into the backward's copies and epilogues), of non-finite
propagation through the ring, and of BASELINE config c1.

The fused path must give the SAME BITS as the unfused composition it
replaces: apply_rotary on q and k (src/avgen/models/rope.py:297-338), the
ring's per-chunk op and merge (torch/.../_context_parallel/_attention.py
:182-183, :468-474, :567-575) and autograd through the rotation.  Against
the CPU oracle the bar is the usual one: output max-abs <= 2e-2, LSE <= 1e-3,
gradients <= 2e-2 x max |reference|.
"""

from __future__ import annotations

import math

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


def _rand(shape, seed, scale, device="cuda"):
    g = torch.Generator()
    g.manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16).to(device)


def _coords(frames, height, width, batch):
    t = torch.arange(frames, dtype=torch.float32) / 8.0
    r = torch.arange(height, dtype=torch.float32) * 2.0
    c = torch.arange(width, dtype=torch.float32) * 2.0
    g = torch.stack(torch.meshgrid(t, r, c, indexing="ij"), -1).reshape(1, -1, 3)
    return g.expand(batch, -1, -1).contiguous()


def _run(amd, q, k, v, do, cp, mask, tq, tk, fused):
    qg, kg, vg = (t.clone().requires_grad_(True) for t in (q, k, v))
    if fused:
        out, lse = amd.ring.ring_attention(qg, kg, vg, cp=cp, key_mask=mask, tables_q=tq, tables_k=tk)
    else:
        out, lse = amd.ring.ring_attention(amd.rope.apply_rotary(qg, tq), amd.rope.apply_rotary(kg, tk), vg, cp=cp,
                                           key_mask=mask)
    out.backward(do)
    torch.cuda.synchronize()
    return out.detach(), lse.detach(), qg.grad, kg.grad, vg.grad


CASES = [
    # (B, Hq, Hkv, grid (F, H, W), Lq rows of shard 0, cp, D, masked)
    (1, 4, 4, (4, 10, 25), 250, 4, 128, False),
    (2, 4, 2, (3, 8, 16), 96, 4, 64, True),
    (1, 2, 2, (2, 9, 20), 360, 1, 128, False),
    # 2 x 4 x 35 = 280 key blocks per chunk: the dK/dV grid's last round is
    # split (partial sums, then dk rotated back in the reduction)
    (2, 4, 4, (7, 32, 40), 512, 2, 128, True),
    # 8 heads x 34 blocks of 256 query rows, 2 x 8 x 35 key blocks: a long
    # query shard (the oracle checks every 16th row)
    (1, 8, 8, (5, 40, 44), 8465, 2, 64, True),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"B{c[0]}Hq{c[1]}Hkv{c[2]}cp{c[5]}D{c[6]}m{int(c[7])}")
def test_fused_ring_bitwise_equals_unfused(amd, case):
    B, Hq, Hkv, grid, Lq, cp, D, masked = case
    L = grid[0] * grid[1] * grid[2]
    print(f"fused ring case {case}", flush=True)
    tables = amd.rope.build_rotary_tables(_coords(*grid, B).cuda(), head_dim=D)
    tq, tk = tables.slice(0, Lq), tables
    q = _rand((B, Hq, Lq, D), 1, 0.7)
    k, v = _rand((B, Hkv, L, D), 2, 0.7), _rand((B, Hkv, L, D), 3, 0.7)
    do = _rand((B, Hq, Lq, D), 4, 1.0)
    mask = None
    if masked:
        g = torch.Generator()
        g.manual_seed(5)
        mask = (torch.rand((B, L), generator=g) > 0.3).cuda()
        mask[0, : L // cp] = False  # a whole chunk without valid keys for batch 0
    fu = _run(amd, q, k, v, do, cp, mask, tq, tk, fused=True)
    un = _run(amd, q, k, v, do, cp, mask, tq, tk, fused=False)
    for name, a, b in zip(("out", "lse", "dq", "dk", "dv"), fu, un):
        assert torch.equal(a, b), name
    # and against the oracle (rotated in float32 exactly as the reference), on
    # at most ~512 query rows (rows are independent)
    step = max(1, Lq // 512)
    cq, sq = (x.cpu().numpy()[:, :, ::step] for x in (tq.cos, tq.sin))
    ck, sk = (x.cpu().numpy() for x in (tk.cos, tk.sin))
    qr = R.apply_rotary_bf16(q.float().cpu().numpy()[:, :, ::step], cq, sq)
    kr = R.apply_rotary_bf16(k.float().cpu().numpy(), ck, sk)
    vv = v.float().cpu().numpy()
    bounds = [R.shard_bounds(L, cp, r) for r in range(cp)]
    mk = None if mask is None else mask.cpu().numpy()
    ro, rl = R.ring_forward_f64(qr, [kr[:, :, a:b] for a, b in bounds], [vv[:, :, a:b] for a, b in bounds],
                                None if mk is None else [mk[:, a:b] for a, b in bounds])
    assert np.abs(fu[0].float().cpu().numpy()[:, :, ::step] - ro).max() <= OUT_TOL
    assert np.abs(fu[1].cpu().numpy()[:, :, ::step] - rl).max() <= LSE_TOL


def test_ring_nan_in_one_key_row_of_chunk_2(amd):
    """A NaN in one key row of chunk 2 of a 4-chunk ring makes every query row
    of that head NaN (out and lse), as torch's SDPA and merge give; a NaN in
    one query row poisons only that row.  Checked through the fused ring and
    through the per-chunk op + separate merge kernel."""
    B, H, Lq, L, D, cp = 1, 2, 256, 1024, 128, 4
    q = _rand((B, H, Lq, D), 11, 0.7)
    k, v = _rand((B, H, L, D), 12, 0.7), _rand((B, H, L, D), 13, 0.7)
    k[0, 0, 2 * (L // cp) + 17] = float("nan")
    q[0, 1, 5, 3] = float("nan")
    print("ring NaN propagation", flush=True)
    out_f, lse_f = amd.ring.ring_attention(q, k, v, cp=cp)  # per-chunk op + lse_merge kernel
    bounds = [R.shard_bounds(L, cp, r) for r in range(cp)]
    ones = amd.rope.build_rotary_tables(torch.zeros(B, L, 3, device="cuda"), head_dim=D)  # identity rotation
    out_u, lse_u = amd.ring.ring_attention(q, k, v, cp=cp, tables_q=ones.slice(0, Lq), tables_k=ones)
    torch.cuda.synchronize()
    ro, rl = R.ring_forward_f64(*(t.float().cpu().numpy() for t in (q,)),
                                [k.float().cpu().numpy()[:, :, a:b] for a, b in bounds],
                                [v.float().cpu().numpy()[:, :, a:b] for a, b in bounds])
    for out, lse in ((out_f, lse_f), (out_u, lse_u)):
        o, l = out.float().cpu().numpy(), lse.cpu().numpy()
        assert np.isnan(o[0, 0]).all() and np.isnan(l[0, 0]).all()
        assert np.array_equal(np.isnan(o), np.isnan(ro)) and np.array_equal(np.isnan(l), np.isnan(rl))
        assert np.isnan(o[0, 1, 5]).all() and np.isnan(l[0, 1, 5])
        fin = ~np.isnan(ro)
        assert np.abs(o[fin] - ro[fin]).max() <= OUT_TOL
        assert np.abs(l[~np.isnan(rl)] - rl[~np.isnan(rl)]).max() <= LSE_TOL
    # an all-masked row is still 0 / -inf, not NaN
    m = torch.ones(B, L, dtype=torch.bool, device="cuda")
    m[:, :] = False
    out0, lse0 = amd.ops.flash_fwd(q[:, :, :, :].clone().nan_to_num_(0.0), k.nan_to_num(0.0), v, m, None, None,
                                   D ** -0.5)
    assert (out0 == 0).all() and torch.isneginf(lse0).all()


# The forward kernel's own error on bf16 inputs (test_c1_cpu_smoke_config).
KERNEL_OUT_TOL = 5e-3
KERNEL_LSE_TOL = 5e-5


def test_c1_cpu_smoke_config(amd):
    """BASELINE config c1: one non-chunked self-attention, B=1, 4 heads,
    head_dim 64, a 4x16x16 latent (1,024 tokens), N(0,1) inputs, 3D RoPE
    theta 1e4 with the head_dim-64 split rope_axis_pairs(64) = (12, 10, 10)
    (the config's 22/21/21 is the head_dim-128 split), no mask, forward out +
    LSE.  The config's tensors are float32 (run as such on the fp32 path by
    tests/test_gpu_f32.py::test_c1_config_in_float32); here they are cast to
    bf16 for the bf16 kernels, whose own error is bounded separately from
    the cast's.  (1)
    Against the float64 oracle of the bf16-cast inputs, the kernel's
    arithmetic alone: bf16 probabilities into the P V product and one bf16
    rounding of the output (half an ulp: 3.9e-3 for |out| in [1, 2)), an fp32
    LSE: out <= KERNEL_OUT_TOL, LSE <= KERNEL_LSE_TOL, four and twenty times
    tighter than the bf16 bar, so a kernel error well below that bar trips
    it.  (2) Against the float32 config itself (float64 rotation of the
    float32 inputs): the cast alone moves the LSE by ~2.5e-3 at these N(0,1)
    inputs, and the kernel may add no more than its own bound (1) on top."""
    B, H, D, grid = 1, 4, 64, (4, 16, 16)
    L = grid[0] * grid[1] * grid[2]
    assert R.rope_axis_pairs(D) == (12, 10, 10)
    g = torch.Generator()
    g.manual_seed(0)
    q32, k32, v32 = (torch.randn((B, H, L, D), generator=g) for _ in range(3))
    coords = _coords(*grid, B)
    tables = amd.rope.build_rotary_tables(coords.cuda(), head_dim=D)
    q, k, v = (t.to(torch.bfloat16).cuda() for t in (q32, k32, v32))
    out, lse = amd.ops.flash_fwd(q, amd.rope.apply_rotary(k, tables), v, None, tables.cos, tables.sin, D ** -0.5)
    torch.cuda.synchronize()
    o, l = out.float().cpu().numpy(), lse.cpu().numpy()
    # (1) the oracle on the bf16-cast inputs, rotated as the reference rotates bf16 tensors
    cos, sin = (x.cpu().numpy() for x in (tables.cos, tables.sin))
    qr = R.apply_rotary_bf16(q.float().cpu().numpy(), cos, sin)
    kr = R.apply_rotary_bf16(k.float().cpu().numpy(), cos, sin)
    ro, rl = R.attention_f64(qr, kr, v.float().cpu().numpy())
    k_o, k_l = np.abs(o - ro).max(), np.abs(l - rl).max()
    print(f"c1 kernel vs oracle on the bf16-cast inputs: out {k_o:.2e} lse {k_l:.2e}", flush=True)
    assert k_o <= KERNEL_OUT_TOL and k_l <= KERNEL_LSE_TOL
    # (2) the float32 config itself: float64 rotation of the float32 inputs
    c64, s64 = R.rotary_tables_f64(coords.numpy(), D)

    def rot64(x):
        x = x.numpy().astype(np.float64)
        e, od = x[..., 0::2], x[..., 1::2]
        y = np.empty_like(x)
        y[..., 0::2] = e * c64 - od * s64
        y[..., 1::2] = e * s64 + od * c64
        return y

    fo, fl = R.attention_f64(rot64(q32), rot64(k32), v32.numpy().astype(np.float64))
    err_o, err_l = np.abs(o - fo).max(), np.abs(l - fl).max()
    cast_o, cast_l = np.abs(ro - fo).max(), np.abs(rl - fl).max()  # what the bf16 cast alone does
    print(f"c1 vs float32 config: kernel out {err_o:.2e} lse {err_l:.2e}; bf16 cast alone out {cast_o:.2e} "
          f"lse {cast_l:.2e}", flush=True)
    assert err_o <= cast_o + KERNEL_OUT_TOL and err_l <= cast_l + KERNEL_LSE_TOL
