"""Run-to-run bit reproducibility on the GPU: the kernels use no atomics and
fixed reduction orders (the dK/dV tail split sums its fp32 partials in part
order, dQ from staged dS sums key blocks in order), so the same call on the
same inputs, budget and device gives the same bits every time.  Each case
runs twice, with other work in between, and compares every output with
torch.equal: the plain forward and backward (staged dS in one pass, in
passes of one (batch, kv head) pair, and the recomputing dQ; a shape whose
dK/dV grid has a split last round), the windowed backward with the compact
dS layout, the fp8 forward and the RoPE-fused ring."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def amd():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    import avgen_amd

    return avgen_amd


def _rand(shape, seed, scale=0.7):
    g = torch.Generator()
    g.manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16).cuda()


def _churn():
    """Unrelated device work between the two runs (other allocations, other
    values in the caching allocator's blocks)."""
    x = torch.randn(1 << 22, device="cuda")
    (x * 3).sum().item()


def _same(a, b, names):
    for n, x, y in zip(names, a, b):
        assert torch.equal(x, y), n


@pytest.mark.parametrize("budget", ["one_pass", "one_pair", "recompute"])
def test_plain_fwd_bwd_bits_repeat(amd, budget):
    # 3 batch rows x 2 kv heads x 60 key blocks = 360 dK/dV workgroups: the
    # last round on 256 CUs is split over query-tile ranges
    B, Hq, Hkv, L, D = 3, 4, 2, 7600, 128
    q, k, v, do = _rand((B, Hq, L, D), 1), _rand((B, Hkv, L, D), 2), _rand((B, Hkv, L, D), 3), _rand((B, Hq, L, D), 4)
    mask = torch.ones(B, L, dtype=torch.bool, device="cuda")
    mask[1, 5000:] = False
    dev = torch.device("cuda", 0)
    nbytes = {"one_pass": None, "one_pair": 1, "recompute": 0}[budget]
    print(f"determinism plain budget={budget}", flush=True)
    ops = amd.ops

    def run():
        ops.set_ds_budget(nbytes, dev)
        try:
            out, lse = ops.flash_fwd(q, k, v, mask, None, None, D ** -0.5)
            dq, dk, dv = ops.flash_bwd(do, q, k, v, out, lse, mask, D ** -0.5)
        finally:
            ops.set_ds_budget(None, dev)
        torch.cuda.synchronize()
        return out, lse, dq, dk, dv

    first = run()
    _churn()
    _same(first, run(), ("out", "lse", "dq", "dk", "dv"))


def test_windowed_compact_bits_repeat(amd):
    B, H, L, D = 2, 4, 3000, 128
    q, k, v, do = (_rand((B, H, L, D), s) for s in (5, 6, 7, 8))
    t = torch.arange(L, device="cuda") // 150  # 20 "frames" of 150 tokens
    lo = torch.searchsorted(t, t - 2, right=False).to(torch.int32)
    hi = torch.searchsorted(t, t + 2, right=True).to(torch.int32)
    print("determinism windowed", flush=True)
    ops = amd.ops

    def run():
        out, lse = ops.flash_fwd_windowed(q, k, v, lo, hi, None, D ** -0.5)
        grads = ops.flash_bwd_windowed(do, q, k, v, out, lse, lo, hi, None, D ** -0.5)
        torch.cuda.synchronize()
        return (out, lse, *grads)

    first = run()
    _churn()
    _same(first, run(), ("out", "lse", "dq", "dk", "dv"))


def test_fp8_forward_bits_repeat(amd):
    B, H, L, D = 2, 4, 4000, 128
    q, k, v = (_rand((B, H, L, D), s) for s in (9, 10, 11))
    qs, ks = amd.ops.fp8_absmax_scales(q), amd.ops.fp8_absmax_scales(k)
    print("determinism fp8", flush=True)

    def run():
        r = amd.ops.flash_fwd_fp8(q, k, v, None, qs, ks, D ** -0.5)
        torch.cuda.synchronize()
        return r

    first = run()
    _churn()
    _same(first, run(), ("out", "lse"))


def test_fused_ring_bits_repeat(amd):
    B, H, D, cp = 1, 4, 128, 4
    F, Hh, W = 8, 16, 20
    L = F * Hh * W
    t = torch.arange(F, dtype=torch.float32) / 8.0
    r = torch.arange(Hh, dtype=torch.float32) * 2.0
    c = torch.arange(W, dtype=torch.float32) * 2.0
    coords = torch.stack(torch.meshgrid(t, r, c, indexing="ij"), -1).reshape(1, L, 3).cuda()
    tables = amd.rope.build_rotary_tables(coords, head_dim=D)
    Lq = L // cp
    tq = tables.slice(0, Lq)
    q, k, v, do = _rand((B, H, Lq, D), 12), _rand((B, H, L, D), 13), _rand((B, H, L, D), 14), _rand((B, H, Lq, D), 15)
    print("determinism fused ring", flush=True)

    def run():
        qg, kg, vg = (x.clone().requires_grad_(True) for x in (q, k, v))
        out, lse = amd.ring.ring_attention(qg, kg, vg, cp=cp, tables_q=tq, tables_k=tables)
        out.backward(do)
        torch.cuda.synchronize()
        return out.detach(), lse.detach(), qg.grad, kg.grad, vg.grad

    first = run()
    _churn()
    _same(first, run(), ("out", "lse", "dq", "dk", "dv"))
