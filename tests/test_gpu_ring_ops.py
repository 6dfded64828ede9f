"""The ring's per-chunk steps as ``torch.library`` ops.

A rank inside PyTorch's ring (torch/.../_context_parallel/_attention.py
:468-475 forward, :567-575 backward, :182-183 merge) calls
``avgen_amd::ring_fwd_step`` / ``ring_bwd_step`` / ``ring_dq_finish`` /
``lse_merge`` per chunk, and the reference compiles every block
(src/avgen/parallel/apply.py:216-221).  Checked here: the ops' schemas and
fake kernels (``torch.library.opcheck``), and that ``torch.compile(
fullgraph=True)`` over ``ring_attention(..., tables_q, tables_k)`` and over a
hand-written ring loop of the step ops gives the eager bits, forward and
backward.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

TESTS = ("test_schema", "test_faketensor")


@pytest.fixture(scope="module")
def amd():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    import avgen_amd

    return avgen_amd


def _rand(shape, seed, scale=1.0):
    g = torch.Generator()
    g.manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16).cuda()


def _coords(frames, height, width, batch):
    t = torch.arange(frames, dtype=torch.float32) / 8.0
    r = torch.arange(height, dtype=torch.float32) * 2.0
    c = torch.arange(width, dtype=torch.float32) * 2.0
    g = torch.stack(torch.meshgrid(t, r, c, indexing="ij"), -1).reshape(1, -1, 3)
    return g.expand(batch, -1, -1).contiguous()


def _problem(amd, B=2, H=2, Lq=96, L=192, D=64):
    q, k, v = _rand((B, H, Lq, D), 1, 0.7), _rand((B, H, L, D), 2, 0.7), _rand((B, H, L, D), 3, 0.7)
    do = _rand((B, H, Lq, D), 4)
    tables = amd.rope.build_rotary_tables(_coords(4, 6, 8, B).cuda(), head_dim=D)
    mask = torch.ones(B, L, dtype=torch.bool, device="cuda")
    mask[1, L - 30:] = False
    return q, k, v, do, tables, mask


def test_step_ops_pass_opcheck(amd):
    q, k, v, do, tables, mask = _problem(amd)
    B, H, Lq, D = q.shape
    L = k.shape[2]
    tq, tk = tables.slice(0, Lq), tables.slice(0, L)
    scale = amd.ops.default_scale(D)
    acc = torch.zeros(q.shape, dtype=torch.float32, device="cuda")
    lse = torch.zeros((B, H, Lq), dtype=torch.float32, device="cuda")
    out = torch.empty_like(q)
    ops = torch.ops.avgen_amd
    torch.library.opcheck(ops.ring_fwd_step.default,
                          (q, k, v, mask, tq.cos, tq.sin, tk.cos, tk.sin, scale, acc, lse, out, True, True),
                          test_utils=TESTS)
    amd.ops.ring_fwd_step_(q, k, v, mask, tq, tk, scale, acc, lse, out, first=True, last=True)
    dq_acc = torch.zeros(q.shape, dtype=torch.float32, device="cuda")
    dk, dv = torch.empty_like(k), torch.empty_like(v)
    B_, Hq, Hkv = B, H, H
    nbytes, _ = amd.ops.bwd_workspace_plan(B_, Hq, Hkv, Lq, L, D, q.device)
    ws = amd.ops._workspace(nbytes, q.device)
    torch.library.opcheck(ops.ring_bwd_step.default,
                          (do, q, k, v, out, lse, mask, tq.cos, tq.sin, tk.cos, tk.sin, scale, dq_acc, dk, dv, ws,
                           False), test_utils=TESTS)
    dq = torch.empty_like(q)
    torch.library.opcheck(ops.ring_dq_finish.default, (dq_acc, tq.cos, tq.sin, dq), test_utils=TESTS)
    o2 = torch.randn(q.shape, device="cuda").to(torch.bfloat16)
    l2 = torch.randn((B, H, Lq), device="cuda")
    torch.library.opcheck(ops.lse_merge.default, (acc.clone(), lse.clone(), o2, l2), test_utils=TESTS)
    qg, kg, vg = (t.clone().requires_grad_(True) for t in (q, k, v))
    torch.library.opcheck(ops.ring_attention_rope.default,
                          (qg, kg, vg, mask, tq.cos, tq.sin, tk.cos, tk.sin, 2, scale),
                          test_utils=TESTS + ("test_autograd_registration",))
    torch.library.opcheck(ops.ring_attention_rope_bwd.default,
                          (do, q, k, v, out, lse, mask, tq.cos, tq.sin, tk.cos, tk.sin, 2, scale), test_utils=TESTS)


def _run(fn, q, k, v, do, *args):
    ins = [t.clone().requires_grad_(True) for t in (q, k, v)]
    out, lse = fn(*ins, *args)
    out.backward(do)
    torch.cuda.synchronize()
    return out.detach(), lse.detach(), [t.grad for t in ins]


def test_compiled_ring_attention_with_tables_gives_eager_bits(amd):
    q, k, v, do, tables, mask = _problem(amd)
    Lq = q.shape[2]

    def fn(q, k, v, tq, tk, m):
        return amd.ring.ring_attention(q, k, v, cp=2, key_mask=m, tables_q=tq, tables_k=tk)

    tq, tk = tables.slice(0, Lq), tables
    ref = _run(fn, q, k, v, do, tq, tk, mask)
    torch._dynamo.reset()
    compiled = torch.compile(fn, fullgraph=True, dynamic=False)
    got = _run(compiled, q, k, v, do, tq, tk, mask)
    assert torch.equal(got[0], ref[0]) and torch.equal(got[1], ref[1])
    for a, b in zip(got[2], ref[2]):
        assert torch.equal(a, b)


def test_compiled_loop_of_step_ops_gives_eager_bits(amd):
    """What a rank does inside the torch ring, per arriving chunk: the forward
    step with the merge, then per chunk the backward step into the fp32 dq
    accumulator and the chunk's dk/dv slices, then one dq finish."""
    q, k, v, do, tables, mask = _problem(amd)
    B, H, Lq, D = q.shape
    L, cp = k.shape[2], 3
    c = L // cp
    scale = amd.ops.default_scale(D)
    tq = tables.slice(0, Lq)
    nbytes = max(amd.ops.bwd_workspace_plan(B, H, H, Lq, c, D, q.device)[0] for _ in range(cp))

    def ring(q, k, v, m, cos_q, sin_q, cos_k, sin_k, do):
        ops = torch.ops.avgen_amd
        acc = torch.empty(q.shape, dtype=torch.float32, device=q.device)
        lse = torch.empty((B, H, Lq), dtype=torch.float32, device=q.device)
        out = torch.empty_like(q)
        for r in range(cp):
            a, b = r * c, (r + 1) * c
            ops.ring_fwd_step(q, k[:, :, a:b], v[:, :, a:b], m[:, a:b], cos_q, sin_q, cos_k[:, :, a:b],
                              sin_k[:, :, a:b], scale, acc, lse, out, r == 0, r == cp - 1)
        dq_acc = torch.zeros(q.shape, dtype=torch.float32, device=q.device)
        dk, dv = torch.empty_like(k), torch.empty_like(v)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
        for r in range(cp):
            a, b = r * c, (r + 1) * c
            ops.ring_bwd_step(do, q, k[:, :, a:b], v[:, :, a:b], out, lse, m[:, a:b], cos_q, sin_q,
                              cos_k[:, :, a:b], sin_k[:, :, a:b], scale, dq_acc, dk[:, :, a:b], dv[:, :, a:b], ws,
                              r > 0)
        dq = torch.empty_like(q)
        ops.ring_dq_finish(dq_acc, cos_q, sin_q, dq)
        return out, lse, dq, dk, dv

    args = (q, k, v, mask, tq.cos, tq.sin, tables.cos, tables.sin, do)
    ref = ring(*args)
    torch.cuda.synchronize()
    torch._dynamo.reset()
    got = torch.compile(ring, fullgraph=True, dynamic=False)(*args)
    torch.cuda.synchronize()
    for a, b in zip(got, ref):
        assert torch.equal(a, b)
    # and the eager ring of the package (its own chunking and workspace) agrees
    out, lse = amd.ring.ring_attention(q, k, v, cp=cp, key_mask=mask, tables_q=tq, tables_k=tables)
    assert torch.equal(out, ref[0]) and torch.equal(lse, ref[1])
