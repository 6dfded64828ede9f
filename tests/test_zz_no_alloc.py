"""avattn_fwd_noalloc (through the C ABI) against avattn_fwd: the same bits,
on two calls in a row, the second with a smaller problem (the fixed scratch
keeps the first call's contents), with and without a key mask and the fused
query rotation, MHA and GQA, head_dim 128 and 64; a problem beyond the
scratch is refused without writing anything."""

from __future__ import annotations

import ctypes

import pytest
import torch

from avgen_amd import _lib

pytestmark = pytest.mark.gpu


def _rand(shape, seed, scale):
    g = torch.Generator()
    g.manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16).cuda()


def _strides(t):
    return _lib.i64_array(t.stride()[:3])


def _call(lib, fn, q, k, v, mask, tables, out, lse, ws=None):
    B, Hq, Lq, D = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    mptr = None if mask is None else mask.data_ptr()
    msb = 0 if mask is None else mask.stride(0)
    cos = sin = None
    rsb = 0
    if tables is not None:
        cos, sin = tables.cos.data_ptr(), tables.sin.data_ptr()
        rsb = 0 if tables.cos.shape[0] == 1 else tables.cos.stride(0)
    stream = torch.cuda.current_stream().cuda_stream
    args = [q.data_ptr(), k.data_ptr(), v.data_ptr(), _strides(q), _strides(k), _strides(v), B, Hq, Hkv, Lq, Lk, D,
            mptr, msb, cos, sin, rsb, ctypes.c_float(D ** -0.5), out.data_ptr(), _strides(out), lse.data_ptr()]
    if fn == "avattn_fwd":
        args += [ws.data_ptr(), ws.numel()]
    return getattr(lib, fn)(*args, stream)


CASES = [
    # B, Hq, Hkv, Lq, Lk, D, masked, rotated
    (2, 4, 2, 300, 1500, 128, True, True),   # first call: the larger problem
    (1, 2, 2, 100, 70, 64, False, False),    # second call: smaller, stale scratch from the first
    (1, 8, 8, 513, 4097, 128, False, True),
]


def test_noalloc_forward_equals_workspace_forward():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    import avgen_amd

    lib = _lib.load()
    for i, (B, Hq, Hkv, Lq, Lk, D, masked, rotated) in enumerate(CASES):
        print(f"noalloc case {i}: B={B} Hq={Hq} Hkv={Hkv} Lq={Lq} Lk={Lk} D={D} mask={masked} rope={rotated}",
              flush=True)
        q = _rand((B, Hq, Lq, D), 10 * i + 1, 0.7)
        k, v = _rand((B, Hkv, Lk, D), 10 * i + 2, 0.7), _rand((B, Hkv, Lk, D), 10 * i + 3, 0.7)
        mask = None
        if masked:
            g = torch.Generator()
            g.manual_seed(i)
            mask = (torch.rand((B, Lk), generator=g) > 0.2).cuda().view(torch.uint8)
            mask[-1, Lk // 2:] = 0
        tables = None
        if rotated:
            coords = torch.rand((B, Lq, 3), generator=torch.Generator().manual_seed(i)).cuda() * 10
            tables = avgen_amd.rope.build_rotary_tables(coords, head_dim=D)
        need = lib.avattn_fwd_workspace_size(B, Hkv, Lk, D)
        assert 0 < need <= _lib.FWD_NOALLOC_SCRATCH
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        out_a, out_b = torch.empty_like(q), torch.full_like(q, float("nan"))
        lse_a = torch.empty((B, Hq, Lq), device="cuda")
        lse_b = torch.full_like(lse_a, float("nan"))
        assert _call(lib, "avattn_fwd", q, k, v, mask, tables, out_a, lse_a, ws) == _lib.OK
        before = torch.cuda.memory_allocated()
        assert _call(lib, "avattn_fwd_noalloc", q, k, v, mask, tables, out_b, lse_b) == _lib.OK
        torch.cuda.synchronize()
        assert torch.cuda.memory_allocated() == before
        assert torch.equal(out_a, out_b) and torch.equal(lse_a, lse_b)
        assert torch.isfinite(out_b).all()
    # beyond the scratch: refused, outputs untouched
    B, Hq, Hkv, Lq, Lk, D = 1, 2, 2, 64, 1 << 17, 128
    q = _rand((B, Hq, Lq, D), 99, 0.7)
    k = v = torch.zeros((B, Hkv, Lk, D), dtype=torch.bfloat16, device="cuda")
    out = torch.full_like(q, 7.0)
    lse = torch.full((B, Hq, Lq), 7.0, device="cuda")
    assert _call(lib, "avattn_fwd_noalloc", q, k, v, None, None, out, lse) == _lib.ERR_SCRATCH
    torch.cuda.synchronize()
    assert (out == 7.0).all() and (lse == 7.0).all()


def test_noalloc_forward_under_graph_capture():
    """The entry point inside a captured HIP graph (torch.cuda.graph): after
    one eager call (the first call per device looks the scratch array up),
    a capture of avattn_fwd_noalloc replays three times, with eager work
    between the replays, each time giving avattn_fwd's bits."""
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    import avgen_amd

    lib = _lib.load()
    B, Hq, Hkv, Lq, Lk, D = 2, 4, 2, 300, 1500, 128
    print(f"noalloc graph capture: B={B} Hq={Hq} Hkv={Hkv} Lq={Lq} Lk={Lk} D={D} mask rope", flush=True)
    q = _rand((B, Hq, Lq, D), 71, 0.7)
    k, v = _rand((B, Hkv, Lk, D), 72, 0.7), _rand((B, Hkv, Lk, D), 73, 0.7)
    g = torch.Generator()
    g.manual_seed(7)
    mask = (torch.rand((B, Lk), generator=g) > 0.2).cuda().view(torch.uint8)
    coords = torch.rand((B, Lq, 3), generator=torch.Generator().manual_seed(7)).cuda() * 10
    tables = avgen_amd.rope.build_rotary_tables(coords, head_dim=D)
    ws = torch.empty(lib.avattn_fwd_workspace_size(B, Hkv, Lk, D), dtype=torch.uint8, device="cuda")
    out_a, lse_a = torch.empty_like(q), torch.empty((B, Hq, Lq), device="cuda")
    assert _call(lib, "avattn_fwd", q, k, v, mask, tables, out_a, lse_a, ws) == _lib.OK
    out_b, lse_b = torch.empty_like(q), torch.empty((B, Hq, Lq), device="cuda")
    assert _call(lib, "avattn_fwd_noalloc", q, k, v, mask, tables, out_b, lse_b) == _lib.OK  # warm-up
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = _call(lib, "avattn_fwd_noalloc", q, k, v, mask, tables, out_b, lse_b)
    assert rc == _lib.OK
    for rep in range(3):
        out_b.fill_(float("nan"))
        lse_b.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_a, out_b) and torch.equal(lse_a, lse_b), rep
