"""GPU tests of the drop-in at the block level and of its framework
integration.

* The DiT block loop (src/avgen/models/dit.py:474-504, :491-493;
  src/avgen/models/blocks.py:173-227, :214-215): rotary tables and the key
  mask are built ONCE per forward and reused by every block, whose attention
  output enters the residual stream behind an adaLN gate.  Two blocks through
  ``self_attention_core`` against the oracle's composition.
* ``torch.library`` integration: ``opcheck`` of the custom ops, a
  ``torch.compile(fullgraph=True)`` of a SelfAttention-shaped function (the
  reference compiles every block, src/avgen/parallel/apply.py:216-221), and
  selective activation checkpointing that saves the attention op by name
  (src/avgen/parallel/activation.py:62-74 lists the aten SDPA ops).
"""

from __future__ import annotations

import functools

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


def test_two_block_loop_reuses_tables_and_key_mask(amd):
    B, H, D, grid = 2, 2, 64, (2, 6, 8)
    L, W = grid[0] * grid[1] * grid[2], 2 * 64
    coords = _coords(*grid, B).cuda()
    valid = torch.ones(B, L, dtype=torch.bool, device="cuda")
    valid[1, L - 20:] = False  # batch 1 carries padding
    # built once per forward, as dit.py:491-493
    tables = amd.rope.RotaryEmbedding(D)(coords)
    assert torch.equal(tables.cos, amd.rope.build_rotary_tables(coords, head_dim=D).cos)
    key_mask = amd.attention.key_padding_mask(valid)
    assert key_mask is not None and key_mask.shape == (B, 1, 1, L)
    assert amd.attention.key_padding_mask(torch.ones(B, L, dtype=torch.bool, device="cuda")) is None
    blocks = []
    for i in range(2):
        s = 100 + 10 * i
        blocks.append(dict(wq=_rand((W, W), s, W ** -0.5), wk=_rand((W, W), s + 1, W ** -0.5),
                           wv=_rand((W, W), s + 2, W ** -0.5), wo=_rand((W, W), s + 3, W ** -0.5),
                           gq=_rand((D,), s + 4, 0.1) + 1, gk=_rand((D,), s + 5, 0.1) + 1,
                           gate=_rand((B, 1, W), s + 6, 0.5)))
    hidden0 = _rand((B, L, W), 7, 1.0)

    def forward(hidden, per_block_tables=False):
        for blk in blocks:
            t = amd.rope.build_rotary_tables(coords, head_dim=D) if per_block_tables else tables
            attn = amd.layers.self_attention_core(hidden @ blk["wq"], hidden @ blk["wk"], hidden @ blk["wv"],
                                                  head_dim=D, q_norm_weight=blk["gq"], k_norm_weight=blk["gk"],
                                                  rope=t, key_mask=key_mask)
            hidden = hidden + blk["gate"] * (attn @ blk["wo"])  # blocks.py:214-215
        return hidden

    out = forward(hidden0)
    torch.cuda.synchronize()
    # reusing the tables is exactly rebuilding them per block
    assert torch.equal(out, forward(hidden0, per_block_tables=True))

    # oracle composition in float64 (bf16 rounding where the reference's
    # tensors are bf16: projections, normed q/k, rotated q/k, attention output)
    cos, sin = (x.cpu().numpy() for x in (tables.cos, tables.sin))
    vm = valid.cpu().numpy()
    h = hidden0.float().cpu().numpy().astype(np.float64)

    def bf(x):
        return R.bf16_round(np.asarray(x, np.float32)).astype(np.float64)

    def heads(x):
        return x.reshape(B, L, H, D).transpose(0, 2, 1, 3)

    for blk in blocks:
        w = {k: v.float().cpu().numpy().astype(np.float64) for k, v in blk.items()}
        hb = bf(h)
        q, k, v = (heads(bf(hb @ w[n])) for n in ("wq", "wk", "wv"))
        q = R.apply_rotary_bf16(R.rms_norm_bf16(q.astype(np.float32), w["gq"].astype(np.float32)), cos, sin)
        k = R.apply_rotary_bf16(R.rms_norm_bf16(k.astype(np.float32), w["gk"].astype(np.float32)), cos, sin)
        o, _ = R.attention_f64(q, k, v, vm)
        o = bf(o).transpose(0, 2, 1, 3).reshape(B, L, W)
        h = bf(hb + bf(w["gate"] * bf(o @ w["wo"])))
    got = out.float().cpu().numpy()
    err = np.abs(got - h).max() / np.abs(h).max()
    print(f"two-block loop: max error {err:.2e} of max |hidden|", flush=True)
    assert err <= 2e-2


def test_custom_ops_pass_opcheck(amd):
    """Schema, fake (meta) kernels and autograd registration of the ops the
    block path calls, checked by torch.library.opcheck on small inputs."""
    D, scale = 64, 0.125
    q, k, v = (_rand((1, 2, 96, D), s, 0.7) for s in (1, 2, 3))
    tables = amd.rope.build_rotary_tables(_coords(2, 6, 8, 1).cuda(), head_dim=D)
    qg = q.clone().requires_grad_(True)
    kg = k.clone().requires_grad_(True)
    vg = v.clone().requires_grad_(True)
    tests = ("test_schema", "test_faketensor", "test_autograd_registration")
    mask = torch.ones(1, 96, dtype=torch.bool, device="cuda")
    mask[0, 90:] = False
    torch.library.opcheck(torch.ops.avgen_amd.flash_fwd.default, (qg, kg, vg, mask, tables.cos, tables.sin, scale),
                          test_utils=tests)
    out, lse = amd.ops.flash_fwd(q, k, v, None, None, None, scale)
    do = _rand(q.shape, 4, 1.0)
    torch.library.opcheck(torch.ops.avgen_amd.flash_bwd.default, (do, q, k, v, out, lse, None, scale),
                          test_utils=tests)
    torch.library.opcheck(torch.ops.avgen_amd.rope_apply.default, (qg, tables.cos, tables.sin, False),
                          test_utils=tests)
    x = _rand((1, 96, 2, D), 5, 1.0).transpose(1, 2).requires_grad_(True)  # (B, H, L, D) view of (B, L, H, D)
    wgt = (_rand((D,), 6, 0.1) + 1).requires_grad_(True)
    torch.library.opcheck(torch.ops.avgen_amd.qk_norm_rope.default, (x, wgt, 1e-6, tables.cos, tables.sin),
                          test_utils=tests)


def _self_attention(amd, q_proj, k_proj, v_proj, gq, gk, tables, key_mask):
    return amd.layers.self_attention_core(q_proj, k_proj, v_proj, head_dim=64, q_norm_weight=gq, k_norm_weight=gk,
                                          rope=tables, key_mask=key_mask)


def test_compiled_block_and_selective_checkpoint(amd):
    """torch.compile(fullgraph=True) traces through the custom ops without a
    graph break and gives the eager bits; a selective-AC policy that saves
    avgen_amd::flash_fwd by name (as the reference's policy saves the aten
    SDPA ops) gives the eager gradients and does not rerun the forward."""
    from torch.utils.checkpoint import CheckpointPolicy, checkpoint, create_selective_checkpoint_contexts

    B, L, H, D = 2, 96, 2, 64
    tables = amd.rope.build_rotary_tables(_coords(2, 6, 8, B).cuda(), head_dim=D)
    valid = torch.ones(B, L, dtype=torch.bool, device="cuda")
    valid[1, 80:] = False
    key_mask = amd.attention.key_padding_mask(valid)
    qp, kp, vp = (_rand((B, L, H * D), s, 1.0) for s in (11, 12, 13))
    gq, gk = _rand((D,), 14, 0.1) + 1, _rand((D,), 15, 0.1) + 1
    do = _rand((B, L, H * D), 16, 1.0)
    fn = functools.partial(_self_attention, amd)

    def grads(f):
        ins = [t.clone().requires_grad_(True) for t in (qp, kp, vp)]
        out = f(*ins, gq, gk, tables, key_mask)
        out.backward(do)
        torch.cuda.synchronize()
        return out.detach(), [t.grad for t in ins]

    ref_out, ref_grads = grads(fn)
    torch._dynamo.reset()
    compiled = torch.compile(fn, fullgraph=True, dynamic=False)
    c_out, c_grads = grads(compiled)
    assert torch.equal(c_out, ref_out)
    for a, b in zip(c_grads, ref_grads):
        assert torch.equal(a, b)

    calls = {"n": 0}
    save = {torch.ops.avgen_amd.flash_fwd.default, torch.ops.avgen_amd.qk_norm_rope.default}

    def policy(ctx, op, *args, **kwargs):
        if op is torch.ops.avgen_amd.flash_fwd.default and not ctx.is_recompute:
            calls["n"] += 1
        return CheckpointPolicy.MUST_SAVE if op in save else CheckpointPolicy.PREFER_RECOMPUTE

    def checkpointed(*args):
        return checkpoint(fn, *args, use_reentrant=False,
                          context_fn=functools.partial(create_selective_checkpoint_contexts, policy))

    s_out, s_grads = grads(checkpointed)
    assert calls["n"] == 1
    assert torch.equal(s_out, ref_out)
    for a, b in zip(s_grads, ref_grads):
        assert torch.equal(a, b)


def test_dispatch_helpers_compose_on_the_device(amd):
    """src/avgen/models/attention.py:264 runs every call under
    ``sdpa_context(query.device, backends=backends)`` with the list from
    ``attention_backends``: the same composition here gives the kernel's bits
    whatever list is pinned, eagerly and compiled, and the device classifies
    as the reference classifies it."""
    from torch.nn.attention import SDPBackend

    A = amd.attention
    major, minor = torch.cuda.get_device_capability()
    cap = 10 * major + minor
    expect = "blackwell" if cap >= 100 else "hopper" if cap >= 90 else "ada" if cap >= 89 else (
        "ampere" if cap >= 80 else "legacy")
    print(f"device capability {(major, minor)} -> {A.device_arch('cuda')}", flush=True)
    assert A.device_arch("cuda") == expect == A.device_arch(None)
    dev = torch.device("cuda")
    backends = A.attention_backends(dev)
    assert backends[-1] is SDPBackend.MATH
    q, k, v = (_rand((2, 2, 96, 64), s, 0.7) for s in (21, 22, 23))
    valid = torch.ones(2, 96, dtype=torch.bool, device="cuda")
    valid[0, 70:] = False
    mask = A.key_padding_mask(valid)
    ref = A.attention(q, k, v, attn_mask=mask)
    assert torch.equal(A.attention(q, k, v, attn_mask=mask, backends=backends), ref)
    with A.sdpa_context(dev, backends=[SDPBackend.MATH]):
        assert not torch.backends.cuda.flash_sdp_enabled()
        assert torch.equal(A.attention(q, k, v, attn_mask=mask, backends=[SDPBackend.MATH]), ref)
    assert torch.backends.cuda.flash_sdp_enabled()  # restored on exit

    def fn(q, k, v, m):
        return A.attention(q, k, v, attn_mask=m, backends=A.attention_backends(q.device, allow_flash=False))

    torch._dynamo.reset()
    assert torch.equal(torch.compile(fn, fullgraph=True, dynamic=False)(q, k, v, mask), ref)
