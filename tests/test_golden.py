"""Golden fixtures (tests/golden/*.npz): written by the pinned oracle, replayed
against the oracle (CPU, exact) and against the HIP kernels (GPU, to the
north-star tolerances; RoPE bit-exact)."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"
NAMES = ["rope_tables_d12", "rope_tables_d128", "rope_tables_d128_ntk", "rope_apply_d64", "attn_d64", "attn_d128",
         "ring_3chunks", "packed_attention", "temporal_attention", "qk_norm_rope_d128", "attn_fp8_d128"]


def load(name: str) -> dict[str, np.ndarray]:
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def bits_to_bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits.astype(np.int16).copy()).view(torch.bfloat16)


def test_fixtures_reproduce_from_oracle():
    from tests.golden import make_golden

    fresh = make_golden.build()
    assert sorted(fresh) == sorted(NAMES)
    for name in NAMES:
        stored = load(name)
        assert sorted(stored) == sorted(fresh[name]), name
        for key, arr in fresh[name].items():
            assert np.array_equal(np.asarray(arr), stored[key]), f"{name}.{key} drifted"


def test_attention_fixtures_agree_with_torch_cpu():
    # Independent check of the stored expectations with PyTorch's SDPA.
    import torch.nn.functional as F

    for name in ("attn_d64", "attn_d128"):
        g = load(name)
        q, k, v = (torch.from_numpy(bits_to_f32(g[f"{t}_bits"]).astype(np.float64)) for t in "qkv")
        m = torch.from_numpy(g["mask"])
        rep = q.shape[1] // k.shape[1]
        ref = F.scaled_dot_product_attention(q, k.repeat_interleave(rep, 1), v.repeat_interleave(rep, 1),
                                             attn_mask=m[:, None, None, :])
        assert np.abs(ref.numpy() - g["out"]).max() < 1e-6


def test_fp8_fixture_operands_agree_with_torch_float8():
    # The stored e4m3 operands, independently of the oracle's e4m3_round:
    # torch's float8_e4m3fn cast of the fp32 products the kernels form.
    g = load("attn_fp8_d128")
    q, k = bits_to_f32(g["q_bits"]), bits_to_f32(g["k_bits"])
    H, Hk = q.shape[1], k.shape[1]
    ks_h = g["k_scale"][np.arange(H) // (H // Hk)]
    gq = (np.float32(g["scale"]) * np.float32(1.4426950408889634) * ks_h).astype(np.float32)
    mult = np.ldexp(gq, -g["eq"]).astype(np.float32)
    q8 = torch.from_numpy((q * mult[None, :, None, None]).astype(np.float32)).to(torch.float8_e4m3fn).float()
    assert np.array_equal(q8.numpy(), g["q8"])
    kinv = (np.float32(1) / g["k_scale"]).astype(np.float32)
    k8 = torch.from_numpy((k * kinv[None, :, None, None]).astype(np.float32)).to(torch.float8_e4m3fn).float()
    assert np.array_equal(k8.numpy(), g["k8"])
    assert np.all(np.ldexp(1.0, g["eq"]) >= (gq * g["q_scale"]).astype(np.float32))


@pytest.fixture(scope="module")
def amd():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    import avgen_amd

    return avgen_amd


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["attn_d64", "attn_d128"])
def test_gpu_attention_matches_golden(amd, name):
    g = load(name)
    q, k, v, do = (bits_to_bf16(g[f"{t}_bits"]).cuda() for t in ("q", "k", "v", "do"))
    mask = torch.from_numpy(g["mask"]).cuda()
    d = q.shape[-1]
    out, lse = amd.ops.flash_fwd(q, k, v, mask, None, None, d ** -0.5)
    o = out.float().cpu().numpy()
    l = lse.cpu().numpy().astype(np.float64)
    assert np.abs(o - g["out"]).max() <= 2e-2
    fin = np.isfinite(g["lse"])
    assert np.array_equal(np.isneginf(l), ~fin)
    assert np.abs(l[fin] - g["lse"][fin]).max() <= 1e-3
    assert np.all(o[1] == 0)  # batch 1 has every key masked
    dq, dk, dv = amd.ops.flash_bwd(do, q, k, v, out, lse, mask, d ** -0.5)
    for got, key in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
        ref = g[key]
        assert np.abs(got.float().cpu().numpy() - ref).max() <= 2e-2 * max(np.abs(ref).max(), 1e-3), key
    masked = ~g["mask"][:, None, :, None]
    assert np.all(dk.float().cpu().numpy()[np.broadcast_to(masked, dk.shape)] == 0)


@pytest.mark.gpu
def test_gpu_rope_matches_golden(amd):
    g = load("rope_apply_d64")
    x = bits_to_bf16(g["x_bits"]).cuda()
    cos, sin = torch.from_numpy(g["cos"]).cuda(), torch.from_numpy(g["sin"]).cuda()
    got = amd.ops.rope_apply(x, cos, sin, False).cpu().view(torch.int16).numpy().astype(np.uint16)
    assert np.array_equal(got, g["out_bits"])
    inv = amd.ops.rope_apply(x, cos, sin, True).cpu().view(torch.int16).numpy().astype(np.uint16)
    assert np.array_equal(inv, g["inv_bits"])
    for name in ("rope_tables_d12", "rope_tables_d128"):
        t = load(name)
        if t["cos"].shape[-1] * 2 not in (12, 128):
            continue
        tabs = amd.rope.build_rotary_tables(torch.from_numpy(t["coords"]).cuda(), head_dim=t["cos"].shape[-1] * 2)
        assert np.abs(tabs.cos.cpu().numpy() - t["cos"]).max() < 2e-6
        assert np.abs(tabs.sin.cpu().numpy() - t["sin"]).max() < 2e-6
    t = load("rope_tables_d128_ntk")
    tabs = amd.rope.build_rotary_tables(torch.from_numpy(t["coords"]).cuda(), head_dim=128, time_scale=1.5,
                                        scaling=amd.rope.RoPEScaling("ntk", 2.0, 1.5))
    assert np.abs(tabs.cos.cpu().numpy() - t["cos"]).max() < 2e-6


@pytest.mark.gpu
def test_gpu_ring_matches_golden(amd):
    g = load("ring_3chunks")
    q, k, v = (bits_to_bf16(g[f"{t}_bits"]).cuda() for t in "qkv")
    out, lse = amd.ring.ring_attention(q, k, v, cp=3)
    assert np.abs(out.float().cpu().numpy() - g["out"]).max() <= 2e-2
    assert np.abs(lse.cpu().numpy() - g["lse"]).max() <= 1e-3
    # the merge kernel on the first two chunks' exact outputs
    o1 = torch.from_numpy(g["merge01_out"]).clone()
    keys = k.split(20, dim=2)
    vals = v.split(20, dim=2)
    a_out, a_lse = amd.ops.flash_fwd(q, keys[0].contiguous(), vals[0].contiguous(), None, None, None, 64 ** -0.5)
    b_out, b_lse = amd.ops.flash_fwd(q, keys[1].contiguous(), vals[1].contiguous(), None, None, None, 64 ** -0.5)
    acc = a_out.float().contiguous()
    acc_lse = a_lse.clone()
    amd.ops.lse_merge_(acc, acc_lse, b_out, b_lse)
    assert np.abs(acc.cpu().numpy() - o1.numpy()).max() <= 2e-2
    assert np.abs(acc_lse.cpu().numpy() - g["merge01_lse"]).max() <= 1e-3


def test_packed_fixture_is_the_reference_layout():
    """tests/test_data.py:640-667 of the reference: ids and cu_seqlens."""
    g = load("packed_attention")
    assert g["segment_ids"].tolist() == [0] * 3 + [1] * 4 + [2] * 2 + [-1] * 3
    assert g["cu_seqlens"].tolist() == [0, 3, 7, 9]


@pytest.mark.gpu
def test_gpu_varlen_matches_golden(amd):
    g = load("packed_attention")
    q, k, v, do = (bits_to_bf16(g[f"{t}_bits"]).cuda().requires_grad_(t != "do") for t in ("q", "k", "v", "do"))
    out = amd.attention.varlen_attention(q, k, v, torch.from_numpy(g["cu_seqlens"]))
    assert np.abs(out.float().detach().cpu().numpy() - g["out"]).max() <= 2e-2
    assert (out[:, :, 9:] == 0).all()
    out.backward(do)
    for t, key in ((q, "dq"), (k, "dk"), (v, "dv")):
        ref = g[key]
        assert np.abs(t.grad.float().cpu().numpy() - ref).max() <= 2e-2 * np.abs(ref).max(), key


@pytest.mark.gpu
def test_gpu_temporal_matches_golden(amd):
    g = load("temporal_attention")
    assert g["mask"][:, 0].all(axis=-1).any(), "the fixture has fallback rows"
    q, k, v = (bits_to_bf16(g[f"{t}_bits"]).cuda() for t in "qkv")
    out = amd.attention.temporal_neighbour_attention(
        q, k, v, torch.from_numpy(g["query_seconds"]).cuda(), torch.from_numpy(g["key_seconds"]).cuda(),
        window_seconds=float(g["window_seconds"]), key_mask=torch.from_numpy(g["key_mask"]).cuda(), enable_gqa=True)
    assert np.abs(out.float().cpu().numpy() - g["out"]).max() <= 2e-2


@pytest.mark.gpu
def test_gpu_qk_norm_matches_golden(amd):
    g = load("qk_norm_rope_d128")
    xp = bits_to_bf16(g["x_bits"]).cuda()
    x = amd.layers.split_heads(xp.flatten(2), 128).requires_grad_(True)
    w = bits_to_bf16(g["w_bits"]).cuda()
    cos, sin = torch.from_numpy(g["cos"]).cuda(), torch.from_numpy(g["sin"]).cuda()
    y = amd.ops.qk_norm_rope(x, w, float(g["eps"]), cos, sin)
    got = y.detach().float().cpu().numpy()
    ref = bits_to_bf16(g["out_bits"]).float().numpy()
    diff = np.abs(got - ref)
    assert (diff <= np.abs(ref) * 2.0 ** -7 + 1e-6).all() and (diff > 0).mean() < 1e-3
    dx, dw = amd.ops.qk_norm_rope_bwd(bits_to_bf16(g["dy_bits"]).cuda(), x.detach(), w, float(g["eps"]), cos, sin)
    assert np.abs(dx.float().cpu().numpy() - g["dx"]).max() <= 2e-2 * np.abs(g["dx"]).max()
    assert np.abs(dw.cpu().numpy() - g["dw"]).max() <= 1e-3 * np.abs(g["dw"]).max()


@pytest.mark.gpu
def test_gpu_fp8_matches_golden(amd):
    g = load("attn_fp8_d128")
    q, k, v = (bits_to_bf16(g[f"{t}_bits"]).cuda() for t in "qkv")
    qs, ks = torch.from_numpy(g["q_scale"]).cuda(), torch.from_numpy(g["k_scale"]).cuda()
    out, lse = amd.ops.flash_fwd_fp8(q, k, v, torch.from_numpy(g["mask"]).cuda(), qs, ks, float(g["scale"]))
    o = out.float().cpu().numpy()
    l = lse.cpu().numpy().astype(np.float64)
    assert np.abs(o - g["out"]).max() <= 2e-2
    fin = np.isfinite(g["lse"])
    assert np.array_equal(np.isneginf(l), ~fin)
    assert np.abs(l[fin] - g["lse"][fin]).max() <= 1e-3
    assert np.all(o[1] == 0)  # batch 1 has every key masked
