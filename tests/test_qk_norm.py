"""QK RMSNorm: the oracle's restatement pinned against the library routine
the reference calls (torch's F.rms_norm, src/avgen/models/layers.py:106-118)
and against float64 autograd of the same formula; the C ABI's validation
paths for the fused norm + rotation entry points (no GPU needed)."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import reference as R


def _bf16(shape, seed, scale=1.0):
    g = torch.Generator()
    g.manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


@pytest.mark.parametrize("D,scale", [(128, 1.0), (64, 3.0), (128, 1e-3)])
def test_rms_norm_oracle_matches_torch_rms_norm(D, scale):
    """bf16 activation and bf16 gain through F.rms_norm on the CPU: the
    oracle's float32 chain gives the same bf16 values (a rare 1-ulp
    difference allowed where torch sums the squares in another order)."""
    x = _bf16((2, 3, 257, D), 1, scale)
    w = (torch.rand(D, generator=torch.Generator().manual_seed(2)) + 0.5).to(torch.bfloat16)
    ref = F.rms_norm(x, (D,), w, 1e-6).float().numpy()
    got = R.rms_norm_bf16(x.float().numpy(), w.float().numpy(), 1e-6)
    diff = np.abs(got - ref)
    ulp = np.abs(ref) * 2.0 ** -7 + 1e-30
    assert (diff <= ulp).all()
    assert (diff > 0).mean() < 1e-3
    # without a gain
    ref = F.rms_norm(x, (D,), None, 1e-6).float().numpy()
    got = R.rms_norm_bf16(x.float().numpy(), None, 1e-6)
    assert (np.abs(got - ref) <= np.abs(ref) * 2.0 ** -7 + 1e-30).all()


def test_rms_norm_hand_worked():
    """x = (3, 4): mean square 12.5, so with eps 0 the row becomes
    (3, 4)/sqrt(12.5) = (0.8485.., 1.1313..); a zero row stays zero."""
    x = np.array([[3.0, 4.0], [0.0, 0.0]], np.float32)
    got = R.rms_norm_bf16(x, None, 0.0 + 1e-30)
    np.testing.assert_allclose(got[0], R.bf16_round(np.array([3, 4], np.float32) / np.float32(np.sqrt(12.5))))
    assert (got[1] == 0).all()
    got = R.rms_norm_bf16(x, np.array([2.0, -1.0], np.float32), 1e-30)
    np.testing.assert_allclose(got[0], R.bf16_round(np.array([6, -4], np.float32) / np.float32(np.sqrt(12.5))),
                               rtol=2 ** -7)


def test_rms_norm_f64_matches_torch_and_autograd_with_an_fp32_gain():
    """The float32 model's norm: F.rms_norm in float64 with a gain that is
    not a bf16 value (so a stray bf16 rounding of the gain would show), its
    autograd gradients against rms_norm_bwd_f64 with round_gain=False."""
    x = torch.randn(2, 7, 128, dtype=torch.float64, requires_grad=True)
    w = (torch.rand(128, dtype=torch.float64) + 0.5 + 1e-4).requires_grad_(True)
    assert not torch.equal(w.to(torch.bfloat16).double(), w)
    np.testing.assert_allclose(R.rms_norm_f64(x.detach().numpy(), w.detach().numpy(), 1e-6),
                               F.rms_norm(x, (128,), w, 1e-6).detach().numpy(), rtol=1e-13, atol=1e-15)
    np.testing.assert_allclose(R.rms_norm_f64(x.detach().numpy(), None, 1e-6),
                               F.rms_norm(x, (128,), None, 1e-6).detach().numpy(), rtol=1e-13, atol=1e-15)
    g = torch.randn(2, 7, 128, dtype=torch.float64)
    F.rms_norm(x, (128,), w, 1e-6).backward(g)
    dx, dw = R.rms_norm_bwd_f64(x.detach().numpy(), w.detach().numpy(), g.numpy(), 1e-6, round_gain=False)
    np.testing.assert_allclose(dx, x.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dw, w.grad.numpy(), rtol=1e-10, atol=1e-12)
    # the default rounds the gain: a different (wrong here) dx
    dx_r, _ = R.rms_norm_bwd_f64(x.detach().numpy(), w.detach().numpy(), g.numpy(), 1e-6)
    assert np.abs(dx_r - x.grad.numpy()).max() > 1e-6


def test_rms_norm_backward_oracle_matches_autograd():
    x = torch.randn(3, 5, 64, dtype=torch.float64, requires_grad=True)
    w = (torch.rand(64, dtype=torch.float64) + 0.5).to(torch.bfloat16).double().requires_grad_(True)
    g = torch.randn(3, 5, 64, dtype=torch.float64)
    F.rms_norm(x, (64,), w, 1e-6).backward(g)
    dx, dw = R.rms_norm_bwd_f64(x.detach().numpy(), w.detach().numpy(), g.numpy(), 1e-6)
    np.testing.assert_allclose(dx, x.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dw, w.grad.numpy(), rtol=1e-10, atol=1e-12)
    x.grad = None
    F.rms_norm(x, (64,), None, 1e-6).backward(g)
    dx, dw = R.rms_norm_bwd_f64(x.detach().numpy(), None, g.numpy(), 1e-6)
    np.testing.assert_allclose(dx, x.grad.numpy(), rtol=1e-10, atol=1e-12)
    assert dw is None


def test_qk_norm_abi_validation():
    from avgen_amd import _lib

    try:
        lib = _lib.load()
    except RuntimeError:
        pytest.skip("libavattn.so not built")
    if torch.cuda.is_available():
        pytest.skip("validation-only test; would launch on a GPU")
    s = _lib.i64_array([1 << 20, 128, 1 << 12])

    def fwd(**o):
        a = dict(x=16, xs=s, B=1, H=2, L=4, D=128, w=16, eps=1e-6, cos=None, sin=None, tsb=0, out=16, os=s)
        a.update(o)
        return lib.avattn_qk_norm_rope(a["x"], a["xs"], a["B"], a["H"], a["L"], a["D"], a["w"], a["eps"], a["cos"],
                                       a["sin"], a["tsb"], a["out"], a["os"], None)

    assert fwd(D=96) == _lib.ERR_HEAD_DIM
    assert fwd(L=-1) == _lib.ERR_BAD_SHAPE
    assert fwd(eps=-1.0) == _lib.ERR_ARGUMENT
    assert fwd(eps=float("nan")) == _lib.ERR_ARGUMENT
    assert fwd(cos=16) == _lib.ERR_NULL_POINTER
    assert fwd(x=None) == _lib.ERR_NULL_POINTER
    assert fwd(out=None) == _lib.ERR_NULL_POINTER
    assert fwd(x=8) == _lib.ERR_LAYOUT
    assert fwd(w=8) == _lib.ERR_LAYOUT
    assert fwd(cos=16, sin=16, tsb=2) == _lib.ERR_LAYOUT
    assert fwd(os=_lib.i64_array([1 << 20, 128, 100])) == _lib.ERR_LAYOUT
    assert fwd(L=0) == _lib.OK
    assert lib.avattn_qk_norm_rope_bwd_workspace_size(128) == 4096 * 128 * 4
    assert lib.avattn_qk_norm_rope_bwd_workspace_size(96) == 0

    def bwd(ws=256, wsb=1 << 20, dw=16, w=16):
        return lib.avattn_qk_norm_rope_bwd(16, s, 16, s, 1, 2, 4, 128, w, 1e-6, None, None, 0, 16, s, dw, ws, wsb,
                                           None)

    assert bwd(dw=None) == _lib.ERR_NULL_POINTER
    assert bwd(ws=None) == _lib.ERR_WORKSPACE
    assert bwd(wsb=100) == _lib.ERR_WORKSPACE


def test_self_attention_composition_oracle_matches_torch_cpu():
    """src/avgen/models/layers.py:530-545 restated with torch CPU ops (split
    heads, F.rms_norm with the bf16 gain, the reference's float32 rotation
    chain, SDPA in float64, flatten) against the oracle's composition
    (rms_norm_bf16 -> apply_rotary_bf16 -> attention_f64)."""
    from oracle import torch_path as T

    B, L, H, D = 1, 48, 2, 64
    coords = torch.from_numpy(R.video_coords(2, 4, 6))
    cos, sin = T.rotary_tables(coords, D)
    qp, kp, vp = (_bf16((B, L, H * D), s) for s in (21, 22, 23))
    wq = (torch.rand(D, generator=torch.Generator().manual_seed(24)) + 0.5).to(torch.bfloat16)
    wk = (torch.rand(D, generator=torch.Generator().manual_seed(25)) + 0.5).to(torch.bfloat16)

    def heads(t):
        return t.unflatten(-1, (-1, D)).transpose(1, 2)

    q = T.apply_rotary(F.rms_norm(heads(qp), (D,), wq, 1e-6), cos, sin)
    k = T.apply_rotary(F.rms_norm(heads(kp), (D,), wk, 1e-6), cos, sin)
    ref = F.scaled_dot_product_attention(q.double(), k.double(), heads(vp).double())
    ref = ref.transpose(1, 2).flatten(2).numpy()

    c, s = cos.numpy(), sin.numpy()
    qn = R.apply_rotary_bf16(R.rms_norm_bf16(heads(qp).float().numpy(), wq.float().numpy()), c, s)
    kn = R.apply_rotary_bf16(R.rms_norm_bf16(heads(kp).float().numpy(), wk.float().numpy()), c, s)
    o, _ = R.attention_f64(qn, kn, heads(vp).float().numpy())
    got = o.transpose(0, 2, 1, 3).reshape(B, L, H * D)
    assert np.abs(got - ref).max() <= 1e-2
    # exact where the normalised operands agree bit for bit
    assert (qn == q.float().numpy()).mean() > 0.999 and (kn == k.float().numpy()).mean() > 0.999
