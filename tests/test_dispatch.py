"""Backend-dispatch helpers (src/avgen/models/attention.py:53-180, called at
:264): the classification, the backend lists and their composition with
``attention(..., backends=...)`` / ``sdpa_context``.  CPU only; the GPU side
(capability of the real device, the call through the kernel) is in
tests/test_gpu_blocks.py."""

from __future__ import annotations

import pytest
import torch
from torch.nn.attention import SDPBackend

from avgen_amd import attention as A

FLASH, EFF, MATH, CUDNN = (SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION, SDPBackend.MATH,
                           SDPBackend.CUDNN_ATTENTION)


@pytest.fixture
def fake_gpu(monkeypatch):
    """Pretend a GPU of a given capability is present (no device is touched)."""
    state = {"cap": (9, 5)}
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(torch.cuda, "current_device", lambda: 0)
    monkeypatch.setattr(torch.cuda, "get_device_capability", lambda index=None: state["cap"])
    monkeypatch.setattr(A, "_arch_by_index", {})
    return state


def test_cpu_classification_and_list():
    assert A.device_arch("cpu") == "cpu"
    assert A.attention_backends("cpu") == (MATH,)
    assert A.attention_backends("cpu", allow_flash=False) == (MATH,)
    if not torch.cuda.is_available():
        assert A.device_arch(None) == "cpu"


# Capability -> family, at and around each floor of the reference's table
# (src/avgen/models/attention.py:53-59: "at least this capability").
@pytest.mark.parametrize(
    "cap,arch",
    [((12, 0), "blackwell"), ((10, 0), "blackwell"), ((9, 5), "hopper"), ((9, 0), "hopper"),
     ((8, 9), "ada"), ((8, 6), "ampere"), ((8, 0), "ampere"), ((7, 5), "legacy"), ((6, 0), "legacy")],
)
def test_capability_floors(fake_gpu, cap, arch):
    fake_gpu["cap"] = cap
    assert A.device_arch("cuda") == arch
    assert A.device_arch("cuda:0") == arch  # memoised per index, same answer


def test_backend_lists_match_reference_order(fake_gpu):
    # src/avgen/models/attention.py:63-91: MATH last everywhere; cuDNN first
    # from Hopper on; no cuDNN before Hopper.
    expect = {
        (10, 0): (CUDNN, FLASH, EFF, MATH),
        (9, 5): (CUDNN, FLASH, EFF, MATH),
        (8, 9): (FLASH, EFF, MATH),
        (8, 0): (FLASH, EFF, MATH),
        (7, 0): (EFF, MATH),
    }
    for cap, backends in expect.items():
        fake_gpu["cap"] = cap
        A._arch_by_index.clear()
        got = A.attention_backends("cuda")
        assert got == backends
        assert got[-1] is MATH
        no_flash = A.attention_backends("cuda", allow_flash=False)
        assert FLASH not in no_flash and no_flash == tuple(b for b in backends if b is not FLASH)


def test_sdpa_context_pins_torch_backends(fake_gpu):
    # On a GPU the context is torch's sdpa_kernel over the list: inside it
    # only the listed backends are enabled for torch's own SDPA calls.
    with A.sdpa_context("cuda", backends=[MATH]):
        assert torch.backends.cuda.math_sdp_enabled()
        assert not torch.backends.cuda.flash_sdp_enabled()
        assert not torch.backends.cuda.mem_efficient_sdp_enabled()
    with A.sdpa_context("cuda"):  # default list of a (9, 5) device: all but none
        assert torch.backends.cuda.flash_sdp_enabled() and torch.backends.cuda.math_sdp_enabled()
    # On CPU it is a no-op whatever the list.
    before = torch.backends.cuda.flash_sdp_enabled()
    with A.sdpa_context("cpu", backends=[MATH]):
        assert torch.backends.cuda.flash_sdp_enabled() == before


def test_attention_enters_sdpa_context_with_callers_backends(monkeypatch):
    """``attention(q, k, v, backends=attention_backends(dev))`` composes as the
    reference's call site (:264) uses it: the kernel launch runs inside
    ``sdpa_context(query.device, backends=...)`` with exactly the caller's list."""
    seen = []

    class Ctx:
        def __init__(self, device, backends):
            seen.append(("enter", torch.device(device).type, None if backends is None else tuple(backends)))

        def __enter__(self):
            return None

        def __exit__(self, *exc):
            seen.append(("exit",))
            return False

    def fake_fwd(q, k, v, mask, cos, sin, scale):
        seen.append(("launch", tuple(q.shape)))
        return torch.zeros_like(q), torch.zeros(q.shape[:3])

    monkeypatch.setattr(A, "sdpa_context", lambda device=None, *, backends=None: Ctx(device, backends))
    monkeypatch.setattr(A.ops, "flash_fwd", fake_fwd)
    q = torch.zeros(1, 2, 8, 64, dtype=torch.bfloat16)
    backends = A.attention_backends(q.device)
    A.attention(q, q, q, backends=backends)
    assert seen == [("enter", "cpu", backends), ("launch", (1, 2, 8, 64)), ("exit",)]
    seen.clear()
    A.attention(q, q, q)  # default: the context is still entered, with None
    assert seen[0] == ("enter", "cpu", None) and seen[-1] == ("exit",)
    seen.clear()
    # zero-length inputs return zeros before any dispatch (:261-262)
    out = A.attention(q[:, :, :0], q, q, backends=backends)
    assert out.shape == (1, 2, 0, 64) and seen == []
