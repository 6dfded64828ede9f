"""The staged-dS memory plan of the backward (CPU: the library's size
functions and the host plan only; no launch).

* the default budget keeps the benchmark's shapes in the pass counts the
  plan states (c3 ring chunk and c2 block in one pass, 76k-token pairs five
  per pass), whatever the device's total memory above 192 GiB;
* passes are equal, the fewest that fit;
* a workspace the allocator cannot provide is retried with half the pairs
  per pass down to one, then (staging optional) without staging, and raises
  only where staging is required.
"""

from __future__ import annotations

import pytest
import torch

from avgen_amd import _lib, ops

GIB = 1 << 30


@pytest.fixture
def device_props(monkeypatch):
    """A fake device index 0 of a given total memory (no GPU touched)."""
    state = {"total": 288 * 10 ** 9}

    class Props:
        @property
        def total_memory(self):
            return state["total"]

    monkeypatch.setattr(torch.cuda, "get_device_properties", lambda idx: Props())
    monkeypatch.setattr(torch.cuda, "current_device", lambda: 0)
    monkeypatch.delenv("AVGEN_AMD_DS_BUDGET_GB", raising=False)
    monkeypatch.setattr(ops, "_ds_budgets", {})
    return state


DEV = torch.device("cuda", 0)


def test_default_budget_pass_counts(device_props):
    assert ops._ds_budget(DEV) == 64 * GIB
    # c3 ring chunk: 40 pairs of 18,944 x 18,944 bf16 = 26.7 GiB, one pass
    per = ops.ds_bytes_per_pair(1, 18900, 18900)
    assert per == 18944 * 18944 * 2 and 40 * per < 64 * GIB
    assert ops._staged_pairs(1, 40, 40, 18900, 18900, 128, DEV) == 40
    # c2 block: (2, 20, 16384) -> 40 pairs of 512 MiB, one pass
    assert ops._staged_pairs(2, 20, 20, 16384, 16384, 128, DEV) == 40
    # c4: 76,112 tokens, 10.8 GiB per pair -> 5 per pass (80 pairs: 16 passes)
    per4 = ops.ds_bytes_per_pair(1, 76112, 76112)
    assert 5 * per4 <= 64 * GIB < 6 * per4
    assert ops._staged_pairs(2, 40, 40, 76112, 76112, 128, DEV) == 5
    # the plan's workspace: the library's staged size for that many pairs
    nbytes, staged = ops.bwd_workspace_plan(1, 40, 40, 18900, 18900, 128, DEV)
    assert staged and nbytes == _lib.load().avattn_bwd_staged_workspace_size(1, 40, 40, 18900, 18900, 128, 40)
    # a small device takes a third of its memory
    device_props["total"] = 48 * GIB
    ops._ds_budgets.clear()
    assert ops._ds_budget(DEV) == 16 * GIB
    assert ops._staged_pairs(1, 40, 40, 18900, 18900, 128, DEV) == 20  # 2 equal passes


def test_equal_passes_and_overrides(device_props):
    per = ops.ds_bytes_per_pair(1, 1000, 1000)
    ops.set_ds_budget(7 * per, DEV)  # 7 fit -> 3 passes of 6, 6, 6 -> 6 per pass for 18 pairs
    assert ops._staged_pairs(1, 18, 18, 1000, 1000, 64, DEV) == 6
    ops.set_ds_budget(0, DEV)
    assert ops._staged_pairs(1, 18, 18, 1000, 1000, 64, DEV) == 0
    assert ops._staged_pairs(1, 18, 18, 1000, 1000, 64, DEV, stage_ds=True) == 1
    ops.set_ds_budget(None, DEV)
    assert ops._ds_budget(DEV) == 64 * GIB
    assert ops._staged_pairs(1, 18, 18, 1000, 1000, 64, DEV, stage_ds=False) == 0


def _fake_alloc(monkeypatch, limit):
    sizes = []

    def alloc(nbytes, device):
        sizes.append(int(nbytes))
        if nbytes > limit:
            raise torch.OutOfMemoryError("fake: out of memory")
        return torch.empty(max(int(nbytes), 256), dtype=torch.uint8)

    monkeypatch.setattr(ops, "_workspace", alloc)
    return sizes


def test_out_of_memory_halves_the_pairs(device_props, monkeypatch):
    lib = _lib.load()
    shape = (1, 40, 40, 18900, 18900, 128)
    staged = [lib.avattn_bwd_staged_workspace_size(*shape, p) for p in (40, 20, 10, 5)]
    sizes = _fake_alloc(monkeypatch, staged[2])  # 10 pairs fit, 20 do not
    ws = ops._alloc_bwd_workspace(*shape, DEV)
    assert sizes == staged[:3] and ws.numel() == staged[2]


def test_out_of_memory_falls_back_to_recompute_or_raises(device_props, monkeypatch):
    lib = _lib.load()
    shape = (1, 4, 4, 1000, 1000, 64)
    base = lib.avattn_bwd_workspace_size(*shape)
    one = lib.avattn_bwd_staged_workspace_size(*shape, 1)
    sizes = _fake_alloc(monkeypatch, base)  # not even one pair's dS fits
    ws = ops._alloc_bwd_workspace(*shape, DEV)
    assert ws.numel() == max(base, 256) and sizes[-2] == one and sizes[-1] == base
    # staging required (the windowed backward): the error surfaces
    with pytest.raises(torch.OutOfMemoryError):
        ops._alloc_bwd_workspace(*shape, DEV, stage_ds=True)
    # staging off: the base workspace, one attempt
    sizes.clear()
    ops._alloc_bwd_workspace(*shape, DEV, stage_ds=False)
    assert sizes == [base]
