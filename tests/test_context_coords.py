"""CPU tests of the context-parallel shard rules (src/avgen/parallel/context.py
:58-139, 142-175, 213-229) and of the token coordinate rule
(src/avgen/core/patchify.py:45-105) in the package, against the oracle's
restatements and the reference's own test cases
(tests/test_parallel.py:122-156, tests/test_core_contracts.py:142-149)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from avgen_amd import context as C
from avgen_amd.coords import PatchLayout, build_temporal_coords
from oracle import reference as R


def test_sharded_length_refuses_a_ragged_split():
    # reference tests/test_parallel.py:122-125
    assert C.sharded_length(64, 8) == 8
    with pytest.raises(ValueError, match="not divisible"):
        C.sharded_length(65, 8)
    with pytest.raises(ValueError, match="not divisible"):
        R.sharded_length(65, 8)
    assert C.shard_bounds(75600, 4, 3) == R.shard_bounds(75600, 4, 3) == (56700, 75600)
    with pytest.raises(ValueError):
        C.shard_bounds(64, 8, 8)


def test_pad_to_multiple_masks_the_padding():
    # reference tests/test_parallel.py:127-136: 10 tokens pad to 12, the two
    # padding positions are masked, an aligned stream is returned as is
    g = torch.Generator().manual_seed(0)
    tokens = torch.randn(2, 10, 6, generator=g)
    coords = torch.randn(2, 10, 3, generator=g)
    mask = torch.ones(2, 10, dtype=torch.bool)
    mask[1, 7:] = False
    t, c, m = C.pad_to_multiple(tokens, coords, mask, 4)
    assert t.shape == (2, 12, 6) and c.shape == (2, 12, 3) and m.shape == (2, 12)
    assert m[0, 10:].tolist() == [False, False] and m[0, :10].all()
    assert (t[:, 10:] == 0).all() and (c[:, 10:] == 0).all()
    assert torch.equal(t[:, :10], tokens) and torch.equal(m[:, :10], mask)
    rt, rc, rm = R.pad_to_multiple(tokens.numpy(), coords.numpy(), mask.numpy(), 4)
    assert np.array_equal(t.numpy(), rt) and np.array_equal(c.numpy(), rc) and np.array_equal(m.numpy(), rm)
    t8, c8, m8 = tokens[:, :8], coords[:, :8], mask[:, :8]
    out = C.pad_to_multiple(t8, c8, m8, 4)
    assert out[0] is t8 and out[1] is c8 and out[2] is m8
    with pytest.raises(ValueError):
        C.pad_to_multiple(tokens, coords, mask, 0)
    # the padded stream now splits; a ragged one does not
    assert C.sharded_length(t.shape[1], 4) == 3
    with pytest.raises(ValueError, match="not divisible"):
        C.shard_sequence(tokens, 4, 0)


def test_shard_takes_a_contiguous_slice_and_gathers_back():
    # reference tests/test_parallel.py:138-150
    stream = torch.arange(16, dtype=torch.float32)[None, :, None]
    seen = [C.shard_sequence(stream, 4, r).flatten().tolist() for r in range(4)]
    assert seen[0] == [0.0, 1.0, 2.0, 3.0]
    assert seen[3] == [12.0, 13.0, 14.0, 15.0]
    assert torch.equal(C.gather_tokens([C.shard_sequence(stream, 4, r) for r in range(4)]), stream)


def test_coords_carry_seconds_not_indices():
    # reference tests/test_core_contracts.py:142-149
    layout = PatchLayout(frames=4, height=4, width=4)
    positions = torch.tensor([[0.0, 0.04, 0.08, 0.12]])
    coords = build_temporal_coords(positions, layout)
    assert coords.shape == (1, layout.num_tokens, 3) and coords.dtype is torch.float32
    first = coords[0, : layout.grid[1] * layout.grid[2], 0]
    assert torch.equal(first, torch.zeros_like(first))
    assert torch.equal(coords[0, -1], torch.tensor([0.12, 2.0, 2.0]))


@pytest.mark.parametrize("patch,normalize", [((1, 2, 2), False), ((2, 2, 2), False), ((1, 1, 1), True),
                                             ((3, 2, 4), True), ((3, 2, 4), False)])
def test_coords_match_the_oracle_loop(patch, normalize):
    F_, H_, W_ = 6, 8, 12
    g = torch.Generator().manual_seed(1)
    positions = torch.sort(torch.rand(2, F_, generator=g) * 3.0, dim=1).values
    layout = PatchLayout(F_, H_, W_, *patch)
    got = build_temporal_coords(positions, layout, normalize_space=normalize).numpy()
    ref = R.temporal_coords(positions.numpy(), F_, H_, W_, patch, normalize)
    assert got.shape == ref.shape
    # spatial coordinates exactly; times are a mean of patch_frames values (one float32 rounding)
    assert np.array_equal(got[..., 1:], ref[..., 1:])
    assert np.abs(got[..., 0] - ref[..., 0]).max() <= 4e-7 * max(1.0, float(np.abs(ref[..., 0]).max()))
    if patch[0] == 1:
        assert np.array_equal(got[..., 0], ref[..., 0])
    if normalize:
        assert got[..., 1].min() == 0.0 and got[..., 1].max() == 1.0
        assert got[..., 2].min() == 0.0 and got[..., 2].max() == 1.0


def test_coords_closed_forms_and_errors():
    layout = PatchLayout(frames=4, height=4, width=6, patch_frames=2, patch_height=2, patch_width=3)
    assert layout.grid == (2, 2, 2) and layout.num_tokens == 8
    pos = torch.tensor([[0.0, 1.0, 2.0, 4.0]])
    c = build_temporal_coords(pos, layout)
    assert c[0, :, 0].tolist() == [0.5] * 4 + [3.0] * 4  # mean of each temporal patch
    assert c[0, :4, 1].tolist() == [0.0, 0.0, 2.0, 2.0]  # row * patch_height
    assert c[0, :4, 2].tolist() == [0.0, 3.0, 0.0, 3.0]  # column * patch_width
    with pytest.raises(ValueError, match="frames"):
        build_temporal_coords(torch.zeros(1, 3), layout)
    with pytest.raises(ValueError, match="divisible"):
        PatchLayout(frames=4, height=7, width=8, patch_height=2)


def test_benchmark_and_oracle_grids_follow_the_rule():
    """The synthetic coordinates of the benchmark and of the oracle (8 fps,
    2x2 patches, patch_frames 1) are build_temporal_coords of frame times f/8."""
    import bench

    F_, gh, gw = 3, 5, 7
    layout = PatchLayout(F_, 2 * gh, 2 * gw)
    ref = build_temporal_coords((torch.arange(F_, dtype=torch.float32) / 8.0)[None].expand(2, F_), layout)
    assert torch.equal(bench.video_coords(F_, gh, gw, 2, "cpu"), ref)
    assert np.array_equal(R.video_coords(F_, gh, gw, batch=2), ref.numpy())
