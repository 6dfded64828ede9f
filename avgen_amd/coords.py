"""Token coordinates of a patchified video latent: the producer of the
``(seconds, row, column)`` positions the 3D RoPE tables are built from
(src/avgen/core/patchify.py:45-105, ``build_temporal_coords``; geometry of
src/avgen/core/tokens.py:43-111, ``PatchLayout``).

Host-side tensor code (any device): it runs once per forward, before the
rotary tables, and is not on the kernel path.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

__all__ = ["PatchLayout", "build_temporal_coords"]


@dataclass(frozen=True)
class PatchLayout:
    """Latent grid and patch sizes (src/avgen/core/tokens.py:43-111): the
    fields the coordinate rule reads, with the reference's defaults (patch
    1 x 2 x 2)."""

    frames: int
    height: int
    width: int
    patch_frames: int = 1
    patch_height: int = 2
    patch_width: int = 2

    def __post_init__(self) -> None:
        for name in ("frames", "height", "width", "patch_frames", "patch_height", "patch_width"):
            value = getattr(self, name)
            if not isinstance(value, int) or value < 1:
                raise ValueError(f"{name} must be a positive integer; got {value!r}")
        for size, patch in (("frames", "patch_frames"), ("height", "patch_height"), ("width", "patch_width")):
            if getattr(self, size) % getattr(self, patch) != 0:
                raise ValueError(f"{size}={getattr(self, size)} is not divisible by {patch}={getattr(self, patch)}")

    @property
    def grid(self) -> tuple[int, int, int]:
        """Post-patch ``(frames, height, width)``."""
        return (self.frames // self.patch_frames, self.height // self.patch_height, self.width // self.patch_width)

    @property
    def num_tokens(self) -> int:
        f, h, w = self.grid
        return f * h * w


def build_temporal_coords(
    positions: torch.Tensor, layout: PatchLayout, *, normalize_space: bool = False
) -> torch.Tensor:
    """``(batch, tokens, 3)`` float32 ``(seconds, row, column)`` per token, in
    token order time -> row -> column (src/avgen/core/patchify.py:45-105).

    ``positions``: ``(batch, frames)`` physical time in seconds of each latent
    frame before temporal patching.  A temporal patch's time is the mean of
    the frames it covers; rows and columns are grid indices times the patch
    size, or indices scaled into [0, 1] by the grid extent with
    ``normalize_space``.

    Raises:
        ValueError: ``positions`` does not have ``layout.frames`` frames.
    """
    batch, frames = tuple(positions.shape)
    if frames != layout.frames:
        raise ValueError(f"positions has {frames} frames but layout declares {layout.frames}")
    gf, gh, gw = layout.grid
    device = positions.device
    time = positions.reshape(batch, gf, layout.patch_frames).mean(dim=2)
    rows = torch.arange(gh, device=device, dtype=torch.float32)
    cols = torch.arange(gw, device=device, dtype=torch.float32)
    if normalize_space:
        rows = rows / max(gh - 1, 1)
        cols = cols / max(gw - 1, 1)
    else:
        rows = rows * layout.patch_height
        cols = cols * layout.patch_width
    shape = (batch, gf, gh, gw)
    return torch.stack(
        (
            time[:, :, None, None].expand(shape).reshape(batch, -1),
            rows[None, None, :, None].expand(shape).reshape(batch, -1),
            cols[None, None, None, :].expand(shape).reshape(batch, -1),
        ),
        dim=-1,
    ).to(torch.float32)
