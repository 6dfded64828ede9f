"""Axial 3D rotary embeddings from physical coordinates, on gfx950 kernels.

Drop-in for ``avgen.models.rope`` (src/avgen/models/rope.py): same names,
signatures, argument meaning and exceptions.  Table construction
(:func:`build_rotary_tables`) and the rotation (:func:`apply_rotary`) run as
HIP kernels through ``libavattn.so``; the rotation is bit-identical to the
reference's fp32 elementwise chain (each product rounded separately, one
round to bf16), and differentiable.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import nn

from . import ops

__all__ = [
    "ROPE_SCALING_MODES",
    "RoPEScaling",
    "RotaryEmbedding",
    "RotaryTables",
    "apply_rotary",
    "build_rotary_tables",
    "inverse_frequencies",
    "rope_axis_pairs",
]

#: Frequency-scaling modes (src/avgen/models/rope.py:58).
ROPE_SCALING_MODES: tuple[str, ...] = ("none", "linear", "ntk")


@dataclass(frozen=True)
class RoPEScaling:
    """Frequency scaling for extrapolation (src/avgen/models/rope.py:61-125).

    ``"linear"`` divides positions by the factor; ``"ntk"`` raises the base by
    ``factor ** (dim / (dim - 2))``.  Time uses ``time_factor``; height and
    width use ``spatial_factor``.

    Raises:
        ValueError: unknown mode or a non-positive factor.
    """

    mode: str = "none"
    time_factor: float = 1.0
    spatial_factor: float = 1.0

    def __post_init__(self) -> None:
        if self.mode not in ROPE_SCALING_MODES:
            raise ValueError(f"mode must be one of {ROPE_SCALING_MODES}; got {self.mode!r}")
        for name in ("time_factor", "spatial_factor"):
            value = float(getattr(self, name))
            if not value > 0.0:
                raise ValueError(f"{name} must be positive; got {value!r}")

    @property
    def is_identity(self) -> bool:
        """Whether the frequencies are left untouched."""
        return self.mode == "none" or (self.time_factor == 1.0 and self.spatial_factor == 1.0)

    def factors(self) -> tuple[float, float, float]:
        """Per-axis factors ``(time, height, width)``."""
        return (self.time_factor, self.spatial_factor, self.spatial_factor)


def rope_axis_pairs(head_dim: int) -> tuple[int, int, int]:
    """Rotation-pair budgets ``(time, height, width)`` (src/avgen/models/rope.py:128-157).

    ``pairs = head_dim // 2``; height and width get ``pairs // 3`` each and time
    takes the remainder: 64 -> (12, 10, 10), 128 -> (22, 21, 21).

    Raises:
        ValueError: ``head_dim`` odd or below 6.
    """
    if head_dim < 6 or head_dim % 2 != 0:
        raise ValueError(
            f"head_dim must be an even integer of at least 6 so each rotary axis "
            f"gets at least one channel pair; got {head_dim!r}"
        )
    pairs = head_dim // 2
    spatial = pairs // 3
    return (pairs - 2 * spatial, spatial, spatial)


@dataclass(frozen=True)
class RotaryTables:
    """Per-pair cos/sin tables ``(batch, 1, length, pairs)`` float32
    (src/avgen/models/rope.py:160-216)."""

    cos: torch.Tensor
    sin: torch.Tensor

    @property
    def pairs(self) -> int:
        return int(self.cos.shape[-1])

    @property
    def length(self) -> int:
        return int(self.cos.shape[-2])

    @property
    def device(self) -> torch.device:
        return self.cos.device

    def validate(self) -> None:
        """Raise ValueError (rank/shape) or TypeError (dtype) like the reference."""
        if self.cos.ndim != 4 or self.sin.ndim != 4:
            raise ValueError(
                f"rotary tables must have rank 4 (batch, 1, length, pairs); got "
                f"{tuple(self.cos.shape)} and {tuple(self.sin.shape)}"
            )
        if self.cos.shape != self.sin.shape:
            raise ValueError(
                f"cos and sin must have the same shape; got {tuple(self.cos.shape)} and {tuple(self.sin.shape)}"
            )
        for name, tensor in (("cos", self.cos), ("sin", self.sin)):
            if tensor.dtype is not torch.float32:
                raise TypeError(f"{name} must be float32; got {tensor.dtype}")

    def slice(self, start: int, stop: int) -> "RotaryTables":
        """Tables for tokens ``[start, stop)`` (a context-parallel shard or KV chunk)."""
        return RotaryTables(cos=self.cos[:, :, start:stop], sin=self.sin[:, :, start:stop])


def inverse_frequencies(
    head_dim: int, *, theta: float = 10000.0, scaling: RoPEScaling | None = None
) -> tuple[list[float], list[int], tuple, tuple]:
    """Host-side frequency plan for :func:`build_rotary_tables`.

    Returns ``(inv_freq, axis_of_pair, pos_mul, pos_div)`` where inv_freq is
    computed with the reference's fp32 operations
    (src/avgen/models/rope.py:287-290: ``arange(pairs)/pairs`` then
    ``pow(float32(theta_axis), -exponent)``), evaluated on the CPU.  pos_mul
    is filled in by the caller (time_scale); pos_div[a] is the linear factor
    or None.
    """
    plan = scaling if scaling is not None else RoPEScaling()
    budgets = rope_axis_pairs(head_dim)
    inv: list[float] = []
    axes: list[int] = []
    divs: list[float | None] = [None, None, None]
    for axis, (pairs, factor) in enumerate(zip(budgets, plan.factors())):
        axis_theta = theta
        if plan.mode == "linear" and factor != 1.0:
            divs[axis] = float(factor)
        elif plan.mode == "ntk" and factor != 1.0:
            dim = 2 * pairs
            if dim > 2:
                axis_theta = theta * factor ** (dim / (dim - 2))
        exponent = torch.arange(pairs, dtype=torch.float32) / pairs
        freq = torch.pow(torch.tensor(axis_theta, dtype=torch.float32), -exponent)
        inv.extend(float(f) for f in freq.tolist())
        axes.extend([axis] * pairs)
    return inv, axes, (None, None, None), tuple(divs)


def build_rotary_tables(
    coords: torch.Tensor,
    *,
    head_dim: int,
    theta: float = 10000.0,
    time_scale: float = 1.0,
    scaling: RoPEScaling | None = None,
) -> RotaryTables:
    """Tables from ``coords (batch, length, 3)`` float32 (src/avgen/models/rope.py:218-294).

    Raises:
        ValueError: coords not ``(batch, length, 3)``.
        TypeError: coords not float32.
    """
    if coords.ndim != 3 or coords.shape[-1] != 3:
        raise ValueError(
            f"coords must be (batch, length, 3) as (seconds, row, column); got {tuple(coords.shape)}"
        )
    if coords.dtype is not torch.float32:
        raise TypeError(f"coords must be float32; got {coords.dtype}")
    inv, axes, _, divs = inverse_frequencies(head_dim, theta=theta, scaling=scaling)
    muls = (float(time_scale) if time_scale != 1.0 else None, None, None)
    cos, sin = ops.rope_tables(coords, inv, axes, muls, divs)
    return RotaryTables(cos=cos, sin=sin)


def apply_rotary(x: torch.Tensor, tables: RotaryTables) -> torch.Tensor:
    """Interleaved-pair rotation of ``x (batch, heads, length, head_dim)``
    (src/avgen/models/rope.py:297-338); returns a new tensor in x's dtype.

    Raises:
        ValueError: rank != 4, head_dim or length disagreeing with the tables.
    """
    if x.ndim != 4:
        raise ValueError(f"rotary input must be (batch, heads, length, head_dim); got {tuple(x.shape)}")
    if x.shape[-1] != 2 * tables.pairs:
        raise ValueError(
            f"head_dim {x.shape[-1]} does not match rotary tables built for head_dim {2 * tables.pairs}"
        )
    if x.shape[-2] != tables.length:
        raise ValueError(
            f"sequence length {x.shape[-2]} does not match rotary tables built for length {tables.length}; "
            "under context parallelism the tables must be built from the local coordinate shard"
        )
    return ops.rope_apply(x, tables.cos, tables.sin, False)


class RotaryEmbedding(nn.Module):
    """Stateless coords -> tables module (src/avgen/models/rope.py:341-401)."""

    def __init__(
        self,
        head_dim: int,
        *,
        theta: float = 10000.0,
        time_scale: float = 1.0,
        scaling: RoPEScaling | None = None,
    ) -> None:
        super().__init__()
        rope_axis_pairs(head_dim)
        self.head_dim = head_dim
        self.theta = theta
        self.time_scale = time_scale
        self.scaling = scaling if scaling is not None else RoPEScaling()

    def forward(self, coords: torch.Tensor) -> RotaryTables:
        return build_rotary_tables(
            coords, head_dim=self.head_dim, theta=self.theta, time_scale=self.time_scale, scaling=self.scaling
        )

    def extra_repr(self) -> str:
        budgets = rope_axis_pairs(self.head_dim)
        return (
            f"head_dim={self.head_dim}, pairs(t,h,w)={budgets}, theta={self.theta}, "
            f"time_scale={self.time_scale}, scaling={self.scaling.mode}"
        )
