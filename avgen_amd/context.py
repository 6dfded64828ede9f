"""Context-parallel sequence sharding rules the ring local step depends on.

Restates the contiguous-shard contract of src/avgen/parallel/context.py on
plain tensors (the TokenStream container is outside this package): shard r
of ``cp`` holds tokens ``[r*L/cp, (r+1)*L/cp)``; ragged lengths are rejected;
explicit right-padding carries a False mask and zero coordinates/features.
The emulated ring splits keys/values into chunks by exactly this rule, so a
chunk's rotary tables are the same contiguous slice of the full tables.
"""

from __future__ import annotations

from collections.abc import Sequence

import torch

__all__ = [
    "gather_tokens",
    "pad_to_multiple",
    "shard_bounds",
    "shard_sequence",
    "sharded_length",
]


def sharded_length(total: int, shards: int) -> int:
    """Per-shard length, requiring an exact split (src/avgen/parallel/context.py:58-80).

    Raises:
        ValueError: ``total`` not divisible by ``shards``.
    """
    if total % shards != 0:
        raise ValueError(
            f"sequence length {total} is not divisible by context-parallel "
            f"degree {shards}; pad the sequence with pad_to_multiple() at the "
            "data boundary so the padding is explicit and masked"
        )
    return total // shards


def shard_bounds(total: int, shards: int, index: int) -> tuple[int, int]:
    """``[start, stop)`` of shard ``index`` (src/avgen/parallel/context.py:159-163)."""
    if not 0 <= index < shards:
        raise ValueError(f"shard index {index} out of range for {shards} shards")
    local = sharded_length(total, shards)
    return index * local, (index + 1) * local


def shard_sequence(tensor: torch.Tensor, shards: int, index: int, dim: int = 1) -> torch.Tensor:
    """Contiguous slice ``index`` of ``shards`` along ``dim`` (a view)."""
    start, stop = shard_bounds(tensor.shape[dim], shards, index)
    return tensor.narrow(dim, start, stop - start)


def gather_tokens(parts: Sequence[torch.Tensor], dim: int = 1) -> torch.Tensor:
    """Single-GPU stand-in for the all-gather along the sequence
    (src/avgen/parallel/context.py:213-229): concatenation in shard order."""
    return torch.cat(list(parts), dim=dim)


def pad_to_multiple(
    tokens: torch.Tensor, coords: torch.Tensor, mask: torch.Tensor, multiple: int
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Right-pad ``(B, L, ...)`` tokens/coords and ``(B, L)`` mask so L divides
    ``multiple`` (src/avgen/parallel/context.py:83-139): padding tokens and
    coordinates are zero and the mask is False.

    Raises:
        ValueError: ``multiple`` not positive.
    """
    if multiple < 1:
        raise ValueError(f"multiple must be positive; got {multiple!r}")
    length = tokens.shape[1]
    remainder = length % multiple
    if remainder == 0:
        return tokens, coords, mask
    pad = multiple - remainder

    def _pad(t: torch.Tensor) -> torch.Tensor:
        shape = list(t.shape)
        shape[1] = pad
        return torch.cat((t, torch.zeros(shape, dtype=t.dtype, device=t.device)), dim=1)

    return _pad(tokens), _pad(coords), _pad(mask)
