"""MI355X (gfx950)-native video-DiT attention hot path.

Hand-written HIP kernels (``csrc/``) behind the C ABI in ``include/avattn.h``
(``libavattn.so``), with host modules that mirror the reference's Python
interfaces:

* :mod:`avgen_amd.attention` — ``attention`` / ``key_padding_mask`` (drop-in
  for ``avgen.models.attention``) and the fused ``rotary_attention``;
* :mod:`avgen_amd.rope` — 3D RoPE tables and rotation (``avgen.models.rope``);
* :mod:`avgen_amd.ring` — ring local step, LSE merger, emulated ring;
* :mod:`avgen_amd.context` — contiguous context-parallel shard rules;
* :mod:`avgen_amd.ops` — the ``torch.library`` ops over the C ABI.
"""

from . import attention, context, layers, ops, ring, rope
from .attention import attention as attention_fn
from .attention import key_padding_mask, rotary_attention
from .ring import SDPAMerger, flash_attention_backward_op, flash_attention_op, ring_attention
from .rope import RotaryEmbedding, RotaryTables, apply_rotary, build_rotary_tables, rope_axis_pairs

__all__ = [
    "RotaryEmbedding",
    "RotaryTables",
    "SDPAMerger",
    "apply_rotary",
    "attention",
    "attention_fn",
    "build_rotary_tables",
    "context",
    "flash_attention_backward_op",
    "flash_attention_op",
    "key_padding_mask",
    "layers",
    "ops",
    "ring",
    "ring_attention",
    "rope",
    "rope_axis_pairs",
    "rotary_attention",
]
