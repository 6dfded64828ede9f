"""ctypes binding of ``libavattn.so`` (declared in ``include/avattn.h``).

The library is loaded lazily on first use and never silently replaced: if it
is missing or fails to load, every operation raises.  There is no CPU or
PyTorch fallback for the attention path.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

_PKG = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("AVATTN_LIB", _PKG / "libavattn.so"))

c_i32 = ctypes.c_int32
c_i64 = ctypes.c_int64
c_ptr = ctypes.c_void_p
c_f32 = ctypes.c_float
c_size = ctypes.c_size_t
c_i64p = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes); must mirror include/avattn.h exactly.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "avattn_strerror": (ctypes.c_char_p, [ctypes.c_int]),
    "avattn_abi_version": (ctypes.c_int, []),
    "avattn_fwd": (
        ctypes.c_int,
        [c_ptr, c_ptr, c_ptr, c_i64p, c_i64p, c_i64p,
         c_i32, c_i32, c_i32, c_i32, c_i32, c_i32,
         c_ptr, c_i64,
         c_ptr, c_ptr, c_i64,
         c_f32,
         c_ptr, c_i64p,
         c_ptr,
         c_ptr, c_size,
         c_ptr],
    ),
    "avattn_fwd_noalloc": (
        ctypes.c_int,
        [c_ptr, c_ptr, c_ptr, c_i64p, c_i64p, c_i64p,
         c_i32, c_i32, c_i32, c_i32, c_i32, c_i32,
         c_ptr, c_i64,
         c_ptr, c_ptr, c_i64,
         c_f32,
         c_ptr, c_i64p,
         c_ptr,
         c_ptr],
    ),
    "avattn_fwd_windowed": (
        ctypes.c_int,
        [c_ptr, c_ptr, c_ptr, c_i64p, c_i64p, c_i64p,
         c_i32, c_i32, c_i32, c_i32, c_i32, c_i32,
         c_ptr, c_i64,
         c_ptr, c_ptr, c_i64,
         c_f32,
         c_ptr, c_i64p, c_ptr,
         c_ptr, c_size,
         c_ptr],
    ),
    "avattn_fwd_workspace_size": (c_size, [c_i32, c_i32, c_i32, c_i32]),
    "avattn_fwd_fp8": (
        ctypes.c_int,
        [c_ptr, c_ptr, c_ptr, c_i64p, c_i64p, c_i64p,
         c_i32, c_i32, c_i32, c_i32, c_i32, c_i32,
         c_ptr, c_i64,
         c_ptr, c_ptr,
         c_f32,
         c_ptr, c_i64p,
         c_ptr,
         c_ptr, c_size,
         c_ptr],
    ),
    "avattn_fwd_fp8_workspace_size": (c_size, [c_i32, c_i32, c_i32, c_i32]),
    "avattn_fp8_absmax_scales": (ctypes.c_int, [c_ptr, c_i64p, c_i32, c_i32, c_i32, c_i32, c_ptr, c_ptr]),
    "avattn_bwd_workspace_size": (c_size, [c_i32, c_i32, c_i32, c_i32, c_i32, c_i32]),
    "avattn_bwd_staged_workspace_size": (c_size, [c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32]),
    "avattn_bwd_dq_staged": (
        ctypes.c_int,
        [c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, ctypes.c_float, c_ptr, c_i64p, c_ptr, c_size, ctypes.c_uint32,
         c_ptr],
    ),
    "avattn_bwd": (
        ctypes.c_int,
        [c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr,
         c_i64p, c_i64p, c_i64p, c_i64p, c_i64p,
         c_i32, c_i32, c_i32, c_i32, c_i32, c_i32,
         c_ptr, c_i64,
         c_f32,
         c_ptr, c_i64p, c_ptr, c_i64p, c_ptr, c_i64p,
         c_ptr, c_size,
         ctypes.c_uint32,
         c_ptr],
    ),
    "avattn_bwd_windowed": (
        ctypes.c_int,
        [c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr,
         c_i64p, c_i64p, c_i64p, c_i64p, c_i64p,
         c_i32, c_i32, c_i32, c_i32, c_i32, c_i32,
         c_ptr, c_i64,
         c_ptr, c_ptr, c_i64,
         c_f32,
         c_ptr, c_i64p, c_ptr, c_i64p, c_ptr, c_i64p,
         c_ptr, c_size,
         ctypes.c_uint32,
         c_ptr],
    ),
    "avattn_bwd_windowed_compact": (
        ctypes.c_int,
        [c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr,
         c_i64p, c_i64p, c_i64p, c_i64p, c_i64p,
         c_i32, c_i32, c_i32, c_i32, c_i32, c_i32,
         c_ptr, c_i64,
         c_ptr, c_ptr, c_i64,
         c_ptr, c_i64, c_i64,
         c_f32,
         c_ptr, c_i64p, c_ptr, c_i64p, c_ptr, c_i64p,
         c_ptr, c_size,
         ctypes.c_uint32,
         c_ptr],
    ),
    "avattn_bwd_compact_workspace_size": (c_size, [c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_i64]),
    "avattn_ring_fwd_step": (
        ctypes.c_int,
        [c_ptr, c_ptr, c_ptr, c_i64p, c_i64p, c_i64p,
         c_i32, c_i32, c_i32, c_i32, c_i32, c_i32,
         c_ptr, c_i64,
         c_ptr, c_ptr, c_i64,
         c_ptr, c_ptr, c_i64,
         c_f32,
         c_ptr, c_ptr,
         c_ptr, c_i64p,
         ctypes.c_uint32,
         c_ptr, c_size,
         c_ptr],
    ),
    "avattn_ring_bwd_step": (
        ctypes.c_int,
        [c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr,
         c_i64p, c_i64p, c_i64p, c_i64p, c_i64p,
         c_i32, c_i32, c_i32, c_i32, c_i32, c_i32,
         c_ptr, c_i64,
         c_ptr, c_ptr, c_i64,
         c_ptr, c_ptr, c_i64,
         c_f32,
         c_ptr, c_i64p, c_ptr, c_i64p, c_ptr, c_i64p,
         c_ptr, c_size,
         ctypes.c_uint32,
         c_ptr],
    ),
    "avattn_ring_dq_finish": (
        ctypes.c_int,
        [c_ptr, c_i64p, c_i32, c_i32, c_i32, c_i32, c_ptr, c_ptr, c_i64, c_ptr, c_i64p, c_ptr],
    ),
    "avattn_lse_merge": (ctypes.c_int, [c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i32, c_i32, c_ptr]),
    "avattn_rope_tables": (
        ctypes.c_int,
        [c_ptr, c_i64, c_i64, c_i32, c_i32, c_i32,
         c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr,
         c_ptr, c_ptr, c_ptr],
    ),
    "avattn_rope_apply": (
        ctypes.c_int,
        [c_ptr, c_i64p, c_i32, c_i32, c_i32, c_i32,
         c_ptr, c_ptr, c_i64, c_i32,
         c_ptr, c_i64p, c_ptr],
    ),
    "avattn_qk_norm_rope": (
        ctypes.c_int,
        [c_ptr, c_i64p, c_i32, c_i32, c_i32, c_i32, c_ptr, c_f32,
         c_ptr, c_ptr, c_i64, c_ptr, c_i64p, c_ptr],
    ),
    "avattn_qk_norm_rope_bwd_workspace_size": (c_size, [c_i32]),
    "avattn_qk_norm_rope_bwd": (
        ctypes.c_int,
        [c_ptr, c_i64p, c_ptr, c_i64p, c_i32, c_i32, c_i32, c_i32, c_ptr, c_f32,
         c_ptr, c_ptr, c_i64, c_ptr, c_i64p, c_ptr, c_ptr, c_size, c_ptr],
    ),
    "avattn_timing_begin": (ctypes.c_int, [c_i32]),
    "avattn_timing_end": (ctypes.c_int, []),
    "avattn_timing_read": (ctypes.c_int, [c_i32, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int32)]),
    "avattn_timing_reset": (ctypes.c_int, []),
    "avattn_diag_dq_partials": (ctypes.c_int, [ctypes.c_void_p] + [c_i32] * 6 + [ctypes.c_void_p]),
    "avattn_fwd_f32": (
        ctypes.c_int,
        [c_ptr, c_ptr, c_ptr, c_i64p, c_i64p, c_i64p,
         c_i32, c_i32, c_i32, c_i32, c_i32, c_i32,
         c_ptr, c_i64,
         c_f32,
         c_ptr, c_i64p,
         c_ptr,
         c_ptr],
    ),
    "avattn_bwd_f32_workspace_size": (c_size, [c_i32, c_i32, c_i32]),
    "avattn_bwd_f32_staged_workspace_size": (c_size, [c_i32, c_i32, c_i32, c_i32, c_i32, c_i32]),
    "avattn_bwd_f32": (
        ctypes.c_int,
        [c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr,
         c_i64p, c_i64p, c_i64p, c_i64p, c_i64p,
         c_i32, c_i32, c_i32, c_i32, c_i32, c_i32,
         c_ptr, c_i64,
         c_f32,
         c_ptr, c_i64p, c_ptr, c_i64p, c_ptr, c_i64p,
         c_ptr, c_size,
         c_ptr],
    ),
    "avattn_fwd_windowed_f32": (
        ctypes.c_int,
        [c_ptr, c_ptr, c_ptr, c_i64p, c_i64p, c_i64p,
         c_i32, c_i32, c_i32, c_i32, c_i32, c_i32,
         c_ptr, c_i64,
         c_ptr, c_ptr, c_i64,
         c_f32,
         c_ptr, c_i64p,
         c_ptr,
         c_ptr],
    ),
    "avattn_bwd_windowed_f32": (
        ctypes.c_int,
        [c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr,
         c_i64p, c_i64p, c_i64p, c_i64p, c_i64p,
         c_i32, c_i32, c_i32, c_i32, c_i32, c_i32,
         c_ptr, c_i64,
         c_ptr, c_ptr, c_i64,
         c_f32,
         c_ptr, c_i64p, c_ptr, c_i64p, c_ptr, c_i64p,
         c_ptr, c_size,
         c_ptr],
    ),
    "avattn_qk_norm_rope_f32": (
        ctypes.c_int,
        [c_ptr, c_i64p, c_i32, c_i32, c_i32, c_i32, c_ptr, c_f32, c_ptr, c_ptr, c_i64,
         c_ptr, c_i64p, c_ptr],
    ),
    "avattn_qk_norm_rope_bwd_f32": (
        ctypes.c_int,
        [c_ptr, c_i64p, c_ptr, c_i64p, c_i32, c_i32, c_i32, c_i32, c_ptr, c_f32, c_ptr, c_ptr, c_i64,
         c_ptr, c_i64p, c_ptr, c_ptr, c_size, c_ptr],
    ),
    "avattn_rope_apply_f32": (
        ctypes.c_int,
        [c_ptr, c_i64p, c_i32, c_i32, c_i32, c_i32,
         c_ptr, c_ptr, c_i64, c_i32,
         c_ptr, c_i64p, c_ptr],
    ),
}

# Status codes (include/avattn.h).
OK = 0
ERR_NULL_POINTER = 1
ERR_BAD_SHAPE = 2
ERR_HEAD_DIM = 3
ERR_GQA = 4
ERR_LAYOUT = 5
ERR_WORKSPACE = 6
ERR_LAUNCH = 7
ERR_TOO_LARGE = 8
ERR_ARGUMENT = 9
ERR_SCRATCH = 10

#: Bytes of avattn_fwd_noalloc's fixed per-GPU scratch (AVATTN_FWD_NOALLOC_SCRATCH).
FWD_NOALLOC_SCRATCH = 64 << 20

# avattn_bwd flags (include/avattn.h).
BWD_REUSE_QUERY_SIDE = 1
BWD_DQ_ACCUMULATE_F32 = 2
BWD_STAGE_DS = 4
BWD_DEFER_DQ = 8

# avattn_ring_fwd_step flags (include/avattn.h).
RING_FIRST = 1
RING_LAST = 2

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class AvattnError(RuntimeError):
    """A C-ABI call returned a non-zero status."""

    def __init__(self, status: int, where: str, message: str) -> None:
        super().__init__(f"{where}: {message} (avattn status {status})")
        self.status = status


def load() -> ctypes.CDLL:
    """Load and bind the library once; raise if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"avattn HIP library not found at {LIB_PATH}; build it with "
                "`python -m avgen_amd.build` (no fallback path exists)"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def strerror(status: int) -> str:
    """Text of a status code."""
    return load().avattn_strerror(status).decode()


def check(status: int, where: str) -> None:
    """Raise :class:`AvattnError` (or a mapped builtin) for a failing status."""
    if status == OK:
        return
    msg = strerror(status)
    if status in (ERR_BAD_SHAPE, ERR_HEAD_DIM, ERR_GQA, ERR_TOO_LARGE):
        raise ValueError(f"{where}: {msg}")
    raise AvattnError(status, where, msg)


def i64_array(values) -> ctypes.Array:
    """A C ``int64_t[]`` holding ``values``."""
    vals = [int(v) for v in values]
    return (ctypes.c_int64 * len(vals))(*vals)


#: Kernel ids of the launch timer (include/avattn.h).
KERNEL_IDS = {
    "attn_fwd": 0,
    "bwd_preprocess": 1,
    "bwd_dkdv": 2,
    "bwd_dq": 3,
    "lse_merge": 4,
    "rope_apply": 5,
    "rope_tables": 6,
    "transpose": 7,
    "attn_fwd_fp8": 8,
    "fp8_absmax": 9,
    "bwd_dq_ds": 10,
    "qk_norm": 11,
    "qk_norm_bwd": 12,
    "ring_dq_finish": 13,
    "dkv_reduce": 14,
    "diag_dq_partials": 15,
}


class LaunchTiming:
    """Context manager: per-kernel HIP-event timing of this library's launches.

    ``with LaunchTiming(4096) as t: ...; t.read("attn_fwd") -> (total_ms, launches)``.
    Reading synchronizes on the recorded events.
    """

    def __init__(self, capacity: int = 4096) -> None:
        self.capacity = capacity

    def __enter__(self) -> "LaunchTiming":
        check(load().avattn_timing_begin(self.capacity), "avattn_timing_begin")
        return self

    def __exit__(self, *exc) -> None:
        load().avattn_timing_end()

    def read(self, kernel: str) -> tuple[float, int]:
        ms = ctypes.c_double()
        n = ctypes.c_int32()
        check(load().avattn_timing_read(KERNEL_IDS[kernel], ctypes.byref(ms), ctypes.byref(n)), "avattn_timing_read")
        return ms.value, n.value

    def close(self) -> None:
        load().avattn_timing_reset()
