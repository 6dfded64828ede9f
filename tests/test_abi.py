"""The C-ABI library: loads without a GPU, exports every symbol declared in
include/avattn.h, and rejects bad arguments before touching the device.

None of these calls launches a kernel: every case returns from argument
validation, which runs before any HIP API call.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from avgen_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "avattn.h"


def _declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(avattn_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} not built; run `python -m avgen_amd.build`")
    return _lib.load()


def _no_device() -> bool:
    import torch

    return not torch.cuda.is_available()


# The validation cases pass fake device addresses.  They are meant to return
# from argument checking, but if a check regressed the call would launch a
# kernel on garbage pointers, so they only run where no GPU is visible.
cpu_only = pytest.mark.skipif(not _no_device(), reason="fake-pointer validation tests run only without a GPU")


def test_every_declared_symbol_is_exported_and_bound(lib):
    names = _declared_functions()
    assert names == sorted(_lib.SIGNATURES), "ctypes signature table out of sync with include/avattn.h"
    for name in names:
        assert hasattr(lib, name), name


def test_strerror_and_version(lib):
    assert lib.avattn_abi_version() == 14
    for code in range(0, 11):
        assert lib.avattn_strerror(code)
    assert b"unknown" in lib.avattn_strerror(12345)


def _round256(x: int) -> int:
    return (x + 255) // 256 * 256


def _pad64(n: int) -> int:
    return (n + 63) // 64 * 64


def _key_regions(B: int, lkp: int) -> int:
    # key bias (B, Lkp) floats and (B, Lkp/32) int flags, each + a 64-entry tail pad
    return _round256((B * lkp + 64) * 4) + _round256((B * (lkp // 32) + 64) * 4)


def test_workspace_size(lib):
    # Sequences pad to whole 64-row tiles: 18900 -> 18944; every region starts
    # on a 256-byte boundary.
    lp = _pad64(18900)
    assert lp == 18944
    copy = 2 * 40 * 128 * lp * 2  # one bf16 copy of a (2, 40, 18900, 128) tensor
    stats = 2 * 40 * lp * 4
    # backward: lse2 + ndelta, q/dout row copies, k/v rows + k^T, and when the dK/dV grid (one workgroup per 128 keys of a (batch,
    # kv head)) has more than 256 workgroups, 512 slots of 256 x head_dim
    # fp32 partial sums for the split of the grid's last round
    def split(D):
        return 512 * 256 * D * 4

    assert lib.avattn_bwd_workspace_size(2, 40, 40, 18900, 18900, 128) == (
        2 * stats + 5 * copy + _key_regions(2, lp) + split(128))
    # exactly 256 dK/dV blocks (1 x 2 x 128 of 128 keys) and 2 dQ blocks: no region
    lp2 = _pad64(128 * 128)
    assert lib.avattn_bwd_workspace_size(1, 2, 2, 64, 128 * 128, 64) == (
        2 * (2 * 64 * 4) + 2 * (2 * 64 * 64 * 2) + 3 * (2 * 64 * lp2 * 2) + _key_regions(1, lp2))
    lp3 = _pad64(128 * 128 + 1)
    assert lib.avattn_bwd_workspace_size(1, 2, 2, 64, 128 * 128 + 1, 64) == (
        2 * (2 * 64 * 4) + 2 * (2 * 64 * 64 * 2) + 3 * (2 * 64 * lp3 * 2) + _key_regions(1, lp3) + split(64))
    # one dK/dV block per head (40 x 74 dQ workgroups do not count): no region
    assert lib.avattn_bwd_workspace_size(1, 40, 40, 18900, 64, 128) == (
        2 * (40 * lp * 4) + 2 * (40 * 128 * lp * 2) + 3 * (40 * 128 * 64 * 2) + _key_regions(1, 64))
    # GQA: k/v copies have heads_kv heads (len_k 70 pads to 128, len_q 10 to 64).
    got = lib.avattn_bwd_workspace_size(1, 4, 2, 10, 70, 64)
    assert got == 2 * (4 * 64 * 4) + 2 * (4 * 64 * 64 * 2) + 3 * (2 * 64 * 128 * 2) + _key_regions(1, 128)
    assert lib.avattn_bwd_workspace_size(1, 1, 1, 1, 1, 64) == 2 * 256 + 5 * 64 * 64 * 2 + _key_regions(1, 64)
    assert lib.avattn_bwd_workspace_size(0, 40, 40, 10, 10, 128) == 0
    # forward: k rows + v^T copies of (B, Hkv, Lk, D), key bias/flags, one
    # max squared k row norm per (b, kv head, 64-key tile)
    assert lib.avattn_fwd_workspace_size(2, 8, 18900, 128) == (
        2 * (2 * 8 * 128 * lp * 2) + _key_regions(2, lp) + _round256(2 * 8 * (lp // 64) * 4))
    assert lib.avattn_fwd_workspace_size(1, 1, 0, 128) == 0
    # fp8 forward: the k copy is e4m3 (one byte per element)
    assert lib.avattn_fwd_fp8_workspace_size(2, 8, 18900, 128) == (
        2 * 8 * 128 * lp + 2 * 8 * 128 * lp * 2 + _key_regions(2, lp) + _round256(2 * 8 * (lp // 64) * 4))
    assert lib.avattn_fwd_fp8_workspace_size(1, 1, 70, 64) == (
        _round256(128 * 64) + 128 * 64 * 2 + _key_regions(1, 128) + 256)
    assert lib.avattn_fwd_fp8_workspace_size(1, 1, 0, 128) == 0


def test_staged_workspace_size(lib):
    # base workspace rounded up to 4 KB, then 8 KB per (query head, 32-row
    # group of the 64-padded rows, 128-key block) for each pair of a pass
    def r4k(x):
        return (x + 4095) // 4096 * 4096

    base = lib.avattn_bwd_workspace_size(2, 40, 40, 18900, 18900, 128)
    per = (18944 // 32) * ((18900 + 127) // 128) * 8192
    assert per == 18944 * 18944 * 2
    assert lib.avattn_bwd_staged_workspace_size(2, 40, 40, 18900, 18900, 128, 1) == r4k(base) + per
    assert lib.avattn_bwd_staged_workspace_size(2, 40, 40, 18900, 18900, 128, 8) == r4k(base) + 8 * per
    assert lib.avattn_bwd_staged_workspace_size(2, 40, 40, 18900, 18900, 128, 1000) == r4k(base) + 80 * per
    # GQA: every query head of the pair's group (2 here); len_q 10 -> 64 rows, len_k 70 -> one block
    base = lib.avattn_bwd_workspace_size(1, 4, 2, 10, 70, 64)
    assert lib.avattn_bwd_staged_workspace_size(1, 4, 2, 10, 70, 64, 2) == r4k(base) + 2 * (2 * 2 * 1 * 8192)
    assert lib.avattn_bwd_staged_workspace_size(1, 4, 2, 10, 70, 64, 0) == 0
    assert lib.avattn_bwd_staged_workspace_size(0, 4, 2, 10, 70, 64, 1) == 0
    assert lib.avattn_bwd_staged_workspace_size(1, 4, 2, 0, 70, 64, 1) == 0


def _fwd(lib, **over):
    s = _lib.i64_array([1024 * 128, 1024 * 128, 128])
    args = dict(q=16, k=16, v=16, qs=s, ks=s, vs=s, B=1, Hq=2, Hkv=2, Lq=4, Lk=4, D=128, mask=None, msb=0,
                cos=None, sin=None, rsb=0, scale=0.125, out=16, os=s, lse=16, ws=256, wsb=1 << 20, stream=None)
    args.update(over)
    return lib.avattn_fwd(args["q"], args["k"], args["v"], args["qs"], args["ks"], args["vs"], args["B"],
                          args["Hq"], args["Hkv"], args["Lq"], args["Lk"], args["D"], args["mask"], args["msb"],
                          args["cos"], args["sin"], args["rsb"], args["scale"], args["out"], args["os"],
                          args["lse"], args["ws"], args["wsb"], args["stream"])


@cpu_only
def test_fwd_validation_paths(lib):
    # Fake (never dereferenced) but aligned addresses; each case fails validation.
    assert _fwd(lib, D=96) == _lib.ERR_HEAD_DIM
    assert _fwd(lib, Hq=3, Hkv=2) == _lib.ERR_GQA
    assert _fwd(lib, Lq=-1) == _lib.ERR_BAD_SHAPE
    assert _fwd(lib, scale=0.0) == _lib.ERR_ARGUMENT
    assert _fwd(lib, scale=float("nan")) == _lib.ERR_ARGUMENT
    assert _fwd(lib, cos=16) == _lib.ERR_ARGUMENT
    assert _fwd(lib, q=None) == _lib.ERR_NULL_POINTER
    assert _fwd(lib, qs=None) == _lib.ERR_NULL_POINTER
    assert _fwd(lib, q=8) == _lib.ERR_LAYOUT
    assert _fwd(lib, qs=_lib.i64_array([1024 * 128, 1024 * 128, 100])) == _lib.ERR_LAYOUT
    assert _fwd(lib, k=None) == _lib.ERR_NULL_POINTER
    assert _fwd(lib, mask=16, msb=2) == _lib.ERR_ARGUMENT
    assert _fwd(lib, B=1, Hq=1 << 30, Hkv=1, Lq=1 << 20) == _lib.ERR_TOO_LARGE
    # 32-bit buffer ranges: one padded (b, head) slice of k (Lkp*D*2 bytes).
    # The query heads of one group (group*Lqp*D*2) bound only the backward.
    assert _fwd(lib, Lk=(1 << 24) - 64) == _lib.ERR_WORKSPACE  # 4 GiB - 16 KiB per slice: still addressable
    assert _fwd(lib, Lk=1 << 24) == _lib.ERR_TOO_LARGE
    # lengths within 63 of INT32_MAX: the padded length is computed in 64 bits
    assert _fwd(lib, Lk=(1 << 31) - 1) == _lib.ERR_TOO_LARGE
    assert _fwd(lib, Lk=(1 << 31) - 40) == _lib.ERR_TOO_LARGE
    # MQA with a long query: 40 * 420k rows * 256 B >= 2^32, fine for the forward
    assert _fwd(lib, Hq=40, Hkv=1, Lq=420_000, ws=8) == _lib.ERR_WORKSPACE
    assert _fwd(lib, Hq=40, Hkv=1, Lq=400_000, ws=8) == _lib.ERR_WORKSPACE
    assert _fwd(lib, ws=None) == _lib.ERR_WORKSPACE
    assert _fwd(lib, wsb=100) == _lib.ERR_WORKSPACE  # needs more than 2 * (2*128*64*2) bytes
    assert _fwd(lib, ws=8) == _lib.ERR_WORKSPACE
    # empty problems succeed without any launch
    assert _fwd(lib, Lq=0) == _lib.OK
    assert _fwd(lib, B=0) == _lib.OK


@cpu_only
def test_fwd_noalloc_rejects_before_any_device_call(lib):
    """Shape errors and problems beyond the fixed scratch return before the
    library touches the device (no GPU here: a HIP call would fail)."""
    s = _lib.i64_array([1 << 30, 1 << 20, 128])

    def call(B=1, Hq=2, Hkv=2, Lq=4, Lk=4, D=128):
        return lib.avattn_fwd_noalloc(16, 16, 16, s, s, s, B, Hq, Hkv, Lq, Lk, D, None, 0, None, None, 0, 0.125,
                                      16, s, 16, None)

    assert call(D=96) == _lib.ERR_HEAD_DIM
    assert call(Hq=3) == _lib.ERR_GQA
    assert call(Lk=-1) == _lib.ERR_BAD_SHAPE
    # k and v copies of (1, 2, 2^17, 128) bf16 are 128 MiB > 64 MiB
    assert lib.avattn_fwd_workspace_size(1, 2, 1 << 17, 128) > _lib.FWD_NOALLOC_SCRATCH
    assert call(Lk=1 << 17) == _lib.ERR_SCRATCH
    assert lib.avattn_fwd_workspace_size(1, 2, 60000, 128) <= _lib.FWD_NOALLOC_SCRATCH
    assert call(Lq=0) == _lib.OK
    assert b"64 MiB" in lib.avattn_strerror(_lib.ERR_SCRATCH)


def _fwd_windowed(lib, lo=32, hi=32, wb=0, **over):
    s = _lib.i64_array([1024 * 128, 1024 * 128, 128])
    a = dict(q=16, k=16, v=16, qs=s, ks=s, vs=s, B=2, Hq=2, Hkv=2, Lq=4, Lk=4, D=128, mask=None, msb=0,
             scale=0.125, out=16, os=s, lse=16, ws=256, wsb=1 << 20, stream=None)
    a.update(over)
    return lib.avattn_fwd_windowed(a["q"], a["k"], a["v"], a["qs"], a["ks"], a["vs"], a["B"], a["Hq"], a["Hkv"],
                                   a["Lq"], a["Lk"], a["D"], a["mask"], a["msb"], lo, hi, wb, a["scale"],
                                   a["out"], a["os"], a["lse"], a["ws"], a["wsb"], a["stream"])


@cpu_only
def test_windowed_validation_paths(lib):
    assert _fwd_windowed(lib, lo=None) == _lib.ERR_NULL_POINTER
    assert _fwd_windowed(lib, hi=None) == _lib.ERR_NULL_POINTER
    assert _fwd_windowed(lib, lo=34) == _lib.ERR_LAYOUT
    assert _fwd_windowed(lib, wb=3) == _lib.ERR_ARGUMENT  # batch stride below len_q
    assert _fwd_windowed(lib, wb=4, ws=8) == _lib.ERR_WORKSPACE  # valid windows reach the workspace check
    assert _fwd_windowed(lib, wb=0, ws=8) == _lib.ERR_WORKSPACE
    assert _fwd_windowed(lib, D=96) == _lib.ERR_HEAD_DIM
    assert _fwd_windowed(lib, Lq=0) == _lib.OK
    s = _lib.i64_array([1 << 17, 1 << 17, 128])
    staged = lib.avattn_bwd_staged_workspace_size(1, 2, 2, 4, 4, 128, 2)

    def bwd(lo, hi, wb, ws_bytes, flags):
        return lib.avattn_bwd_windowed(16, 16, 16, 16, 16, 16, s, s, s, s, s, 1, 2, 2, 4, 4, 128, None, 0,
                                       lo, hi, wb, 0.125, 16, s, 16, s, 16, s, 16, ws_bytes, flags, None)

    assert bwd(None, 32, 0, staged, _lib.BWD_STAGE_DS) == _lib.ERR_NULL_POINTER
    assert bwd(32, 32, 0, staged, 0) == _lib.ERR_ARGUMENT  # windows need staged dS
    assert bwd(32, 32, 0, staged, _lib.BWD_STAGE_DS | _lib.BWD_DEFER_DQ) == _lib.ERR_ARGUMENT
    assert bwd(32, 32, 2, staged, _lib.BWD_STAGE_DS) == _lib.ERR_ARGUMENT
    assert bwd(34, 32, 0, staged, _lib.BWD_STAGE_DS) == _lib.ERR_LAYOUT
    one_pair = lib.avattn_bwd_staged_workspace_size(1, 2, 2, 4, 4, 128, 1)
    assert bwd(32, 32, 0, one_pair - 1, _lib.BWD_STAGE_DS) == _lib.ERR_WORKSPACE


@cpu_only
def test_bwd_validation_paths(lib):
    s = _lib.i64_array([1 << 17, 1 << 17, 128])
    base = [16, 16, 16, 16, 16, 16, s, s, s, s, s, 1, 2, 2, 4, 4, 128, None, 0, 0.125,
            16, s, 16, s, 16, s, 16, 8, 0, None]
    assert lib.avattn_bwd(*base) == _lib.ERR_WORKSPACE  # 8 bytes < 2*1*2*4*4
    # the query heads of one group go through one 32-bit range in the backward
    mqa = list(base)
    mqa[12], mqa[13], mqa[14] = 40, 1, 420_000  # heads_q, heads_kv, len_q
    assert lib.avattn_bwd(*mqa) == _lib.ERR_TOO_LARGE
    mqa[14] = 400_000  # 40 * 400k rows * 256 B < 2^32: valid, fails on the workspace
    assert lib.avattn_bwd(*mqa) == _lib.ERR_WORKSPACE
    assert lib.avattn_bwd_dq_staged(1, 40, 1, 420_000, 4, 128, 0.125, 16, s, 16, 1 << 20, 0, None) == \
        _lib.ERR_TOO_LARGE
    bad = list(base)
    bad[28] = 8  # unknown flag
    assert lib.avattn_bwd(*bad) == _lib.ERR_ARGUMENT
    # staged dS needs the base workspace (4 KB aligned) plus one pair's dS
    bad = list(base)
    bad[28] = _lib.BWD_STAGE_DS
    need = lib.avattn_bwd_workspace_size(1, 2, 2, 4, 4, 128)
    bad[27] = need
    assert lib.avattn_bwd(*bad) == _lib.ERR_WORKSPACE
    bad[27] = lib.avattn_bwd_staged_workspace_size(1, 2, 2, 4, 4, 128, 1) - 1
    assert lib.avattn_bwd(*bad) == _lib.ERR_WORKSPACE
    # a deferred dq needs staging, and every pair's dS at once (2 pairs here)
    bad[28] = _lib.BWD_DEFER_DQ
    assert lib.avattn_bwd(*bad) == _lib.ERR_ARGUMENT
    bad[28] = _lib.BWD_STAGE_DS | _lib.BWD_DEFER_DQ
    bad[27] = lib.avattn_bwd_staged_workspace_size(1, 2, 2, 4, 4, 128, 1)
    assert lib.avattn_bwd(*bad) == _lib.ERR_WORKSPACE
    bad[20] = None  # dq is not used by a deferred backward: still fails on the workspace, not the pointer
    assert lib.avattn_bwd(*bad) == _lib.ERR_WORKSPACE
    # avattn_bwd_dq_staged: flags, pointers, workspace
    dq_s = _lib.i64_array([1 << 17, 1 << 17, 128])
    full = lib.avattn_bwd_staged_workspace_size(1, 2, 2, 4, 4, 128, 2)
    assert lib.avattn_bwd_dq_staged(1, 2, 2, 4, 4, 128, 0.125, 16, dq_s, 256, full, 1, None) == _lib.ERR_ARGUMENT
    assert lib.avattn_bwd_dq_staged(1, 2, 2, 4, 4, 128, 0.125, None, dq_s, 256, full, 0, None) == _lib.ERR_NULL_POINTER
    assert lib.avattn_bwd_dq_staged(1, 2, 2, 4, 4, 128, 0.125, 16, dq_s, 256, full - 1, 0, None) == _lib.ERR_WORKSPACE
    assert lib.avattn_bwd_dq_staged(1, 2, 2, 4, 4, 128, 0.0, 16, dq_s, 256, full, 0, None) == _lib.ERR_ARGUMENT
    assert lib.avattn_bwd_dq_staged(1, 3, 2, 4, 4, 128, 0.125, 16, dq_s, 256, full, 0, None) == _lib.ERR_GQA
    assert lib.avattn_bwd_dq_staged(1, 2, 2, 0, 4, 128, 0.125, None, dq_s, None, 0, 0, None) == _lib.OK
    # fp32 dq accumulator: strides in floats, multiples of 4 (not 8)
    bad = list(base)
    bad[28] = _lib.BWD_DQ_ACCUMULATE_F32
    bad[21] = _lib.i64_array([1 << 16, 1 << 16, 132])
    assert lib.avattn_bwd(*bad) == _lib.ERR_WORKSPACE  # layout accepted, reaches the workspace check
    bad[21] = _lib.i64_array([1 << 16, 1 << 16, 130])
    assert lib.avattn_bwd(*bad) == _lib.ERR_LAYOUT
    bad = list(base)
    bad[16] = 80
    assert lib.avattn_bwd(*bad) == _lib.ERR_HEAD_DIM
    bad = list(base)
    bad[20] = None
    assert lib.avattn_bwd(*bad) == _lib.ERR_NULL_POINTER
    bad = list(base)
    bad[0] = 24
    bad[27] = 1 << 20
    assert lib.avattn_bwd(*bad) == _lib.ERR_LAYOUT


@cpu_only
def test_merge_and_rope_validation_paths(lib):
    assert lib.avattn_lse_merge(16, 16, 16, 16, 10, 96, 1, None) == _lib.ERR_HEAD_DIM
    assert lib.avattn_lse_merge(None, 16, 16, 16, 10, 128, 1, None) == _lib.ERR_NULL_POINTER
    assert lib.avattn_lse_merge(8, 16, 16, 16, 10, 128, 1, None) == _lib.ERR_LAYOUT
    assert lib.avattn_lse_merge(16, 16, 16, 16, 0, 128, 1, None) == _lib.OK
    s = _lib.i64_array([1 << 16, 1 << 14, 128])
    assert lib.avattn_rope_apply(16, s, 1, 1, 4, 100, 16, 16, 0, 0, 16, s, None) == _lib.ERR_HEAD_DIM
    assert lib.avattn_rope_apply(None, s, 1, 1, 4, 128, 16, 16, 0, 0, 16, s, None) == _lib.ERR_NULL_POINTER
    assert lib.avattn_rope_apply(16, s, 1, 1, 4, 128, 16, 16, 2, 0, 16, s, None) == _lib.ERR_LAYOUT
    f = (ctypes.c_float * 64)()
    ax = (ctypes.c_int32 * 64)(*([3] * 64))
    z = (ctypes.c_int32 * 3)()
    f3 = (ctypes.c_float * 3)()
    cast = lambda a: ctypes.cast(a, ctypes.c_void_p)  # noqa: E731
    assert lib.avattn_rope_tables(16, 3, 3, 1, 4, 64, cast(f), cast(ax), cast(z), cast(f3), cast(z), cast(f3),
                                  16, 16, None) == _lib.ERR_ARGUMENT
    assert lib.avattn_rope_tables(16, 3, 3, 1, 4, 2, cast(f), cast(ax), cast(z), cast(f3), cast(z), cast(f3),
                                  16, 16, None) == _lib.ERR_HEAD_DIM


def _ring_fwd(lib, **over):
    s = _lib.i64_array([1024 * 128, 1024 * 128, 128])
    a = dict(q=16, k=16, v=16, qs=s, ks=s, vs=s, B=1, Hq=2, Hkv=2, Lq=4, Lk=4, D=128, mask=None, msb=0,
             cq=16, sq=16, rqb=0, ck=16, sk=16, rkb=0, scale=0.125, acc=16, lacc=16, out=16, os=s,
             flags=_lib.RING_FIRST | _lib.RING_LAST, ws=256, wsb=1 << 20, stream=None)
    a.update(over)
    return lib.avattn_ring_fwd_step(a["q"], a["k"], a["v"], a["qs"], a["ks"], a["vs"], a["B"], a["Hq"], a["Hkv"],
                                    a["Lq"], a["Lk"], a["D"], a["mask"], a["msb"], a["cq"], a["sq"], a["rqb"],
                                    a["ck"], a["sk"], a["rkb"], a["scale"], a["acc"], a["lacc"], a["out"], a["os"],
                                    a["flags"], a["ws"], a["wsb"], a["stream"])


@cpu_only
def test_ring_step_validation_paths(lib):
    assert _ring_fwd(lib, ws=8) == _lib.ERR_WORKSPACE  # valid up to the workspace
    assert _ring_fwd(lib, flags=4) == _lib.ERR_ARGUMENT
    assert _ring_fwd(lib, Lk=0) == _lib.ERR_BAD_SHAPE  # a ring chunk holds keys
    assert _ring_fwd(lib, Lq=0) == _lib.OK
    assert _ring_fwd(lib, acc=None) == _lib.ERR_NULL_POINTER
    assert _ring_fwd(lib, acc=8) == _lib.ERR_LAYOUT
    assert _ring_fwd(lib, lacc=18) == _lib.ERR_LAYOUT
    assert _ring_fwd(lib, sq=None) == _lib.ERR_NULL_POINTER
    assert _ring_fwd(lib, ck=24) == _lib.ERR_LAYOUT
    assert _ring_fwd(lib, rkb=2) == _lib.ERR_LAYOUT
    assert _ring_fwd(lib, out=None) == _lib.ERR_NULL_POINTER  # the last step writes the output
    assert _ring_fwd(lib, out=None, os=None, flags=_lib.RING_FIRST, ws=8) == _lib.ERR_WORKSPACE  # not needed
    assert _ring_fwd(lib, cq=None, sq=None, ck=None, sk=None, ws=8) == _lib.ERR_WORKSPACE  # no rotation
    s = _lib.i64_array([1 << 17, 1 << 17, 128])
    fs = _lib.i64_array([1 << 17, 1 << 17, 132])  # fp32 accumulator strides: multiples of 4

    def bwd(flags=0, ws_bytes=8, dq_s=fs, cq=16):
        return lib.avattn_ring_bwd_step(16, 16, 16, 16, 16, 16, s, s, s, s, s, 1, 2, 2, 4, 4, 128, None, 0,
                                        cq, 16, 0, 16, 16, 0, 0.125, 16, dq_s, 16, s, 16, s, 16, ws_bytes, flags,
                                        None)

    assert bwd() == _lib.ERR_WORKSPACE
    assert bwd(flags=_lib.BWD_DEFER_DQ) == _lib.ERR_ARGUMENT  # dq always accumulates here
    assert bwd(flags=_lib.BWD_DQ_ACCUMULATE_F32) == _lib.ERR_ARGUMENT
    assert bwd(dq_s=_lib.i64_array([1 << 17, 1 << 17, 130])) == _lib.ERR_LAYOUT
    assert bwd(cq=None) == _lib.ERR_NULL_POINTER
    one = lib.avattn_bwd_staged_workspace_size(1, 2, 2, 4, 4, 128, 1)
    assert bwd(flags=_lib.BWD_STAGE_DS, ws_bytes=one - 1) == _lib.ERR_WORKSPACE
    f = lib.avattn_ring_dq_finish
    assert f(16, fs, 1, 2, 4, 96, 16, 16, 0, 16, s, None) == _lib.ERR_HEAD_DIM
    assert f(16, fs, -1, 2, 4, 128, 16, 16, 0, 16, s, None) == _lib.ERR_BAD_SHAPE
    assert f(None, fs, 1, 2, 4, 128, 16, 16, 0, 16, s, None) == _lib.ERR_NULL_POINTER
    assert f(16, fs, 1, 2, 4, 128, 16, None, 0, 16, s, None) == _lib.ERR_NULL_POINTER
    assert f(16, _lib.i64_array([1 << 17, 1 << 17, 130]), 1, 2, 4, 128, 16, 16, 0, 16, s, None) == _lib.ERR_LAYOUT
    assert f(16, fs, 1, 2, 4, 128, 16, 16, 0, 16, _lib.i64_array([1 << 17, 1 << 17, 132]), None) == _lib.ERR_LAYOUT
    assert f(16, fs, 1, 0, 4, 128, 16, 16, 0, 16, s, None) == _lib.OK


def _fwd_fp8(lib, **over):
    s = _lib.i64_array([1024 * 128, 1024 * 128, 128])
    args = dict(q=16, k=16, v=16, qs=s, ks=s, vs=s, B=1, Hq=2, Hkv=2, Lq=4, Lk=4, D=128, mask=None, msb=0,
                qsc=16, ksc=16, scale=0.125, out=16, os=s, lse=16, ws=256, wsb=1 << 20, stream=None)
    args.update(over)
    return lib.avattn_fwd_fp8(args["q"], args["k"], args["v"], args["qs"], args["ks"], args["vs"], args["B"],
                              args["Hq"], args["Hkv"], args["Lq"], args["Lk"], args["D"], args["mask"], args["msb"],
                              args["qsc"], args["ksc"], args["scale"], args["out"], args["os"], args["lse"],
                              args["ws"], args["wsb"], args["stream"])


@cpu_only
def test_fwd_fp8_validation_paths(lib):
    assert _fwd_fp8(lib, D=96) == _lib.ERR_HEAD_DIM
    assert _fwd_fp8(lib, Hq=3, Hkv=2) == _lib.ERR_GQA
    assert _fwd_fp8(lib, scale=-1.0) == _lib.ERR_ARGUMENT
    assert _fwd_fp8(lib, qsc=None) == _lib.ERR_NULL_POINTER
    assert _fwd_fp8(lib, ksc=None) == _lib.ERR_NULL_POINTER
    assert _fwd_fp8(lib, qsc=18) == _lib.ERR_LAYOUT
    assert _fwd_fp8(lib, q=8) == _lib.ERR_LAYOUT
    assert _fwd_fp8(lib, ws=None) == _lib.ERR_WORKSPACE
    assert _fwd_fp8(lib, wsb=1000) == _lib.ERR_WORKSPACE
    assert _fwd_fp8(lib, Lq=0) == _lib.OK


@cpu_only
def test_fp8_absmax_validation_paths(lib):
    s = _lib.i64_array([1 << 17, 1 << 17, 128])
    f = lib.avattn_fp8_absmax_scales
    assert f(16, s, 1, 2, 4, 96, 16, None) == _lib.ERR_HEAD_DIM
    assert f(16, s, -1, 2, 4, 128, 16, None) == _lib.ERR_BAD_SHAPE
    assert f(16, None, 1, 2, 4, 128, 16, None) == _lib.ERR_NULL_POINTER
    assert f(16, s, 1, 2, 4, 128, None, None) == _lib.ERR_NULL_POINTER
    assert f(None, s, 1, 2, 4, 128, 16, None) == _lib.ERR_NULL_POINTER
    assert f(8, s, 1, 2, 4, 128, 16, None) == _lib.ERR_LAYOUT
    assert f(16, s, 1, 2, 4, 128, 18, None) == _lib.ERR_LAYOUT
    assert f(16, s, 1, 1 << 17, 4, 128, 16, None) == _lib.ERR_TOO_LARGE
    assert f(16, s, 1, 0, 4, 128, 16, None) == _lib.OK


def _fwd_f32(lib, **over):
    s = _lib.i64_array([1024 * 128, 1024 * 128, 128])
    args = dict(q=16, k=16, v=16, qs=s, ks=s, vs=s, B=1, Hq=2, Hkv=2, Lq=4, Lk=4, D=128, mask=None, msb=0,
                scale=0.125, out=16, os=s, lse=16, stream=None)
    args.update(over)
    return lib.avattn_fwd_f32(args["q"], args["k"], args["v"], args["qs"], args["ks"], args["vs"], args["B"],
                              args["Hq"], args["Hkv"], args["Lq"], args["Lk"], args["D"], args["mask"], args["msb"],
                              args["scale"], args["out"], args["os"], args["lse"], args["stream"])


@cpu_only
def test_fwd_f32_validation_paths(lib):
    assert _fwd_f32(lib, D=96) == _lib.ERR_HEAD_DIM
    assert _fwd_f32(lib, Hq=3, Hkv=2) == _lib.ERR_GQA
    assert _fwd_f32(lib, Lq=-1) == _lib.ERR_BAD_SHAPE
    assert _fwd_f32(lib, qs=None) == _lib.ERR_NULL_POINTER
    assert _fwd_f32(lib, q=None) == _lib.ERR_NULL_POINTER
    assert _fwd_f32(lib, lse=None) == _lib.ERR_NULL_POINTER
    assert _fwd_f32(lib, q=8) == _lib.ERR_LAYOUT
    assert _fwd_f32(lib, os=_lib.i64_array([1024 * 128, 1024 * 128, 130])) == _lib.ERR_LAYOUT
    assert _fwd_f32(lib, scale=0.0) == _lib.ERR_ARGUMENT
    assert _fwd_f32(lib, scale=float("inf")) == _lib.ERR_ARGUMENT
    assert _fwd_f32(lib, k=None) == _lib.ERR_NULL_POINTER
    assert _fwd_f32(lib, v=24) == _lib.ERR_LAYOUT
    assert _fwd_f32(lib, mask=16, msb=2) == _lib.ERR_ARGUMENT
    # nothing to compute: success without a launch
    assert _fwd_f32(lib, Lq=0) == _lib.OK
    assert _fwd_f32(lib, B=0) == _lib.OK


def _bwd_f32(lib, **over):
    s = _lib.i64_array([1024 * 128, 1024 * 128, 128])
    args = dict(do=16, q=16, k=16, v=16, o=16, lse=16, B=1, Hq=2, Hkv=2, Lq=4, Lk=4, D=128, mask=None, msb=0,
                scale=0.125, dq=16, dk=16, dv=16, ws=256, wsb=1 << 20, stream=None)
    args.update(over)
    st = {k_: args.get(k_ + "s", s) for k_ in ("do", "q", "k", "v", "o", "dq", "dk", "dv")}
    return lib.avattn_bwd_f32(args["do"], args["q"], args["k"], args["v"], args["o"], args["lse"],
                              st["do"], st["q"], st["k"], st["v"], st["o"],
                              args["B"], args["Hq"], args["Hkv"], args["Lq"], args["Lk"], args["D"],
                              args["mask"], args["msb"], args["scale"],
                              args["dq"], st["dq"], args["dk"], st["dk"], args["dv"], st["dv"],
                              args["ws"], args["wsb"], args["stream"])


@cpu_only
def test_bwd_f32_validation_paths(lib):
    assert lib.avattn_bwd_f32_workspace_size(2, 40, 18900) == 2 * _round256(2 * 40 * 18900 * 4)
    assert lib.avattn_bwd_f32_workspace_size(0, 4, 10) == 0
    base = 2 * _round256(2 * 40 * 18900 * 4)
    per = 4 * 2 * 18912 * 18944  # group 2: rows to 32, keys to 128
    assert lib.avattn_bwd_f32_staged_workspace_size(2, 40, 20, 18900, 18900, 3) == (base + 4095) // 4096 * 4096 + 3 * per
    assert lib.avattn_bwd_f32_staged_workspace_size(2, 40, 20, 18900, 18900, 99) == (base + 4095) // 4096 * 4096 + 40 * per
    assert lib.avattn_bwd_f32_staged_workspace_size(2, 40, 20, 18900, 18900, 0) == base
    assert lib.avattn_bwd_f32_staged_workspace_size(0, 40, 20, 18900, 18900, 1) == 0
    assert _bwd_f32(lib, D=32) == _lib.ERR_HEAD_DIM
    assert _bwd_f32(lib, Hq=4, Hkv=3) == _lib.ERR_GQA
    assert _bwd_f32(lib, Lk=-2) == _lib.ERR_BAD_SHAPE
    assert _bwd_f32(lib, qs=None) == _lib.ERR_NULL_POINTER
    assert _bwd_f32(lib, scale=-1.0) == _lib.ERR_ARGUMENT
    assert _bwd_f32(lib, lse=None) == _lib.ERR_NULL_POINTER
    assert _bwd_f32(lib, dv=None) == _lib.ERR_NULL_POINTER
    assert _bwd_f32(lib, o=40) == _lib.ERR_LAYOUT
    assert _bwd_f32(lib, dks=_lib.i64_array([1024 * 128, 1024 * 128, 126])) == _lib.ERR_LAYOUT
    assert _bwd_f32(lib, mask=16, msb=1) == _lib.ERR_ARGUMENT
    assert _bwd_f32(lib, ws=None) == _lib.ERR_WORKSPACE
    assert _bwd_f32(lib, wsb=16) == _lib.ERR_WORKSPACE
    assert _bwd_f32(lib, ws=272) == _lib.ERR_LAYOUT  # the row statistics need 256-byte alignment
    assert _bwd_f32(lib, Lq=0, Lk=0) == _lib.OK


@cpu_only
def test_rope_f32_validation_paths(lib):
    s = _lib.i64_array([1024 * 128, 1024 * 128, 128])

    def call(**over):
        a = dict(x=16, xs=s, B=1, H=2, L=4, D=128, c=16, sn=16, tsb=0, inv=0, out=16, os=s)
        a.update(over)
        return lib.avattn_rope_apply_f32(a["x"], a["xs"], a["B"], a["H"], a["L"], a["D"], a["c"], a["sn"],
                                         a["tsb"], a["inv"], a["out"], a["os"], None)

    assert call(D=130) == _lib.ERR_HEAD_DIM
    assert call(D=6) == _lib.ERR_HEAD_DIM
    assert call(L=-1) == _lib.ERR_BAD_SHAPE
    assert call(c=None) == _lib.ERR_NULL_POINTER
    assert call(x=8) == _lib.ERR_LAYOUT
    assert call(os=_lib.i64_array([1024 * 128, 1024 * 128, 2])) == _lib.ERR_LAYOUT
    assert call(tsb=-4) == _lib.ERR_LAYOUT
    assert call(L=0) == _lib.OK


@cpu_only
def test_windowed_f32_validation_paths(lib):
    s = _lib.i64_array([1024 * 128, 1024 * 128, 128])

    def fwd(**over):
        a = dict(q=16, k=16, v=16, B=1, Hq=2, Hkv=2, Lq=4, Lk=4, D=128, mask=None, msb=0, lo=16, hi=32, wsb=0,
                 scale=0.125, out=16, lse=16)
        a.update(over)
        return lib.avattn_fwd_windowed_f32(a["q"], a["k"], a["v"], s, s, s, a["B"], a["Hq"], a["Hkv"], a["Lq"],
                                           a["Lk"], a["D"], a["mask"], a["msb"], a["lo"], a["hi"], a["wsb"],
                                           a["scale"], a["out"], s, a["lse"], None)

    def bwd(**over):
        a = dict(lo=16, hi=32, wsb=0, D=128, ws=256, wsb_ws=1 << 20)
        a.update(over)
        return lib.avattn_bwd_windowed_f32(16, 16, 16, 16, 16, 16, s, s, s, s, s, 1, 2, 2, 4, 4, a["D"], None, 0,
                                           a["lo"], a["hi"], a["wsb"], 0.125, 16, s, 16, s, 16, s, a["ws"],
                                           a["wsb_ws"], None)

    assert fwd(D=96) == _lib.ERR_HEAD_DIM
    assert fwd(lo=None) == _lib.ERR_NULL_POINTER  # one bound without the other
    assert fwd(hi=None) == _lib.ERR_NULL_POINTER
    assert fwd(lo=18) == _lib.ERR_LAYOUT  # int32 windows 4-byte aligned
    assert fwd(wsb=2) == _lib.ERR_ARGUMENT  # a batch stride shorter than len_q
    assert fwd(wsb=-4) == _lib.ERR_ARGUMENT
    assert fwd(q=8) == _lib.ERR_LAYOUT
    assert fwd(Lq=0) == _lib.OK
    assert bwd(D=96) == _lib.ERR_HEAD_DIM
    assert bwd(hi=None) == _lib.ERR_NULL_POINTER
    assert bwd(wsb=3) == _lib.ERR_ARGUMENT
    assert bwd(ws=None) == _lib.ERR_WORKSPACE


@cpu_only
def test_qk_norm_f32_validation_paths(lib):
    s = _lib.i64_array([1 << 20, 128, 1 << 12])

    def fwd(**o):
        a = dict(x=16, xs=s, B=1, H=2, L=4, D=128, w=16, eps=1e-6, cos=None, sin=None, tsb=0, out=16, os=s)
        a.update(o)
        return lib.avattn_qk_norm_rope_f32(a["x"], a["xs"], a["B"], a["H"], a["L"], a["D"], a["w"], a["eps"],
                                           a["cos"], a["sin"], a["tsb"], a["out"], a["os"], None)

    def bwd(ws=256, wsb=4096 * 128 * 4, dw=16, w=16, x=16):
        return lib.avattn_qk_norm_rope_bwd_f32(x, s, 16, s, 1, 2, 4, 128, w, 1e-6, None, None, 0, 16, s, dw, ws,
                                               wsb, None)

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
    assert fwd(os=_lib.i64_array([1 << 20, 128, 102])) == _lib.ERR_LAYOUT  # rows 16-byte aligned: 4 floats
    assert fwd(L=0) == _lib.OK
    assert bwd(dw=None) == _lib.ERR_NULL_POINTER
    assert bwd(ws=None) == _lib.ERR_WORKSPACE
    assert bwd(wsb=100) == _lib.ERR_WORKSPACE
    assert bwd(ws=8) == _lib.ERR_WORKSPACE  # workspace 16-byte aligned
    assert bwd(x=8) == _lib.ERR_LAYOUT
