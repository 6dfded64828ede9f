"""The compact staged-dS layout of the windowed backward (CPU).

``ops.compact_ds_table`` lays out, per 64-row query tile, the 128-key blocks
whose dS the dK/dV kernel writes.  It must equal, block for block, the set of
blocks the kernel visits the tile from, restated here by brute force from the
kernel's own rule (attn_bwd.hip, dK/dV with windows: block kt, keys [k0, k1)
with k1 = min(k0 + 128, Lk), visits tile T iff clamp(lo[first row]) < k1 and
clamp(hi[last row]) > k0, with windows clamped into 0 <= lo <= hi <= Lk), and
it must contain every 64-key stage the dQ kernel multiplies for each 32-row
group (that group's window union).  Bases and the per-head unit count follow
as prefix sums.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from avgen_amd import ops


def _visited_blocks(lo, hi, T, Lq, Lk):
    f, l = 64 * T, min(64 * T + 63, Lq - 1)
    lof = min(max(int(lo[f]), 0), Lk)
    lol = min(max(int(lo[l]), 0), Lk)
    hil = min(max(int(hi[l]), lol), Lk)
    out = []
    for kt in range((Lk + 127) // 128):
        k0, k1 = 128 * kt, min(128 * kt + 128, Lk)
        if lof < k1 and hil > k0:
            out.append(kt)
    return out


def _group_stages(lo, hi, g, Lq, Lk):
    """The 64-key stages the dQ kernel multiplies for 32-row group g."""
    r0, r1 = 32 * g, min(32 * g + 32, Lq)
    if r1 <= r0:
        return range(0)
    l = min(max(int(lo[r0]), 0), Lk)
    lol = min(max(int(lo[r1 - 1]), 0), Lk)
    h = min(max(int(hi[r1 - 1]), lol), Lk)
    return range(l // 64, (h + 63) // 64) if h > l else range(0)


def _check(lo_rows, hi_rows, Lq, Lk):
    lo_t = torch.tensor(np.asarray(lo_rows), dtype=torch.int32)
    hi_t = torch.tensor(np.asarray(hi_rows), dtype=torch.int32)
    table, units = ops.compact_ds_table(lo_t, hi_t, Lq, Lk)
    lo2, hi2 = lo_t.reshape(-1, Lq).numpy(), hi_t.reshape(-1, Lq).numpy()
    tiles = (Lq + 63) // 64
    assert table.dtype == torch.int32 and tuple(table.shape) == (lo2.shape[0], tiles, 4)
    tab = table.numpy()
    need = 1
    for r in range(lo2.shape[0]):
        base = 0
        for T in range(tiles):
            kb_lo, nblk, gbase, pad = (int(x) for x in tab[r, T])
            vis = _visited_blocks(lo2[r], hi2[r], T, Lq, Lk)
            assert list(range(kb_lo, kb_lo + nblk)) == vis or (nblk == 0 and vis == []), (r, T, kb_lo, nblk, vis)
            assert gbase == base and pad == 0
            base += 2 * nblk
            for g in (2 * T, 2 * T + 1):
                for s in _group_stages(lo2[r], hi2[r], g, Lq, Lk):
                    assert kb_lo <= s // 2 < kb_lo + nblk, (r, T, g, s)
        need = max(need, base)
    assert units == need


def _monotone(rng, Lq, Lk, width):
    lo = np.sort(rng.integers(-5, Lk + 5, Lq))
    hi = np.maximum(lo + rng.integers(-3, width, Lq), lo)  # may be empty
    hi = np.maximum.accumulate(hi)
    return lo, hi


@pytest.mark.parametrize("seed", range(6))
def test_random_monotone_windows(seed):
    rng = np.random.default_rng(seed)
    Lq, Lk = int(rng.integers(1, 700)), int(rng.integers(1, 900))
    lo, hi = _monotone(rng, Lq, Lk, int(rng.integers(1, 400)))
    _check(lo, hi, Lq, Lk)


def test_per_batch_rows_and_edges():
    Lq, Lk = 333, 300  # neither a multiple of 64 / 128
    rows_lo, rows_hi = [], []
    # temporal-style windows
    t = np.repeat(np.arange(12), 30)[:Lq] / 8.0
    k = np.repeat(np.arange(10), 30)[:Lk] / 8.0
    rows_lo.append(np.searchsorted(k, t - 0.25, side="left"))
    rows_hi.append(np.searchsorted(k, t + 0.25, side="right"))
    # empty windows pinned at the end (lo = hi = Lk), at block boundaries, at 0
    lo = np.full(Lq, Lk)
    hi = np.full(Lq, Lk)
    lo[:100], hi[:100] = 128, 128
    lo[:50], hi[:50] = 0, 0
    rows_lo.append(lo)
    rows_hi.append(hi)
    # full windows
    rows_lo.append(np.zeros(Lq, dtype=np.int64))
    rows_hi.append(np.full(Lq, Lk))
    _check(np.stack(rows_lo), np.stack(rows_hi), Lq, Lk)


def test_packed_windows_layout_and_size():
    """Varlen windows (packed_windows): the compact units per head are the
    admitted blocks, far fewer than the dense layout's."""
    from avgen_amd.attention import packed_windows

    segs = [2880, 2160, 1440, 900]
    Lq = sum(segs) + 180
    cu = torch.tensor([0, *np.cumsum(segs).tolist()], dtype=torch.int32)
    lo, hi = packed_windows(cu, Lq)
    _check(lo.numpy(), hi.numpy(), Lq, Lq)
    _, units = ops.compact_ds_table(lo, hi, Lq, Lq)
    dense = ((Lq + 63) // 64 * 2) * ((Lq + 127) // 128)
    assert units < 0.4 * dense
    assert ops.ds_bytes_per_pair(1, Lq, Lq, units) == units * 8192
