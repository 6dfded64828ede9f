"""Query-dependent masks as per-row key windows: the oracle's restatements
of the reference masks pinned against the reference's own expectations and
hand-worked cases, and the window builders (host logic, run here on CPU
tensors) checked against those masks element by element."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from avgen_amd import attention as A
from oracle import reference as R


def _window_mask(lo, hi, Lk):
    j = np.arange(Lk)
    return (j >= np.asarray(lo)[..., None]) & (j < np.asarray(hi)[..., None])


def test_packed_mask_matches_the_reference_test():
    """tests/test_data.py:640-667 of the reference: segments of 3, 4 and 2
    tokens in a capacity of 12."""
    ids = R.packed_segment_ids([3, 4, 2], 12)
    assert ids.tolist() == [0] * 3 + [1] * 4 + [2] * 2 + [R.PADDING_SEGMENT] * 3
    assert R.packed_cu_seqlens([3, 4, 2]).tolist() == [0, 3, 7, 9]
    mask = R.packed_attention_mask([3, 4, 2], 12)
    assert mask.shape == (12, 12)
    for row in range(12):
        for col in range(12):
            expected = ids[row] != R.PADDING_SEGMENT and ids[row] == ids[col]
            assert bool(mask[row, col]) is bool(expected), (row, col)


@pytest.mark.parametrize("lengths,capacity", [([3, 4, 2], 12), ([5], 5), ([1, 1, 1], 4), ([64, 200, 7, 129], 512)])
def test_packed_windows_give_the_block_diagonal_mask(lengths, capacity):
    cu = torch.tensor(R.packed_cu_seqlens(lengths))
    lo, hi = A.packed_windows(cu, capacity)
    assert lo.dtype is torch.int32 and hi.dtype is torch.int32
    assert (lo[1:] >= lo[:-1]).all() and (hi[1:] >= hi[:-1]).all()
    np.testing.assert_array_equal(_window_mask(lo.numpy(), hi.numpy(), capacity),
                                  R.packed_attention_mask(lengths, capacity))


def test_temporal_mask_hand_worked():
    """|tq - tk| <= w with exactly representable times; the last query has no
    key within the window and falls back to every key
    (src/avgen/models/blocks.py:97-104)."""
    tq = np.array([[0.0, 1.0, 2.0, 5.0]], np.float32)
    tk = np.array([[0.0, 0.5, 1.5, 2.0, 2.6]], np.float32)
    T, F = True, False
    m = R.temporal_neighbour_mask(tq, tk, 0.5)
    assert m.shape == (1, 1, 4, 5)
    assert m[0, 0].tolist() == [[T, T, F, F, F], [F, T, T, F, F], [F, F, T, T, F], [T, T, T, T, T]]
    km = np.array([[T, T, F, T, T]])
    m = R.temporal_neighbour_mask(tq, tk, 0.5, km)
    assert m[0, 0].tolist() == [[T, T, F, F, F], [F, T, F, F, F], [F, F, F, T, F], [T, T, T, T, T]]
    # a window holding only masked keys also falls back to every key
    km = np.array([[F, F, T, T, T]])
    m = R.temporal_neighbour_mask(tq, tk, 0.5, km)
    assert m[0, 0, 0].tolist() == [T, T, T, T, T]
    # window <= 0: no mask, or the key mask alone (:92-95)
    assert R.temporal_neighbour_mask(tq, tk, 0.0) is None
    assert R.temporal_neighbour_mask(tq, tk, -1.0, np.ones((1, 5), bool)) is None
    assert R.temporal_neighbour_mask(tq, tk, 0.0, km).shape == (1, 1, 1, 5)


def _stream_times(n, rate, start=0.0, per_step=1):
    steps = np.arange(n) // per_step
    return (start + steps / rate).astype(np.float32)


@pytest.mark.parametrize("window", [1 / 24, 0.25, 1.0, 1e-6, 30.0])
def test_temporal_windows_select_the_reference_keys(window):
    """Video times repeat per frame (many tokens share one time), audio runs at
    another rate: the windows hold exactly the keys the dense mask holds,
    boundary roundings included; rows with none are the fallback rows."""
    tq = np.stack([_stream_times(600, 24.0, per_step=40), _stream_times(600, 24.0, 0.3, per_step=16)])
    tk = np.stack([_stream_times(257, 43.07), _stream_times(257, 43.07, 0.01)])
    lo, hi = A.temporal_neighbour_windows(torch.from_numpy(tq), torch.from_numpy(tk), window_seconds=window)
    lo, hi = lo.numpy(), hi.numpy()
    assert (np.diff(lo, axis=1) >= 0).all() and (np.diff(hi, axis=1) >= 0).all()
    ref = R.temporal_neighbour_mask(tq, tk, window)[:, 0]
    wm = _window_mask(lo, hi, tk.shape[1])
    empty = hi == lo
    np.testing.assert_array_equal(wm[~empty], ref[~empty])
    assert ref[empty].all()  # fallback rows attend to everything


def test_temporal_windows_at_rounding_boundaries():
    """Differences that round onto the window edge: the bound search uses the
    reference's own float32 predicate, so it agrees where tq - w would not."""
    rng = np.random.default_rng(3)
    tk = np.sort(rng.uniform(0, 2, (1, 4000)).astype(np.float32), axis=1)
    w = 0.1
    tq = np.sort((tk[:, rng.integers(0, 4000, 700)] + np.float32(w)).astype(np.float32), axis=1)
    lo, hi = A.temporal_neighbour_windows(torch.from_numpy(tq), torch.from_numpy(tk), window_seconds=w)
    ref = R.temporal_neighbour_mask(tq, tk, w)[:, 0]
    wm = _window_mask(lo.numpy(), hi.numpy(), tk.shape[1])
    np.testing.assert_array_equal(wm, ref)


def test_temporal_windows_without_keys_are_empty():
    lo, hi = A.temporal_neighbour_windows(torch.zeros(2, 5), torch.zeros(2, 0), window_seconds=1.0)
    assert lo.shape == (2, 5) and (lo == 0).all() and (hi == 0).all()


def test_window_builders_validate():
    with pytest.raises(ValueError):
        A.temporal_neighbour_windows(torch.zeros(3), torch.zeros(1, 3), window_seconds=1.0)
    with pytest.raises(ValueError):
        A.packed_windows(torch.zeros((2, 2), dtype=torch.int32), 4)


@pytest.mark.parametrize("shuffle", [False, True])
def test_temporal_neighbourhood_reproduces_the_mask(shuffle):
    """Host side of the build-once neighbourhood (CPU tensors): windows over
    the time-sorted keys plus the fallback rows give back the reference mask
    row by row, in the caller's token order."""
    rng = np.random.default_rng(7)
    tq = np.stack([_stream_times(90, 24.0, per_step=6), _stream_times(90, 24.0, 0.4, per_step=6)])
    tk = np.stack([_stream_times(14, 20.0), _stream_times(14, 20.0, 0.1)])
    km = rng.random((2, 14)) < 0.7
    if shuffle:
        tq = tq[:, rng.permutation(90)]
        tk = tk[:, rng.permutation(14)]
    nb = A.temporal_neighbourhood(torch.from_numpy(tq), torch.from_numpy(tk), window_seconds=0.1,
                                  key_mask=torch.from_numpy(km))
    assert (nb.query_order is not None) == shuffle and (nb.key_order is not None) == shuffle
    ref = R.temporal_neighbour_mask(tq, tk, 0.1, km)[:, 0]
    qo = np.arange(90)[None].repeat(2, 0) if nb.query_order is None else nb.query_order.numpy()
    ko = np.arange(14)[None].repeat(2, 0) if nb.key_order is None else nb.key_order.numpy()
    kms = np.take_along_axis(km, ko, 1)
    win = _window_mask(nb.lo.numpy(), nb.hi.numpy(), 14) & kms[:, None, :]
    fb = np.zeros((2, 90), bool)
    for b, r in nb.fallback:
        fb[b, r.numpy()] = True
    assert fb.any(), "the case must have fallback rows"
    for b in range(2):
        for i in range(90):
            row = ref[b, qo[b, i]][ko[b]]  # reference row in sorted key order
            if fb[b, i]:
                assert row.all()
            else:
                np.testing.assert_array_equal(win[b, i], row)


def test_oracle_dense_mask_attention_matches_torch_sdpa():
    """attention_f64 / attention_bwd_f64 with a query-dependent boolean mask
    against torch's float64 SDPA and autograd with the same mask (rows with
    no admitted key excluded: SDPA returns NaN there, the oracle 0 / -inf)."""
    import torch.nn.functional as F

    rng = np.random.default_rng(11)
    B, H, Lq, Lk, D = 2, 2, 19, 23, 16
    q, k, v, do = (rng.standard_normal(s) for s in ((B, H, Lq, D), (B, H, Lk, D), (B, H, Lk, D), (B, H, Lq, D)))
    m = rng.random((B, 1, Lq, Lk)) < 0.4
    m[0, 0, 3] = False  # one row with no key
    km = rng.random((B, Lk)) < 0.9
    full = m & km[:, None, None, :]
    o, lse = R.attention_f64(q, k, v, km, attn_mask=m)
    tq, tk, tv = (torch.tensor(a, requires_grad=True) for a in (q, k, v))
    ref = F.scaled_dot_product_attention(tq, tk, tv, attn_mask=torch.from_numpy(full))
    ok = full.any(-1)[:, 0]  # (B, Lq)
    np.testing.assert_allclose(o.transpose(0, 2, 1, 3)[ok], ref.detach().numpy().transpose(0, 2, 1, 3)[ok],
                               rtol=1e-10, atol=1e-12)
    assert (o[0, :, 3] == 0).all() and np.isneginf(lse[0, :, 3]).all()
    g = np.where(ok[:, None, :, None], do, 0.0)
    ref.backward(torch.from_numpy(np.where(ok[:, None, :, None], do, 0.0)))
    dq, dk, dv = R.attention_bwd_f64(g, q, k, v, o, lse, km, attn_mask=m)
    for got, want in ((dq, tq.grad), (dk, tk.grad), (dv, tv.grad)):
        w = np.nan_to_num(want.numpy())
        np.testing.assert_allclose(got, w, rtol=1e-9, atol=1e-11)
