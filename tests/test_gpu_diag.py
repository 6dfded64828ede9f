"""GPU check of the dQ-accumulation diagnostic (avattn_diag_dq_partials):
with atomics every element of a (head, query tile) ends up incremented by
the number of key blocks that visit the tile (block kb visits tiles
2*kb .. 2*kb + tiles_per_block - 1, mod the tile count); plain stores write
1.0 exactly on the visited tiles and leave the others alone."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    from avgen_amd import _lib

    return _lib


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("atomic", [0, 1])
def test_diag_dq_partials(lib, D, atomic):
    H, nkb, ntiles, tpb = 3, 5, 7, 3
    acc = torch.full((H, ntiles, 64 * D), -2.0, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    print(f"diag dq partials D={D} atomic={atomic}", flush=True)
    for _ in range(2):
        lib.check(lib.load().avattn_diag_dq_partials(acc.data_ptr(), H, nkb, ntiles, tpb, D, atomic, stream),
                  "avattn_diag_dq_partials")
    torch.cuda.synchronize()
    t = torch.arange(ntiles)
    kb = torch.arange(nkb)
    visits = (((t[None, :] - 2 * kb[:, None]) % ntiles) < tpb).sum(0).float()
    if atomic:
        want = -2.0 + 2 * visits
    else:
        want = torch.where(visits > 0, torch.tensor(1.0), torch.tensor(-2.0))
    assert torch.equal(acc.cpu(), want[None, :, None].expand(H, ntiles, 64 * D))


def test_diag_dq_partials_rejects_bad_arguments(lib):
    acc = torch.zeros(64 * 128, dtype=torch.float32, device="cuda")
    L = lib.load()
    assert L.avattn_diag_dq_partials(None, 1, 1, 1, 1, 128, 1, None) != 0
    assert L.avattn_diag_dq_partials(acc.data_ptr(), 1, 1, 1, 2, 128, 1, None) != 0  # more tiles than exist
    assert L.avattn_diag_dq_partials(acc.data_ptr(), 1, 1, 1, 1, 96, 1, None) != 0  # head_dim
