"""Dense legal-mask rows <-> id lists on an MI355X (junqi_amd.masks over
jq_mask_count / jq_mask_to_ids / jq_ids_to_mask), against numpy restatements
of junqi_rl/training/rollout_gpu.py:119-198."""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

D = 16641


@pytest.fixture(scope="module")
def masks():
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a machine without a visible GPU")
    from junqi_amd import masks as M
    return M


def _np_csr(mask: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
    ids = np.zeros((mask.shape[0], k), np.int32)
    counts = mask.sum(1).astype(np.int32)
    for r in range(mask.shape[0]):
        cols = np.flatnonzero(mask[r])
        ids[r, :len(cols)] = cols
    return ids, counts


def _random_masks(rng, n, k_max):
    m = np.zeros((n, D), bool)
    for r in range(n):
        kind = r % 5
        if kind == 0:
            continue                                   # empty row
        cnt = int(rng.integers(1, k_max + 1)) if kind != 4 else k_max
        m[r, rng.choice(D, cnt, replace=False)] = True
    m[1, [0, 1, 2, 15, 16, D - 16, D - 1]] = True          # row ends and word boundaries
    return m


def test_dense_mask_to_csr_matches_numpy(masks):
    rng = np.random.default_rng(0)
    n, k = 53, 300                                      # 16641-byte rows start at every alignment
    m = _random_masks(rng, n, k)
    want_ids, want_counts = _np_csr(m, k)
    dm = torch.from_numpy(m).cuda()
    ids = torch.full((n, k), -7, dtype=torch.int32, device="cuda")
    counts = torch.full((n,), -7, dtype=torch.int32, device="cuda")
    masks.dense_mask_to_csr(dm, ids, counts)
    assert np.array_equal(counts.cpu().numpy(), want_counts)
    assert np.array_equal(ids.cpu().numpy(), want_ids)
    # overflow raises before any output is written
    m[3, :k + 1] = True
    ids.fill_(-7)
    counts.fill_(-7)
    with pytest.raises(ValueError, match="overflow"):
        masks.dense_mask_to_csr(torch.from_numpy(m).cuda(), ids, counts)
    assert (ids == -7).all() and (counts == -7).all()


def test_csr_to_dense_selected_matches_numpy(masks):
    rng = np.random.default_rng(1)
    rows, k = 40, 64
    m = _random_masks(rng, rows, k)
    ids, counts = _np_csr(m, k)
    idx = np.array([5, 0, 39, 5, 17, 2, 2], np.int64)
    got = masks.csr_to_dense_selected(torch.from_numpy(ids).cuda(), torch.from_numpy(counts).cuda(),
                                      torch.from_numpy(idx).cuda(), D)
    assert got.dtype == torch.bool and got.shape == (len(idx), D)
    assert np.array_equal(got.cpu().numpy(), m[idx])


def test_round_trip_of_legal_masks(masks):
    """The legal masks of live games survive mask -> ids -> mask."""
    import junqi_amd
    b = junqi_amd.JunqiBatch(24, show_mode=2)
    b.reset(5)
    out = b.legal(mask_bool=True)
    lm = out["mask_bool"].bool()
    ids = torch.empty((24, 512), dtype=torch.int32, device="cuda")
    cnt = torch.empty(24, dtype=torch.int32, device="cuda")
    masks.dense_mask_to_csr(lm, ids, cnt)
    assert torch.equal(cnt.cpu(), lm.sum(1, dtype=torch.int32).cpu())
    back = masks.csr_to_dense_selected(ids, cnt, torch.arange(24, device="cuda"), D)
    assert torch.equal(back, lm)
    b.close()
