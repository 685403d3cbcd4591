"""GPU tests of ogn_index_facts (sortedness, min, max of an int64 index in
one pass), which gates the sorted-index paths of scatter / segment_coo and
the COO -> CSR conversion.  Checked against numpy on sorted inputs with one
inversion placed at every position class (inside a 16-byte pair, across
pairs, at the first and last element), on 16-byte aligned and 8-byte
aligned views, and on sizes around the per-thread pair split."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _facts(t):
    from ops_gnn import _native

    return _native.index_probe(t)


def _want(a):
    return (bool((np.diff(a) < 0).any()), int(a.min()), int(a.max()))


@pytest.mark.parametrize("n", [1, 2, 3, 4, 5, 7, 8, 9, 63, 64, 65, 1000, 100_003])
@pytest.mark.parametrize("offset", [0, 1])
def test_index_facts_sorted_and_single_inversions(n, offset):
    rng = np.random.default_rng(n)
    base = np.sort(rng.integers(-50, 50, n + 1)).astype(np.int64)
    dev = torch.from_numpy(base).cuda()
    view = dev[offset: offset + n]  # offset 1: 8-byte aligned only
    assert _facts(view) == _want(base[offset: offset + n])
    positions = sorted({0, 1, 2, n // 2, n - 2, n - 1} & set(range(n - 1))) if n > 1 else []
    for j in positions:  # swap j, j+1 after making them distinct
        a = base.copy()[offset: offset + n]
        a[j], a[j + 1] = a[j + 1] + 1, a[j]
        full = base.copy()
        full[offset: offset + n] = a
        t = torch.from_numpy(full).cuda()[offset: offset + n]
        assert _facts(t) == _want(a), (n, offset, j)


def test_index_facts_extremes():
    a = np.array([np.iinfo(np.int64).min, -1, 0, np.iinfo(np.int64).max], dtype=np.int64)
    assert _facts(torch.from_numpy(a).cuda()) == (False, int(a[0]), int(a[-1]))
    assert _facts(torch.from_numpy(a[::-1].copy()).cuda()) == (True, int(a[0]), int(a[-1]))
