"""GPU tests of ogn_sort_rows, the stable bounded-key sort behind COO -> CSR
and CSR -> CSC (the reference sorts with a stable argsort,
python/ops_gnn/torch_sparse_spmm.py:273-342).  Sorted keys and the
permutation must equal torch.sort(keys, stable=True) exactly, including the
order of equal keys, for key ranges from one bit to 32 bits."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [1, 7, 1000, 1_000_003])
@pytest.mark.parametrize("max_key", [0, 1, 255, 256, 65_535, 1_000_000, 2**32 - 1])
def test_sort_rows_matches_stable_sort(n, max_key):
    from ops_gnn import _native

    rng = np.random.default_rng(n + max_key % 97)
    # few distinct values as well as the full range: long runs of equal keys
    hi = min(max_key, 50) if n > 100 and max_key > 1_000 else max_key
    keys = torch.from_numpy(rng.integers(0, hi, n, endpoint=True).astype(np.int64))
    if n > 2:
        keys[0], keys[-1] = max_key, 0  # both ends of the range
    want_k, want_p = torch.sort(keys, stable=True)
    got_k, got_p = _native.sort_rows(keys.cuda(), max_key)
    assert torch.equal(got_k.cpu(), want_k)
    assert torch.equal(got_p.cpu(), want_p)


def test_sort_rows_c_abi_without_sorted_keys_and_small_workspace():
    from ops_gnn import _lib

    lib = _lib.lib
    n, max_key = 5000, 999
    keys = torch.randint(0, max_key + 1, (n,), device="cuda")
    nbytes = lib.ogn_sort_rows_workspace_size(n, max_key)
    assert nbytes > 0
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    perm = torch.empty(n, dtype=torch.int64, device="cuda")
    rc = lib.ogn_sort_rows(_lib.dptr(keys), n, max_key, None, _lib.dptr(perm), _lib.dptr(ws), nbytes,
                           _lib.stream_of(keys))
    _lib.check(rc, "sort_rows")
    assert torch.equal(perm.cpu(), torch.sort(keys.cpu(), stable=True)[1])
    rc = lib.ogn_sort_rows(_lib.dptr(keys), n, max_key, None, _lib.dptr(perm), _lib.dptr(ws), nbytes - 1,
                           _lib.stream_of(keys))
    assert rc == 1  # OGN_EINVAL


def test_coo_and_transposed_layouts_use_the_sort(ogn):
    # unsorted COO -> CSR through the torch_sparse frontend: same permutation as a stable argsort
    from ops_gnn import torch_sparse_spmm as tss

    rng = np.random.default_rng(3)
    m, e = 500, 20_000
    index = torch.from_numpy(np.stack([rng.integers(0, m, e), rng.integers(0, m, e)]).astype(np.int64)).cuda()
    ptr, col, perm = tss._coo_layout_uncached(index, m)
    want_perm = torch.sort(index[0].cpu(), stable=True)[1]
    assert torch.equal(perm.cpu(), want_perm)
    assert torch.equal(col.cpu(), index[1].cpu()[want_perm])
    counts = torch.bincount(index[0].cpu(), minlength=m)
    assert torch.equal(ptr.cpu(), torch.cat([torch.zeros(1, dtype=torch.int64), counts.cumsum(0)]))
