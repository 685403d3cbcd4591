"""GPU tests of ogn_sort_rows, the stable bounded-key sort behind COO -> CSR
and CSR -> CSC (the reference sorts with a stable argsort and indexes the
columns and values by it, python/ops_gnn/torch_sparse_spmm.py:273-342).
Sorted keys, the permutation and the permuted companion arrays must equal
torch.sort(keys, stable=True) and indexing by it exactly, including the
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
    got_k, got_p, _ = _native.sort_rows(keys.cuda(), max_key)
    assert torch.equal(got_k.cpu(), want_k)
    assert torch.equal(got_p.cpu(), want_p)


@pytest.mark.parametrize("dtypes", [(torch.int64,), (torch.int64, torch.float32), (torch.int32, torch.float64),
                                    (torch.float16,), (torch.int64, torch.float32, torch.bfloat16)])
@pytest.mark.parametrize("n", [1, 5, 4097, 300_001])
def test_sort_rows_companions(dtypes, n):
    # 4- / 8-byte 1-D companions are permuted in the sort's last pass (at
    # most two), the rest by indexing; all must equal c[perm] bit for bit
    from ops_gnn import _native

    rng = np.random.default_rng(n)
    keys = torch.from_numpy(rng.integers(0, 999, n).astype(np.int64))
    comps = [torch.from_numpy(rng.standard_normal(n) * 1e6).to(dt) for dt in dtypes]
    comps[0] = comps[0] if dtypes[0].is_floating_point else torch.from_numpy(rng.integers(-2**31, 2**31 - 1, n)).to(dtypes[0])
    perm = torch.sort(keys, stable=True)[1]
    _, got_p, outs = _native.sort_rows(keys.cuda(), 998, tuple(c.cuda() for c in comps))
    assert torch.equal(got_p.cpu(), perm)
    for c, o in zip(comps, outs):
        assert o.dtype == c.dtype and torch.equal(o.cpu(), c[perm])


def test_sort_rows_c_abi_errors_and_small_workspace():
    from ops_gnn import _lib

    lib = _lib.lib
    n, max_key = 5000, 999
    keys = torch.randint(0, max_key + 1, (n,), device="cuda")
    nbytes = lib.ogn_sort_rows_workspace_size(n, max_key, 0, 0)
    assert nbytes > 0
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    perm = torch.empty(n, dtype=torch.int64, device="cuda")
    rc = lib.ogn_sort_rows(_lib.dptr(keys), n, max_key, None, _lib.dptr(perm), None, None, 0, None, None, 0,
                           _lib.dptr(ws), nbytes, _lib.stream_of(keys))
    _lib.check(rc, "sort_rows")
    assert torch.equal(perm.cpu(), torch.sort(keys.cpu(), stable=True)[1])
    rc = lib.ogn_sort_rows(_lib.dptr(keys), n, max_key, None, _lib.dptr(perm), None, None, 0, None, None, 0,
                           _lib.dptr(ws), nbytes - 1, _lib.stream_of(keys))
    assert rc == 1  # OGN_EINVAL: workspace too small


def test_coo_and_transposed_layouts_use_the_sort(ogn):
    # unsorted COO -> CSR through the torch_sparse frontend: same permutation as a stable argsort
    from ops_gnn import torch_sparse_spmm as tss

    rng = np.random.default_rng(3)
    m, e = 500, 20_000
    index = torch.from_numpy(np.stack([rng.integers(0, m, e), rng.integers(0, m, e)]).astype(np.int64)).cuda()
    value = torch.from_numpy(rng.standard_normal(e).astype(np.float32)).cuda()
    ptr, col, val = tss.coo_to_csr(index, value, m)
    want_perm = torch.sort(index[0].cpu(), stable=True)[1]
    assert torch.equal(col.cpu(), index[1].cpu()[want_perm])
    assert torch.equal(val.cpu(), value.cpu()[want_perm])
    counts = torch.bincount(index[0].cpu(), minlength=m)
    assert torch.equal(ptr.cpu(), torch.cat([torch.zeros(1, dtype=torch.int64), counts.cumsum(0)]))
    ptr2, col2, perm2, _ = tss._coo_layout_uncached(index, m)
    assert torch.equal(perm2.cpu(), want_perm) and torch.equal(col2, col) and torch.equal(ptr2, ptr)
