"""GPU parity of ind2ptr / ptr2ind (bit-exact) against the oracle, on the
reference's own case tables (test/sparse/arch35/test_sparse.py:261-332) and
random / power-law inputs, plus the reference's error contract."""

import numpy as np
import pytest
import torch

from test_oracle import IND2PTR_CASES, PTR2IND_CASES

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("ind,rows", IND2PTR_CASES)
def test_ind2ptr_table(ogn, oracle, ind, rows):
    out = ogn.ind2ptr(torch.tensor(ind, dtype=torch.long, device="cuda"), rows)
    assert out.dtype == torch.int64 and out.shape == (rows + 1,)
    np.testing.assert_array_equal(out.cpu().numpy(), oracle.ind2ptr(np.array(ind, dtype=np.int64), rows))


@pytest.mark.parametrize("ptr,edges", PTR2IND_CASES)
def test_ptr2ind_table(ogn, oracle, ptr, edges):
    out = ogn.ptr2ind(torch.tensor(ptr, dtype=torch.long, device="cuda"), edges)
    assert out.dtype == torch.int64 and out.shape == (edges,)
    np.testing.assert_array_equal(out.cpu().numpy(), oracle.ptr2ind(np.array(ptr, dtype=np.int64), edges))


@pytest.mark.parametrize("edges,rows,seed", [(1, 7, 0), (1025, 64, 1), (4096, 1025, 42), (100_000, 257, 3),
                                             (257, 100_000, 4)])
def test_random_round_trip(ogn, oracle, edges, rows, seed):
    g = torch.Generator().manual_seed(seed)
    ind = torch.sort(torch.randint(0, rows, (edges,), generator=g)).values
    ptr = ogn.ind2ptr(ind.cuda(), rows)
    np.testing.assert_array_equal(ptr.cpu().numpy(), oracle.ind2ptr(ind.numpy(), rows))
    back = ogn.ptr2ind(ptr, edges)
    assert torch.equal(back.cpu(), ind)


def test_noncontiguous_inputs(ogn):
    ind = torch.tensor([0, 9, 0, 9, 2, 9, 2, 9, 3, 9], device="cuda")[::2]
    assert torch.equal(ogn.ind2ptr(ind, 4).cpu(), torch.tensor([0, 2, 2, 4, 5]))
    ptr = torch.tensor([0, 9, 2, 9, 2, 9, 5, 9], device="cuda")[::2]
    assert torch.equal(ogn.ptr2ind(ptr, 5).cpu(), torch.tensor([0, 0, 2, 2, 2]))


def test_powerlaw_round_trip_large(ogn):
    from ops_gnn.synthetic import cfg3_powerlaw_degrees

    deg, _ = cfg3_powerlaw_degrees(seed=5, m=200_000, nnz=5_000_000, cap=100_000)
    ptr = torch.from_numpy(np.concatenate([[0], np.cumsum(deg)])).cuda()
    ind = ogn.ptr2ind(ptr, int(deg.sum()))
    expected = torch.repeat_interleave(torch.arange(200_000, device="cuda"), torch.from_numpy(deg).cuda())
    assert torch.equal(ind, expected)
    assert torch.equal(ogn.ind2ptr(ind, 200_000), ptr)


@pytest.mark.parametrize("ptr,edges,msg", [
    ([1, 2], 2, "start with 0"), ([0, 2], 3, "end with num_edges"), ([0, 2, 1, 2], 2, "non-decreasing"),
    ([0, -1, 2], 2, "out-of-range"),
])
def test_ptr2ind_rejects_bad_pointer(ogn, ptr, edges, msg):
    with pytest.raises(RuntimeError, match=msg):
        ogn.ptr2ind(torch.tensor(ptr, device="cuda"), edges)


def test_argument_errors(ogn):
    with pytest.raises(RuntimeError, match="1-D"):
        ogn.ind2ptr(torch.zeros(2, 2, dtype=torch.long, device="cuda"), 3)
    with pytest.raises(RuntimeError, match="int64"):
        ogn.ind2ptr(torch.zeros(2, dtype=torch.int32, device="cuda"), 3)
    with pytest.raises(RuntimeError, match="non-negative"):
        ogn.ind2ptr(torch.zeros(2, dtype=torch.long, device="cuda"), -1)
    with pytest.raises(RuntimeError, match="at least one"):
        ogn.ptr2ind(torch.zeros(0, dtype=torch.long, device="cuda"), 0)


def test_ptr2ind_tiles_with_empty_row_runs(ogn, oracle):
    # tiles of 2048 edges stage their pointer entries in LDS (up to 2176);
    # long runs of empty rows inside a tile take the global search instead
    rng = np.random.default_rng(8)
    deg = rng.integers(0, 5, 30_000)
    deg[5000:15000] = 0          # 10 000 empty rows inside one tile
    deg[20000] = 7000            # a row spanning several tiles
    ptr = np.concatenate([[0], np.cumsum(deg)])
    edges = int(ptr[-1])
    out = ogn.ptr2ind(torch.from_numpy(ptr).cuda(), edges)
    np.testing.assert_array_equal(out.cpu().numpy(), oracle.ptr2ind(ptr, edges))
