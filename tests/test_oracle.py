"""Pin the CPU oracle (oracle/oracle.c) before trusting it as the checker.

Each oracle function is checked against (1) the known-answer tables the
reference's own tests hold, transcribed as literals with their file:line,
(2) an independent library routine (torch.sparse, torch.segment_reduce,
numpy.searchsorted / repeat), and (3) brute-force Python loops on tiny inputs
for the tie / NaN / empty-row rules.  These run on the CPU only.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as orc

INF, NAN = float("inf"), float("nan")


# ----------------------------------------------------------------- SpMM
def _brute_spmm(ptr, col, val, mat, reduce):
    """Literal per-edge loop of the torch_sparse golden rules."""
    m, k = len(ptr) - 1, mat.shape[-1]
    nnz = ptr[-1]
    out = np.zeros((m, k))
    arg = np.full((m, k), nnz, dtype=np.int64)
    for r in range(m):
        for j in range(k):
            terms = [(e, float(mat[col[e], j]) * (1.0 if val is None else float(val[e])))
                     for e in range(ptr[r], ptr[r + 1])]
            if reduce in ("sum", "mean"):
                s = sum(t for _, t in terms)
                out[r, j] = s / len(terms) if (reduce == "mean" and terms) else s
            else:
                best = None
                for e, t in terms:
                    if t != t:
                        continue
                    if best is None or (t < best[1] if reduce == "min" else t > best[1]):
                        best = (e, t)
                if best is not None:
                    out[r, j], arg[r, j] = best[1], best[0]
    return out, arg


@pytest.mark.parametrize("reduce", ["min", "max"])
def test_spmm_extrema_policy_kat(reduce):
    # reference test/torch_sparse_spmm/arch35/test_torch_sparse_spmm.py:518-536
    p = np.array([0, 2, 2, 3])
    c = np.array([0, 1, 2])
    b = np.array([[2.0, NAN, INF], [2.0, 3.0, -INF], [NAN, NAN, NAN]], dtype=np.float32)
    out, arg = orc.spmm_csr(p, c, None, b, reduce)
    expected = np.array([[2.0, 3.0, -INF if reduce == "min" else INF], [0, 0, 0], [0, 0, 0]])
    np.testing.assert_array_equal(out, expected)
    np.testing.assert_array_equal(arg, [[0, 1, 1 if reduce == "min" else 0], [3, 3, 3], [3, 3, 3]])


@pytest.mark.parametrize("reduce", ["min", "max"])
@pytest.mark.parametrize("features", [64, 128, 256, 512])
def test_spmm_first_tie_kat(reduce, features):
    # reference test/torch_sparse_spmm/arch35/test_torch_sparse_spmm.py:719-744
    ptr = np.array([0, 0, 9, 10])
    col = np.array([0] * 8 + [1, 2])
    values = np.ones(10, dtype=np.float32)
    mat = np.full((3, features), 2.0, dtype=np.float32)
    mat[0, 1] = NAN
    mat[1, 1] = 3.0
    mat[0, 2] = INF
    mat[1, 2] = -INF
    mat[2] = NAN
    out, arg = orc.spmm_csr(ptr, col, values, mat, reduce)
    expected = np.zeros((3, features))
    expected[1] = 2.0
    expected[1, 1] = 3.0
    expected[1, 2] = -INF if reduce == "min" else INF
    expected_arg = np.full((3, features), 10)
    expected_arg[1] = 0
    expected_arg[1, 1] = 8
    expected_arg[1, 2] = 8 if reduce == "min" else 0
    np.testing.assert_array_equal(out, expected)
    np.testing.assert_array_equal(arg, expected_arg)


def _random_csr(rng, m, n, avg, dup=True):
    deg = rng.poisson(avg, size=m)
    deg[rng.random(m) < 0.2] = 0
    col = np.concatenate([np.sort(rng.integers(0, n, d)) for d in deg]) if deg.sum() else \
        np.zeros(0, np.int64)
    ptr = np.concatenate([[0], np.cumsum(deg)]).astype(np.int64)
    return ptr, col.astype(np.int64)


@pytest.mark.parametrize("weighted", [False, True])
def test_spmm_sum_matches_torch_sparse(weighted):
    rng = np.random.default_rng(0)
    ptr, col = _random_csr(rng, 300, 200, 6)
    val = rng.standard_normal(col.size).astype(np.float32) if weighted else None
    mat = rng.standard_normal((200, 33)).astype(np.float32)
    out, arg = orc.spmm_csr(ptr, col, val, mat, "sum")
    assert arg is None
    a = torch.sparse_csr_tensor(torch.from_numpy(ptr), torch.from_numpy(col),
                                torch.from_numpy(val).double() if weighted else torch.ones(col.size, dtype=torch.float64),
                                size=(300, 200))
    ref = (a @ torch.from_numpy(mat).double()).numpy()
    np.testing.assert_allclose(out, ref, rtol=1e-12, atol=1e-12)
    mean, _ = orc.spmm_csr(ptr, col, val, mat, "mean")
    deg = np.diff(ptr)[:, None]
    np.testing.assert_allclose(mean, np.where(deg > 0, ref / np.maximum(deg, 1), 0.0), rtol=1e-12, atol=1e-12)


def test_spmm_batched_feature_weights_closed_form():
    rng = np.random.default_rng(1)
    ptr, col = _random_csr(rng, 40, 30, 4)
    val = rng.standard_normal((col.size, 7)).astype(np.float32)
    mat = rng.standard_normal((2, 3, 30, 7)).astype(np.float32)
    out, _ = orc.spmm_csr(ptr, col, val, mat, "sum")
    rows = np.repeat(np.arange(40), np.diff(ptr))
    ref = np.zeros((2, 3, 40, 7))
    np.add.at(ref, (slice(None), slice(None), rows), mat[:, :, col].astype(np.float64) * val)
    np.testing.assert_allclose(out, ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("reduce", ["sum", "mean", "min", "max"])
def test_spmm_matches_brute_force_with_ties_and_nans(reduce):
    rng = np.random.default_rng(2)
    ptr, col = _random_csr(rng, 25, 9, 5)
    mat = rng.integers(-2, 3, size=(9, 5)).astype(np.float32)  # many ties
    mat[rng.random(mat.shape) < 0.1] = NAN
    mat[0, 0], mat[1, 1] = INF, -INF
    val = rng.integers(-1, 2, size=col.size).astype(np.float32)
    out, arg = orc.spmm_csr(ptr, col, val, mat, reduce)
    ref, ref_arg = _brute_spmm(ptr, col, val, mat, reduce)
    np.testing.assert_allclose(out, ref, equal_nan=True)
    if reduce in ("min", "max"):
        np.testing.assert_array_equal(arg, ref_arg)


# ----------------------------------------------------------------- ind2ptr / ptr2ind
# Input tables: reference test/sparse/arch35/test_sparse.py:261-282 and :299-315.
IND2PTR_CASES = [
    ([], 0), ([], 1), ([0], 1), ([0], 8), ([7], 8), ([0, 0], 3), ([1, 1, 1], 3), ([0, 1], 2),
    ([0, 1, 2], 3), ([0, 0, 1, 1], 2), ([2, 2, 4, 5, 5, 6], 8), ([0, 0, 1, 3, 3, 3, 7], 8),
    ([0] * 16, 4), ([3] * 16, 4), (list(range(64)), 64), ([0, 2, 4, 6, 8, 10], 12),
    ([1, 3, 5, 7, 9, 11], 12), ([0] * 100 + [50] * 100 + [99] * 100, 100),
    (list(range(0, 256, 2)), 256), ([0] + [255] * 31, 256),
]
PTR2IND_CASES = [
    ([0], 0), ([0, 0], 0), ([0, 1], 1), ([0, 0, 0, 0], 0), ([0, 5], 5), ([0, 0, 0, 5, 5], 5),
    ([0, 0, 0, 2, 2, 3, 5, 6, 6], 6), ([0, 1, 2, 3, 4, 5], 5), ([0, 2, 4, 6, 8], 8),
    ([0, 0, 2, 2, 3, 3], 3), ([0, 10, 10, 20, 30], 30), ([0] + list(range(1, 65)), 64),
    ([0] + [16] * 4 + [64], 64), ([0, 0, 100, 100, 100], 100), ([0, 50, 50, 50, 100], 100),
]


@pytest.mark.parametrize("ind,rows", IND2PTR_CASES)
def test_ind2ptr_closed_form(ind, rows):
    got = orc.ind2ptr(np.array(ind, dtype=np.int64), rows)
    ref = np.searchsorted(np.array(ind, dtype=np.int64), np.arange(rows + 1), side="left")
    np.testing.assert_array_equal(got, ref)


def test_ind2ptr_docstring_kat():
    # reference python/ops_gnn/ind2ptr.py:51-55
    np.testing.assert_array_equal(orc.ind2ptr(np.array([2, 2, 4, 5, 5, 6]), 8), [0, 0, 0, 2, 2, 3, 5, 6, 6])


@pytest.mark.parametrize("ptr,edges", PTR2IND_CASES)
def test_ptr2ind_closed_form(ptr, edges):
    p = np.array(ptr, dtype=np.int64)
    got = orc.ptr2ind(p, edges)
    np.testing.assert_array_equal(got, np.repeat(np.arange(len(ptr) - 1), np.diff(p)))


def test_ptr2ind_docstring_kat():
    # reference python/ops_gnn/ptr2ind.py:51-55
    np.testing.assert_array_equal(orc.ptr2ind(np.array([0, 0, 0, 2, 2, 3, 5, 6, 6]), 6), [2, 2, 4, 5, 5, 6])


def test_convert_round_trip_random():
    rng = np.random.default_rng(3)
    ind = np.sort(rng.integers(0, 500, 5000))
    ptr = orc.ind2ptr(ind, 500)
    np.testing.assert_array_equal(orc.ptr2ind(ptr, ind.size), ind)


# ----------------------------------------------------------------- segment_csr
def test_segment_arg_first_occurrence_kat():
    # reference test/segment_csr/arch35/test_segment_csr.py:435-445
    src = np.array([[5.0, 1.0, 1.0, 5.0, 2.0], [3.0, 3.0, 3.0, 3.0, 3.0]], dtype=np.float32)
    indptr = np.array([0, 5])
    out, arg = orc.segment_csr(src, indptr, "min")
    np.testing.assert_array_equal(arg, [[1, 0, 0, 1, 0]])
    np.testing.assert_array_equal(out, [[3.0, 1.0, 1.0, 3.0, 2.0]])
    out, arg = orc.segment_csr(src, indptr, "max")
    np.testing.assert_array_equal(arg, [[0, 1, 1, 0, 1]])
    np.testing.assert_array_equal(out, [[5.0, 3.0, 3.0, 5.0, 3.0]])


def test_segment_readme_example():
    # reference docs/en/api_reference.md:290-296 (values computed by hand)
    src = np.array([[1.0, 4.0], [2.0, 3.0], [5.0, 6.0]], dtype=np.float32)
    indptr = np.array([0, 2, 3])
    out, _ = orc.segment_csr(src, indptr, "sum")
    np.testing.assert_array_equal(out, [[3.0, 7.0], [5.0, 6.0]])
    out, arg = orc.segment_csr(src, indptr, "max")
    np.testing.assert_array_equal(out, [[2.0, 4.0], [5.0, 6.0]])
    np.testing.assert_array_equal(arg, [[1, 0], [2, 2]])


@pytest.mark.parametrize("reduce", ["sum", "mean", "max", "min"])
def test_segment_matches_torch_segment_reduce(reduce):
    rng = np.random.default_rng(4)
    lengths = rng.poisson(5, size=50)
    lengths[::7] = 0
    src = rng.standard_normal((int(lengths.sum()), 6)).astype(np.float32)
    indptr = np.concatenate([[0], np.cumsum(lengths)])
    out, arg = orc.segment_csr(src, indptr, reduce)
    red = {"sum": "sum", "mean": "mean", "max": "max", "min": "min"}[reduce]
    ref = torch.segment_reduce(torch.from_numpy(src).double(), red, lengths=torch.from_numpy(lengths),
                               axis=0, unsafe=True).numpy()
    ref[lengths == 0] = 0.0  # reference empty-segment contract: value 0
    np.testing.assert_allclose(out, ref, rtol=1e-12, atol=1e-12)
    if arg is not None:
        # arg points at an element equal to the value, and it is the first such one
        for s in range(50):
            for j in range(6):
                a, z = indptr[s], indptr[s + 1]
                if a == z:
                    assert arg[s, j] == src.shape[0]
                else:
                    assert src[arg[s, j], j] == out[s, j]
                    assert arg[s, j] == a + int(np.argmax(src[a:z, j] == out[s, j]))


def test_segment_broadcast_batched_pointer():
    rng = np.random.default_rng(5)
    src = rng.standard_normal((3, 10, 4)).astype(np.float32)
    indptr = np.array([[0, 3, 3, 10]])
    out, _ = orc.segment_csr(src, indptr, "sum")
    s64 = src.astype(np.float64)
    ref = np.stack([s64[:, 0:3].sum(1), np.zeros((3, 4)), s64[:, 3:10].sum(1)], axis=1)
    np.testing.assert_allclose(out, ref, rtol=1e-6)
