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


@pytest.mark.parametrize("reduce", ["sum", "mean", "min", "max"])
@pytest.mark.parametrize("out_dtype", ["int32", "float32"])
def test_spmm_int8_output_cast_brute_force(reduce, out_dtype):
    """int8 SpMM to int32 or float32 (reference golden.py:80-88,114-115):
    exact integer arithmetic with Python ints / Fractions, an int32 mean
    truncated toward zero, a float32 mean rounded from the exact quotient."""
    from fractions import Fraction

    rng = np.random.default_rng(7)
    ptr, col = _random_csr(rng, 40, 11, 6)
    mat = rng.integers(-128, 128, size=(11, 3)).astype(np.int8)
    val = rng.integers(-128, 128, size=col.size).astype(np.int8)
    out, arg = orc.spmm_csr(ptr, col, val, mat, reduce)
    got = orc.spmm_output_cast(out, out_dtype)
    assert got.dtype == np.dtype(out_dtype)
    for r in range(len(ptr) - 1):
        for j in range(3):
            terms = [int(mat[col[e], j]) * int(val[e]) for e in range(ptr[r], ptr[r + 1])]
            if not terms:
                exact = Fraction(0)
            elif reduce == "sum":
                exact = Fraction(sum(terms))
            elif reduce == "mean":
                exact = Fraction(sum(terms), len(terms))
            else:
                exact = Fraction(min(terms) if reduce == "min" else max(terms))
            want = int(exact) if out_dtype == "int32" else np.float32(float(exact))
            assert got[r, j] == want, (r, j, reduce, out_dtype)
    assert ("int8", "float32") in orc.SPMM_DTYPE_COMBOS and ("float32", "float16") not in orc.SPMM_DTYPE_COMBOS


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


# ----------------------------------------------------------------- segment_coo (Ascend 950 rules)
@pytest.mark.parametrize("mode", ["sum", "mean", "min", "max"])
def test_segment_coo_unequal_segments_kat(mode):
    # reference test/segment_coo/arch35/test_segment_coo.py:892-911
    x = np.array([[2, 5], [2, 1], [3, 6], [4, 6], [1, 2]], dtype=np.float32)
    idx = np.array([0, 0, 2, 2, 2])
    out, arg = orc.segment_coo(x, idx, 4, mode)
    ref = {"sum": [[4, 6], [0, 0], [8, 14], [0, 0]], "mean": [[2, 3], [0, 0], [8 / 3, 14 / 3], [0, 0]],
           "min": [[2, 1], [0, 0], [1, 2], [0, 0]], "max": [[2, 5], [0, 0], [4, 6], [0, 0]]}[mode]
    np.testing.assert_allclose(out, ref, rtol=1e-12)
    if arg is not None:
        expected = {"min": [[1, 1], [5, 5], [4, 4], [5, 5]], "max": [[1, 0], [5, 5], [3, 3], [5, 5]]}[mode]
        np.testing.assert_array_equal(arg, expected)


def test_segment_coo_matches_segment_reduce_and_later_tie_rule():
    rng = np.random.default_rng(11)
    idx = np.sort(rng.integers(0, 30, 400))
    src = rng.integers(-3, 4, size=(2, 400, 3)).astype(np.float32)  # ties everywhere
    lengths = np.bincount(idx, minlength=30)
    for mode in ("sum", "mean", "min", "max"):
        out, arg = orc.segment_coo(src, idx[None, :], 30, mode)
        ref = torch.segment_reduce(torch.from_numpy(src).double(), mode,
                                   lengths=torch.from_numpy(np.tile(lengths, (2, 1))), axis=1, unsafe=True).numpy()
        ref[:, lengths == 0] = 0.0
        np.testing.assert_allclose(out, ref, rtol=1e-12, atol=1e-12)
        if arg is not None:
            ptr = np.concatenate([[0], np.cumsum(lengths)])
            for b in range(2):
                for s in range(30):
                    for f in range(3):
                        a, z = ptr[s], ptr[s + 1]
                        if a == z:
                            assert arg[b, s, f] == 400
                        else:
                            hits = np.nonzero(src[b, a:z, f] == out[b, s, f])[0]
                            assert arg[b, s, f] == a + hits[-1]  # the LAST extremum


def test_segment_coo_out_seeds():
    x = np.array([[1.0], [5.0], [2.0]], dtype=np.float32)
    idx = np.array([0, 0, 2])
    seed = np.array([[3.0], [7.0], [-1.0]])
    out, arg = orc.segment_coo(x, idx, 3, "max", out=seed)
    np.testing.assert_array_equal(out, [[5.0], [7.0], [2.0]])
    np.testing.assert_array_equal(arg, [[1], [3], [2]])
    out, _ = orc.segment_coo(x, idx, 3, "mean", out=seed)
    np.testing.assert_allclose(out, [[(3 + 1 + 5) / 2], [7.0], [(-1 + 2) / 1]])
    out, _ = orc.segment_coo(x, idx, 3, "sum", out=seed)  # sum overwrites
    np.testing.assert_array_equal(out, [[6.0], [0.0], [2.0]])


# ----------------------------------------------------------------- scatter (torch_scatter)
def test_scatter_later_writer_tie_kat():
    # reference test/scatter/arch35/test_scatter.py:322-331
    src = np.array([4.0, 2.0, 2.0, 5.0, 5.0], dtype=np.float32)
    index = np.array([0, 0, 0, 1, 1])
    mn, amin = orc.scatter(src, index, 0, 2, "min")
    mx, amax = orc.scatter(src, index, 0, 2, "max")
    np.testing.assert_array_equal(mn, [2.0, 5.0])
    np.testing.assert_array_equal(mx, [4.0, 5.0])
    np.testing.assert_array_equal(amin, [2, 4])
    np.testing.assert_array_equal(amax, [0, 4])


def test_scatter_docs_example():
    # reference docs/en/api_reference.md:1032-1048
    src = np.array([1.0, 2.0, 3.0, 4.0], dtype=np.float32)
    index = np.array([0, 1, 0, 1])
    np.testing.assert_array_equal(orc.scatter(src, index, 0, 2, "sum")[0], [4.0, 6.0])
    v, a = orc.scatter(src, index, 0, 2, "max")
    np.testing.assert_array_equal(v, [3.0, 4.0])
    np.testing.assert_array_equal(a, [2, 3])


@pytest.mark.parametrize("reduce,torch_reduce", [("sum", "sum"), ("mean", "mean"), ("min", "amin"),
                                                 ("max", "amax"), ("mul", "prod")])
def test_scatter_matches_torch_scatter_reduce(reduce, torch_reduce):
    rng = np.random.default_rng(12)
    src = rng.standard_normal((3, 50, 4)).astype(np.float32)
    index = rng.integers(0, 12, size=(3, 50, 4))
    out, arg = orc.scatter(src, index, 1, 15, reduce)
    ref = torch.zeros(3, 15, 4, dtype=torch.float64).scatter_reduce(
        1, torch.from_numpy(index), torch.from_numpy(src).double(), torch_reduce, include_self=False)
    written = torch.zeros(3, 15, 4, dtype=torch.bool).scatter_(1, torch.from_numpy(index), True).numpy()
    ref = ref.numpy()
    if reduce == "mul":
        ref = np.where(written, ref, 1.0)
    else:
        ref = np.where(written, ref, 0.0)
    np.testing.assert_allclose(out, ref, rtol=1e-12, atol=1e-12)
    if arg is not None:
        for b in range(3):
            for t in range(15):
                for f in range(4):
                    hits = [l for l in range(50) if index[b, l, f] == t and src[b, l, f] == out[b, t, f]]
                    assert arg[b, t, f] == (hits[-1] if hits else 50)


def test_scatter_out_is_accumulated():
    src = np.array([1.0, 2.0, 3.0], dtype=np.float32)
    index = np.array([0, 0, 1])
    seed = np.array([10.0, 20.0, 30.0])
    np.testing.assert_array_equal(orc.scatter(src, index, 0, 3, "sum", out=seed)[0], [13.0, 23.0, 30.0])
    np.testing.assert_allclose(orc.scatter(src, index, 0, 3, "mean", out=seed)[0], [13 / 2, 23.0, 30.0])
    v, a = orc.scatter(src, index, 0, 3, "max", out=seed)
    np.testing.assert_array_equal(v, [10.0, 20.0, 30.0])
    np.testing.assert_array_equal(a, [3, 3, 3])


# ----------------------------------------------------------------- log-sum-exp / grouped softmax
def test_segment_logsumexp_matches_torch():
    rng = np.random.default_rng(13)
    lengths = rng.poisson(4, size=40)
    lengths[::9] = 0
    src = (rng.standard_normal((int(lengths.sum()), 5)) * 30).astype(np.float32)
    ptr = np.concatenate([[0], np.cumsum(lengths)])
    out = orc.segment_logsumexp(src, ptr)
    for s in range(40):
        a, z = ptr[s], ptr[s + 1]
        ref = torch.logsumexp(torch.from_numpy(src[a:z]).double(), 0).numpy() if z > a else np.full(5, -np.inf)
        np.testing.assert_allclose(out[s], ref, rtol=1e-12)


def test_segment_logsumexp_special_values():
    src = np.array([[-np.inf], [-np.inf], [np.inf], [1.0], [np.nan], [2.0]], dtype=np.float32)
    out = orc.segment_logsumexp(src, np.array([0, 2, 4, 6, 6]))
    assert out[0, 0] == -np.inf and out[1, 0] == np.inf and np.isnan(out[2, 0]) and out[3, 0] == -np.inf


@pytest.mark.parametrize("mode", ["softmax", "log_softmax", "logsumexp"])
def test_group_softmax_matches_torch_per_group(mode):
    rng = np.random.default_rng(14)
    src = (rng.standard_normal((2, 30, 3)) * 5).astype(np.float32)
    index = rng.integers(0, 8, size=30)
    index[index == 5] = 6  # group 5 empty
    out = orc.group_softmax(src, index, 1, 8, mode)
    t = torch.from_numpy(src).double()
    for g in range(8):
        pos = np.nonzero(index == g)[0]
        if mode == "logsumexp":
            ref = torch.logsumexp(t[:, pos], 1).numpy() if pos.size else np.full((2, 3), -np.inf)
            np.testing.assert_allclose(out[:, g], ref, rtol=1e-12)
        elif pos.size:
            fn = torch.softmax if mode == "softmax" else torch.log_softmax
            np.testing.assert_allclose(out[:, pos], fn(t[:, pos], 1).numpy(), rtol=1e-12, atol=1e-15)


def test_group_softmax_special_values_follow_torch():
    src = np.array([np.inf, 1.0, -np.inf, 2.0, np.nan, 0.0, -np.inf, -np.inf], dtype=np.float32)
    index = np.array([0, 0, 1, 1, 2, 2, 3, 3])
    t = torch.from_numpy(src).double()
    for mode, fn in (("softmax", torch.softmax), ("log_softmax", torch.log_softmax)):
        out = orc.group_softmax(src, index, 0, 4, mode)
        ref = np.concatenate([fn(t[2 * g:2 * g + 2], 0).numpy() for g in range(4)])
        np.testing.assert_array_equal(np.isnan(out), np.isnan(ref))
        np.testing.assert_allclose(out[~np.isnan(ref)], ref[~np.isnan(ref)])


# ----------------------------------------------------------------- SDDMM
def _csr_small(rng, m, n, avg):
    deg = rng.poisson(avg, size=m)
    deg[::5] = 0
    col = np.concatenate([np.sort(rng.integers(0, n, d)) for d in deg]).astype(np.int64)
    return np.concatenate([[0], np.cumsum(deg)]).astype(np.int64), col


def test_sddmm_dot_matches_sampled_addmm():
    rng = np.random.default_rng(61)
    ptr, col = _csr_small(rng, 40, 30, 5)
    q = rng.standard_normal((40, 8)).astype(np.float32)
    k = rng.standard_normal((30, 8)).astype(np.float32)
    got = orc.sddmm(ptr, col, q, k, "dot", 0, 2)
    a = torch.sparse_csr_tensor(torch.from_numpy(ptr), torch.from_numpy(col), torch.zeros(col.size, dtype=torch.float64),
                                size=(40, 30))
    ref = torch.sparse.sampled_addmm(a, torch.from_numpy(q).double(), torch.from_numpy(k).double().t()).values()
    np.testing.assert_allclose(got, ref.numpy(), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("op", ["dot", "add", "sub", "mul", "div", "copy_lhs", "copy_rhs"])
@pytest.mark.parametrize("lt,rt", [(0, 2), (2, 0), (1, 0), (2, 1)])
def test_sddmm_brute_force(op, lt, rt):
    rng = np.random.default_rng(62)
    ptr, col = _csr_small(rng, 12, 10, 3)
    nnz = col.size
    rows = {0: 12, 1: nnz, 2: 10}
    lhs = rng.standard_normal((rows[lt], 3)).astype(np.float32)
    rhs = (rng.standard_normal((rows[rt], 3)) + 3).astype(np.float32)
    got = orc.sddmm(ptr, col, lhs if op != "copy_rhs" else None, rhs if op != "copy_lhs" else None, op, lt, rt)
    for r in range(12):
        for e in range(ptr[r], ptr[r + 1]):
            pick = lambda t: r if t == 0 else (e if t == 1 else col[e])
            a = lhs[pick(lt)].astype(np.float64)
            b = rhs[pick(rt)].astype(np.float64)
            ref = {"dot": (a * b).sum(), "add": a + b, "sub": a - b, "mul": a * b, "div": a / b,
                   "copy_lhs": a, "copy_rhs": b}[op]
            np.testing.assert_allclose(got[e], ref, rtol=1e-12)


# ----------------------------------------------------------------- DGL spmm
@pytest.mark.parametrize("reduce,torch_reduce", [("max", "amax"), ("min", "amin")])
def test_spmm_dgl_extrema_propagate_nan_like_scatter_reduce(reduce, torch_reduce):
    rng = np.random.default_rng(63)
    ptr, col = _csr_small(rng, 30, 20, 4)
    x = rng.standard_normal((20, 6)).astype(np.float32)
    x[rng.random(x.shape) < 0.05] = np.nan
    got = orc.spmm_dgl(ptr, col, x, None, "copy_lhs", reduce)
    rows = torch.repeat_interleave(torch.arange(30), torch.from_numpy(np.diff(ptr)))
    init = float("-inf") if reduce == "max" else float("inf")
    ref = torch.full((30, 6), init, dtype=torch.float64).scatter_reduce(
        0, rows[:, None].expand(-1, 6), torch.from_numpy(x).double()[torch.from_numpy(col)], torch_reduce,
        include_self=True)
    ref[torch.from_numpy(np.diff(ptr)) == 0] = 0
    np.testing.assert_array_equal(np.isnan(got), torch.isnan(ref).numpy())
    np.testing.assert_allclose(got, ref.numpy(), equal_nan=True)


@pytest.mark.parametrize("op", ["add", "sub", "mul", "div", "copy_rhs"])
@pytest.mark.parametrize("width", [1, 4])
def test_spmm_dgl_messages_brute_force(op, width):
    rng = np.random.default_rng(64)
    ptr, col = _csr_small(rng, 15, 9, 3)
    x = rng.standard_normal((9, 4)).astype(np.float32)
    w = (rng.standard_normal((col.size, width)) + 2).astype(np.float32)
    for reduce in ("sum", "mean", "max"):
        got = orc.spmm_dgl(ptr, col, None if op == "copy_rhs" else x, w if width == 4 or op != "copy_rhs" else
                           np.repeat(w, 4, axis=1), op, reduce)
        for r in range(15):
            msgs = []
            for e in range(ptr[r], ptr[r + 1]):
                a = x[col[e]].astype(np.float64)
                b = np.broadcast_to(w[e].astype(np.float64), (4,))
                msgs.append({"add": a + b, "sub": a - b, "mul": a * b, "div": a / b, "copy_rhs": b}[op])
            if not msgs:
                ref = np.zeros(4)
            else:
                arr = np.stack(msgs)
                ref = {"sum": arr.sum(0), "mean": arr.mean(0), "max": arr.max(0)}[reduce]
            np.testing.assert_allclose(got[r], ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("mode", ["softmax", "log_softmax", "logsumexp"])
def test_group_softmax_backward_matches_torch_autograd(mode):
    # autograd of torch's own float64 per-group softmax / log_softmax / logsumexp
    rng = np.random.default_rng(15)
    src = (rng.standard_normal((2, 25, 3)) * 4).astype(np.float32)
    index = rng.integers(0, 6, size=25)
    index[index == 2] = 3  # group 2 empty
    gshape = (2, 6, 3) if mode == "logsumexp" else src.shape
    grad = rng.standard_normal(gshape).astype(np.float32)
    got = orc.group_softmax_backward(src, grad, index, 1, 6, mode)
    t = torch.from_numpy(src).double().requires_grad_(True)
    g = torch.from_numpy(grad).double()
    outs = []
    for grp in range(6):
        pos = torch.from_numpy(np.nonzero(index == grp)[0])
        if mode == "logsumexp":
            if pos.numel():
                outs.append((torch.logsumexp(t[:, pos], 1) * g[:, grp]).sum())
        elif pos.numel():
            fn = torch.softmax if mode == "softmax" else torch.log_softmax
            outs.append((fn(t[:, pos], 1) * g[:, pos]).sum())
    torch.stack(outs).sum().backward()
    np.testing.assert_allclose(got, t.grad.numpy(), rtol=1e-12, atol=1e-14)


def test_group_softmax_backward_special_values_follow_torch():
    # +inf / -inf groups give NaN gradients exactly where torch's autograd does
    src = np.array([np.inf, 1.0, -np.inf, -np.inf, 0.5, 2.0], dtype=np.float32)
    index = np.array([0, 0, 1, 1, 2, 2])
    for mode in ("softmax", "log_softmax", "logsumexp"):
        gshape = (3,) if mode == "logsumexp" else (6,)
        grad = np.linspace(0.5, 1.5, gshape[0]).astype(np.float32)
        got = orc.group_softmax_backward(src, grad, index, 0, 3, mode)
        t = torch.from_numpy(src).double().requires_grad_(True)
        g = torch.from_numpy(grad).double()
        tot = 0
        for grp in range(3):
            sl = slice(2 * grp, 2 * grp + 2)
            if mode == "logsumexp":
                tot = tot + torch.logsumexp(t[sl], 0) * g[grp]
            else:
                fn = torch.softmax if mode == "softmax" else torch.log_softmax
                tot = tot + (fn(t[sl], 0) * g[sl]).sum()
        tot.backward()
        ref = t.grad.numpy()
        np.testing.assert_array_equal(np.isnan(got), np.isnan(ref), err_msg=mode)
        np.testing.assert_allclose(got[~np.isnan(ref)], ref[~np.isnan(ref)], rtol=1e-12, err_msg=mode)


# ----------------------------------------------------------------- gather_csr / gather_coo
# reference test/gather_csr/arch35/golden.py:23-51 (CASES: src, coo index, indptr, expected)
GATHER_CASES = [
    ([1, 2, 3, 4], [0, 0, 1, 1, 1, 3], [0, 2, 5, 5, 6], [1, 1, 2, 2, 2, 4]),
    ([[1, 2], [3, 4], [5, 6], [7, 8]], [0, 0, 1, 1, 1, 3], [0, 2, 5, 5, 6],
     [[1, 2], [1, 2], [3, 4], [3, 4], [3, 4], [7, 8]]),
    ([[1, 3, 5, 7], [2, 4, 6, 8]], [[0, 0, 1, 1, 1, 3], [0, 0, 0, 1, 1, 2]],
     [[0, 2, 5, 5, 6], [0, 3, 5, 6, 6]], [[1, 1, 3, 3, 3, 7], [2, 2, 2, 4, 4, 6]]),
    ([[[1, 2], [3, 4], [5, 6]], [[7, 9], [10, 11], [12, 13]]], [[0, 0, 1], [0, 2, 2]],
     [[0, 2, 3, 3], [0, 1, 1, 3]], [[[1, 2], [1, 2], [3, 4]], [[7, 9], [12, 13], [12, 13]]]),
    ([[1], [2]], [[0, 0], [0, 0]], [[0, 2], [0, 2]], [[1, 1], [2, 2]]),
    ([[[1, 1]], [[2, 2]]], [[0, 0], [0, 0]], [[0, 2], [0, 2]], [[[1, 1], [1, 1]], [[2, 2], [2, 2]]]),
]


@pytest.mark.parametrize("case", range(len(GATHER_CASES)))
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32, torch.float64, torch.int32,
                                   torch.int64])
def test_gather_official_cases(case, dtype):
    src, coo, ptr, expected = GATHER_CASES[case]
    s = torch.tensor(src).to(dtype)
    want = torch.tensor(expected).to(dtype)
    assert torch.equal(orc.gather_csr(s, np.array(ptr)), want)
    assert torch.equal(orc.gather_coo(s, np.array(coo)), want)


def test_gather_csr_uncovered_prefix_kat():
    # reference test/gather_csr/arch35/test_gather_csr.py:278-283
    got = orc.gather_csr(torch.tensor([3, 5], dtype=torch.int32), np.array([2, 4, 6]))
    assert torch.equal(got, torch.tensor([0, 0, 3, 3, 5, 5], dtype=torch.int32))


def test_gather_matches_repeat_interleave_and_index_select():
    rng = np.random.default_rng(16)
    lengths = rng.integers(0, 5, 40)
    ptr = np.concatenate([[0], np.cumsum(lengths)])
    src = torch.from_numpy(rng.standard_normal((40, 7)))
    want = src.repeat_interleave(torch.from_numpy(lengths), dim=0)
    assert torch.equal(orc.gather_csr(src, ptr), want)
    idx = np.repeat(np.arange(40), lengths)
    assert torch.equal(orc.gather_coo(src, idx), src.index_select(0, torch.from_numpy(idx)))
