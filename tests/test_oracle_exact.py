"""Pins of the exact-dtype (integer, float64) oracle functions.

Known-answer tests come from the reference's own tests
(test/segment_csr/arch35/test_segment_csr_golden.py:20-56,
test/segment_coo/arch35/test_segment_coo.py:493-531 and :772-826,
test/scatter/arch35/test_scatter.py:345-349); sums, extrema and float64
folds are checked against numpy's own routines (np.add.reduceat /
np.add.at / np.minimum.at / argmin), which share no code with the oracle.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as orc

INT_DTYPES = [np.int8, np.uint8, np.int16, np.int32, np.int64]


# ------------------------------------------------------------------ segment_csr KATs
@pytest.mark.parametrize("value", [16_777_217, -16_777_217, 9_007_199_254_740_993, -9_007_199_254_740_993])
def test_csr_int64_mean_keeps_exact_integer(value):
    # reference test_segment_csr_golden.py:21-29
    out, _ = orc.segment_csr(np.array([value], np.int64), np.array([0, 1]), "mean")
    assert out.tolist() == [value]


@pytest.mark.parametrize("dtype,count,expected", [(np.int8, 200, -1), (np.int8, 256, 0), (np.uint8, 256, 0)])
def test_csr_narrow_mean_wraps_count(dtype, count, expected):
    # reference test_segment_csr_golden.py:31-40
    src = np.zeros(count, dtype)
    src[0] = 100
    out, _ = orc.segment_csr(src, np.array([0, count]), "mean")
    assert out.tolist() == [expected]


def test_csr_integer_mean_truncates_and_int8_sum_wraps_first():
    # reference test_segment_csr_golden.py:42-56
    assert orc.segment_csr(np.array([-1, -2], np.int64), np.array([0, 2]), "mean")[0].tolist() == [-1]
    assert orc.segment_csr(np.array([100, 100], np.int8), np.array([0, 2]), "mean")[0].tolist() == [-28]


@pytest.mark.parametrize("dtype", INT_DTYPES)
def test_csr_sum_min_max_match_numpy(dtype):
    rng = np.random.default_rng(3)
    info = np.iinfo(dtype)
    lengths = rng.integers(0, 40, 60)
    ptr = np.concatenate([[0], np.cumsum(lengths)])
    src = rng.integers(info.min, info.max, (ptr[-1], 5), dtype=np.int64, endpoint=True).astype(dtype)
    got, _ = orc.segment_csr(src, ptr, "sum")
    for s in range(60):
        rows = src[ptr[s]:ptr[s + 1]].astype(np.int64)
        want = rows.sum(0).astype(dtype) if len(rows) else np.zeros(5, dtype)
        assert np.array_equal(got[s].astype(dtype), want)
    for reduce, fn, argfn in (("min", np.min, np.argmin), ("max", np.max, np.argmax)):
        got, arg = orc.segment_csr(src, ptr, reduce)
        for s in range(60):
            rows = src[ptr[s]:ptr[s + 1]]
            if len(rows) == 0:
                assert (got[s] == 0).all() and (arg[s] == src.shape[0]).all()
            else:  # numpy's argmin / argmax return the first occurrence
                assert np.array_equal(got[s], fn(rows, 0)) and np.array_equal(arg[s], ptr[s] + argfn(rows, 0))


# ------------------------------------------------------------------ segment_coo KATs
INTEGER_MEAN_COUNTS = (1, 0, 2, 3, 4, 7, 8, 16, 31, 32, 63, 64, 127, 128, 255, 256, 257, 511, 512, 513)


def integer_mean_extremes_case(dtype, channels, with_out):
    """The reference's closed-form case (test_segment_coo.py:772-826):
    one non-zero entry per segment, truncating mean of (value + seed)."""
    counts = INTEGER_MEAN_COUNTS
    index = np.repeat(np.arange(len(counts)), counts)
    info = np.iinfo(dtype)
    src = np.zeros((len(index), channels), dtype)
    initial = np.zeros((len(counts), channels), dtype)
    expected = np.zeros_like(initial)
    begin = 0
    for seg, count in enumerate(counts):
        values = [info.min, info.max, -count - 1, count + 1, -count + 1, count - 1, -1, 1]
        for ch in range(channels):
            value = values[(ch + seg) % len(values)]
            seed = (3 if value < 0 else -3) if with_out else 0
            initial[seg, ch] = seed
            if count:
                src[begin, ch] = value
                num = value + seed
                q = abs(num) // count
                expected[seg, ch] = -q if num < 0 else q
            else:
                expected[seg, ch] = seed
        begin += count
    return src, index, (initial if with_out else None), expected


@pytest.mark.parametrize("dtype", [np.int32, np.int64])
@pytest.mark.parametrize("channels", [1, 8, 96])
@pytest.mark.parametrize("with_out", [False, True])
def test_coo_integer_mean_extremes_kat(dtype, channels, with_out):
    src, index, initial, expected = integer_mean_extremes_case(dtype, channels, with_out)
    got, _ = orc.segment_coo(src, index, len(INTEGER_MEAN_COUNTS), "mean", out=initial)
    assert np.array_equal(got.astype(dtype), expected)


@pytest.mark.parametrize("dtype", [np.int8, np.uint8])
def test_coo_byte_mean_zero_narrowed_count_is_exact(dtype):
    # reference test_segment_coo.py:516-524: 256 threes -> 3
    got, _ = orc.segment_coo(np.full((256, 4), 3, dtype), np.zeros(256, np.int64), 1, "mean")
    assert (got == 3).all()


@pytest.mark.parametrize("dtype", [np.int8, np.uint8])
def test_coo_byte_mean_narrows_both_operands(dtype):
    # 200 ones: typed sum and count both narrow (int8: -56 / -56 = 1; uint8: 200 / 200)
    got, _ = orc.segment_coo(np.ones((200, 1), dtype), np.zeros(200, np.int64), 1, "mean")
    assert got.tolist() == [[1]]
    # 257 entries of 2: typed sum 514 -> 2, count 257 -> 1
    got, _ = orc.segment_coo(np.full((257, 1), 2, dtype), np.zeros(257, np.int64), 1, "mean")
    assert got.tolist() == [[2]]


def test_coo_later_tie_and_seed_rules():
    src = np.array([[4], [2], [2], [7], [7], [1]], np.int32)
    index = np.array([0, 0, 0, 2, 2, 2])
    v, a = orc.segment_coo(src, index, 3, "min")
    assert v[:, 0].tolist() == [2, 0, 1] and a[:, 0].tolist() == [2, 6, 5]
    v, a = orc.segment_coo(src, index, 3, "max")
    assert v[:, 0].tolist() == [4, 0, 7] and a[:, 0].tolist() == [0, 6, 4]
    v, a = orc.segment_coo(src, index, 3, "min", out=np.array([[2], [9], [0]], np.int32))
    assert v[:, 0].tolist() == [2, 9, 0] and a[:, 0].tolist() == [2, 6, 6]


# ------------------------------------------------------------------ scatter KATs
def test_scatter_integer_floor_mean_kat():
    # reference test_scatter.py:345-349
    src = np.array([[-3, -2, 4], [-2, -1, 5]], np.int32)
    got, _ = orc.scatter(src, np.broadcast_to(np.array([0, 0, 1]), src.shape), 1, 2, "mean")
    assert got.tolist() == [[-3, 4], [-2, 5]]


def test_scatter_narrow_wraps_and_counts():
    assert orc.scatter(np.array([100, 100], np.int8), np.array([0, 0]), 0, 1, "sum")[0].tolist() == [-56]
    assert orc.scatter(np.array([16, 16], np.int8), np.array([0, 0]), 0, 1, "mul")[0].tolist() == [0]
    # int8 count 200 narrows to -56 and clamps to 1: the mean is the typed sum
    assert orc.scatter(np.ones(200, np.int8), np.zeros(200, np.int64), 0, 1, "mean")[0].tolist() == [-56]
    # uint8 count 300 narrows to 44; sum of 300 ones wraps to 44 -> 1
    assert orc.scatter(np.ones(300, np.uint8), np.zeros(300, np.int64), 0, 1, "mean")[0].tolist() == [1]


@pytest.mark.parametrize("dtype", INT_DTYPES)
def test_scatter_matches_numpy_ufunc_at(dtype):
    rng = np.random.default_rng(5)
    info = np.iinfo(dtype)
    src = rng.integers(info.min, info.max, (3, 50, 4), dtype=np.int64, endpoint=True).astype(dtype)
    idx = rng.integers(0, 12, (3, 50, 4))
    for reduce, ufunc, start in (("sum", np.add, 0), ("mul", np.multiply, 1), ("min", np.minimum, info.max),
                                 ("max", np.maximum, info.min)):
        want = np.full((3, 12, 4), start, dtype)
        b, _, f = np.meshgrid(np.arange(3), np.arange(50), np.arange(4), indexing="ij")
        with np.errstate(over="ignore"):
            ufunc.at(want, (b, idx, f), src)
        got, arg = orc.scatter(src, idx, 1, 12, reduce)
        if reduce in ("min", "max"):
            touched = np.zeros((3, 12, 4), bool)
            touched[b, idx, f] = True
            want[~touched] = 0
            assert ((arg == 50) == ~touched).all()
        assert np.array_equal(got.astype(dtype), want), reduce


def test_scatter_f64_matches_numpy_in_order():
    rng = np.random.default_rng(6)
    src = rng.standard_normal((2, 300, 3))
    idx = rng.integers(0, 7, (2, 300, 3))
    b, _, f = np.meshgrid(np.arange(2), np.arange(300), np.arange(3), indexing="ij")
    want = np.zeros((2, 7, 3))
    np.add.at(want, (b, idx, f), src)  # unbuffered, element order: the golden's fold
    got, _ = orc.scatter(src, idx, 1, 7, "sum")
    assert np.array_equal(got, want)
    cnt = np.zeros((2, 7, 3))
    np.add.at(cnt, (b, idx, f), 1.0)
    got, _ = orc.scatter(src, idx, 1, 7, "mean")
    assert np.array_equal(got, np.where(cnt > 0, want / np.maximum(cnt, 1), 0.0))
    got, arg = orc.scatter(src, idx, 1, 7, "max")
    want = np.full((2, 7, 3), -np.inf)
    np.maximum.at(want, (b, idx, f), src)
    assert np.array_equal(got, np.where(np.isinf(want), 0.0, want))


def test_torch_tensors_accepted():
    got, _ = orc.segment_csr(torch.tensor([1, 2, 3], dtype=torch.int8), torch.tensor([0, 3]), "sum")
    assert got.tolist() == [6]
