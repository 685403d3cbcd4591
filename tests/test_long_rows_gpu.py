"""GPU parity for rows whose records span many engine chunks.

A row spanning more than 64 chunks is finished in two stages: its interior
chunks' partial records are first folded in runs of 32 (one run per aligned
group of 32 chunks), then the fix-up folds the row's first record, the run
records and its last record.  Inside such a row, whole 64-position windows
take the engine's long-run loop (contiguous mode).  These tests force small
chunks (OGN_ENGINE_CHUNK=64) so that modest inputs hit every boundary case:
a row spanning exactly 64 chunks (not long) and 65 chunks (long), long rows
starting exactly on a chunk boundary, two long rows meeting inside one group
of 32 chunks, empty rows between them, and batched pointers.  Same bars as
the other parity tests: min/max values and args bit-exact, sums within
rel 1e-5 (fp32) / 1e-2 (fp16, bf16) of the oracle.
"""

import os

import numpy as np
import pytest
import torch

from _util import assert_exact, assert_sum_close, cast_like

pytestmark = pytest.mark.gpu

CH = 64
# positions: 5 | 0 | 70 chunks from offset 5 | up to a chunk boundary | 65
# chunks exactly (span 64: not long) | 66 chunks from a boundary (span 65:
# long) | short rows | long | two adjacent long rows | a short tail
LENGTHS = np.array([5, 0, 70 * CH, CH - 5, 65 * CH, 66 * CH, 2, 200 * CH + 17, 0, 0, 33, 130 * CH, 130 * CH,
                    1, 7000, 3], dtype=np.int64)


@pytest.fixture
def small_chunks():
    old = os.environ.get("OGN_ENGINE_CHUNK")
    os.environ["OGN_ENGINE_CHUNK"] = str(CH)
    yield
    if old is None:
        del os.environ["OGN_ENGINE_CHUNK"]
    else:
        os.environ["OGN_ENGINE_CHUNK"] = old


def _src(rng, n, feat, dtype, ties):
    if ties:
        a = rng.integers(-4, 5, size=(n, feat)).astype(np.float32)
    else:
        a = rng.standard_normal((n, feat)).astype(np.float32)
    return torch.from_numpy(a).to(dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("reduce", ["sum", "mean", "min", "max"])
@pytest.mark.parametrize("feat", [1, 4, 32, 33, 128])
def test_segment_csr_long_rows(ogn, oracle, small_chunks, dtype, reduce, feat):
    rng = np.random.default_rng(feat)
    indptr = torch.from_numpy(np.concatenate([[0], np.cumsum(LENGTHS)]))
    src = _src(rng, int(LENGTHS.sum()), feat, dtype, reduce in ("min", "max"))
    res = getattr(ogn, f"segment_{reduce}_csr")(src.cuda(), indptr.cuda())
    out, arg = res if isinstance(res, tuple) else (res, None)
    gold, garg = oracle.segment_csr(src, indptr, reduce)
    what = f"long/{dtype}/{reduce}/f{feat}"
    if arg is not None:
        assert_exact(out, cast_like(gold, dtype), what + " values")
        assert_exact(arg, garg, what + " arg")
    else:
        scale, _ = oracle.segment_csr(src.float().abs(), indptr, reduce)
        assert_sum_close(out, gold, scale, dtype, what)


@pytest.mark.parametrize("reduce", ["sum", "mean", "min", "max"])
@pytest.mark.parametrize("feat", [1, 32])
def test_segment_coo_long_rows_with_out(ogn, oracle, small_chunks, reduce, feat):
    # later-tie rule and out seeds through the pre-folded runs
    rng = np.random.default_rng(3 + feat)
    m = LENGTHS.size
    index = np.repeat(np.arange(m), LENGTHS)
    src = _src(rng, index.size, feat, torch.float32, True)
    out = torch.from_numpy(rng.integers(-4, 5, size=(m, feat)).astype(np.float32))
    res = getattr(ogn, f"segment_{reduce}_coo")(src.cuda(), torch.from_numpy(index).cuda(), out.clone().cuda(), m)
    got, arg = res if isinstance(res, tuple) else (res, None)
    gold, garg = oracle.segment_coo(src, index, m, reduce, out.double().numpy())
    if arg is not None:
        assert_exact(got, gold, "coo values")
        assert_exact(arg, garg, "coo arg")
    else:
        scale, _ = oracle.segment_coo(src.abs(), index, m, reduce, out.double().abs().numpy())
        assert_sum_close(got, gold, scale, torch.float32, "coo")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("feat", [1, 32, 128])
def test_segment_logsumexp_long_rows(ogn, oracle, small_chunks, dtype, feat):
    rng = np.random.default_rng(11)
    indptr = torch.from_numpy(np.concatenate([[0], np.cumsum(LENGTHS)]))
    src = torch.from_numpy((rng.standard_normal((int(LENGTHS.sum()), feat)) * 4).astype(np.float32)).to(dtype)
    src[100, 0] = float("inf")  # the first long row: +inf
    src[70 * CH + 50, -1] = float("nan")  # inside a long row: NaN
    got = ogn.segment_logsumexp(src.cuda(), indptr.cuda()).float().cpu().numpy()
    gold = cast_like(oracle.segment_logsumexp(src, indptr), dtype)
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    np.testing.assert_allclose(got, gold, rtol=tol, atol=tol)


def test_segment_csr_long_rows_batched_pointers(ogn, oracle, small_chunks):
    # per-batch pointer rows: batch 1 has its long rows elsewhere
    rng = np.random.default_rng(5)
    l0 = LENGTHS
    l1 = np.concatenate([l0[::-1][:-1], [l0[0]]])
    assert l1.sum() == l0.sum()
    indptr = torch.from_numpy(np.stack([np.concatenate([[0], np.cumsum(l)]) for l in (l0, l1)]))
    src = _src(rng, int(l0.sum()), 8, torch.float32, True).view(1, -1, 8).repeat(2, 1, 1).contiguous()
    src[1] = _src(rng, int(l0.sum()), 8, torch.float32, True)
    for reduce in ("sum", "max"):
        res = getattr(ogn, f"segment_{reduce}_csr")(src.cuda(), indptr.cuda())
        out, arg = res if isinstance(res, tuple) else (res, None)
        for b in range(2):
            gold, garg = oracle.segment_csr(src[b], indptr[b], reduce)
            if arg is not None:
                assert_exact(out[b], gold, f"batch{b} values")
                assert_exact(arg[b], garg, f"batch{b} arg")
            else:
                scale, _ = oracle.segment_csr(src[b].abs(), indptr[b], reduce)
                assert_sum_close(out[b], gold, scale, torch.float32, f"batch{b}")


@pytest.mark.parametrize("reduce", ["sum", "mean", "min", "max"])
@pytest.mark.parametrize("dtype,k", [(torch.float32, 128), (torch.bfloat16, 32), (torch.float16, 8)])
def test_spmm_long_rows(ogn, oracle, small_chunks, reduce, dtype, k):
    # gather mode: one chunk is 64 edges, so every long row pre-folds
    rng = np.random.default_rng(k)
    n = 3000
    col = np.concatenate([np.sort(rng.integers(0, n, d)) for d in LENGTHS]).astype(np.int64)
    ptr = torch.from_numpy(np.concatenate([[0], np.cumsum(LENGTHS)]))
    mat = _src(rng, n, k, dtype, reduce in ("min", "max"))
    val = torch.from_numpy(rng.integers(1, 3, col.size).astype(np.float32)).to(dtype)
    res = ogn.csr_spmm(ptr.cuda(), torch.from_numpy(col).cuda(), val.cuda(), mat.cuda(), reduce)
    got, arg = res if reduce in ("min", "max") else (res, None)
    gold, garg = oracle.spmm_csr(ptr, torch.from_numpy(col), val, mat, reduce)
    what = f"spmm/{dtype}/k{k}/{reduce}"
    if arg is not None:
        assert_exact(got, cast_like(gold, dtype), what + " values")
        assert_exact(arg, garg, what + " arg")
    else:
        scale, _ = oracle.spmm_csr(ptr, torch.from_numpy(col), val.float().abs(), mat.float().abs(), reduce)
        assert_sum_close(got, gold, scale, dtype, what)


@pytest.mark.parametrize("reduce", ["sum", "mean"])
def test_spmm_int8_long_rows(ogn, oracle, small_chunks, reduce):
    # int32 records through the pre-fold; exact
    rng = np.random.default_rng(8)
    n, k = 2000, 16
    col = np.concatenate([np.sort(rng.integers(0, n, d)) for d in LENGTHS]).astype(np.int64)
    ptr = torch.from_numpy(np.concatenate([[0], np.cumsum(LENGTHS)]))
    mat = torch.from_numpy(rng.integers(-128, 128, (n, k)).astype(np.int8))
    val = torch.from_numpy(rng.integers(-128, 128, col.size).astype(np.int8))
    got = ogn.csr_spmm(ptr.cuda(), torch.from_numpy(col).cuda(), val.cuda(), mat.cuda(), reduce,
                       output_dtype=torch.int32)
    gold, _ = oracle.spmm_csr(ptr, torch.from_numpy(col), val, mat, reduce)
    assert_exact(got, oracle.spmm_output_cast(gold, torch.int32), "int8 long rows")


@pytest.mark.parametrize("reduce", ["sum", "max"])
def test_scatter_hub_default_chunks(ogn, oracle, reduce):
    # default chunk sizes: a 300 000-position hub row spans ~590 chunks
    rng = np.random.default_rng(21)
    lengths = np.array([4, 300_000, 0, 9, 130_000, 1], dtype=np.int64)
    index = np.repeat(np.arange(lengths.size), lengths)
    src = _src(rng, index.size, 32, torch.float32, reduce == "max")
    res = ogn.scatter(src.cuda(), torch.from_numpy(index).cuda(), 0, dim_size=lengths.size, reduce=reduce)
    got = res[0] if isinstance(res, tuple) else res
    gold, _ = oracle.scatter(src.numpy(), index[:, None], 0, lengths.size, reduce)
    if reduce == "max":
        assert_exact(got, gold, "scatter max")
    else:
        scale, _ = oracle.scatter(np.abs(src.numpy()), index[:, None], 0, lengths.size, reduce)
        assert_sum_close(got, gold, scale, torch.float32, "scatter sum")
