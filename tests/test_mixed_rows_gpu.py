"""GPU parity for engine chunks that mix short rows with long ones.

A contiguous-mode chunk holding two or more row boundaries has its rows
dealt to the wave's sub-groups, one row each, except rows with more than
L positions in the chunk (twice the chunk's mean row length, at least 16),
which the whole wave folds afterwards with a position-ordered merge of the
sub-group partials.  These inputs put long rows (17 .. 3000 positions)
between runs of 0-3 position rows, at forced small chunks (64 and 256
positions: long rows then also cross chunk edges, leaving head / tail
records from the wave fold) and at the default chunk size.  Same bars as
the other parity tests: min/max values and args bit-exact, sums within
rel 1e-5 (fp32) / 1e-2 (fp16, bf16) of the oracle.
"""

import os

import numpy as np
import pytest
import torch

from _util import assert_exact, assert_sum_close, cast_like

pytestmark = pytest.mark.gpu


def _lengths(seed, rows=4000):
    rng = np.random.default_rng(seed)
    kind = rng.random(rows)
    lengths = np.where(kind < 0.2, 0, rng.integers(1, 4, rows))
    mid = kind > 0.9
    lengths[mid] = rng.integers(4, 40, int(mid.sum()))
    long_ = kind > 0.98
    lengths[long_] = rng.integers(17, 3000, int(long_.sum()))
    lengths[5] = 5000  # one long row near the start
    return lengths.astype(np.int64)


@pytest.fixture(params=[64, 256, None], ids=["chunk64", "chunk256", "default"])
def chunk(request):
    old = os.environ.get("OGN_ENGINE_CHUNK")
    if request.param is not None:
        os.environ["OGN_ENGINE_CHUNK"] = str(request.param)
    yield request.param
    if old is None:
        os.environ.pop("OGN_ENGINE_CHUNK", None)
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
def test_segment_csr_mixed_rows(ogn, oracle, chunk, dtype, reduce, feat):
    lengths = _lengths(feat)
    rng = np.random.default_rng(100 + feat)
    indptr = torch.from_numpy(np.concatenate([[0], np.cumsum(lengths)]))
    src = _src(rng, int(lengths.sum()), feat, dtype, reduce in ("min", "max"))
    res = getattr(ogn, f"segment_{reduce}_csr")(src.cuda(), indptr.cuda())
    out, arg = res if isinstance(res, tuple) else (res, None)
    gold, garg = oracle.segment_csr(src, indptr, reduce)
    what = f"mixed/{chunk}/{dtype}/{reduce}/f{feat}"
    if arg is not None:
        assert_exact(out, cast_like(gold, dtype), what + " values")
        assert_exact(arg, garg, what + " arg")
    else:
        scale, _ = oracle.segment_csr(src.float().abs(), indptr, reduce)
        assert_sum_close(out, gold, scale, dtype, what)


@pytest.mark.parametrize("reduce", ["sum", "mean", "min", "max"])
@pytest.mark.parametrize("feat", [1, 32])
def test_scatter_and_coo_mixed_rows(ogn, oracle, chunk, reduce, feat):
    # later-tie rule (scatter / segment_coo) and out seeds through the wave fold
    lengths = _lengths(7 + feat)
    rng = np.random.default_rng(3 + feat)
    m = lengths.size
    index = np.repeat(np.arange(m), lengths)
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
    res = ogn.scatter(src.cuda(), torch.from_numpy(index).cuda(), 0, dim_size=m, reduce=reduce)
    got = res[0] if isinstance(res, tuple) else res
    gold, _ = oracle.scatter(src.numpy(), index[:, None], 0, m, reduce)
    if reduce in ("min", "max"):
        assert_exact(got, gold, "scatter")
    else:
        scale, _ = oracle.scatter(np.abs(src.numpy()), index[:, None], 0, m, reduce)
        assert_sum_close(got, gold, scale, torch.float32, "scatter")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("feat", [1, 32, 33])
def test_segment_logsumexp_mixed_rows(ogn, oracle, chunk, dtype, feat):
    lengths = _lengths(11)
    rng = np.random.default_rng(11)
    indptr = torch.from_numpy(np.concatenate([[0], np.cumsum(lengths)]))
    src = torch.from_numpy((rng.standard_normal((int(lengths.sum()), feat)) * 4).astype(np.float32)).to(dtype)
    long_rows = np.nonzero(lengths > 100)[0]
    r0, r1 = int(long_rows[0]), int(long_rows[-1])
    src[int(indptr[r0]) + 40, 0] = float("inf")  # inside a long row: +inf
    src[int(indptr[r1]) + 70, -1] = float("nan")  # inside another: NaN
    got = ogn.segment_logsumexp(src.cuda(), indptr.cuda()).float().cpu().numpy()
    gold = cast_like(oracle.segment_logsumexp(src, indptr), dtype)
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    np.testing.assert_allclose(got, gold, rtol=tol, atol=tol)


@pytest.mark.parametrize("reduce", ["sum", "mean", "min", "max"])
@pytest.mark.parametrize("feat", [4, 32, 33])
def test_segment_csr_mixed_rows_batched_pointers(ogn, oracle, chunk, reduce, feat):
    # one pointer row per batch (different row layouts, the last starting
    # past position 0): the finished rows of every batch, staged and written
    # in groups, land in that batch's output
    rng = np.random.default_rng(40 + feat)
    n = 6000
    rows = []
    for bi in range(3):
        lengths = _lengths(bi + feat, rows=1500)
        lead = 0 if bi < 2 else 17
        lengths = lengths[np.cumsum(lengths) + lead <= n]
        ptr = np.concatenate([[lead], lead + np.cumsum(lengths)])
        rows.append(ptr)
    m = min(r.size for r in rows) - 1
    indptr = np.stack([r[: m + 1] for r in rows])
    ties = reduce in ("min", "max")
    src = _src(rng, 3 * n, feat, torch.float32, ties).reshape(3, n, feat)
    res = getattr(ogn, f"segment_{reduce}_csr")(src.cuda(), torch.from_numpy(indptr).cuda())
    out, arg = res if isinstance(res, tuple) else (res, None)
    for bi in range(3):
        gold, garg = oracle.segment_csr(src[bi], indptr[bi], reduce)
        what = f"batched/{chunk}/{reduce}/f{feat}/b{bi}"
        if ties:
            assert_exact(out[bi], gold, what + " values")
            assert_exact(arg[bi], garg, what + " arg")
        else:
            scale, _ = oracle.segment_csr(src[bi].abs(), indptr[bi], reduce)
            assert_sum_close(out[bi], gold, scale, torch.float32, what)


@pytest.mark.parametrize("reduce", ["sum", "max", "logsumexp"])
@pytest.mark.parametrize("feat", [1, 32, 33])
def test_staged_and_direct_row_stores_agree(ogn, chunk, reduce, feat):
    # OGN_ENGINE_NO_STAGE=1 writes each finished short row directly; the
    # default stages rows in LDS and writes them in groups: same bits
    lengths = _lengths(50 + feat)
    rng = np.random.default_rng(60 + feat)
    indptr = torch.from_numpy(np.concatenate([[0], np.cumsum(lengths)])).cuda()
    src = _src(rng, int(lengths.sum()), feat, torch.float32, reduce == "max").cuda()

    def run():
        if reduce == "logsumexp":
            return (ogn.segment_logsumexp(src, indptr),)
        res = getattr(ogn, f"segment_{reduce}_csr")(src, indptr)
        return res if isinstance(res, tuple) else (res,)

    staged = run()
    os.environ["OGN_ENGINE_NO_STAGE"] = "1"
    try:
        direct = run()
    finally:
        os.environ.pop("OGN_ENGINE_NO_STAGE", None)
    for a, b in zip(staged, direct):
        assert torch.equal(a.view(torch.int32) if a.dtype == torch.float32 else a,
                           b.view(torch.int32) if b.dtype == torch.float32 else b)


@pytest.mark.parametrize("op", ["sum", "max", "logsumexp", "scatter_max"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("feat", [1, 32, 33])
def test_nontemporal_and_plain_source_loads_agree(ogn, oracle, chunk, op, dtype, feat):
    # the library reads a contiguous source above 256 MiB with non-temporal
    # loads (separate kernel instances) and a smaller one with plain loads;
    # OGN_ENGINE_NT=1 / 0 forces either: same bits, and the oracle's values
    lengths = _lengths(70 + feat)
    rng = np.random.default_rng(80 + feat)
    ptr_np = np.concatenate([[0], np.cumsum(lengths)])
    indptr = torch.from_numpy(ptr_np).cuda()
    src = _src(rng, int(lengths.sum()), feat, dtype, op in ("max", "scatter_max"))
    dsrc = src.cuda()
    index = torch.from_numpy(np.repeat(np.arange(lengths.size), lengths)).cuda()

    def run():
        if op == "logsumexp":
            return (ogn.segment_logsumexp(dsrc, indptr),)
        if op == "scatter_max":
            return ogn.scatter_max(dsrc, index, 0, None, lengths.size)
        res = getattr(ogn, f"segment_{op}_csr")(dsrc, indptr)
        return res if isinstance(res, tuple) else (res,)

    outs = {}
    for mode in ("1", "0"):
        os.environ["OGN_ENGINE_NT"] = mode
        try:
            outs[mode] = [t.cpu() for t in run()]
        finally:
            os.environ.pop("OGN_ENGINE_NT", None)
    for a, b in zip(outs["1"], outs["0"]):
        assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                           b.view(torch.int16) if b.dtype == torch.bfloat16 else b)
    if op == "max":
        gold, garg = oracle.segment_csr(src, ptr_np, "max")
        assert_exact(outs["1"][0], cast_like(gold, dtype), "nt max values")
        assert_exact(outs["1"][1], garg, "nt max arg")
