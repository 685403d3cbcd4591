"""GPU parity of segment_csr / segment_coo / segment_reduce / segment_logsumexp
against the CPU oracle.  Cases follow the reference tests
(test/segment_csr/arch35/test_segment_csr.py, test/segment_coo/arch35/test_segment_coo.py,
test/segment_logsumexp/test_segment_logsumexp.py): KATs, random graphs per
dtype and reduction, broadcast / per-batch pointers, empty segments, `out`
identity, non-contiguous inputs, long segments spanning many wavefront chunks,
determinism and error contracts.  Sum/mean: |a - g| <= rtol * sum|x| (rtol
1e-5 fp32, 1e-2 fp16/bf16); min/max values and args bit-exact.
"""

import numpy as np
import pytest
import torch

from _util import assert_exact, assert_sum_close, cast_like

pytestmark = pytest.mark.gpu

DT = [torch.float32, torch.float16, torch.bfloat16]
REDUCES = ["sum", "mean", "min", "max"]
LSE_TOL = {torch.float32: 1e-5, torch.float16: 1e-2, torch.bfloat16: 1e-2}


def _lengths(rng, segs, mean, empty_every=7, long_every=None, long_len=0):
    lengths = rng.poisson(mean, size=segs)
    lengths[::empty_every] = 0
    if long_every:
        lengths[::long_every] = long_len
    return lengths


def _csr_check(ogn, oracle, src, indptr, reduce, what=""):
    fn = getattr(ogn, f"segment_{reduce}_csr")
    res = fn(src.cuda(), indptr.cuda())
    out, arg = res if isinstance(res, tuple) else (res, None)
    gold, garg = oracle.segment_csr(src, indptr, reduce)
    if reduce in ("min", "max"):
        assert_exact(out, cast_like(gold, src.dtype), what + " values")
        assert_exact(arg, garg, what + " arg")
    else:
        scale, _ = oracle.segment_csr(src.float().abs(), indptr, reduce)
        assert_sum_close(out, gold, scale, src.dtype, what)


def test_arg_first_occurrence_kat(ogn):
    # reference test/segment_csr/arch35/test_segment_csr.py:435-445
    src = torch.tensor([[5.0, 1.0, 1.0, 5.0, 2.0], [3.0, 3.0, 3.0, 3.0, 3.0]], device="cuda")
    indptr = torch.tensor([0, 5], device="cuda")
    out, arg = ogn.segment_min_csr(src, indptr)
    assert arg.cpu().tolist() == [[1, 0, 0, 1, 0]] and out.cpu().tolist() == [[3.0, 1.0, 1.0, 3.0, 2.0]]
    out, arg = ogn.segment_max_csr(src, indptr)
    assert arg.cpu().tolist() == [[0, 1, 1, 0, 1]] and out.cpu().tolist() == [[5.0, 3.0, 3.0, 5.0, 3.0]]


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("reduce", REDUCES)
@pytest.mark.parametrize("feat", [1, 3, 8, 64, 128, 200])
def test_segment_csr_random(ogn, oracle, dtype, reduce, feat):
    rng = np.random.default_rng(feat)
    lengths = _lengths(rng, 300, 9, long_every=97, long_len=3000)
    src = torch.from_numpy(rng.standard_normal((int(lengths.sum()), feat)).astype(np.float32)).to(dtype)
    indptr = torch.from_numpy(np.concatenate([[0], np.cumsum(lengths)]))
    _csr_check(ogn, oracle, src, indptr, reduce, f"csr/{dtype}/{reduce}/f{feat}")


@pytest.mark.parametrize("reduce", REDUCES)
def test_segment_csr_ties(ogn, oracle, reduce):
    rng = np.random.default_rng(5)
    lengths = _lengths(rng, 200, 30)
    src = torch.from_numpy(rng.integers(-2, 3, size=(int(lengths.sum()), 16)).astype(np.float32))
    indptr = torch.from_numpy(np.concatenate([[0], np.cumsum(lengths)]))
    _csr_check(ogn, oracle, src, indptr, reduce, "ties")


@pytest.mark.parametrize("reduce", REDUCES)
def test_segment_csr_broadcast_and_batched_pointers(ogn, oracle, reduce):
    rng = np.random.default_rng(6)
    src = torch.from_numpy(rng.standard_normal((3, 500, 8)).astype(np.float32))
    shared = torch.tensor([[0, 100, 100, 420, 500]])
    _csr_check(ogn, oracle, src, shared, reduce, "shared")
    per_batch = torch.tensor([[0, 10, 300, 500], [0, 0, 250, 499], [5, 5, 400, 450]])
    _csr_check(ogn, oracle, src, per_batch, reduce, "per-batch")


@pytest.mark.parametrize("reduce", REDUCES)
def test_segment_csr_pointer_offsets_and_out(ogn, oracle, reduce):
    # rows before indptr[0] and after indptr[-1] belong to no segment
    src = torch.randn(1000, 16, generator=torch.Generator().manual_seed(3))
    indptr = torch.tensor([37, 37, 300, 301, 900])
    _csr_check(ogn, oracle, src, indptr, reduce, "offsets")
    out = torch.empty(4, 16, device="cuda")
    res = ogn.segment_csr(src.cuda(), indptr.cuda(), out=out, reduce=reduce)
    assert res.data_ptr() == out.data_ptr()


def test_segment_csr_noncontiguous_src_and_out(ogn, oracle):
    base = torch.randn(400, 32, generator=torch.Generator().manual_seed(4))
    src = base[:, ::2]
    indptr = torch.tensor([0, 50, 50, 399, 400])
    out = torch.zeros(4, 32, device="cuda")[:, ::2]
    res = ogn.segment_csr(src.cuda(), indptr.cuda(), out=out, reduce="sum")
    assert res is out or res.data_ptr() == out.data_ptr()
    gold, _ = oracle.segment_csr(src, indptr, "sum")
    scale, _ = oracle.segment_csr(src.abs(), indptr, "sum")
    assert_sum_close(out, gold, scale, torch.float32, "noncontig")


def test_segment_csr_determinism_bitwise(ogn):
    # reference test/segment_csr/arch35/test_segment_csr.py:416-433
    torch.manual_seed(7)
    src = torch.randn(100000, 64)
    indptr = torch.zeros(257, dtype=torch.long)
    indptr[1:] = torch.cumsum(torch.randint(0, 1200, (256,)), 0)
    indptr = torch.clamp(indptr, max=100000)
    indptr[-1] = 100000
    for dtype in DT:
        s = src.to(dtype).cuda()
        for reduce in ("sum", "mean", "min", "max"):
            outs = [ogn.segment_csr(s, indptr.cuda(), reduce=reduce) for _ in range(4)]
            for o in outs[1:]:
                assert torch.equal(outs[0], o), (dtype, reduce)


def test_segment_csr_empty_and_errors(ogn):
    out = ogn.segment_csr(torch.empty(0, 4, device="cuda"), torch.zeros(3, dtype=torch.long, device="cuda"))
    assert out.shape == (2, 4) and bool((out == 0).all())
    with pytest.raises(RuntimeError, match="int64"):
        ogn.segment_csr(torch.ones(4, 2, device="cuda"), torch.tensor([0, 4], dtype=torch.int32, device="cuda"))
    with pytest.raises(RuntimeError, match="nondecreasing"):
        ogn.segment_csr(torch.ones(4, 2, device="cuda"), torch.tensor([0, 3, 2], device="cuda"))
    with pytest.raises(RuntimeError, match="non-negative"):
        ogn.segment_csr(torch.ones(4, 2, device="cuda"), torch.tensor([-1, 3], device="cuda"))
    # ends past src.size(dim) are clamped
    out = ogn.segment_csr(torch.ones(4, 2, device="cuda"), torch.tensor([0, 3, 9], device="cuda"))
    assert out.cpu().tolist() == [[3.0, 3.0], [1.0, 1.0]]
    with pytest.raises(ValueError, match="not valid"):
        ogn.segment_csr(torch.ones(4, 2, device="cuda"), torch.tensor([0, 4], device="cuda"), reduce="mul")
    with pytest.raises(TypeError):
        ogn.segment_csr(torch.ones(4, 2, dtype=torch.float64, device="cuda"), torch.tensor([0, 4], device="cuda"))


@pytest.mark.parametrize("reduce", ["sum", "mean", "max"])
def test_segment_csr_ends_past_source_with_chunk_crossing(ogn, oracle, reduce):
    """Segment ends past src.size(0) are clamped (the golden slices
    src[start:end]); the last segments, clamped, also span many wavefront
    chunks, so the chunk-row pass, the main kernel and the fix-up must agree
    on where the data ends."""
    rng = np.random.default_rng(77)
    length = 40_000
    src = torch.from_numpy(rng.standard_normal((length, 8)).astype(np.float32))
    lengths = rng.poisson(30, size=600)
    ptr = np.concatenate([[0], np.cumsum(lengths)])
    ptr = np.concatenate([ptr[ptr < length - 15_000], [length - 15_000, length - 5, length + 9_000, length + 20_000]])
    indptr = torch.from_numpy(ptr.astype(np.int64))
    clamped = indptr.clamp(max=length)
    _csr_check(ogn, oracle, src, clamped, reduce, f"clamped reference/{reduce}")
    fn = getattr(ogn, f"segment_{reduce}_csr")
    res = fn(src.cuda(), indptr.cuda())
    out, arg = res if isinstance(res, tuple) else (res, None)
    gold, garg = oracle.segment_csr(src, clamped, reduce)
    if reduce == "max":
        assert_exact(out, cast_like(gold, src.dtype), "ends past src values")
        assert_exact(arg, garg, "ends past src arg")
    else:
        scale, _ = oracle.segment_csr(src.abs(), clamped, reduce)
        assert_sum_close(out, gold, scale, torch.float32, f"ends past src/{reduce}")


def test_segment_reduce_and_legacy_max(ogn, oracle):
    rng = np.random.default_rng(8)
    lengths = _lengths(rng, 50, 6)
    src = torch.from_numpy(rng.standard_normal((int(lengths.sum()), 5)).astype(np.float32))
    offsets = torch.from_numpy(np.concatenate([[0], np.cumsum(lengths)])).int()
    out = ogn.segment_reduce(src.cuda(), offsets.cuda(), reduce="mean")
    gold, _ = oracle.segment_csr(src, offsets.long(), "mean")
    scale, _ = oracle.segment_csr(src.abs(), offsets.long(), "mean")
    assert_sum_close(out, gold, scale, torch.float32, "segment_reduce")
    # legacy int32 entry: value-only max; optional_out seeds max(src, out)
    # (reference golden test/segment_max_csr/arch35/golden.py:16-41)
    legacy = ogn.segment_max_csr(src.cuda(), offsets.cuda())
    gmax, _ = oracle.segment_csr(src, offsets.long(), "max")
    assert_exact(legacy, gmax.astype(np.float32))
    seed = torch.full((50, 5), 0.5, device="cuda")
    seeded = ogn.segment_max_csr_legacy(src.cuda(), offsets.cuda(), seed)
    assert_exact(seeded, np.maximum(gmax, 0.5).astype(np.float32))


# ----------------------------------------------------------------- segment_coo
@pytest.mark.parametrize("mode", REDUCES)
def test_segment_coo_unequal_segments_kat(ogn, mode):
    # reference test/segment_coo/arch35/test_segment_coo.py:892-911
    x = torch.tensor([[2, 5], [2, 1], [3, 6], [4, 6], [1, 2]], dtype=torch.float32, device="cuda")
    idx = torch.tensor([0, 0, 2, 2, 2], device="cuda")
    out = ogn.segment_coo(x, idx, dim_size=4, reduce=mode).cpu()
    ref = {"sum": [[4, 6], [0, 0], [8, 14], [0, 0]], "mean": [[2, 3], [0, 0], [8 / 3, 14 / 3], [0, 0]],
           "min": [[2, 1], [0, 0], [1, 2], [0, 0]], "max": [[2, 5], [0, 0], [4, 6], [0, 0]]}[mode]
    torch.testing.assert_close(out, torch.tensor(ref, dtype=torch.float32), rtol=1e-6, atol=1e-6)
    if mode in ("min", "max"):
        _, arg = getattr(ogn, "segment_" + mode + "_coo")(x, idx, dim_size=4)
        expected = {"min": [[1, 1], [5, 5], [4, 4], [5, 5]], "max": [[1, 0], [5, 5], [3, 3], [5, 5]]}[mode]
        assert torch.equal(arg.cpu(), torch.tensor(expected))


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("mode", REDUCES)
@pytest.mark.parametrize("with_out", [False, True])
def test_segment_coo_random(ogn, oracle, dtype, mode, with_out):
    rng = np.random.default_rng(21)
    idx = np.sort(rng.integers(0, 200, 6000))
    idx[:2500] = np.sort(rng.integers(0, 3, 2500))  # a few long segments
    idx = np.sort(idx)
    src = torch.from_numpy(rng.integers(-4, 5, size=(2, 6000, 24)).astype(np.float32)).to(dtype)
    seed = torch.from_numpy(rng.standard_normal((2, 210, 24)).astype(np.float32)).to(dtype) if with_out else None
    index = torch.from_numpy(idx)
    fn = getattr(ogn, f"segment_{mode}_coo")
    dev_out = seed.cuda() if with_out else None
    res = fn(src.cuda(), index.unsqueeze(0).cuda(), out=dev_out, dim_size=None if with_out else 210)
    out, arg = res if isinstance(res, tuple) else (res, None)
    if with_out:
        assert out.data_ptr() == dev_out.data_ptr()
    gold, garg = oracle.segment_coo(src, index.unsqueeze(0), 210, mode,
                                    out=None if seed is None else seed.double().numpy())
    if mode in ("min", "max"):
        assert_exact(out, cast_like(gold, dtype), "coo values")
        assert_exact(arg, garg, "coo arg")
    else:
        scale, _ = oracle.segment_coo(src.float().abs(), index.unsqueeze(0), 210, mode,
                                      out=None if seed is None else seed.double().abs().numpy())
        assert_sum_close(out, gold, scale, dtype, f"coo/{mode}")


def test_segment_coo_batched_index_and_inferred_size(ogn, oracle):
    rng = np.random.default_rng(22)
    idx = np.stack([np.sort(rng.integers(0, 40, 300)), np.sort(rng.integers(0, 40, 300))])
    src = torch.from_numpy(rng.standard_normal((2, 300, 4)).astype(np.float32))
    out = ogn.segment_sum_coo(src.cuda(), torch.from_numpy(idx).cuda())
    segs = int(idx.max()) + 1
    assert out.shape == (2, segs, 4)
    gold, _ = oracle.segment_coo(src, idx, segs, "sum")
    scale, _ = oracle.segment_coo(src.abs(), idx, segs, "sum")
    assert_sum_close(out, gold, scale, torch.float32, "coo batched")


def test_segment_coo_index_validation(ogn):
    # reference csrc/npu/segment_coo/op_host/segment_coo.cpp:97-100
    src = torch.ones(4, 2, device="cuda")
    with pytest.raises(RuntimeError, match="non-negative"):
        ogn.segment_sum_coo(src, torch.tensor([-1, 0, 0, 1], device="cuda"))
    with pytest.raises(RuntimeError, match="sorted"):
        ogn.segment_sum_coo(src, torch.tensor([0, 2, 1, 3], device="cuda"))
    with pytest.raises(RuntimeError, match="exceed"):
        ogn.segment_sum_coo(src, torch.tensor([0, 1, 2, 3], device="cuda"), dim_size=3)
    # each row of a batched index is sorted on its own (row ends may drop)
    s2 = torch.ones(2, 3, device="cuda")
    got = ogn.segment_sum_coo(s2, torch.tensor([[0, 1, 1], [0, 0, 2]], device="cuda"))
    assert got.cpu().tolist() == [[1.0, 2.0, 0.0], [2.0, 0.0, 1.0]]
    with pytest.raises(RuntimeError, match="sorted"):
        ogn.segment_sum_coo(s2, torch.tensor([[0, 1, 1], [2, 0, 2]], device="cuda"))
    # the cached facts follow in-place changes of the index
    idx = torch.tensor([0, 0, 1, 1], device="cuda")
    ogn.segment_sum_coo(src, idx)
    idx[1] = 5
    with pytest.raises(RuntimeError, match="sorted"):
        ogn.segment_sum_coo(src, idx)


# ----------------------------------------------------------------- segment_logsumexp
@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("feat", [1, 16, 128])
def test_segment_logsumexp_random(ogn, oracle, dtype, feat):
    rng = np.random.default_rng(31)
    lengths = _lengths(rng, 500, 12, long_every=101, long_len=5000)
    src = torch.from_numpy((rng.standard_normal((int(lengths.sum()), feat)) * 4).astype(np.float32)).to(dtype)
    indptr = torch.from_numpy(np.concatenate([[0], np.cumsum(lengths)]))
    out = ogn.segment_logsumexp(src.cuda(), indptr.cuda())
    gold = cast_like(oracle.segment_logsumexp(src, indptr), dtype)
    tol = LSE_TOL[dtype]
    np.testing.assert_allclose(out.float().cpu().numpy(), gold, rtol=tol, atol=tol)


def test_segment_logsumexp_special_values_and_out(ogn):
    src = torch.tensor([[-float("inf")], [-float("inf")], [float("inf")], [1.0], [float("nan")], [2.0]],
                       device="cuda")
    out = torch.empty(4, 1, device="cuda")
    res = ogn.segment_logsumexp(src, torch.tensor([0, 2, 4, 6, 6], device="cuda"), out=out)
    assert res is out
    v = out.cpu().flatten().tolist()
    assert v[0] == -float("inf") and v[1] == float("inf") and v[2] != v[2] and v[3] == -float("inf")


def test_segment_logsumexp_errors(ogn):
    src = torch.ones(4, 2, device="cuda")
    with pytest.raises(ValueError, match="non-negative"):
        ogn.segment_logsumexp(src, torch.tensor([-1, 4], device="cuda"))
    with pytest.raises(ValueError, match="nondecreasing"):
        ogn.segment_logsumexp(src, torch.tensor([0, 3, 2, 4], device="cuda"))
    with pytest.raises(ValueError, match="must equal"):
        ogn.segment_logsumexp(src, torch.tensor([0, 3], device="cuda"))
    with pytest.raises(TypeError):
        ogn.segment_logsumexp(src.double(), torch.tensor([0, 4], device="cuda"))


# ------------------------------------------------------------------ mixed short / hub rows
def _mixed_lengths(rng, segs, hub):
    """Config-5-like rows: mostly 1-3 positions (chunks of them take the
    short-row kernel), a few medium rows, and one hub row that spans many
    chunks (folded by the fix-up across its lane groups)."""
    lengths = np.minimum(rng.zipf(1.8, size=segs), 300)
    lengths[rng.integers(0, segs, segs // 20)] = 0
    lengths[segs // 3] = hub
    return lengths


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("reduce", REDUCES)
@pytest.mark.parametrize("feat", [1, 4, 32, 33, 128])
def test_segment_csr_short_rows_and_hub(ogn, oracle, dtype, reduce, feat):
    rng = np.random.default_rng(100 + feat)
    lengths = _mixed_lengths(rng, 4000, 60000 if feat <= 4 else 9000)
    src = torch.from_numpy(rng.standard_normal((int(lengths.sum()), feat)).astype(np.float32)).to(dtype)
    if reduce in ("min", "max"):
        src = torch.from_numpy(rng.integers(-3, 4, size=tuple(src.shape)).astype(np.float32)).to(dtype)  # ties
    indptr = torch.from_numpy(np.concatenate([[0], np.cumsum(lengths)]))
    _csr_check(ogn, oracle, src, indptr, reduce, f"mixed/{dtype}/{reduce}/f{feat}")


@pytest.mark.parametrize("reduce", REDUCES)
@pytest.mark.parametrize("with_out", [False, True])
@pytest.mark.parametrize("feat", [1, 32])
def test_segment_coo_short_rows_and_hub(ogn, oracle, reduce, with_out, feat):
    # later-tie rule and seeds on the short-row kernel and the grouped fix-up
    rng = np.random.default_rng(7 + feat)
    lengths = _mixed_lengths(rng, 3000, 40000)
    index = np.repeat(np.arange(3000), lengths)
    src = torch.from_numpy(rng.integers(-3, 4, size=(index.size, feat)).astype(np.float32))
    out = torch.from_numpy(rng.integers(-3, 4, size=(3000, feat)).astype(np.float32)) if with_out else None
    fn = getattr(ogn, f"segment_{reduce}_coo")
    res = fn(src.cuda(), torch.from_numpy(index).cuda(), None if out is None else out.clone().cuda(), 3000)
    got, arg = res if isinstance(res, tuple) else (res, None)
    gold, garg = oracle.segment_coo(src, index, 3000, reduce, None if out is None else out.double().numpy())
    if arg is not None:
        assert_exact(got, gold, "coo values")
        assert_exact(arg, garg, "coo arg")
    else:
        scale, _ = oracle.segment_coo(src.abs(), index, 3000, reduce,
                                      None if out is None else out.double().abs().numpy())
        assert_sum_close(got, gold, scale, torch.float32, "coo")


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("feat", [1, 32])
def test_segment_logsumexp_short_rows_and_hub(ogn, oracle, dtype, feat):
    rng = np.random.default_rng(9)
    lengths = _mixed_lengths(rng, 3000, 40000)
    src = torch.from_numpy((rng.standard_normal((int(lengths.sum()), feat)) * 3).astype(np.float32)).to(dtype)
    indptr = torch.from_numpy(np.concatenate([[0], np.cumsum(lengths)]))
    got = ogn.segment_logsumexp(src.cuda(), indptr.cuda())
    gold = oracle.segment_logsumexp(src, indptr)
    g = got.float().cpu().numpy()
    np.testing.assert_allclose(g, cast_like(gold, dtype), rtol=LSE_TOL[dtype], atol=LSE_TOL[dtype])
