"""GPU parity of the exact-dtype reductions (int8 / uint8 / int16 / int32 /
int64, float64 scatter) against the oracle: bit-exact everywhere except the
order-dependent float64 sums of the unsorted (atomic) scatter.

Cases follow the reference tests: segment_csr integer mean regressions
(test/segment_csr/arch35/test_segment_csr_golden.py), segment_coo byte mean
narrowing, integer mean extremes, later ties and out seeds
(test/segment_coo/arch35/test_segment_coo.py:486-826), scatter's integer floor
mean, documented dtypes and collapsed-index mean counts
(test/scatter/arch35/test_scatter.py:185-349).
"""

import numpy as np
import pytest
import torch

from test_oracle_exact import INTEGER_MEAN_COUNTS, integer_mean_extremes_case

pytestmark = pytest.mark.gpu

SEG_DTYPES = [torch.int8, torch.uint8, torch.int32, torch.int64]
SCAT_DTYPES = [torch.int8, torch.uint8, torch.int16, torch.int32, torch.int64]


def _rand(shape, dtype, rng, small=False):
    if dtype == torch.float64:
        return torch.from_numpy(rng.standard_normal(shape))
    info = torch.iinfo(dtype)
    lo, hi = (-5 if info.min < 0 else 0, 6) if small else (info.min, info.max)
    vals = rng.integers(lo, hi, shape, dtype=np.int64, endpoint=True)
    if dtype == torch.int64 and not small:
        vals = vals * 3 + 1  # exercise the high bits
    return torch.from_numpy(vals).to(dtype)


def _eq(got, want, what=""):
    want = torch.as_tensor(np.ascontiguousarray(want))
    got = got.cpu()
    assert got.shape == tuple(want.shape), what
    if got.dtype.is_floating_point:
        assert torch.equal(got, want.to(got.dtype)), what
    else:
        assert torch.equal(got, want.to(torch.int64).to(got.dtype)), what


def _powerlaw_ptr(rng, segs, empty=10):
    lengths = np.minimum(rng.zipf(1.7, segs), 700)
    lengths[rng.integers(0, segs, empty)] = 0
    return np.concatenate([[0], np.cumsum(lengths)])


# ------------------------------------------------------------------ segment_csr
@pytest.mark.parametrize("dtype", SEG_DTYPES)
@pytest.mark.parametrize("reduce", ["sum", "mean", "min", "max"])
@pytest.mark.parametrize("feat", [1, 3, 16, 48])
def test_segment_csr_random(ogn, oracle, dtype, reduce, feat):
    rng = np.random.default_rng(11)
    ptr = _powerlaw_ptr(rng, 400)
    src = _rand((int(ptr[-1]), feat), dtype, rng)
    got = ogn.segment_csr(src.cuda(), torch.from_numpy(ptr).cuda(), reduce=reduce)
    want, warg = oracle.segment_csr(src, ptr, reduce)
    _eq(got, want, f"{dtype} {reduce}")
    if reduce in ("min", "max"):
        fn = ogn.segment_min_csr if reduce == "min" else ogn.segment_max_csr
        v, a = fn(src.cuda(), torch.from_numpy(ptr).cuda())
        _eq(v, want)
        _eq(a, warg, "arg")


@pytest.mark.parametrize("dtype", SEG_DTYPES)
@pytest.mark.parametrize("reduce", ["sum", "mean", "min", "max"])
def test_segment_csr_batched_pointers(ogn, oracle, dtype, reduce):
    rng = np.random.default_rng(12)
    src = _rand((3, 90, 5, 4), dtype, rng)
    ptr = np.stack([np.sort(rng.integers(0, 91, 13)) for _ in range(3)])
    ptr[:, 0] = rng.integers(0, 3, 3)  # leading rows outside any segment
    got = ogn.segment_csr(src.cuda(), torch.from_numpy(ptr).cuda(), reduce=reduce)
    want, _ = oracle.segment_csr(src, ptr, reduce)
    _eq(got, want)
    shared = np.sort(rng.integers(0, 91, 9))
    got = ogn.segment_csr(src.cuda(), torch.from_numpy(shared).view(1, -1).cuda(), reduce=reduce)
    want, _ = oracle.segment_csr(src, shared.reshape(1, -1), reduce)
    _eq(got, want)


@pytest.mark.parametrize("value", [16_777_217, -16_777_217, 9_007_199_254_740_993, -9_007_199_254_740_993])
def test_segment_csr_int64_mean_exact(ogn, value):
    src = torch.tensor([value], dtype=torch.int64, device="cuda")
    assert ogn.segment_csr(src, torch.tensor([0, 1], device="cuda"), reduce="mean").cpu().tolist() == [value]


@pytest.mark.parametrize("dtype,count,expected", [(torch.int8, 200, -1), (torch.int8, 256, 0), (torch.uint8, 256, 0)])
def test_segment_csr_narrow_mean_kat(ogn, dtype, count, expected):
    src = torch.zeros(count, dtype=dtype)
    src[0] = 100
    got = ogn.segment_csr(src.cuda(), torch.tensor([0, count], device="cuda"), reduce="mean")
    assert got.cpu().tolist() == [expected]
    got = ogn.segment_csr(torch.tensor([100, 100], dtype=torch.int8, device="cuda"),
                          torch.tensor([0, 2], device="cuda"), reduce="mean")
    assert got.cpu().tolist() == [-28]
    got = ogn.segment_csr(torch.tensor([-1, -2], device="cuda"), torch.tensor([0, 2], device="cuda"), reduce="mean")
    assert got.cpu().tolist() == [-1]


@pytest.mark.parametrize("offset", [1, 3])
def test_segment_csr_unaligned_views(ogn, oracle, offset):
    # 16-byte packets need aligned rows; offset views take the scalar path
    rng = np.random.default_rng(13)
    ptr = _powerlaw_ptr(rng, 50, empty=3)
    base = _rand((int(ptr[-1]) * 16 + offset,), torch.int8, rng)
    src = base[offset:].view(-1, 16)
    dev = base.cuda()[offset:].view(-1, 16)
    assert dev.data_ptr() % 16 != 0
    got = ogn.segment_csr(dev, torch.from_numpy(ptr).cuda())
    want, _ = oracle.segment_csr(src, ptr, "sum")
    _eq(got, want)


# ------------------------------------------------------------------ segment_coo
@pytest.mark.parametrize("dtype", SEG_DTYPES)
@pytest.mark.parametrize("reduce", ["sum", "mean", "min", "max"])
@pytest.mark.parametrize("with_out", [False, True])
def test_segment_coo_random(ogn, oracle, dtype, reduce, with_out):
    rng = np.random.default_rng(21)
    src = _rand((2, 600, 32), dtype, rng)
    index = np.sort(rng.integers(0, 40, (2, 600)) * 2, axis=1)  # uneven segments with holes
    out = _rand((2, 80, 32), dtype, rng) if with_out else None
    fn = {"sum": ogn.segment_sum_coo, "mean": ogn.segment_mean_coo, "min": ogn.segment_min_coo,
          "max": ogn.segment_max_coo}[reduce]
    dev_out = None if out is None else out.clone().cuda()
    res = fn(src.cuda(), torch.from_numpy(index).cuda(), dev_out, 80)
    got, arg = res if isinstance(res, tuple) else (res, None)
    if dev_out is not None:
        assert got.data_ptr() == dev_out.data_ptr()
    want, warg = oracle.segment_coo(src, index, 80, reduce, out=out)
    _eq(got, want, f"{dtype} {reduce} {with_out}")
    if arg is not None:
        _eq(arg, warg, "arg")


@pytest.mark.parametrize("dtype", [torch.int32, torch.int64])
@pytest.mark.parametrize("channels", [1, 8, 32, 96, 128])
@pytest.mark.parametrize("with_out", [False, True])
def test_segment_coo_integer_mean_extremes(ogn, dtype, channels, with_out):
    npdt = np.int32 if dtype == torch.int32 else np.int64
    src, index, initial, expected = integer_mean_extremes_case(npdt, channels, with_out)
    out = None if initial is None else torch.from_numpy(initial).cuda()
    got = ogn.segment_mean_coo(torch.from_numpy(src).cuda(), torch.from_numpy(index).cuda(), out=out,
                               dim_size=len(INTEGER_MEAN_COUNTS))
    assert torch.equal(got.cpu(), torch.from_numpy(expected))


@pytest.mark.parametrize("dtype", [torch.int8, torch.uint8])
@pytest.mark.parametrize("channels", [1, 8, 32])
@pytest.mark.parametrize("kind", ["random", "positive", "boundary"])
def test_segment_coo_byte_mean_narrowing(ogn, oracle, dtype, channels, kind):
    counts = np.array([0, 1, 2, 7, 17, 31, 33, 127, 129, 257, 0])
    index = np.repeat(np.arange(len(counts)), counts)
    if kind == "boundary":
        src = torch.full((len(index), channels), torch.iinfo(dtype).max // 4, dtype=dtype)
    else:
        low = -5 if dtype == torch.int8 and kind == "random" else 0
        src = torch.randint(low, 6, (len(index), channels), dtype=dtype, generator=torch.Generator().manual_seed(923))
    got = ogn.segment_mean_coo(src.cuda(), torch.from_numpy(index).cuda(), dim_size=len(counts))
    want, _ = oracle.segment_coo(src, index, len(counts), "mean")
    _eq(got, want)
    # 256 equal entries: the narrowed count is 0 and the exact mean is kept
    got = ogn.segment_mean_coo(torch.full((256, channels), 3, dtype=dtype, device="cuda"),
                               torch.zeros(256, dtype=torch.int64, device="cuda"), dim_size=1)
    assert (got.cpu() == 3).all()


# ------------------------------------------------------------------ scatter
def _scatter(ogn, reduce, src, index, dim, out, size):
    fn = {"sum": ogn.scatter_sum, "mean": ogn.scatter_mean, "mul": ogn.scatter_mul,
          "min": ogn.scatter_min, "max": ogn.scatter_max}[reduce]
    res = fn(src, index, dim, out, size)
    return res if isinstance(res, tuple) else (res, None)


@pytest.mark.parametrize("dtype", SCAT_DTYPES + [torch.float64])
@pytest.mark.parametrize("reduce", ["sum", "mean", "mul", "min", "max"])
@pytest.mark.parametrize("sorted_index", [True, False])
@pytest.mark.parametrize("with_out", [False, True])
def test_scatter_compact_index(ogn, oracle, dtype, reduce, sorted_index, with_out):
    rng = np.random.default_rng(31)
    idx = rng.integers(0, 120, 3000)
    idx[:400] = 5  # hot target
    if sorted_index:
        idx = np.sort(idx)
    src = _rand((3000, 16), dtype, rng, small=reduce == "mul")
    out = _rand((130, 16), dtype, rng) if with_out else None
    dev_out = None if out is None else out.clone().cuda()
    got, arg = _scatter(ogn, reduce, src.cuda(), torch.from_numpy(idx).cuda(), 0, dev_out, 130)
    full = np.broadcast_to(idx.reshape(-1, 1), (3000, 16))
    want, warg = oracle.scatter(src, full, 0, 130, reduce, out)
    what = f"{dtype} {reduce} sorted={sorted_index} out={with_out}"
    if dtype == torch.float64 and reduce in ("sum", "mean", "mul") and not sorted_index:
        np.testing.assert_allclose(got.cpu().numpy(), want, rtol=1e-12, atol=1e-12, err_msg=what)
    else:
        _eq(got, want, what)
    if arg is not None:
        _eq(arg, warg, what + " arg")


@pytest.mark.parametrize("dtype", SCAT_DTYPES + [torch.float64])
@pytest.mark.parametrize("reduce", ["sum", "mean", "mul", "min", "max"])
def test_scatter_full_shape_index(ogn, oracle, dtype, reduce):
    rng = np.random.default_rng(32)
    src = _rand((3, 70, 5), dtype, rng, small=reduce == "mul")
    index = rng.integers(0, 9, (3, 70, 5))
    got, arg = _scatter(ogn, reduce, src.cuda(), torch.from_numpy(index).cuda(), -2, None, 9)
    want, warg = oracle.scatter(src, index, 1, 9, reduce)
    if dtype == torch.float64 and reduce in ("sum", "mean", "mul"):
        np.testing.assert_allclose(got.cpu().numpy(), want, rtol=1e-12, atol=1e-12)
    else:
        _eq(got, want)
    if arg is not None:
        _eq(arg, warg, "arg")


def test_scatter_integer_floor_mean_kat(ogn):
    # reference test/scatter/arch35/test_scatter.py:345-349
    src = torch.tensor([[-3, -2, 4], [-2, -1, 5]], dtype=torch.int32, device="cuda")
    got = ogn.scatter_mean(src, torch.tensor([0, 0, 1], device="cuda"), dim=-1)
    assert torch.equal(got.cpu(), torch.tensor([[-3, 4], [-2, 5]], dtype=torch.int32))
    # the unsorted (atomic) path gives the same
    got = ogn.scatter_mean(src, torch.tensor([0, 1, 0], device="cuda"), dim=-1)
    assert torch.equal(got.cpu(), torch.tensor([[0, -2], [1, -1]], dtype=torch.int32))  # floor(1/2), floor(3/2)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32, torch.float64, torch.int8,
                                   torch.int16, torch.int32, torch.int64, torch.uint8])
@pytest.mark.parametrize("reduce", ["sum", "add", "mul", "mean", "min", "max"])
def test_scatter_all_documented_dtypes(ogn, dtype, reduce):
    # reference test/scatter/arch35/test_scatter.py:333-342
    src = torch.tensor([1, 2, 3, 4], dtype=dtype, device="cuda")
    got = ogn.scatter(src, torch.tensor([0, 0, 1, 1], device="cuda"), dim=0, dim_size=3, reduce=reduce)
    assert got.dtype == dtype and got.shape == (3,)
    want = {"sum": [3, 7, 0], "add": [3, 7, 0], "mul": [2, 12, 1], "mean": [1, 3, 0], "min": [1, 3, 0],
            "max": [2, 4, 0]}[reduce]
    if reduce == "mean" and dtype.is_floating_point:
        want = [1.5, 3.5, 0]
    assert got.cpu().double().tolist() == want


@pytest.mark.parametrize("dtype", [torch.float32, torch.int32])
@pytest.mark.parametrize("reduce", ["sum", "mul", "mean", "min", "max"])
def test_scatter_collapsed_index_mean_counts(ogn, dtype, reduce):
    # reference test/scatter/arch35/test_scatter.py:185-237: the mean counts
    # over the index's own shape, so an index of extent 1 along dim gives the sum
    src = torch.tensor([[[1, 2], [3, 4], [5, 6]], [[7, 8], [9, 10], [11, 12]]], dtype=dtype, device="cuda")
    index = torch.tensor([[[0, 1]], [[1, 0]]], device="cuda")
    want = {"sum": [[[9, 0], [0, 12]], [[0, 30], [27, 0]]],
            "mul": [[[15, 1], [1, 48]], [[1, 960], [693, 1]]],
            "mean": [[[9, 0], [0, 12]], [[0, 30], [27, 0]]],
            "min": [[[1, 0], [0, 2]], [[0, 8], [7, 0]]],
            "max": [[[5, 0], [0, 6]], [[0, 12], [11, 0]]]}[reduce]
    got = ogn.scatter(src, index, dim=1, dim_size=2, reduce=reduce)
    assert torch.equal(got.cpu(), torch.tensor(want, dtype=dtype))
    if reduce == "mean":
        s = torch.tensor([[[1, 2, 3], [4, 5, 6]]], dtype=dtype, device="cuda")
        got = ogn.scatter_mean(s, torch.tensor([0], device="cuda"), dim=2)
        assert torch.equal(got.cpu(), torch.tensor([[[6], [15]]], dtype=dtype))


def test_scatter_int_wrap_kats(ogn):
    dev = "cuda"
    assert ogn.scatter_sum(torch.tensor([100, 100], dtype=torch.int8, device=dev),
                           torch.tensor([0, 0], device=dev)).cpu().tolist() == [-56]
    assert ogn.scatter_mul(torch.tensor([16, 16], dtype=torch.int8, device=dev),
                           torch.tensor([0, 0], device=dev)).cpu().tolist() == [0]
    assert ogn.scatter_mean(torch.ones(200, dtype=torch.int8, device=dev),
                            torch.zeros(200, dtype=torch.int64, device=dev)).cpu().tolist() == [-56]
    # unsorted: same exact result
    idx = torch.tensor([1, 0] * 100, device=dev)
    assert ogn.scatter_mean(torch.ones(200, dtype=torch.uint8, device=dev), idx).cpu().tolist() == [1, 1]


def test_scatter_f64_signed_zero_later_writer(ogn):
    # ties between -0.0 and +0.0: the later writer's value and position win,
    # on the sorted (segment) and the unsorted (atomic) path alike
    f64 = dict(dtype=torch.float64, device="cuda")
    v, a = ogn.scatter_min(torch.tensor([-0.0, 0.0, 3.0], **f64), torch.tensor([0, 0, 1], device="cuda"))
    assert a.cpu().tolist() == [1, 2] and str(v.cpu()[0].item()) == "0.0"
    v, a = ogn.scatter_min(torch.tensor([-0.0, 3.0, 0.0], **f64), torch.tensor([0, 1, 0], device="cuda"))
    assert a.cpu().tolist() == [2, 1] and str(v.cpu()[0].item()) == "0.0"
    v, a = ogn.scatter_max(torch.tensor([3.0, 0.0, -0.0], **f64), torch.tensor([1, 0, 0], device="cuda"))
    assert a.cpu().tolist() == [2, 0] and str(v.cpu()[0].item()) == "-0.0"


def test_unsupported_dtypes_raise(ogn):
    with pytest.raises(TypeError):
        ogn.segment_csr(torch.ones(3, dtype=torch.int16, device="cuda"), torch.tensor([0, 3], device="cuda"))
    with pytest.raises(TypeError):
        ogn.segment_csr(torch.ones(3, dtype=torch.float64, device="cuda"), torch.tensor([0, 3], device="cuda"))
    with pytest.raises(TypeError):
        ogn.scatter_sum(torch.ones(3, dtype=torch.bool, device="cuda"), torch.tensor([0, 1, 1], device="cuda"))
