"""GPU parity of gather_csr / gather_coo against the CPU oracle (bit-exact).

Cases follow the reference's tests (test/gather_csr/arch35/test_gather_csr.py,
test/gather_coo/arch35/test_gather_coo.py): the official table, every dtype,
NaN payloads, feature tails, ranks 1..8, broadcast pointers, empty segments,
an uncovered prefix, `out` (identity, aliasing), and the error contract.
"""

import numpy as np
import pytest
import torch

from test_oracle import GATHER_CASES

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.bfloat16, torch.float32, torch.float64, torch.int8, torch.int16, torch.int32,
          torch.int64, torch.uint8]


def _bits(t):
    t = t.detach().cpu().contiguous()
    return t.view(torch.uint8).reshape(-1)


def _assert_bitwise(actual, expected):
    assert actual.shape == expected.shape and actual.dtype == expected.dtype
    assert torch.equal(_bits(actual), _bits(expected))


def _make_src(shape, dtype, seed=0):
    g = torch.Generator().manual_seed(seed)
    if dtype.is_floating_point:
        return torch.randn(shape, generator=g).to(dtype)
    return (torch.arange(int(np.prod(shape))) % 127).reshape(shape).to(dtype)


@pytest.mark.parametrize("case", range(len(GATHER_CASES)))
@pytest.mark.parametrize("dtype", DTYPES)
def test_official_cases(ogn, case, dtype):
    src, coo, ptr, expected = GATHER_CASES[case]
    s = torch.tensor(src).to(dtype).cuda()
    want = torch.tensor(expected).to(dtype)
    _assert_bitwise(ogn.gather_csr(s, torch.tensor(ptr).cuda()), want)
    _assert_bitwise(ogn.gather_coo(s, torch.tensor(coo).cuda()), want)


@pytest.mark.parametrize("feat", [1, 3, 7, 31, 33, 127, 129, 4097])
def test_feature_tail_and_tiles(ogn, oracle, feat):
    src = torch.arange(4 * feat, dtype=torch.float32).reshape(4, feat)
    ptr = np.array([0, 1, 4, 4, 7])
    _assert_bitwise(ogn.gather_csr(src.cuda(), torch.from_numpy(ptr).cuda()), oracle.gather_csr(src, ptr))


@pytest.mark.parametrize("dtype", DTYPES)
def test_random_power_law(ogn, oracle, dtype):
    rng = np.random.default_rng(70)
    lengths = np.minimum(rng.zipf(1.8, 3000), 5000)
    lengths[rng.integers(0, 3000, 30)] = 0
    ptr = np.concatenate([[0], np.cumsum(lengths)])
    src = _make_src((3000, 24), dtype)
    _assert_bitwise(ogn.gather_csr(src.cuda(), torch.from_numpy(ptr).cuda()), oracle.gather_csr(src, ptr))
    idx = np.sort(rng.integers(0, 3000, 20000))
    _assert_bitwise(ogn.gather_coo(src.cuda(), torch.from_numpy(idx).cuda()), oracle.gather_coo(src, idx))


def test_nan_payload_preserved(ogn):
    raw = torch.tensor([0x7FF8000000000123, 0x7FF0000000000001, -1], dtype=torch.int64)
    src = raw.view(torch.float64)
    got = ogn.gather_csr(src.cuda(), torch.tensor([0, 2, 3, 5]).cuda())
    assert torch.equal(got.cpu().view(torch.int64), raw[[0, 0, 1, 2, 2]])
    got = ogn.gather_coo(src.cuda(), torch.tensor([2, 1, 0]).cuda())
    assert torch.equal(got.cpu().view(torch.int64), raw[[2, 1, 0]])


@pytest.mark.parametrize("rank", range(1, 9))
def test_rank_1_to_8(ogn, oracle, rank):
    shape = [2] * (rank - 1) + [3]
    src = _make_src(shape, torch.float32, rank)
    dim = rank - 1 if rank > 1 else 0
    width = shape[dim] + 1
    ptr = torch.tensor([0, 2, 2, 5][:width]).expand(*shape[:dim], width).contiguous()
    _assert_bitwise(ogn.gather_csr(src.cuda(), ptr.cuda()), oracle.gather_csr(src, ptr.numpy()))


def test_broadcast_and_batched_indptr(ogn, oracle):
    src = _make_src((3, 4, 5), torch.float32)
    shared = torch.tensor([[0, 1, 1, 3, 6]])
    _assert_bitwise(ogn.gather_csr(src.cuda(), shared.cuda()), oracle.gather_csr(src, shared.numpy()))
    per = torch.tensor([[0, 1, 1, 3, 6], [0, 0, 0, 6, 6], [1, 2, 3, 4, 6]])
    _assert_bitwise(ogn.gather_csr(src.cuda(), per.cuda()), oracle.gather_csr(src, per.numpy()))
    src4 = _make_src((2, 3, 4, 2), torch.float16)
    mid = torch.tensor([[0, 2, 2, 3, 3], [0, 0, 1, 2, 3], [0, 1, 1, 1, 3]]).reshape(1, 3, 5)
    want = oracle.gather_csr(src4, np.broadcast_to(mid.numpy(), (2, 3, 5)))
    _assert_bitwise(ogn.gather_csr(src4.cuda(), mid.cuda()), want)


@pytest.mark.parametrize("ptr", [[0, 0, 0, 0, 0], [0, 2, 2, 2, 5], [0, 0, 3, 3, 3]])
def test_empty_segments(ogn, oracle, ptr):
    src = torch.arange(12, dtype=torch.float32).reshape(4, 3)
    _assert_bitwise(ogn.gather_csr(src.cuda(), torch.tensor(ptr).cuda()), oracle.gather_csr(src, np.array(ptr)))


def test_uncovered_prefix_zeroed(ogn):
    got = ogn.gather_csr(torch.tensor([3, 5], dtype=torch.int32).cuda(), torch.tensor([2, 4, 6]).cuda())
    assert torch.equal(got.cpu(), torch.tensor([0, 0, 3, 3, 5, 5], dtype=torch.int32))
    out = torch.full((2,), 7, dtype=torch.int32, device="cuda")
    res = ogn.gather_csr(torch.empty(0, dtype=torch.int32, device="cuda"), torch.tensor([2]).cuda(), out)
    assert res.data_ptr() == out.data_ptr() and bool((out == 0).all())


def test_out_identity_and_alias_snapshot(ogn):
    src = torch.tensor([4, 3, 2, 1], dtype=torch.int32, device="cuda")
    ptr = torch.tensor([0, 2, 2, 3, 4], device="cuda")
    out = torch.empty(4, dtype=torch.int32, device="cuda")
    v0 = out._version
    res = ogn.gather_csr(src, ptr, out)
    assert res.data_ptr() == out.data_ptr() and out._version > v0
    assert torch.equal(out.cpu(), torch.tensor([4, 4, 2, 1], dtype=torch.int32))
    res = ogn.gather_csr(src, ptr, src)  # out aliases src: reads a snapshot
    assert res.data_ptr() == src.data_ptr()
    assert torch.equal(src.cpu(), torch.tensor([4, 4, 2, 1], dtype=torch.int32))
    s2 = torch.arange(6, dtype=torch.float32, device="cuda").reshape(3, 2)
    o2 = torch.empty(2, 3, device="cuda").t()  # non-contiguous out
    ogn.gather_coo(s2, torch.tensor([2, 0, 0], device="cuda"), o2)
    assert torch.equal(o2.cpu(), torch.tensor([[4.0, 5.0], [0.0, 1.0], [0.0, 1.0]]))


def test_deterministic_and_stream(ogn):
    src = torch.randn(5000, 40, device="cuda")
    lengths = torch.randint(0, 9, (5000,))
    ptr = torch.cat([torch.zeros(1, dtype=torch.long), lengths.cumsum(0)]).cuda()
    a = ogn.gather_csr(src, ptr)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        b = ogn.gather_csr(src, ptr)
    s.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("src,indptr,error", [
    (torch.ones(2), torch.tensor([0, 1, 2], dtype=torch.int32), "dtype must be int64"),
    (torch.ones(3), torch.tensor([0, 2, 1, 3]), "non-decreasing"),
    (torch.ones(2), torch.tensor([0, -1, 2]), "out of range"),
    (torch.ones(2), torch.tensor([0, 4, 3]), "out of range"),
    (torch.ones(3), torch.tensor([0, 1, 2]), "must equal"),
])
def test_invalid_indptr(ogn, src, indptr, error):
    # reference test/gather_csr/arch35/test_gather_csr.py:409-423
    with pytest.raises(RuntimeError, match=error):
        ogn.gather_csr(src.cuda(), indptr.cuda())


def test_validation_contract(ogn):
    src = torch.ones((2, 3), device="cuda")
    ptr = torch.tensor([0, 1, 2], device="cuda")
    with pytest.raises(RuntimeError, match="same endpoint"):
        ogn.gather_csr(torch.ones((2, 2), device="cuda"), torch.tensor([[0, 1, 2], [0, 1, 3]], device="cuda"))
    with pytest.raises(RuntimeError, match="out byte span overflows"):
        ogn.gather_csr(torch.ones((2, 8), device="cuda"), torch.tensor([0, 1, 2 ** 63 - 1], device="cuda"))
    with pytest.raises(RuntimeError, match="out dtype"):
        ogn.gather_csr(src, ptr, torch.empty((2, 3), dtype=torch.float16, device="cuda"))
    with pytest.raises(RuntimeError, match="out.size"):
        ogn.gather_csr(src, ptr, torch.empty((3, 3), device="cuda"))
    with pytest.raises(RuntimeError, match="out rank"):
        ogn.gather_csr(src, ptr, torch.empty((2, 3, 1), device="cuda"))
    with pytest.raises(RuntimeError, match="outside dimension"):
        ogn.gather_csr(src, ptr, torch.empty((2, 4), device="cuda"))
    with pytest.raises(RuntimeError, match="GPU tensor"):
        ogn.gather_csr(src, ptr, torch.empty((2, 3)))
    with pytest.raises(RuntimeError, match="unsupported src dtype"):
        ogn.gather_csr(torch.ones(2, dtype=torch.bool, device="cuda"), ptr)
    with pytest.raises(RuntimeError, match="cannot broadcast"):
        ogn.gather_csr(torch.ones((2, 2), device="cuda"), torch.ones((3, 3), dtype=torch.int64, device="cuda"))
    with pytest.raises(RuntimeError, match="indptr rank"):
        ogn.gather_csr(torch.ones((2, 2), device="cuda"), torch.zeros((1, 1, 3), dtype=torch.int64, device="cuda"))
    s3 = torch.ones((2, 5, 3), device="cuda")
    good = torch.zeros((2, 4), dtype=torch.int64, device="cuda")
    with pytest.raises(RuntimeError, match="int64"):
        ogn.gather_coo(s3, good.to(torch.int32))
    with pytest.raises(RuntimeError, match="prefix shapes"):
        ogn.gather_coo(s3, torch.zeros((3, 4), dtype=torch.int64, device="cuda"))
    with pytest.raises(RuntimeError, match="shape mismatch"):
        ogn.gather_coo(s3, good, out=torch.empty((2, 3, 3), device="cuda"))
    with pytest.raises(RuntimeError, match="zero rows"):
        ogn.gather_coo(torch.empty((2, 0, 3), device="cuda"), torch.zeros((2, 1), dtype=torch.int64, device="cuda"))


def test_empty_shapes(ogn):
    out = ogn.gather_csr(torch.randn(0, 0, 0, 16, device="cuda"), torch.tensor([], dtype=torch.int64, device="cuda"))
    assert out.shape == (0, 0, 0, 16)
    out = ogn.gather_csr(torch.empty((2, 0), device="cuda"), torch.tensor([0, 1, 3], device="cuda"))
    assert out.shape == (3, 0)
    out = ogn.gather_coo(torch.randn(3, 4, device="cuda"), torch.empty(0, dtype=torch.int64, device="cuda"))
    assert out.shape == (0, 4)


def test_gather_csr_long_empty_segment_runs(ogn, oracle):
    # a 64-row tile stages up to 128 pointer entries in LDS; a run of 5000
    # empty segments inside one tile takes the global search instead
    lengths = np.array([3] * 40 + [0] * 5000 + [7] * 30 + [0] * 200 + [1] * 500)
    ptr = np.concatenate([[0], np.cumsum(lengths)])
    src = _make_src((lengths.size, 6), torch.float32, 5)
    _assert_bitwise(ogn.gather_csr(src.cuda(), torch.from_numpy(ptr).cuda()), oracle.gather_csr(src, ptr))
