"""GPU parity of the integer segment reductions on segments longer than the
4096-row threshold, which are folded in parallel pieces of 2048 positions
and then combined in position order.

Boundary cases: a long segment starting inside a piece and one starting
exactly on a piece boundary, a segment of exactly 4096 rows (serial) and
one of 4097 (pieces), two long segments meeting inside one piece, empty
and one-row segments between them, rows before the first segment, and
batched pointers.  Every result is bit-exact against the oracle (integer
sums and products wrap, extremum positions follow each operator's tie
rule), and the workspace-less call (serial fold of every segment) and the
short-segments hint give the same bits through the C ABI.
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DTYPES = [torch.int8, torch.uint8, torch.int32, torch.int64]
# start 3 | 9000 from offset 3 | empty | up to the piece boundary at 10240 |
# 4097 from the boundary | exactly 4096 | 5000 and 6000 meeting inside a piece |
# 1 | 20000 | 2
LENGTHS = np.array([3, 9000, 0, 1237, 4097, 4096, 5000, 6000, 1, 20000, 2], dtype=np.int64)


def _rand(shape, dtype, rng, small):
    info = torch.iinfo(dtype)
    lo, hi = (-3 if info.min < 0 else 0, 3) if small else (info.min, info.max)
    vals = rng.integers(lo, hi, shape, dtype=np.int64, endpoint=True)
    return torch.from_numpy(vals).to(dtype)


def _eq(got, want, what=""):
    want = torch.as_tensor(np.ascontiguousarray(want))
    got = got.cpu()
    assert got.shape == tuple(want.shape), what
    assert torch.equal(got, want.to(torch.int64).to(got.dtype)), what


def _ptr(lengths, lead=0):
    return np.concatenate([[lead], lead + np.cumsum(lengths)])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("reduce", ["sum", "mean", "min", "max"])
@pytest.mark.parametrize("feat", [1, 3, 16])
def test_segment_csr_long_integer_segments(ogn, oracle, dtype, reduce, feat):
    rng = np.random.default_rng(feat)
    ptr = _ptr(LENGTHS)
    # few distinct values for min / max: many ties, so the first-wins rule matters
    src = _rand((int(ptr[-1]), feat), dtype, rng, small=reduce in ("min", "max"))
    want, warg = oracle.segment_csr(src, ptr, reduce)
    if reduce in ("min", "max"):
        fn = ogn.segment_min_csr if reduce == "min" else ogn.segment_max_csr
        v, a = fn(src.cuda(), torch.from_numpy(ptr).cuda())
        _eq(v, want, f"{dtype} {reduce} values")
        _eq(a, warg, f"{dtype} {reduce} arg")
    else:
        got = ogn.segment_csr(src.cuda(), torch.from_numpy(ptr).cuda(), reduce=reduce)
        _eq(got, want, f"{dtype} {reduce}")


@pytest.mark.parametrize("dtype", [torch.int8, torch.int32, torch.int64])
@pytest.mark.parametrize("reduce", ["sum", "mean", "min", "max"])
@pytest.mark.parametrize("with_out", [False, True])
def test_segment_coo_long_integer_segments(ogn, oracle, dtype, reduce, with_out):
    # last-wins ties, out seeds
    rng = np.random.default_rng(7)
    m = LENGTHS.size
    index = np.repeat(np.arange(m), LENGTHS)
    src = _rand((index.size, 8), dtype, rng, small=reduce in ("min", "max"))
    out = _rand((m, 8), dtype, rng, small=True) if with_out else None
    fn = {"sum": ogn.segment_sum_coo, "mean": ogn.segment_mean_coo, "min": ogn.segment_min_coo,
          "max": ogn.segment_max_coo}[reduce]
    res = fn(src.cuda(), torch.from_numpy(index).cuda(), None if out is None else out.clone().cuda(), m)
    got, arg = res if isinstance(res, tuple) else (res, None)
    want, warg = oracle.segment_coo(src, index, m, reduce, out=out)
    _eq(got, want, f"{dtype} {reduce} out={with_out}")
    if arg is not None:
        _eq(arg, warg, "arg")


@pytest.mark.parametrize("dtype", [torch.uint8, torch.int16, torch.int32, torch.int64])
@pytest.mark.parametrize("reduce", ["sum", "mean", "mul", "min", "max"])
def test_scatter_sorted_long_integer_segments(ogn, oracle, dtype, reduce):
    rng = np.random.default_rng(9)
    m = LENGTHS.size
    idx = np.repeat(np.arange(m), LENGTHS)
    src = _rand((idx.size, 4), dtype, rng, small=reduce in ("mul", "min", "max"))
    out = _rand((m + 2, 4), dtype, rng, small=True)
    fn = {"sum": ogn.scatter_sum, "mean": ogn.scatter_mean, "mul": ogn.scatter_mul,
          "min": ogn.scatter_min, "max": ogn.scatter_max}[reduce]
    res = fn(src.cuda(), torch.from_numpy(idx).cuda(), 0, out.clone().cuda(), m + 2)
    got, arg = res if isinstance(res, tuple) else (res, None)
    full = np.broadcast_to(idx.reshape(-1, 1), src.shape)
    want, warg = oracle.scatter(src, full, 0, m + 2, reduce, out)
    _eq(got, want, f"{dtype} {reduce}")
    if arg is not None:
        _eq(arg, warg, "arg")


@pytest.mark.parametrize("reduce", ["sum", "max"])
def test_segment_csr_long_batched_pointers(ogn, oracle, reduce):
    # batch 1 has its long segments elsewhere and rows before its first segment
    rng = np.random.default_rng(13)
    l0 = LENGTHS
    l1 = np.concatenate([l0[::-1][:-1], [0]])
    n = int(l0.sum())
    ptr = np.stack([_ptr(l0), _ptr(l1, lead=n - int(l1.sum()))])
    src = _rand((2, n, 4), torch.int32, rng, small=reduce == "max")
    got = ogn.segment_csr(src.cuda(), torch.from_numpy(ptr).cuda(), reduce=reduce)
    for b in range(2):
        want, _ = oracle.segment_csr(src[b], ptr[b], reduce)
        _eq(got[b], want, f"batch {b}")


@pytest.mark.parametrize("reduce", ["sum", "min"])
def test_c_abi_pieces_equal_serial(ogn, reduce):
    # pieces (full workspace), serial (no workspace) and the short-segments
    # hint (serial) give the same bits
    from ops_gnn import _lib

    lib = _lib.lib
    rng = np.random.default_rng(17)
    ptr = torch.from_numpy(_ptr(LENGTHS)).cuda()
    e, k = int(LENGTHS.sum()), 16
    src = _rand((e, k), torch.int32, rng, small=reduce == "min").cuda()
    code = _lib.TORCH_TO_OGN[torch.int32]
    red = _lib.R_SUM if reduce == "sum" else _lib.R_MIN
    segs = LENGTHS.size
    nbytes = lib.ogn_segment_reduce_workspace_size(1, e, segs, k, 1, code, red)
    assert nbytes > 0
    ws = torch.full((nbytes,), 0x5A, dtype=torch.uint8, device="cuda")
    outs = []
    for wsp, wsb, flags in [(ws, nbytes, 0), (None, 0, 0), (ws, nbytes, _lib.SEG_SHORT_SEGMENTS)]:
        out = torch.empty((segs, k), dtype=torch.int32, device="cuda")
        arg = torch.empty((segs, k), dtype=torch.int64, device="cuda") if reduce == "min" else None
        rc = lib.ogn_segment_reduce(_lib.dptr(ptr), 1, _lib.dptr(src), code, 1, e, segs, k, _lib.dptr(out),
                                    _lib.dptr(arg), red, _lib.SEM_SEGMENT_CSR, flags,
                                    None if wsp is None else _lib.dptr(wsp), wsb, _lib.stream_of(src))
        _lib.check(rc, "segment_reduce")
        outs.append((out, arg))
    for out, arg in outs[1:]:
        assert torch.equal(out, outs[0][0])
        if arg is not None:
            assert torch.equal(arg, outs[0][1])
