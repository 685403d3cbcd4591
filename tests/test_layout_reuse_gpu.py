"""GPU tests of the kept chunk layout (OGN_SEG_KEEP_LAYOUT / OGN_SEG_REUSE_LAYOUT)
and the short-segment hint (OGN_SEG_SHORT_SEGMENTS) of ogn_segment_reduce.

A graph reduced many times keeps its engine workspace, whose chunk layout
(row of each chunk's first position, rows crossing chunk ends) is then not
recomputed.  Every case is checked against the oracle: repeated calls, an
indptr changed in place (new tensor version), two graphs alternating, a
plan change from a misaligned src view, and through the C ABI a REUSE call
whose workspace never held a layout and one whose recorded pointer differs.
Sums within rel 1e-5 (fp32); min/max values and args bit-exact.
"""

import numpy as np
import pytest
import torch

from _util import assert_exact, assert_sum_close

pytestmark = pytest.mark.gpu


def _graph(seed, segs=3000, mean=16, hub=0):
    rng = np.random.default_rng(seed)
    lengths = rng.poisson(mean, size=segs)
    lengths[::37] = 0
    if hub:
        lengths[segs // 2] = hub
    return torch.from_numpy(np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)), rng


def _check(ogn, oracle, src, indptr, reduce, what):
    res = getattr(ogn, f"segment_{reduce}_csr")(src, indptr)
    out, arg = res if isinstance(res, tuple) else (res, None)
    gold, garg = oracle.segment_csr(src.cpu(), indptr.cpu(), reduce)
    if arg is not None:
        assert_exact(out, gold, what + " values")
        assert_exact(arg, garg, what + " arg")
    else:
        scale, _ = oracle.segment_csr(src.cpu().abs(), indptr.cpu(), reduce)
        assert_sum_close(out, gold, scale, torch.float32, what)


@pytest.mark.parametrize("reduce", ["sum", "max"])
@pytest.mark.parametrize("hub", [0, 40_000])
def test_repeated_calls_and_inplace_change(ogn, oracle, reduce, hub):
    indptr, rng = _graph(1, hub=hub)
    e = int(indptr[-1])
    src = torch.from_numpy(rng.integers(-5, 6, (e, 64)).astype(np.float32)).cuda()
    ptr = indptr.cuda()
    for i in range(3):
        _check(ogn, oracle, src, ptr, reduce, f"repeat {i}")
    # move one boundary in place: same tensor, new version, new layout
    lengths = indptr.diff().numpy()
    j = int(np.nonzero(lengths[: len(lengths) // 2] >= 3)[0][-1]) + 1  # segment j - 1 keeps >= 0 rows
    ptr[j] -= 3
    assert bool((ptr[1:] >= ptr[:-1]).all())
    for i in range(2):
        _check(ogn, oracle, src, ptr, reduce, f"after change {i}")


def test_alternating_graphs_and_plan_change(ogn, oracle):
    pa, rng = _graph(2)
    pb, _ = _graph(3)
    pb = pb * int(pa[-1]) // int(pb[-1])  # same total length, other boundaries
    e = int(pa[-1])
    big = torch.from_numpy(rng.standard_normal((e + 1) * 32).astype(np.float32)).cuda()
    src = big[: e * 32].view(e, 32)
    mis = big[1: e * 32 + 1].view(e, 32)  # 4-byte offset: the scalar plan
    a, b = pa.cuda(), pb.cuda()
    for i in range(3):
        _check(ogn, oracle, src, a, "sum", f"a {i}")
        _check(ogn, oracle, src, b, "sum", f"b {i}")
        _check(ogn, oracle, mis, a, "sum", f"a misaligned {i}")
        _check(ogn, oracle, src, a, "mean", f"a mean {i}")


def test_logsumexp_and_scatter_repeat(ogn, oracle):
    indptr, rng = _graph(4, hub=30_000)
    e = int(indptr[-1])
    src = torch.from_numpy(rng.standard_normal((e, 32)).astype(np.float32)).cuda()
    ptr = indptr.cuda()
    gold = oracle.segment_logsumexp(src.cpu(), indptr)
    for _ in range(3):
        got = ogn.segment_logsumexp(src, ptr).cpu().numpy()
        np.testing.assert_allclose(got, gold, rtol=1e-5, atol=1e-5)
    index = torch.repeat_interleave(torch.arange(indptr.numel() - 1), indptr.diff()).cuda()
    g2, _ = oracle.scatter(src.cpu().numpy(), index.cpu().numpy()[:, None], 0, indptr.numel() - 1, "max")
    for _ in range(3):
        assert_exact(ogn.scatter(src, index, 0, dim_size=indptr.numel() - 1, reduce="max"), g2, "scatter max")


def _raw_call(ogn, src, ptr, out, ws, flags):
    from ops_gnn import _lib

    lib = _lib.lib
    e, k = src.shape
    segs = ptr.numel() - 1
    rc = lib.ogn_segment_reduce(_lib.dptr(ptr), 1, _lib.dptr(src), _lib.TORCH_TO_OGN[torch.float32], 1, e, segs, k, _lib.dptr(out),
                                None, _lib.R_SUM, _lib.SEM_SEGMENT_CSR, flags, _lib.dptr(ws), ws.numel(),
                                _lib.stream_of(src))
    _lib.check(rc, "segment_reduce")


def test_c_abi_reuse_without_keep_and_other_pointer(ogn, oracle):
    from ops_gnn import _lib

    pa, rng = _graph(5, hub=20_000)
    pb, _ = _graph(6, hub=20_000)
    pb = pb * int(pa[-1]) // int(pb[-1])
    e = int(pa[-1])
    src = torch.from_numpy(rng.standard_normal((e, 16)).astype(np.float32)).cuda()
    segs = pa.numel() - 1
    nbytes = _lib.lib.ogn_segment_reduce_workspace_size(1, e, segs, 16, 1, _lib.TORCH_TO_OGN[torch.float32], _lib.R_SUM)
    ws = torch.full((nbytes,), 0xAB, dtype=torch.uint8, device="cuda")  # garbage layout
    a, b = pa.cuda(), pb.cuda()
    for ptr, host, flags in [(a, pa, _lib.SEG_REUSE_LAYOUT),  # never kept: recomputed
                             (a, pa, _lib.SEG_REUSE_LAYOUT),  # kept now
                             (b, pb, _lib.SEG_REUSE_LAYOUT),  # other pointer: recomputed
                             (b, pb, _lib.SEG_KEEP_LAYOUT),
                             (a, pa, _lib.SEG_REUSE_LAYOUT)]:
        out = torch.empty((segs, 16), device="cuda")
        _raw_call(ogn, src, ptr, out, ws, flags)
        gold, _ = oracle.segment_csr(src.cpu(), host, "sum")
        scale, _ = oracle.segment_csr(src.cpu().abs(), host, "sum")
        assert_sum_close(out, gold, scale, torch.float32, f"raw flags {flags}")


def test_short_segments_hint_matches(ogn, oracle):
    # the hint only drops the pre-fold launch; results equal the plain call bit for bit
    from ops_gnn import _lib

    indptr, rng = _graph(7, segs=20_000)
    e = int(indptr[-1])
    src = torch.from_numpy(rng.standard_normal((e, 128)).astype(np.float32)).cuda()
    segs = indptr.numel() - 1
    nbytes = _lib.lib.ogn_segment_reduce_workspace_size(1, e, segs, 128, 1, _lib.TORCH_TO_OGN[torch.float32], _lib.R_SUM)
    ws = torch.empty((nbytes,), dtype=torch.uint8, device="cuda")
    ptr = indptr.cuda()
    o1 = torch.empty((segs, 128), device="cuda")
    o2 = torch.empty((segs, 128), device="cuda")
    _raw_call(ogn, src, ptr, o1, ws, 0)
    _raw_call(ogn, src, ptr, o2, ws, _lib.SEG_SHORT_SEGMENTS)
    assert torch.equal(o1, o2)
