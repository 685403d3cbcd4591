"""GPU parity of the scatter family and the grouped softmax family against the
oracle.  Both execution paths are covered: a sorted 1-D index (segment
engine) and unsorted / full-shape indices (atomic kernels).  Cases follow the
reference tests (test/scatter/arch35/test_scatter.py,
test/scatter_softmax/*, test/scatter_log_softmax/*, test/scatter_logsumexp/*).
"""

import numpy as np
import pytest
import torch

from _util import assert_exact, assert_sum_close, cast_like

pytestmark = pytest.mark.gpu

DT = [torch.float32, torch.float16, torch.bfloat16]
SOFT_TOL = {torch.float32: 1e-5, torch.float16: 1e-2, torch.bfloat16: 1e-2}
INF, NAN = float("inf"), float("nan")


def test_later_writer_tie_kat(ogn):
    # reference test/scatter/arch35/test_scatter.py:322-331
    src = torch.tensor([4.0, 2.0, 2.0, 5.0, 5.0], device="cuda")
    index = torch.tensor([0, 0, 0, 1, 1], device="cuda")
    min_out, arg_min = ogn.scatter_min(src, index)
    max_out, arg_max = ogn.scatter_max(src, index)
    assert torch.equal(min_out.cpu(), torch.tensor([2.0, 5.0]))
    assert torch.equal(max_out.cpu(), torch.tensor([4.0, 5.0]))
    assert torch.equal(arg_min.cpu(), torch.tensor([2, 4]))
    assert torch.equal(arg_max.cpu(), torch.tensor([0, 4]))
    # same data, unsorted order -> atomic path
    perm = torch.tensor([3, 0, 4, 1, 2], device="cuda")
    v, a = ogn.scatter_min(src[perm], index[perm])
    assert torch.equal(v.cpu(), torch.tensor([2.0, 5.0])) and torch.equal(a.cpu(), torch.tensor([4, 2]))


def test_docs_example(ogn):
    # reference docs/en/api_reference.md:1032-1048
    src = torch.tensor([1.0, 2.0, 3.0, 4.0], device="cuda")
    index = torch.tensor([0, 1, 0, 1], device="cuda")
    assert torch.equal(ogn.scatter_sum(src, index).cpu(), torch.tensor([4.0, 6.0]))
    values, arg = ogn.scatter_max(src, index)
    assert torch.equal(values.cpu(), torch.tensor([3.0, 4.0])) and torch.equal(arg.cpu(), torch.tensor([2, 3]))


def _check(ogn, oracle, src, index, dim, size, reduce, out=None, what=""):
    fn = {"sum": ogn.scatter_sum, "mean": ogn.scatter_mean, "mul": ogn.scatter_mul,
          "min": ogn.scatter_min, "max": ogn.scatter_max}[reduce]
    dev_out = None if out is None else out.clone().cuda()
    res = fn(src.cuda(), index.cuda(), dim, dev_out, size)
    got, arg = res if isinstance(res, tuple) else (res, None)
    if dev_out is not None:
        assert got.data_ptr() == dev_out.data_ptr()
    d = dim % src.dim()
    from ops_gnn.scatter import broadcast
    idx_b = broadcast(index, src, d)
    name = {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16"}[src.dtype]
    gold, garg = oracle.scatter(src, idx_b, d, size, reduce, None if out is None else out.double().numpy(), name)
    if reduce in ("min", "max"):
        assert_exact(got, cast_like(gold, src.dtype), what + " values")
        assert_exact(arg, garg, what + " arg")
    elif reduce == "mul":
        np.testing.assert_allclose(got.float().cpu().numpy(), cast_like(gold, src.dtype), rtol=2e-2 if src.dtype != torch.float32 else 1e-3, atol=1e-6)
    else:
        sc, _ = oracle.scatter(src.float().abs(), idx_b, d, size, reduce,
                               None if out is None else out.double().abs().numpy(), name)
        assert_sum_close(got, gold, sc, src.dtype, what)


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("reduce", ["sum", "mean", "min", "max", "mul"])
@pytest.mark.parametrize("sorted_index", [True, False])
def test_compact_index(ogn, oracle, dtype, reduce, sorted_index):
    rng = np.random.default_rng(41)
    idx = rng.integers(0, 300, 5000)
    idx[:1500] = 7  # hot target
    if sorted_index:
        idx = np.sort(idx)
    src_np = rng.integers(-3, 4, size=(5000, 16)).astype(np.float32)
    if reduce == "mul":
        src_np = rng.uniform(0.9, 1.1, size=(5000, 16)).astype(np.float32)
    src = torch.from_numpy(src_np).to(dtype)
    _check(ogn, oracle, src, torch.from_numpy(idx), 0, 310, reduce, what=f"{reduce}/{sorted_index}")


@pytest.mark.parametrize("reduce", ["sum", "mean", "min", "max"])
@pytest.mark.parametrize("sorted_index", [True, False])
def test_out_is_accumulated(ogn, oracle, reduce, sorted_index):
    rng = np.random.default_rng(42)
    idx = rng.integers(0, 50, 800)
    if sorted_index:
        idx = np.sort(idx)
    src = torch.from_numpy(rng.standard_normal((800, 8)).astype(np.float32))
    out = torch.from_numpy(rng.standard_normal((60, 8)).astype(np.float32))
    _check(ogn, oracle, src, torch.from_numpy(idx), 0, 60, reduce, out=out, what=f"out/{reduce}")


@pytest.mark.parametrize("reduce", ["sum", "mean", "min", "max"])
def test_full_shape_index_and_negative_dim(ogn, oracle, reduce):
    rng = np.random.default_rng(43)
    src = torch.from_numpy(rng.standard_normal((3, 40, 6)).astype(np.float32))
    index = torch.from_numpy(rng.integers(0, 9, size=(3, 40, 6)))
    _check(ogn, oracle, src, index, -2, 9, reduce, what="full")
    # 1-D index along the last dim
    idx1 = torch.from_numpy(rng.integers(0, 4, size=6))
    _check(ogn, oracle, src, idx1, -1, 4, reduce, what="last dim")


@pytest.mark.parametrize("reduce", ["sum", "mean", "min", "max"])
@pytest.mark.parametrize("sorted_index", [True, False])
def test_broadcast_view_index_matches_oracle(ogn, oracle, reduce, sorted_index):
    # torch_scatter's usual call: index.view(-1, 1).expand_as(src) -- a
    # stride-0 view on the GPU, which takes the 1-D path (segment engine
    # when sorted) and must give the oracle's result
    rng = np.random.default_rng(64)
    idx = rng.integers(0, 50, 700)
    if sorted_index:
        idx = np.sort(idx)
    src = torch.from_numpy(rng.standard_normal((700, 6)).astype(np.float32))
    fn = {"sum": ogn.scatter_sum, "mean": ogn.scatter_mean, "min": ogn.scatter_min, "max": ogn.scatter_max}[reduce]
    dsrc = src.cuda()
    view = torch.from_numpy(idx).cuda().view(-1, 1).expand_as(dsrc)
    assert view.stride(1) == 0
    res = fn(dsrc, view, 0, None, 50)
    got, arg = res if isinstance(res, tuple) else (res, None)
    full = torch.from_numpy(idx).view(-1, 1).expand(700, 6).contiguous()
    gold, garg = oracle.scatter(src, full, 0, 50, reduce)
    if reduce in ("min", "max"):
        assert_exact(got, cast_like(gold, src.dtype), "broadcast view values")
        assert_exact(arg, garg, "broadcast view arg")
    else:
        scale, _ = oracle.scatter(src.abs(), full, 0, 50, "sum")
        if reduce == "mean":
            cnt, _ = oracle.scatter(torch.ones_like(src), full, 0, 50, "sum")
            scale = scale / np.maximum(cnt, 1)
        assert_sum_close(got, gold, scale, src.dtype, "broadcast view")


def test_scatter_dim_size_inference_and_empty(ogn):
    src = torch.randn(5, 3, device="cuda")
    out = ogn.scatter(src, torch.tensor([0, 4, 4, 1, 0], device="cuda"), dim=0)
    assert out.shape == (5, 3)
    empty = ogn.scatter(torch.empty(0, 3, device="cuda"), torch.empty(0, dtype=torch.long, device="cuda"), 0,
                        dim_size=4)
    assert empty.shape == (4, 3) and bool((empty == 0).all())
    with pytest.raises(ValueError):
        ogn.scatter(src, torch.zeros(5, dtype=torch.long, device="cuda"), reduce="median")
    with pytest.raises(TypeError):
        ogn.scatter(src, torch.zeros(5, dtype=torch.int32, device="cuda"))


# ----------------------------------------------------------------- grouped softmax family
def _softmax_check(ogn, oracle, src, index, dim, groups, mode, tol):
    fn = {"softmax": ogn.scatter_softmax, "log_softmax": ogn.scatter_log_softmax,
          "logsumexp": ogn.scatter_logsumexp}[mode]
    got = fn(src.cuda(), index.cuda(), dim, groups)
    gold = cast_like(oracle.group_softmax(src, index.long(), dim, groups, mode), src.dtype)
    g = got.float().cpu().numpy()
    np.testing.assert_array_equal(np.isnan(g), np.isnan(gold))
    np.testing.assert_allclose(g, gold, rtol=tol, atol=tol, equal_nan=True)


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("mode", ["softmax", "log_softmax", "logsumexp"])
@pytest.mark.parametrize("sorted_index", [True, False])
@pytest.mark.parametrize("index_dtype", [torch.int64, torch.int32])
def test_grouped_softmax(ogn, oracle, dtype, mode, sorted_index, index_dtype):
    rng = np.random.default_rng(51)
    idx = rng.integers(0, 64, 3000)
    idx[idx == 9] = 10  # an empty group
    if sorted_index:
        idx = np.sort(idx)
    src = torch.from_numpy((rng.standard_normal((2, 3000, 5)) * 6).astype(np.float32)).to(dtype)
    _softmax_check(ogn, oracle, src, torch.from_numpy(idx).to(index_dtype), 1, 64, mode, SOFT_TOL[dtype])


@pytest.mark.parametrize("mode", ["softmax", "log_softmax", "logsumexp"])
def test_grouped_softmax_edge_rows(ogn, oracle, mode):
    # GAT layout: one score per edge, grouped by destination row
    rng = np.random.default_rng(52)
    deg = rng.poisson(40, size=500)
    deg[::50] = 4000
    idx = np.repeat(np.arange(500), deg)
    src = torch.from_numpy((rng.standard_normal(idx.size) * 3).astype(np.float32))
    _softmax_check(ogn, oracle, src, torch.from_numpy(idx), 0, 500, mode, 1e-5)


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("mode", ["softmax", "log_softmax", "logsumexp"])
@pytest.mark.parametrize("before", [1, 2])
@pytest.mark.parametrize("mean_len", [90, 300, 1200])
def test_grouped_softmax_long_edge_rows(ogn, oracle, dtype, mode, before, mean_len):
    # one score per edge, rows averaging >= 128 edges (the GAT regime of
    # config 4): the row-per-wavefront statistics kernel; rows start at
    # arbitrary (unaligned) positions, some are empty, some hold +-inf / NaN
    rng = np.random.default_rng(53)
    deg = np.maximum(rng.lognormal(np.log(mean_len) - 0.5, 1.0, 300).astype(np.int64), 1)
    deg[[3, 77, 150]] = 0
    deg[10] = 30 * mean_len
    idx = np.repeat(np.arange(300), deg)
    x = (rng.standard_normal((before, idx.size)) * 4).astype(np.float32)
    starts = np.concatenate([[0], np.cumsum(deg)])
    x[0, starts[20] + 5] = INF
    x[0, starts[21]:starts[22]] = -INF
    x[-1, starts[30] + 1] = NAN
    src = torch.from_numpy(x).to(dtype)
    _softmax_check(ogn, oracle, src, torch.from_numpy(idx), 1, 300, mode, SOFT_TOL[dtype])


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("mode", ["softmax", "log_softmax"])
def test_grouped_softmax_register_row_sizes(ogn, oracle, dtype, mode):
    # one-feature rows whose packet counts straddle every register tier of
    # the fused row kernel (64 / 128 / 256 / 512 packets of 4 or 8 positions)
    # and the two-pass path beyond, at unaligned starts
    v = 8 if dtype != torch.float32 else 4
    sizes = [1, v - 1, v, v + 1, 64 * v - 1, 64 * v, 64 * v + 1, 128 * v + 3, 256 * v, 256 * v + 5,
             512 * v - 2, 512 * v, 512 * v + 1, 1500 * v, 3]
    rng = np.random.default_rng(54)
    deg = np.array(sizes, dtype=np.int64)
    idx = np.repeat(np.arange(deg.size), deg)
    x = (rng.standard_normal((2, idx.size)) * 5).astype(np.float32)
    src = torch.from_numpy(x).to(dtype)
    _softmax_check(ogn, oracle, src, torch.from_numpy(idx), 1, deg.size, mode, SOFT_TOL[dtype])


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("mode", ["softmax", "log_softmax"])
@pytest.mark.parametrize("before", [1, 2])
def test_grouped_softmax_repeated_calls(ogn, oracle, dtype, mode, before):
    # Repeated calls with one index tensor (its group pointers are cached):
    # rows straddling the register tiers of the row and long-row kernels, a
    # poisoned long row; every call is checked, and again after the index
    # changes in place (new version, pointers rebuilt).
    v = 8 if dtype != torch.float32 else 4
    sizes = [1, 64 * v, 256 * v, 256 * v + 1, 512 * v + 3, 1024 * v, 1024 * v + 1, 3000 * v, 0, 7, 300,
             256 * v + 1, 5, 2048 * v + 9]
    rng = np.random.default_rng(55)
    deg = np.array(sizes, dtype=np.int64)
    idx = np.repeat(np.arange(deg.size), deg)
    x = (rng.standard_normal((before, idx.size)) * 5).astype(np.float32)
    starts = np.concatenate([[0], np.cumsum(deg)])
    x[0, starts[7] + 100] = INF  # a long row poisoned
    src = torch.from_numpy(x).to(dtype)
    index = torch.from_numpy(idx).cuda()
    fn = ogn.scatter_softmax if mode == "softmax" else ogn.scatter_log_softmax
    for step in range(5):
        if step == 3:
            # move a boundary in place: the list is rebuilt for the new version
            j = int(starts[2])
            index[j: j + 40] = 1
            idx[j: j + 40] = 1
        got = fn(src.cuda(), index, 1, deg.size).float().cpu().numpy()
        gold = cast_like(oracle.group_softmax(src, torch.from_numpy(idx), 1, deg.size, mode), dtype)
        np.testing.assert_array_equal(np.isnan(got), np.isnan(gold))
        np.testing.assert_allclose(got, gold, rtol=SOFT_TOL[dtype], atol=SOFT_TOL[dtype], equal_nan=True,
                                   err_msg=f"call {step}")


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("mode", ["softmax", "log_softmax"])
@pytest.mark.parametrize("before", [1, 3])
def test_grouped_softmax_binned_rows(ogn, oracle, dtype, mode, before):
    # The first call bins the rows by packet count into a kept plan; later
    # calls with the same index run them binned: 8 / 16 / 32-lane groups for
    # rows of up to 8 / 16 / 32 packets (several rows per wavefront, the last
    # wavefront of a class partly empty), one wavefront for up to 256 packets,
    # a block beyond.  Sizes straddle every class edge at unaligned starts,
    # with empty rows and +-inf / NaN in short rows.
    v = 8 if dtype != torch.float32 else 4
    edges = [8, 16, 32, 64, 128, 192, 256]
    sizes = [0, 1, 2, v - 1, v + 1]
    for e in edges:
        sizes += [e * v - 3, e * v, e * v + 2]
    sizes += [300 * v, 1500 * v + 5]
    rng = np.random.default_rng(56)
    deg = np.array([sizes[i] for i in rng.integers(0, len(sizes), 400)] + sizes, dtype=np.int64)
    deg = np.maximum(deg, 0)
    idx = np.repeat(np.arange(deg.size), deg)
    x = (rng.standard_normal((before, idx.size)) * 4).astype(np.float32)
    starts = np.concatenate([[0], np.cumsum(deg)])
    short = [r for r in range(deg.size) if 2 <= deg[r] <= 8 * v][:3]
    x[0, starts[short[0]]] = INF
    x[-1, starts[short[1]] + 1] = NAN
    x[0, starts[short[2]]: starts[short[2] + 1]] = -INF
    src = torch.from_numpy(x).to(dtype)
    index = torch.from_numpy(idx).cuda()
    fn = ogn.scatter_softmax if mode == "softmax" else ogn.scatter_log_softmax
    gold = cast_like(oracle.group_softmax(src, torch.from_numpy(idx), 1, deg.size, mode), dtype)
    for step in range(3):
        got = fn(src.cuda(), index, 1, deg.size).float().cpu().numpy()
        np.testing.assert_array_equal(np.isnan(got), np.isnan(gold), err_msg=f"call {step}")
        np.testing.assert_allclose(got, gold, rtol=SOFT_TOL[dtype], atol=SOFT_TOL[dtype], equal_nan=True,
                                   err_msg=f"call {step}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("before", [1, 2])
def test_grouped_softmax_kept_plan_row_order(ogn, oracle, dtype, before):
    # A kept plan with few short rows runs the rows one wavefront each in
    # row order and takes its long rows (> 256 packets) from the plan's
    # bounds, with no list-building launch.
    v = 8 if dtype != torch.float32 else 4
    rng = np.random.default_rng(57)
    deg = rng.integers(33 * v, 256 * v, 300)
    deg[::40] = rng.integers(257 * v, 900 * v, deg[::40].size)
    deg[7] = 3
    deg[8] = 0
    idx = np.repeat(np.arange(deg.size), deg)
    src = torch.from_numpy((rng.standard_normal((before, idx.size)) * 4).astype(np.float32)).to(dtype)
    index = torch.from_numpy(idx).cuda()
    gold = cast_like(oracle.group_softmax(src, torch.from_numpy(idx), 1, deg.size, "log_softmax"), dtype)
    for step in range(3):
        got = ogn.scatter_log_softmax(src.cuda(), index, 1, deg.size).float().cpu().numpy()
        np.testing.assert_allclose(got, gold, rtol=SOFT_TOL[dtype], atol=SOFT_TOL[dtype], err_msg=f"call {step}")


@pytest.mark.parametrize("sorted_index", [True, False])
def test_grouped_softmax_special_values(ogn, oracle, sorted_index):
    src = torch.tensor([INF, 1.0, -INF, 2.0, NAN, 0.0, -INF, -INF])
    index = torch.tensor([0, 0, 1, 1, 2, 2, 3, 3])
    if not sorted_index:
        perm = torch.tensor([5, 2, 7, 0, 3, 6, 1, 4])
        src, index = src[perm], index[perm]
    for mode in ("softmax", "log_softmax", "logsumexp"):
        _softmax_check(ogn, oracle, src, index, 0, 4, mode, 1e-6)


# Gradient tolerance: the reference's grouped-softmax tolerances
# (test/common/grouped_softmax_golden.py:24-28), rtol = atol.
GRAD_TOL = {torch.float32: 1e-5, torch.float16: 2e-2, torch.bfloat16: 4e-2}


def _softmax_grad_check(ogn, oracle, src, index, dim, groups, mode, tol, seed=0):
    fn = {"softmax": ogn.scatter_softmax, "log_softmax": ogn.scatter_log_softmax,
          "logsumexp": ogn.scatter_logsumexp}[mode]
    x = src.cuda().requires_grad_(True)
    out = fn(x, index.cuda(), dim, groups)
    g = torch.from_numpy(np.random.default_rng(seed).standard_normal(tuple(out.shape)).astype(np.float32))
    g = g.to(src.dtype)
    out.backward(g.cuda())
    assert x.grad.dtype == src.dtype and x.grad.shape == src.shape
    gold = oracle.group_softmax_backward(src, g, index.long(), dim, groups, mode)
    got = x.grad.float().cpu().numpy()
    np.testing.assert_array_equal(np.isnan(got), np.isnan(gold))
    np.testing.assert_allclose(got, gold, rtol=tol, atol=tol, equal_nan=True)


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("mode", ["softmax", "log_softmax", "logsumexp"])
@pytest.mark.parametrize("sorted_index", [True, False])
def test_grouped_softmax_backward(ogn, oracle, dtype, mode, sorted_index):
    rng = np.random.default_rng(53)
    idx = rng.integers(0, 40, 2000)
    idx[idx == 7] = 8  # an empty group
    if sorted_index:
        idx = np.sort(idx)
    src = torch.from_numpy((rng.standard_normal((3, 2000, 4)) * 3).astype(np.float32)).to(dtype)
    _softmax_grad_check(ogn, oracle, src, torch.from_numpy(idx), 1, 40, mode, GRAD_TOL[dtype])


@pytest.mark.parametrize("mode", ["softmax", "log_softmax", "logsumexp"])
def test_grouped_softmax_backward_edge_rows(ogn, oracle, mode):
    # GAT layout: one score per edge grouped by destination row, hub rows of 4000
    rng = np.random.default_rng(54)
    deg = rng.poisson(40, size=300)
    deg[::30] = 4000
    idx = np.repeat(np.arange(300), deg)
    src = torch.from_numpy((rng.standard_normal(idx.size) * 3).astype(np.float32))
    _softmax_grad_check(ogn, oracle, src, torch.from_numpy(idx), 0, 300, mode, 1e-5, seed=1)


@pytest.mark.parametrize("sorted_index", [True, False])
def test_grouped_softmax_backward_special_values(ogn, oracle, sorted_index):
    src = torch.tensor([INF, 1.0, -INF, -INF, 0.5, 2.0])
    index = torch.tensor([0, 0, 1, 1, 2, 2])
    if not sorted_index:
        perm = torch.tensor([3, 5, 0, 2, 4, 1])
        src, index = src[perm], index[perm]
    for mode in ("softmax", "log_softmax", "logsumexp"):
        _softmax_grad_check(ogn, oracle, src, index, 0, 3, mode, 1e-6)


def test_grouped_softmax_backward_matches_torch_autograd(ogn):
    # the same gradient as torch's own softmax autograd over one group per row
    x = torch.randn(6, 50, dtype=torch.float32, device="cuda")
    idx = torch.arange(6, device="cuda").repeat_interleave(50)
    a = x.reshape(-1).clone().requires_grad_(True)
    b = x.clone().requires_grad_(True)
    g = torch.randn(300, device="cuda")
    ogn.scatter_softmax(a, idx).backward(g)
    torch.softmax(b, 1).reshape(-1).backward(g)
    torch.testing.assert_close(a.grad, b.grad.reshape(-1), rtol=1e-5, atol=1e-6)


def test_grouped_softmax_errors(ogn):
    src = torch.randn(6, device="cuda")
    with pytest.raises(ValueError, match="non-negative"):
        ogn.scatter_softmax(src, torch.tensor([0, -1, 0, 0, 0, 0], device="cuda"))
    with pytest.raises(ValueError, match="smaller than dim_size"):
        ogn.scatter_softmax(src, torch.tensor([0, 3, 0, 0, 0, 0], device="cuda"), dim_size=2)
    with pytest.raises(ValueError, match="must match"):
        ogn.scatter_log_softmax(src, torch.tensor([0, 1], device="cuda"))
    with pytest.raises(ValueError, match="1-D"):
        ogn.scatter_logsumexp(src, torch.zeros(2, 3, dtype=torch.long, device="cuda"))
    with pytest.raises(TypeError):
        ogn.scatter_softmax(src.double(), torch.zeros(6, dtype=torch.long, device="cuda"))
    with pytest.raises(IndexError):
        ogn.scatter_softmax(src, torch.zeros(6, dtype=torch.long, device="cuda"), dim=3)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.int32, torch.int64, torch.uint8])
@pytest.mark.parametrize("layout", ["sorted", "unsorted", "full_shape"])
@pytest.mark.parametrize("reduce", ["sum", "max"])
def test_index_out_of_range_raises(ogn, dtype, layout, reduce):
    """A negative index, or one at or past the output size, raises IndexError
    on every path (reference python/ops_gnn/scatter.py:406-422); nothing is
    silently dropped."""
    src = torch.arange(12, device="cuda").reshape(6, 2).to(dtype)
    base = [0, 0, 1, 2, 2, 3] if layout == "sorted" else [2, 0, 3, 1, 0, 2]

    def make(values):
        idx = torch.tensor(values, device="cuda")
        return idx.view(-1, 1).expand(6, 2).contiguous() if layout == "full_shape" else idx

    bad_neg = list(base)
    bad_neg[3] = -1
    with pytest.raises(IndexError, match="negative value \\(-1\\)"):
        ogn.scatter(src, make(bad_neg), dim=0, reduce=reduce)
    with pytest.raises(IndexError, match="index value 3 is out of bounds for output size 3 at dimension 0"):
        ogn.scatter(src, make(base), dim=0, dim_size=3, reduce=reduce)
    out = torch.zeros(2, 2, device="cuda").to(dtype)
    with pytest.raises(IndexError, match="out of bounds for output size 2"):
        ogn.scatter(src, make(base), dim=0, out=out, reduce=reduce)
    # in range: dim_size = max + 1 is accepted
    ok = ogn.scatter(src, make(base), dim=0, dim_size=4, reduce=reduce)
    assert ok.shape == (4, 2)
