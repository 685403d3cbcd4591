"""GPU parity of CSR SpMM (torch_sparse semantics) against the CPU oracle.

Cases follow the reference's own SpMM tests
(test/torch_sparse_spmm/arch35/test_torch_sparse_spmm.py): the 4-row sample,
the documented extrema policy, the 7/8/9-edge prefetch boundaries, batches
and per-feature weights, plus power-law graphs whose hub rows span many
chunks, empty graphs, int32 indices, unaligned features and determinism.
Sum/mean are compared with |a - g| <= rtol * sum|terms| (rtol 1e-5 fp32,
1e-2 fp16/bf16); min/max values and arg indices must be bit-exact.
"""

import numpy as np
import pytest
import torch

from _util import assert_exact, assert_sum_close, cast_like

pytestmark = pytest.mark.gpu

DT = [torch.float32, torch.float16, torch.bfloat16]
INF, NAN = float("inf"), float("nan")


def _sample(dtype, batch=False, feature_values=False):
    # reference test/torch_sparse_spmm/arch35/golden.py:119-131 (shapes; our seed)
    g = torch.Generator().manual_seed(41)
    ptr = torch.tensor([0, 3, 3, 4, 7], dtype=torch.long)
    col = torch.tensor([2, 0, 2, 1, 3, 0, 1], dtype=torch.long)
    shape = (2, 3, 4, 17) if batch else (4, 17)
    vs = (7, 17) if feature_values else (7,)
    mat = torch.randn(shape, generator=g).to(dtype)
    v = torch.randn(vs, generator=g).to(dtype)
    return ptr, col, v, mat


def check_spmm(ogn, oracle, ptr, col, val, mat, reduce, out_dtype=None, what=""):
    out_dtype = out_dtype or mat.dtype
    dev = "cuda"
    res = ogn.csr_spmm(ptr.to(dev), col.to(dev), None if val is None else val.to(dev), mat.to(dev), reduce,
                       output_dtype=out_dtype)
    actual, arg = res if reduce in ("min", "max") else (res, None)
    assert actual.dtype == out_dtype and actual.device.type == "cuda"
    golden, garg = oracle.spmm_csr(ptr, col, val, mat, reduce)
    if reduce in ("min", "max"):
        assert_exact(actual, cast_like(golden, out_dtype), what + " values")
        assert_exact(arg, garg, what + " arg")
    else:
        scale, _ = oracle.spmm_csr(ptr, col, None if val is None else val.float().abs(), mat.float().abs(),
                                   reduce)
        assert_sum_close(actual, golden, scale, out_dtype, what)
    return actual, arg


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("reduce", ["sum", "mean", "min", "max"])
@pytest.mark.parametrize("batch,feature_values", [(False, False), (True, True)])
def test_sample_forward(ogn, oracle, dtype, reduce, batch, feature_values):
    ptr, col, v, mat = _sample(dtype, batch, feature_values)
    check_spmm(ogn, oracle, ptr, col, v, mat, reduce, what=f"sample/{dtype}/{reduce}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("reduce", ["sum", "max"])
def test_low_precision_input_fp32_output(ogn, oracle, dtype, reduce):
    ptr, col, v, mat = _sample(dtype)
    check_spmm(ogn, oracle, ptr, col, v, mat, reduce, out_dtype=torch.float32)


@pytest.mark.parametrize("reduce", ["min", "max"])
def test_extrema_documented_special_policy(ogn, reduce):
    # reference test/torch_sparse_spmm/arch35/test_torch_sparse_spmm.py:518-536
    p = torch.tensor([0, 2, 2, 3], device="cuda")
    c = torch.tensor([0, 1, 2], device="cuda")
    b = torch.tensor([[2.0, NAN, INF], [2.0, 3.0, -INF], [NAN, NAN, NAN]], device="cuda")
    out, arg = ogn.csr_spmm(p, c, None, b, reduce)
    expected = torch.tensor([[2.0, 3.0, -INF if reduce == "min" else INF], [0.0, 0.0, 0.0], [0.0, 0.0, 0.0]])
    assert torch.equal(out.cpu(), expected)
    assert torch.equal(arg.cpu(), torch.tensor([[0, 1, 1 if reduce == "min" else 0], [3, 3, 3], [3, 3, 3]]))


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("reduce", ["sum", "mean", "min", "max"])
@pytest.mark.parametrize("features", [64, 128, 256, 512])
def test_prefetch_widths_and_eight_edge_boundary(ogn, oracle, dtype, reduce, features):
    # reference test/torch_sparse_spmm/arch35/test_torch_sparse_spmm.py:704-716
    ptr = torch.tensor([0, 0, 7, 15, 24, 41], dtype=torch.int64)
    col = torch.arange(41, dtype=torch.int64).remainder(5)
    values = torch.arange(41).remainder(7).sub(3).to(dtype)
    mat = torch.arange(5 * features).reshape(5, features).remainder(11).sub(5).to(dtype)
    check_spmm(ogn, oracle, ptr, col, values, mat, reduce)


@pytest.mark.parametrize("reduce", ["min", "max"])
@pytest.mark.parametrize("features", [64, 128, 256, 512])
def test_prefetch_extrema_special_values_and_first_tie(ogn, reduce, features):
    # reference test/torch_sparse_spmm/arch35/test_torch_sparse_spmm.py:719-744
    ptr = torch.tensor([0, 0, 9, 10], dtype=torch.int64)
    col = torch.tensor([0] * 8 + [1, 2], dtype=torch.int64)
    values = torch.ones(10)
    mat = torch.full((3, features), 2.0)
    mat[0, 1] = NAN
    mat[1, 1] = 3.0
    mat[0, 2] = INF
    mat[1, 2] = -INF
    mat[2] = NAN
    actual, arg = ogn.csr_spmm(ptr.cuda(), col.cuda(), values.cuda(), mat.cuda(), reduce)
    expected = torch.zeros((3, features))
    expected[1] = 2.0
    expected[1, 1] = 3.0
    expected[1, 2] = -INF if reduce == "min" else INF
    expected_arg = torch.full((3, features), 10, dtype=torch.int64)
    expected_arg[1] = 0
    expected_arg[1, 1] = 8
    expected_arg[1, 2] = 8 if reduce == "min" else 0
    assert torch.equal(actual.cpu(), expected)
    assert torch.equal(arg.cpu(), expected_arg)


def _powerlaw(m, n, nnz, cap, seed):
    from ops_gnn.synthetic import powerlaw_csr

    ptr, col, rng = powerlaw_csr(m, n, nnz, cap, seed)
    return torch.from_numpy(ptr), torch.from_numpy(col), rng


@pytest.mark.parametrize("k", [1, 4, 8, 17, 32, 40, 64, 96, 128, 200, 256, 512, 1024])
@pytest.mark.parametrize("reduce", ["sum", "mean", "max"])
def test_powerlaw_feature_widths(ogn, oracle, k, reduce):
    ptr, col, rng = _powerlaw(3000, 2500, 60_000, 6000, seed=k)
    mat = torch.from_numpy(rng.standard_normal((2500, k), dtype=np.float32))
    val = torch.from_numpy(rng.random(col.numel(), dtype=np.float32))
    check_spmm(ogn, oracle, ptr, col, val, mat, reduce, what=f"powerlaw/k{k}/{reduce}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("k", [4, 8, 16])
@pytest.mark.parametrize("reduce", ["sum", "max"])
@pytest.mark.parametrize("feature_values", [False, True])
def test_narrow_rows_16bit(ogn, oracle, dtype, k, reduce, feature_values):
    # K * 2 bytes <= 32: one or two lanes per row, 64 / 32 positions per step
    ptr, col, rng = _powerlaw(4000, 3000, 90_000, 9000, seed=10 + k)
    mat = torch.from_numpy(rng.standard_normal((3000, k), dtype=np.float32)).to(dtype)
    shape = (col.numel(), k) if feature_values else (col.numel(),)
    val = torch.from_numpy(rng.random(shape, dtype=np.float32)).to(dtype)
    check_spmm(ogn, oracle, ptr, col, val, mat, reduce, what=f"narrow/{dtype}/k{k}/{reduce}")


def _check_int8(ogn, oracle, ptr, col, val, mat, reduce, out_dtype, what):
    """int8 SpMM against the golden's cast of the fp64 result: int32 truncates,
    float32 rounds once (reference golden.py:80-88,114-115).  Bit-exact."""
    res = ogn.csr_spmm(ptr.cuda(), col.cuda(), None if val is None else val.cuda(), mat.cuda(), reduce,
                       output_dtype=out_dtype)
    got, arg = res if reduce in ("min", "max") else (res, None)
    assert got.dtype == out_dtype
    gold, garg = oracle.spmm_csr(ptr, col, val, mat, reduce)
    want = oracle.spmm_output_cast(gold, out_dtype)
    assert_exact(got, want, what + " values")
    if arg is not None:
        assert_exact(arg, garg, what + " arg")


@pytest.mark.parametrize("out_dtype", [torch.int32, torch.float32])
@pytest.mark.parametrize("reduce", ["sum", "mean", "min", "max"])
@pytest.mark.parametrize("k,feature_values", [(16, False), (128, False), (32, True), (5, False)])
def test_int8_powerlaw(ogn, oracle, reduce, k, feature_values, out_dtype):
    # reference golden test/torch_sparse_spmm/arch35/golden.py:91-116: int8
    # mat / value, fp64 arithmetic, then trunc (int32) or one rounding (fp32)
    ptr, col, rng = _powerlaw(3000, 2000, 70_000, 9000, seed=20 + k)
    mat = torch.from_numpy(rng.integers(-128, 128, (2000, k)).astype(np.int8))
    shape = (col.numel(), k) if feature_values else (col.numel(),)
    val = torch.from_numpy(rng.integers(-128, 128, shape).astype(np.int8))
    _check_int8(ogn, oracle, ptr, col, val, mat, reduce, out_dtype, f"int8/{reduce}/k{k}/{out_dtype}")


@pytest.mark.parametrize("out_dtype", [torch.int32, torch.float32])
@pytest.mark.parametrize("reduce", ["sum", "mean", "min", "max"])
@pytest.mark.parametrize("batch,feature_values", [(False, False), (True, True)])
def test_int8_sample(ogn, oracle, reduce, batch, feature_values, out_dtype):
    # the reference's sample (golden.py:119-131) for its (int8, int32) and
    # (int8, float32) COMBOS
    ptr, col, _, _ = _sample(torch.float32, batch, feature_values)
    g = torch.Generator().manual_seed(5)
    mat = torch.randint(-128, 128, (2, 3, 4, 17) if batch else (4, 17), generator=g).to(torch.int8)
    val = torch.randint(-128, 128, (7, 17) if feature_values else (7,), generator=g).to(torch.int8)
    _check_int8(ogn, oracle, ptr, col, val, mat, reduce, out_dtype, f"int8 sample/{reduce}")


@pytest.mark.parametrize("out_dtype", [torch.int32, torch.float32])
@pytest.mark.parametrize("reduce", ["sum", "mean", "min", "max"])
@pytest.mark.parametrize("features", [64, 128, 256, 512])
def test_int8_prefetch_boundaries(ogn, oracle, reduce, features, out_dtype):
    # reference test/torch_sparse_spmm/arch35/test_torch_sparse_spmm.py:704-716
    # with the int8 COMBOS; the 7 / 8 / 9 / 17-edge rows give non-integer means
    ptr = torch.tensor([0, 0, 7, 15, 24, 41], dtype=torch.int64)
    col = torch.arange(41, dtype=torch.int64).remainder(5)
    values = torch.arange(41).remainder(7).sub(3).to(torch.int8)
    mat = torch.arange(5 * features).reshape(5, features).remainder(11).sub(5).to(torch.int8)
    _check_int8(ogn, oracle, ptr, col, values, mat, reduce, out_dtype, f"int8 prefetch/{reduce}/{features}")


def test_output_dtype_table(ogn):
    """The reference's input -> output table (torch_sparse_spmm.cpp:88-90):
    f32 -> f32; f16 -> f16 | f32; bf16 -> bf16 | f32; int8 -> int32 | f32."""
    ptr = torch.tensor([0, 1, 2], device="cuda")
    col = torch.tensor([0, 1], device="cuda")
    allowed = {torch.float32: {torch.float32}, torch.float16: {torch.float16, torch.float32},
               torch.bfloat16: {torch.bfloat16, torch.float32}, torch.int8: {torch.int32, torch.float32}}
    for src, outs in allowed.items():
        mat = torch.ones((2, 4), device="cuda").to(src)
        for out_dtype in (torch.float32, torch.float16, torch.bfloat16, torch.int32):
            if out_dtype in outs:
                got = ogn.csr_spmm(ptr, col, None, mat, "sum", output_dtype=out_dtype)
                assert got.dtype == out_dtype and torch.equal(got.cpu().double(), torch.ones(2, 4).double())
            else:
                with pytest.raises(ValueError, match="dtype"):
                    ogn.csr_spmm(ptr, col, None, mat, "sum", output_dtype=out_dtype)


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("reduce", ["sum", "min", "max"])
def test_powerlaw_k128_dtypes(ogn, oracle, dtype, reduce):
    ptr, col, rng = _powerlaw(20_000, 20_000, 400_000, 20_000, seed=3)
    mat = torch.from_numpy(rng.standard_normal((20_000, 128), dtype=np.float32)).to(dtype)
    val = torch.from_numpy(rng.random(col.numel(), dtype=np.float32)).to(dtype)
    check_spmm(ogn, oracle, ptr, col, val, mat, reduce, what=f"powerlaw128/{dtype}/{reduce}")


def test_single_hub_row_spans_many_chunks(ogn, oracle):
    # one 50 000-edge row between short rows: carries through ~200 chunks
    deg = np.array([3, 0, 50_000, 1, 0, 7], dtype=np.int64)
    rng = np.random.default_rng(9)
    col = np.concatenate([np.sort(rng.integers(0, 1000, d)) for d in deg])
    ptr = torch.from_numpy(np.concatenate([[0], np.cumsum(deg)]))
    mat = torch.from_numpy(rng.standard_normal((1000, 128), dtype=np.float32))
    for reduce in ("sum", "mean", "min", "max"):
        check_spmm(ogn, oracle, ptr, torch.from_numpy(col), None, mat, reduce, what=f"hub/{reduce}")


def test_poisson_config1(ogn, oracle):
    from ops_gnn.synthetic import cfg1_spmm_small

    ptr, col, val, mat = map(torch.from_numpy, cfg1_spmm_small())
    check_spmm(ogn, oracle, ptr, col, val, mat, "sum", what="cfg1")


@pytest.mark.parametrize("reduce", ["sum", "mean", "min", "max"])
def test_empty_graph_and_empty_rows(ogn, reduce):
    ptr = torch.zeros(6, dtype=torch.int64, device="cuda")
    col = torch.empty(0, dtype=torch.int64, device="cuda")
    mat = torch.randn(4, 33, device="cuda")
    res = ogn.csr_spmm(ptr, col, None, mat, reduce)
    out, arg = res if reduce in ("min", "max") else (res, None)
    assert torch.equal(out.cpu(), torch.zeros(5, 33))
    if arg is not None:
        assert torch.equal(arg.cpu(), torch.zeros(5, 33, dtype=torch.int64))


def test_int32_indices_native_entry(ogn, oracle):
    from ops_gnn import _native

    ptr, col, rng = _powerlaw(2000, 1500, 30_000, 3000, seed=5)
    mat = torch.from_numpy(rng.standard_normal((1500, 64), dtype=np.float32))
    out, _ = _native.spmm_forward(ptr.int().cuda(), col.int().cuda(), None, mat.cuda(), 0, torch.float32)
    golden, _ = oracle.spmm_csr(ptr, col, None, mat, "sum")
    scale, _ = oracle.spmm_csr(ptr, col, None, mat.abs(), "sum")
    assert_sum_close(out, golden, scale, torch.float32, "int32")


def test_unaligned_mat_uses_scalar_path(ogn, oracle):
    ptr, col, rng = _powerlaw(500, 400, 5000, 800, seed=6)
    base = torch.from_numpy(rng.standard_normal(400 * 64 + 1, dtype=np.float32))
    mat = base[1:].reshape(400, 64)  # storage offset 4 bytes: not 16-byte aligned on the GPU
    dev = base.cuda()[1:].reshape(400, 64)
    assert dev.data_ptr() % 16 != 0
    res = ogn.csr_spmm(ptr.cuda(), col.cuda(), None, dev, "max")
    golden, garg = oracle.spmm_csr(ptr, col, None, mat, "max")
    assert_exact(res[0], golden.astype(np.float32), "unaligned values")
    assert_exact(res[1], garg, "unaligned arg")


def test_determinism_bitwise(ogn):
    ptr, col, rng = _powerlaw(20_000, 20_000, 400_000, 20_000, seed=8)
    mat = torch.from_numpy(rng.standard_normal((20_000, 128), dtype=np.float32)).cuda()
    p, c = ptr.cuda(), col.cuda()
    outs = [ogn.csr_spmm(p, c, None, mat, "sum") for _ in range(4)]
    for o in outs[1:]:
        assert torch.equal(o, outs[0])


def test_non_default_stream(ogn):
    # reference test/conftest.py:217-230 (stream ordering)
    stream = torch.cuda.Stream()
    ptr = torch.tensor([0, 1, 2], device="cuda")
    idx = torch.tensor([1, 0], device="cuda")
    x = torch.ones(2, 17, device="cuda")
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        x = x * -3
        result = ogn.csr_spmm(ptr, idx, None, x) + 2
    torch.cuda.current_stream().wait_stream(stream)
    assert torch.equal(result.cpu(), torch.full((2, 17), -1.0))


def test_torch_sparse_registration(ogn, oracle):
    ptr, col, v, mat = _sample(torch.float32)
    row = torch.repeat_interleave(torch.arange(4), ptr[1:] - ptr[:-1])
    d = lambda t: t.cuda()
    out = torch.ops.torch_sparse.spmm_sum(d(row), d(ptr), d(col), d(v), None, None, d(mat))
    golden, _ = oracle.spmm_csr(ptr, col, v, mat, "sum")
    scale, _ = oracle.spmm_csr(ptr, col, v.abs(), mat.abs(), "sum")
    assert_sum_close(out, golden, scale, torch.float32, "registered sum")
    counts = ptr[1:] - ptr[:-1]
    out = torch.ops.torch_sparse.spmm_mean(d(row), d(ptr), d(col), d(v), d(counts), None, None, d(mat))
    golden, _ = oracle.spmm_csr(ptr, col, v, mat, "mean")
    assert_sum_close(out, golden, scale, torch.float32, "registered mean")
    out, arg = torch.ops.torch_sparse.spmm_max(d(ptr), d(col), d(v), d(mat))
    golden, garg = oracle.spmm_csr(ptr, col, v, mat, "max")
    assert_exact(out, golden.astype(np.float32))
    assert_exact(arg, garg)
    assert torch.equal(torch.ops.torch_sparse.ind2ptr(d(row), 4).cpu(), ptr)
    assert torch.equal(torch.ops.torch_sparse.ptr2ind(d(ptr), 7).cpu(), row)


def test_coo_spmm_unsorted_rows(ogn):
    index = torch.tensor([[2, 0, 0, 1], [1, 2, 0, 1]], dtype=torch.int64)
    values = torch.tensor([1.0, -2.0, 0.5, 3.0])
    mat = torch.arange(12, dtype=torch.float32).reshape(3, 4) - 5
    expected = torch.zeros(3, 4, dtype=torch.float64)
    expected.index_add_(0, index[0], mat.double()[index[1]] * values.double()[:, None])
    out = ogn.coo_spmm(index.cuda(), values.cuda(), 3, 3, mat.cuda())
    torch.testing.assert_close(out.cpu().double(), expected, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("ptr,col", [
    # reference test/conftest.py:37-45 (SPMM_BAD_CSR_CASES)
    ([1, 1], [0]), ([0, 2], [0]), ([0, 2, 1, 2], [0, 0]), ([0, -1, 1], [0]), ([0, 1], [-1]),
    ([0, 1], [2]), ([0, 1], [2**32]), ([0, 2**32], [0]),
])
def test_bad_csr_rejected(ogn, ptr, col):
    with pytest.raises(ValueError, match="invalid CSR"):
        ogn.csr_spmm(torch.tensor(ptr, device="cuda"), torch.tensor(col, device="cuda"), None,
                     torch.ones(2, 17, device="cuda"))
