"""GPU tests of the torch_sparse boundary: the ``_pybind.torch_sparse_spmm``
extension called directly (reference csrc/pybind.cpp:245-257 signatures)
against the oracle, the torch_sparse operator schemas' metadata contract
(reference python/ops_gnn/torch_sparse_spmm.py:96-149), autograd of every
reduction against float64 PyTorch, and the frontend adaptation with a real
SparseTensor-shaped operand on the GPU.
"""

import sys

import numpy as np
import pytest
import torch

import _stub_frontends as stub
from _util import assert_exact, assert_sum_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _graph(m=300, n=250, mean=9, seed=0, hub=None):
    rng = np.random.default_rng(seed)
    deg = rng.poisson(mean, m)
    deg[rng.integers(0, m, 5)] = 0
    if hub is not None:
        deg[7] = hub
    col = np.concatenate([np.sort(rng.integers(0, n, d)) for d in deg]).astype(np.int64)
    ptr = np.concatenate([[0], np.cumsum(deg)]).astype(np.int64)
    return torch.from_numpy(ptr), torch.from_numpy(col), rng


# ------------------------------------------------------------------ the extension itself
@pytest.mark.parametrize("reduce", [0, 1, 2, 3])
@pytest.mark.parametrize("mat_dtype,outtype", [(torch.float32, 0), (torch.float16, 1), (torch.bfloat16, 0),
                                               (torch.int8, 4), (torch.int8, 0)])
def test_extension_forward(ogn, oracle, reduce, mat_dtype, outtype):
    from ops_gnn import _pybind

    ptr, col, rng = _graph(seed=reduce, hub=3000)
    if mat_dtype == torch.int8:
        mat = torch.from_numpy(rng.integers(-128, 128, (250, 64)).astype(np.int8))
        val = torch.from_numpy(rng.integers(-128, 128, col.numel()).astype(np.int8))
    else:
        mat = torch.from_numpy(rng.standard_normal((250, 64), dtype=np.float32)).to(mat_dtype)
        val = torch.from_numpy(rng.random(col.numel(), dtype=np.float32)).to(mat_dtype)
    out, arg = _pybind.torch_sparse_spmm.forward(ptr.to(DEV), col.to(DEV), val.to(DEV), mat.to(DEV), reduce, outtype)
    name = {0: "sum", 1: "mean", 2: "min", 3: "max"}[reduce]
    out_dtype = {0: torch.float32, 1: torch.float16, 4: torch.int32}[outtype]
    assert out.dtype == out_dtype
    gold, garg = oracle.spmm_csr(ptr, col, val, mat, name)
    if reduce >= 2 or mat_dtype == torch.int8:
        assert_exact(out, oracle.spmm_output_cast(gold, "float16" if outtype == 1 else str(out_dtype)), "forward")
        if reduce >= 2:
            assert_exact(arg, garg, "forward arg")
    else:
        scale, _ = oracle.spmm_csr(ptr, col, val.float().abs(), mat.float().abs(), name)
        assert_sum_close(out, gold, scale, out_dtype if out_dtype != torch.float32 else mat_dtype, "forward")
        assert arg.numel() == 0


def test_extension_rejects_unsupported_dtype_pairs(ogn):
    from ops_gnn import _pybind

    ptr = torch.tensor([0, 1], device=DEV)
    col = torch.tensor([0], device=DEV)
    for dtype, outtype in ((torch.float32, 1), (torch.float32, 4), (torch.float16, 2), (torch.int8, 1)):
        with pytest.raises(RuntimeError, match="dtype combination"):
            _pybind.torch_sparse_spmm.forward(ptr, col, None, torch.ones(1, 4, device=DEV).to(dtype), 0, outtype)


def test_extension_validate_convert_permute_version(ogn, oracle):
    from ops_gnn import _pybind

    C = _pybind.torch_sparse_spmm
    ptr, col, _ = _graph(seed=3)
    p, c = ptr.to(DEV), col.to(DEV)
    assert int(C.validate(p, c, 250).item()) == 0
    assert int(C.validate(p, c, 10).item()) == 2             # columns past n
    bad = p.clone()
    bad[5] = bad[6] + 1
    assert int(C.validate(bad, c, 250).item()) == 1
    row = C.convert(p, col.numel(), False)
    assert_exact(row, oracle.ptr2ind(ptr, col.numel()), "convert ptr2ind")
    assert_exact(C.convert(row, ptr.numel(), True), ptr.numpy(), "convert ind2ptr")
    perm = torch.randperm(col.numel(), device=DEV)
    for shape in ((col.numel(),), (col.numel(), 3)):
        v = torch.randn(shape, device=DEV).half()
        assert torch.equal(C.permute_values(v, perm), v[perm])
    t = torch.zeros(3)
    v0 = C.tensor_version(t)
    t.add_(1)
    assert C.tensor_version(t) == v0 + 1
    with torch.inference_mode():
        assert C.tensor_version(torch.zeros(2)) is None


@pytest.mark.parametrize("reduce", [0, 1])
@pytest.mark.parametrize("width", [1, 32])
def test_extension_value_backward(ogn, reduce, width):
    from ops_gnn import _pybind

    ptr, col, rng = _graph(seed=4, hub=2000)
    mat = torch.from_numpy(rng.standard_normal((2, 250, 32), dtype=np.float32))
    grad = torch.from_numpy(rng.standard_normal((2, 300, 32), dtype=np.float32))
    dv = _pybind.torch_sparse_spmm.value_backward(ptr.to(DEV), col.to(DEV), mat.to(DEV), grad.to(DEV), reduce, width)
    row = torch.repeat_interleave(torch.arange(300), ptr.diff())
    prod = grad.double()[:, row, :] * mat.double()[:, col, :]          # [B, E, K]
    if reduce == 1:
        prod = prod / ptr.diff().clamp_min(1).double()[row].view(1, -1, 1)
    want = prod.sum(0) if width > 1 else prod.sum((0, 2))
    torch.testing.assert_close(dv.cpu().double(), want, rtol=1e-5, atol=1e-4)


# ------------------------------------------------------------------ operator schema metadata contract
def test_schema_requires_gradient_metadata(ogn):
    ptr, col, _ = _graph(seed=5)
    p, c = ptr.to(DEV), col.to(DEV)
    e, m = col.numel(), ptr.numel() - 1
    mat = torch.randn(250, 8, device=DEV, requires_grad=True)
    value = torch.rand(e, device=DEV)
    with pytest.raises(ValueError, match=r"row must be int64 \[%d\]" % e):
        torch.ops.torch_sparse.spmm_sum(None, p, c, value, None, None, mat)
    row = torch.repeat_interleave(torch.arange(m, device=DEV), p.diff())
    with pytest.raises(ValueError, match="colptr must be int64"):
        torch.ops.torch_sparse.spmm_sum(row, p, c, value, None, None, mat)
    perm = torch.argsort(c, stable=True)
    colptr = torch.ops.torch_sparse.ind2ptr(c[perm], 250)
    out = torch.ops.torch_sparse.spmm_sum(row, p, c, value, colptr, perm, mat)
    with pytest.raises(ValueError, match="rowcount must be int64"):
        torch.ops.torch_sparse.spmm_mean(row, p, c, value, None, colptr, perm, mat)
    # wrong contents are caught
    with pytest.raises(ValueError, match="row disagrees"):
        torch.ops.torch_sparse.spmm_sum(row.flip(0), p, c, value, colptr, perm, mat)
    with pytest.raises(ValueError, match="permutation"):
        torch.ops.torch_sparse.spmm_sum(row, p, c, value, colptr, torch.zeros_like(perm), mat)
    with pytest.raises(ValueError, match="order edges by column"):
        torch.ops.torch_sparse.spmm_sum(row, p, c, value, colptr, perm.flip(0), mat)
    with pytest.raises(ValueError, match="colptr disagrees"):
        torch.ops.torch_sparse.spmm_sum(row, p, c, value, colptr + 1, perm, mat)
    with pytest.raises(ValueError, match="rowcount disagrees"):
        torch.ops.torch_sparse.spmm_mean(row, p, c, value, p.diff() + 1, colptr, perm, mat)
    # without gradients, omitted metadata is fine
    with torch.no_grad():
        torch.ops.torch_sparse.spmm_sum(None, p, c, value, None, None, mat)
    out.sum().backward()
    assert mat.grad is not None


# ------------------------------------------------------------------ autograd vs float64 PyTorch
def _ref_spmm(ptr, col, value, mat, reduce):
    m = ptr.numel() - 1
    row = torch.repeat_interleave(torch.arange(m), ptr.diff())
    msg = mat[..., col, :] * (value.reshape(col.numel(), -1) if value is not None else 1.0)
    shape = list(mat.shape)
    shape[-2] = m
    idx = row.view(-1, 1).expand(-1, mat.size(-1))
    if mat.dim() == 3:
        idx = idx.unsqueeze(0).expand(mat.size(0), -1, -1)
    if reduce in ("sum", "mean"):
        out = torch.zeros(shape, dtype=mat.dtype).scatter_add(-2, idx, msg)
        if reduce == "mean":
            out = out / ptr.diff().clamp_min(1).to(mat.dtype).unsqueeze(-1)
        return out
    return torch.zeros(shape, dtype=mat.dtype).scatter_reduce(-2, idx, msg, "amax" if reduce == "max" else "amin",
                                                            include_self=False)


@pytest.mark.parametrize("reduce", ["sum", "mean", "min", "max"])
@pytest.mark.parametrize("width,batch", [(1, False), (16, False), (1, True)])
def test_csr_spmm_gradients(ogn, reduce, width, batch):
    ptr, col, rng = _graph(seed=6, hub=900)
    e = col.numel()
    shape = (2, 250, 16) if batch else (250, 16)
    mat64 = torch.from_numpy(rng.standard_normal(shape))
    val64 = torch.from_numpy(rng.uniform(0.5, 1.5, (e, width) if width > 1 else (e,)))
    grad64 = torch.from_numpy(rng.standard_normal(shape[:-2] + (300, 16)))
    m_ref = mat64.clone().requires_grad_(True)
    v_ref = val64.clone().requires_grad_(True)
    _ref_spmm(ptr, col, v_ref, m_ref, reduce).backward(grad64)
    mat = mat64.float().to(DEV).requires_grad_(True)
    val = val64.float().to(DEV).requires_grad_(True)
    res = ogn.csr_spmm(ptr.to(DEV), col.to(DEV), val, mat, reduce)
    out = res[0] if reduce in ("min", "max") else res
    out.backward(grad64.float().to(DEV))
    torch.testing.assert_close(mat.grad.cpu().double(), m_ref.grad, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(val.grad.cpu().double(), v_ref.grad, rtol=1e-4, atol=1e-4)


# ------------------------------------------------------------------ frontends on the GPU
@pytest.fixture
def adapted():
    from ops_gnn import torch_sparse_spmm as m

    ts, pyg, mods = stub.make("gpu_stub_torch_sparse", "gpu_stub_torch_geometric")
    m.adapt_frontends(ts, pyg)
    yield m, ts, pyg, mods
    for name in mods:
        sys.modules.pop(name, None)
    stub.CALLS.clear()


@pytest.mark.parametrize("storage_kind", ["rowptr", "row_only", "with_metadata"])
def test_sparse_tensor_matmul_reaches_the_kernels(ogn, oracle, adapted, storage_kind):
    m, ts, pyg, mods = adapted
    ptr, col, rng = _graph(seed=7, hub=1500)
    e = col.numel()
    p, c = ptr.to(DEV), col.to(DEV)
    val = torch.from_numpy(rng.random(e, dtype=np.float32)).to(DEV)
    mat = torch.from_numpy(rng.standard_normal((250, 32), dtype=np.float32)).to(DEV)
    meta = {}
    if storage_kind == "rowptr":
        storage = stub.SparseStorage(rowptr=p, col=c, value=val, sparse_sizes=(300, 250))
    elif storage_kind == "row_only":
        row = torch.repeat_interleave(torch.arange(300, device=DEV), p.diff())
        storage = stub.SparseStorage(row=row, col=c, value=val, sparse_sizes=(300, 250))
    else:
        perm = torch.argsort(c, stable=True)
        meta = dict(rowcount=p.diff(), colptr=torch.ops.torch_sparse.ind2ptr(c[perm], 250), csr2csc=perm)
        storage = stub.SparseStorage(rowptr=p, row=torch.repeat_interleave(torch.arange(300, device=DEV), p.diff()),
                                     col=c, value=val, sparse_sizes=(300, 250), **meta)
    a = ts.SparseTensor(storage)
    gold, _ = oracle.spmm_csr(ptr, col, val, mat, "sum")
    scale, _ = oracle.spmm_csr(ptr, col, val.abs(), mat.abs(), "sum")
    assert_sum_close(a @ mat, gold, scale, torch.float32, "SparseTensor @ mat")
    assert_sum_close(ts.matmul(a, mat), gold, scale, torch.float32, "torch_sparse.matmul")
    assert_sum_close(mods[pyg.__name__ + ".nn.conv.gcn_conv"].spmm(a, mat), gold, scale, torch.float32, "PyG")
    vmax = a.spmm(mat, "max")
    gmax, _ = oracle.spmm_csr(ptr, col, val, mat, "max")
    assert_exact(vmax, gmax.astype(np.float32), "SparseTensor.spmm max (values only)")
    assert stub.CALLS == []
    # backward through the frontend reuses / builds the transposed metadata
    mg = mat.clone().requires_grad_(True)
    (a @ mg).sum().backward()
    want = torch.zeros(250, 32, dtype=torch.float64).index_add_(0, col, val.double().cpu().unsqueeze(1).expand(-1, 32))
    torch.testing.assert_close(mg.grad.cpu().double(), want, rtol=1e-5, atol=1e-5)


def test_sparse_tensor_row_checks(ogn, adapted):
    m, ts, pyg, mods = adapted
    row = torch.tensor([0, 2, 1], device=DEV)
    col = torch.tensor([0, 1, 1], device=DEV)
    mat = torch.ones(2, 4, device=DEV)
    a = ts.SparseTensor(stub.SparseStorage(row=row, col=col, value=None, sparse_sizes=(3, 2)))
    with pytest.raises(ValueError, match="sorted"):
        a @ mat
    a = ts.SparseTensor(stub.SparseStorage(row=torch.tensor([0, 1, 5], device=DEV), col=col, sparse_sizes=(3, 2)))
    with pytest.raises(ValueError, match="out of range"):
        a @ mat
    a = ts.SparseTensor(stub.SparseStorage(row=torch.tensor([0, 1, 1], device=DEV), col=col, sparse_sizes=(3, 3)))
    with pytest.raises(ValueError, match="sparse columns must match"):
        a @ mat


def test_coo_spmm_layout_cache_and_gradients(ogn):
    from ops_gnn import torch_sparse_spmm as m

    m.clear_validation_cache()
    rng = np.random.default_rng(8)
    e = 4000
    index = torch.from_numpy(np.stack([rng.integers(0, 120, e), rng.integers(0, 90, e)])).to(DEV)
    value = torch.rand(e, device=DEV, requires_grad=True)
    mat = torch.randn(90, 24, device=DEV, requires_grad=True)
    out = ogn.coo_spmm(index, value, 120, 90, mat)
    assert m.validation_cache_info().coo_entries == 1
    out2 = ogn.coo_spmm(index, value, 120, 90, mat)
    assert m.validation_cache_info().coo_entries == 1
    assert torch.equal(out, out2)
    want = torch.zeros(120, 24, dtype=torch.float64, device=DEV).index_add_(
        0, index[0], value.detach().double().unsqueeze(1) * mat.detach().double()[index[1]])
    torch.testing.assert_close(out.double(), want, rtol=1e-5, atol=1e-5)
    g = torch.randn(120, 24, device=DEV)
    out.backward(g)
    v64 = value.detach().double().requires_grad_(True)
    m64 = mat.detach().double().requires_grad_(True)
    torch.zeros(120, 24, dtype=torch.float64, device=DEV).index_add(
        0, index[0].clone(), v64.unsqueeze(1) * m64[index[1].clone()]).backward(g.double())
    torch.testing.assert_close(value.grad.double(), v64.grad, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(mat.grad.double(), m64.grad, rtol=1e-4, atol=1e-4)
    index.add_(0)                                   # a write bumps the version: new layout
    ogn.coo_spmm(index, value.detach(), 120, 90, mat.detach())
    del index
    import gc

    gc.collect()
    assert m.validation_cache_info().coo_entries == 0  # entries die with their index
