"""GPU parity of sddmm_csr, the DGL-style spmm / bspmm and the SpMM autograd
paths against the oracle (reference test/sddmm_csr/arch22/test_sddmm_csr.py,
test/spmm_*/arch22, test/unified_spmm/arch22, and the gradient tests of
test/torch_sparse_spmm/arch35/test_torch_sparse_spmm.py:480-516)."""

import numpy as np
import pytest
import torch

from _util import assert_sum_close, cast_like

pytestmark = pytest.mark.gpu

DT = [torch.float32, torch.float16, torch.bfloat16]
TOL = {torch.float32: 1e-5, torch.float16: 1e-2, torch.bfloat16: 1e-2}


def _csr(m, n, avg, seed, hub=0):
    rng = np.random.default_rng(seed)
    deg = rng.poisson(avg, size=m)
    deg[::7] = 0
    if hub:
        deg[1] = hub
    col = np.concatenate([np.sort(rng.integers(0, n, d)) for d in deg]).astype(np.int64)
    return torch.from_numpy(np.concatenate([[0], np.cumsum(deg)]).astype(np.int64)), torch.from_numpy(col), rng


# ----------------------------------------------------------------- sddmm
@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("k", [1, 5, 8, 64, 100, 128])
def test_sddmm_dot(ogn, oracle, dtype, k):
    ptr, col, rng = _csr(400, 300, 12, seed=k, hub=3000)
    q = torch.from_numpy(rng.standard_normal((400, k)).astype(np.float32)).to(dtype)
    kk = torch.from_numpy(rng.standard_normal((300, k)).astype(np.float32)).to(dtype)
    got = ogn.sddmm_csr(ptr.cuda(), col.cuda(), q.cuda(), kk.cuda())
    gold = oracle.sddmm(ptr, col, q, kk, "dot", 0, 2)
    scale = oracle.sddmm(ptr, col, q.float().abs(), kk.float().abs(), "dot", 0, 2)
    assert got.shape == (col.numel(),) and got.dtype == dtype
    assert_sum_close(got, gold, scale, dtype, f"dot/{dtype}/k{k}")


@pytest.mark.parametrize("op", ["add", "sub", "mul", "div", "copy_lhs", "copy_rhs"])
@pytest.mark.parametrize("lt,rt", [(0, 2), (2, 0), (1, 2), (0, 1)])
def test_sddmm_ops_and_targets(ogn, oracle, op, lt, rt):
    ptr, col, rng = _csr(60, 50, 5, seed=3)
    nnz = col.numel()
    rows = {0: 60, 1: nnz, 2: 50}
    lhs = torch.from_numpy(rng.standard_normal((rows[lt], 16)).astype(np.float32))
    rhs = torch.from_numpy((rng.standard_normal((rows[rt], 16)) + 3).astype(np.float32))
    args = dict(lhs=None if op == "copy_rhs" else lhs.cuda(), rhs=None if op == "copy_lhs" else rhs.cuda())
    got = ogn.sddmm_csr(ptr.cuda(), col.cuda(), op=op, lhs_target=lt, rhs_target=rt, **args)
    gold = oracle.sddmm(ptr, col, lhs if op != "copy_rhs" else None, rhs if op != "copy_lhs" else None, op, lt, rt)
    np.testing.assert_allclose(got.cpu().numpy(), gold, rtol=1e-6, atol=1e-6)


def test_sddmm_aliases_1d_operands_and_out(ogn, oracle):
    ptr, col, rng = _csr(30, 20, 4, seed=4)
    lhs = torch.from_numpy(rng.standard_normal(30).astype(np.float32))
    rhs = torch.from_numpy(rng.standard_normal(20).astype(np.float32))
    got = ogn.sddmm_csr(ptr.cuda(), col.cuda(), lhs.cuda(), rhs.cuda(), op="add", lhs_target="u", rhs_target="v")
    assert got.shape == (col.numel(),)
    np.testing.assert_allclose(got.cpu().numpy(), oracle.sddmm(ptr, col, lhs, rhs, "add", 0, 2)[:, 0], rtol=1e-6)
    out = torch.empty(col.numel(), device="cuda")
    res = ogn.sddmm_csr(ptr.cuda(), col.cuda(), lhs.cuda(), rhs.cuda(), "dot", "src", "dst", out=out)
    assert res.data_ptr() == out.data_ptr()


def test_sddmm_int32_and_special_values(ogn, oracle):
    # reference test/sddmm_csr/arch22/test_sddmm_csr.py:253-269
    ptr = torch.tensor([0, 2, 4, 5])
    idx = torch.tensor([0, 1, 1, 0, 0])
    lhs = torch.tensor([[float("inf"), float("nan"), 1, -2], [-float("inf"), 3, 4, float("nan")],
                        [0, 1, -1, 2], [float("nan"), -3, 5, 6]])
    rhs = torch.tensor([[1, 0, float("inf"), -3], [2, float("nan"), -4, 5], [0, -1, 2, float("nan")],
                        [3, 4, 5, 6]], dtype=torch.float32)
    for op in ("dot", "add", "div"):
        got = ogn.sddmm_csr(ptr.int().cuda(), idx.int().cuda(), lhs.cuda(), rhs.cuda(), op=op)
        gold = oracle.sddmm(ptr, idx, lhs, rhs, op, 0, 2)
        np.testing.assert_allclose(got.cpu().numpy(), gold, rtol=1e-6, equal_nan=True)


@pytest.mark.parametrize("ptr_values,index_values", [
    # reference test/sddmm_csr/arch22/test_sddmm_csr.py:291-302
    ([1, 1], [0]), ([0, 2], [0]), ([0, 2, 1, 2], [0, 0]), ([0, -1, 1], [0]), ([0, 1], [-1]), ([0, 1], [4]),
    ([0, 1], [2**32]),
])
def test_sddmm_bad_csr(ogn, ptr_values, index_values):
    lhs = torch.ones(4, 3, device="cuda")
    with pytest.raises(RuntimeError, match="sddmm_csr"):
        ogn.sddmm_csr(torch.tensor(ptr_values, device="cuda"), torch.tensor(index_values, device="cuda"), lhs, lhs)


# ----------------------------------------------------------------- DGL spmm / bspmm
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("reduce", ["sum", "mean", "max", "min"])
@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64])
def test_dgl_copy_lhs(ogn, oracle, dtype, reduce, index_dtype):
    ptr, col, rng = _csr(500, 400, 9, seed=5, hub=5000)
    x = torch.from_numpy(rng.standard_normal((400, 64)).astype(np.float32)).to(dtype)
    x[3, 5] = float("nan")
    got = ogn.spmm(ptr.to(index_dtype).cuda(), col.to(index_dtype).cuda(), x.cuda(), reduce=reduce)
    gold = oracle.spmm_dgl(ptr, col, x, None, "copy_lhs", reduce)
    if reduce in ("max", "min"):
        g = got.float().cpu().numpy()
        np.testing.assert_array_equal(np.isnan(g), np.isnan(gold))
        np.testing.assert_array_equal(g[~np.isnan(g)], cast_like(gold, dtype)[~np.isnan(g)])
    else:
        scale = oracle.spmm_dgl(ptr, col, x.float().abs(), None, "copy_lhs", reduce)
        assert_sum_close(got, gold, scale, dtype, f"dgl/{reduce}")


# copy_rhs aggregates the edge features as given: only the full edge shape
_MSG_CASES = [(op, shape) for op in ("add", "sub", "mul", "div") for shape in ("scalar", "column", "full")] + \
    [("copy_rhs", "full")]


@pytest.mark.parametrize("op,edge_shape", _MSG_CASES)
@pytest.mark.parametrize("reduce", ["sum", "mean", "max", "min"])
def test_dgl_binary_messages(ogn, oracle, op, reduce, edge_shape):
    ptr, col, rng = _csr(200, 150, 6, seed=6)
    nnz = col.numel()
    x = torch.from_numpy(rng.standard_normal((150, 8)).astype(np.float32))
    w_full = torch.from_numpy((rng.standard_normal((nnz, 8)) + 3).astype(np.float32))
    w = {"scalar": w_full[:, 0].contiguous(), "column": w_full[:, :1].contiguous(), "full": w_full}[edge_shape]
    if op == "copy_rhs":
        got = ogn.spmm(ptr.cuda(), col.cuda(), None, op="copy_rhs", reduce=reduce, rhs=w.cuda())
        gold = oracle.spmm_dgl(ptr, col, None, w, "copy_rhs", reduce)
    else:
        got = ogn.spmm(ptr.cuda(), col.cuda(), x.cuda(), op, reduce, rhs=w.cuda())
        gold = oracle.spmm_dgl(ptr, col, x, w, op, reduce)
    if reduce in ("max", "min"):
        np.testing.assert_array_equal(got.cpu().numpy(), gold.astype(np.float32))
    else:
        abs_op = {"add": "add", "sub": "add", "mul": "mul", "div": "div", "copy_rhs": "copy_rhs"}[op]
        scale = oracle.spmm_dgl(ptr, col, None if op == "copy_rhs" else x.abs(), w.abs(), abs_op, reduce)
        assert_sum_close(got, gold, scale, torch.float32, f"{op}/{reduce}/{edge_shape}")


def test_bspmm_rank3(ogn, oracle):
    # reference test/conftest.py:150-170 (assert_bspmm_case layout)
    ptr = torch.tensor([0, 0, 3, 4])
    idx = torch.tensor([0, 2, 1, 2])
    base = (torch.arange(3 * 17 * 2).reshape(3, 17, 2) % 7) - 3
    x = base.transpose(1, 2).to(torch.float16)  # [3, 2, 17]
    for reduce in ("sum", "max", "min", "mean"):
        out = torch.empty((3, 2, 17), dtype=torch.float16, device="cuda")
        res = ogn.bspmm(ptr.cuda(), idx.cuda(), x.cuda(), reduce=reduce, out=out)
        assert res.data_ptr() == out.data_ptr()
        gold = oracle.spmm_dgl(ptr, idx, x.reshape(3, 34), None, "copy_lhs", reduce).reshape(3, 2, 17)
        np.testing.assert_allclose(res.float().cpu().numpy(), gold, rtol=1e-3, atol=1e-3)


def test_dgl_errors(ogn):
    ptr = torch.tensor([0, 1, 2], device="cuda")
    idx = torch.tensor([0, 1], device="cuda")
    x = torch.ones(2, 17, device="cuda")
    with pytest.raises(RuntimeError, match="op must be"):
        ogn.spmm(ptr, idx, x, op="pow")
    with pytest.raises(RuntimeError, match="reduce must be"):
        ogn.spmm(ptr, idx, x, reduce="prod")
    with pytest.raises(RuntimeError, match="bspmm"):
        ogn.spmm(ptr, idx, x.reshape(2, 1, 17))
    with pytest.raises(RuntimeError, match="out of range"):
        ogn.spmm(ptr, torch.tensor([0, 5], device="cuda"), x)
    with pytest.raises(RuntimeError, match="start at zero"):
        ogn.spmm(torch.tensor([1, 1, 2], device="cuda"), idx, x)
    with pytest.raises(ValueError, match="requires both"):
        ogn.spmm(ptr, idx, x, op="mul")


# ----------------------------------------------------------------- autograd
def _dense_grads(ptr, col, val, mat, g, reduce):
    """Library reference: torch.sparse CSR (fp64, CPU) autograd."""
    m, n = ptr.numel() - 1, mat.size(0)
    v = val.double().clone().requires_grad_(True)
    x = mat.double().clone().requires_grad_(True)
    rows = torch.repeat_interleave(torch.arange(m), ptr[1:] - ptr[:-1])
    a = torch.zeros(m, n, dtype=torch.float64).index_put((rows, col), v, accumulate=True)
    out = a @ x
    if reduce == "mean":
        out = out / (ptr[1:] - ptr[:-1]).clamp_min(1).double().unsqueeze(-1)
    (out * g.double()).sum().backward()
    return v.grad, x.grad


@pytest.mark.parametrize("reduce", ["sum", "mean"])
def test_torch_sparse_backward(ogn, reduce):
    ptr, col, rng = _csr(80, 60, 5, seed=7)
    val = torch.from_numpy(rng.standard_normal(col.numel()).astype(np.float32))
    mat = torch.from_numpy(rng.standard_normal((60, 16)).astype(np.float32))
    g = torch.from_numpy(rng.standard_normal((80, 16)).astype(np.float32))
    v = val.cuda().requires_grad_(True)
    x = mat.cuda().requires_grad_(True)
    out = ogn.csr_spmm(ptr.cuda(), col.cuda(), v, x, reduce)
    out.backward(g.cuda())
    dv, dx = _dense_grads(ptr, col, val, mat, g, reduce)
    np.testing.assert_allclose(v.grad.cpu().numpy(), dv.numpy(), rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(x.grad.cpu().numpy(), dx.numpy(), rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("reduce", ["sum", "mean"])
@pytest.mark.parametrize("op", ["copy_lhs", "mul"])
def test_dgl_backward(ogn, reduce, op):
    ptr, col, rng = _csr(70, 50, 4, seed=8)
    val = torch.from_numpy(rng.standard_normal(col.numel()).astype(np.float32))
    mat = torch.from_numpy(rng.standard_normal((50, 8)).astype(np.float32))
    g = torch.from_numpy(rng.standard_normal((70, 8)).astype(np.float32))
    x = mat.cuda().requires_grad_(True)
    w = val.cuda().requires_grad_(True) if op == "mul" else None
    out = ogn.spmm(ptr.cuda(), col.cuda(), x, op, reduce, rhs=w)
    out.backward(g.cuda())
    dv, dx = _dense_grads(ptr, col, val if op == "mul" else torch.ones(col.numel()), mat, g, reduce)
    np.testing.assert_allclose(x.grad.cpu().numpy(), dx.numpy(), rtol=1e-4, atol=1e-4)
    if w is not None:
        np.testing.assert_allclose(w.grad.cpu().numpy(), dv.numpy(), rtol=1e-4, atol=1e-4)


def _torch_composition(ptr, col, x, w, op, reduce):
    """The reference's torch composition (python/ops_gnn/spmm.py:148-208) in
    float64 on the CPU: gather, message op with rank alignment, then
    index_add (sum / mean) or per-row max / min over dim 0."""
    m = ptr.numel() - 1
    gathered = None if x is None else x.index_select(0, col)
    if op == "copy_lhs":
        msg = gathered
    elif op == "copy_rhs":
        msg = w
    else:
        rank = max(gathered.dim(), w.dim()) - 1
        pad = lambda v: v.reshape((v.shape[0],) + (1,) * (rank - v.dim() + 1) + tuple(v.shape[1:]))
        a, b = pad(gathered), pad(w)
        msg = {"add": a + b, "sub": a - b, "mul": a * b, "div": a / b}[op]
    counts = ptr.diff()
    if reduce in ("sum", "mean"):
        rows = torch.repeat_interleave(torch.arange(m), counts)
        out = msg.new_zeros((m,) + tuple(msg.shape[1:])).index_add(0, rows, msg)
        if reduce == "mean":
            out = out / counts.clamp(min=1).to(out.dtype).reshape((m,) + (1,) * (msg.dim() - 1))
        return out
    parts = []
    for r in range(m):
        a, b = int(ptr[r]), int(ptr[r + 1])
        if a == b:
            parts.append(msg.new_zeros(msg.shape[1:]))
        else:
            seg = msg[a:b]
            parts.append(seg.max(dim=0).values if reduce == "max" else seg.min(dim=0).values)
    return torch.stack(parts)


_GRAD_CASES = [
    # (op, x feature shape, w feature shape, batched)
    ("copy_lhs", (6,), None, False),
    ("copy_rhs", None, (6,), False),
    ("add", (6,), (6,), False),
    ("sub", (6,), (1,), False),
    ("mul", (6,), (), False),
    ("div", (6,), (6,), False),
    ("mul", (3, 4), (3, 1), True),
    ("add", (1, 4), (3, 4), True),
    ("div", (3, 4), (), True),
    ("copy_lhs", (2, 5), None, True),
]


@pytest.mark.parametrize("op,xs,ws,batched", _GRAD_CASES)
@pytest.mark.parametrize("reduce", ["sum", "mean", "max", "min"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_dgl_gradients_every_op_and_reduce(ogn, op, xs, ws, batched, reduce, dtype):
    """spmm / bspmm gradients for every message op and reduction, against
    float64 autograd through the reference's composition (no ties: random
    continuous data, divisors kept away from zero)."""
    ptr, col, rng = _csr(90, 70, 5, seed=17, hub=60)
    e = col.numel()
    x64 = None if xs is None else torch.from_numpy(rng.standard_normal((70,) + xs))
    w64 = None if ws is None else torch.from_numpy(rng.uniform(0.5, 2.0, (e,) + ws)
                                                   * rng.choice([-1.0, 1.0], (e,) + ws))
    if dtype == torch.float16:  # compare on the exact fp16 inputs
        x64 = None if x64 is None else x64.half().double()
        w64 = None if w64 is None else w64.half().double()
    leaves = [t.clone().requires_grad_(True) for t in (x64, w64) if t is not None]
    x_ref = leaves[0] if x64 is not None else None
    w_ref = leaves[-1] if w64 is not None else None
    ref = _torch_composition(ptr, col, x_ref, w_ref, op, reduce)
    g = torch.from_numpy(rng.standard_normal(tuple(ref.shape)))
    ref.backward(g)
    xg = None if x64 is None else x64.to(dtype).cuda().requires_grad_(True)
    wg = None if w64 is None else w64.to(dtype).cuda().requires_grad_(True)
    fn = ogn.bspmm if batched else ogn.spmm
    if op == "copy_rhs":
        out = fn(ptr.cuda(), col.cuda(), None, op=op, reduce=reduce, rhs=wg)
    else:
        out = fn(ptr.cuda(), col.cuda(), xg, op=op, reduce=reduce, rhs=wg)
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    torch.testing.assert_close(out.double().cpu(), ref.detach(), rtol=tol, atol=tol)
    out.backward(g.to(dtype).cuda())
    if xg is not None:
        torch.testing.assert_close(xg.grad.double().cpu(), x_ref.grad, rtol=tol, atol=tol)
    if wg is not None:
        torch.testing.assert_close(wg.grad.double().cpu(), w_ref.grad, rtol=tol, atol=tol)
