"""Training drop-in: GNN layers built on the ops (forward and every gradient)
against the same layers in plain PyTorch float64 on the CPU.

Follows the reference's PyG layer test (test/torch_sparse_spmm/arch35/
test_torch_sparse_spmm.py:764-794: GCNConv / GINConv over a SparseTensor,
forward, input and parameter gradients at rtol 1e-4 / atol 1e-5).  PyG is
not installed, so the layers are written out: GCN = A (x W) + b, GIN =
MLP((1 + eps) x + A x), and a GAT-style head (edge scores, scatter_softmax
over each row's edges, attention-weighted aggregation) that exercises the
softmax backward and the SpMM value gradient.
"""

import copy

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _graph(n, seed, mean_degree=6):
    rng = np.random.default_rng(seed)
    deg = rng.poisson(mean_degree, n)
    deg[rng.integers(0, n, 3)] = 0
    rowptr = np.concatenate([[0], np.cumsum(deg)])
    col = np.concatenate([np.sort(rng.choice(n, d, replace=False)) for d in deg])
    value = rng.uniform(0.1, 1.0, len(col))
    return torch.from_numpy(rowptr), torch.from_numpy(col), torch.from_numpy(value)


def _dense_aggregate(rowptr, col, value, mat):
    """Reference sum aggregation: out[r] = sum_e value[e] * mat[col[e]]."""
    row = torch.repeat_interleave(torch.arange(len(rowptr) - 1), rowptr[1:] - rowptr[:-1])
    msg = mat[col] * value.unsqueeze(-1)
    return torch.zeros(len(rowptr) - 1, mat.size(-1), dtype=mat.dtype).index_add(0, row, msg)


class GCN(torch.nn.Module):
    def __init__(self, fin, fout):
        super().__init__()
        self.lin = torch.nn.Linear(fin, fout, bias=False)
        self.bias = torch.nn.Parameter(torch.randn(fout) * 0.1)

    def forward(self, x, adj, agg):
        return agg(*adj, self.lin(x)) + self.bias


class GIN(torch.nn.Module):
    def __init__(self, fin, fout):
        super().__init__()
        self.mlp = torch.nn.Sequential(torch.nn.Linear(fin, 12), torch.nn.ReLU(), torch.nn.Linear(12, fout))
        self.eps = torch.nn.Parameter(torch.tensor(0.25))

    def forward(self, x, adj, agg):
        rowptr, col, value = adj
        return self.mlp((1 + self.eps) * x + agg(rowptr, col, torch.ones_like(value), x))


class GATHead(torch.nn.Module):
    def __init__(self, fin, fout):
        super().__init__()
        self.lin = torch.nn.Linear(fin, fout, bias=False)
        self.att_src = torch.nn.Parameter(torch.randn(fout) * 0.3)
        self.att_dst = torch.nn.Parameter(torch.randn(fout) * 0.3)

    def forward(self, x, adj, agg, softmax):
        rowptr, col, _ = adj
        h = self.lin(x)
        row = torch.repeat_interleave(torch.arange(len(rowptr) - 1, device=x.device), rowptr[1:] - rowptr[:-1])
        score = torch.nn.functional.leaky_relu((h * self.att_dst).sum(-1)[row] + (h * self.att_src).sum(-1)[col], 0.2)
        alpha = softmax(score, row, len(rowptr) - 1)
        return agg(rowptr, col, alpha, h)


def _ref_softmax(score, row, n):
    out = torch.empty_like(score)
    for r in torch.unique(row).tolist():
        sel = row == r
        out[sel] = torch.softmax(score[sel], 0)
    return out


@pytest.mark.parametrize("kind", ["gcn", "gin", "gat"])
def test_layer_forward_and_gradients(ogn, kind):
    torch.manual_seed(123)
    n, fin, fout = 300, 8, 5
    rowptr, col, value = _graph(n, 5)
    cls = {"gcn": GCN, "gin": GIN, "gat": GATHead}[kind]
    ref = cls(fin, fout).double()
    dut = copy.deepcopy(ref).float().cuda()
    x = torch.randn(n, fin, dtype=torch.float64, requires_grad=True)
    xd = x.detach().float().cuda().requires_grad_()
    adj_ref = (rowptr, col, value)
    adj_dut = (rowptr.cuda(), col.cuda(), value.float().cuda())

    def agg(p, c, v, m):
        return ogn.csr_spmm(p, c, v, m, "sum")

    def sm(score, row, size):
        return ogn.scatter_softmax(score, row, dim=0, dim_size=size)

    if kind == "gat":
        expected = ref(x, adj_ref, _dense_aggregate, _ref_softmax)
        actual = dut(xd, adj_dut, agg, sm)
    else:
        expected = ref(x, adj_ref, _dense_aggregate)
        actual = dut(xd, adj_dut, agg)
    torch.testing.assert_close(actual.double().cpu(), expected, rtol=1e-4, atol=1e-5)
    expected.square().sum().backward()
    actual.square().sum().backward()
    torch.testing.assert_close(xd.grad.double().cpu(), x.grad, rtol=1e-4, atol=1e-5)
    for (name, a), b in zip(dut.named_parameters(), ref.parameters()):
        torch.testing.assert_close(a.grad.double().cpu(), b.grad, rtol=1e-4, atol=1e-5, msg=name)


def test_gcn_training_loop_tracks_reference(ogn):
    # a few SGD steps: the GPU model follows the float64 CPU model
    torch.manual_seed(7)
    n, fin, fout = 500, 16, 4
    rowptr, col, value = _graph(n, 9)
    ref = GCN(fin, fout).double()
    dut = copy.deepcopy(ref).float().cuda()
    x = torch.randn(n, fin, dtype=torch.float64)
    target = torch.randn(n, fout, dtype=torch.float64)
    opt_r = torch.optim.SGD(ref.parameters(), lr=1e-3)
    opt_d = torch.optim.SGD(dut.parameters(), lr=1e-3)
    adj_d = (rowptr.cuda(), col.cuda(), value.float().cuda())
    losses = []
    for _ in range(5):
        opt_r.zero_grad()
        opt_d.zero_grad()
        lr_ = (ref(x, (rowptr, col, value), _dense_aggregate) - target).square().mean()
        ld = (dut(x.float().cuda(), adj_d, lambda p, c, v, m: ogn.csr_spmm(p, c, v, m, "sum"))
              - target.float().cuda()).square().mean()
        lr_.backward()
        ld.backward()
        opt_r.step()
        opt_d.step()
        losses.append((lr_.item(), ld.item()))
    for a, b in losses:
        assert abs(a - b) <= 1e-5 * max(1.0, abs(a))
    assert losses[-1][1] < losses[0][1]
