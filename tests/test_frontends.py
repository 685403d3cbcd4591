"""Host logic of the torch_sparse / PyG frontend adaptation and the proof
caches (CPU; no kernel runs).  The GPU half (real SparseTensor @ GPU dense
through the kernels) is in test_spmm_gpu.py.

Routing follows the reference's adaptation (python/ops_gnn/torch_sparse_spmm.py
:345-459): GPU dense operands go to this package, everything else to the
original frontend; a second adaptation (module reload) never wraps an adapter.
"""

import sys

import pytest
import torch

import _stub_frontends as stub


@pytest.fixture
def tss(monkeypatch):
    from ops_gnn import torch_sparse_spmm as m

    ts, pyg, mods = stub.make()
    yield m, ts, pyg, mods
    for name in mods:
        sys.modules.pop(name, None)
    stub.CALLS.clear()


def _sparse(ts):
    ptr = torch.tensor([0, 2, 3])
    col = torch.tensor([0, 1, 1])
    return ts.SparseTensor(stub.SparseStorage(rowptr=ptr, col=col, value=torch.ones(3), sparse_sizes=(2, 2)))


def test_cpu_operands_keep_the_original_frontends(tss):
    m, ts, pyg, mods = tss
    assert m.adapt_frontends(ts, pyg)
    a = _sparse(ts)
    dense = torch.ones(2, 3)
    assert a @ dense == "original"
    assert a.spmm(dense, "max") == "original"
    assert a.matmul(dense) == "original"
    assert ts.matmul(a, dense, "mean") == "original"
    assert mods[ts.__name__ + ".matmul"].spmm(a, dense) == "original"
    assert ts.spmm(torch.zeros(2, 3, dtype=torch.long), None, 2, 2, dense) == "original"
    assert mods[pyg.__name__ + ".nn.conv.gcn_conv"].spmm(a, dense) == "original"
    assert mods[pyg.__name__ + ".utils"].spmm(a, dense) == "original"
    kinds = [c[0] for c in stub.CALLS]
    assert kinds == ["SparseTensor.__matmul__", "SparseTensor.spmm", "SparseTensor.matmul", "matmul.matmul",
                     "matmul.spmm", "torch_sparse.spmm", "pyg.spmm", "pyg.spmm"]


def test_gpu_operands_reach_this_package(tss, monkeypatch):
    m, ts, pyg, mods = tss
    m.adapt_frontends(ts, pyg)
    seen = []
    monkeypatch.setattr(m, "_on_gpu", lambda t: isinstance(t, torch.Tensor))
    monkeypatch.setattr(m, "_sparse_tensor_spmm", lambda src, other, reduce="sum": seen.append(("csr", reduce)) or "ours")
    monkeypatch.setattr(m, "coo_spmm", lambda *a: seen.append(("coo",)) or "ours")
    a = _sparse(ts)
    dense = torch.ones(2, 3)
    assert a @ dense == "ours"
    assert a.spmm(dense, "max") == "ours"
    assert a.matmul(dense, "min") == "ours"
    assert ts.matmul(a, dense) == "ours"
    assert ts.spmm(torch.zeros(2, 3, dtype=torch.long), None, 2, 2, dense) == "ours"
    assert mods[ts.__name__ + ".spmm"].spmm(torch.zeros(2, 3, dtype=torch.long), None, 2, 2, dense) == "ours"
    for alias in (".utils", ".utils._spmm", ".nn.conv.gcn_conv", ".nn.conv.gin_conv"):
        assert mods[pyg.__name__ + alias].spmm(a, dense) == "ours"
    # PyG adapts only SparseTensor sources; anything else stays with PyG
    assert mods[pyg.__name__ + ".nn.conv.gin_conv"].spmm(torch.ones(2, 2), dense) == "original"
    assert [s[0] for s in seen] == ["csr"] * 4 + ["coo"] * 2 + ["csr"] * 4
    assert [s[1] for s in seen[:4]] == ["sum", "max", "min", "sum"]
    assert stub.CALLS == [("pyg.spmm", "sum")]


def test_second_adaptation_wraps_the_original_not_the_adapter(tss):
    m, ts, pyg, mods = tss
    m.adapt_frontends(ts, pyg)
    first = ts.SparseTensor.__matmul__
    m.adapt_frontends(ts, pyg)
    second = ts.SparseTensor.__matmul__
    assert first is not second
    assert second.__ops_gnn_original__ is first.__ops_gnn_original__
    assert second.__ops_gnn_original__ is stub.SparseTensor.__matmul__
    assert _sparse(ts) @ torch.ones(2, 1) == "original"
    assert len(stub.CALLS) == 1


def test_absent_torch_sparse_is_not_adapted():
    from ops_gnn import torch_sparse_spmm as m

    if "torch_sparse" in sys.modules:
        pytest.skip("a real torch_sparse is installed")
    assert m.adapt_frontends() is False


def test_coo_spmm_on_cpu_without_torch_sparse_raises():
    from ops_gnn import torch_sparse_spmm as m

    m._ORIGINALS.pop("torch_sparse.spmm", None)
    with pytest.raises(ValueError, match="GPU"):
        m.coo_spmm(torch.zeros(2, 1, dtype=torch.long), None, 1, 1, torch.ones(1, 2))


def test_proof_cache_hits_misses_and_release():
    from ops_gnn.torch_sparse_spmm import _MISS, _ProofCache

    cache = _ProofCache(2)
    a, b = torch.arange(4), torch.arange(5)
    cache.store((a, b), (7,), "ab")
    assert cache.lookup((a, b), (7,)) == "ab"
    assert cache.lookup((a, b), (8,)) is _MISS          # other parameters
    assert cache.lookup((b, a), (7,)) is _MISS          # other order
    a.add_(1)                                           # version bump
    assert cache.lookup((a, b), (7,)) is _MISS
    c = torch.arange(3)
    cache.store((c,), (), "c")
    assert len(cache) == 2
    del c                                               # freed tensor -> entry gone
    assert len(cache) == 1
    cache.store((a,), (), "a1")
    cache.store((b,), (), "b1")
    assert len(cache) == 2                              # capacity bound (LRU)
    with torch.inference_mode():
        inf = torch.arange(3)
    cache.store((inf,), (), "never")                    # no version counter: not cached
    assert cache.lookup((inf,), ()) is _MISS
    view = a[:2]
    cache.store((view,), (), "view")
    assert cache.lookup((a[:2],), ()) is _MISS          # a new view object is a new identity
