"""Minimal stand-ins for the torch_sparse and PyG frontends (neither is
installed here), shaped like the parts the adaptation touches:

- ``torch_sparse.SparseTensor`` whose ``storage`` answers ``has_*()`` and
  ``rowptr() / row() / col() / value() / rowcount() / colptr() / csr2csc()``
  (rowptr built lazily from row through ``torch.ops.torch_sparse.ind2ptr``,
  as torch_sparse's SparseStorage does);
- module functions ``torch_sparse.spmm`` (COO), ``torch_sparse.matmul``,
  ``torch_sparse.matmul.{spmm, matmul}``, ``torch_sparse.spmm.spmm``;
- ``torch_geometric.utils.spmm`` / ``utils._spmm.spmm`` and the aliases in
  ``nn.conv.gcn_conv`` / ``gin_conv``.

The original implementations only record their calls (``CALLS``), so tests
can tell which path a call took.
"""

import sys
import types

import torch

CALLS = []


class SparseStorage:
    def __init__(self, rowptr=None, row=None, col=None, value=None, sparse_sizes=None, **meta):
        self._rowptr, self._row, self._col, self._value = rowptr, row, col, value
        self._meta = meta
        self.sparse_sizes = sparse_sizes

    def has_rowptr(self):
        return self._rowptr is not None

    def has_row(self):
        return self._row is not None

    def rowptr(self):
        if self._rowptr is None:
            self._rowptr = torch.ops.torch_sparse.ind2ptr(self._row, self.sparse_sizes[0])
        return self._rowptr

    def row(self):
        return self._row

    def col(self):
        return self._col

    def value(self):
        return self._value

    def has_value(self):
        return self._value is not None


for _name in ("rowcount", "colptr", "csr2csc"):
    setattr(SparseStorage, "has_" + _name, lambda self, n=_name: self._meta.get(n) is not None)
    setattr(SparseStorage, _name, lambda self, n=_name: self._meta.get(n))


class SparseTensor:
    def __init__(self, storage):
        self.storage = storage

    def sparse_size(self, dim):
        return self.storage.sparse_sizes[dim]

    def spmm(self, other, reduce="sum"):
        CALLS.append(("SparseTensor.spmm", reduce))
        return "original"

    def matmul(self, other, reduce="sum"):
        CALLS.append(("SparseTensor.matmul", reduce))
        return "original"

    def __matmul__(self, other):
        CALLS.append(("SparseTensor.__matmul__",))
        return "original"


def make(prefix="stub_torch_sparse", pyg_prefix="stub_torch_geometric"):
    """Fresh stub packages registered in sys.modules under the given names."""
    ts = types.ModuleType(prefix)
    ts.__path__ = []
    mm = types.ModuleType(prefix + ".matmul")
    coo = types.ModuleType(prefix + ".spmm")

    def coo_spmm(index, value, m, n, matrix):
        CALLS.append(("torch_sparse.spmm", m, n))
        return "original"

    def mm_spmm(src, other, reduce="sum"):
        CALLS.append(("matmul.spmm", reduce))
        return "original"

    def mm_matmul(src, other, reduce="sum"):
        CALLS.append(("matmul.matmul", reduce))
        return "original"

    coo.spmm = coo_spmm
    mm.spmm, mm.matmul = mm_spmm, mm_matmul
    ts.spmm, ts.matmul = coo_spmm, mm_matmul
    ts.SparseTensor = type("SparseTensor", (SparseTensor,), {})
    ts.SparseStorage = SparseStorage

    pyg = types.ModuleType(pyg_prefix)
    pyg.__path__ = []
    utils = types.ModuleType(pyg_prefix + ".utils")
    utils.__path__ = []
    inner = types.ModuleType(pyg_prefix + ".utils._spmm")
    nn = types.ModuleType(pyg_prefix + ".nn")
    nn.__path__ = []
    conv = types.ModuleType(pyg_prefix + ".nn.conv")
    conv.__path__ = []

    def pyg_spmm(src, other, reduce="sum"):
        CALLS.append(("pyg.spmm", reduce))
        return "original"

    inner.spmm = utils.spmm = pyg_spmm
    mods = {prefix: ts, prefix + ".matmul": mm, prefix + ".spmm": coo, pyg_prefix: pyg,
            pyg_prefix + ".utils": utils, pyg_prefix + ".utils._spmm": inner, pyg_prefix + ".nn": nn,
            pyg_prefix + ".nn.conv": conv}
    for name in ("gcn_conv", "gin_conv"):
        m = types.ModuleType(f"{pyg_prefix}.nn.conv.{name}")
        m.spmm = pyg_spmm
        mods[m.__name__] = m
    sys.modules.update(mods)
    return ts, pyg, mods
