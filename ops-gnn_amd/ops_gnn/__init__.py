"""ops_gnn for AMD MI355X (gfx950): the sparse message-passing hot path of
ops-gnn -- CSR SpMM, SDDMM, segment / scatter reductions, grouped softmax and
index conversions -- as hand-written HIP kernels behind a C ABI
(include/ogn.h, libogn_hip.so).

Public names and argument contracts follow the reference package
(python/ops_gnn/__init__.py:44-174).  Tensors live on the torch "cuda" device
(HIP on ROCm).  Importing this package registers the ``torch_sparse::spmm_*``,
``ind2ptr`` and ``ptr2ind`` operators for the CUDA dispatch keys.
"""

from . import _lib
from ._lib import arch
from .convert import ind2ptr, ptr2ind
from . import torch_sparse_spmm
from .torch_sparse_spmm import csr_spmm, coo_spmm, coo_to_csr

__version__ = "0.1.0"

native_available = True

__all__ = [
    "arch",
    "ind2ptr",
    "ptr2ind",
    "csr_spmm",
    "coo_spmm",
    "coo_to_csr",
    "torch_sparse_spmm",
    "native_available",
]
