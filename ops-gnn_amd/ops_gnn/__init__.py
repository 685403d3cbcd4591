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
from .segment import (
    segment_csr, segment_sum_csr, segment_add_csr, segment_mean_csr, segment_min_csr, segment_max_csr,
    segment_max_csr_legacy, segment_reduce,
    segment_coo, segment_sum_coo, segment_add_coo, segment_mean_coo, segment_min_coo, segment_max_coo,
    segment_logsumexp,
)
from .scatter import (
    scatter, scatter_sum, scatter_add, scatter_mul, scatter_mean, scatter_min, scatter_max,
)
from .softmax import scatter_softmax, scatter_log_softmax, scatter_logsumexp
from .sddmm_csr import sddmm_csr
from .spmm import spmm, bspmm
from .gather import gather_csr, gather_coo

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
    "segment_csr", "segment_sum_csr", "segment_add_csr", "segment_mean_csr", "segment_min_csr",
    "segment_max_csr", "segment_max_csr_legacy", "segment_reduce",
    "segment_coo", "segment_sum_coo", "segment_add_coo", "segment_mean_coo", "segment_min_coo",
    "segment_max_coo", "segment_logsumexp",
    "scatter", "scatter_sum", "scatter_add", "scatter_mul", "scatter_mean", "scatter_min", "scatter_max",
    "scatter_softmax", "scatter_log_softmax", "scatter_logsumexp",
    "sddmm_csr", "spmm", "bspmm",
    "gather_csr", "gather_coo",
]
