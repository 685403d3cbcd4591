"""Tensor-level wrappers over the C ABI -- the counterpart of the reference's
pybind module ``_pybind`` (reference csrc/pybind.cpp:92-349).

Each function takes torch tensors, checks what the kernel assumes (device,
dtype, contiguity, shapes), allocates outputs and workspaces with torch's
caching allocator, and launches on torch's current stream.  ctypes drops the
GIL for the duration of each foreign call, matching the reference's
``py::gil_scoped_release`` guards.
"""

import math
from typing import Optional, Tuple

import torch

from . import _lib
from ._lib import check, dptr, lib, stream_of

SPMM_INPUT_DTYPES = (torch.float32, torch.float16, torch.bfloat16)
SPMM_OUTPUT_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def _index_code(t: torch.Tensor) -> int:
    if t.dtype == torch.int64:
        return _lib.I64
    if t.dtype == torch.int32:
        return _lib.I32
    raise ValueError("index tensors must be int32 or int64")


def validate_csr(ptr: torch.Tensor, col: torch.Tensor, n: int) -> torch.Tensor:
    """Device CSR check; returns an int32 [1] status tensor (0 ok, 1 bad rowptr,
    2 column out of range).  Reference TorchSparseSpmmValidate
    (csrc/npu/torch_sparse_spmm/op_host/torch_sparse_spmm.cpp:136-147)."""
    ptr = ptr.contiguous()
    col = col.contiguous()
    if col.dtype != ptr.dtype:
        col = col.to(ptr.dtype)
    status = torch.empty(1, dtype=torch.int32, device=ptr.device)
    m = ptr.numel() - 1
    if m < 0:
        status.fill_(1)
        return status
    rc = lib.ogn_validate_csr(dptr(ptr), dptr(col), _index_code(ptr), m, col.numel(), int(n),
                              dptr(status), stream_of(ptr))
    check(rc, "validate_csr")
    return status


def spmm_forward(ptr: torch.Tensor, col: torch.Tensor, value: Optional[torch.Tensor],
                 mat: torch.Tensor, reduce: int, out_dtype: torch.dtype,
                 out: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Weighted CSR SpMM; reference TorchSparseSpmmForward
    (csrc/npu/torch_sparse_spmm/op_host/torch_sparse_spmm.cpp:97-135).

    mat [..., N, K]; value None / [E] / [E, K] (any trailing shape of width 1
    or K); returns (out [..., M, K], arg [..., M, K] int64 for min/max, else an
    empty int64 tensor).
    """
    if mat.dtype not in SPMM_INPUT_DTYPES:
        raise ValueError("mat must be float32, float16 or bfloat16")
    if out_dtype not in SPMM_OUTPUT_DTYPES:
        raise ValueError("unsupported output dtype")
    mat = mat.contiguous()
    ptr = ptr.contiguous()
    col = col.contiguous()
    if col.dtype != ptr.dtype:
        col = col.to(ptr.dtype)
    m = ptr.numel() - 1
    n, k = mat.size(-2), mat.size(-1)
    lead = tuple(mat.shape[:-2])
    batch = math.prod(lead)
    nnz = col.numel()
    width = 1
    if value is not None:
        value = value.contiguous()
        width = value.numel() // nnz if nnz else 1
    shape = lead + (m, k)
    if out is None:
        out = torch.empty(shape, dtype=out_dtype, device=mat.device)
    minmax = reduce >= 2
    arg = torch.empty(shape if minmax else (0,), dtype=torch.int64, device=mat.device)
    if out.numel() == 0:
        return out, arg
    ws_bytes = lib.ogn_spmm_csr_workspace_size(m, nnz, k, batch, _lib.TORCH_TO_OGN[mat.dtype], reduce)
    ws = _lib.workspace(ws_bytes, mat.device)
    rc = lib.ogn_spmm_csr(dptr(ptr), dptr(col), _index_code(ptr), dptr(value), width, dptr(mat),
                          _lib.TORCH_TO_OGN[mat.dtype], batch, m, n, k, nnz, dptr(out),
                          _lib.TORCH_TO_OGN[out_dtype], dptr(arg) if minmax else None, reduce,
                          dptr(ws), ws_bytes, stream_of(mat))
    check(rc, "spmm")
    return out, arg
