"""ind2ptr / ptr2ind -- torch_sparse index conversions on the GPU.

Public API and error contract of the reference python/ops_gnn/ind2ptr.py:26-72,
python/ops_gnn/ptr2ind.py:27-72 and the host checks of
csrc/npu/ind2ptr/op_host/ind2ptr.cpp:20-40, csrc/npu/ptr2ind/op_host/ptr2ind.cpp:20-55.
"""

import torch

from . import _lib
from ._lib import check, dptr, lib, stream_of


def ind2ptr_tensor(ind: torch.Tensor, num_rows: int) -> torch.Tensor:
    """Kernel call without argument checks (inputs already known valid)."""
    out = torch.empty(num_rows + 1, dtype=torch.int64, device=ind.device)
    if ind.numel() == 0:
        return out.zero_()
    ind = ind.contiguous()
    code = _lib.I64 if ind.dtype == torch.int64 else _lib.I32
    check(lib.ogn_ind2ptr(dptr(ind), code, ind.numel(), num_rows, dptr(out), stream_of(ind)), "ind2ptr")
    return out


def ptr2ind_tensor(ptr: torch.Tensor, num_edges: int) -> torch.Tensor:
    out = torch.empty(num_edges, dtype=torch.int64, device=ptr.device)
    if num_edges == 0:
        return out
    ptr = ptr.contiguous()
    code = _lib.I64 if ptr.dtype == torch.int64 else _lib.I32
    check(lib.ogn_ptr2ind(dptr(ptr), code, ptr.numel() - 1, num_edges, dptr(out), stream_of(ptr)),
          "ptr2ind")
    return out


def ind2ptr(ind: torch.Tensor, num_rows: int) -> torch.Tensor:
    """Convert sorted row indices to a CSR row pointer of length num_rows + 1.

    Drop-in for ``torch.ops.torch_sparse.ind2ptr(ind, M)``; asynchronous on the
    current stream.

    >>> ind2ptr(torch.tensor([2, 2, 4, 5, 5, 6], device='cuda'), 8)
    tensor([0, 0, 0, 2, 2, 3, 5, 6, 6], device='cuda:0')
    """
    _lib.require_gpu(ind, what="ind2ptr")
    if ind.dim() != 1:
        raise RuntimeError("ind2ptr: ind must be 1-D")
    if ind.dtype != torch.int64:
        raise RuntimeError("ind2ptr: ind must be int64 (torch.long)")
    num_rows = int(num_rows)
    if num_rows < 0:
        raise RuntimeError("ind2ptr: M must be non-negative")
    return ind2ptr_tensor(ind, num_rows)


def ptr2ind(ptr: torch.Tensor, num_edges: int) -> torch.Tensor:
    """Convert a CSR row pointer to the row index of every edge.

    Drop-in for ``torch.ops.torch_sparse.ptr2ind(ptr, E)``.  Like the
    reference, the pointer is validated first (one 4-byte device-to-host read).

    >>> ptr2ind(torch.tensor([0, 0, 0, 2, 2, 3, 5, 6, 6], device='cuda'), 6)
    tensor([2, 2, 4, 5, 5, 6], device='cuda:0')
    """
    _lib.require_gpu(ptr, what="ptr2ind")
    if ptr.dim() != 1:
        raise RuntimeError("ptr2ind: ptr must be 1-D")
    if ptr.dtype != torch.int64:
        raise RuntimeError("ptr2ind: ptr must be int64 (torch.long)")
    num_edges = int(num_edges)
    if num_edges < 0:
        raise RuntimeError("ptr2ind: E must be non-negative")
    if ptr.numel() < 1:
        raise RuntimeError("ptr2ind: ptr must have at least one element")
    ptr = ptr.contiguous()
    # Validate rowptr only (no columns): status 1 covers start/end/range/order.
    status = torch.empty(1, dtype=torch.int32, device=ptr.device)
    rc = lib.ogn_validate_csr(dptr(ptr), None, _lib.I64, ptr.numel() - 1, num_edges, 0, dptr(status),
                              stream_of(ptr))
    check(rc, "ptr2ind")
    if int(status.item()) != 0:
        first, last = ptr[0].item(), ptr[-1].item()
        if first != 0:
            raise RuntimeError("ptr2ind: ptr must start with 0")
        if last != num_edges:
            raise RuntimeError("ptr2ind: ptr must end with num_edges")
        if bool(((ptr < 0) | (ptr > num_edges)).any()):
            raise RuntimeError("ptr2ind: ptr contains an out-of-range value")
        raise RuntimeError("ptr2ind: ptr must be non-decreasing")
    return ptr2ind_tensor(ptr, num_edges)
