"""gather_csr / gather_coo: expand segment rows back over their positions.

Public API and argument contract of the reference
(python/ops_gnn/gather_csr.py, python/ops_gnn/gather_coo.py; host checks
csrc/npu/gather_csr/op_host/gather_csr.cpp:84-306 and
csrc/npu/gather_coo/op_host/gather_coo.cpp:87-180).  The copy is raw bytes
(every dtype, NaN payloads preserved) on the HIP kernels ogn_gather_csr /
ogn_gather_coo; there is no autograd, as in the reference.

gather_csr(src, indptr, out=None): the segment dim is indptr.dim() - 1;
out.size(dim) = indptr[..., -1] (one endpoint shared by every broadcast
pointer row); rows before indptr[..., 0] are zero.
gather_coo(src, index, out=None): the gather dim is index.dim() - 1 and the
prefix shapes of src and index match; out.size(dim) = index.size(-1).
"""

import math
from typing import Optional

import torch

from . import _lib, _native
from ._lib import check, dptr, lib, stream_of

_DTYPES = (torch.float16, torch.bfloat16, torch.float32, torch.float64, torch.int8, torch.int16, torch.int32,
           torch.int64, torch.uint8)
_MAX_RANK = 8
_INT64_MAX = 2 ** 63 - 1

# (endpoint min, endpoint max, value min, value max, decreasing?, first > 0?)
_PTR_CHECKS = _native._VersionCache(limit=128)


def _require_gpu(t, name):
    if not isinstance(t, torch.Tensor):
        raise RuntimeError(f"gather: {name} must be defined")
    if t.device.type != "cuda":
        raise RuntimeError(f"gather: {name} must be a GPU tensor")


def _overlaps(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Whether the byte ranges of two tensors' storages intersect."""
    if a.numel() == 0 or b.numel() == 0:
        return False
    sa, sb = a.untyped_storage(), b.untyped_storage()
    a0, b0 = sa.data_ptr(), sb.data_ptr()
    return a0 < b0 + sb.nbytes() and b0 < a0 + sa.nbytes()


def _ptr_facts(indptr: torch.Tensor, width: int):
    def compute():
        p = indptr.reshape(-1, width)
        ends = p[:, -1]
        dec = (p[:, 1:] < p[:, :-1]).any() if width > 1 else torch.zeros((), dtype=torch.bool, device=p.device)
        vals = torch.stack((ends.min(), ends.max(), p.min(), p.max(), dec.to(torch.int64),
                            (p[:, 0] > 0).any().to(torch.int64)))
        return tuple(int(v) for v in vals.tolist())
    return _PTR_CHECKS.get(indptr, compute)


def _validate_ptr(indptr: torch.Tensor, width: int):
    """Endpoint and uncovered-prefix flag; errors as the reference's
    ValidateIndptr (gather_csr.cpp:154-184)."""
    e_min, e_max, v_min, v_max, dec, prefix = _ptr_facts(indptr, width)
    if e_min < 0:
        raise RuntimeError("gather_csr: indptr endpoint must be non-negative")
    if e_min != e_max:
        raise RuntimeError("gather_csr: all broadcasted indptr rows must have the same endpoint")
    if v_min < 0 or v_max > e_max:
        raise RuntimeError(f"gather_csr: indptr value out of range: expected [0, {e_max}]")
    if dec:
        raise RuntimeError("gather_csr: indptr must be non-decreasing")
    return e_max, bool(prefix)


def _check_out_shape(out, src, dim, rows, op):
    _require_gpu(out, "out")
    if out.device != src.device:
        raise RuntimeError(f"{op}: out and src must be on the same GPU")
    if out.dtype != src.dtype:
        raise RuntimeError(f"{op}: out dtype must match src dtype")
    if out.dim() != src.dim():
        raise RuntimeError(f"{op}: out rank must match src rank")
    for axis in range(src.dim()):
        if axis != dim and out.size(axis) != src.size(axis):
            raise RuntimeError(f"{op}: out.size({axis}) must equal src.size({axis}) outside dimension {dim}")
    if out.size(dim) != rows:
        raise RuntimeError(f"{op}: out.size({dim}) must equal {rows}, got {out.size(dim)}")


def _result(res3, out, shape):
    res = res3.reshape(shape)
    if out is None:
        return res
    if res.data_ptr() != out.data_ptr() or not out.is_contiguous():
        out.copy_(res)
    else:
        # written through a raw pointer: record the in-place write for autograd
        torch._C._increment_version(out)
    return out


def gather_csr(src: torch.Tensor, indptr: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Expand segment features according to int64 CSR index pointers."""
    op = "gather_csr"
    _require_gpu(src, "src")
    _require_gpu(indptr, "indptr")
    if src.device != indptr.device:
        raise RuntimeError("gather_csr: src and indptr must be on the same GPU")
    if src.dtype not in _DTYPES:
        raise RuntimeError(f"gather_csr: unsupported src dtype {src.dtype}")
    if indptr.dtype != torch.int64:
        raise RuntimeError("gather_csr: indptr dtype must be int64")
    if not 1 <= src.dim() <= _MAX_RANK:
        raise RuntimeError(f"gather_csr: src rank must be in [1, {_MAX_RANK}], got {src.dim()}")
    if not 1 <= indptr.dim() <= src.dim():
        raise RuntimeError(f"gather_csr: indptr rank must be in [1, src.dim()], got {indptr.dim()}")
    dim = indptr.dim() - 1
    for axis in range(dim):
        if indptr.size(axis) not in (1, src.size(axis)):
            raise RuntimeError(f"gather_csr: indptr dimension {axis} with size {indptr.size(axis)} cannot "
                               f"broadcast to src size {src.size(axis)}")
    width = indptr.size(-1)
    if width == 0:
        if src.size(dim) != 0:
            raise RuntimeError(f"gather_csr: an empty indptr requires src.size({dim}) to be 0, got {src.size(dim)}")
    elif src.size(dim) != width - 1:
        raise RuntimeError(f"gather_csr: src.size({dim}) must equal indptr.size(-1) - 1; got {src.size(dim)} "
                           f"and {width - 1}")
    rows, prefix = (0, False) if indptr.numel() == 0 else _validate_ptr(indptr, width)
    before, segs, feat = math.prod(src.shape[:dim]), src.size(dim), math.prod(src.shape[dim + 1:])
    row_bytes = feat * src.element_size()
    if before and rows and row_bytes and rows > _INT64_MAX // (before * row_bytes):
        raise RuntimeError("gather_csr: out byte span overflows int64")
    shape = list(src.shape)
    shape[dim] = rows
    if out is not None:
        if src.numel() == 0 and isinstance(out, torch.Tensor) and out.dim() == src.dim() and \
                out.size(dim) != rows:
            raise RuntimeError(f"gather_csr: out.size({dim}) must equal indptr endpoint {rows} for an empty src, "
                               f"got {out.size(dim)}")
        _check_out_shape(out, src, dim, rows, op)
    if src.numel() == 0 or math.prod(shape) == 0:
        if out is not None:
            if prefix:
                out.zero_()
            return out
        return torch.zeros(shape, dtype=src.dtype, device=src.device)
    if out is not None and (_overlaps(out, src) or _overlaps(out, indptr)):
        src, indptr = src.clone(), indptr.clone()  # the reference reads a snapshot
    src3 = src.contiguous()
    if all(indptr.size(a) == 1 for a in range(dim)):
        ptr2 = indptr.contiguous().reshape(1, width)
    else:
        ptr2 = indptr.expand(*src.shape[:dim], width).reshape(-1, width).contiguous()
    direct = out is not None and out.is_contiguous()
    res = out if direct else torch.empty(shape, dtype=src.dtype, device=src.device)
    rc = lib.ogn_gather_csr(dptr(ptr2), ptr2.size(0), dptr(src3), before, segs, row_bytes, rows, dptr(res),
                            stream_of(src3))
    check(rc, op)
    return _result(res, out, shape)


def gather_coo(src: torch.Tensor, index: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Gather rows from ``src`` according to a sorted COO index tensor."""
    op = "gather_coo"
    _require_gpu(src, "src")
    _require_gpu(index, "index")
    if src.device != index.device:
        raise RuntimeError("gather_coo: src and index must be on the same GPU")
    if index.dtype != torch.int64:
        raise RuntimeError("gather_coo: index must have dtype torch.int64")
    if src.dtype not in _DTYPES:
        raise RuntimeError(f"gather_coo does not support dtype {src.dtype}")
    if not 1 <= src.dim() <= _MAX_RANK:
        raise RuntimeError(f"gather_coo: src rank must be in [1, {_MAX_RANK}]")
    if not 1 <= index.dim() <= src.dim():
        raise RuntimeError("gather_coo: index rank must be in [1, src.dim()]")
    dim = index.dim() - 1
    for axis in range(dim):
        if src.size(axis) != index.size(axis):
            raise RuntimeError(f"gather_coo: src and index prefix shapes must match at dim {axis}")
    before, src_rows, feat = math.prod(src.shape[:dim]), src.size(dim), math.prod(src.shape[dim + 1:])
    entries = index.size(dim)
    if before * entries > 0 and src_rows == 0:
        raise RuntimeError("gather_coo: index contains entries but src has zero rows along the gather dimension")
    shape = list(src.shape)
    shape[dim] = entries
    if out is not None:
        _require_gpu(out, "out")
        if out.device != src.device:
            raise RuntimeError("gather_coo: out must be on the same GPU as src")
        if out.dtype != src.dtype:
            raise RuntimeError("gather_coo: out dtype must match src dtype")
        if list(out.shape) != shape:
            raise RuntimeError(f"gather_coo: out shape mismatch: expected {tuple(shape)}, got {tuple(out.shape)}")
    if math.prod(shape) == 0:
        return out if out is not None else torch.empty(shape, dtype=src.dtype, device=src.device)
    if out is not None and (_overlaps(out, src) or _overlaps(out, index)):
        src, index = src.clone(), index.clone()
    src3 = src.contiguous()
    idx = index.contiguous()
    direct = out is not None and out.is_contiguous()
    res = out if direct else torch.empty(shape, dtype=src.dtype, device=src.device)
    rc = lib.ogn_gather_coo(dptr(idx), dptr(src3), before, src_rows, entries, feat * src.element_size(), dptr(res),
                            stream_of(src3))
    check(rc, op)
    return _result(res, out, shape)
