"""torch_sparse SpMM adapter for MI355X.

Mirror of the reference module python/ops_gnn/torch_sparse_spmm.py: the same
public helpers (csr_spmm, coo_spmm, coo_to_csr, clear_validation_cache,
validation_cache_info), the same argument checks and error messages, the same
validation cache keyed by tensor identity + version, and registrations of
``torch_sparse::spmm_{sum,mean,min,max}``, ``ind2ptr`` and ``ptr2ind`` -- here
for the CUDA (HIP) and AutogradCUDA dispatch keys instead of PrivateUse1.

When the third-party ``torch_sparse`` package is not importable, the operator
schemas are defined here (same signatures as torch_sparse's), so that
``torch.ops.torch_sparse.*`` callers work unchanged.
"""

__all__ = ["csr_spmm", "coo_spmm", "coo_to_csr", "clear_validation_cache", "validation_cache_info"]

from collections import OrderedDict
from numbers import Integral
from typing import NamedTuple, Optional, Tuple, Union
import weakref

import torch

from . import _native

try:  # optional third-party frontend
    import torch_sparse  # type: ignore
except ImportError:  # the normal case in this image
    torch_sparse = None

_REDUCE = {"sum": 0, "add": 0, "mean": 1, "min": 2, "max": 3}
_VALIDATED = OrderedDict()
_METADATA_VALIDATED = OrderedDict()
_COO_LAYOUTS = OrderedDict()
_INPUT_DTYPES = _native.SPMM_INPUT_DTYPES


def _check_mat(mat):
    """reference python/ops_gnn/torch_sparse_spmm.py:35-37."""
    if mat.device.type != "cuda" or mat.dim() < 2 or mat.dtype not in _INPUT_DTYPES:
        raise ValueError("mat must be a GPU fp32/fp16/bf16/int8 tensor [...,N,K]")


def _check_value(value, edges, mat):
    """reference python/ops_gnn/torch_sparse_spmm.py:40-51."""
    if value is None:
        return
    if value.dtype not in _INPUT_DTYPES or value.dtype != mat.dtype:
        raise ValueError("value dtype must be supported and match mat dtype")
    if value.device != mat.device or value.dim() < 1 or value.size(0) != edges:
        raise ValueError("value must be on the same GPU and have leading length E")
    width = 1
    for size in value.shape[1:]:
        width *= size
    if width not in (1, mat.size(-1)):
        raise ValueError("value must contain 1 or K weights per edge")


def _version(t):
    try:
        return t._version
    except (AttributeError, RuntimeError):  # inference tensors carry no version
        return None


def _validate(ptr, col, n):
    """Check CSR contents on the device; only the 4-byte status reaches the host.

    Same cache policy as the reference (python/ops_gnn/torch_sparse_spmm.py:58-76):
    up to 128 (identity, version) entries; in-place mutation through PyTorch
    bumps the version and invalidates the entry.
    """
    key = (id(ptr), id(col), _version(ptr), _version(col), n)
    cached = _VALIDATED.get(key)
    if cached is not None and cached[0]() is ptr and cached[1]() is col:
        _VALIDATED.move_to_end(key)
        return
    if ptr.dtype != torch.int64 or col.dtype != torch.int64 or ptr.dim() != 1 or col.dim() != 1:
        raise ValueError("invalid CSR rowptr or column index out of range")
    status = _native.validate_csr(ptr, col, n)
    if int(status.max().item()):
        raise ValueError("invalid CSR rowptr or column index out of range")
    if key[2] is not None and key[3] is not None:
        _VALIDATED[key] = (weakref.ref(ptr), weakref.ref(col))
        if len(_VALIDATED) > 128:
            _VALIDATED.popitem(last=False)


def clear_validation_cache() -> None:
    _VALIDATED.clear()
    _METADATA_VALIDATED.clear()
    _COO_LAYOUTS.clear()


class _CacheInfo(NamedTuple):
    csr_entries: int
    metadata_entries: int
    coo_entries: int


def validation_cache_info() -> _CacheInfo:
    return _CacheInfo(len(_VALIDATED), len(_METADATA_VALIDATED), len(_COO_LAYOUTS))


def _meta_tensor(t, length, name, device):
    if t is None or t.dtype != torch.int64 or t.device != device or t.shape != (length,):
        raise ValueError(f"{name} must be int64 [{length}] on {device}")


def _grad_meta(ptr, col, value, mat, reduce, *, row, rowcount, colptr, perm):
    """Validate supplied backward metadata; reference
    python/ops_gnn/torch_sparse_spmm.py:103-149 (same rules and messages)."""
    from .convert import ind2ptr_tensor, ptr2ind_tensor

    gradients = torch.is_grad_enabled() and reduce < 2
    need_v = gradients and value is not None and value.requires_grad
    need_m = gradients and mat.requires_grad
    e, m, n = col.numel(), ptr.numel() - 1, mat.size(-2)
    if row is not None or need_v or need_m:
        _meta_tensor(row, e, "row", col.device)
    if colptr is not None or need_m:
        _meta_tensor(colptr, n + 1, "colptr", col.device)
    if perm is not None or need_m:
        _meta_tensor(perm, e, "csr2csc", col.device)
    if rowcount is not None or (need_m and reduce == 1):
        _meta_tensor(rowcount, m, "rowcount", col.device)
    slots = (ptr, col, row, rowcount, colptr, perm)
    supplied = [t for t in slots if t is not None]
    if len(supplied) == 2:
        return
    key = (n, tuple(None if t is None else (id(t), _version(t)) for t in slots))
    cached = _METADATA_VALIDATED.get(key)
    if cached is not None and all(ref() is t for ref, t in zip(cached, supplied)):
        _METADATA_VALIDATED.move_to_end(key)
        return
    if row is not None and not torch.equal(row, ptr2ind_tensor(ptr, e)):
        raise ValueError("row disagrees with rowptr")
    if rowcount is not None and not torch.equal(rowcount, ptr[1:] - ptr[:-1]):
        raise ValueError("rowcount disagrees with rowptr")
    sorted_col = None
    if perm is not None:
        if not torch.equal(perm.sort().values, torch.arange(e, device=col.device)):
            raise ValueError("csr2csc must be a permutation of [0,E)")
        sorted_col = col[perm]
        if e > 1 and bool((sorted_col[1:] < sorted_col[:-1]).any().item()):
            raise ValueError("csr2csc must order edges by column")
    if colptr is not None:
        if sorted_col is None:
            sorted_col = col.sort().values
        if not torch.equal(colptr, ind2ptr_tensor(sorted_col, n)):
            raise ValueError("colptr disagrees with col and csr2csc")
    if all(item is None or item[1] is not None for item in key[1]):
        _METADATA_VALIDATED[key] = tuple(weakref.ref(t) for t in supplied)
        if len(_METADATA_VALIDATED) > 128:
            _METADATA_VALIDATED.popitem(last=False)


class _SpmmMetadata(NamedTuple):
    ptr: torch.Tensor
    col: torch.Tensor
    row: Optional[torch.Tensor]
    colptr: Optional[torch.Tensor]
    perm: Optional[torch.Tensor]
    reduce: int
    output_dtype: torch.dtype


class _Spmm(torch.autograd.Function):
    """Autograd for sum/mean; reference _Spmm (python/ops_gnn/torch_sparse_spmm.py:162-202).

    dvalue[e] = <grad[row(e)], mat[col(e)]> (/ deg for mean), computed by the
    SDDMM kernel; dmat is a forward SpMM over the transposed graph
    (colptr, row[csr2csc], value[csr2csc]).
    """

    @staticmethod
    def forward(ctx, value, mat, metadata):
        ptr, col, row, colptr, perm, reduce, output_dtype = metadata
        out, arg = _native.spmm_forward(ptr, col, value, mat, reduce, output_dtype)
        ctx.save_for_backward(ptr, col, value if value is not None else col, mat,
                              row if row is not None else col,
                              colptr if colptr is not None else col,
                              perm if perm is not None else col, arg)
        ctx.has_value, ctx.reduce = value is not None, reduce
        ctx.mark_non_differentiable(arg)
        return out, arg

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad, unused_arg):
        from .sddmm_csr import value_grad

        ptr, col, saved_value, mat, row, colptr, perm, arg = ctx.saved_tensors
        value = saved_value if ctx.has_value else None
        dv = dm = None
        if ctx.reduce >= 2:
            raise NotImplementedError("min/max backward is outside this extension's supported contract")
        if ctx.needs_input_grad[0]:
            width = 1
            for size in value.shape[1:]:
                width *= size
            dv = value_grad(ptr, col, mat, grad, ctx.reduce, width).reshape_as(value).to(value.dtype)
        if ctx.needs_input_grad[1]:
            g = grad.float()
            if ctx.reduce == 1:
                degree = (ptr[1:] - ptr[:-1]).clamp_min(1).float()
                g = g / degree.unsqueeze(-1)
            tv = None if value is None else value[perm].float()
            dm = _native.spmm_forward(colptr, row[perm], tv, g.contiguous(), 0, torch.float32)[0]
            dm = dm.to(mat.dtype)
        return dv, dm, None


def _dispatch(ptr, col, value, mat, reduce, *, row=None, rowcount=None, colptr=None, perm=None,
              output_dtype=None):
    """reference python/ops_gnn/torch_sparse_spmm.py:205-219."""
    _check_mat(mat)
    _check_value(value, col.numel(), mat)
    if ptr.device != mat.device or col.device != mat.device:
        raise ValueError("indices and mat must be on the same GPU")
    _validate(ptr, col, mat.size(-2))
    if reduce < 2:
        _grad_meta(ptr, col, value, mat, reduce, row=row, rowcount=rowcount, colptr=colptr, perm=perm)
    dtype = output_dtype or (torch.int32 if mat.dtype == torch.int8 else mat.dtype)
    if dtype not in _native.SPMM_OUTPUT_DTYPES or ((mat.dtype == torch.int8) != (dtype == torch.int32)):
        raise ValueError("unsupported output dtype")
    if not torch.is_grad_enabled() or not (mat.requires_grad or (value is not None and value.requires_grad)):
        return _native.spmm_forward(ptr, col, value, mat, reduce, dtype)
    metadata = _SpmmMetadata(ptr, col, row, colptr, perm, reduce, dtype)
    return _Spmm.apply(value, mat, metadata)


def csr_spmm(rowptr: torch.Tensor, col: torch.Tensor, value: Optional[torch.Tensor], mat: torch.Tensor,
             reduce: str = "sum", *, output_dtype: Optional[torch.dtype] = None
             ) -> Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]:
    """CSR SpMM; min/max return (out, arg), sum/mean return out.  Empty rows
    are zero with arg = E.  reference python/ops_gnn/torch_sparse_spmm.py:222-256.

    Missing backward metadata (row, csr2csc, colptr, rowcount) is built on the
    GPU when a gradient is required.
    """
    from .convert import ind2ptr_tensor, ptr2ind_tensor

    _check_mat(mat)
    _check_value(value, col.numel(), mat)
    if rowptr.device != mat.device or col.device != mat.device:
        raise ValueError("indices and mat must be on the same GPU")
    if not isinstance(reduce, str) or reduce not in _REDUCE:
        raise ValueError("reduce must be sum/add/mean/min/max")
    r = _REDUCE[reduce]
    row = rowcount = cp = perm = None
    _validate(rowptr, col, mat.size(-2))
    if r < 2 and torch.is_grad_enabled():
        if mat.requires_grad or (value is not None and value.requires_grad):
            row = ptr2ind_tensor(rowptr, col.numel())
            if mat.requires_grad:
                perm = torch.argsort(col, stable=True)
                cp = ind2ptr_tensor(col[perm], mat.size(-2))
                rowcount = rowptr[1:] - rowptr[:-1]
    result = _dispatch(rowptr, col, value, mat, r, row=row, rowcount=rowcount, colptr=cp, perm=perm,
                       output_dtype=output_dtype)
    return result if r >= 2 else result[0]


def _build_coo_layout(index, m):
    """reference python/ops_gnn/torch_sparse_spmm.py:273-281."""
    from .convert import ind2ptr_tensor

    if bool(((index[0] < 0) | (index[0] >= m)).any().item()):
        raise ValueError("COO row out of range")
    row = index[0]
    if row.numel() < 2 or not bool((row[1:] < row[:-1]).any().item()):
        return ind2ptr_tensor(row.contiguous(), m), index[1].clone(), None
    perm = torch.argsort(row, stable=True)
    row, col = row[perm], index[1][perm]
    return ind2ptr_tensor(row.contiguous(), m), col, perm


def coo_to_csr(index: torch.Tensor, value: Optional[torch.Tensor], m: int
               ) -> Tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    """Convert COO rows to CSR without caching (columns stably ordered by row)."""
    ptr, col, perm = _build_coo_layout(index, m)
    return ptr, col, None if value is None else (value.clone() if perm is None else value[perm])


def _cached_coo_layout(index, m):
    """Topology-only cache (reference :296-317); values are read on every call."""
    version = _version(index)
    if version is None:
        return _build_coo_layout(index, m)
    key = (id(index), version, m)
    cached = _COO_LAYOUTS.get(key)
    if cached is not None and cached[0]() is index:
        _COO_LAYOUTS.move_to_end(key)
        return cached[1:]
    layout = _build_coo_layout(index, m)

    def release(ref):
        entry = _COO_LAYOUTS.get(key)
        if entry is not None and entry[0] is ref:
            _COO_LAYOUTS.pop(key, None)

    _COO_LAYOUTS[key] = (weakref.ref(index, release), *layout)
    if len(_COO_LAYOUTS) > 32:
        _COO_LAYOUTS.popitem(last=False)
    return layout


def coo_spmm(index: torch.Tensor, value: Optional[torch.Tensor], m: int, n: int,
             matrix: torch.Tensor) -> torch.Tensor:
    """torch_sparse.spmm(index, value, m, n, matrix) on the GPU; reference :320-342."""
    if matrix.device.type != "cuda":
        if torch_sparse is not None:
            return torch_sparse.spmm(index, value, m, n, matrix)
        raise ValueError("coo_spmm: matrix must be a GPU tensor")
    _check_mat(matrix)
    if any(isinstance(x, bool) or not isinstance(x, Integral) or x < 0 for x in (m, n)):
        raise ValueError("COO m and n must be nonnegative integers")
    if index.dtype != torch.int64 or index.dim() != 2 or index.size(0) != 2:
        raise ValueError("COO index must be int64 [2,E] and dimensions nonnegative")
    if index.device != matrix.device or matrix.dim() < 2 or matrix.size(-2) != n:
        raise ValueError("COO device or dense shape mismatch")
    _check_value(value, index.size(1), matrix)
    ptr, col, perm = _cached_coo_layout(index, m)
    if value is None:
        weights = None
    elif perm is None:
        snapshot = torch.is_grad_enabled() and (value.requires_grad or matrix.requires_grad)
        weights = value.clone() if snapshot else value
    else:
        weights = value[perm]
    return csr_spmm(ptr, col, weights, matrix)


# ---------------------------------------------------------------- registration
def _spmm_sum_impl(row, ptr, col, value, cp, perm, mat):
    return _dispatch(ptr, col, value, mat, 0, row=row, colptr=cp, perm=perm)[0]


def _spmm_mean_impl(row, ptr, col, value, counts, cp, perm, mat):
    return _dispatch(ptr, col, value, mat, 1, row=row, rowcount=counts, colptr=cp, perm=perm)[0]


def _spmm_min_impl(ptr, col, value, mat):
    out, arg = _dispatch(ptr, col, value, mat, 2)
    return out, arg


def _spmm_max_impl(ptr, col, value, mat):
    out, arg = _dispatch(ptr, col, value, mat, 3)
    return out, arg


def _ind2ptr_impl(ind, m):
    from .convert import ind2ptr_tensor
    return ind2ptr_tensor(ind, m)


def _ptr2ind_impl(ptr, e):
    from .convert import ptr2ind_tensor
    return ptr2ind_tensor(ptr, e)


_SCHEMAS = {
    "spmm_sum": "spmm_sum(Tensor? row, Tensor rowptr, Tensor col, Tensor? value, Tensor? colptr, "
                "Tensor? csr2csc, Tensor mat) -> Tensor",
    "spmm_mean": "spmm_mean(Tensor? row, Tensor rowptr, Tensor col, Tensor? value, Tensor? rowcount, "
                 "Tensor? colptr, Tensor? csr2csc, Tensor mat) -> Tensor",
    "spmm_min": "spmm_min(Tensor rowptr, Tensor col, Tensor? value, Tensor mat) -> (Tensor, Tensor)",
    "spmm_max": "spmm_max(Tensor rowptr, Tensor col, Tensor? value, Tensor mat) -> (Tensor, Tensor)",
    "ind2ptr": "ind2ptr(Tensor ind, int M) -> Tensor",
    "ptr2ind": "ptr2ind(Tensor ptr, int E) -> Tensor",
}
_IMPLS = {
    "spmm_sum": _spmm_sum_impl,
    "spmm_mean": _spmm_mean_impl,
    "spmm_min": _spmm_min_impl,
    "spmm_max": _spmm_max_impl,
    "ind2ptr": _ind2ptr_impl,
    "ptr2ind": _ptr2ind_impl,
}

_LIBRARIES = []


def _op_exists(name):
    try:
        torch._C._dispatch_find_schema_or_throw("torch_sparse::" + name, "")
        return True
    except RuntimeError:
        return False


def _register():
    if _LIBRARIES:
        return
    missing = [name for name in _SCHEMAS if not _op_exists(name)]
    if missing:
        lib_def = torch.library.Library("torch_sparse", "FRAGMENT")
        for name in missing:
            lib_def.define(_SCHEMAS[name])
        _LIBRARIES.append(lib_def)
    for key in ("CUDA", "AutogradCUDA"):
        lib_impl = torch.library.Library("torch_sparse", "IMPL", key)
        for name, fn in _IMPLS.items():
            lib_impl.impl(name, fn)
        _LIBRARIES.append(lib_impl)


_register()
