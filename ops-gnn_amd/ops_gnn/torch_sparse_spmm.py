"""torch_sparse SpMM on MI355X.

Three layers, all over the ``_pybind.torch_sparse_spmm`` extension (the HIP
kernels of libogn_hip.so):

* ``csr_spmm`` / ``coo_spmm`` / ``coo_to_csr``: the public helpers of the
  reference module (python/ops_gnn/torch_sparse_spmm.py:222-342), with its
  argument checks and error messages, which callers match on.
* ``torch.ops.torch_sparse.spmm_{sum,mean,min,max}`` / ``ind2ptr`` /
  ``ptr2ind`` implemented for the CUDA (HIP) and AutogradCUDA dispatch keys
  (reference :407-431 registers PrivateUse1).  When the third-party
  ``torch_sparse`` package is absent, the schemas are defined here.
* the frontend adaptation: when ``torch_sparse`` (and PyG) are importable,
  their SpMM entry points route GPU operands here and everything else to the
  original implementation (reference :345-459).

Design.  A CSR operand travels as one ``_Csr`` record: the pointer, the
columns, the dense row count, and any backward metadata a torch_sparse
storage already holds (row, rowcount, colptr, csr2csc).  Proofs about
tensors (CSR validity, metadata consistency, COO layouts) live in bounded
``_ProofCache`` tables whose keys stamp each tensor by identity, version
counter, storage address and layout; an entry dies with any of its tensors.
Transposed (CSC) metadata is built on the GPU only when a backward pass
asks for a mat gradient, not when the forward runs.
"""

__all__ = ["csr_spmm", "coo_spmm", "coo_to_csr", "clear_validation_cache", "validation_cache_info",
           "adapt_frontends"]

import importlib
import importlib.util
import math
import sys
from collections import OrderedDict
from numbers import Integral
from typing import NamedTuple, Optional, Tuple, Union
import weakref

import torch

from . import _lib, _native
from . import _pybind

_C = _pybind.torch_sparse_spmm

# Reduction codes and output-type codes shared with the extension (reference
# python/ops_gnn/torch_sparse_spmm.py:27-28).
_REDUCE = {"sum": 0, "add": 0, "mean": 1, "min": 2, "max": 3}
_OUT_CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2, torch.int8: 3, torch.int32: 4}
_MAT_DTYPES = tuple(_native.SPMM_OUTPUTS_FOR)


# ---------------------------------------------------------------- proof caches
def _stamp(t: torch.Tensor):
    """What must be unchanged for a proof about `t` to still hold: the object,
    its version counter, storage address and offset, and layout.  None for
    tensors without a version counter (inference tensors): never cached."""
    version = _C.tensor_version(t)
    if version is None:
        return None
    return (id(t), version, t.data_ptr(), t.storage_offset(), tuple(t.shape), tuple(t.stride()))


_MISS = object()


class _ProofCache:
    """Bounded LRU of facts proven about a tuple of tensors (plus plain
    parameters).  A hit requires the same live tensor objects with unchanged
    stamps; an entry is dropped as soon as one of its tensors is freed."""

    def __init__(self, capacity: int):
        self.capacity = capacity
        self._table = OrderedDict()

    def _key(self, tensors, params):
        stamps = tuple(None if t is None else _stamp(t) for t in tensors)
        if any(s is None for s, t in zip(stamps, tensors) if t is not None):
            return None
        return stamps, params

    def lookup(self, tensors, params=()):
        key = self._key(tensors, params)
        entry = None if key is None else self._table.get(key)
        if entry is None:
            return _MISS
        refs, value = entry
        if any((r() if r is not None else None) is not t for r, t in zip(refs, tensors)):
            return _MISS
        self._table.move_to_end(key)
        return value

    def store(self, tensors, params, value) -> None:
        key = self._key(tensors, params)
        if key is None:
            return
        table = self._table

        def forget(dead_ref, key=key):
            entry = table.get(key)
            if entry is not None and any(r is dead_ref for r in entry[0]):
                del table[key]

        refs = tuple(None if t is None else weakref.ref(t, forget) for t in tensors)
        table[key] = (refs, value)
        table.move_to_end(key)
        while len(table) > self.capacity:
            table.popitem(last=False)

    def clear(self) -> None:
        self._table.clear()

    def __len__(self) -> int:
        return len(self._table)


# capacities of the reference's caches (python/ops_gnn/torch_sparse_spmm.py:75,148,315)
_CSR_PROOFS = _ProofCache(128)
_META_PROOFS = _ProofCache(128)
_COO_LAYOUTS = _ProofCache(32)


def clear_validation_cache() -> None:
    _CSR_PROOFS.clear()
    _META_PROOFS.clear()
    _COO_LAYOUTS.clear()


class _CacheInfo(NamedTuple):
    csr_entries: int
    metadata_entries: int
    coo_entries: int


def validation_cache_info() -> _CacheInfo:
    """Entry counts of the three proof caches (no tensors are exposed)."""
    return _CacheInfo(len(_CSR_PROOFS), len(_META_PROOFS), len(_COO_LAYOUTS))


# ---------------------------------------------------------------- operand checks
# Messages are the reference's (python/ops_gnn/torch_sparse_spmm.py:35-51), with NPU -> GPU.
def _on_gpu(t) -> bool:
    return isinstance(t, torch.Tensor) and t.device.type == "cuda"


def _check_mat(mat):
    if not _on_gpu(mat) or mat.dim() < 2 or mat.dtype not in _MAT_DTYPES:
        raise ValueError("mat must be a GPU fp32/fp16/bf16/int8 tensor [...,N,K]")


def _check_value(value, edges, mat):
    if value is None:
        return
    if value.dtype != mat.dtype:
        raise ValueError("value dtype must be supported and match mat dtype")
    if value.device != mat.device or value.dim() < 1 or value.size(0) != edges:
        raise ValueError("value must be on the same GPU and have leading length E")
    if math.prod(value.shape[1:]) not in (1, mat.size(-1)):
        raise ValueError("value must contain 1 or K weights per edge")


def _check_reduce(reduce) -> int:
    if not isinstance(reduce, str) or reduce not in _REDUCE:
        raise ValueError("reduce must be sum/add/mean/min/max")
    return _REDUCE[reduce]


def _output_code(mat, output_dtype) -> int:
    allowed = _native.SPMM_OUTPUTS_FOR[mat.dtype]
    dtype = allowed[0] if output_dtype is None else output_dtype
    if dtype not in allowed:
        raise ValueError("unsupported output dtype")
    return _OUT_CODE[dtype]


class _Csr:
    """A CSR operand and whatever backward metadata came with it."""

    __slots__ = ("ptr", "col", "n", "row", "rowcount", "colptr", "perm")

    def __init__(self, ptr, col, n, row=None, rowcount=None, colptr=None, perm=None):
        self.ptr, self.col, self.n = ptr, col, n
        self.row, self.rowcount, self.colptr, self.perm = row, rowcount, colptr, perm

    @property
    def rows(self) -> int:
        return self.ptr.numel() - 1

    @property
    def edges(self) -> int:
        return self.col.numel()

    def prove_valid(self) -> None:
        """Device check of the pointer and columns; only a 4-byte status is
        read back, and only when the pair is not already proven."""
        if _CSR_PROOFS.lookup((self.ptr, self.col), (self.n,)) is not _MISS:
            return
        if self.ptr.dtype != torch.int64 or self.col.dtype != torch.int64 or self.ptr.dim() != 1 \
                or self.col.dim() != 1 or self.ptr.numel() == 0:
            raise ValueError("invalid CSR rowptr or column index out of range")
        if int(_C.validate(self.ptr, self.col, self.n).item()):
            raise ValueError("invalid CSR rowptr or column index out of range")
        _CSR_PROOFS.store((self.ptr, self.col), (self.n,), True)

    def check_metadata(self, reduce: int, value, mat, required: bool) -> None:
        """Shape / dtype / device of every supplied metadata tensor, and, when
        `required` (the torch_sparse operator schemas), the presence of those a
        gradient of this call needs (reference :103-120).  Contents are then
        proven consistent with (ptr, col) once per tensor version."""
        grads = required and reduce < 2 and torch.is_grad_enabled()
        need_row = grads and ((value is not None and value.requires_grad) or mat.requires_grad)
        need_t = grads and mat.requires_grad
        slots = (("row", self.row, self.edges, need_row),
                 ("colptr", self.colptr, self.n + 1, need_t),
                 ("csr2csc", self.perm, self.edges, need_t),
                 ("rowcount", self.rowcount, self.rows, need_t and reduce == 1))
        device = self.col.device
        for name, t, length, needed in slots:
            if t is None and not needed:
                continue
            if t is None or t.dtype != torch.int64 or t.device != device or tuple(t.shape) != (length,):
                raise ValueError(f"{name} must be int64 [{length}] on {device}")
        meta = (self.row, self.rowcount, self.colptr, self.perm)
        if all(t is None for t in meta):
            return
        tensors = (self.ptr, self.col) + meta
        if _META_PROOFS.lookup(tensors, (self.n,)) is not _MISS:
            return
        self._prove_metadata()
        _META_PROOFS.store(tensors, (self.n,), True)

    def _prove_metadata(self) -> None:
        e, n = self.edges, self.n
        if self.row is not None and not torch.equal(self.row, _C.convert(self.ptr, e, False)):
            raise ValueError("row disagrees with rowptr")
        if self.rowcount is not None and not torch.equal(self.rowcount, self.ptr.diff()):
            raise ValueError("rowcount disagrees with rowptr")
        if self.perm is not None:
            perm = self.perm
            in_range = e == 0 or bool(((perm >= 0) & (perm < e)).all().item())
            if not in_range or (e and not bool((torch.bincount(perm, minlength=e) == 1).all().item())):
                raise ValueError("csr2csc must be a permutation of [0,E)")
            if e > 1 and bool((self.col[perm].diff() < 0).any().item()):
                raise ValueError("csr2csc must order edges by column")
        if self.colptr is not None:
            # column counts need no sort: colptr = [0, cumsum(bincount(col))]
            counts = torch.bincount(self.col, minlength=n) if e else torch.zeros(n, dtype=torch.int64,
                                                                                   device=self.col.device)
            expect = torch.cat([counts.new_zeros(1), counts.cumsum(0)])
            if not torch.equal(self.colptr, expect):
                raise ValueError("colptr disagrees with col and csr2csc")

    def transposed(self):
        """(colptr, row of each edge in column order, csr2csc), built on the
        GPU from (ptr, col) where the caller supplied none."""
        e = self.edges
        row = self.row if self.row is not None else _C.convert(self.ptr, e, False)
        perm = self.perm
        if perm is None:
            # columns lie in [0, n) (validated with the CSR): bounded-key sort
            sorted_col, perm, (row_t,) = _native.sort_rows(self.col, max(self.n - 1, 0), (row,))
        else:
            sorted_col, row_t = self.col[perm], row[perm]
        colptr = self.colptr if self.colptr is not None else _C.convert(sorted_col, self.n + 1, True)
        return colptr, row_t, perm


# ---------------------------------------------------------------- autograd
class _SpmmFunction(torch.autograd.Function):
    """out = R_e value[e] * mat[col[e]] with gradients for value and mat.

    sum / mean (reference _Spmm, python/ops_gnn/torch_sparse_spmm.py:162-202):
      dvalue[e] = <grad[row(e)], mat[col(e)]> (/ deg for mean): the SDDMM
      kernel through ``value_backward``; dmat = the forward SpMM over the
      transposed graph with (grad / deg) as the dense operand.
    min / max: the gradient flows to the arg edge of every output element
      (upstream torch_sparse's rule; the reference rejects it).
    """

    @staticmethod
    def forward(ctx, value, mat, csr, reduce, out_code):
        out, arg = _forward(csr.ptr, csr.col, value, mat, reduce, out_code)
        ctx.csr, ctx.reduce = csr, reduce
        ctx.value_shape = None if value is None else value.shape
        ctx.save_for_backward(value, mat, arg)
        ctx.mark_non_differentiable(arg)
        return out, arg

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad, _grad_arg):
        value, mat, arg = ctx.saved_tensors
        csr, reduce = ctx.csr, ctx.reduce
        want_v, want_m = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        if reduce >= 2:
            return _extremum_backward(csr, value, mat, arg, grad, want_v, want_m) + (None, None, None)
        d_value = d_mat = None
        if want_v:
            width = math.prod(value.shape[1:])
            d_value = _C.value_backward(csr.ptr, csr.col, mat, grad, reduce, width)
            d_value = d_value.reshape(ctx.value_shape).to(value.dtype)
        if want_m:
            g = grad.float()
            if reduce == 1:
                g = g / csr.ptr.diff().clamp_min(1).to(torch.float32).unsqueeze(-1)
            colptr, row_t, perm = csr.transposed()
            w_t = None if value is None else _C.permute_values(value.float(), perm)
            d_mat = _C.forward(colptr, row_t, w_t, g.contiguous(), 0, 0)[0].to(mat.dtype)
        return d_value, d_mat, None, None, None


def _extremum_backward(csr, value, mat, arg, grad, want_v, want_m):
    """Gradients of min / max: each output element (b, r, k) took its value
    from edge arg = a (a == E for an empty row): out = w[a] * mat[b, col[a], k]."""
    e = csr.edges
    k = mat.size(-1)
    g = grad.float().reshape(-1, csr.rows, k)
    a = arg.reshape(-1, csr.rows, k)
    hit = a < e
    a_safe = torch.where(hit, a, torch.zeros_like(a))
    g = torch.where(hit, g, torch.zeros_like(g))
    d_value = d_mat = None
    w = None
    width = 1 if value is None else math.prod(value.shape[1:])
    if value is not None:
        wf = value.float().reshape(e, width)
        kk = torch.arange(k, device=mat.device) if width > 1 else torch.zeros(k, dtype=torch.long, device=mat.device)
        w = wf[a_safe, kk]
    if want_m:
        src_rows = csr.col[a_safe]                                   # [B, M, K] source row of each element
        contrib = g if w is None else g * w
        flat = mat.reshape(-1, mat.size(-2), k)
        d = torch.zeros(flat.shape, dtype=torch.float32, device=mat.device)
        d.scatter_add_(1, src_rows, contrib)
        d_mat = d.reshape(mat.shape).to(mat.dtype)
    if want_v and value is not None:
        flat = mat.float().reshape(-1, mat.size(-2), k)
        x = torch.gather(flat, 1, csr.col[a_safe])
        contrib = (g * x).reshape(-1)
        target = a_safe if width == 1 else a_safe * k + torch.arange(k, device=mat.device)
        dv = torch.zeros(e * width, dtype=torch.float32, device=mat.device)
        dv.index_add_(0, target.reshape(-1), contrib)
        d_value = dv.reshape(value.shape).to(value.dtype)
    return d_value, d_mat


def _forward(ptr, col, value, mat, reduce: int, out_code: int):
    """``_C.forward``, or for a weighted sum over one 2-D operand the
    XCD-tiled SpMM when the graph and table sizes call for it
    (``_native.spmm_sum_xcd``; include/ogn.h ogn_spmm_sum_xcd)."""
    if reduce == 0 and mat.dim() == 2 and value is not None and value.dim() == 1 and col.dtype == ptr.dtype:
        out_dtype = _OUT_DTYPES.get(out_code)
        if out_dtype is not None and mat.dtype in _native.SEGMENT_DTYPES and out_dtype in (mat.dtype, torch.float32):
            out = torch.empty((ptr.numel() - 1, mat.size(1)), dtype=out_dtype, device=mat.device)
            if _native.spmm_sum_xcd(ptr.contiguous(), col.contiguous(), value.contiguous(), mat.contiguous(), out):
                return out, torch.empty(0, dtype=torch.int64, device=mat.device)
    return _C.forward(ptr, col, value, mat, reduce, out_code)


_OUT_DTYPES = {code: dt for dt, code in _lib.TORCH_TO_OGN.items()}


def _run(csr: _Csr, value, mat, reduce: int, out_code: int):
    """(out, arg) through autograd when a gradient is wanted, else directly."""
    if torch.is_grad_enabled() and (mat.requires_grad or (value is not None and value.requires_grad)):
        return _SpmmFunction.apply(value, mat, csr, reduce, out_code)
    return _forward(csr.ptr, csr.col, value, mat, reduce, out_code)


def _prove_and_run(csr: _Csr, value, mat, reduce: int, output_dtype=None, required_metadata=False):
    csr.prove_valid()
    if reduce < 2:
        csr.check_metadata(reduce, value, mat, required_metadata)
    return _run(csr, value, mat, reduce, _output_code(mat, output_dtype))


def _checked_call(csr: _Csr, value, mat, reduce: int, *, required_metadata=False):
    """The operator entry: operand checks (reference :205-219), then run."""
    _check_mat(mat)
    _check_value(value, csr.edges, mat)
    if csr.ptr.device != mat.device or csr.col.device != mat.device:
        raise ValueError("indices and mat must be on the same GPU")
    return _prove_and_run(csr, value, mat, reduce, required_metadata=required_metadata)


# ---------------------------------------------------------------- public helpers
def csr_spmm(rowptr: torch.Tensor, col: torch.Tensor, value: Optional[torch.Tensor], mat: torch.Tensor,
             reduce: str = "sum", *, output_dtype: Optional[torch.dtype] = None
             ) -> Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]:
    """CSR SpMM: ``out[..., r, k] = R_{e in row r} value[e, (k)] * mat[..., col[e], k]``.

    reduce sum/add/mean return ``out``; min/max return ``(out, arg)`` with
    arg = the first extremal edge, E for an empty row (value 0).  Output
    dtypes follow the reference table: fp32 -> fp32; fp16 -> fp16 | fp32;
    bf16 -> bf16 | fp32; int8 -> int32 | fp32.  Reference
    python/ops_gnn/torch_sparse_spmm.py:222-256.
    """
    _check_mat(mat)
    _check_value(value, col.numel(), mat)
    if rowptr.device != mat.device or col.device != mat.device:
        raise ValueError("indices and mat must be on the same GPU")
    r = _check_reduce(reduce)
    out, arg = _prove_and_run(_Csr(rowptr, col, mat.size(-2)), value, mat, r, output_dtype)
    return (out, arg) if r >= 2 else out


def _coo_layout_uncached(index: torch.Tensor, m: int, value: Optional[torch.Tensor] = None):
    """(ptr, col, perm or None, value in row order or None) of a COO index
    [2, E]; rows ordered stably.  One device probe gives the row range and
    sortedness together; the columns (and a 1-D 4- or 8-byte value) are
    permuted inside the sort's last pass."""
    row = index[0]
    if row.numel() == 0:
        return (torch.zeros(m + 1, dtype=torch.int64, device=index.device), index[1].clone(), None,
                None if value is None else value.clone())
    unsorted, lo, hi = _native.index_probe(row)
    if lo < 0 or hi >= m:
        raise ValueError("COO row out of range")
    if not unsorted:
        return _C.convert(row, m + 1, True), index[1].clone(), None, None if value is None else value.clone()
    carried = (index[1],) if value is None else (index[1], value)
    sorted_row, perm, outs = _native.sort_rows(row, m - 1, carried)
    return _C.convert(sorted_row, m + 1, True), outs[0], perm, None if value is None else outs[1]


def coo_to_csr(index: torch.Tensor, value: Optional[torch.Tensor], m: int
               ) -> Tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    """COO [2, E] -> (rowptr, col, value) with columns stably ordered by row;
    nothing is cached (reference :284-294)."""
    ptr, col, _, vals = _coo_layout_uncached(index, m, value)
    return ptr, col, vals


def _coo_layout(index: torch.Tensor, m: int):
    """Topology only is cached; values and dense inputs are read every call."""
    hit = _COO_LAYOUTS.lookup((index,), (m,))
    if hit is not _MISS:
        return hit
    layout = _coo_layout_uncached(index, m)[:3]
    _COO_LAYOUTS.store((index,), (m,), layout)
    return layout


def coo_spmm(index: torch.Tensor, value: Optional[torch.Tensor], m: int, n: int,
             matrix: torch.Tensor) -> torch.Tensor:
    """``torch_sparse.spmm(index, value, m, n, matrix)`` for a GPU matrix
    (reference :320-342); other devices go to torch_sparse when present."""
    if not _on_gpu(matrix):
        original = _ORIGINALS.get("torch_sparse.spmm")
        if original is not None:
            return original(index, value, m, n, matrix)
        raise ValueError("coo_spmm: matrix must be a GPU tensor")
    _check_mat(matrix)
    if any(isinstance(x, bool) or not isinstance(x, Integral) or x < 0 for x in (m, n)):
        raise ValueError("COO m and n must be nonnegative integers")
    if index.dtype != torch.int64 or index.dim() != 2 or index.size(0) != 2:
        raise ValueError("COO index must be int64 [2,E] and dimensions nonnegative")
    if index.device != matrix.device or matrix.dim() < 2 or matrix.size(-2) != n:
        raise ValueError("COO device or dense shape mismatch")
    _check_value(value, index.size(1), matrix)  # before a permutation could hide extra entries
    ptr, col, perm = _coo_layout(index, m)
    weights = value
    if value is not None:
        grad_wanted = torch.is_grad_enabled() and (value.requires_grad or matrix.requires_grad)
        if perm is not None:
            weights = value[perm] if grad_wanted and value.requires_grad else _C.permute_values(value, perm)
        elif grad_wanted:
            weights = value.clone()  # the backward reads the weights as they were at forward time
    return csr_spmm(ptr, col, weights, matrix)


# ---------------------------------------------------------------- torch_sparse operators
def _op_spmm_sum(row, rowptr, col, value, colptr, csr2csc, mat):
    csr = _Csr(rowptr, col, mat.size(-2), row=row, colptr=colptr, perm=csr2csc)
    return _checked_call(csr, value, mat, 0, required_metadata=True)[0]


def _op_spmm_mean(row, rowptr, col, value, rowcount, colptr, csr2csc, mat):
    csr = _Csr(rowptr, col, mat.size(-2), row=row, rowcount=rowcount, colptr=colptr, perm=csr2csc)
    return _checked_call(csr, value, mat, 1, required_metadata=True)[0]


def _op_spmm_min(rowptr, col, value, mat):
    return tuple(_checked_call(_Csr(rowptr, col, mat.size(-2)), value, mat, 2))


def _op_spmm_max(rowptr, col, value, mat):
    return tuple(_checked_call(_Csr(rowptr, col, mat.size(-2)), value, mat, 3))


def _op_ind2ptr(ind, m):
    return _C.convert(ind, m + 1, True)


def _op_ptr2ind(ptr, e):
    return _C.convert(ptr, e, False)


# name -> (schema, implementation); the schemas are torch_sparse's own.
_OPERATORS = {
    "spmm_sum": ("spmm_sum(Tensor? row, Tensor rowptr, Tensor col, Tensor? value, Tensor? colptr, "
                 "Tensor? csr2csc, Tensor mat) -> Tensor", _op_spmm_sum),
    "spmm_mean": ("spmm_mean(Tensor? row, Tensor rowptr, Tensor col, Tensor? value, Tensor? rowcount, "
                  "Tensor? colptr, Tensor? csr2csc, Tensor mat) -> Tensor", _op_spmm_mean),
    "spmm_min": ("spmm_min(Tensor rowptr, Tensor col, Tensor? value, Tensor mat) -> (Tensor, Tensor)",
                 _op_spmm_min),
    "spmm_max": ("spmm_max(Tensor rowptr, Tensor col, Tensor? value, Tensor mat) -> (Tensor, Tensor)",
                 _op_spmm_max),
    "ind2ptr": ("ind2ptr(Tensor ind, int M) -> Tensor", _op_ind2ptr),
    "ptr2ind": ("ptr2ind(Tensor ptr, int E) -> Tensor", _op_ptr2ind),
}
_LIBRARIES = []  # torch.library handles must stay alive


def _schema_known(name: str) -> bool:
    try:
        torch._C._dispatch_find_schema_or_throw("torch_sparse::" + name, "")
    except RuntimeError:
        return False
    return True


def _register_operators() -> None:
    if _LIBRARIES:
        return
    undefined = [name for name in _OPERATORS if not _schema_known(name)]
    if undefined:
        fragment = torch.library.Library("torch_sparse", "FRAGMENT")
        for name in undefined:
            fragment.define(_OPERATORS[name][0])
        _LIBRARIES.append(fragment)
    for key in ("CUDA", "AutogradCUDA"):
        impl = torch.library.Library("torch_sparse", "IMPL", key)
        for name, (_schema, fn) in _OPERATORS.items():
            impl.impl(name, fn)
        _LIBRARIES.append(impl)


# ---------------------------------------------------------------- frontend adaptation
_ORIGINALS = {}  # "module.attr" -> the implementation that was there before adaptation


def _install(owner, attr: str, label: str, make_adapter) -> None:
    """Replace owner.attr by make_adapter(original).  The original is looked
    through any adapter installed earlier (a reload adapts the original
    again, never an adapter)."""
    current = getattr(owner, attr)
    original = getattr(current, "__ops_gnn_original__", current)
    adapter = make_adapter(original)
    adapter.__ops_gnn_original__ = original
    adapter.__name__ = getattr(original, "__name__", attr)
    adapter.__doc__ = getattr(original, "__doc__", None)
    setattr(owner, attr, adapter)
    _ORIGINALS[label] = original


def _rowptr_of(src, other):
    """The CSR pointer of a SparseTensor: its cached rowptr, or one built from
    its (sorted, in-range) row index by the registered ind2ptr."""
    storage = src.storage
    if storage.has_rowptr():
        return storage.rowptr()
    row = storage.row() if storage.has_row() else None
    if row is None or row.dtype != torch.int64 or row.device != other.device:
        raise ValueError("SparseTensor row must be int64 on the same GPU")
    if row.numel():
        unsorted, lo, hi = _native.index_probe(row)
        if lo < 0 or hi >= src.sparse_size(0):
            raise ValueError("SparseTensor row out of range")
        if unsorted:
            raise ValueError("SparseTensor row must be sorted")
    return storage.rowptr()


def _sparse_tensor_spmm(src, other, reduce="sum"):
    """SparseTensor @ GPU dense (reference _sparse_spmm, :366-393): the
    storage's own metadata is checked when present and reused by backward."""
    _check_mat(other)
    r = _check_reduce(reduce)
    if other.size(-2) != src.sparse_size(1):
        raise ValueError("sparse columns must match dense N")
    storage = src.storage
    ptr = _rowptr_of(src, other)
    col, value = storage.col(), storage.value()

    def present(name):
        return getattr(storage, name)() if getattr(storage, "has_" + name)() else None

    csr = _Csr(ptr, col, other.size(-2), row=present("row"), rowcount=present("rowcount"),
               colptr=present("colptr"), perm=present("csr2csc"))
    _check_value(value, csr.edges, other)
    if ptr.device != other.device or col.device != other.device:
        raise ValueError("indices and mat must be on the same GPU")
    out, _arg = _prove_and_run(csr, value, other, r)
    return out


def adapt_frontends(torch_sparse_module=None, pyg_module=None) -> bool:
    """Route the torch_sparse (and PyG) SpMM frontends to this module for GPU
    operands; returns True when torch_sparse was adapted.  Run at import;
    callable again (e.g. after torch_sparse is imported later)."""
    ts = torch_sparse_module
    if ts is None:
        if importlib.util.find_spec("torch_sparse") is None:
            return False
        ts = importlib.import_module("torch_sparse")
    mm = sys.modules.get(ts.__name__ + ".matmul") or importlib.import_module(ts.__name__ + ".matmul")
    coo = sys.modules.get(ts.__name__ + ".spmm") or importlib.import_module(ts.__name__ + ".spmm")

    def coo_adapter(original):
        def spmm(index, value, m, n, matrix):
            if _on_gpu(matrix):
                return coo_spmm(index, value, m, n, matrix)
            return original(index, value, m, n, matrix)
        return spmm

    def spmm_adapter(original):
        def spmm(src, other, reduce="sum"):
            if _on_gpu(other):
                return _sparse_tensor_spmm(src, other, reduce)
            return original(src, other, reduce)
        return spmm

    def matmul_adapter(original):
        def matmul(src, other, reduce="sum"):
            if _on_gpu(other):
                return _sparse_tensor_spmm(src, other, reduce)
            return original(src, other, reduce)
        return matmul

    def dunder_adapter(original):
        def __matmul__(self, other):
            if _on_gpu(other):
                return _sparse_tensor_spmm(self, other, "sum")
            return original(self, other)
        return __matmul__

    _install(ts, "spmm", "torch_sparse.spmm", coo_adapter)
    _install(coo, "spmm", "torch_sparse.spmm.spmm", coo_adapter)
    _install(mm, "spmm", "torch_sparse.matmul.spmm", spmm_adapter)
    _install(mm, "matmul", "torch_sparse.matmul.matmul", matmul_adapter)
    _install(ts, "matmul", "torch_sparse.matmul", matmul_adapter)
    _install(ts.SparseTensor, "spmm", "SparseTensor.spmm", spmm_adapter)
    _install(ts.SparseTensor, "matmul", "SparseTensor.matmul", matmul_adapter)
    _install(ts.SparseTensor, "__matmul__", "SparseTensor.__matmul__", dunder_adapter)

    # PyG captures `spmm` by value in its utils and in the GCN / GIN modules
    # (reference :442-459); adapt each alias for SparseTensor x GPU operands.
    pyg = pyg_module
    if pyg is None and importlib.util.find_spec("torch_geometric") is not None:
        pyg = importlib.import_module("torch_geometric")
    if pyg is not None:
        utils = importlib.import_module(pyg.__name__ + ".utils")
        inner = importlib.import_module(pyg.__name__ + ".utils._spmm")

        def pyg_adapter(original):
            def spmm(src, other, reduce="sum"):
                if isinstance(src, ts.SparseTensor) and _on_gpu(other):
                    return _sparse_tensor_spmm(src, other, reduce)
                return original(src, other, reduce)
            return spmm

        _install(inner, "spmm", "torch_geometric.utils._spmm.spmm", pyg_adapter)
        utils.spmm = inner.spmm
        for conv in ("gcn_conv", "gin_conv"):
            module = importlib.import_module(f"{pyg.__name__}.nn.conv.{conv}")
            _install(module, "spmm", f"torch_geometric.nn.conv.{conv}.spmm", pyg_adapter)
    return True


_register_operators()
adapt_frontends()
