"""DGL-style generalised CSR aggregation: spmm / bspmm.

Mirror of the reference python/ops_gnn/spmm.py:292-321 and bspmm.py:17-28:
the same call options (op, reduce, out, rhs), operand rules (copy_rhs may take
its edge features through ``x``), rank alignment, error messages and
reduction semantics (sum / mean / max / min; max and min propagate NaN; empty
rows give 0).  Every case runs on HIP kernels:
  copy_lhs and the binary messages (mul / add / sub / div with an edge
  operand) -> the CSR engine in gather mode (ogn_spmm_csr_ex, DGL semantics);
  copy_rhs -> the contiguous-segment engine over the edge rows.
fp16 accumulates in fp32 (the reference's fp16 kernels accumulate in fp16;
the fp32 result is the more accurate one and is compared by tolerance).
Autograd: sum / mean with copy_lhs or mul run backward on the same kernels
(transposed SpMM for the node operand, SDDMM for the edge operand); other
combinations raise NotImplementedError when a gradient is required.
"""

import math
from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from . import _lib, _native

_MESSAGE_OPS = {"copy_lhs", "copy_rhs", "add", "sub", "mul", "div"}
_REDUCE_OPS = {"sum", "max", "min", "mean"}
_R = {"sum": _lib.R_SUM, "mean": _lib.R_MEAN, "min": _lib.R_MIN, "max": _lib.R_MAX}
_MSG = {"mul": _lib.MSG_MUL, "add": _lib.MSG_ADD, "sub": _lib.MSG_SUB, "div": _lib.MSG_DIV,
        "copy_lhs": _lib.MSG_MUL}
_FEATURE_DTYPES = (torch.float16, torch.float32, torch.bfloat16)


@dataclass(frozen=True)
class _SpmmRequest:
    indptr: torch.Tensor
    indices: torch.Tensor
    x: Optional[torch.Tensor]
    op: str
    reduce: str
    out: Optional[torch.Tensor]
    rhs: Optional[torch.Tensor]
    batched: bool


def _normalize_operands(x, rhs, op):
    if op == "copy_lhs":
        if x is None or rhs is not None:
            raise ValueError("copy_lhs requires x and does not accept rhs")
        return x, None
    if op == "copy_rhs":
        if rhs is not None:
            if x is not None:
                raise ValueError("copy_rhs accepts edge features through either x or rhs, not both")
            return None, rhs
        if x is None:
            raise ValueError("copy_rhs requires edge features")
        return None, x
    if x is None or rhs is None:
        raise ValueError(f"{op} requires both x and rhs")
    return x, rhs


def _validate(request: _SpmmRequest, lhs, rhs):
    features = [v for v in (lhs, rhs) if v is not None]
    for name, value in (("indptr", request.indptr), ("indices", request.indices)):
        if not isinstance(value, torch.Tensor):
            raise TypeError(f"{name} must be a Tensor")
    device = features[0].device
    if device.type != "cuda" or any(v.device != device for v in features):
        raise RuntimeError("spmm: feature tensors must be on the same GPU")
    if request.indptr.device != device or request.indices.device != device:
        raise RuntimeError("spmm: CSR tensors and features must be on the same GPU")
    indptr, indices = request.indptr, request.indices
    if indptr.dim() != 1 or indices.dim() != 1:
        raise RuntimeError("spmm: CSR tensors must be one-dimensional")
    if indptr.numel() == 0:
        raise RuntimeError("spmm: indptr must be nonempty")
    if indptr.dtype not in (torch.int32, torch.int64) or indices.dtype != indptr.dtype:
        raise RuntimeError("spmm: CSR tensors must have the same int32 or int64 dtype")
    if any(v.dtype not in _FEATURE_DTYPES for v in features):
        raise RuntimeError("spmm: features must use float16 or float32")
    if lhs is not None and rhs is not None and lhs.dtype != rhs.dtype:
        raise RuntimeError("x and rhs must have the same dtype")
    ranks = [v.dim() for v in features]
    if any(r < 1 for r in ranks):
        raise RuntimeError("spmm feature tensors must have at least one dimension")
    if request.batched:
        if max(ranks) < 3:
            raise RuntimeError("bspmm requires at least one feature tensor with rank 3 or higher")
    elif any(r > 2 for r in ranks):
        raise RuntimeError("spmm supports scalar or two-dimensional features; use bspmm for higher-rank features")
    rows, edges = indptr.numel() - 1, indices.numel()
    if rhs is not None and rhs.size(0) != edges:
        raise RuntimeError("rhs.size(0) must equal indices.numel()")
    n = lhs.size(0) if lhs is not None else (1 << 62)

    def compute():
        status = torch.empty(1, dtype=torch.int32, device=device)
        _lib.check(_lib.lib.ogn_validate_csr(
            _lib.dptr(indptr.contiguous()), _lib.dptr(indices.contiguous()),
            _lib.I64 if indptr.dtype == torch.int64 else _lib.I32, rows, edges, n, _lib.dptr(status),
            _lib.stream_of(indptr)), "spmm")
        return int(status.item())

    code = compute()
    if code == 1:
        first, last = int(indptr[0].item()), int(indptr[-1].item())
        if first != 0 or last != edges:
            raise RuntimeError("indptr must start at zero and end at indices.numel()")
        raise RuntimeError("indptr must be non-decreasing")
    if code == 2:
        raise RuntimeError("indices are out of range for x")


def _align(lhs, rhs):
    """Pad missing feature dims right after the item axis (reference spmm.py:133-146)."""
    rank = max(lhs.dim(), rhs.dim()) - 1

    def pad(v):
        extra = rank - (v.dim() - 1)
        return v if extra == 0 else v.reshape((v.shape[0],) + (1,) * extra + tuple(v.shape[1:]))

    return pad(lhs), pad(rhs)


def _forward(request: _SpmmRequest, lhs, rhs) -> torch.Tensor:
    indptr = request.indptr.contiguous()
    indices = request.indices.contiguous()
    rows, edges = indptr.numel() - 1, indices.numel()
    reduce = _R[request.reduce]
    if request.op == "copy_rhs":
        feat = tuple(rhs.shape[1:])
        k = math.prod(feat)
        src3 = rhs.contiguous().reshape(1, edges, k)
        out3, _ = _native.segment_reduce(src3, indptr.to(torch.int64).reshape(1, -1), rows, reduce,
                                         _lib.SEM_DGL)
        return out3.reshape((rows,) + feat)
    if request.op == "copy_lhs":
        x, w, wshape = lhs, None, None
        feat = tuple(lhs.shape[1:])
    else:
        x, w = _align(lhs, rhs)
        feat = tuple(torch.broadcast_shapes(x.shape[1:], w.shape[1:]))
        if tuple(x.shape[1:]) != feat:
            x = x.expand((x.shape[0],) + feat)
        if math.prod(w.shape[1:]) != 1 and tuple(w.shape[1:]) != feat:
            w = w.expand((edges,) + feat)
    k = math.prod(feat)
    n = x.size(0)
    mat = x.contiguous().reshape(n, k)
    value, width = None, 1
    if w is not None:
        width = 1 if math.prod(w.shape[1:]) == 1 else k
        value = w.contiguous().reshape(edges, width) if width > 1 else w.contiguous().reshape(edges)
    out = torch.empty((rows, k), dtype=mat.dtype, device=mat.device)
    if out.numel():
        ws_bytes = _lib.lib.ogn_spmm_csr_workspace_size(rows, edges, k, 1, _lib.TORCH_TO_OGN[mat.dtype], reduce)
        ws = _lib.workspace(ws_bytes, mat.device)
        rc = _lib.lib.ogn_spmm_csr_ex(
            _lib.dptr(indptr), _lib.dptr(indices), _lib.I64 if indptr.dtype == torch.int64 else _lib.I32,
            _lib.dptr(value), width, _lib.dptr(mat), _lib.TORCH_TO_OGN[mat.dtype], 1, rows, n, k, edges,
            _lib.dptr(out), _lib.TORCH_TO_OGN[mat.dtype], None, reduce, _MSG[request.op], _lib.SPMM_DGL,
            _lib.dptr(ws), ws_bytes, _lib.stream_of(mat))
        _lib.check(rc, "spmm")
    return out.reshape((rows,) + feat)


class _DglSpmm(torch.autograd.Function):
    """sum / mean aggregation of copy_lhs or mul messages with gradients."""

    @staticmethod
    def forward(ctx, x, w, request):
        out = _forward(request, x, w)
        ctx.request = request
        ctx.save_for_backward(x, w if w is not None else x)
        ctx.has_w = w is not None
        return out

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad):
        from .convert import ind2ptr_tensor, ptr2ind_tensor
        from .sddmm_csr import sddmm_csr

        request = ctx.request
        x, w_saved = ctx.saved_tensors
        w = w_saved if ctx.has_w else None
        indptr = request.indptr.to(torch.int64)
        indices = request.indices.to(torch.int64)
        rows, edges = indptr.numel() - 1, indices.numel()
        g = grad.float().reshape(rows, -1)
        if request.reduce == "mean":
            g = g / (indptr[1:] - indptr[:-1]).clamp_min(1).to(torch.float32).unsqueeze(-1)
        dx = dw = None
        if ctx.needs_input_grad[0]:
            perm = torch.argsort(indices, stable=True)
            colptr = ind2ptr_tensor(indices[perm], x.size(0))
            row = ptr2ind_tensor(indptr, edges)
            tw = None
            if w is not None:
                tw = w.reshape(edges, -1).float()[perm].contiguous()
                tw = tw.reshape(edges) if tw.size(1) == 1 else tw
            dx = _native.spmm_forward(colptr, row[perm].contiguous(), tw, g.contiguous(), 0, torch.float32)[0]
            dx = dx.reshape(x.shape).to(x.dtype)
        if ctx.needs_input_grad[1] and w is not None:
            xf = x.float().reshape(x.size(0), -1).contiguous()
            width = w.reshape(edges, -1).size(1)
            dw = sddmm_csr(indptr, indices, g.contiguous(), xf, "dot" if width == 1 else "mul", 0, 2)
            dw = dw.reshape(w.shape).to(w.dtype)
        return dx, dw, None


def _spmm(request: _SpmmRequest) -> torch.Tensor:
    api = "bspmm" if request.batched else "spmm"
    for name, value in (("indptr", request.indptr), ("indices", request.indices), ("x", request.x),
                        ("rhs", request.rhs), ("out", request.out)):
        if value is not None and not isinstance(value, torch.Tensor):
            raise TypeError(f"{api}: {name} must be a Tensor")
    if not isinstance(request.op, str) or request.op not in _MESSAGE_OPS:
        raise RuntimeError(f"{api}: op must be copy_lhs, copy_rhs, add, sub, mul or div")
    if not isinstance(request.reduce, str) or request.reduce not in _REDUCE_OPS:
        raise RuntimeError(f"{api}: reduce must be sum, max, min or mean")
    lhs, edge = _normalize_operands(request.x, request.rhs, request.op)
    _validate(request, lhs, edge)
    grad_required = torch.is_grad_enabled() and any(v is not None and v.requires_grad for v in (lhs, edge))
    if grad_required:
        if request.reduce in ("sum", "mean") and request.op in ("copy_lhs", "mul"):
            result = _DglSpmm.apply(lhs, edge, request)
        else:
            raise NotImplementedError(f"{api}: gradients of op={request.op}, reduce={request.reduce} are not "
                                      "implemented on the GPU path")
    else:
        result = _forward(request, lhs, edge)
    out = request.out
    if out is None:
        return result
    if grad_required:
        raise RuntimeError("out is not supported when feature tensors require gradients")
    if out.shape != result.shape or out.dtype != result.dtype or out.device != result.device:
        raise RuntimeError("out must match the result shape, dtype and device")
    if not out.is_contiguous() or out.requires_grad:
        raise RuntimeError("out must be contiguous and must not require gradients")
    out.copy_(result)
    return out


def _parse_call_options(api: str, args: tuple, kwargs: dict) -> Tuple:
    names = ("op", "reduce", "out", "rhs")
    if len(args) > len(names):
        raise TypeError(f"{api} accepts at most seven positional arguments")
    options = {"op": "copy_lhs", "reduce": "sum", "out": None, "rhs": None}
    for name, value in zip(names, args):
        if name in kwargs:
            raise TypeError(f"{api} got multiple values for argument '{name}'")
        options[name] = value
    unexpected = set(kwargs) - set(names)
    if unexpected:
        raise TypeError(f"{api} got an unexpected keyword argument '{sorted(unexpected)[0]}'")
    options.update(kwargs)
    return options["op"], options["reduce"], options["out"], options["rhs"]


def spmm(indptr: torch.Tensor, indices: torch.Tensor, x: Optional[torch.Tensor] = None, *args, **kwargs):
    """Generalised CSR aggregation: out[r] = reduce_{e in row r} msg(x[indices[e]], rhs[e])."""
    op, reduce, out, rhs = _parse_call_options("spmm", args, kwargs)
    return _spmm(_SpmmRequest(indptr, indices, x, op, reduce, out, rhs, False))


def bspmm(indptr: torch.Tensor, indices: torch.Tensor, x: Optional[torch.Tensor] = None, *args, **kwargs):
    """Batched form of :func:`spmm`: at least one feature tensor has rank >= 3;
    trailing feature dims broadcast after the item axis."""
    op, reduce, out, rhs = _parse_call_options("bspmm", args, kwargs)
    return _spmm(_SpmmRequest(indptr, indices, x, op, reduce, out, rhs, True))
