"""DGL-style generalised CSR aggregation: spmm / bspmm.

Drop-in for the reference's python/ops_gnn/spmm.py:292-321 and
bspmm.py:17-28 call contract: the same call options (op, reduce, out, rhs),
operand rules (copy_rhs may take its edge features through ``x``), rank
alignment, error messages and reduction semantics (sum / mean / max / min;
max and min propagate NaN; empty rows give 0).  Every case runs on HIP
kernels:
  copy_lhs and the binary messages (mul / add / sub / div with an edge
  operand) -> the CSR engine in gather mode (ogn_spmm_csr_ex, DGL semantics);
  copy_rhs -> the contiguous-segment engine over the edge rows.
fp16 accumulates in fp32 (the reference's fp16 kernels accumulate in fp16;
the fp32 result is the more accurate one and is compared by tolerance).
Autograd covers every op x reduce (see _DglSpmm): transposed SpMM for the
node operand, SDDMM for the edge operand, and the forward's arg edges for
max / min.
"""

import math
from typing import NamedTuple, Optional, Tuple

import torch

from . import _lib, _native

_MESSAGE_OPS = {"copy_lhs", "copy_rhs", "add", "sub", "mul", "div"}
_REDUCE_OPS = {"sum", "max", "min", "mean"}
_R = {"sum": _lib.R_SUM, "mean": _lib.R_MEAN, "min": _lib.R_MIN, "max": _lib.R_MAX}
_MSG = {"mul": _lib.MSG_MUL, "add": _lib.MSG_ADD, "sub": _lib.MSG_SUB, "div": _lib.MSG_DIV,
        "copy_lhs": _lib.MSG_MUL}
_FEATURE_DTYPES = (torch.float16, torch.float32, torch.bfloat16)

# Call options after (indptr, indices, x), in positional order, with defaults.
_OPTIONS = (("op", "copy_lhs"), ("reduce", "sum"), ("out", None), ("rhs", None))


class _Call(NamedTuple):
    """One spmm / bspmm call: the CSR pattern and the message / reduction
    (the feature operands travel separately, as autograd inputs)."""
    api: str  # "spmm" or "bspmm"
    indptr: torch.Tensor
    indices: torch.Tensor
    op: str
    reduce: str

    @property
    def batched(self) -> bool:
        return self.api == "bspmm"


def _bind_options(api: str, args: tuple, kwargs: dict) -> dict:
    """The call options from the extra positional and keyword arguments,
    refused as Python refuses a bad call of a function with this signature."""
    names = [name for name, _ in _OPTIONS]
    if len(args) > len(names):
        raise TypeError(f"{api} accepts at most seven positional arguments")
    given = dict(zip(names, args))
    twice = [name for name in given if name in kwargs]
    if twice:
        raise TypeError(f"{api} got multiple values for argument '{twice[0]}'")
    unknown = sorted(set(kwargs).difference(names))
    if unknown:
        raise TypeError(f"{api} got an unexpected keyword argument '{unknown[0]}'")
    return {**dict(_OPTIONS), **given, **kwargs}


def _operands(op: str, x, rhs):
    """(node, edge): the operand gathered per edge through `indices`, and the
    one holding a row per edge.  copy_rhs takes its edge rows from whichever
    of x / rhs was given."""
    if op == "copy_rhs":
        supplied = [t for t in (rhs, x) if t is not None]
        if len(supplied) > 1:
            raise ValueError("copy_rhs accepts edge features through either x or rhs, not both")
        if not supplied:
            raise ValueError("copy_rhs requires edge features")
        return None, supplied[0]
    if op == "copy_lhs":
        if x is None or rhs is not None:
            raise ValueError("copy_lhs requires x and does not accept rhs")
        return x, None
    if x is None or rhs is None:
        raise ValueError(f"{op} requires both x and rhs")
    return x, rhs


def _check_arguments(api: str, tensors: dict, op, reduce) -> None:
    """Argument kinds and option values, before any operand is looked at."""
    for name, value in tensors.items():
        if value is not None and not isinstance(value, torch.Tensor):
            raise TypeError(f"{api}: {name} must be a Tensor")
    if not (isinstance(op, str) and op in _MESSAGE_OPS):
        raise RuntimeError(f"{api}: op must be copy_lhs, copy_rhs, add, sub, mul or div")
    if not (isinstance(reduce, str) and reduce in _REDUCE_OPS):
        raise RuntimeError(f"{api}: reduce must be sum, max, min or mean")


def _deliver(result: torch.Tensor, out: Optional[torch.Tensor], grad_required: bool) -> torch.Tensor:
    """The result, or `out` holding it (refused under autograd, or when it
    does not match the result exactly)."""
    if out is None:
        return result
    refusals = (
        (lambda: grad_required, "out is not supported when feature tensors require gradients"),
        (lambda: (out.shape, out.dtype, out.device) != (result.shape, result.dtype, result.device),
         "out must match the result shape, dtype and device"),
        (lambda: not out.is_contiguous() or out.requires_grad,
         "out must be contiguous and must not require gradients"),
    )
    for refused, message in refusals:
        if refused():
            raise RuntimeError(message)
    return out.copy_(result)


def _validate(request: _Call, lhs, rhs):
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


def _forward(request: _Call, lhs, rhs, want_arg: bool = False):
    """(out, arg): out [rows, *feat]; arg [rows, k] int64 (the edge each
    max / min element came from, E for an empty row; the first NaN edge for
    a NaN result; the first extremal edge among ties) when `want_arg`."""
    indptr = request.indptr.contiguous()
    indices = request.indices.contiguous()
    rows, edges = indptr.numel() - 1, indices.numel()
    reduce = _R[request.reduce]
    if request.op == "copy_rhs":
        feat = tuple(rhs.shape[1:])
        k = math.prod(feat)
        src3 = rhs.contiguous().reshape(1, edges, k)
        out3, arg3 = _native.segment_reduce(src3, indptr.to(torch.int64).reshape(1, -1), rows, reduce,
                                            _lib.SEM_DGL, need_arg=want_arg)
        return out3.reshape((rows,) + feat), (None if arg3 is None else arg3.reshape(rows, k))
    if request.op == "copy_lhs":
        x, w = lhs, None
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
    arg = torch.empty((rows, k), dtype=torch.int64, device=mat.device) if want_arg else None
    if out.numel():
        ws_bytes = _lib.lib.ogn_spmm_csr_workspace_size(rows, edges, k, 1, _lib.TORCH_TO_OGN[mat.dtype], reduce)
        ws = _lib.workspace(ws_bytes, mat.device)
        rc = _lib.lib.ogn_spmm_csr_ex(
            _lib.dptr(indptr), _lib.dptr(indices), _lib.I64 if indptr.dtype == torch.int64 else _lib.I32,
            _lib.dptr(value), width, _lib.dptr(mat), _lib.TORCH_TO_OGN[mat.dtype], 1, rows, n, k, edges,
            _lib.dptr(out), _lib.TORCH_TO_OGN[mat.dtype], _lib.dptr(arg), reduce, _MSG[request.op], _lib.SPMM_DGL,
            _lib.dptr(ws), ws_bytes, _lib.stream_of(mat))
        _lib.check(rc, "spmm")
    return out.reshape((rows,) + feat), arg


def _message_shapes(request: _Call, x, w):
    """(feat, aligned x shape, aligned w shape) of the forward's messages."""
    if request.op == "copy_rhs":
        return tuple(w.shape[1:]), None, tuple(w.shape)
    if request.op == "copy_lhs":
        return tuple(x.shape[1:]), tuple(x.shape), None
    xa, wa = _align(x, w)
    return tuple(torch.broadcast_shapes(xa.shape[1:], wa.shape[1:])), tuple(xa.shape), tuple(wa.shape)


class _DglSpmm(torch.autograd.Function):
    """Gradients of every op x reduce, matching the reference's torch
    composition (python/ops_gnn/spmm.py:148-208): message m_e = phi(x[col[e]],
    w[e]) with phi in {x, w, x + w, x - w, x * w, x / w}, reduced per row.

    sum / mean: each message's gradient is g_e = grad[row(e)] (/ deg).  The
      node gradient is a transposed SpMM of g with edge weights d phi / dx
      (none, or w, or 1 / w); the edge gradient is g_e * d phi / dw, formed
      with the SDDMM kernels (a dot when w has one weight per edge).
    max / min: only the edge each output element came from (the forward's
      arg) receives that element's gradient; scattered with index_add.
    Gradients are summed back over broadcast feature dims; fp32 throughout,
    cast to the operand dtype at the end.
    """

    @staticmethod
    def forward(ctx, x, w, request):
        extremum = request.reduce in ("max", "min")
        out, arg = _forward(request, x, w, want_arg=extremum)
        ctx.request = request
        ctx.save_for_backward(x, w, arg)
        if arg is not None:
            ctx.mark_non_differentiable(arg)
        return out

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad):
        from .convert import ind2ptr_tensor, ptr2ind_tensor
        from .sddmm_csr import sddmm_csr

        request = ctx.request
        x, w, arg = ctx.saved_tensors
        op = request.op
        want_x = ctx.needs_input_grad[0] and x is not None
        want_w = ctx.needs_input_grad[1] and w is not None
        indptr = request.indptr.to(torch.int64).contiguous()
        col = request.indices.to(torch.int64).contiguous()
        rows, edges = indptr.numel() - 1, col.numel()
        feat, x_shape, w_shape = _message_shapes(request, x, w)
        k = math.prod(feat)
        g = grad.float().reshape(rows, k)
        # operands as the forward saw them: x [N, k]; w [E, width] (width 1 or k)
        xk = None if x is None else x.float().reshape(x_shape).expand((x.size(0),) + feat).reshape(x.size(0), k)
        width = 1 if w is None or math.prod(w.shape[1:]) == 1 else k
        wk = None
        if w is not None:
            wk = w.float().reshape(edges, 1) if width == 1 else \
                w.float().reshape(w_shape).expand((edges,) + feat).reshape(edges, k)
        dx = torch.zeros_like(xk) if want_x else None
        dw = torch.zeros((edges, width), dtype=torch.float32, device=g.device) if want_w else None
        if request.reduce in ("sum", "mean"):
            if request.reduce == "mean":
                g = g / indptr.diff().clamp_min(1).to(torch.float32).unsqueeze(-1)
            g = g.contiguous()
            if want_x:
                # d phi / dx per edge: 1 (copy_lhs, add, sub), w (mul), 1 / w (div)
                scale = wk if op == "mul" else (1.0 / wk if op == "div" else None)
                sorted_col, perm = torch.sort(col, stable=True)
                colptr = ind2ptr_tensor(sorted_col, x.size(0))
                row_t = ptr2ind_tensor(indptr, edges)[perm].contiguous()
                tw = None
                if scale is not None:
                    tw = scale[perm].contiguous()
                    tw = tw.reshape(edges) if width == 1 else tw
                dx = _native.spmm_forward(colptr, row_t, tw, g, 0, torch.float32)[0]
            if want_w:
                if op in ("copy_rhs", "add", "sub"):
                    if width == 1:
                        gw = ptr2ind_tensor(indptr, edges)
                        dw = g.sum(-1).index_select(0, gw).unsqueeze(-1)
                    else:
                        dw = sddmm_csr(indptr, col, g, None, "copy_lhs", 0, 2).reshape(edges, k).float()
                    if op == "sub":
                        dw = -dw
                else:  # mul: g_e * x[col]; div: -g_e * x[col] / w^2
                    xc = xk.contiguous()
                    if width == 1:
                        dw = sddmm_csr(indptr, col, g, xc, "dot", 0, 2).float().unsqueeze(-1)
                    else:
                        dw = sddmm_csr(indptr, col, g, xc, "mul", 0, 2).reshape(edges, k).float()
                    if op == "div":
                        dw = -dw / (wk * wk)
        else:
            hit = arg < edges
            a = torch.where(hit, arg, torch.zeros_like(arg))
            ge = torch.where(hit, g, torch.zeros_like(g))
            feature = torch.arange(k, device=g.device).expand(rows, k)
            wv = None if wk is None else (wk[a, 0] if width == 1 else wk[a, feature])
            src = col[a] if xk is not None else None
            if want_x:
                dphi_dx = ge if op in ("copy_lhs", "add", "sub") else (ge * wv if op == "mul" else ge / wv)
                dx.view(-1).index_add_(0, (src * k + feature).reshape(-1), dphi_dx.reshape(-1))
            if want_w:
                if op in ("copy_rhs", "add"):
                    dphi_dw = ge
                elif op == "sub":
                    dphi_dw = -ge
                else:
                    xv = xk[src, feature]
                    dphi_dw = ge * xv if op == "mul" else -ge * xv / (wv * wv)
                slot = a if width == 1 else a * k + feature
                dw.view(-1).index_add_(0, slot.reshape(-1), dphi_dw.reshape(-1))
        gx = gw_out = None
        if want_x:
            gx = dx.reshape((x.size(0),) + feat).sum_to_size(x_shape).reshape(x.shape).to(x.dtype)
        if want_w:
            if width == 1:
                gw_out = dw.reshape(w.shape).to(w.dtype)
            else:
                gw_out = dw.reshape((edges,) + feat).sum_to_size(w_shape).reshape(w.shape).to(w.dtype)
        return gx, gw_out, None


def _aggregate(api: str, indptr, indices, x, args: tuple, kwargs: dict) -> torch.Tensor:
    options = _bind_options(api, args, kwargs)
    op, reduce, out, rhs = options["op"], options["reduce"], options["out"], options["rhs"]
    _check_arguments(api, {"indptr": indptr, "indices": indices, "x": x, "rhs": rhs, "out": out}, op, reduce)
    node, edge = _operands(op, x, rhs)
    call = _Call(api, indptr, indices, op, reduce)
    _validate(call, node, edge)
    grad_required = torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (node, edge))
    result = _DglSpmm.apply(node, edge, call) if grad_required else _forward(call, node, edge)[0]
    return _deliver(result, out, grad_required)


def spmm(indptr: torch.Tensor, indices: torch.Tensor, x: Optional[torch.Tensor] = None, *args, **kwargs):
    """Generalised CSR aggregation: out[r] = reduce_{e in row r} msg(x[indices[e]], rhs[e])."""
    return _aggregate("spmm", indptr, indices, x, args, kwargs)


def bspmm(indptr: torch.Tensor, indices: torch.Tensor, x: Optional[torch.Tensor] = None, *args, **kwargs):
    """Batched form of :func:`spmm`: at least one feature tensor has rank >= 3;
    trailing feature dims broadcast after the item axis."""
    return _aggregate("bspmm", indptr, indices, x, args, kwargs)
