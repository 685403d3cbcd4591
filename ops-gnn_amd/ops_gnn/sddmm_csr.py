"""Generalised sampled dense-dense matrix multiplication on a CSR graph.

Mirror of the reference python/ops_gnn/sddmm_csr.py:126-173 (argument
contract, target aliases, 1-D operand squeezing, `out` handling) over the
HIP kernel ogn_sddmm_csr.  float16 / float32 as in the reference, plus
bfloat16; fp32 compute with one final rounding.
"""

from typing import Optional, Tuple

import torch

from . import _lib, _native
from ._lib import check, dptr, lib, stream_of

_MESSAGE_OPS = {"dot", "add", "sub", "mul", "div", "copy_lhs", "copy_rhs"}
_TARGET_ALIASES = {"u": 0, "src": 0, "e": 1, "edge": 1, "v": 2, "dst": 2}
_DTYPES = (torch.float16, torch.float32, torch.bfloat16)


def _normalize_target(target, name: str) -> int:
    if isinstance(target, bool):
        raise ValueError(f"sddmm_csr: {name} must be 0, 1, 2, u, e or v")
    if isinstance(target, int):
        if target in (0, 1, 2):
            return target
        raise ValueError(f"sddmm_csr: {name} must be 0, 1, 2, u, e or v")
    if isinstance(target, str):
        alias = _TARGET_ALIASES.get(target.lower())
        if alias is not None:
            return alias
    raise ValueError(f"sddmm_csr: {name} must be 0, 1, 2, u, e or v")


def _operand_flags(op: str) -> Tuple[bool, bool]:
    if op not in _MESSAGE_OPS:
        raise ValueError("sddmm_csr: op must be dot, add, sub, mul, div, copy_lhs or copy_rhs")
    if op == "copy_lhs":
        return True, False
    if op == "copy_rhs":
        return False, True
    return True, True


def _check_operand(name: str, value, required: bool) -> None:
    if not required:
        if value is not None:
            raise ValueError(f"sddmm_csr: {name} is not used by this op")
        return
    if value is None:
        raise ValueError(f"sddmm_csr: {name} is required by this op")
    if not isinstance(value, torch.Tensor):
        raise TypeError(f"sddmm_csr: {name} must be a Tensor")
    if value.dim() not in (1, 2):
        raise ValueError(f"sddmm_csr: {name} must be one- or two-dimensional")
    if value.dtype not in _DTYPES:
        raise ValueError(f"sddmm_csr: {name} must be float16, bfloat16 or float32")


# Validation results per (indices version, indptr version, dst rows): the
# reference re-validates on every call (sddmm_csr.cpp:78-126); a mutated
# tensor bumps its version and is checked again.
_CSR_CHECKS = _native._VersionCache(limit=128)


def _csr_status(indptr, indices, m, nnz, n) -> int:
    import weakref

    per_indices = _CSR_CHECKS.get(indices, dict)
    key = (id(indptr), indptr.data_ptr(), indptr._version, n)
    hit = per_indices.get(key)
    if hit is not None and hit[0]() is indptr:
        return hit[1]
    status = torch.empty(1, dtype=torch.int32, device=indptr.device)
    check(lib.ogn_validate_csr(dptr(indptr.contiguous()), dptr(indices.contiguous()),
                               _lib.I64 if indptr.dtype == torch.int64 else _lib.I32, m, nnz, n, dptr(status),
                               stream_of(indptr)), "sddmm_csr")
    code = int(status.item())
    if len(per_indices) > 8:
        per_indices.clear()
    per_indices[key] = (weakref.ref(indptr), code)
    return code


def _check_csr(indptr, indices, lhs, rhs, lt, rt, use_l, use_r):
    """reference csrc/npu/sddmm_csr/op_host/sddmm_csr.cpp:78-126 (CheckCsr) and
    CheckTargetRange: one fused device check, one small host read."""
    if indptr.dim() != 1 or indices.dim() != 1 or indptr.numel() < 1:
        raise RuntimeError("sddmm_csr: indptr and indices must be one-dimensional; indptr must be nonempty")
    if indptr.dtype not in (torch.int32, torch.int64) or indices.dtype != indptr.dtype:
        raise RuntimeError("sddmm_csr: indptr and indices must have the same int32/int64 dtype")
    m, nnz = indptr.numel() - 1, indices.numel()
    dst_rows = []
    if use_l and lt == 2:
        dst_rows.append(lhs.size(0))
    if use_r and rt == 2:
        dst_rows.append(rhs.size(0))
    n = min(dst_rows) if dst_rows else (1 << 62)
    code = _csr_status(indptr, indices, m, nnz, n)
    if code == 2:
        raise RuntimeError("sddmm_csr: CSR indices are out of range for dst features")
    if code:
        raise RuntimeError("sddmm_csr: invalid CSR (indptr/indices)")
    for name, value, target, used in (("lhs", lhs, lt, use_l), ("rhs", rhs, rt, use_r)):
        if not used:
            continue
        need = m if target == 0 else (nnz if target == 1 else None)
        if need is not None and value.size(0) < need:
            raise RuntimeError(f"sddmm_csr: {name} has too few rows for its target")


def sddmm_csr(indptr: torch.Tensor, indices: torch.Tensor, lhs: Optional[torch.Tensor] = None,
              rhs: Optional[torch.Tensor] = None, op: str = "dot", lhs_target=0, rhs_target=2,
              out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Run generalised SDDMM on a CSR graph.

    ``lhs`` / ``rhs`` are gathered by their targets (0/'u'/'src' = the CSR row,
    1/'e'/'edge' = the edge position, 2/'v'/'dst' = the CSR column).  ``dot``
    reduces the feature axis and returns ``(nnz,)``; the other ops return
    ``(nnz, k)``.  One-dimensional operands are treated as ``(rows, 1)`` and
    the trailing axis is squeezed from non-dot results.
    """
    if not isinstance(indptr, torch.Tensor):
        raise TypeError("sddmm_csr: indptr must be a Tensor")
    if not isinstance(indices, torch.Tensor):
        raise TypeError("sddmm_csr: indices must be a Tensor")
    use_l, use_r = _operand_flags(op)
    _check_operand("lhs", lhs, use_l)
    _check_operand("rhs", rhs, use_r)
    lt = _normalize_target(lhs_target, "lhs_target")
    rt = _normalize_target(rhs_target, "rhs_target")
    l2 = lhs.unsqueeze(-1) if use_l and lhs.dim() == 1 else lhs
    r2 = rhs.unsqueeze(-1) if use_r and rhs.dim() == 1 else rhs
    if use_l and use_r:
        if l2.device != r2.device:
            raise ValueError("sddmm_csr: lhs and rhs must be on the same device")
        if l2.dtype != r2.dtype:
            raise ValueError("sddmm_csr: lhs and rhs must have the same dtype")
        if l2.size(1) != r2.size(1):
            raise ValueError("sddmm_csr: lhs and rhs must have the same feature dim")
    feature = l2 if use_l else r2
    _lib.require_gpu(indptr, indices, feature, what="sddmm_csr")
    if indptr.device != feature.device or indices.device != feature.device:
        raise RuntimeError("sddmm_csr: indptr must be on the same GPU")
    k = feature.size(1)
    if k == 0:
        raise ValueError("sddmm_csr: the feature dim must be positive")
    nnz = indices.numel()
    is_dot = op == "dot"
    squeeze = (not is_dot) and ((lhs is None or lhs.dim() == 1) if use_l else True) and \
        ((rhs is None or rhs.dim() == 1) if use_r else True)
    final_shape = (nnz,) if (is_dot or squeeze) else (nnz, k)
    if out is not None:
        if not isinstance(out, torch.Tensor):
            raise TypeError("sddmm_csr: out must be a Tensor")
        if tuple(out.shape) != final_shape:
            raise ValueError(f"sddmm_csr: out must have shape {tuple(final_shape)}, got {tuple(out.shape)}")
        if out.dtype != feature.dtype or out.device != feature.device:
            raise RuntimeError("sddmm_csr: out must match the feature dtype and device")
        if not out.is_contiguous():
            raise RuntimeError("sddmm_csr: out must be contiguous")
    _check_csr(indptr, indices, l2, r2, lt, rt, use_l, use_r)
    result = out if out is not None else torch.empty(final_shape, dtype=feature.dtype, device=feature.device)
    if nnz == 0 or k == 0:
        return result
    l2c = l2.contiguous() if use_l else None
    r2c = r2.contiguous() if use_r else None
    ptr = indptr.contiguous()
    col = indices.contiguous()
    if is_dot and lt == 0 and rt == 2 and _native.sddmm_dot_xcd(ptr, col, l2c, r2c, result):
        return result
    ws_bytes = lib.ogn_sddmm_csr_workspace_size(nnz, k, _lib.TORCH_TO_OGN[feature.dtype])
    ws = _lib.workspace(ws_bytes, feature.device)
    rc = lib.ogn_sddmm_csr(dptr(ptr), dptr(col), _lib.I64 if ptr.dtype == torch.int64 else _lib.I32, ptr.numel() - 1,
                           nnz, dptr(l2c), 0 if l2c is None else l2c.size(0), lt, dptr(r2c),
                           0 if r2c is None else r2c.size(0), rt, k, _lib.TORCH_TO_OGN[feature.dtype],
                           _lib.SDDMM_OPS[op], dptr(result), dptr(ws), ws_bytes, stream_of(feature))
    check(rc, "sddmm_csr")
    return result


def value_grad(ptr: torch.Tensor, col: torch.Tensor, mat: torch.Tensor, grad: torch.Tensor, reduce: int,
               width: int) -> torch.Tensor:
    """SpMM edge-weight gradient (reference ValueGradCompute,
    csrc/npu/torch_sparse_spmm/op_kernel/arch35/torch_sparse_spmm_kernel.h:326-395):
    dv[e] = sum_b <grad[b, row(e)], mat[b, col(e)]> (/ deg for mean), or the
    per-feature product for k-wide weights.  One SDDMM per batch."""
    k = mat.size(-1)
    g = grad.float().reshape(-1, grad.size(-2), k)
    x = mat.float().reshape(-1, mat.size(-2), k)
    if reduce == 1:
        deg = (ptr[1:] - ptr[:-1]).clamp_min(1).to(torch.float32)
        g = g / deg.reshape(1, -1, 1)
    total = None
    for b in range(g.size(0)):
        part = sddmm_csr(ptr, col, g[b].contiguous(), x[b].contiguous(), "dot" if width == 1 else "mul", 0, 2)
        total = part if total is None else total + part
    return total
