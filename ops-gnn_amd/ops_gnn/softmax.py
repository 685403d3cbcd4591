"""Grouped softmax family: scatter_softmax, scatter_log_softmax, scatter_logsumexp.

Argument handling and error contract of the reference
(python/ops_gnn/_grouped_softmax.py:33-155, scatter_softmax.py:46-75,
scatter_log_softmax.py:49-79, scatter_logsumexp.py:86-127): `index` is a
1-D int32/int64 vector along `dim` (length src.size(dim)), groups =
`dim_size` (default index.max() + 1), every index value must lie in
[0, dim_size).

Forward, all HIP: per-(batch, group, feature) statistics m = max and
s = sum(exp(x - clamp(m))) -- from the contiguous-segment engine when the
index is sorted (deterministic), from atomics otherwise -- then one
elementwise pass (softmax / log_softmax) or one pass over the groups
(logsumexp).  A sorted index over one-feature rows that average >= 64
positions (per-edge attention scores) takes one fused kernel, a wavefront
per row, instead.  fp32 math for every dtype.

Backward (reference python/ops_gnn/_grouped_softmax.py:102-133,
scatter_logsumexp.py:57-84), all HIP: softmax out * (g - sum_group(out * g)),
log_softmax g - exp(out) * sum_group(g), logsumexp g[group] * exp(x - out[group]).
"""

from typing import Optional

import math
import torch

from . import _lib, _native

SUPPORTED_DTYPES = (torch.float16, torch.float32, torch.bfloat16)
SUPPORTED_INDEX_DTYPES = (torch.int32, torch.int64)


def normalize_dim(dim: int, rank: int) -> int:
    if not isinstance(dim, int) or isinstance(dim, bool):
        raise TypeError(f"dim must be an int, got {type(dim).__name__}")
    if dim < -rank or dim >= rank:
        raise IndexError(f"Dimension out of range (expected to be in range of [-{rank}, {rank - 1}], but got {dim})")
    return dim + rank if dim < 0 else dim


def check_inputs(op: str, src: torch.Tensor, index: torch.Tensor, dim: int) -> None:
    if src.dim() < 1:
        raise ValueError("src must have at least one dimension")
    if index.dim() != 1:
        raise ValueError(f"index must be 1-D, got {index.dim()}-D")
    if src.dtype not in SUPPORTED_DTYPES:
        raise TypeError(f"src dtype must be one of float16, float32, bfloat16; got {src.dtype}")
    if index.dtype not in SUPPORTED_INDEX_DTYPES:
        raise TypeError(f"index dtype must be int32 or int64, got {index.dtype}")
    if src.device != index.device:
        raise ValueError(f"src and index must be on the same device, got {src.device} and {index.device}")
    if src.device.type != "cuda":
        raise RuntimeError(f"{op} requires GPU tensors")
    if index.numel() != src.size(dim):
        raise ValueError(f"index length ({index.numel()}) must match src.size({dim}) ({src.size(dim)})")


def resolve_dim_size(index: torch.Tensor, dim_size: Optional[int], facts) -> int:
    if dim_size is None:
        return facts[2] + 1 if index.numel() > 0 else 0
    if not isinstance(dim_size, int) or isinstance(dim_size, bool):
        raise TypeError(f"dim_size must be an int, got {type(dim_size).__name__}")
    if dim_size < 0:
        raise ValueError(f"dim_size must be non-negative, got {dim_size}")
    if dim_size > 2 ** 31 - 1:
        raise ValueError(f"dim_size must fit the int32 index range, got {dim_size}")
    return dim_size


def _facts(index: torch.Tensor):
    if index.numel() == 0:
        return (True, 0, -1)
    return _native.index_facts(index)


def _prepare(op, src, index, dim, dim_size):
    if not isinstance(src, torch.Tensor):
        raise TypeError(f"src must be a torch.Tensor, got {type(src).__name__}")
    if not isinstance(index, torch.Tensor):
        raise TypeError(f"index must be a torch.Tensor, got {type(index).__name__}")
    dim = normalize_dim(dim, src.dim())
    check_inputs(op, src, index, dim)
    facts = _facts(index)
    groups = resolve_dim_size(index, dim_size, facts)
    if index.numel():
        if facts[1] < 0:
            raise ValueError("index must be non-negative")
        if facts[2] >= groups:
            raise ValueError(f"index values must be smaller than dim_size ({groups})")
    before, length, after = math.prod(src.shape[:dim]), src.size(dim), math.prod(src.shape[dim + 1:])
    src3 = src.contiguous().reshape(before, length, after)
    return dim, groups, facts[0], src3


def _stats(src3, index, groups, is_sorted):
    return _native.group_stats(src3, index, groups, is_sorted)


class _GroupedSoftmax(torch.autograd.Function):
    """softmax / log_softmax over index groups with the analytic grouped Jacobian."""

    @staticmethod
    def forward(ctx, src, index, groups, is_sorted, log_softmax, shape3):
        src3 = src.contiguous().reshape(shape3)
        if is_sorted and _native.fused_row_softmax_ok(src3, groups):
            # one feature per position, long rows: statistics and output in one pass per row
            ptr = _native.sorted_index_ptr(index, groups)
            out3 = _native.group_softmax_rows(src3, ptr, groups, log_softmax, key=ptr)
        else:
            m, s = _stats(src3, index, groups, is_sorted)
            out3 = _native.group_softmax_apply(src3, index, groups, m, s, log_softmax)
        ctx.save_for_backward(out3, index)
        ctx.groups, ctx.log_softmax, ctx.shape3 = groups, log_softmax, src3.shape
        return out3.reshape(src.shape)

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad):
        out3, index = ctx.saved_tensors
        g3 = grad.to(out3.dtype).contiguous().reshape(ctx.shape3)
        gsrc = _native.group_softmax_backward(out3, g3, index, ctx.groups, 1 if ctx.log_softmax else 0)
        return gsrc.reshape(grad.shape), None, None, None, None, None


class _GroupedLogSumExp(torch.autograd.Function):
    """log-sum-exp over index groups; gradient g[group] * exp(x - out[group])."""

    @staticmethod
    def forward(ctx, src, index, groups, is_sorted, shape3, shape):
        src3 = src.contiguous().reshape(shape3)
        if is_sorted:
            ptr = _native.sorted_index_ptr(index, groups)
            res3, _ = _native.segment_reduce(src3, ptr, groups, _lib.R_LSE, _lib.SEM_SEGMENT_CSR, key=ptr)
        else:
            m, s = _stats(src3, index, groups, False)
            res3 = _native.group_lse_from_stats(m, s, src.dtype)
        ctx.save_for_backward(src3, res3, index)
        ctx.groups, ctx.src_shape = groups, src.shape
        return res3.reshape(shape)

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad):
        src3, res3, index = ctx.saved_tensors
        g3 = grad.to(res3.dtype).contiguous().reshape(res3.shape)
        gsrc = _native.group_softmax_backward(src3, g3, index, ctx.groups, 2, reduced3=res3)
        return gsrc.reshape(ctx.src_shape), None, None, None, None, None


def scatter_softmax(src: torch.Tensor, index: torch.Tensor, dim: int = 0,
                    dim_size: Optional[int] = None) -> torch.Tensor:
    """Softmax over the groups of ``src`` along ``dim`` defined by ``index``."""
    dim, groups, is_sorted, src3 = _prepare("scatter_softmax", src, index, dim, dim_size)
    if src.numel() == 0:
        return torch.zeros_like(src)
    return _GroupedSoftmax.apply(src, index, groups, is_sorted, False, src3.shape)


def scatter_log_softmax(src: torch.Tensor, index: torch.Tensor, dim: int = 0,
                        dim_size: Optional[int] = None) -> torch.Tensor:
    """Log-softmax over the groups of ``src`` along ``dim`` defined by ``index``."""
    dim, groups, is_sorted, src3 = _prepare("scatter_log_softmax", src, index, dim, dim_size)
    if src.numel() == 0:
        return torch.zeros_like(src)
    return _GroupedSoftmax.apply(src, index, groups, is_sorted, True, src3.shape)


def scatter_logsumexp(src: torch.Tensor, index: torch.Tensor, dim: int = 0,
                      dim_size: Optional[int] = None) -> torch.Tensor:
    """log(sum(exp(src))) per group; src.size(dim) is replaced by dim_size,
    empty groups give -inf."""
    dim, groups, is_sorted, src3 = _prepare("scatter_logsumexp", src, index, dim, dim_size)
    shape = list(src.shape)
    shape[dim] = groups
    if src3.numel() == 0 or groups == 0:
        return torch.full(shape, float("-inf"), dtype=src.dtype, device=src.device)
    return _GroupedLogSumExp.apply(src, index, groups, is_sorted, src3.shape, shape)
