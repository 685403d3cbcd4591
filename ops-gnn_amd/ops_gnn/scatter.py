"""torch_scatter-compatible scatter family on the GPU.

Public API and rules of the reference python/ops_gnn/scatter.py:555-674
(torch_scatter 2.1.2 semantics with the Ascend 950 "later writer wins" tie
rule for min/max): index broadcast (`broadcast`), negative dims, `out`
updated in place (identity preserved), dim_size inferred from the index,
positions never written by min/max get arg = src.size(dim) and value 0 when
`out` is omitted.

Two execution paths, both HIP:
  * sorted 1-D index along `dim` (the common message-passing layout) -> the
    deterministic contiguous-segment engine (include/ogn.h ogn_segment_reduce
    with OGN_SEM_SCATTER);
  * any other index -> the atomic scatter (ogn_scatter_atomic).
Index sortedness and bounds come from one cached device probe per index
version.  float32 / float16 / bfloat16 (fp32 arithmetic), float64, and
int8 / uint8 / int16 / int32 / int64 (exact, wrapping in the dtype; the mean
floors, with 8/16-bit counts narrowed as torch_scatter does, reference
python/ops_gnn/scatter.py:430-458); other dtypes raise TypeError.
"""

import math
from typing import Optional, Tuple

import torch

from . import _lib, _native
from ._native import SCATTER_DTYPES

_REDUCE_CODE = {"sum": _lib.R_SUM, "add": _lib.R_SUM, "mul": _lib.R_PROD, "mean": _lib.R_MEAN,
                "min": _lib.R_MIN, "max": _lib.R_MAX}


def native_available() -> bool:
    return True


def broadcast(src: torch.Tensor, other: torch.Tensor, dim: int) -> torch.Tensor:
    """Broadcast ``src`` to ``other`` with torch_scatter's index rules."""
    if dim < 0:
        dim = other.dim() + dim
    if src.dim() == 1:
        for _ in range(0, dim):
            src = src.unsqueeze(0)
    for _ in range(src.dim(), other.dim()):
        src = src.unsqueeze(-1)
    return src.expand(other.size())


def _index_extent(index: torch.Tensor, dim: int) -> int:
    """Size of `index` along `dim` once `broadcast` has placed its dims."""
    if index.dim() == 1:
        return index.numel()
    return index.size(dim) if index.dim() > dim else 1


def _normalize_dim(src: torch.Tensor, dim: int) -> int:
    if not isinstance(dim, int) or isinstance(dim, bool):
        raise TypeError("dim must be an int")
    if src.dim() < 1 or src.dim() > 8:
        raise ValueError("src must have between 1 and 8 dimensions")
    if dim < -src.dim() or dim >= src.dim():
        raise IndexError(f"Dimension out of range (expected to be in range of [-{src.dim()}, {src.dim() - 1}], "
                         f"but got {dim})")
    return dim + src.dim() if dim < 0 else dim


def _scatter_forward(src: torch.Tensor, index: torch.Tensor, dim: int, out: Optional[torch.Tensor],
                     dim_size: Optional[int], reduce: str) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    if reduce not in _REDUCE_CODE:
        raise ValueError("reduce must be one of 'sum', 'add', 'mul', 'mean', 'min', or 'max'")
    dim = _normalize_dim(src, dim)
    if index.dtype != torch.int64:
        raise TypeError(f"index must have dtype torch.int64, got {index.dtype}")
    if src.dtype not in SCATTER_DTYPES:
        raise TypeError(f"scatter: unsupported dtype {src.dtype}")
    _lib.require_gpu(src, index, what="scatter")
    if reduce == "mean" and src.size(dim) > 1 and _index_extent(index, dim) == 1:
        # torch_scatter counts the mean's denominators over the index's own
        # shape (reference python/ops_gnn/scatter.py:437-449): an index of
        # extent 1 along dim, broadcast over it, counts each target once, so
        # the mean of such a scatter is its sum.
        reduce = "sum"
    expanded = broadcast(index, src, dim)
    compact = index.dim() == 1 and index.numel() == src.size(dim)
    line = index
    if not compact and expanded.dim() == src.dim() and all(
            expanded.stride(d) == 0 or expanded.size(d) == 1 for d in range(src.dim()) if d != dim):
        # an index broadcast along every other dim (torch_scatter's usual
        # `index.view(-1, 1).expand_as(src)`) is one 1-D vector along dim
        line = expanded
        for d in reversed(range(src.dim())):
            if d != dim:
                line = line.select(d, 0)
        compact = line.numel() == src.size(dim)
    # Exact index bounds (one cached device probe per index version); both
    # paths below rely on every index lying in [0, size) (reference
    # python/ops_gnn/scatter.py:406-422, same errors).
    checked = index.numel() > 0 and expanded.numel() > 0
    mn, mx = _native.index_facts(line, key=index)[1:] if checked else (0, -1)
    if mn < 0:
        raise IndexError(f"index contains a negative value ({mn})")
    if out is not None:
        size = out.size(dim)
    elif dim_size is not None:
        size = int(dim_size)
    else:
        size = mx + 1
    if mx >= size:
        raise IndexError(f"index value {mx} is out of bounds for output size {size} at dimension {dim}")
    shape = list(src.shape)
    shape[dim] = size
    if out is not None:
        if out.dtype != src.dtype or list(out.shape) != shape or out.device != src.device:
            raise ValueError("out must match src's dtype and device and have the scatter output shape")
    before, length, after = math.prod(src.shape[:dim]), src.size(dim), math.prod(src.shape[dim + 1:])
    code = _REDUCE_CODE[reduce]
    has_out = out is not None
    is_minmax = reduce in ("min", "max")
    if has_out:
        out3 = out.view(before, size, after) if out.is_contiguous() else out.contiguous().view(before, size, after)
    else:
        out3 = torch.empty((before, size, after), dtype=src.dtype, device=src.device)
    if out3.numel() == 0:
        arg = torch.full(shape, length, dtype=torch.int64, device=src.device) if is_minmax else None
        return (out if has_out else out3.reshape(shape)), arg
    src3 = src.contiguous().reshape(before, length, after)
    arg3 = None
    use_segments = False
    if compact and checked:
        use_segments = _native.index_facts(line, key=index)[0]
    if use_segments:
        ptr = _native.sorted_index_ptr(index, size, line.reshape(1, -1))
        res3, arg3 = _native.segment_reduce(src3, ptr, size, code, _lib.SEM_SCATTER, out3, has_out, is_minmax,
                                            key=ptr)
    elif (compact and checked and before == 1 and length >= _native.SORT_PATH_MIN_LENGTH and length < 2**31
          and size <= 2**32 and src.dtype in (torch.float32, torch.float16, torch.bfloat16)):
        # unsorted: a stable sort of the index (cached per index version),
        # then every output row folded by the engine through the
        # permutation -- no contended atomics, and sums in a fixed order
        ptr, perm = _native.sorted_layout(line, size, index)
        arg2 = _native.segment_reduce_gather(ptr, perm, src3[0], size, code, out3[0], has_out, is_minmax)
        res3, arg3 = out3, None if arg2 is None else arg2.view(1, size, after)
    else:
        if compact:
            idx, strides = line.contiguous(), (0, 1, 0)
        else:
            idx, strides = expanded.contiguous(), (length * after, after, 1)
        arg3 = _native.scatter_atomic(src3, idx, strides, size, code, out3, has_out)
        res3 = out3
    result = res3.reshape(shape)
    if has_out and result.data_ptr() != out.data_ptr():
        out.copy_(result)
        result = out
    elif has_out:
        result = out
    return result, (None if arg3 is None else arg3.reshape(shape))


def scatter_sum(src, index, dim: int = -1, out=None, dim_size=None) -> torch.Tensor:
    return _scatter_forward(src, index, dim, out, dim_size, "sum")[0]


def scatter_add(src, index, dim: int = -1, out=None, dim_size=None) -> torch.Tensor:
    return scatter_sum(src, index, dim, out, dim_size)


def scatter_mul(src, index, dim: int = -1, out=None, dim_size=None) -> torch.Tensor:
    return _scatter_forward(src, index, dim, out, dim_size, "mul")[0]


def scatter_mean(src, index, dim: int = -1, out=None, dim_size=None) -> torch.Tensor:
    return _scatter_forward(src, index, dim, out, dim_size, "mean")[0]


def scatter_min(src, index, dim: int = -1, out=None, dim_size=None) -> Tuple[torch.Tensor, torch.Tensor]:
    return _scatter_forward(src, index, dim, out, dim_size, "min")


def scatter_max(src, index, dim: int = -1, out=None, dim_size=None) -> Tuple[torch.Tensor, torch.Tensor]:
    return _scatter_forward(src, index, dim, out, dim_size, "max")


def scatter(src, index, dim: int = -1, out=None, dim_size=None, reduce: str = "sum") -> torch.Tensor:
    """``torch_scatter.scatter(src, index, dim, out, dim_size, reduce)``."""
    return _scatter_forward(src, index, dim, out, dim_size, reduce)[0]
