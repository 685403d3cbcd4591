"""segment_csr / segment_coo / segment_reduce / segment_logsumexp on the GPU.

Public names, signatures and return conventions follow the reference
(python/ops_gnn/segment_csr.py:35-91, segment_reduce.py:32-66,
segment_coo.py:33-128, segment_logsumexp.py:108-155,
segment_max_csr.py:19-50).  Every reduction runs on the contiguous-segment
CSR engine (include/ogn.h ogn_segment_reduce): deterministic, one writer per
output, nnz-balanced across wavefronts.  segment_csr / segment_coo take
float32, float16, bfloat16 (fp32 arithmetic) and int8, uint8, int32, int64
(exact integer arithmetic wrapping in the dtype, on the exact-dtype segment
kernel); segment_logsumexp takes the floating dtypes.  Other dtypes raise
TypeError -- there is no CPU fallback.
"""

import math
from typing import Optional, Tuple

import torch

from . import _lib, _native
from ._native import SEGMENT_DTYPES, SEGMENT_EXACT_DTYPES

_REDUCE_OPS = ("sum", "add", "mean", "min", "max")
_CODE = {"sum": _lib.R_SUM, "add": _lib.R_SUM, "mean": _lib.R_MEAN, "min": _lib.R_MIN, "max": _lib.R_MAX}

_PTR_FACTS = _native._VersionCache()
_LSE_FACTS = _native._VersionCache()


def _check_reduce(reduce: str) -> None:
    if reduce not in _REDUCE_OPS:
        raise ValueError(f"reduce value '{reduce}' is not valid (use one of {_REDUCE_OPS})")


def _check_dtype(src: torch.Tensor, op: str) -> None:
    if src.dtype not in SEGMENT_DTYPES + SEGMENT_EXACT_DTYPES:
        raise TypeError(f"{op}: unsupported dtype {src.dtype} (float32, float16, bfloat16, int8, uint8, int32 "
                        f"and int64 run on the GPU)")


def _split(shape, dim):
    return math.prod(shape[:dim]), shape[dim], math.prod(shape[dim + 1:])


def _pointer_facts(ptr2d: torch.Tensor):
    """(non-decreasing and >= 0, max, longest segment) of a pointer tensor:
    one small device-to-host read, cached per tensor version.  Pass the
    caller's own tensor (not a fresh view of it) so that the cache can hit."""
    def compute():
        p = ptr2d
        bad = (p < 0).any()
        longest = torch.zeros((), dtype=p.dtype, device=p.device)
        if p.size(-1) > 1:
            steps = p[..., 1:] - p[..., :-1]
            bad = bad | (steps < 0).any()
            longest = steps.max()
        flags = torch.stack((bad.to(torch.int64), p.max().to(torch.int64), longest.to(torch.int64))).tolist()
        return flags[0] == 0, flags[1], flags[2]
    return _PTR_FACTS.get(ptr2d, compute)


def _prepare_out(out, shape, src, op):
    if out is None:
        return None
    if not isinstance(out, torch.Tensor):
        raise TypeError(f"{op}: out must be a torch.Tensor")
    if out.dtype != src.dtype:
        raise RuntimeError(f"out dtype ({out.dtype}) must match src ({src.dtype})")
    if tuple(out.shape) != tuple(shape):
        raise RuntimeError(f"out shape {tuple(out.shape)} must be {tuple(shape)}")
    if out.device != src.device:
        raise RuntimeError("out must live on src's device")
    return out


def _finish(result3, out, shape):
    result = result3.reshape(shape)
    if out is None:
        return result
    if result.data_ptr() != out.data_ptr():
        out.copy_(result)
    return out


# ------------------------------------------------------------------ A2 (arch22) semantics
# The reference's Atlas A2 build binds segment_csr / segment_coo with other
# forward rules than the Ascend 950 build (docs/en/api_reference.md:1778-1795,
# goldens test/segment_csr/arch22/golden.py:68-153 and
# test/segment_coo/arch22/golden.py:63-160).  semantics="a2" selects them.
# They are derived on the GPU from the first-tie, NaN-ignoring segment
# kernels (SEM_SEGMENT_CSR) plus elementwise passes:
#   * extrema update only on strict improvement, from the supplied out
#     (segment_coo) or from the work dtype's finite identity; a result still
#     equal to the identity is the identity (segment_csr) or zero (segment_coo
#     without out);
#   * the arg of an element without an improvement carries the last
#     improving position of the same feature across the flattened
#     (batch, segment) order, starting from 0; empty segments give the
#     length sentinel;
#   * segment_coo seeds sum / mean with out, the segment holding position 0 of
#     a batch reads out[batch, 0], and its mean divides by the count narrowed
#     to the source dtype (zero when that is zero); segment_csr's fp16 / bf16
#     mean narrows the sum before the division.
_SEMANTICS = ("arch35", "a2")


def _check_semantics(semantics: str) -> None:
    if semantics not in _SEMANTICS:
        raise ValueError(f"semantics must be one of {_SEMANTICS}, got {semantics!r}")


def _work_dtype(dtype):
    return torch.float32 if dtype in (torch.float16, torch.bfloat16) else dtype


def _identity(dtype, reduce):
    work = _work_dtype(dtype)
    info = torch.finfo(work) if work.is_floating_point else torch.iinfo(work)
    return info.max if reduce == "min" else info.min


def _strictly_better(v, ref, reduce):
    """v strictly improves on ref (NaN never does), compared in the work dtype."""
    work = _work_dtype(v.dtype)
    a = v.to(work)
    b = ref.to(work) if isinstance(ref, torch.Tensor) else ref
    return a < b if reduce == "min" else a > b


def _carry_args(arg3, improved3, nonempty2, length):
    """A2 arg state: improving elements keep their position; other elements
    of nonempty segments take the last improving position of their feature in
    flattened (batch, segment) order (0 before any); empty segments take
    `length`."""
    b, s, f = arg3.shape
    flat = arg3.reshape(b * s, f)
    imp = improved3.reshape(b * s, f)
    pos = torch.arange(b * s, device=arg3.device).view(-1, 1).expand(b * s, f)
    last = torch.where(imp, pos, torch.full_like(pos, -1)).cummax(0).values
    carried = torch.where(last >= 0, flat.gather(0, last.clamp_min(0)), torch.zeros_like(flat))
    ne = nonempty2.reshape(b * s, 1)
    res = torch.where(ne, torch.where(imp, flat, carried), torch.full_like(flat, length))
    return res.reshape(b, s, f)


def _segment_counts(ptr2d, before, segs):
    counts = ptr2d[:, 1:] - ptr2d[:, :-1]
    return counts.expand(before, segs) if counts.size(0) != before else counts


# ------------------------------------------------------------------ segment_csr
def _segment_csr(src, indptr, out, reduce, return_arg, semantics="arch35"):
    _lib.require_gpu(src, indptr, what="segment_csr")
    if indptr.dtype != torch.int64:
        raise RuntimeError(f"indptr must be int64, got {indptr.dtype}")
    if indptr.dim() < 1:
        raise RuntimeError("indptr must have at least 1 dim")
    if src.dim() < indptr.dim():
        raise RuntimeError(f"src.dim() ({src.dim()}) must be >= indptr.dim() ({indptr.dim()})")
    if indptr.size(-1) < 1:
        raise RuntimeError("indptr last dim must be >= 1")
    dim = indptr.dim() - 1
    for i in range(dim):
        if indptr.size(i) not in (1, src.size(i)):
            raise RuntimeError(f"indptr leading dim {i} ({indptr.size(i)}) must be 1 or src.size({i}) "
                               f"({src.size(i)})")
    _check_dtype(src, "segment_csr")
    segs = indptr.size(-1) - 1
    before, length, after = _split(src.shape, dim)
    shape = list(src.shape)
    shape[dim] = segs
    out = _prepare_out(out, shape, src, "segment_csr")
    if src.numel() == 0 or segs == 0:
        if out is not None:
            res = out
        else:
            res = torch.zeros(shape, dtype=src.dtype, device=src.device)
        arg = torch.full(shape, length, dtype=torch.int64, device=src.device)
        return res, arg
    if all(indptr.size(i) == 1 for i in range(dim)):
        ptr2d = indptr.reshape(1, -1).contiguous()
    else:
        ptr2d = indptr.expand(*src.shape[:dim], segs + 1).reshape(before, segs + 1).contiguous()
    # broadcasting repeats pointer rows, so the facts of indptr are those of ptr2d
    ok, top, longest = _pointer_facts(indptr)
    if not ok:
        raise RuntimeError("indptr must be nondecreasing and non-negative")
    if top > length:
        # segment ends past src.size(dim) are clamped, as the golden does
        # (reference test/segment_csr/arch35/golden.py:64)
        ptr2d = ptr2d.clamp(max=length)
    src3 = src.contiguous().reshape(before, length, after)
    direct = out is not None and out.is_contiguous()
    out3 = out.view(before, segs, after) if direct else None
    if semantics == "a2":
        res3, arg3 = _segment_csr_a2(src3, ptr2d, segs, reduce, return_arg)
        result = _finish(res3, out, shape)
        return result, (None if arg3 is None else arg3.reshape(shape))
    res3, arg3 = _native.segment_reduce(src3, ptr2d, segs, _CODE[reduce], _lib.SEM_SEGMENT_CSR, out3,
                                        False, return_arg and reduce in ("min", "max"), key=indptr,
                                        max_len=longest)
    result = _finish(res3, out, shape)
    return result, (None if arg3 is None else arg3.reshape(shape))


def _segment_csr_a2(src3, ptr2d, segs, reduce, return_arg):
    """A2 segment_csr values / args (reference test/segment_csr/arch22/golden.py:68-153)."""
    before, length, _ = src3.shape
    extremum = reduce in ("min", "max")
    res3, arg3 = _native.segment_reduce(src3, ptr2d, segs, _CODE[reduce], _lib.SEM_SEGMENT_CSR, None, False,
                                        extremum)
    counts = _segment_counts(ptr2d, before, segs)
    if reduce == "mean" and src3.dtype in (torch.float16, torch.bfloat16):
        # the sum is narrowed to the source dtype, then divided by the count
        # (itself converted to that dtype)
        total, _ = _native.segment_reduce(src3, ptr2d, segs, _lib.R_SUM, _lib.SEM_SEGMENT_CSR)
        div = counts.clamp_min(1).to(torch.float32).to(src3.dtype).unsqueeze(-1)
        return total / div, None
    if not extremum:
        return res3, None
    nonempty = (counts > 0).unsqueeze(-1)
    improved = _strictly_better(res3, _identity(src3.dtype, reduce), reduce) & nonempty
    ident = torch.tensor(_identity(src3.dtype, reduce), dtype=_work_dtype(src3.dtype)).to(src3.dtype)
    values = torch.where(improved, res3, torch.where(nonempty, ident.to(src3.device), torch.zeros_like(res3)))
    args = _carry_args(arg3, improved, counts > 0, length) if return_arg else None
    return values, args


def segment_sum_csr(src: torch.Tensor, indptr: torch.Tensor, out: Optional[torch.Tensor] = None, *,
                    semantics: str = "arch35") -> torch.Tensor:
    _check_semantics(semantics)
    return _segment_csr(src, indptr, out, "sum", False, semantics)[0]


def segment_add_csr(src: torch.Tensor, indptr: torch.Tensor, out: Optional[torch.Tensor] = None, *,
                    semantics: str = "arch35") -> torch.Tensor:
    _check_semantics(semantics)
    return _segment_csr(src, indptr, out, "add", False, semantics)[0]


def segment_mean_csr(src: torch.Tensor, indptr: torch.Tensor, out: Optional[torch.Tensor] = None, *,
                     semantics: str = "arch35") -> torch.Tensor:
    _check_semantics(semantics)
    return _segment_csr(src, indptr, out, "mean", False, semantics)[0]


def segment_min_csr(src: torch.Tensor, indptr: torch.Tensor, out: Optional[torch.Tensor] = None, *,
                    semantics: str = "arch35") -> Tuple[torch.Tensor, torch.Tensor]:
    _check_semantics(semantics)
    return _segment_csr(src, indptr, out, "min", True, semantics)


def segment_max_csr(src: torch.Tensor, indptr: torch.Tensor, out: Optional[torch.Tensor] = None, *,
                    semantics: str = "arch35") -> Tuple[torch.Tensor, torch.Tensor]:
    """Values and first indices of the segment maxima.

    An int32 indptr selects the legacy value-only entry (segment_max_csr_legacy),
    as in the reference (python/ops_gnn/segment_csr.py:64-77).
    """
    if isinstance(indptr, torch.Tensor) and indptr.dtype == torch.int32:
        return segment_max_csr_legacy(src, indptr, out)
    _check_semantics(semantics)
    return _segment_csr(src, indptr, out, "max", True, semantics)


def segment_csr(src: torch.Tensor, indptr: torch.Tensor, out: Optional[torch.Tensor] = None,
                reduce: str = "sum", *, semantics: str = "arch35") -> torch.Tensor:
    """Reduce CSR segments along ``indptr.dim() - 1``; values only.
    semantics="a2" selects the reference's Atlas A2 rules (see above)."""
    _check_reduce(reduce)
    _check_semantics(semantics)
    return _segment_csr(src, indptr, out, reduce, False, semantics)[0]


def segment_reduce(src: torch.Tensor, offsets: torch.Tensor, out: Optional[torch.Tensor] = None,
                   reduce: str = "sum") -> torch.Tensor:
    """DGL ``segment_reduce``: promote int32 offsets to int64 and call segment_csr."""
    if offsets.dtype != torch.int64:
        offsets = offsets.to(torch.int64)
    return segment_csr(src, offsets, out, reduce)


def segment_max_csr_legacy(src: torch.Tensor, indptr: torch.Tensor, optional_out: Optional[torch.Tensor] = None):
    """Legacy value-only segment max (reference python/ops_gnn/segment_max_csr.py:19-50,
    golden test/segment_max_csr/arch35/golden.py:16-41): empty segments give 0;
    a non-empty ``optional_out`` seeds the result as max(segment max, optional_out)."""
    ptr = indptr.to(torch.int64)
    values, _ = _segment_csr(src, ptr, None, "max", False)
    if optional_out is not None and optional_out.numel() > 0:
        if optional_out.shape != values.shape:
            raise RuntimeError("optional_out must have the output shape")
        values = torch.maximum(values, optional_out.to(values.dtype))
    return values


# ------------------------------------------------------------------ segment_coo
_COO_FACTS = _native._VersionCache()


def _coo_index_facts(index: torch.Tensor):
    """(min, max, sorted along the last dim) of a COO index, one small
    device-to-host read cached per index version (reference
    csrc/npu/segment_coo/op_host/segment_coo.cpp:65-109 ValidateIndex)."""
    def compute():
        if index.dim() == 1:
            ok, mn, mx = _native.index_facts(index)
            return mn, mx, ok
        bad = (index[..., 1:] < index[..., :-1]).any() if index.size(-1) > 1 else index.new_zeros((), dtype=torch.bool)
        mn, mx, uns = torch.stack((index.min(), index.max(), bad.to(torch.int64))).tolist()
        return mn, mx, uns == 0
    return _COO_FACTS.get(index, compute)


def _segment_coo(src, index, out, dim_size, reduce, return_arg, semantics="arch35"):
    _lib.require_gpu(src, index, what="segment_coo")
    if index.dtype != torch.int64:
        raise ValueError("indices must be an int64 tensor with valid rank")
    if index.dim() < 1 or index.dim() > src.dim():
        raise ValueError("indices must be an int64 tensor with valid rank")
    if reduce not in _CODE:
        raise ValueError("segment_coo supports sum/add/mean/min/max, not " + str(reduce))
    _check_dtype(src, "segment_coo")
    dim = index.dim() - 1
    for i in range(dim + 1):
        if index.size(i) not in (1, src.size(i)) or (i == dim and index.size(i) != src.size(i)):
            raise ValueError("index shape must broadcast to src")
    before, length, after = _split(src.shape, dim)
    facts = _coo_index_facts(index) if index.numel() else None
    if facts is not None:
        # the reference's checks and messages (segment_coo.cpp:97-100)
        if facts[0] < 0:
            raise RuntimeError("index values must be non-negative")
        if not facts[2]:
            raise RuntimeError("index must be sorted along its last dimension")
    if out is not None:
        segs = out.size(dim)
    elif dim_size is not None:
        segs = int(dim_size)
    else:
        segs = facts[1] + 1 if facts is not None else 0
    if facts is not None and (out is not None or dim_size is not None) and facts[1] >= segs:
        raise RuntimeError("index values exceed output size")
    shape = list(src.shape)
    shape[dim] = segs
    out = _prepare_out(out, shape, src, "segment_coo")
    if all(index.size(i) == 1 for i in range(dim)):
        idx2d = index.reshape(1, -1)
    else:
        idx2d = index.expand(*src.shape[:dim], length).reshape(before, length)
    if src.numel() == 0 or segs == 0:
        res = out if out is not None else torch.zeros(shape, dtype=src.dtype, device=src.device)
        return res, torch.full(shape, length, dtype=torch.int64, device=src.device)
    ptr2d = _native.sorted_index_ptr(index, segs, idx2d)
    src3 = src.contiguous().reshape(before, length, after)
    if semantics == "a2":
        seeds = None if out is None else out.contiguous().reshape(before, segs, after)
        res3, arg3 = _segment_coo_a2(src3, ptr2d, idx2d, segs, reduce, return_arg, seeds)
        result = _finish(res3, out, shape)
        return result, (None if arg3 is None else arg3.reshape(shape))
    has_out = out is not None
    direct = has_out and out.is_contiguous()
    if has_out:
        out3 = out.view(before, segs, after) if direct else out.contiguous().reshape(before, segs, after)
    else:
        out3 = None
    res3, arg3 = _native.segment_reduce(src3, ptr2d, segs, _CODE[reduce], _lib.SEM_SEGMENT_COO, out3, has_out,
                                        return_arg and reduce in ("min", "max"), key=ptr2d)
    result = _finish(res3, out, shape)
    return result, (None if arg3 is None else arg3.reshape(shape))


def _segment_coo_a2(src3, ptr2d, idx2d, segs, reduce, return_arg, seeds3):
    """A2 segment_coo values / args (reference test/segment_coo/arch22/golden.py:63-160)."""
    before, length, after = src3.shape
    reduce = "sum" if reduce == "add" else reduce
    extremum = reduce in ("min", "max")
    counts = _segment_counts(ptr2d, before, segs)
    nonempty = (counts > 0).unsqueeze(-1)
    work = _work_dtype(src3.dtype)
    if seeds3 is not None:
        # the segment holding a batch's position 0 starts from out[batch, 0]
        seeds = seeds3.clone()
        first = idx2d[:, :1].expand(before, 1) if idx2d.size(0) != before else idx2d[:, :1]
        seeds.scatter_(1, first.unsqueeze(-1).expand(before, 1, after), seeds3[:, :1, :])
    if extremum:
        v, arg3 = _native.segment_reduce(src3, ptr2d, segs, _CODE[reduce], _lib.SEM_SEGMENT_CSR, None, False, True)
        if seeds3 is None:
            ident = torch.tensor(_identity(src3.dtype, reduce), dtype=work, device=src3.device)
            improved = _strictly_better(v, ident, reduce) & nonempty
            values = torch.where(improved, v, torch.zeros_like(v))
        else:
            improved = _strictly_better(v, seeds, reduce) & nonempty
            values = torch.where(improved, v, seeds3.where(~nonempty, seeds))
        args = _carry_args(arg3, improved, counts > 0, length) if return_arg else None
        return values, args
    total, _ = _native.segment_reduce(src3, ptr2d, segs, _lib.R_SUM, _lib.SEM_SEGMENT_CSR)
    if seeds3 is not None:
        total = (seeds.to(work) + total.to(work)).to(src3.dtype) if work != src3.dtype else seeds + total
    if reduce == "mean":
        div = counts.to(src3.dtype).unsqueeze(-1)
        zero = div == 0
        if src3.dtype.is_floating_point:
            mean = total / torch.where(zero, torch.ones_like(div), div)
        else:
            mean = torch.div(total.to(torch.int64), torch.where(zero, torch.ones_like(div), div).to(torch.int64),
                             rounding_mode="trunc").to(src3.dtype)
        total = torch.where(zero, torch.zeros_like(mean), mean)
    if seeds3 is not None:
        total = torch.where(nonempty, total, seeds3)
    else:
        total = torch.where(nonempty, total, torch.zeros_like(total))
    return total, None


def segment_sum_coo(src, index, out=None, dim_size=None, *, semantics: str = "arch35") -> torch.Tensor:
    """Sum segments of a sorted index (a supplied out is overwritten, Ascend 950
    rule; with semantics="a2" it seeds the sums)."""
    _check_semantics(semantics)
    return _segment_coo(src, index, out, dim_size, "sum", False, semantics)[0]


def segment_add_coo(src, index, out=None, dim_size=None, *, semantics: str = "arch35") -> torch.Tensor:
    return segment_sum_coo(src, index, out, dim_size, semantics=semantics)


def segment_mean_coo(src, index, out=None, dim_size=None, *, semantics: str = "arch35") -> torch.Tensor:
    """Segment means; a supplied out seeds the numerator."""
    _check_semantics(semantics)
    return _segment_coo(src, index, out, dim_size, "mean", False, semantics)[0]


def segment_min_coo(src, index, out=None, dim_size=None, *, semantics: str = "arch35"
                    ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Minima and int64 positions; later ties win (Ascend 950 convention;
    semantics="a2": first strict improvement, carried arg state)."""
    _check_semantics(semantics)
    return _segment_coo(src, index, out, dim_size, "min", True, semantics)


def segment_max_coo(src, index, out=None, dim_size=None, *, semantics: str = "arch35"
                    ) -> Tuple[torch.Tensor, torch.Tensor]:
    _check_semantics(semantics)
    return _segment_coo(src, index, out, dim_size, "max", True, semantics)


def segment_coo(src, index, out=None, dim_size=None, reduce: str = "sum", *,
                semantics: str = "arch35") -> torch.Tensor:
    """Reduce along ``index.dim() - 1`` over a sorted int64 index; values only."""
    if reduce not in _CODE:
        raise ValueError("segment_coo supports sum/add/mean/min/max, not " + str(reduce))
    _check_semantics(semantics)
    return _segment_coo(src, index, out, dim_size, reduce, False, semantics)[0]


# ------------------------------------------------------------------ segment_logsumexp
_MAX_POINTER = 2 ** 31 - 1


def segment_logsumexp(src: torch.Tensor, indptr: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """log(sum(exp(src))) over CSR segments along dim 0 (fp32 math, shift
    clamped to +-FLT_MAX; empty segments give -inf).  Argument checks and
    messages follow the reference (python/ops_gnn/segment_logsumexp.py:44-105)."""
    if not isinstance(src, torch.Tensor):
        raise TypeError(f"src must be a torch.Tensor, got {type(src).__name__}")
    if not isinstance(indptr, torch.Tensor):
        raise TypeError(f"indptr must be a torch.Tensor, got {type(indptr).__name__}")
    if src.dim() < 1:
        raise ValueError("src must have at least one dimension")
    if indptr.dim() != 1:
        raise ValueError(f"indptr must be 1-D, got {indptr.dim()}-D")
    if src.dtype not in SEGMENT_DTYPES:
        raise TypeError(f"src dtype must be one of float16, float32, bfloat16; got {src.dtype}")
    if indptr.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"indptr dtype must be int32 or int64, got {indptr.dtype}")
    if src.device != indptr.device:
        raise ValueError(f"src and indptr must be on the same device, got {src.device} and {indptr.device}")
    _lib.require_gpu(src, what="segment_logsumexp")
    if indptr.numel() < 1:
        raise ValueError("indptr must contain at least one boundary")
    ptr = indptr.to(torch.int64).contiguous()

    def compute():
        # the reference reads these back on every call (segment_logsumexp.py:75-84);
        # here once per indptr version
        steps = ptr[1:] - ptr[:-1]
        longest = steps.max() if steps.numel() else torch.zeros((), dtype=torch.int64, device=ptr.device)
        return tuple(int(v) for v in torch.stack(((ptr < 0).any().to(torch.int64),
                                                  (steps < 0).any().to(torch.int64), ptr[-1],
                                                  longest)).tolist())
    flags = _LSE_FACTS.get(indptr, compute)
    if int(flags[0]):
        raise ValueError("indptr must be non-negative")
    if int(flags[1]):
        raise ValueError("indptr must be nondecreasing")
    if int(flags[2]) != src.size(0):
        raise ValueError(f"indptr[-1] ({int(flags[2])}) must equal src.size(0) ({src.size(0)})")
    if src.size(0) > _MAX_POINTER:
        raise ValueError(f"src.size(0) must fit the int32 pointer range, got {src.size(0)}")
    segs = ptr.numel() - 1
    shape = (segs,) + tuple(src.shape[1:])
    if out is not None:
        if not isinstance(out, torch.Tensor):
            raise TypeError(f"out must be a torch.Tensor, got {type(out).__name__}")
        if tuple(out.shape) != shape:
            raise ValueError(f"out shape must be {shape}, got {tuple(out.shape)}")
        if out.dtype != src.dtype:
            raise TypeError(f"out dtype must match src ({src.dtype}), got {out.dtype}")
        if out.device != src.device:
            raise ValueError(f"out device must match src ({src.device}), got {out.device}")
    if segs == 0:
        result = torch.empty(shape, dtype=src.dtype, device=src.device)
    elif src.numel() == 0:
        result = torch.full(shape, float("-inf"), dtype=src.dtype, device=src.device)
    else:
        length = src.size(0)
        after = math.prod(src.shape[1:])
        res3, _ = _native.segment_reduce(src.contiguous().reshape(1, length, after), ptr.reshape(1, -1), segs,
                                         _lib.R_LSE, _lib.SEM_SEGMENT_CSR, key=indptr, max_len=int(flags[3]))
        result = res3.reshape(shape)
    if out is not None:
        out.copy_(result)
        return out
    return result
