"""Python face of the CPU oracle (oracle.c) -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, as the checker and the timed CPU baseline.  The product package
(ops_gnn) never imports it.

Functions take numpy arrays (or CPU torch tensors), widen floating inputs to
float32 (exact for fp16/bf16), and return float64 values (+ int64 arg) so the
caller can apply the reference golden's final cast.
"""

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle.so"

_i64p = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_lib = None

REDUCE = {"sum": 0, "add": 0, "mean": 1, "min": 2, "max": 3}


def build() -> Path:
    """Compile oracle.c with the committed Makefile (gcc + OpenMP)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        l = ctypes.CDLL(str(LIB_PATH))
        vp = ctypes.c_void_p
        i64 = ctypes.c_int64
        l.oracle_spmm_csr.argtypes = [_i64p, _i64p, vp, i64, _f32p, i64, i64, i64, i64,
                                      ctypes.c_int, _f64p, vp]
        l.oracle_spmm_csr.restype = None
        l.oracle_ind2ptr.argtypes = [_i64p, i64, i64, _i64p]
        l.oracle_ptr2ind.argtypes = [_i64p, i64, i64, _i64p]
        l.oracle_segment_csr.argtypes = [_f32p, _i64p, i64, i64, i64, i64, i64, ctypes.c_int,
                                         _f64p, vp]
        l.oracle_segment_coo.argtypes = [_f32p, _i64p, i64, i64, i64, i64, i64, ctypes.c_int,
                                         ctypes.c_int, _f64p, vp]
        l.oracle_scatter.argtypes = [_f32p, _i64p, i64, i64, i64, i64, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_double, _f64p, vp]
        l.oracle_scatter_f64.argtypes = [_f64p, _i64p, i64, i64, i64, i64, ctypes.c_int, ctypes.c_int, _f64p, vp]
        ci = ctypes.c_int
        l.oracle_int_segment_csr.argtypes = [_i64p, _i64p, i64, i64, i64, i64, i64, ci, ci, ci, _i64p, vp]
        l.oracle_int_segment_coo.argtypes = [_i64p, _i64p, i64, i64, i64, i64, i64, ci, ci, ci, ci, _i64p, vp]
        l.oracle_int_scatter.argtypes = [_i64p, _i64p, i64, i64, i64, i64, ci, ci, ci, ci, _i64p, vp]
        l.oracle_segment_lse.argtypes = [_f32p, _i64p, i64, i64, i64, i64, i64, _f64p]
        l.oracle_group_softmax.argtypes = [_f32p, _i64p, i64, i64, i64, i64, ctypes.c_int, _f64p]
        u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
        l.oracle_gather_csr.argtypes = [_i64p, i64, u8p, i64, i64, i64, i64, u8p]
        l.oracle_gather_coo.argtypes = [_i64p, u8p, i64, i64, i64, i64, u8p]
        l.oracle_group_softmax_backward.argtypes = [_f32p, _f32p, _i64p, i64, i64, i64, i64, ctypes.c_int,
                                                    _f64p]
        l.oracle_sddmm.argtypes = [_i64p, _i64p, i64, vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, i64,
                                   _f64p]
        l.oracle_spmm_dgl.argtypes = [_i64p, _i64p, i64, vp, vp, i64, ctypes.c_int, ctypes.c_int, i64, _f64p]
        _lib = l
    return _lib


def _np(x, dtype=None):
    if hasattr(x, "detach"):  # torch tensor
        x = x.detach().cpu()
        if dtype is not None and x.is_floating_point() and x.dtype != __import__("torch").float64:
            x = x.float()  # fp16 / bf16 widen exactly; numpy has no bf16
        x = x.numpy()
    x = np.asarray(x)
    if dtype is not None:
        x = x.astype(dtype, copy=False)
    return np.ascontiguousarray(x)


def _int_kind(x):
    """(bits, is_unsigned) of an integer array / tensor, or None for floats."""
    dt = x.dtype
    if hasattr(x, "detach"):  # torch dtype -> numpy dtype
        if dt.is_floating_point or dt.is_complex or dt == __import__("torch").bool:
            return None
        dt = np.dtype(str(dt).replace("torch.", ""))
    dt = np.dtype(dt)
    if dt.kind not in "iu":
        return None
    return dt.itemsize * 8, int(dt.kind == "u")


def _is_f64(x):
    return str(x.dtype) in ("float64", "torch.float64")


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def spmm_csr(ptr, col, value, mat, reduce="sum"):
    """torch_sparse SpMM golden (reference test/torch_sparse_spmm/arch35/golden.py:91-116).

    mat: [..., N, K]; value: None, [E] or [E, K].  Returns (out float64
    [..., M, K], arg int64 [..., M, K] or None for sum/mean).
    """
    ptr = _np(ptr, np.int64)
    col = _np(col, np.int64)
    mat = _np(mat, np.float32)
    lead = mat.shape[:-2]
    n, k = mat.shape[-2], mat.shape[-1]
    batch = int(np.prod(lead)) if lead else 1
    m = ptr.shape[0] - 1
    width = 0
    v = None
    if value is not None:
        v = _np(value, np.float32).reshape(col.shape[0], -1)
        width = v.shape[1]
        if width not in (1, k):
            raise ValueError("value width must be 1 or K")
        v = np.ascontiguousarray(v)
    r = REDUCE[reduce]
    out = np.zeros(lead + (m, k), dtype=np.float64)
    arg = np.zeros(lead + (m, k), dtype=np.int64) if r >= 2 else None
    lib().oracle_spmm_csr(ptr, col, _ptr(v), width, mat, batch, m, n, k, r, out, _ptr(arg))
    return out, arg


def ind2ptr(ind, rows):
    """reference test/sparse/arch35/golden.py:6-27."""
    ind = _np(ind, np.int64)
    out = np.zeros(rows + 1, dtype=np.int64)
    lib().oracle_ind2ptr(ind, ind.shape[0], rows, out)
    return out


def ptr2ind(ptr, numel):
    """reference test/sparse/arch35/golden.py:30-43."""
    ptr = _np(ptr, np.int64)
    out = np.zeros(numel, dtype=np.int64)
    lib().oracle_ptr2ind(ptr, ptr.shape[0] - 1, numel, out)
    return out


def segment_csr(src, indptr, reduce="sum"):
    """segment_csr golden (reference test/segment_csr/arch35/golden.py:21-103).

    Returns (values float64 -- int64 already wrapped to the dtype for integer
    src --, arg int64 or None).  Reduction axis is indptr.dim() - 1; leading
    indptr dims broadcast to src's.
    """
    kind = _int_kind(src)
    src = _np(src, np.int64 if kind else np.float32)
    ip = _np(indptr, np.int64)
    dim = ip.ndim - 1
    lead = src.shape[:dim]
    length = src.shape[dim]
    feat = int(np.prod(src.shape[dim + 1:])) if src.ndim > dim + 1 else 1
    batch = int(np.prod(lead)) if lead else 1
    segs = ip.shape[-1] - 1
    if ip.ndim > 1 and int(np.prod(ip.shape[:-1])) != 1:
        ip = np.ascontiguousarray(np.broadcast_to(ip, lead + (ip.shape[-1],)))
        stride = ip.shape[-1]
    else:
        ip = np.ascontiguousarray(ip.reshape(-1))
        stride = 0
    r = REDUCE[reduce]
    shape = lead + (segs,) + src.shape[dim + 1:]
    arg = np.zeros(shape, dtype=np.int64) if r >= 2 else None
    if kind:
        out = np.zeros(shape, dtype=np.int64)
        lib().oracle_int_segment_csr(np.ascontiguousarray(src.reshape(-1)), ip.reshape(-1), stride, batch, length,
                                     feat, segs, r, kind[0], kind[1], out, _ptr(arg))
        return out, arg
    out = np.zeros(shape, dtype=np.float64)
    lib().oracle_segment_csr(np.ascontiguousarray(src.reshape(-1)), ip.reshape(-1), stride, batch,
                             length, feat, segs, r, out, _ptr(arg))
    return out, arg


def _split(shape, dim):
    before = int(np.prod(shape[:dim])) if dim > 0 else 1
    after = int(np.prod(shape[dim + 1:])) if dim + 1 < len(shape) else 1
    return before, shape[dim], after


FINFO_MAX = {"float32": 3.4028234663852886e38, "float16": 65504.0, "bfloat16": 3.3895313892515355e38}


def segment_coo(src, index, segments, reduce="sum", out=None):
    """Ascend 950 segment_coo rules (reference csrc/npu/segment_coo/op_kernel/arch35/segment_coo.cpp:114-153).

    index: [..., L] sorted along its last dim (reduction dim = index.ndim - 1),
    leading dims 1 or equal to src's.  out: optional seed values (float64
    array of the output shape).  Returns (values float64, arg int64 | None).
    """
    kind = _int_kind(src)
    src = _np(src, np.int64 if kind else np.float32)
    idx = _np(index, np.int64)
    dim = idx.ndim - 1
    before, length, after = _split(src.shape, dim)
    ib = int(np.prod(idx.shape[:-1])) if idx.ndim > 1 else 1
    if ib not in (1, before):
        raise ValueError("index leading dims must broadcast")
    r = REDUCE[reduce]
    shape = src.shape[:dim] + (segments,) + src.shape[dim + 1:]
    arg = np.zeros(shape, np.int64) if r >= 2 else None
    if kind:
        o = np.zeros(shape, np.int64) if out is None else _np(out, np.int64).reshape(shape).copy()
        lib().oracle_int_segment_coo(np.ascontiguousarray(src.reshape(-1)), np.ascontiguousarray(idx.reshape(-1)),
                                     ib, before, length, after, segments, r, 0 if out is None else 1, kind[0],
                                     kind[1], o, _ptr(arg))
        return o, arg
    o = np.zeros(shape, np.float64) if out is None else np.array(out, dtype=np.float64).reshape(shape).copy()
    lib().oracle_segment_coo(np.ascontiguousarray(src.reshape(-1)), np.ascontiguousarray(idx.reshape(-1)), ib,
                             before, length, after, segments, r, 0 if out is None else 1, o, _ptr(arg))
    return o, arg


def scatter(src, index, dim, size, reduce="sum", out=None, dtype_name="float32"):
    """torch_scatter fold (reference test/scatter/arch35/golden.py:35-127).

    index must already have src's shape (broadcast by the caller).  reduce
    codes as torch_scatter: sum/add/mean/min/max/mul.  Returns (values, arg|None).
    """
    kind = _int_kind(src)
    f64 = _is_f64(src)
    src = _np(src, np.int64 if kind else (np.float64 if f64 else np.float32))
    idx = np.ascontiguousarray(np.broadcast_to(_np(index, np.int64), src.shape))
    before, length, after = _split(src.shape, dim)
    code = {"sum": 0, "add": 0, "mean": 1, "min": 2, "max": 3, "mul": 4}[reduce]
    shape = src.shape[:dim] + (size,) + src.shape[dim + 1:]
    arg = np.zeros(shape, np.int64) if code in (2, 3) else None
    flat = np.ascontiguousarray(src.reshape(-1))
    if kind:
        o = np.zeros(shape, np.int64) if out is None else _np(out, np.int64).reshape(shape).copy()
        lib().oracle_int_scatter(flat, idx.reshape(-1), before, length, after, size, code, 0 if out is None else 1,
                                 kind[0], kind[1], o, _ptr(arg))
        return o, arg
    o = np.zeros(shape, np.float64) if out is None else _np(out, np.float64).reshape(shape).copy()
    if f64:
        lib().oracle_scatter_f64(flat, idx.reshape(-1), before, length, after, size, code,
                                 0 if out is None else 1, o, _ptr(arg))
        return o, arg
    lib().oracle_scatter(flat, idx.reshape(-1), before, length, after, size,
                         code, 0 if out is None else 1, FINFO_MAX[dtype_name], o, _ptr(arg))
    return o, arg


def segment_logsumexp(src, indptr):
    """reference test/segment_logsumexp/golden.py:25-44 (1-D indptr along dim 0)."""
    src = _np(src, np.float32)
    ip = _np(indptr, np.int64).reshape(-1)
    length = src.shape[0]
    feat = int(np.prod(src.shape[1:])) if src.ndim > 1 else 1
    segs = ip.shape[0] - 1
    out = np.zeros((segs,) + src.shape[1:], np.float64)
    lib().oracle_segment_lse(np.ascontiguousarray(src.reshape(-1)), ip, 0, 1, length, feat, segs, out)
    return out


def group_softmax(src, index, dim, groups, mode):
    """Grouped softmax family (reference test/common/grouped_softmax_golden.py:31-82).

    mode: "softmax", "log_softmax" (src-shaped output) or "logsumexp"
    (output with src.size(dim) replaced by `groups`).
    """
    src = _np(src, np.float32)
    idx = _np(index, np.int64).reshape(-1)
    dim = dim % src.ndim
    before, length, after = _split(src.shape, dim)
    m = {"softmax": 0, "log_softmax": 1, "logsumexp": 2}[mode]
    shape = src.shape if m < 2 else src.shape[:dim] + (groups,) + src.shape[dim + 1:]
    out = np.zeros(shape, np.float64)
    lib().oracle_group_softmax(np.ascontiguousarray(src.reshape(-1)), idx, before, length, after, groups, m, out)
    return out


def group_softmax_backward(src, grad, index, dim, groups, mode):
    """Gradient of group_softmax w.r.t. src from the float64 forward.  `grad`
    has the forward output's shape (src-shaped, or `groups` along dim for
    logsumexp).  Returns float64, src-shaped."""
    src = _np(src, np.float32)
    grad = _np(grad, np.float32)
    idx = _np(index, np.int64).reshape(-1)
    dim = dim % src.ndim
    before, length, after = _split(src.shape, dim)
    m = {"softmax": 0, "log_softmax": 1, "logsumexp": 2}[mode]
    out = np.zeros(src.shape, np.float64)
    lib().oracle_group_softmax_backward(np.ascontiguousarray(src.reshape(-1)), np.ascontiguousarray(grad.reshape(-1)),
                                        idx, before, length, after, groups, m, out)
    return out


SDDMM_OPS = {"dot": 0, "add": 1, "sub": 2, "mul": 3, "div": 4, "copy_lhs": 5, "copy_rhs": 6}


def sddmm(ptr, col, lhs, rhs, op="dot", lhs_target=0, rhs_target=2):
    """reference test/sddmm_csr/arch22/golden.py:74-90; operands [rows, k]
    (1-D operands are [rows, 1]).  Returns float64 [nnz] (dot) or [nnz, k]."""
    ptr = _np(ptr, np.int64)
    col = _np(col, np.int64)
    l = None if lhs is None else _np(lhs, np.float32)
    r = None if rhs is None else _np(rhs, np.float32)
    feat = l if l is not None else r
    k = 1 if feat.ndim == 1 else feat.shape[1]
    nnz = col.shape[0]
    code = SDDMM_OPS[op]
    out = np.zeros((nnz,) if code == 0 else (nnz, k), np.float64)
    lib().oracle_sddmm(ptr, col, ptr.shape[0] - 1, _ptr(l), _ptr(r), lhs_target, rhs_target, code, k, out)
    return out


DGL_MSG = {"copy_lhs": 0, "add": 1, "sub": 2, "mul": 3, "div": 4, "copy_rhs": 5}


# Input -> output dtype pairs of torch_sparse SpMM (reference golden
# test/torch_sparse_spmm/arch35/golden.py:80-88, COMBOS).
SPMM_DTYPE_COMBOS = (("float32", "float32"), ("float16", "float16"), ("bfloat16", "bfloat16"),
                     ("float16", "float32"), ("bfloat16", "float32"), ("int8", "int32"), ("int8", "float32"))


def spmm_output_cast(out, out_dtype):
    """The golden's final cast of the fp64 result (reference
    test/torch_sparse_spmm/arch35/golden.py:114-115): an int32 output
    truncates toward zero; every other output is one rounding of the fp64
    value.  `out_dtype` is a numpy dtype name; 'bfloat16' returns the fp64
    values rounded to bf16 (as float32 numbers)."""
    name = str(out_dtype).replace("torch.", "")
    out = np.asarray(out, dtype=np.float64)
    if name == "int32":
        return np.trunc(out).astype(np.int32)
    if name == "bfloat16":
        import torch
        return torch.from_numpy(out).to(torch.bfloat16).float().numpy()
    return out.astype(np.dtype(name))


def spmm_dgl(ptr, col, x, rhs, op, reduce):
    """DGL-style aggregation (reference test/unified_spmm/arch22/golden.py:13-92).

    x [N, k] (None for copy_rhs); rhs [E], [E, 1] or [E, k] (None for copy_lhs).
    Returns float64 [M, k]."""
    ptr = _np(ptr, np.int64)
    col = _np(col, np.int64)
    xs = None if x is None else _np(x, np.float32)
    w = None if rhs is None else _np(rhs, np.float32)
    nnz = col.shape[0]
    if xs is not None:
        k = int(np.prod(xs.shape[1:])) if xs.ndim > 1 else 1
        xs = np.ascontiguousarray(xs.reshape(xs.shape[0], k))
    else:
        k = int(np.prod(w.shape[1:])) if w.ndim > 1 else 1
    width = 0
    if w is not None:
        width = int(np.prod(w.shape[1:])) if w.ndim > 1 else 1
        w = np.ascontiguousarray(w.reshape(nnz, width))
    m = ptr.shape[0] - 1
    out = np.zeros((m, k), np.float64)
    lib().oracle_spmm_dgl(ptr, col, m, _ptr(xs), _ptr(w), width, DGL_MSG[op], REDUCE[reduce], k, out)
    return out


def threads() -> int:
    return int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))


def _raw(t):
    """numpy view of a tensor / array as raw bytes (C order) and its dtype."""
    import torch

    if isinstance(t, torch.Tensor):
        t = t.detach().cpu().contiguous()
        return t.view(torch.uint8).numpy().reshape(-1), t.dtype
    a = np.ascontiguousarray(t)
    return a.view(np.uint8).reshape(-1), a.dtype


def gather_csr(src, indptr):
    """reference test/gather_csr/arch35/golden.py:63-90; returns a torch CPU tensor."""
    import torch

    src_t = src if isinstance(src, torch.Tensor) else torch.from_numpy(np.asarray(src))
    ptr = _np(indptr, np.int64)
    dim = ptr.ndim - 1
    before = int(np.prod(src_t.shape[:dim])) if dim else 1
    width = ptr.shape[-1]
    ptr2 = np.ascontiguousarray(np.broadcast_to(ptr, tuple(src_t.shape[:dim]) + (width,)).reshape(-1, width))
    segs = width - 1
    rows = int(ptr2[0, -1]) if ptr2.size else 0
    feat = int(np.prod(src_t.shape[dim + 1:])) if src_t.dim() > dim + 1 else 1
    shape = list(src_t.shape)
    shape[dim] = rows
    out = torch.zeros(shape, dtype=src_t.dtype)
    if out.numel() == 0 or segs <= 0:
        return out
    raw, _ = _raw(src_t)
    ob = np.zeros(out.numel() * out.element_size(), np.uint8)
    lib().oracle_gather_csr(ptr2, ptr2.shape[0], raw, before, segs, feat * src_t.element_size(), rows, ob)
    return torch.from_numpy(ob).view(src_t.dtype).reshape(shape)


def gather_coo(src, index):
    """reference test/gather_coo/arch35/test_gather_coo.py:87-106; torch CPU tensor."""
    import torch

    src_t = src if isinstance(src, torch.Tensor) else torch.from_numpy(np.asarray(src))
    idx = np.ascontiguousarray(_np(index, np.int64))
    dim = idx.ndim - 1
    before = int(np.prod(src_t.shape[:dim])) if dim else 1
    feat = int(np.prod(src_t.shape[dim + 1:])) if src_t.dim() > dim + 1 else 1
    shape = list(src_t.shape)
    shape[dim] = idx.shape[-1]
    out = torch.zeros(shape, dtype=src_t.dtype)
    if out.numel() == 0:
        return out
    raw, _ = _raw(src_t)
    ob = np.zeros(out.numel() * out.element_size(), np.uint8)
    lib().oracle_gather_coo(idx.reshape(-1), raw, before, src_t.size(dim), idx.shape[-1],
                            feat * src_t.element_size(), ob)
    return torch.from_numpy(ob).view(src_t.dtype).reshape(shape)
