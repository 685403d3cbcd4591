"""Tensor-level wrappers over the C ABI -- the counterpart of the reference's
pybind module ``_pybind`` (reference csrc/pybind.cpp:92-349).

Each function takes torch tensors, checks what the kernel assumes (device,
dtype, contiguity, shapes), allocates outputs and workspaces with torch's
caching allocator, and launches on torch's current stream.  ctypes drops the
GIL for the duration of each foreign call, matching the reference's
``py::gil_scoped_release`` guards.
"""

import math
from typing import Optional, Tuple

import torch

from . import _lib
from ._lib import check, dptr, lib, stream_of

SPMM_INPUT_DTYPES = (torch.float32, torch.float16, torch.bfloat16, torch.int8)
SPMM_OUTPUT_DTYPES = (torch.float32, torch.float16, torch.bfloat16, torch.int32)
SPMM_FLOAT_DTYPES = (torch.float32, torch.float16, torch.bfloat16)
# Output dtypes each mat dtype may produce (reference
# csrc/npu/torch_sparse_spmm/op_host/torch_sparse_spmm.cpp:88-90); the first
# one is the default (python/ops_gnn/torch_sparse_spmm.py:213).
SPMM_OUTPUTS_FOR = {
    torch.float32: (torch.float32,),
    torch.float16: (torch.float16, torch.float32),
    torch.bfloat16: (torch.bfloat16, torch.float32),
    torch.int8: (torch.int32, torch.float32),
}


def _index_code(t: torch.Tensor) -> int:
    if t.dtype == torch.int64:
        return _lib.I64
    if t.dtype == torch.int32:
        return _lib.I32
    raise ValueError("index tensors must be int32 or int64")


def validate_csr(ptr: torch.Tensor, col: torch.Tensor, n: int) -> torch.Tensor:
    """Device CSR check; returns an int32 [1] status tensor (0 ok, 1 bad rowptr,
    2 column out of range).  Reference TorchSparseSpmmValidate
    (csrc/npu/torch_sparse_spmm/op_host/torch_sparse_spmm.cpp:136-147)."""
    ptr = ptr.contiguous()
    col = col.contiguous()
    if col.dtype != ptr.dtype:
        col = col.to(ptr.dtype)
    status = torch.empty(1, dtype=torch.int32, device=ptr.device)
    m = ptr.numel() - 1
    if m < 0:
        status.fill_(1)
        return status
    rc = lib.ogn_validate_csr(dptr(ptr), dptr(col), _index_code(ptr), m, col.numel(), int(n),
                              dptr(status), stream_of(ptr))
    check(rc, "validate_csr")
    return status


def spmm_forward(ptr: torch.Tensor, col: torch.Tensor, value: Optional[torch.Tensor],
                 mat: torch.Tensor, reduce: int, out_dtype: torch.dtype,
                 out: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Weighted CSR SpMM; reference TorchSparseSpmmForward
    (csrc/npu/torch_sparse_spmm/op_host/torch_sparse_spmm.cpp:97-135).

    mat [..., N, K]; value None / [E] / [E, K] (any trailing shape of width 1
    or K); returns (out [..., M, K], arg [..., M, K] int64 for min/max, else an
    empty int64 tensor).
    """
    if mat.dtype not in SPMM_INPUT_DTYPES:
        raise ValueError("mat must be float32, float16, bfloat16 or int8")
    if out_dtype not in SPMM_OUTPUTS_FOR[mat.dtype]:
        raise ValueError("unsupported input/output dtype combination")
    mat = mat.contiguous()
    ptr = ptr.contiguous()
    col = col.contiguous()
    if col.dtype != ptr.dtype:
        col = col.to(ptr.dtype)
    m = ptr.numel() - 1
    n, k = mat.size(-2), mat.size(-1)
    lead = tuple(mat.shape[:-2])
    batch = math.prod(lead)
    nnz = col.numel()
    width = 1
    if value is not None:
        value = value.contiguous()
        width = value.numel() // nnz if nnz else 1
    shape = lead + (m, k)
    if out is None:
        out = torch.empty(shape, dtype=out_dtype, device=mat.device)
    minmax = reduce >= 2
    arg = torch.empty(shape if minmax else (0,), dtype=torch.int64, device=mat.device)
    if out.numel() == 0:
        return out, arg
    if reduce == _lib.R_SUM and batch == 1 and width == 1 and out.is_contiguous() and \
            spmm_sum_xcd(ptr, col, value, mat.view(n, k), out):
        return out, arg
    ws_bytes = lib.ogn_spmm_csr_workspace_size(m, nnz, k, batch, _lib.TORCH_TO_OGN[mat.dtype], reduce)
    ws = _lib.workspace(ws_bytes, mat.device)
    rc = lib.ogn_spmm_csr(dptr(ptr), dptr(col), _index_code(ptr), dptr(value), width, dptr(mat),
                          _lib.TORCH_TO_OGN[mat.dtype], batch, m, n, k, nnz, dptr(out),
                          _lib.TORCH_TO_OGN[out_dtype], dptr(arg) if minmax else None, reduce,
                          dptr(ws), ws_bytes, stream_of(mat))
    check(rc, "spmm")
    return out, arg


# ------------------------------------------------------------------ XCD tiles
# Column-tiled SDDMM dot / SpMM sum (include/ogn.h, ogn_xcd_*): used when the
# gathered table is larger than one XCD's L2 and an eighth of it fits (8-96 MB),
# on graphs of at least 2^20 edges.  OGN_XCD=0 turns the path off, OGN_XCD=1
# takes it whenever the row width allows (tests).
XCD_TABLE_BYTES = (8 << 20, 96 << 20)
XCD_MIN_EDGES = 1 << 20
_XCD_PLANS = None


def xcd_wanted(table_rows: int, row_bytes: int, nnz: int) -> bool:
    import os

    mode = os.environ.get("OGN_XCD", "")
    if mode == "0" or row_bytes not in (64, 128, 256, 512) or not 0 < nnz < (1 << 31):
        return False
    if mode == "1":
        return True
    return XCD_TABLE_BYTES[0] <= table_rows * row_bytes <= XCD_TABLE_BYTES[1] and nnz >= XCD_MIN_EDGES


def xcd_plan(ptr: torch.Tensor, col: torch.Tensor, n_cols: int):
    """(plan, state) of the kept XCD plan of (ptr, col), or None when a row's
    columns are not sorted (the tiles would not follow column ranges); state
    2 means the plan also holds 16-bit tile-relative columns.  Cached per
    version of col, together with ptr's address, version and n_cols."""
    import ctypes

    global _XCD_PLANS
    if _XCD_PLANS is None:
        _XCD_PLANS = _VersionCache(limit=8)
    per_col = _XCD_PLANS.get(col, dict)
    info = (ptr.data_ptr(), ptr._version, tuple(ptr.shape), ptr.dtype, n_cols)
    hit = per_col.get(info)
    if hit is None:
        m, nnz = ptr.numel() - 1, col.numel()
        plan = _lib.workspace(lib.ogn_xcd_plan_bytes(m, nnz), col.device)
        sorted_flag = ctypes.c_int(0)
        check(lib.ogn_xcd_plan(dptr(ptr), dptr(col), _index_code(ptr), m, n_cols, nnz, dptr(plan), plan.numel(),
                               ctypes.byref(sorted_flag), stream_of(col)), "xcd plan")
        hit = (plan, sorted_flag.value)
        per_col.clear()
        per_col[info] = hit
    return hit if hit[1] > 0 else None


def sddmm_dot_xcd(ptr, col, lhs, rhs, out) -> bool:
    """dot(lhs[row], rhs[col]) into out through the XCD path; False when the
    path does not apply (the caller runs ogn_sddmm_csr)."""
    k = lhs.size(1)
    nnz = col.numel()
    if lhs.dtype not in SEGMENT_DTYPES or not xcd_wanted(rhs.size(0), k * lhs.element_size(), nnz):
        return False
    if lhs.data_ptr() % 16 or rhs.data_ptr() % 16 or ptr.dtype != col.dtype:
        return False
    kept = xcd_plan(ptr, col, rhs.size(0))
    if kept is None:
        return False
    check(lib.ogn_sddmm_dot_xcd(dptr(kept[0]), ptr.numel() - 1, nnz, dptr(col), _index_code(ptr), dptr(lhs),
                                lhs.size(0), dptr(rhs), rhs.size(0), k, _lib.TORCH_TO_OGN[lhs.dtype], dptr(out),
                                kept[1], stream_of(lhs)), "sddmm_csr (xcd)")
    return True


def spmm_sum_xcd(ptr, col, value, mat, out) -> bool:
    """out = A @ mat (sum, one weight per edge, batch 1) through the XCD path;
    False when the path does not apply."""
    m, nnz = ptr.numel() - 1, col.numel()
    n, k = mat.shape
    if mat.dtype not in SEGMENT_DTYPES or out.dtype not in (mat.dtype, torch.float32):
        return False
    if value is None or value.dtype != mat.dtype or value.numel() != nnz:
        return False
    if not xcd_wanted(n, k * mat.element_size(), nnz) or mat.data_ptr() % 16 or out.data_ptr() % 16:
        return False
    kept = xcd_plan(ptr, col, n)
    if kept is None:
        return False
    ws_bytes = lib.ogn_spmm_sum_xcd_workspace_size(m, k)
    ws = _lib.workspace(ws_bytes, mat.device)
    check(lib.ogn_spmm_sum_xcd(dptr(kept[0]), m, nnz, dptr(col), _index_code(ptr), dptr(value), dptr(mat), n, k,
                               _lib.TORCH_TO_OGN[mat.dtype], dptr(out), _lib.TORCH_TO_OGN[out.dtype], dptr(ws),
                               ws_bytes, kept[1], stream_of(mat)), "spmm (xcd)")
    return True


# ------------------------------------------------------------------ segment engine
SEGMENT_DTYPES = (torch.float32, torch.float16, torch.bfloat16)
# exact-arithmetic dtypes of segment_csr / segment_coo (reference
# test/segment_csr/arch35/test_segment_csr.py SUPPORTED_DTYPES) and of scatter
# (test/scatter/arch35/test_scatter.py DTYPES)
SEGMENT_EXACT_DTYPES = (torch.int8, torch.uint8, torch.int32, torch.int64)
SCATTER_DTYPES = SEGMENT_DTYPES + (torch.float64, torch.int8, torch.int16, torch.int32, torch.int64, torch.uint8)


# Engine workspaces kept per pointer tensor version: a graph reduced many
# times reuses its chunk layout (ogn.h OGN_SEG_REUSE_LAYOUT).  Bounded in
# entries and in bytes per workspace.
_LAYOUT_WS = None
_LAYOUT_WS_MAX_BYTES = 256 << 20


def _layout_workspace(key: torch.Tensor, sub: tuple, nbytes: int, device):
    """(workspace, flags): a kept workspace for (key's version, sub) -- REUSE
    when it already holds the layout, else a new one with KEEP."""
    global _LAYOUT_WS
    if _LAYOUT_WS is None:
        _LAYOUT_WS = _VersionCache(limit=8)
    per_key = _LAYOUT_WS.get(key, dict)
    ws = per_key.get(sub)
    if ws is not None:
        return ws, _lib.SEG_REUSE_LAYOUT
    ws = _lib.workspace(nbytes, device)
    per_key.clear()  # one shape / stream per pointer version is the common case
    per_key[sub] = ws
    return ws, _lib.SEG_KEEP_LAYOUT


def segment_reduce(src3: torch.Tensor, ptr2d: torch.Tensor, segments: int, reduce: int, semantics: int,
                   out3: Optional[torch.Tensor] = None, has_out: bool = False, need_arg: bool = False,
                   key: Optional[torch.Tensor] = None, max_len: Optional[int] = None
                   ) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Contiguous-segment reduction (include/ogn.h ogn_segment_reduce).

    src3 [B, L, F] contiguous; ptr2d int64 [1 | B, S+1] contiguous; out3
    [B, S, F] contiguous (holding seeds when has_out).  Returns (out3, arg3).
    key: a tensor whose version certifies ptr2d's contents (the caller's
    pointer or index tensor, or ptr2d itself when it is a cached tensor);
    the engine workspace is then kept with its chunk layout.  max_len: the
    longest segment, when the caller knows it.
    """
    b, length, f = src3.shape
    if out3 is None:
        out3 = torch.empty((b, segments, f), dtype=src3.dtype, device=src3.device)
    arg = torch.empty((b, segments, f), dtype=torch.int64, device=src3.device) if need_arg else None
    if out3.numel() == 0:
        return out3, arg
    pb = ptr2d.shape[0]
    code = _lib.TORCH_TO_OGN[src3.dtype]
    ws_bytes = lib.ogn_segment_reduce_workspace_size(b, length, segments, f, pb, code, reduce)
    flags = _lib.SEG_HAS_OUT if has_out else 0
    if max_len is not None and max_len <= _lib.SHORT_SEGMENT_MAX:
        flags |= _lib.SEG_SHORT_SEGMENTS
    stream = stream_of(src3)
    if key is not None and 0 < ws_bytes <= _LAYOUT_WS_MAX_BYTES and src3.dtype not in SEGMENT_EXACT_DTYPES:
        sub = (ptr2d.data_ptr(), tuple(ptr2d.shape), b, length, segments, f, code, reduce, stream.value, ws_bytes)
        ws, lf = _layout_workspace(key, sub, ws_bytes, src3.device)
        flags |= lf
    else:
        ws = _lib.workspace(ws_bytes, src3.device)
    rc = lib.ogn_segment_reduce(dptr(ptr2d), pb, dptr(src3), code, b, length, segments, f, dptr(out3), dptr(arg),
                                reduce, semantics, flags, dptr(ws), ws_bytes, stream)
    check(rc, "segment reduction")
    return out3, arg


def segment_reduce_gather(ptr: torch.Tensor, rows: torch.Tensor, src2: torch.Tensor, segments: int, reduce: int,
                          out2: torch.Tensor, has_out: bool, need_arg: bool) -> Optional[torch.Tensor]:
    """Scatter-semantics segment reduction over src2 [n, k] rows read through
    `rows` (include/ogn.h ogn_segment_reduce_gather): segment s covers
    positions ptr[s] .. ptr[s+1] - 1, position i being src2[rows[i]].
    Writes out2 [segments, k]; returns the arg (src rows) for min / max."""
    n, k = src2.shape
    length = rows.numel()
    code = _lib.TORCH_TO_OGN[src2.dtype]
    arg = torch.empty((segments, k), dtype=torch.int64, device=src2.device) if need_arg else None
    ws_bytes = lib.ogn_segment_reduce_gather_workspace_size(length, segments, k, code, reduce)
    ws = _lib.workspace(ws_bytes, src2.device)
    rc = lib.ogn_segment_reduce_gather(dptr(ptr), dptr(rows), dptr(src2), code, n, length, segments, k, dptr(out2),
                                       dptr(arg), reduce, _lib.SEM_SCATTER, _lib.SEG_HAS_OUT if has_out else 0,
                                       dptr(ws), ws_bytes, stream_of(src2))
    check(rc, "scatter (sorted gather)")
    return arg


_SORTED_LAYOUTS = None

# Unsorted scatters and grouped statistics over at least this many positions
# sort their index and reduce through the permutation; smaller ones use atomics.
SORT_PATH_MIN_LENGTH = 1 << 16


def sorted_layout(line: torch.Tensor, size: int, key: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(ptr [size + 1], perm) of an unsorted 1-D index with values in
    [0, size): the stable sort's permutation and the segment pointers of the
    sorted index, cached per version of `key` (the caller's index tensor)."""
    global _SORTED_LAYOUTS
    if _SORTED_LAYOUTS is None:
        _SORTED_LAYOUTS = _VersionCache(limit=4)

    def compute():
        keys = line.contiguous()
        if keys.dtype != torch.int64:
            keys = keys.to(torch.int64)
        sorted_keys, perm, _ = sort_rows(keys, max(size - 1, 0))
        ptr = ind2ptr_batched(sorted_keys.reshape(1, -1), size).reshape(-1)
        return ptr, perm

    per_size = _SORTED_LAYOUTS.get(key, dict)  # {size: (ptr, perm)} for this index version
    if size not in per_size:
        per_size[size] = compute()
    return per_size[size]


def ind2ptr_batched(index2d: torch.Tensor, rows: int) -> torch.Tensor:
    ib, numel = index2d.shape
    out = torch.empty((ib, rows + 1), dtype=torch.int64, device=index2d.device)
    if numel == 0:
        return out.zero_()
    index2d = index2d.contiguous()
    check(lib.ogn_ind2ptr_batched(dptr(index2d), ib, numel, rows, dptr(out), stream_of(index2d)), "ind2ptr")
    return out


class _VersionCache:
    """Per-tensor facts keyed by identity + version (the reference's proof /
    bounds caches, e.g. python/ops_gnn/scatter.py:134-178)."""

    def __init__(self, limit=256):
        from collections import OrderedDict
        self._d = OrderedDict()
        self._limit = limit

    def get(self, t, compute):
        import weakref
        try:
            version = t._version
        except (AttributeError, RuntimeError):
            return compute()
        key = (id(t), t.data_ptr(), tuple(t.shape), tuple(t.stride()), version)
        hit = self._d.get(key)
        if hit is not None and hit[0]() is t:
            self._d.move_to_end(key)
            return hit[1]
        value = compute()
        self._d[key] = (weakref.ref(t), value)
        if len(self._d) > self._limit:
            self._d.popitem(last=False)
        return value

    def put(self, t, value):
        import weakref
        try:
            key = (id(t), t.data_ptr(), tuple(t.shape), tuple(t.stride()), t._version)
        except (AttributeError, RuntimeError):
            return
        self._d[key] = (weakref.ref(t), value)
        if len(self._d) > self._limit:
            self._d.popitem(last=False)

    def clear(self):
        self._d.clear()


INDEX_FACTS = _VersionCache()


def index_probe(index: torch.Tensor) -> Tuple[bool, int, int]:
    """(unsorted, min, max) of a nonempty int32 / int64 index in one device
    pass and one 24-byte device-to-host read; not cached."""
    idx = index.contiguous()
    if idx.dtype != torch.int64:
        idx = idx.to(torch.int64)
    facts = torch.empty(3, dtype=torch.int64, device=idx.device)
    check(lib.ogn_index_facts(dptr(idx), idx.numel(), dptr(facts), stream_of(idx)), "index facts")
    unsorted, mn, mx = facts.tolist()
    return (unsorted != 0, mn, mx)


def sort_rows(keys: torch.Tensor, max_key: int, companions: Tuple[torch.Tensor, ...] = ()
              ) -> Tuple[torch.Tensor, torch.Tensor, list]:
    """(sorted keys, perm, permuted companions) of a 1-D int64 key tensor
    with every key in [0, max_key]: a stable sort (equal keys keep their
    order), as torch.sort(keys, stable=True), and each companion c (one
    entry per key along dim 0) returned as c[perm].  Companions of 4- or
    8-byte 1-D elements (at most two) are permuted inside the sort's last
    pass; others by indexing.  Sizes beyond the native sort's range (2^31
    keys, keys of 2^32 or more) take torch.sort on the device."""
    n = keys.numel()
    keys = keys.contiguous()
    fused, outs = [], [None] * len(companions)
    for i, c in enumerate(companions):
        if len(fused) < 2 and c.dim() == 1 and c.element_size() in (4, 8) and c.device == keys.device:
            outs[i] = torch.empty_like(c, memory_format=torch.contiguous_format)
            fused.append((c.contiguous(), outs[i]))
    widths = [src.element_size() for src, _ in fused] + [0] * (2 - len(fused))
    ws_bytes = lib.ogn_sort_rows_workspace_size(n, max_key, *widths) if n > 0 else 0
    if n > 0 and ws_bytes == 0:
        sk, perm = torch.sort(keys, stable=True)
        return sk, perm, [c[perm] for c in companions]
    sorted_keys = torch.empty_like(keys)
    perm = torch.empty(n, dtype=torch.int64, device=keys.device)
    if n == 0:
        return sorted_keys, perm, [c[perm] if o is None else o for c, o in zip(companions, outs)]
    args = []
    for j in range(2):
        if j < len(fused):
            src, dst = fused[j]
            args += [dptr(src), dptr(dst), src.element_size()]
        else:
            args += [None, None, 0]
    ws = _lib.workspace(ws_bytes, keys.device)
    check(lib.ogn_sort_rows(dptr(keys), n, max_key, dptr(sorted_keys), dptr(perm), *args, dptr(ws), ws_bytes,
                            stream_of(keys)), "sort_rows")
    return sorted_keys, perm, [c[perm] if o is None else o for c, o in zip(companions, outs)]


def index_facts(index: torch.Tensor, key: Optional[torch.Tensor] = None) -> Tuple[bool, int, int]:
    """(sorted, min, max) of an int32 / int64 index (index_probe), cached per
    tensor version of `key` (default: `index` itself; pass the caller's
    tensor when `index` is a fresh view of it)."""

    def compute():
        unsorted, mn, mx = index_probe(index)
        return (not unsorted, mn, mx)

    return INDEX_FACTS.get(index if key is None else key, compute)


def scatter_atomic(src3: torch.Tensor, index: torch.Tensor, strides, size: int, reduce: int,
                   out3: torch.Tensor, has_out: bool) -> Optional[torch.Tensor]:
    """Unsorted scatter into out3 [B, size, F] (modified in place); returns arg."""
    b, length, f = src3.shape
    need_arg = reduce in (_lib.R_MIN, _lib.R_MAX)
    arg = torch.empty((b, size, f), dtype=torch.int64, device=src3.device) if need_arg else None
    if out3.numel() == 0:
        return arg
    ws_bytes = lib.ogn_scatter_atomic_workspace_size(b, size, f, reduce)
    ws = _lib.workspace(ws_bytes, src3.device)
    rc = lib.ogn_scatter_atomic(dptr(src3), _lib.TORCH_TO_OGN[src3.dtype], dptr(index), strides[0], strides[1],
                                strides[2], b, length, f, size, dptr(out3), dptr(arg), reduce, 1 if has_out else 0,
                                dptr(ws), ws_bytes, stream_of(src3))
    check(rc, "scatter")
    return arg


_SORTED_PTR = _VersionCache()


def sorted_index_ptr(index: torch.Tensor, groups: int, index2d: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Group pointers [B, groups + 1] of a sorted index (index2d [B, L], by
    default `index` as one row), cached per version of the caller's `index`
    (and group count and shape): repeated calls with the same index skip the
    batched ind2ptr."""
    rows2d = index.reshape(1, -1) if index2d is None else index2d
    shape = tuple(rows2d.shape)

    def compute():
        return (groups, shape, ind2ptr_batched(rows2d.to(torch.int64).contiguous(), groups))

    hit = _SORTED_PTR.get(index, compute)
    if hit[0] != groups or hit[1] != shape:
        hit = compute()
        _SORTED_PTR.put(index, hit)
    return hit[2]


def fused_row_softmax_ok(src3: torch.Tensor, groups: int) -> bool:
    """The one-wavefront-per-row fused softmax applies: one feature, rows
    averaging >= 64 positions, 16-byte aligned rows."""
    b, length, f = src3.shape
    return (f == 1 and groups > 0 and length >= 64 * groups and src3.data_ptr() % 16 == 0
            and (b == 1 or (length * src3.element_size()) % 16 == 0) and b <= 65535)


def group_softmax_rows(src3: torch.Tensor, ptr: torch.Tensor, groups: int, log_softmax: bool,
                       key: Optional[torch.Tensor] = None) -> torch.Tensor:
    b, length, _ = src3.shape
    out = torch.empty_like(src3)
    if out.numel() == 0:
        return out
    code = _lib.TORCH_TO_OGN[src3.dtype]
    ws_bytes = lib.ogn_segment_group_softmax_workspace_size(b, length, groups, code)
    stream = stream_of(src3)
    if key is not None and ws_bytes <= _LAYOUT_WS_MAX_BYTES:
        # a kept row plan: later calls with this pointer tensor bin the rows
        sub = ("softmax", ptr.data_ptr(), b, length, groups, code, stream.value, ws_bytes)
        ws, flags = _layout_workspace(key, sub, ws_bytes, src3.device)
    else:
        ws, flags = _lib.workspace(ws_bytes, src3.device), 0
    rc = lib.ogn_segment_group_softmax(dptr(ptr), dptr(src3), code, b, length, groups, dptr(out),
                                       1 if log_softmax else 0, flags, dptr(ws), ws_bytes, stream)
    check(rc, "grouped softmax")
    return out


def group_stats(src3: torch.Tensor, index: torch.Tensor, groups: int, sorted_index: bool
                ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-(batch, group, feature) max and sum(exp(x - clamp(max))), fp32."""
    b, length, f = src3.shape
    m = torch.empty((b, groups, f), dtype=torch.float32, device=src3.device)
    s = torch.empty_like(m)
    if m.numel() == 0:
        return m, s
    code = _lib.TORCH_TO_OGN[src3.dtype]
    if sorted_index:
        ptr = sorted_index_ptr(index, groups)
        ws_bytes = lib.ogn_segment_reduce_workspace_size(b, length, groups, f, 1, code, _lib.R_LSE)
        ws = _lib.workspace(ws_bytes, src3.device)
        rc = lib.ogn_segment_group_stats(dptr(ptr), dptr(src3), code, b, length, groups, f, dptr(m), dptr(s),
                                         dptr(ws), ws_bytes, stream_of(src3))
    elif b == 1 and index.dim() == 1 and length >= SORT_PATH_MIN_LENGTH and length < 2**31 and groups <= 2**32:
        # unsorted: statistics through the stable sort's permutation (cached
        # per index version) -- no contended atomics
        ptr, perm = sorted_layout(index, groups, index)
        ws_bytes = lib.ogn_segment_reduce_gather_workspace_size(length, groups, f, code, _lib.R_LSE)
        ws = _lib.workspace(ws_bytes, src3.device)
        rc = lib.ogn_segment_group_stats_gather(dptr(ptr), dptr(perm), dptr(src3), code, length, length, groups, f,
                                                dptr(m), dptr(s), dptr(ws), ws_bytes, stream_of(src3))
    else:
        idx = index.contiguous()
        key = torch.empty(m.shape, dtype=torch.int32, device=src3.device)
        rc = lib.ogn_group_stats_atomic(dptr(src3), code, dptr(idx), _index_code(idx), b, length, f, groups,
                                        dptr(m), dptr(s), dptr(key), stream_of(src3))
    check(rc, "group statistics")
    return m, s


def group_softmax_apply(src3, index, groups, m, s, log_softmax: bool) -> torch.Tensor:
    b, length, f = src3.shape
    out = torch.empty_like(src3)
    if out.numel() == 0:
        return out
    idx = index.contiguous()
    rc = lib.ogn_group_softmax_apply(dptr(src3), _lib.TORCH_TO_OGN[src3.dtype], dptr(idx), _index_code(idx), b,
                                     length, f, groups, dptr(m), dptr(s), dptr(out), 1 if log_softmax else 0,
                                     stream_of(src3))
    check(rc, "group softmax")
    return out


def group_lse_from_stats(m, s, dtype) -> torch.Tensor:
    out = torch.empty(m.shape, dtype=dtype, device=m.device)
    if out.numel() == 0:
        return out
    check(lib.ogn_group_lse_from_stats(dptr(m), dptr(s), m.numel(), dptr(out), _lib.TORCH_TO_OGN[dtype],
                                       stream_of(m)), "group logsumexp")
    return out


def group_softmax_backward(saved3, grad3, index, groups, mode, reduced3=None) -> torch.Tensor:
    """Gradient of the grouped softmax family w.r.t. src ([B, L, F] like saved3).

    mode 0 softmax / 1 log_softmax: saved3 = forward output, grad3 = its grad.
    mode 2 logsumexp: saved3 = forward src, reduced3 = forward output
    [B, groups, F], grad3 = its grad (same shape as reduced3)."""
    b, length, f = saved3.shape
    out = torch.empty_like(saved3)
    if out.numel() == 0:
        return out
    idx = index.contiguous()
    cells = b * groups * f if mode != 2 else 0
    code = _lib.TORCH_TO_OGN[saved3.dtype]
    if (mode != 2 and b == 1 and index.dim() == 1 and length >= SORT_PATH_MIN_LENGTH and length < 2**31
            and groups <= 2**32):
        # unsorted index: the group sums through the sort permutation (fp32
        # terms, then the engine), no contended atomics; then the elementwise pass
        ptr, perm = sorted_layout(index, groups, index)
        msg = torch.empty((length, f), dtype=torch.float32, device=saved3.device)
        check(lib.ogn_group_bwd_messages(dptr(saved3), dptr(grad3), code, length * f, mode, dptr(msg),
                                         stream_of(saved3)), "group softmax backward")
        totals = torch.empty((groups, f), dtype=torch.float32, device=saved3.device)
        segment_reduce_gather(ptr, perm, msg, groups, _lib.R_SUM, totals, False, False)
        rc = lib.ogn_group_softmax_backward(dptr(saved3), dptr(grad3), None, code, dptr(idx), _index_code(idx), b,
                                            length, f, groups, mode | _lib.GROUP_BWD_TOTALS_GIVEN, dptr(out),
                                            dptr(totals), totals.numel() * 4, stream_of(saved3))
        check(rc, "group softmax backward")
        return out
    ws = torch.empty(max(cells, 1), dtype=torch.float32, device=saved3.device)
    rc = lib.ogn_group_softmax_backward(dptr(saved3), dptr(grad3), dptr(reduced3), _lib.TORCH_TO_OGN[saved3.dtype],
                                        dptr(idx), _index_code(idx), b, length, f, groups, mode, dptr(out),
                                        dptr(ws), ws.numel() * 4, stream_of(saved3))
    check(rc, "group softmax backward")
    return out
