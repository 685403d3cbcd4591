"""Loader for libogn_hip.so, the gfx950 kernels behind the C ABI in include/ogn.h.

Replaces the reference's npu-smi / CANN_TARGET target selection
(reference python/ops_gnn/_device.py:15-44, python/ops_gnn/__init__.py:27-42):
there is exactly one build, for gfx950, living next to this file.  A missing
or unloadable library raises ImportError -- there is no CPU fallback.
"""

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (loads torch's HIP runtime first so the library shares it)

LIB_NAME = "libogn_hip.so"
LIB_PATH = Path(os.environ.get("OGN_LIB", Path(__file__).resolve().parent / LIB_NAME))

try:
    _so = ctypes.CDLL(str(LIB_PATH))
except OSError as exc:  # pragma: no cover - exercised only on a broken install
    raise ImportError(
        f"ops_gnn: cannot load the gfx950 kernel library {LIB_PATH} ({exc}). "
        "Build it with `python ops-gnn_amd/build.py` (or __graft_entry__.build())."
    ) from exc

arch = "gfx950"

# dtype codes (include/ogn.h ogn_dtype)
F32, F16, BF16, I8, I32, I64, F64, U8, I16 = range(9)
TORCH_TO_OGN = {
    torch.float32: F32,
    torch.float16: F16,
    torch.bfloat16: BF16,
    torch.int8: I8,
    torch.int32: I32,
    torch.int64: I64,
    torch.float64: F64,
    torch.uint8: U8,
    torch.int16: I16,
}

OK, EINVAL, EUNSUPPORTED, EHIP = 0, 1, 2, 3

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_sz = ctypes.c_size_t

# name -> (restype, argtypes); every entry must be declared in include/ogn.h.
SIGNATURES = {
    "ogn_last_error": (ctypes.c_char_p, []),
    "ogn_arch": (ctypes.c_char_p, []),
    "ogn_abi_version": (_int, []),
    "ogn_timing_enable": (_int, [_int]),
    "ogn_timing_query": (_int, [ctypes.c_char_p, _vp, _vp]),
    "ogn_validate_csr": (_int, [_vp, _vp, _int, _i64, _i64, _i64, _vp, _vp]),
    "ogn_spmm_csr_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _int, _int]),
    "ogn_spmm_csr": (_int, [_vp, _vp, _int, _vp, _i64, _vp, _int, _i64, _i64, _i64, _i64, _i64,
                            _vp, _int, _vp, _int, _vp, _sz, _vp]),
    "ogn_spmm_csr_noalloc": (_int, [_vp, _vp, _int, _vp, _i64, _vp, _int, _i64, _i64, _i64, _i64, _i64,
                                    _vp, _int, _vp, _int, _vp]),
    "ogn_spmm_csr_ex": (_int, [_vp, _vp, _int, _vp, _i64, _vp, _int, _i64, _i64, _i64, _i64, _i64,
                               _vp, _int, _vp, _int, _int, _int, _vp, _sz, _vp]),
    "ogn_sddmm_csr_workspace_size": (_sz, [_i64, _i64, _int]),
    "ogn_sddmm_csr": (_int, [_vp, _vp, _int, _i64, _i64, _vp, _i64, _int, _vp, _i64, _int, _i64, _int, _int,
                             _vp, _vp, _sz, _vp]),
    "ogn_ind2ptr": (_int, [_vp, _int, _i64, _i64, _vp, _vp]),
    "ogn_ptr2ind": (_int, [_vp, _int, _i64, _i64, _vp, _vp]),
    "ogn_segment_reduce_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i64, _int, _int]),
    "ogn_segment_reduce": (_int, [_vp, _i64, _vp, _int, _i64, _i64, _i64, _i64, _vp, _vp, _int, _int, _int,
                                  _vp, _sz, _vp]),
    "ogn_ind2ptr_batched": (_int, [_vp, _i64, _i64, _i64, _vp, _vp]),
    "ogn_index_facts": (_int, [_vp, _i64, _vp, _vp]),
    "ogn_sort_rows_workspace_size": (_sz, [_i64, _i64, _int, _int]),
    "ogn_segment_reduce_gather_workspace_size": (_sz, [_i64, _i64, _i64, _int, _int]),
    "ogn_segment_group_stats_gather": (_int, [_vp, _vp, _vp, _int, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _sz, _vp]),
    "ogn_group_bwd_messages": (_int, [_vp, _vp, _int, _i64, _int, _vp, _vp]),
    "ogn_segment_reduce_gather": (_int, [_vp, _vp, _vp, _int, _i64, _i64, _i64, _i64, _vp, _vp, _int, _int, _int,
                                         _vp, _sz, _vp]),
    "ogn_sort_rows": (_int, [_vp, _i64, _i64, _vp, _vp, _vp, _vp, _int, _vp, _vp, _int, _vp, _sz, _vp]),
    "ogn_segment_group_stats": (_int, [_vp, _vp, _int, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _sz, _vp]),
    "ogn_segment_group_softmax_workspace_size": (_sz, [_i64, _i64, _i64, _int]),
    "ogn_segment_group_softmax": (_int, [_vp, _vp, _int, _i64, _i64, _i64, _vp, _int, _int, _vp, _sz, _vp]),
    "ogn_scatter_atomic_workspace_size": (_sz, [_i64, _i64, _i64, _int]),
    "ogn_scatter_atomic": (_int, [_vp, _int, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _int,
                                  _int, _vp, _sz, _vp]),
    "ogn_group_stats_atomic": (_int, [_vp, _int, _vp, _int, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp]),
    "ogn_group_softmax_apply": (_int, [_vp, _int, _vp, _int, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _int,
                                       _vp]),
    "ogn_group_lse_from_stats": (_int, [_vp, _vp, _i64, _vp, _int, _vp]),
    "ogn_gather_csr": (_int, [_vp, _i64, _vp, _i64, _i64, _i64, _i64, _vp, _vp]),
    "ogn_gather_coo": (_int, [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp]),
    "ogn_group_softmax_backward": (_int, [_vp, _vp, _vp, _int, _vp, _int, _i64, _i64, _i64, _i64, _int, _vp,
                                          _vp, _sz, _vp]),
    "ogn_calibrate_gather": (_int, [_vp, _i64, _i64, _vp, _i64, _vp, _vp]),
    "ogn_xcd_plan_bytes": (_sz, [_i64, _i64]),
    "ogn_xcd_plan": (_int, [_vp, _vp, _int, _i64, _i64, _i64, _vp, _sz, _vp, _vp]),
    "ogn_sddmm_dot_xcd": (_int, [_vp, _i64, _i64, _vp, _int, _vp, _i64, _vp, _i64, _i64, _int, _vp, _int, _vp]),
    "ogn_spmm_sum_xcd_workspace_size": (_sz, [_i64, _i64]),
    "ogn_spmm_sum_xcd": (_int, [_vp, _i64, _i64, _vp, _int, _vp, _vp, _i64, _i64, _int, _vp, _int, _vp, _sz, _int,
                                 _vp]),
    "ogn_calibrate_stream": (_int, [_vp, _vp, _i64, _vp, _vp]),
}

# reduce / semantics codes (include/ogn.h)
R_SUM, R_MEAN, R_MIN, R_MAX, R_PROD, R_LSE = range(6)
SEM_SEGMENT_CSR, SEM_SEGMENT_COO, SEM_SCATTER, SEM_DGL = range(4)
GROUP_BWD_TOTALS_GIVEN = 4  # ogn_group_softmax_backward: the workspace holds the group sums
MSG_MUL, MSG_ADD, MSG_SUB, MSG_DIV = range(4)
SPMM_TORCH_SPARSE, SPMM_DGL = range(2)
SDDMM_OPS = {"dot": 0, "add": 1, "sub": 2, "mul": 3, "div": 4, "copy_lhs": 5, "copy_rhs": 6}
SEG_HAS_OUT = 1
SEG_SHORT_SEGMENTS = 2  # no segment holds more than SHORT_SEGMENT_MAX rows
SEG_KEEP_LAYOUT = 4
SEG_REUSE_LAYOUT = 8
SHORT_SEGMENT_MAX = 4096

for _name, (_res, _args) in SIGNATURES.items():
    _fn = getattr(_so, _name)
    _fn.restype = _res
    _fn.argtypes = _args

lib = _so


def check(rc: int, what: str) -> None:
    """Turn a C-ABI status into the exception the reference raises (RuntimeError,
    like its TORCH_CHECK failures)."""
    if rc != OK:
        msg = _so.ogn_last_error().decode(errors="replace")
        raise RuntimeError(f"{what}: {msg or 'error code %d' % rc}")


def dptr(t):
    """Device address of a tensor (None -> NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor):
    """hipStream_t of torch's current stream on the tensor's device."""
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require_gpu(*tensors, what="ops_gnn"):
    for t in tensors:
        if t is not None and (not isinstance(t, torch.Tensor) or t.device.type != "cuda"):
            raise ValueError(f"{what}: tensors must be on the GPU (torch 'cuda' device on ROCm)")


def workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def timing_enable(on: bool) -> None:
    check(_so.ogn_timing_enable(1 if on else 0), "timing_enable")


def timing_query(kernel: str):
    """(total_ms, launches) of the recorded launches of `kernel`."""
    total = ctypes.c_double(0.0)
    count = ctypes.c_int64(0)
    check(_so.ogn_timing_query(kernel.encode(), ctypes.byref(total), ctypes.byref(count)), "timing_query")
    return total.value, count.value
