"""C-ABI surface checks (CPU only: load + symbol table, no kernel launches)."""

import ctypes
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "ogn.h"
LIB = ROOT / "ops-gnn_amd" / "ops_gnn" / "libogn_hip.so"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*[A-Za-z_][\w\s\*]*?\b(ogn_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_functions():
    names = declared_functions()
    assert "ogn_spmm_csr" in names and "ogn_last_error" in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(LIB))
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"declared in ogn.h but not exported: {missing}"


def test_python_bindings_cover_header_exactly():
    import ops_gnn._lib as L

    assert sorted(L.SIGNATURES) == declared_functions()


def test_identification_calls():
    import ops_gnn._lib as L

    assert L.lib.ogn_arch() == b"gfx950"
    assert L.lib.ogn_abi_version() >= 1
    assert L.lib.ogn_last_error() == b""


def test_argument_errors_are_reported_without_gpu():
    import ops_gnn._lib as L

    rc = L.lib.ogn_spmm_csr(None, None, 7, None, 1, None, 0, 1, 1, 1, 1, 0, None, 0, None, 0, None, 0, None)
    assert rc == L.EINVAL
    assert b"index dtype" in L.lib.ogn_last_error()
    rc = L.lib.ogn_ind2ptr(None, L.I64, -1, 3, None, None)
    assert rc == L.EINVAL and b"negative" in L.lib.ogn_last_error()


def test_workspace_query_is_pure_host():
    import ops_gnn._lib as L

    a = L.lib.ogn_spmm_csr_workspace_size(100, 1000, 128, 1, L.F32, 0)
    b = L.lib.ogn_spmm_csr_workspace_size(100, 1000, 128, 1, L.F32, 3)
    assert 0 < a < b


def test_exact_segment_workspace_sizes():
    # integer dtypes: piece records (one int64 per feature and record, two
    # records per 2048-position piece; min/max also keep positions), only
    # when a segment can be longer than 4096 rows; float64: none
    import ops_gnn._lib as L

    i32 = L.TORCH_TO_OGN[__import__("torch").int32]
    f64 = L.TORCH_TO_OGN[__import__("torch").float64]
    size = L.lib.ogn_segment_reduce_workspace_size
    assert size(1, 4096, 10, 8, 1, i32, L.R_SUM) == 0
    s = size(1, 10_000, 10, 8, 1, i32, L.R_SUM)
    assert s >= 5 * 2 * 8 * 8  # 5 pieces
    assert size(1, 10_000, 10, 8, 1, i32, L.R_MAX) == 2 * s
    assert size(2, 10_000, 10, 8, 2, i32, L.R_SUM) >= 2 * 5 * 2 * 8 * 8
    assert size(1, 10_000, 10, 8, 1, f64, L.R_SUM) == 0


def test_sort_rows_refuses_out_of_range_sizes_without_gpu():
    # checked before any device work
    import ops_gnn._lib as L

    assert L.lib.ogn_sort_rows(None, 2**31, 10, None, None, None, None, 0, None, None, 0, None, 0, None) == 2  # OGN_EUNSUPPORTED
    assert L.lib.ogn_sort_rows(None, 10, 2**32, None, None, None, None, 0, None, None, 0, None, 0, None) == 2
    assert L.lib.ogn_sort_rows(None, -1, 10, None, None, None, None, 0, None, None, 0, None, 0, None) == 1  # OGN_EINVAL
    assert L.lib.ogn_sort_rows(None, 0, 10, None, None, None, None, 0, None, None, 0, None, 0, None) == 0  # nothing to sort
    assert L.lib.ogn_sort_rows(None, 10, 5, None, None, None, None, 2, None, None, 0, None, 0, None) == 1
    assert L.lib.ogn_sort_rows_workspace_size(2**31, 10, 0, 0) == 0


def test_sort_rows_companion_rules_without_gpu():
    import ops_gnn._lib as L

    # companion b without a, and a width other than 4 / 8: refused before any device work
    assert L.lib.ogn_sort_rows(None, 10, 5, None, None, None, None, 0, None, None, 4, None, 0, None) == 1
    assert L.lib.ogn_sort_rows_workspace_size(10, 5, 0, 4) == 0
    assert L.lib.ogn_sort_rows_workspace_size(10, 5, 2, 0) == 0


def test_gather_reduction_entry_points_refuse_bad_arguments_without_gpu():
    # checked before any device work
    import ops_gnn._lib as L

    f32 = L.TORCH_TO_OGN[__import__("torch").float32]
    i32 = L.TORCH_TO_OGN[__import__("torch").int32]
    g = L.lib.ogn_segment_reduce_gather
    # (indptr, rows, src, dtype, src_rows, length, segments, k, out, arg, reduce, semantics, flags, ws, bytes, stream)
    assert g(None, None, None, f32, -1, 0, 1, 1, None, None, L.R_SUM, L.SEM_SCATTER, 0, None, 0, None) == 1
    assert g(None, None, None, i32, 1, 1, 1, 1, None, None, L.R_SUM, L.SEM_SCATTER, 0, None, 0, None) == 2
    assert g(None, None, None, f32, 1, 1, 1, 1, None, None, L.R_LSE, L.SEM_SCATTER, 0, None, 0, None) == 2
    assert g(None, None, None, f32, 1, 1, 1, 1, None, None, L.R_SUM, L.SEM_SEGMENT_COO, 0, None, 0, None) == 2
    assert g(None, None, None, f32, 1, 1, 1, 1, None, None, L.R_SUM, L.SEM_SCATTER, 0, None, 0, None) == 1
    assert g(None, None, None, f32, 1, 1, 0, 1, None, None, L.R_SUM, L.SEM_SCATTER, 0, None, 0, None) == 0
    s = L.lib.ogn_segment_group_stats_gather
    assert s(None, None, None, i32, 1, 1, 1, 1, None, None, None, 0, None) == 2
    assert s(None, None, None, f32, 1, 1, 1, 1, None, None, None, 0, None) == 1
    m = L.lib.ogn_group_bwd_messages
    assert m(None, None, f32, 10, 2, None, None) == 1
    assert m(None, None, i32, 10, 0, None, None) == 2
    assert m(None, None, f32, 0, 0, None, None) == 0
    assert L.lib.ogn_segment_reduce_gather_workspace_size(10, 2, 4, i32, L.R_SUM) == 0
    assert L.lib.ogn_segment_reduce_gather_workspace_size(10, 2, 4, f32, L.R_SUM) > 0
