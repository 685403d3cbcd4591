"""ogn_spmm_csr_noalloc (library-owned scratch, no allocation) against
ogn_spmm_csr with a caller workspace, through the C ABI: bitwise equal on
two calls in a row, the second with a smaller input, for sum and max + arg;
a request above the scratch maximum is refused without launching.

This file is collected last (test_zz_*), so that it runs both after every
other GPU test and, alone, in a fresh process.
"""

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

SCRATCH_MAX = 134217728  # OGN_SPMM_NOALLOC_SCRATCH_BYTES in include/ogn.h


def _powerlaw(m, n, nnz, seed):
    from ops_gnn.synthetic import powerlaw_csr

    ptr, col, rng = powerlaw_csr(m, n, nnz, max(nnz // 10, 1), seed)
    return torch.from_numpy(ptr).cuda(), torch.from_numpy(col).cuda(), rng


def _call(L, noalloc, ptr, col, val, mat, reduce, out_dtype):
    m, (n, k), nnz = ptr.numel() - 1, mat.shape, col.numel()
    out = torch.full((m, k), float("nan"), device="cuda").to(out_dtype)
    arg = torch.full((m, k), -7, dtype=torch.int64, device="cuda") if reduce >= 2 else None
    code = L.TORCH_TO_OGN
    common = (L.dptr(ptr), L.dptr(col), L.I64, L.dptr(val), 1, L.dptr(mat), code[mat.dtype], 1, m, n, k, nnz,
              L.dptr(out), code[out_dtype], L.dptr(arg), reduce)
    stream = L.stream_of(mat)
    if noalloc:
        rc = L.lib.ogn_spmm_csr_noalloc(*common, stream)
    else:
        ws_bytes = L.lib.ogn_spmm_csr_workspace_size(m, nnz, k, 1, code[mat.dtype], reduce)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
        rc = L.lib.ogn_spmm_csr(*common, L.dptr(ws), ws_bytes, stream)
    L.check(rc, "noalloc test")
    torch.cuda.synchronize()
    return out, arg


@pytest.mark.parametrize("dtype,reduce", [(torch.float32, 0), (torch.float32, 3), (torch.bfloat16, 0),
                                          (torch.float16, 2), (torch.int8, 1)])
def test_noalloc_matches_workspace_entry(dtype, reduce):
    import ops_gnn._lib as L

    sizes = [(40_000, 30_000, 900_000, 11), (3_000, 2_500, 50_000, 12)]  # second call smaller
    for m, n, nnz, seed in sizes:
        ptr, col, rng = _powerlaw(m, n, nnz, seed)
        if dtype == torch.int8:
            mat = torch.from_numpy(rng.integers(-128, 128, (n, 64)).astype(np.int8)).cuda()
            val = torch.from_numpy(rng.integers(-128, 128, col.numel()).astype(np.int8)).cuda()
            out_dtype = torch.int32
        else:
            mat = torch.from_numpy(rng.standard_normal((n, 64), dtype=np.float32)).cuda().to(dtype)
            val = torch.from_numpy(rng.random(col.numel(), dtype=np.float32)).cuda().to(dtype)
            out_dtype = dtype
        print(f"noalloc case dtype={dtype} reduce={reduce} m={m} nnz={nnz}", flush=True)
        want, want_arg = _call(L, False, ptr, col, val, mat, reduce, out_dtype)
        got, got_arg = _call(L, True, ptr, col, val, mat, reduce, out_dtype)
        assert torch.equal(got.view(torch.uint8) if got.dtype != torch.int32 else got,
                           want.view(torch.uint8) if want.dtype != torch.int32 else want), (m, nnz)
        if reduce >= 2:
            assert torch.equal(got_arg, want_arg)


def test_noalloc_refuses_requests_above_the_maximum():
    import ops_gnn._lib as L

    m, n, k, nnz = 2_450_000, 2_450_000, 128, 62_000_000
    need = L.lib.ogn_spmm_csr_workspace_size(m, nnz, k, 1, L.F32, 3)
    assert need > SCRATCH_MAX
    assert L.lib.ogn_spmm_csr_workspace_size(m, nnz, k, 1, L.F32, 0) <= SCRATCH_MAX  # config-3 sum fits
    marker = torch.full((4,), 5.0, device="cuda")
    # pointers are never dereferenced: the size check comes first
    rc = L.lib.ogn_spmm_csr_noalloc(L.dptr(marker), L.dptr(marker), L.I64, None, 1, L.dptr(marker), L.F32, 1,
                                    m, n, k, nnz, L.dptr(marker), L.F32, L.dptr(marker), 3, L.stream_of(marker))
    assert rc == L.EINVAL
    assert b"maximum" in L.lib.ogn_last_error()
    torch.cuda.synchronize()
    assert torch.equal(marker.cpu(), torch.full((4,), 5.0))
