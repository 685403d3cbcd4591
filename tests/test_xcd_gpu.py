"""GPU parity of the XCD-tiled SDDMM dot and SpMM sum (ogn_xcd_plan,
ogn_sddmm_dot_xcd, ogn_spmm_sum_xcd).

The path is taken automatically for 8-96 MB feature tables on graphs of at
least 2^20 edges; OGN_XCD=1 forces it for smaller cases and OGN_XCD=0 turns
it off.  SDDMM scores must equal the untiled kernel's bit for bit (same packet
dots and sub-group sums per edge) and the oracle within the dtype tolerance;
SpMM sums (per-tile fp32 partials added in tile order) are checked against
the oracle at rel 1e-5 (fp32) / 1e-2 (fp16, bf16) of sum |terms|.  Cases:
every row width (64-512 bytes), fp32 / fp16 / bf16, int32 and int64 indices,
empty rows, a hub row spanning several 8192-edge chunks, rows whose columns
all fall in one tile, unsorted columns (the plan reports it and the path is
not taken; a direct call is still right), repeated calls on one kept plan,
and a graph that selects the path by its size.
"""

import ctypes
import os

import numpy as np
import pytest
import torch

from _util import assert_sum_close, cast_like

pytestmark = pytest.mark.gpu


@pytest.fixture
def force_xcd():
    old = os.environ.get("OGN_XCD")
    os.environ["OGN_XCD"] = "1"
    yield
    if old is None:
        del os.environ["OGN_XCD"]
    else:
        os.environ["OGN_XCD"] = old


def _graph(seed, m=3000, n=2500, mean=40, hub=0, sort=True):
    rng = np.random.default_rng(seed)
    deg = np.maximum(rng.lognormal(np.log(mean), 1.0, m).astype(np.int64), 0)
    deg[::17] = 0
    if hub:
        deg[m // 2] = hub
    cols = [rng.integers(0, n, d) for d in deg]
    # a few rows with every column inside one tile
    for r in range(5, m, 97):
        t = rng.integers(0, 8)
        lo = t * ((n + 7) // 8)
        cols[r] = rng.integers(lo, min(n, lo + (n + 7) // 8), deg[r])
    col = np.concatenate([np.sort(c) if sort else c for c in cols]).astype(np.int64)
    ptr = np.concatenate([[0], np.cumsum(deg)]).astype(np.int64)
    return torch.from_numpy(ptr), torch.from_numpy(col), rng


def _bits(t):
    # raw bits, so that 16-bit results compare exactly through numpy
    t = t.detach().cpu()
    return t.view({2: torch.int16, 4: torch.int32}[t.element_size()]).numpy()


def _untiled(fn):
    old = os.environ.get("OGN_XCD")
    os.environ["OGN_XCD"] = "0"
    try:
        return fn()
    finally:
        if old is None:
            del os.environ["OGN_XCD"]
        else:
            os.environ["OGN_XCD"] = old


CASES = [(torch.float16, 32), (torch.float16, 64), (torch.float16, 128), (torch.float16, 256),
         (torch.bfloat16, 64), (torch.float32, 16), (torch.float32, 32), (torch.float32, 64), (torch.float32, 128)]


@pytest.mark.parametrize("dtype,k", CASES)
@pytest.mark.parametrize("index_dtype", [torch.int64, torch.int32])
def test_sddmm_dot_xcd_matches_untiled_and_oracle(ogn, oracle, force_xcd, dtype, k, index_dtype):
    ptr, col, rng = _graph(k, hub=20_000)
    m, n = ptr.numel() - 1, 2500
    q = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(dtype).cuda()
    kk = torch.from_numpy(rng.standard_normal((n, k)).astype(np.float32)).to(dtype).cuda()
    p, c = ptr.to(index_dtype).cuda(), col.to(index_dtype).cuda()
    got = ogn.sddmm_csr(p, c, q, kk, "dot")
    ref = _untiled(lambda: ogn.sddmm_csr(p, c, q, kk, "dot"))
    assert np.array_equal(_bits(got), _bits(ref)), f"xcd vs untiled {dtype} k{k}"
    gold = oracle.sddmm(ptr.numpy(), col.numpy(), q.float().cpu().numpy(), kk.float().cpu().numpy(), "dot")
    scale = oracle.sddmm(ptr.numpy(), col.numpy(), q.float().abs().cpu().numpy(), kk.float().abs().cpu().numpy(),
                         "dot")
    assert_sum_close(got, cast_like(gold, dtype), scale, dtype, f"xcd sddmm {dtype} k{k}")


@pytest.mark.parametrize("dtype,k", CASES)
@pytest.mark.parametrize("index_dtype", [torch.int64, torch.int32])
def test_spmm_sum_xcd_matches_oracle(ogn, oracle, force_xcd, dtype, k, index_dtype):
    ptr, col, rng = _graph(100 + k, hub=20_000)
    n = 2500
    val = torch.from_numpy(rng.random(col.numel()).astype(np.float32)).to(dtype)
    mat = torch.from_numpy(rng.standard_normal((n, k)).astype(np.float32)).to(dtype)
    p, c = ptr.to(index_dtype).cuda(), col.to(index_dtype).cuda()
    for _ in range(2):  # second call: the kept plan
        if index_dtype == torch.int64:
            got = ogn.csr_spmm(p, c, val.cuda(), mat.cuda(), "sum")
        else:  # torch_sparse takes int64 indices only; int32 through the native layer
            from ops_gnn import _native

            got = torch.empty((p.numel() - 1, k), dtype=dtype, device="cuda")
            assert _native.spmm_sum_xcd(p, c, val.cuda(), mat.cuda(), got)
        gold, _ = oracle.spmm_csr(ptr, col, val, mat, "sum")
        scale, _ = oracle.spmm_csr(ptr, col, val.float().abs(), mat.float().abs(), "sum")
        assert got.dtype == dtype
        assert_sum_close(got, gold, scale, dtype, f"xcd spmm {dtype} k{k}")


def test_spmm_sum_xcd_fp32_output_and_empty_tiles(ogn, oracle, force_xcd):
    # fp16 in, fp32 out; rows with a single edge and many empty rows, so most
    # (row, tile) partials are zeros written by the tile pass
    rng = np.random.default_rng(7)
    m, n, k = 5000, 4000, 64
    deg = rng.integers(0, 3, m)
    col = np.concatenate([np.sort(rng.integers(0, n, d)) for d in deg]).astype(np.int64)
    ptr = torch.from_numpy(np.concatenate([[0], np.cumsum(deg)]).astype(np.int64))
    val = torch.from_numpy(rng.random(col.size).astype(np.float32)).half()
    mat = torch.from_numpy(rng.standard_normal((n, k)).astype(np.float32)).half()
    got = ogn.csr_spmm(ptr.cuda(), torch.from_numpy(col).cuda(), val.cuda(), mat.cuda(), "sum",
                       output_dtype=torch.float32)
    assert got.dtype == torch.float32
    gold, _ = oracle.spmm_csr(ptr, torch.from_numpy(col), val, mat, "sum")
    scale, _ = oracle.spmm_csr(ptr, torch.from_numpy(col), val.float().abs(), mat.float().abs(), "sum")
    assert_sum_close(got, gold, scale, torch.float32, "xcd fp16->fp32")


def test_unsorted_columns_fall_back_and_direct_call_is_right(ogn, oracle, force_xcd):
    from ops_gnn import _lib, _native

    ptr, col, rng = _graph(9, sort=False)
    m, n, k = ptr.numel() - 1, 2500, 64
    p, c = ptr.cuda(), col.cuda()
    assert _native.xcd_plan(p, c, n) is None  # reported unsorted
    q = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).half().cuda()
    kk = torch.from_numpy(rng.standard_normal((n, k)).astype(np.float32)).half().cuda()
    got = ogn.sddmm_csr(p, c, q, kk, "dot")  # untiled path
    gold = oracle.sddmm(ptr.numpy(), col.numpy(), q.float().cpu().numpy(), kk.float().cpu().numpy(), "dot")
    scale = oracle.sddmm(ptr.numpy(), col.numpy(), q.float().abs().cpu().numpy(), kk.float().abs().cpu().numpy(),
                         "dot")
    assert_sum_close(got, cast_like(gold, torch.float16), scale, torch.float16, "unsorted fallback")
    # the tiles partition every row's edges whatever the order: a direct call is right too
    L = _lib.lib
    plan = torch.empty(L.ogn_xcd_plan_bytes(m, col.numel()), dtype=torch.uint8, device="cuda")
    flag = ctypes.c_int(-1)
    _lib.check(L.ogn_xcd_plan(_lib.dptr(p), _lib.dptr(c), _lib.I64, m, n, col.numel(), _lib.dptr(plan), plan.numel(),
                              ctypes.byref(flag), _lib.stream_of(p)), "plan")
    assert flag.value == 0
    out = torch.empty(col.numel(), dtype=torch.float16, device="cuda")
    _lib.check(L.ogn_sddmm_dot_xcd(_lib.dptr(plan), m, col.numel(), _lib.dptr(c), _lib.I64, _lib.dptr(q), m,
                                   _lib.dptr(kk), n, k, _lib.TORCH_TO_OGN[torch.float16], _lib.dptr(out), 0,
                                   _lib.stream_of(q)), "sddmm xcd")
    assert np.array_equal(_bits(out), _bits(got)), "direct call on unsorted columns"


def test_kept_plan_rebuilt_after_inplace_change(ogn, oracle, force_xcd):
    ptr, col, rng = _graph(11)
    n, k = 2500, 64
    p, c = ptr.cuda(), col.cuda()
    val = torch.from_numpy(rng.random(col.numel()).astype(np.float32)).cuda()
    mat = torch.from_numpy(rng.standard_normal((n, k)).astype(np.float32)).cuda()
    ogn.csr_spmm(p, c, val, mat, "sum")
    # change columns in place (rows stay sorted): the plan is rebuilt
    c2 = col.clone()
    for r in range(0, ptr.numel() - 1, 3):
        a, z = int(ptr[r]), int(ptr[r + 1])
        c2[a:z] = torch.sort(torch.from_numpy(np.random.default_rng(r).integers(0, n, z - a)))[0]
    c.copy_(c2.cuda())
    got = ogn.csr_spmm(p, c, val, mat, "sum")
    gold, _ = oracle.spmm_csr(ptr, c2, val.cpu(), mat.cpu(), "sum")
    scale, _ = oracle.spmm_csr(ptr, c2, val.cpu().abs(), mat.cpu().abs(), "sum")
    assert_sum_close(got, gold, scale, torch.float32, "after in-place change")


def test_size_selects_the_path(ogn, oracle):
    # an 8+ MB table and 2^20+ edges take the path without forcing it
    from ops_gnn import _native

    rng = np.random.default_rng(13)
    m, n, k = 40_000, 80_000, 64  # K table: 80 000 x 128 B = 10.2 MB
    deg = rng.poisson(30, m)
    col = np.concatenate([np.sort(rng.integers(0, n, d)) for d in deg]).astype(np.int64)
    ptr = torch.from_numpy(np.concatenate([[0], np.cumsum(deg)]).astype(np.int64))
    assert _native.xcd_wanted(n, k * 2, col.size)
    q = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).half().cuda()
    kk = torch.from_numpy(rng.standard_normal((n, k)).astype(np.float32)).half().cuda()
    p, c = ptr.cuda(), torch.from_numpy(col).cuda()
    got = ogn.sddmm_csr(p, c, q, kk, "dot")
    ref = _untiled(lambda: ogn.sddmm_csr(p, c, q, kk, "dot"))
    assert np.array_equal(_bits(got), _bits(ref)), "size-selected xcd sddmm"
    val = torch.softmax(got.float(), 0).half()
    out = ogn.csr_spmm(p, c, val, kk, "sum")
    ref2 = _untiled(lambda: ogn.csr_spmm(p, c, val, kk, "sum"))
    np.testing.assert_allclose(out.float().cpu().numpy(), ref2.float().cpu().numpy(), rtol=1e-2, atol=1e-3)


def test_wide_tables_read_the_index(ogn, oracle, force_xcd):
    # more than 2^19 columns: tiles wider than 2^16 columns, so the plan keeps
    # no 16-bit columns (state 1) and the kernels read col
    from ops_gnn import _native

    rng = np.random.default_rng(17)
    m, n, k = 2000, 600_000, 16
    deg = rng.poisson(50, m)
    deg[3] = 12_000
    col = np.concatenate([np.sort(rng.integers(0, n, d)) for d in deg]).astype(np.int64)
    ptr = torch.from_numpy(np.concatenate([[0], np.cumsum(deg)]).astype(np.int64))
    p, c = ptr.cuda(), torch.from_numpy(col).cuda()
    kept = _native.xcd_plan(p, c, n)
    assert kept is not None and kept[1] == 1
    q = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).cuda()
    kk = torch.from_numpy(rng.standard_normal((n, k)).astype(np.float32)).cuda()
    got = ogn.sddmm_csr(p, c, q, kk, "dot")
    ref = _untiled(lambda: ogn.sddmm_csr(p, c, q, kk, "dot"))
    assert np.array_equal(_bits(got), _bits(ref)), "wide-table xcd sddmm"
    val = torch.from_numpy(rng.random(col.size).astype(np.float32)).cuda()
    out = ogn.csr_spmm(p, c, val, kk, "sum")
    gold, _ = oracle.spmm_csr(ptr, torch.from_numpy(col), val.cpu(), kk.cpu(), "sum")
    scale, _ = oracle.spmm_csr(ptr, torch.from_numpy(col), val.cpu().abs(), kk.cpu().abs(), "sum")
    assert_sum_close(out, gold, scale, torch.float32, "wide-table xcd spmm")
