"""Seeded random sweeps against the oracle, across the engine's schedules.

Each case draws its own shape: segment / row lengths mixing empty and 1-3
position rows with long ones (Zipf for the SpMM graphs), a forced engine
chunk size (64 .. 512 positions, or the library's choice), the feature
width (1 .. 128), the dtype (fp32 / fp16 / bf16) and the reduction.  That
reaches every path of the CSR engine (step schedule, long runs, sub-group
rows, wave-folded long rows, pre-fold, fix-up), the sorted and the
sort-then-gather scatter, and the softmax family over an unsorted index.
Same bars as the targeted tests: min/max values and args bit-exact, sums
within rel 1e-5 (fp32) / 1e-2 (fp16, bf16), softmax family within the
reference's tolerances (test/common/grouped_softmax_golden.py:24-28).
"""

import os

import numpy as np
import pytest
import torch

from _util import assert_exact, assert_sum_close, cast_like

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]
SOFT_TOL = {torch.float32: 1e-5, torch.float16: 2e-2, torch.bfloat16: 4e-2}


@pytest.fixture
def chunk_env():
    old = os.environ.get("OGN_ENGINE_CHUNK")

    def set_chunk(c):
        if c:
            os.environ["OGN_ENGINE_CHUNK"] = str(c)
        else:
            os.environ.pop("OGN_ENGINE_CHUNK", None)

    yield set_chunk
    if old is None:
        os.environ.pop("OGN_ENGINE_CHUNK", None)
    else:
        os.environ["OGN_ENGINE_CHUNK"] = old


def _values(rng, shape, dtype, ties):
    a = rng.integers(-3, 4, shape) if ties else rng.standard_normal(shape)
    return torch.from_numpy(a.astype(np.float32)).to(dtype)


@pytest.mark.parametrize("seed", range(60))
def test_segment_and_scatter_sweep(ogn, oracle, chunk_env, seed):
    rng = np.random.default_rng(1000 + seed)
    chunk_env(int(rng.choice([64, 128, 192, 256, 512, 0])))
    segs = int(rng.integers(1, 3000))
    kind = rng.random(segs)
    lengths = np.where(kind < 0.3, 0, rng.integers(1, 4, segs))
    big = kind > 0.97
    lengths[big] = rng.integers(10, int(rng.choice([100, 2000, 20000])), int(big.sum()))
    lengths[0] += 1  # at least one position
    feat = int(rng.choice([1, 2, 4, 8, 16, 32, 33, 64, 128]))
    dtype = DTYPES[int(rng.integers(0, 3))]
    reduce = str(rng.choice(["sum", "mean", "min", "max"]))
    ties = reduce in ("min", "max")
    e = int(lengths.sum())
    src = _values(rng, (e, feat), dtype, ties)
    ptr = torch.from_numpy(np.concatenate([[0], np.cumsum(lengths)]))
    what = f"seed {seed} segs {segs} e {e} f {feat} {dtype} {reduce}"
    res = getattr(ogn, f"segment_{reduce}_csr")(src.cuda(), ptr.cuda())
    out, arg = res if isinstance(res, tuple) else (res, None)
    gold, garg = oracle.segment_csr(src, ptr, reduce)
    if ties:
        assert_exact(out, cast_like(gold, dtype), what)
        assert_exact(arg, garg, what + " arg")
    else:
        scale, _ = oracle.segment_csr(src.float().abs(), ptr, reduce)
        assert_sum_close(out, gold, scale, dtype, what)
    idx = np.repeat(np.arange(segs), lengths)
    for order in ("sorted", "shuffled"):
        p = rng.permutation(e) if order == "shuffled" else np.arange(e)
        ix, sx = idx[p], src[torch.from_numpy(p)]
        got = ogn.scatter(sx.cuda(), torch.from_numpy(ix).cuda(), 0, dim_size=segs, reduce=reduce)
        full = np.broadcast_to(ix.reshape(-1, 1), sx.shape)
        want, _ = oracle.scatter(sx.float(), full, 0, segs, reduce)
        if ties:
            assert_exact(got.float(), want, f"{what} scatter {order}")
        else:
            scale, _ = oracle.scatter(sx.float().abs(), full, 0, segs, reduce)
            assert_sum_close(got, want, scale, dtype, f"{what} scatter {order}")


@pytest.mark.parametrize("seed", range(60))
def test_spmm_and_unsorted_softmax_sweep(ogn, oracle, chunk_env, seed):
    rng = np.random.default_rng(5000 + seed)
    chunk_env(int(rng.choice([64, 128, 256, 512, 0])))
    m, n = int(rng.integers(1, 2000)), int(rng.integers(1, 3000))
    deg = np.minimum(rng.zipf(1.8, m), int(rng.choice([50, 5000])))
    deg[rng.random(m) < 0.1] = 0
    deg[0] += 1
    e = int(deg.sum())
    col = np.concatenate([np.sort(rng.integers(0, n, d)) for d in deg]).astype(np.int64)
    ptr = torch.from_numpy(np.concatenate([[0], np.cumsum(deg)]))
    k = int(rng.choice([1, 4, 8, 16, 32, 64, 128]))
    dtype = DTYPES[int(rng.integers(0, 3))]
    reduce = str(rng.choice(["sum", "mean", "min", "max"]))
    ties = reduce in ("min", "max")
    mat = _values(rng, (n, k), dtype, ties)
    val = torch.from_numpy(rng.integers(1, 3, e).astype(np.float32)).to(dtype)
    what = f"seed {seed} m {m} n {n} e {e} k {k} {dtype} {reduce}"
    res = ogn.csr_spmm(ptr.cuda(), torch.from_numpy(col).cuda(), val.cuda(), mat.cuda(), reduce)
    got, arg = res if ties else (res, None)
    gold, garg = oracle.spmm_csr(ptr, torch.from_numpy(col), val, mat, reduce)
    if ties:
        assert_exact(got, cast_like(gold, dtype), what)
        assert_exact(arg, garg, what + " arg")
    else:
        scale, _ = oracle.spmm_csr(ptr, torch.from_numpy(col), val.float().abs(), mat.float().abs(), reduce)
        assert_sum_close(got, gold, scale, dtype, what)
    # the grouped softmax family over a shuffled index of the same groups
    ix = np.repeat(np.arange(m), deg)[rng.permutation(e)]
    src = torch.from_numpy((rng.standard_normal((e, k)) * 3).astype(np.float32)).to(dtype)
    mode = str(rng.choice(["softmax", "log_softmax", "logsumexp"]))
    fn = {"softmax": ogn.scatter_softmax, "log_softmax": ogn.scatter_log_softmax,
          "logsumexp": ogn.scatter_logsumexp}[mode]
    got = fn(src.cuda(), torch.from_numpy(ix).cuda(), 0, m).float().cpu().numpy()
    gold = cast_like(oracle.group_softmax(src, torch.from_numpy(ix), 0, m, mode), dtype)
    tol = SOFT_TOL[dtype]
    np.testing.assert_allclose(got, gold, rtol=tol, atol=tol, equal_nan=True, err_msg=f"{what} {mode}")
