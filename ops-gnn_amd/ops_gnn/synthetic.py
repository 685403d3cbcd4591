"""Seeded synthetic graphs for the benchmark configurations (NumPy PCG64).

cfg1..cfg5 use seeds 1..5.  Every generator returns NumPy arrays (int64
indices, float32 values/features); callers move them to the GPU.  Sorting of
the (row, col) keys -- the slow part at full size -- can be delegated to a
callable (e.g. a GPU sort) through ``sort_keys``; the result is identical.
"""

from typing import Callable, Optional

import numpy as np


def rng_for(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def _rescale_degrees(raw: np.ndarray, target: int, cap: int, lo: int = 1) -> np.ndarray:
    """Find f by bisection so that sum(clip(round(f * raw), lo, cap)) ~= target."""
    raw = raw.astype(np.float64)

    def total(f):
        return int(np.clip(np.rint(f * raw), lo, cap).sum())

    a, b = 0.0, 1.0
    while total(b) < target:
        b *= 2.0
        if b > 1e12:
            break
    for _ in range(100):
        mid = 0.5 * (a + b)
        if total(mid) < target:
            a = mid
        else:
            b = mid
    deg = np.clip(np.rint(b * raw), lo, cap).astype(np.int64)
    return deg


def _fix_total(deg: np.ndarray, target: int, rng: np.random.Generator, cap: int) -> np.ndarray:
    """Spread the remaining difference as +-1 over random rows with room."""
    diff = target - int(deg.sum())
    while diff != 0:
        step = 1 if diff > 0 else -1
        ok = np.nonzero((deg < cap) if step > 0 else (deg > 1))[0]
        pick = rng.choice(ok, size=min(abs(diff), ok.size), replace=False)
        deg[pick] += step
        diff -= step * pick.size
    return deg


def sorted_columns(deg: np.ndarray, n: int, rng: np.random.Generator,
                   sort_keys: Optional[Callable[[np.ndarray], np.ndarray]] = None) -> np.ndarray:
    """Uniform random columns in [0, n), sorted within each row (duplicates allowed)."""
    m = deg.shape[0]
    e = int(deg.sum())
    rows = np.repeat(np.arange(m, dtype=np.int64), deg)
    cols = rng.integers(0, n, size=e, dtype=np.int64)
    keys = rows * np.int64(n) + cols
    del rows, cols
    keys = sort_keys(keys) if sort_keys is not None else np.sort(keys, kind="stable")
    return keys % np.int64(n)


def csr_from_degrees(deg: np.ndarray) -> np.ndarray:
    ptr = np.zeros(deg.shape[0] + 1, dtype=np.int64)
    np.cumsum(deg, out=ptr[1:])
    return ptr


def cfg1_spmm_small(seed: int = 1):
    """10k x 10k, Poisson(10) row lengths, K=64 fp32."""
    rng = rng_for(seed)
    m = n = 10_000
    deg = rng.poisson(10, size=m).astype(np.int64)
    col = sorted_columns(deg, n, rng)
    ptr = csr_from_degrees(deg)
    val = rng.random(col.shape[0], dtype=np.float32)
    mat = rng.standard_normal((n, 64), dtype=np.float32)
    return ptr, col, val, mat


def cfg2_segments(seed: int = 2, rows: int = 1_000_000, segs: int = 62_500, feat: int = 128):
    """src [rows, feat] N(0,1); Poisson(16) segment lengths, 1 % forced empty,
    total fixed to `rows`."""
    rng = rng_for(seed)
    lengths = rng.poisson(rows / segs, size=segs).astype(np.int64)
    empty = rng.choice(segs, size=max(1, segs // 100), replace=False)
    lengths[empty] = 0
    nonempty = np.nonzero(lengths)[0]
    diff = rows - int(lengths.sum())
    while diff != 0:
        step = 1 if diff > 0 else -1
        cand = nonempty if step > 0 else nonempty[lengths[nonempty] > 1]
        pick = rng.choice(cand, size=min(abs(diff), cand.size), replace=False)
        lengths[pick] += step
        diff -= step * pick.size
    indptr = csr_from_degrees(lengths)
    src = rng.standard_normal((rows, feat), dtype=np.float32)
    return src, indptr


def cfg3_powerlaw_degrees(seed: int = 3, m: int = 2_450_000, nnz: int = 62_000_000,
                          cap: int = 20_000, a: float = 2.1):
    rng = rng_for(seed)
    raw = np.minimum(rng.zipf(a, size=m), cap)
    deg = _rescale_degrees(raw, nnz, cap)
    deg = _fix_total(deg, nnz, rng, cap)
    return deg, rng


def cfg3_powerlaw_spmm(seed: int = 3, m: int = 2_450_000, nnz: int = 62_000_000, cap: int = 20_000,
                       k: int = 128, sort_keys=None, with_mat: bool = True):
    """Power-law CSR: Zipf(2.1) degrees capped at `cap`, rescaled to `nnz`
    edges; uniform sorted columns; values U[0,1); B [m, k] N(0,1)."""
    deg, rng = cfg3_powerlaw_degrees(seed, m, nnz, cap)
    col = sorted_columns(deg, m, rng, sort_keys)
    ptr = csr_from_degrees(deg)
    val = rng.random(col.shape[0], dtype=np.float32)
    mat = rng.standard_normal((m, k), dtype=np.float32) if with_mat else None
    return ptr, col, val, mat


def cfg4_gat_graph(seed: int = 4, n: int = 233_000, nnz: int = 114_600_000, feat: int = 64,
                   sort_keys=None):
    """Lognormal degrees (mean ~490, sigma 1) rescaled to `nnz`, capped at n;
    Q, K, V [n, feat] N(0,1) (cast to fp16 by the caller)."""
    rng = rng_for(seed)
    sigma = 1.0
    mu = np.log(nnz / n) - sigma ** 2 / 2
    raw = rng.lognormal(mu, sigma, size=n)
    deg = _rescale_degrees(raw, nnz, n)
    deg = _fix_total(deg, nnz, rng, n)
    col = sorted_columns(deg, n, rng, sort_keys)
    ptr = csr_from_degrees(deg)
    q = rng.standard_normal((n, feat), dtype=np.float32)
    kk = rng.standard_normal((n, feat), dtype=np.float32)
    v = rng.standard_normal((n, feat), dtype=np.float32)
    return ptr, col, q, kk, v


def cfg5_coo_scatter(seed: int = 5, nodes: int = 1_000_000, edges: int = 50_000_000, feat: int = 32,
                     a: float = 1.8):
    """Sorted destination index with Zipf(1.8) in-degree rescaled to `edges`;
    src [edges, feat] N(0,1)."""
    rng = rng_for(seed)
    raw = np.minimum(rng.zipf(a, size=nodes), nodes)
    deg = _rescale_degrees(raw, edges, nodes)
    deg = _fix_total(deg, edges, rng, nodes)
    index = np.repeat(np.arange(nodes, dtype=np.int64), deg)
    src = rng.standard_normal((edges, feat), dtype=np.float32)
    return index, src


def powerlaw_csr(m: int, n: int, nnz: int, cap: int, seed: int, a: float = 2.1):
    """Scaled-down power-law CSR for tests (same recipe as cfg3)."""
    rng = rng_for(seed)
    raw = np.minimum(rng.zipf(a, size=m), cap)
    deg = _rescale_degrees(raw, nnz, cap)
    col = sorted_columns(deg, n, rng)
    return csr_from_degrees(deg), col, rng
