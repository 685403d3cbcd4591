"""Comparison helpers for parity tests (oracle vs HIP)."""

import numpy as np
import torch

# rel 1e-5 for fp32, 1e-2 for fp16/bf16, applied to
# the scale of the summed terms: |a - g| <= rtol * sum|terms| + atol.
RTOL = {torch.float32: 1e-5, torch.float16: 1e-2, torch.bfloat16: 1e-2}
ATOL = {torch.float32: 1e-6, torch.float16: 1e-3, torch.bfloat16: 1e-2}


def to_np(t):
    if isinstance(t, torch.Tensor):
        t = t.detach().cpu()
        if t.dtype in (torch.float16, torch.bfloat16):
            t = t.float()
        return t.numpy()
    return np.asarray(t)


def assert_sum_close(actual, golden, scale, dtype, what=""):
    """Summation parity: |a - g| <= rtol * scale + atol elementwise, where
    `scale` is the same reduction over |terms| (the conditioning of the sum)."""
    a = to_np(actual).astype(np.float64)
    g = np.asarray(golden, dtype=np.float64)
    s = np.abs(np.asarray(scale, dtype=np.float64))
    assert a.shape == g.shape, (what, a.shape, g.shape)
    special = ~np.isfinite(g)
    assert np.array_equal(np.isnan(a), np.isnan(g)), f"{what}: NaN positions differ"
    assert np.array_equal(a[special & ~np.isnan(g)], g[special & ~np.isnan(g)]), f"{what}: inf mismatch"
    fin = np.isfinite(g)
    tol = RTOL[dtype] * s[fin] + ATOL[dtype] + RTOL[dtype] * np.abs(g[fin])
    err = np.abs(a[fin] - g[fin])
    bad = err > tol
    assert not bad.any(), (f"{what}: {bad.sum()} of {bad.size} out of tolerance; "
                           f"max err {err.max():.3e} at {np.argmax(err - tol)}")


def assert_exact(actual, expected, what=""):
    a = to_np(actual)
    e = np.asarray(expected)
    assert a.shape == e.shape, (what, a.shape, e.shape)
    eq = (a == e) | (np.isnan(a.astype(np.float64)) & np.isnan(e.astype(np.float64))) \
        if a.dtype.kind == "f" else (a == e)
    assert eq.all(), f"{what}: {int((~eq).sum())} mismatches, first at {np.argwhere(~eq)[:3].tolist()}"


def cast_like(golden, dtype):
    """Apply the golden's final cast (float64 -> dtype) and return float64."""
    t = torch.from_numpy(np.asarray(golden, dtype=np.float64)).to(dtype)
    return t.double().numpy()
