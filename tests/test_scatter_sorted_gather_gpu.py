"""GPU parity of the unsorted scatter path that sorts the index and reduces
each output row through the permutation (ogn_sort_rows +
ogn_segment_reduce_gather), taken for a 1-D index of at least 2^16
positions.  torch_scatter rules as for the sorted path (reference
test/scatter/arch35/golden.py:47-143): sum / mean / mul accumulate into out
when given, min / max fold with <= / >= so the LATER position wins ties and
its src position is the arg, untouched rows give 0 (or keep out).  Values
and args bit-exact for min / max; sums within rel 1e-5 (fp32) / 1e-2
(fp16, bf16) of the oracle.  Inputs: hub-skewed unsorted indices with few
distinct source values (many ties), empty output rows, a second call on the
same index (cached sort), and the C ABI directly."""

import numpy as np
import pytest
import torch

from _util import assert_exact, assert_sum_close

pytestmark = pytest.mark.gpu

N = 1 << 17  # positions: above the sort-path threshold


def _index(seed, size):
    rng = np.random.default_rng(seed)
    idx = rng.integers(0, size, N)
    idx[rng.random(N) < 0.3] = 7  # a hub
    idx[rng.random(N) < 0.1] = size - 1
    idx[idx == size // 2] = size // 2 + 1  # an empty output row
    return idx.astype(np.int64)


def _src(rng, feat, dtype, ties):
    a = rng.integers(-3, 4, (N, feat)).astype(np.float32) if ties else rng.standard_normal((N, feat)).astype(np.float32)
    return torch.from_numpy(a).to(dtype)


# products over a 40 000-position hub leave the float16 range: mul is run
# for float32 and bfloat16 only
CASES = [(dt, r) for dt in (torch.float32, torch.float16, torch.bfloat16) for r in ("sum", "mean", "mul", "min", "max")
         if not (r == "mul" and dt == torch.float16)]


@pytest.mark.parametrize("dtype,reduce", CASES)
@pytest.mark.parametrize("feat", [1, 16, 33])
@pytest.mark.parametrize("with_out", [False, True])
def test_unsorted_scatter_sort_path(ogn, oracle, dtype, reduce, feat, with_out):
    rng = np.random.default_rng(feat)
    size = 5000
    idx = _index(feat, size)
    src = _src(rng, feat, dtype, reduce in ("min", "max"))
    if reduce == "mul":  # keep products finite and exact-ish: values near 1
        src = torch.from_numpy(rng.choice([0.5, 1.0, 2.0], (N, feat), p=[0.01, 0.98, 0.01]).astype(np.float32)).to(dtype)
    out = torch.from_numpy(rng.integers(-3, 4, (size, feat)).astype(np.float32)).to(dtype) if with_out else None
    fn = {"sum": ogn.scatter_sum, "mean": ogn.scatter_mean, "mul": ogn.scatter_mul, "min": ogn.scatter_min,
          "max": ogn.scatter_max}[reduce]
    dev_idx = torch.from_numpy(idx).cuda()
    for call in range(2):  # the second call reuses the cached sort of the index
        res = fn(src.cuda(), dev_idx, 0, None if out is None else out.clone().cuda(), size)
        got, arg = res if isinstance(res, tuple) else (res, None)
        full = np.broadcast_to(idx.reshape(-1, 1), src.shape)
        want, warg = oracle.scatter(src.float(), full, 0, size, reduce, None if out is None else out.float())
        what = f"{dtype} {reduce} f{feat} out={with_out} call {call}"
        if reduce in ("min", "max"):
            assert_exact(got.float(), want, what + " values")
            assert_exact(arg, warg, what + " arg")
        elif reduce == "mul":
            np.testing.assert_allclose(got.float().cpu().numpy(), want, rtol=1e-2 if dtype != torch.float32 else 1e-5)
        else:
            scale, _ = oracle.scatter(src.float().abs(), full, 0, size, reduce,
                                      None if out is None else out.float().abs())
            assert_sum_close(got, want, scale, dtype, what)


def test_gather_reduce_c_abi_arg_is_src_row(ogn):
    # max through the C ABI with an explicit permutation: arg reports src rows
    from ops_gnn import _lib, _native

    rng = np.random.default_rng(5)
    size, k = 300, 8
    idx = torch.from_numpy(rng.integers(0, size, N)).cuda()
    src = torch.from_numpy(rng.integers(-2, 3, (N, k)).astype(np.float32)).cuda()
    ptr, perm = _native.sorted_layout(idx, size, idx)
    out = torch.empty((size, k), device="cuda")
    arg = _native.segment_reduce_gather(ptr, perm, src, size, _lib.R_MAX, out, False, True)
    # every winner's src row holds the value and belongs to the output row
    rows = torch.arange(size, device="cuda").unsqueeze(1).expand(size, k)
    feat = torch.arange(k, device="cuda").expand(size, k)
    hit = arg < N
    assert bool(hit.all())
    assert torch.equal(src[arg, feat], out)
    assert torch.equal(idx[arg], rows)
    # later tie: the last position of the row holding the maximum
    s = src.cpu().numpy()
    ix = idx.cpu().numpy()
    a = arg.cpu().numpy()
    for r in (0, 7, size - 1):
        pos = np.nonzero(ix == r)[0]
        for f in range(k):
            best = s[pos, f].max()
            assert a[r, f] == pos[s[pos, f] == best][-1]


# ----------------------------------------------------------------- grouped softmax family, unsorted index
SOFT_TOL = {torch.float32: 1e-5, torch.float16: 2e-2, torch.bfloat16: 4e-2}  # reference grouped_softmax_golden.py:24-28


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("mode", ["softmax", "log_softmax", "logsumexp"])
@pytest.mark.parametrize("feat", [1, 32, 33])
def test_unsorted_grouped_softmax_sort_path(ogn, oracle, dtype, mode, feat):
    # statistics through the sort permutation (ogn_segment_group_stats_gather):
    # hub groups, an empty group, +inf / NaN inside a hub group
    from _util import cast_like

    rng = np.random.default_rng(feat)
    groups = 3000
    idx = _index(feat + 1, groups)
    src = torch.from_numpy((rng.standard_normal((N, feat)) * 4).astype(np.float32))
    hub = np.nonzero(idx == 7)[0]
    src[hub[10], 0] = float("inf")
    src[hub[20], -1] = float("nan")
    src = src.to(dtype)
    fn = {"softmax": ogn.scatter_softmax, "log_softmax": ogn.scatter_log_softmax,
          "logsumexp": ogn.scatter_logsumexp}[mode]
    dev_idx = torch.from_numpy(idx).cuda()
    gold = cast_like(oracle.group_softmax(src, torch.from_numpy(idx), 0, groups, mode), dtype)
    for call in range(2):  # the second call reuses the cached sort
        got = fn(src.cuda(), dev_idx, 0, groups).float().cpu().numpy()
        np.testing.assert_array_equal(np.isnan(got), np.isnan(gold))
        tol = SOFT_TOL[dtype]
        np.testing.assert_allclose(got, gold, rtol=tol, atol=tol, equal_nan=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode", ["softmax", "log_softmax", "logsumexp"])
@pytest.mark.parametrize("feat", [1, 32])
def test_unsorted_grouped_softmax_backward_sort_path(ogn, oracle, dtype, mode, feat):
    # the backward's group sums through the sort permutation
    # (ogn_group_bwd_messages + ogn_segment_reduce_gather, then the
    # elementwise pass) against the float64 oracle gradient
    rng = np.random.default_rng(40 + feat)
    groups = 2000
    idx = _index(feat + 3, groups)
    src = torch.from_numpy((rng.standard_normal((N, feat)) * 3).astype(np.float32)).to(dtype)
    fn = {"softmax": ogn.scatter_softmax, "log_softmax": ogn.scatter_log_softmax,
          "logsumexp": ogn.scatter_logsumexp}[mode]
    x = src.cuda().requires_grad_(True)
    out = fn(x, torch.from_numpy(idx).cuda(), 0, groups)
    grad = torch.from_numpy(rng.standard_normal(tuple(out.shape)).astype(np.float32)).to(dtype)
    out.backward(grad.cuda())
    want = oracle.group_softmax_backward(src, grad, torch.from_numpy(idx), 0, groups, mode)
    tol = 1e-4 if dtype == torch.float32 else 5e-2
    scale = np.abs(want).max() + 1.0
    np.testing.assert_allclose(x.grad.float().cpu().numpy() / scale, want / scale, rtol=0, atol=tol)
