"""Parity at the BASELINE configurations' full sizes.

The oracle checks sampled rows (hub rows and random rows) exactly as in the
small tests. Whole outputs are checked through properties that do not
depend on size:

- SpMM sum is linear. C·w must equal A·(B·w) for a random w. The right side
  is computed in fp64 with torch's index_add_, an independent reduction.
- SpMM max: every output equals val[arg]·B[col[arg]] exactly, and no edge of
  the row exceeds it. arg is the first edge attaining it; this is checked
  against a torch scatter_reduce(amin) over all 7.9 G edge-feature products.
- segment_csr (config 2): the full output is compared with the oracle.
- SpMM min is checked like max; bf16 sum by linearity at 1e-2 and sampled
  rows against the oracle on the same bf16 inputs.
- scatter (config 5): sum / mean / max at sampled nodes (hubs included)
  against the oracle, plus per-feature totals; scatter_log_softmax and
  scatter_logsumexp at sampled nodes against the oracle, and exp(log_softmax)
  summing to 1 in every group.
- GAT layer (config 4): sampled edges of the sddmm are compared with fp64
  dots; every softmax group must sum to 1, and the softmax of sampled rows
  (hubs included) is compared edge by edge with the oracle; sampled rows of
  the SpMM are compared with the oracle.

Tolerances as elsewhere: sums |a - g| <= rtol * sum|terms| (rtol 1e-5 fp32,
1e-2 fp16); extrema and args bit-exact.
"""

import numpy as np
import pytest
import torch

from _util import assert_exact, assert_sum_close

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _gpu_sort(keys):
    return torch.sort(torch.from_numpy(keys).to(DEV)).values.cpu().numpy()


@pytest.fixture(scope="module")
def cfg3():
    from ops_gnn.synthetic import cfg3_powerlaw_spmm

    ptr, col, val, mat = cfg3_powerlaw_spmm(sort_keys=_gpu_sort)
    d = {"ptr": torch.from_numpy(ptr).to(DEV), "col": torch.from_numpy(col).to(DEV),
         "val": torch.from_numpy(val).to(DEV), "mat": torch.from_numpy(mat).to(DEV)}
    return (ptr, col, val, mat), d


def _sample_rows(ptr, rng, hubs=48, rand=400):
    deg = np.diff(ptr)
    top = np.argsort(deg)[-hubs:]
    pick = np.unique(np.concatenate([top, rng.integers(0, deg.size, rand), [0, deg.size - 1]]))
    return pick


def _sub_csr(ptr, col, val, rows):
    parts_c, parts_v, sub = [], [], [0]
    for r in rows:
        a, b = ptr[r], ptr[r + 1]
        parts_c.append(col[a:b])
        parts_v.append(val[a:b])
        sub.append(sub[-1] + (b - a))
    return np.array(sub, np.int64), np.concatenate(parts_c), np.concatenate(parts_v)


def test_config3_spmm_sum_full_size(ogn, oracle, cfg3):
    (ptr, col, val, mat), d = cfg3
    out = ogn.csr_spmm(d["ptr"], d["col"], d["val"], d["mat"], "sum")
    # sampled rows against the oracle
    rows = _sample_rows(ptr, np.random.default_rng(31))
    sp, sc, sv = _sub_csr(ptr, col, val, rows)
    gold, _ = oracle.spmm_csr(sp, sc, sv, mat, "sum")
    scale, _ = oracle.spmm_csr(sp, sc, np.abs(sv), np.abs(mat), "sum")
    assert_sum_close(out[torch.from_numpy(rows).to(DEV)], gold, scale, torch.float32, "config-3 sampled rows")
    # linearity over every row: C w == A (B w), fp64 reference via index_add_
    w = torch.randn(mat.shape[1], dtype=torch.float64, device=DEV, generator=torch.Generator(DEV).manual_seed(5))
    m = ptr.size - 1
    row_of = torch.repeat_interleave(torch.arange(m, device=DEV), d["ptr"][1:] - d["ptr"][:-1])
    bw = d["mat"].double() @ w
    babs = d["mat"].double().abs() @ w.abs()
    ref = torch.zeros(m, dtype=torch.float64, device=DEV).index_add_(0, row_of, d["val"].double() * bw[d["col"]])
    bound = torch.zeros(m, dtype=torch.float64, device=DEV).index_add_(
        0, row_of, d["val"].double().abs() * babs[d["col"]])
    got = out.double() @ w
    err = (got - ref).abs() - (1e-5 * bound + 1e-6)
    assert float(err.max()) <= 0, f"config-3 C w differs from A (B w): worst excess {float(err.max()):.3e}"


@pytest.mark.parametrize("reduce", ["max", "min"])
def test_config3_spmm_extremum_full_size(ogn, oracle, cfg3, reduce):
    (ptr, col, val, mat), d = cfg3
    vals, arg = ogn.csr_spmm(d["ptr"], d["col"], d["val"], d["mat"], reduce)
    m, k = vals.shape
    e = col.size
    deg = d["ptr"][1:] - d["ptr"][:-1]
    empty = deg == 0
    # arg inside its row (or E for an empty row)
    lo = d["ptr"][:-1].unsqueeze(1)
    hi = d["ptr"][1:].unsqueeze(1)
    ok = ((arg >= lo) & (arg < hi)) | (empty.unsqueeze(1) & (arg == e))
    assert bool(ok.all()), f"config-3 {reduce} arg outside its row"
    # value attained by arg, exactly: the kernel compares exact fp64 products
    # and rounds the winner once
    a = arg.clamp(max=e - 1)
    best64 = d["val"].double()[a] * d["mat"].double()[d["col"][a], torch.arange(k, device=DEV)]
    attained = best64.float()
    attained[empty] = 0
    assert torch.equal(attained, vals), f"config-3 {reduce} value not val[arg] * B[col[arg]]"
    # extremal over all edges, first edge among ties: amin of attaining edge ids
    row_of = torch.repeat_interleave(torch.arange(m, device=DEV), deg)
    first = torch.full((m, k), e, dtype=torch.int64, device=DEV)
    step = 1 << 22
    for s in range(0, e, step):
        sl = slice(s, min(s + step, e))
        prod = d["val"][sl].double().unsqueeze(1) * d["mat"][d["col"][sl]].double()
        best = best64[row_of[sl]]
        beyond = prod > best if reduce == "max" else prod < best
        assert not bool(beyond.any()), f"config-3 an edge beats the {reduce}"
        ids = torch.arange(s, sl.stop, device=DEV).unsqueeze(1).expand(-1, k)
        cand = torch.where(prod == best, ids, torch.full_like(ids, e))
        first.scatter_reduce_(0, row_of[sl].unsqueeze(1).expand(-1, k), cand, "amin")
        del prod, best, ids, cand, beyond
    assert torch.equal(first, arg), f"config-3 {reduce} arg is not the first extremal edge"
    # sampled rows against the oracle, bit-exact
    rows = _sample_rows(ptr, np.random.default_rng(32), hubs=16, rand=200)
    sp, sc, sv = _sub_csr(ptr, col, val, rows)
    gold, garg = oracle.spmm_csr(sp, sc, sv, mat, reduce)
    assert_exact(vals[torch.from_numpy(rows).to(DEV)], gold.astype(np.float32), f"config-3 sampled {reduce} values")
    base = ptr[rows][:, None]
    sub_base = sp[:-1][:, None]
    expect_arg = np.where(garg == sc.size, e, garg - sub_base + base)
    assert_exact(arg[torch.from_numpy(rows).to(DEV)], expect_arg, f"config-3 sampled {reduce} args")


def test_config3_spmm_sum_bf16_full_size(ogn, oracle, cfg3):
    """Config 3 in bf16 (values cast to bf16 like the mat): linearity over
    every row at the bf16 tolerance 1e-2, and sampled hub / random rows
    against the oracle on the same bf16 inputs."""
    (ptr, col, val, mat), d = cfg3
    vb, mb = d["val"].bfloat16(), d["mat"].bfloat16()
    out = ogn.csr_spmm(d["ptr"], d["col"], vb, mb, "sum")
    assert out.dtype == torch.bfloat16
    rows = _sample_rows(ptr, np.random.default_rng(35))
    sp, sc, _ = _sub_csr(ptr, col, val, rows)
    sel = torch.from_numpy(np.concatenate([np.arange(ptr[r], ptr[r + 1]) for r in rows])).to(DEV)
    sv = vb[sel].float().cpu().numpy()
    mf = mb.float().cpu().numpy()
    gold, _ = oracle.spmm_csr(sp, sc, sv, mf, "sum")
    scale, _ = oracle.spmm_csr(sp, sc, np.abs(sv), np.abs(mf), "sum")
    assert_sum_close(out[torch.from_numpy(rows).to(DEV)], gold, scale, torch.bfloat16, "config-3 bf16 sampled rows")
    w = torch.randn(mat.shape[1], dtype=torch.float64, device=DEV, generator=torch.Generator(DEV).manual_seed(6))
    m = ptr.size - 1
    row_of = torch.repeat_interleave(torch.arange(m, device=DEV), d["ptr"][1:] - d["ptr"][:-1])
    bw = mb.double() @ w
    babs = mb.double().abs() @ w.abs()
    ref = torch.zeros(m, dtype=torch.float64, device=DEV).index_add_(0, row_of, vb.double() * bw[d["col"]])
    bound = torch.zeros(m, dtype=torch.float64, device=DEV).index_add_(0, row_of, vb.double().abs() * babs[d["col"]])
    # the output rounds each element to bf16 once: |C - C_exact| <= 2^-8 |C|
    got = out.double() @ w
    round_bound = (out.double().abs() @ w.abs()) * 2.0 ** -8
    err = (got - ref).abs() - (1e-2 * bound + round_bound + 1e-3)
    assert float(err.max()) <= 0, f"config-3 bf16 C w differs from A (B w): worst excess {float(err.max()):.3e}"


def test_config3_coo_to_csr_full_size(ogn, cfg3):
    # config 3's 62 M edges in random order back to CSR through the
    # torch_sparse frontend: row pointers equal the original, and the columns
    # and values come out in the order of a stable argsort of the rows
    # (the reference's, python/ops_gnn/torch_sparse_spmm.py:273-342), bit for bit
    from ops_gnn import torch_sparse_spmm as tss
    from ops_gnn.convert import ptr2ind_tensor

    _, d = cfg3
    ptr, col, val = d["ptr"], d["col"], d["val"]
    e, m = col.numel(), ptr.numel() - 1
    order = torch.randperm(e, device=DEV, generator=torch.Generator(device=DEV).manual_seed(11))
    row = ptr2ind_tensor(ptr, e)
    index = torch.stack([row[order], col[order]]).contiguous()
    value = val[order].contiguous()
    del row
    got_ptr, got_col, got_val = tss.coo_to_csr(index, value, m)
    assert torch.equal(got_ptr, ptr)
    perm = torch.sort(index[0], stable=True)[1]
    assert torch.equal(got_col, index[1][perm])
    assert torch.equal(got_val, value[perm])


def test_config2_segment_full_size(ogn, oracle):
    from ops_gnn.synthetic import cfg2_segments

    src, ptr = cfg2_segments()
    s, p = torch.from_numpy(src).to(DEV), torch.from_numpy(ptr).to(DEV)
    for reduce in ("sum", "mean"):
        got = ogn.segment_csr(s, p, reduce=reduce)
        gold, _ = oracle.segment_csr(src, ptr, reduce)
        scale, _ = oracle.segment_csr(np.abs(src), ptr, reduce)
        assert_sum_close(got, gold, scale, torch.float32, f"config-2 {reduce}")
    vals, arg = ogn.segment_max_csr(s, p)
    gold, garg = oracle.segment_csr(src, ptr, "max")
    assert_exact(vals, gold.astype(np.float32), "config-2 max values")
    assert_exact(arg, garg, "config-2 max args")
    lse = ogn.segment_logsumexp(s, p)
    gold = oracle.segment_logsumexp(src, ptr)
    np.testing.assert_allclose(lse.cpu().numpy(), gold, rtol=1e-5, atol=1e-5)


@pytest.fixture(scope="module")
def cfg5():
    from ops_gnn.synthetic import cfg5_coo_scatter

    idx, src = cfg5_coo_scatter()
    return idx, src, torch.from_numpy(idx).to(DEV), torch.from_numpy(src).to(DEV)


def _cfg5_nodes(ptr_np, nodes, seed):
    rng = np.random.default_rng(seed)
    deg = np.diff(ptr_np)
    return np.unique(np.concatenate([np.argsort(deg)[-8:], rng.integers(0, nodes, 300), [0, nodes - 1]]))


def test_config5_scatter_full_size(ogn, oracle, cfg5):
    idx, src, index, s = cfg5
    nodes = 1_000_000
    ptr = ogn.ind2ptr(index, nodes)
    assert torch.equal(ogn.ptr2ind(ptr, idx.size), index), "config-5 ind2ptr / ptr2ind round trip"
    ptr_np = ptr.cpu().numpy()
    nodes_pick = _cfg5_nodes(ptr_np, nodes, 33)
    for reduce in ("sum", "mean", "max"):
        res = ogn.scatter(s, index, 0, dim_size=nodes, reduce=reduce)
        got, arg = (res, None) if reduce != "max" else ogn.scatter_max(s, index, 0, None, nodes)
        for n in nodes_pick:
            a, b = ptr_np[n], ptr_np[n + 1]
            sub = src[a:b]
            if reduce != "max":
                gv, _ = oracle.scatter(sub, np.zeros((b - a, 1), np.int64), 0, 1, reduce)
                sv, _ = oracle.scatter(np.abs(sub), np.zeros((b - a, 1), np.int64), 0, 1, reduce)
                assert_sum_close(got[n:n + 1], gv, sv, torch.float32, f"config-5 {reduce} node {n}")
            else:
                gv, ga = oracle.scatter(sub, np.zeros((b - a, 1), np.int64), 0, 1, "max")
                assert_exact(got[n:n + 1], gv.astype(np.float32), f"config-5 max node {n}")
                want = np.where(ga == (b - a), idx.size, ga + a)
                assert_exact(arg[n:n + 1], want, f"config-5 max arg node {n}")
        if reduce == "sum":
            tot = got.double().sum(0)
            ref = s.double().sum(0)
            bound = 1e-5 * s.double().abs().sum(0) + 1e-6
            assert bool(((tot - ref).abs() <= bound).all()), "config-5 per-feature totals"
        if reduce == "mean":
            deg = torch.from_numpy(np.diff(ptr_np)).to(DEV).double().unsqueeze(1)
            tot = (got.double() * deg).sum(0)
            ref = s.double().sum(0)
            bound = 1e-5 * s.double().abs().sum(0) + 1e-4
            assert bool(((tot - ref).abs() <= bound).all()), "config-5 mean x degree totals"
        del res, got, arg


@pytest.mark.parametrize("mode", ["log_softmax", "logsumexp"])
def test_config5_grouped_full_size(ogn, oracle, cfg5, mode):
    """scatter_log_softmax / scatter_logsumexp at 50 M x 32: sampled nodes
    (the 8 largest hubs included) against the oracle at 1e-5, and, over all
    rows, exp(log_softmax) summing to 1 per (node, feature)."""
    idx, src, index, s = cfg5
    nodes = 1_000_000
    ptr_np = ogn.ind2ptr(index, nodes).cpu().numpy()
    fn = ogn.scatter_log_softmax if mode == "log_softmax" else ogn.scatter_logsumexp
    got = fn(s, index, 0, nodes)
    for n in _cfg5_nodes(ptr_np, nodes, 36):
        a, b = ptr_np[n], ptr_np[n + 1]
        gold = oracle.group_softmax(src[a:b], np.zeros(b - a, np.int64), 0, 1, mode)
        part = got[a:b] if mode == "log_softmax" else got[n:n + 1]
        g = part.cpu().numpy()
        if b == a and mode == "logsumexp":
            assert np.isneginf(g).all(), f"config-5 logsumexp empty node {n}"
            continue
        np.testing.assert_allclose(g, gold, rtol=1e-5, atol=1e-5, err_msg=f"config-5 {mode} node {n}")
    if mode == "log_softmax":
        sums = torch.zeros((nodes, s.shape[1]), dtype=torch.float64, device=DEV).index_add_(0, index, got.double().exp())
        nonempty = torch.from_numpy(np.diff(ptr_np) > 0).to(DEV)
        assert bool(((sums[nonempty] - 1).abs() <= 1e-4).all()), "config-5 exp(log_softmax) group sums"


def test_config4_gat_layer_full_size(ogn, oracle):
    from ops_gnn.synthetic import cfg4_gat_graph

    ptr, col, q, k, v = cfg4_gat_graph(sort_keys=_gpu_sort)
    n, f = q.shape
    e = col.size
    dp, dc = torch.from_numpy(ptr).to(DEV), torch.from_numpy(col).to(DEV)
    dq, dk, dv = (torch.from_numpy(a).to(DEV).half() for a in (q, k, v))
    scores = ogn.sddmm_csr(dp, dc, dq, dk, "dot")
    rng = np.random.default_rng(34)
    eids = np.unique(np.concatenate([rng.integers(0, e, 4000), [0, e - 1]]))
    row_of = np.searchsorted(ptr, eids, side="right") - 1
    qh, kh = dq.float().cpu().numpy(), dk.float().cpu().numpy()
    gold = (qh[row_of].astype(np.float64) * kh[col[eids]].astype(np.float64)).sum(1)
    got = scores[torch.from_numpy(eids).to(DEV)].float().cpu().numpy()
    scale = (np.abs(qh[row_of]) * np.abs(kh[col[eids]])).sum(1)
    assert (np.abs(got - gold) <= 1e-2 * scale + 1e-2 * np.abs(gold) + 1e-3).all(), "config-4 sampled sddmm"
    row = ogn.ptr2ind(dp, e)
    att = ogn.scatter_softmax(scores, row, 0, n)
    sums = torch.zeros(n, dtype=torch.float64, device=DEV).index_add_(0, row, att.double())
    nonempty = (dp[1:] - dp[:-1]) > 0
    assert torch.allclose(sums[nonempty], torch.ones_like(sums[nonempty]), atol=2e-2), "config-4 softmax sums"
    # sampled rows (hubs included), every edge against the oracle's grouped
    # softmax of the same fp16 scores, fp16 tolerance 1e-2
    rows = _sample_rows(ptr, rng, hubs=8, rand=200)
    sc_all = scores.float().cpu().numpy()
    att_all = att.float().cpu().numpy()
    for r in rows:
        a, b = ptr[r], ptr[r + 1]
        if a == b:
            continue
        gold = oracle.group_softmax(sc_all[a:b], np.zeros(b - a, np.int64), 0, 1, "softmax")
        gold = torch.from_numpy(gold).half().float().numpy()
        np.testing.assert_allclose(att_all[a:b], gold, rtol=1e-2, atol=1e-2, err_msg=f"config-4 softmax row {r}")
    out = ogn.csr_spmm(dp, dc, att, dv, "sum")
    sp, sc, sa = _sub_csr(ptr, col, att.float().cpu().numpy(), rows)
    gold, _ = oracle.spmm_csr(sp, sc, sa, dv.float().cpu().numpy(), "sum")
    scale, _ = oracle.spmm_csr(sp, sc, np.abs(sa), np.abs(dv.float().cpu().numpy()), "sum")
    assert_sum_close(out[torch.from_numpy(rows).to(DEV)], gold, scale, torch.float16, "config-4 sampled spmm")
