"""Benchmark of the ops-gnn hot path on one MI355X.

Headline (BASELINE.json metric): power-law CSR SpMM sum at K=128, fp32
(configuration 3: 2.45 M rows/cols, Zipf(2.1) degrees capped at 20 000,
rescaled to 62 M edges, uniform sorted columns, values U[0,1), B N(0,1)).
A "step" is one ``ops_gnn.csr_spmm(rowptr, col, value, B, "sum")`` over the
whole graph with every input resident in HBM.

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--dtype f32|bf16]

Prints ONE JSON line.  `value` is effective HBM GB/s: the algorithmic bytes
of one step (rowptr + col + value + one B-row gather per edge + C) divided by
the measured step time.  `roofline` reports the dominant kernel (spmm_main)
timed with HIP events inside the library; `cpu_baseline` times the C/OpenMP
oracle on a bounded slice of the same graph on the host cores.
"""

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "ops-gnn_amd"))
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
TRAFFIC_FILE = ROOT / "profiles" / "spmm_main_powerlaw_k128_{dtype}_traffic.txt"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def spmm_bytes(m, nnz, k, esize, val_esize, out_esize, idx=8):
    """Algorithmic bytes of one SpMM step: rowptr + col + value + B gathers + C."""
    return idx * (m + 1) + idx * nnz + val_esize * nnz + esize * k * nnz + out_esize * k * m


def read_traffic(dtype):
    path = Path(str(TRAFFIC_FILE).format(dtype=dtype))
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def copy_calibration():
    """Three 1 GiB device-to-device copies: known bytes for scaling rocprof's
    FETCH_SIZE / WRITE_SIZE counters in the same process."""
    import torch

    src = torch.empty(1 << 28, dtype=torch.float32, device="cuda:0").fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def _event_ms(fn, reps=5):
    """Mean ms of fn() over `reps` calls after one warm call, HIP events on the current stream."""
    import torch

    fn()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / reps


def _stream_gbs(copy, nbytes=1 << 30):
    """Practical HBM ceilings from the library's streaming kernel
    (ogn_calibrate_stream, 16-byte packets, 8 in flight per thread): a copy
    of `nbytes` (read + write counted) or a read of `nbytes`."""
    import torch

    from ops_gnn import _lib

    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src) if copy else None
    sink = torch.zeros(1, dtype=torch.int32, device="cuda:0")

    def run():
        _lib.check(_lib.lib.ogn_calibrate_stream(_lib.dptr(src), _lib.dptr(dst), nbytes, _lib.dptr(sink),
                                                 _lib.stream_of(src)), "calibrate_stream")
    ms = _event_ms(run)
    del src, dst
    return round((2 if copy else 1) * nbytes / (ms * 1e-3) / 1e9, 1)


def measure_copy_gbs():
    return _stream_gbs(True)


def measure_read_gbs():
    return _stream_gbs(False)


def gather_floor_ms(table, index):
    """Time to read exactly the rows `index` selects from `table` [rows, k]
    and nothing else (ogn_calibrate_gather): the floor of any kernel that
    gathers them."""
    import torch

    from ops_gnn import _lib

    rows = table.shape[0]
    row_bytes = table[0].numel() * table.element_size()
    sink = torch.zeros(1, dtype=torch.int32, device=table.device)

    def run():
        _lib.check(_lib.lib.ogn_calibrate_gather(_lib.dptr(table), rows, row_bytes, _lib.dptr(index), index.numel(),
                                                 _lib.dptr(sink), _lib.stream_of(table)), "calibrate_gather")
    return _event_ms(run)


def torch_sparse_mm_baseline(ptr, col, val, mat, rows):
    """Secondary CPU baseline: torch.sparse.mm (CSR x dense, MKL / ATen) on the
    same prefix of rows, fp32, all host threads."""
    import torch

    e = int(ptr[rows])
    a = torch.sparse_csr_tensor(torch.from_numpy(ptr[: rows + 1].copy()), torch.from_numpy(col[:e].copy()),
                                torch.from_numpy(val[:e].copy()), size=(rows, mat.shape[0]))
    b = torch.from_numpy(mat)
    torch.sparse.mm(a, b)
    t0 = time.perf_counter()
    torch.sparse.mm(a, b)
    dt = time.perf_counter() - t0
    nbytes = spmm_bytes(rows, e, mat.shape[1], 4, 4, 4)
    return {"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "library", "sample": f"torch.sparse.mm (CSR fp32) on rows [0, {rows}) = {e} edges, {dt:.2f} s"}


def cpu_baseline(ptr, col, val, mat, k, budget_s=12.0):
    """Time the oracle (C + OpenMP) on a prefix of rows, growing the sample
    until one run takes >= ~1/4 of the budget; report GB/s of that sample."""
    import numpy as np
    from oracle import oracle

    threads = oracle.threads()
    m = ptr.shape[0] - 1
    rows = max(1, m // 1000)
    while True:
        sp = np.ascontiguousarray(ptr[: rows + 1])
        e = int(sp[-1])
        t0 = time.perf_counter()
        oracle.spmm_csr(sp, col[:e], val[:e], mat, "sum")
        dt = time.perf_counter() - t0
        if dt >= budget_s / 4 or rows >= m:
            break
        rows = min(m, int(rows * max(2.0, (budget_s / 4) / max(dt, 1e-3))))
    nbytes = spmm_bytes(rows, e, k, 4, 4, 8)
    try:
        secondary = torch_sparse_mm_baseline(ptr, col, val, mat, rows)
    except Exception as exc:  # noqa: BLE001 - a missing CPU kernel must not sink the bench
        secondary = {"error": repr(exc)[:200]}
    return {
        "secondary": secondary,
        "value": round(nbytes / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"oracle_spmm_csr (C, OpenMP, fp64 accumulate) on rows [0, {rows}) = {e} edges "
                  f"of the same graph, {dt:.2f} s",
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--dtype", choices=["f32", "bf16"], default="f32")
    ap.add_argument("--reduce", choices=["sum", "max", "min"], default="sum")
    ap.add_argument("--scale", type=float, default=1.0, help="fraction of the config-3 size (testing)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a 1 GiB device copy (rocprof counter calibration)")
    ap.add_argument("--torch-compare", action="store_true",
                    help="also time torch's embedding_bag(sum, per_sample_weights) on the same CSR "
                         "(a library implementation of the same weighted row gather)")
    ap.add_argument("--workload", choices=["spmm", "segment", "gat", "coo", "convert"], default="spmm",
                    help="spmm = config 3 (the headline metric); segment / gat / coo = configs 2 / 4 / 5")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for {args.gpus}); the sparse "
              "hot path has no multi-GPU code here -- see DESIGN.md for how it would shard.",
              file=sys.stderr)
        sys.exit(2)

    if args.workload != "spmm":
        line = {"segment": bench_segment, "gat": bench_gat, "coo": bench_coo,
                "convert": bench_convert}[args.workload](args)
        if args.copy_calibration:
            copy_calibration()

        print(json.dumps(line), flush=True)
        return

    import numpy as np
    import torch

    import ops_gnn
    from ops_gnn import _lib
    from ops_gnn.synthetic import cfg3_powerlaw_spmm

    dev = torch.device("cuda:0")
    m = int(2_450_000 * args.scale)
    nnz = int(62_000_000 * args.scale)
    k = 128
    t0 = time.perf_counter()

    def gpu_sort(keys):
        t = torch.from_numpy(keys).to(dev)
        return torch.sort(t).values.cpu().numpy()

    ptr, col, val, mat = cfg3_powerlaw_spmm(m=m, nnz=nnz, k=k, sort_keys=gpu_sort)
    log(f"bench: generated config-3 graph m={m} nnz={int(ptr[-1])} max_deg={int(np.diff(ptr).max())} "
        f"in {time.perf_counter() - t0:.1f}s")
    tdt = torch.float32 if args.dtype == "f32" else torch.bfloat16
    d_ptr = torch.from_numpy(ptr).to(dev)
    d_col = torch.from_numpy(col).to(dev)
    d_val = torch.from_numpy(val).to(dev).to(tdt)
    d_mat = torch.from_numpy(mat).to(dev).to(tdt)
    nnz = int(ptr[-1])

    def step():
        return ops_gnn.csr_spmm(d_ptr, d_col, d_val, d_mat, args.reduce)

    with torch.no_grad():
        for _ in range(max(args.warmup, 1)):
            step()
        torch.cuda.synchronize()
        t_start = time.perf_counter()
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t_start
        ms = elapsed * 1e3 / args.steps

        # Dominant-kernel timing with HIP events recorded by the library on
        # the launch stream (a second pass, so the headline has no events).
        _lib.timing_enable(True)
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        main_ms, main_n = _lib.timing_query("spmm_main")
        rows_ms, _ = _lib.timing_query("spmm_chunk_rows")
        fix_ms, _ = _lib.timing_query("spmm_fixup")
        _lib.timing_enable(False)

        if args.copy_calibration:
            copy_calibration()
        copy_gbs = measure_copy_gbs()
        read_gbs = measure_read_gbs()
        gather_ms = gather_floor_ms(d_mat, d_col)
        log(f"bench: streaming copy {copy_gbs} GB/s, streaming read {read_gbs} GB/s, gathering the "
            f"{nnz} rows alone {gather_ms:.3f} ms (practical ceilings)")

        torch_ms = None
        if args.torch_compare and args.reduce == "sum":
            offsets = d_ptr[:-1]

            def tstep():
                return torch.nn.functional.embedding_bag(d_col, d_mat, offsets, mode="sum",
                                                         per_sample_weights=d_val)
            ref = tstep()
            torch.cuda.synchronize()
            got = step()
            scale = (got.float() - ref.float()).abs().max().item()
            log(f"bench: torch embedding_bag max |diff| vs csr_spmm = {scale:.3e}")
            for _ in range(2):
                tstep()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(args.steps):
                tstep()
            torch.cuda.synchronize()
            torch_ms = (time.perf_counter() - t0) * 1e3 / args.steps
            log(f"bench: torch embedding_bag {torch_ms:.3f} ms per step")

    esz = 4 if args.dtype == "f32" else 2
    mm = args.reduce in ("min", "max")
    nbytes = spmm_bytes(m, nnz, k, esz, esz, esz) + (8 * m * k if mm else 0)
    gbs = nbytes / (ms * 1e-3) / 1e9
    kernel_ms = main_ms / max(main_n, 1)
    achieved = nbytes / (kernel_ms * 1e-3) / 1e9
    log(f"bench: step {ms:.3f} ms; spmm_main {kernel_ms:.3f} ms, chunk_rows {rows_ms / max(main_n, 1):.3f} ms, "
        f"fixup {fix_ms / max(main_n, 1):.3f} ms per launch")

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(ptr, col, val, mat, k)
        log(f"bench: cpu baseline {cpu}")

    result = {
        "metric": "SpMM effective HBM GB/s (power-law CSR, K=128)",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if args.dtype == "f32" else "bf16",
        "data": "synthetic (seeded PCG64, BASELINE config 3 recipe)",
        "config": {
            "workload": "configs[2]: power-law CSR SpMM " + args.reduce,
            "rows": m, "cols": m, "nnz": nnz, "k": k, "max_degree_cap": 20000,
            "index_dtype": "int64", "reduce": args.reduce,
        },
        "gflops": round(2.0 * nnz * k / (ms * 1e-3) / 1e9, 2),
        "pct_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2),
        "roofline": {
            "bound": "hbm",
            "kernel": "spmm_main",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": read_traffic(args.dtype),
            "algorithmic_bytes_per_launch": nbytes,
            "kernel_ms": round(kernel_ms, 4),
            "copy_ceiling": copy_gbs,
            "read_ceiling": read_gbs,
            # the same rows gathered by ogn_calibrate_gather, nothing else
            # read or written: no SpMM over this graph can take less
            "gather_floor_ms": round(gather_ms, 4),
            "gather_floor_GB/s": round(nnz * k * esz / (gather_ms * 1e-3) / 1e9, 1),
            "kernel_over_gather_floor": round(kernel_ms / gather_ms, 4),
        },
        "cpu_baseline": cpu,
    }
    if torch_ms is not None:
        result["torch_embedding_bag"] = {"ms_per_step": round(torch_ms, 4),
                                         "GB/s": round(nbytes / (torch_ms * 1e-3) / 1e9, 2)}
    print(json.dumps(result), flush=True)



# ---------------------------------------------------------------- configs 2, 4, 5
def _timed(fn, steps, warmup):
    """Mean wall ms of fn() over `steps` calls after `warmup`, synchronised."""
    import torch

    for _ in range(max(warmup, 1)):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def _kernel_ms(fn, steps, names):
    """Average per-call ms of the named library kernels (HIP events on the launch stream)."""
    import torch
    from ops_gnn import _lib

    _lib.timing_enable(True)
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    res = {}
    for n in names:
        ms, cnt = _lib.timing_query(n)
        res[n] = ms / steps if cnt else 0.0
    _lib.timing_enable(False)
    return res


def _line(metric, value, unit, ms, args, dtype, workload, config, ops, roof_kernel, roof_bytes, roof_ms, cpu,
          basis="algorithmic"):
    copy_gbs, read_gbs = measure_copy_gbs(), measure_read_gbs()
    return {
        "metric": metric, "value": round(value, 2), "unit": unit, "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": dtype, "data": "synthetic (seeded PCG64, BASELINE recipe)",
        "config": dict({"workload": workload}, **config), "ops": ops,
        "roofline": {"bound": "hbm", "kernel": roof_kernel, "achieved": round(roof_bytes / roof_ms / 1e6, 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(roof_bytes / roof_ms / 1e6 / HBM_PEAK_GBS, 4), "traffic": None,
                     "algorithmic_bytes_per_launch": roof_bytes, "bytes_basis": basis,
                     "kernel_ms": round(roof_ms, 4), "copy_ceiling": copy_gbs, "read_ceiling": read_gbs},
        "cpu_baseline": cpu,
    }


def _cpu_sample(fn_rows, total_rows, bytes_of, budget_s=8.0):
    """Time fn_rows(r) (the oracle on the first r rows/segments), growing r
    until one run takes ~budget/4; returns (GB/s, rows, seconds)."""
    rows = max(1, total_rows // 1000)
    while True:
        t0 = time.perf_counter()
        fn_rows(rows)
        dt = time.perf_counter() - t0
        if dt >= budget_s / 4 or rows >= total_rows:
            return bytes_of(rows) / dt / 1e9, rows, dt
        rows = min(total_rows, int(rows * max(2.0, (budget_s / 4) / max(dt, 1e-3))))


def bench_segment(args):
    """Config 2: segment_csr sum/mean/max(+arg), segment_max_csr and
    segment_logsumexp over src [1e6, 128] fp32 and 62 500 Poisson(16) segments."""
    import numpy as np
    import torch

    import ops_gnn
    from ops_gnn.synthetic import cfg2_segments

    dev = torch.device("cuda:0")
    src_np, ptr_np = cfg2_segments()
    rows, k = src_np.shape
    segs = ptr_np.shape[0] - 1
    src = torch.from_numpy(src_np).to(dev)
    ptr = torch.from_numpy(ptr_np).to(dev)
    base = 4 * rows * k + 8 * (segs + 1) + 4 * segs * k
    cases = [("sum", lambda: ops_gnn.segment_csr(src, ptr, reduce="sum"), base),
             ("mean", lambda: ops_gnn.segment_csr(src, ptr, reduce="mean"), base),
             ("max", lambda: ops_gnn.segment_max_csr(src, ptr), base + 8 * segs * k),
             ("logsumexp", lambda: ops_gnn.segment_logsumexp(src, ptr), base),
             # the inverse expansion: segment rows back over their positions
             ("gather_csr", lambda: ops_gnn.gather_csr(seg_out, ptr), 4 * segs * k + 8 * (segs + 1) + 4 * rows * k)]
    seg_out = ops_gnn.segment_csr(src, ptr, reduce="sum")
    ops = {}
    with torch.no_grad():
        for name, fn, nbytes in cases:
            ms = _timed(fn, args.steps, args.warmup)
            kname = "gather_csr" if name == "gather_csr" else "segment_main"
            kms = _kernel_ms(fn, args.steps, [kname])[kname]
            ops[name] = {"ms": round(ms, 4), "GB/s": round(nbytes / ms / 1e6, 1), "bytes": nbytes,
                         "kernel_ms": round(kms, 4), "kernel_GB/s": round(nbytes / kms / 1e6, 1) if kms else None}
            log(f"bench segment {name}: {ms:.4f} ms, {nbytes / ms / 1e6:.1f} GB/s ({kname} {kms:.4f} ms)")
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import oracle

        gbs, r, dt = _cpu_sample(
            lambda r: oracle.segment_csr(src_np[: ptr_np[r]], ptr_np[: r + 1], "sum"), segs,
            lambda r: 4 * int(ptr_np[r]) * k + 8 * (r + 1) + 4 * r * k)
        cpu = {"value": round(gbs, 3), "unit": "GB/s", "cores": oracle.threads(), "kind": "port",
               "sample": f"oracle_segment_csr sum (C, OpenMP, fp64 accumulate) on segments [0, {r}) "
                         f"= {int(ptr_np[r])} rows of the same input, {dt:.2f} s"}
    s = ops["sum"]
    return _line("segment_csr sum effective HBM GB/s (config 2)", s["GB/s"], "GB/s", s["ms"], args, "f32",
                 "configs[1]: segment reductions", {"rows": rows, "segments": segs, "k": k}, ops,
                 "segment_main", base, s["kernel_ms"], cpu)


def bench_gat(args):
    """Config 4: one GAT-style layer -- sddmm_csr(dot) of Q[row], K[col];
    scatter_softmax over the edges of each row; SpMM-sum of the weights with V.
    233 000 nodes, 114.6 M edges (lognormal degrees), fp16 features [., 64]."""
    import numpy as np
    import torch

    import ops_gnn
    from ops_gnn.synthetic import cfg4_gat_graph

    dev = torch.device("cuda:0")

    def gpu_sort(keys):
        t = torch.from_numpy(keys).to(dev)
        return torch.sort(t).values.cpu().numpy()

    ptr_np, col_np, q_np, k_np, v_np = cfg4_gat_graph(sort_keys=gpu_sort)
    n, f = q_np.shape
    e = int(ptr_np[-1])
    ptr = torch.from_numpy(ptr_np).to(dev)
    col = torch.from_numpy(col_np).to(dev)
    q = torch.from_numpy(q_np).to(dev).half()
    kk = torch.from_numpy(k_np).to(dev).half()
    v = torch.from_numpy(v_np).to(dev).half()
    row = ops_gnn.ptr2ind(ptr, e)  # graph metadata: row of every edge (not timed)
    log(f"bench gat: n={n} e={e} max_deg={int(np.diff(ptr_np).max())}")
    state = {}

    def sddmm():
        state["s"] = ops_gnn.sddmm_csr(ptr, col, q, kk, "dot")

    def softmax():
        state["a"] = ops_gnn.scatter_softmax(state["s"], row, 0, n)

    def spmm():
        state["o"] = ops_gnn.csr_spmm(ptr, col, state["a"], v, "sum")

    def layer():
        sddmm()
        softmax()
        spmm()

    eff = {"sddmm": 8 * e + 2 * e * f + 2 * e + 2 * n * f + 8 * (n + 1),
           "softmax": 2 * e + 2 * e + 8 * e,
           "spmm": 8 * e + 2 * e + 2 * e * f + 2 * n * f + 8 * (n + 1)}
    comp = {"sddmm": 8 * e + 2 * e + 2 * 2 * n * f + 8 * (n + 1),
            # the sorted-index fused pass reads the cached row pointers, not the index
            "softmax": 2 * e + 2 * e + 8 * (n + 1),
            "spmm": 8 * e + 2 * e + 2 * 2 * n * f + 8 * (n + 1)}
    ops = {}
    with torch.no_grad():
        layer()
        for name, fn in (("sddmm", sddmm), ("softmax", softmax), ("spmm", spmm)):
            ms = _timed(fn, args.steps, args.warmup)
            ops[name] = {"ms": round(ms, 4), "effective_GB/s": round(eff[name] / ms / 1e6, 1),
                         "compulsory_GB/s": round(comp[name] / ms / 1e6, 1)}
            log(f"bench gat {name}: {ms:.4f} ms, effective {eff[name] / ms / 1e6:.1f} GB/s, "
                f"compulsory {comp[name] / ms / 1e6:.1f} GB/s")
        ms = _timed(layer, args.steps, args.warmup)
        km = _kernel_ms(layer, args.steps, ["sddmm_main", "spmm_main", "sddmm_xcd", "spmm_xcd", "spmm_xcd_combine",
                                            "segment_softmax", "group_apply", "segment_stats_main"])
        # the XCD-tiled kernels replace sddmm_main / spmm_main when the graph and table sizes select them
        sddmm_kernel = "sddmm_xcd" if km["sddmm_xcd"] > 0 else "sddmm_main"
        gfloor = gather_floor_ms(kk, col)
        log(f"bench gat: gathering the {e} K rows alone {gfloor:.3f} ms")
    tot_eff = sum(eff.values())
    ops["layer"] = {"ms": round(ms, 4), "kernels_ms": {k2: round(v2, 4) for k2, v2 in km.items()}}
    ops["gather_floor"] = {"ms": round(gfloor, 4), "GB/s": round(2 * e * f / (gfloor * 1e-3) / 1e9, 1),
                           "note": "the e K (or V) rows of 128 B that sddmm (SpMM) gathers, read alone"}
    log(f"bench gat layer: {ms:.4f} ms; kernels {km}")
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import oracle

        qf, kf = q.float().cpu().numpy(), kk.float().cpu().numpy()

        def cpu_rows(r):
            oracle.sddmm(ptr_np[: r + 1], col_np[: ptr_np[r]], qf, kf, "dot")

        gbs, r, dt = _cpu_sample(cpu_rows, n, lambda r: 8 * int(ptr_np[r]) + 2 * int(ptr_np[r]) * f)
        cpu = {"value": round(gbs, 3), "unit": "GB/s", "cores": oracle.threads(), "kind": "port",
               "sample": f"oracle_sddmm dot (C) on rows [0, {r}) = {int(ptr_np[r])} edges, {dt:.2f} s"}
    return _line("GAT layer (sddmm + scatter_softmax + SpMM) effective GB/s (config 4)", tot_eff / ms / 1e6,
                 "GB/s", ms, args, "f16", "configs[3]: GAT-style attention layer",
                 {"nodes": n, "nnz": e, "k": f}, ops, sddmm_kernel, comp["sddmm"], km[sddmm_kernel], cpu,
                 basis="compulsory: col + scores + Q and K read once (the per-edge K-row gathers hit the "
                       "256 MB MALL, since K is 29.8 MB)")


def bench_convert(args):
    """COO -> CSR of config 3's graph (2.45 M rows, 62 M edges, fp32 values)
    given in a random edge order, through the torch_sparse frontend's
    coo_to_csr: the stable sort by row (ogn_sort_rows), the row pointers and
    the column and value permutation."""
    import numpy as np
    import torch

    from ops_gnn import torch_sparse_spmm as tss
    from ops_gnn.convert import ptr2ind_tensor
    from ops_gnn.synthetic import cfg3_powerlaw_spmm

    dev = torch.device("cuda:0")

    def gpu_sort(keys):
        t = torch.from_numpy(keys).to(dev)
        return torch.sort(t).values.cpu().numpy()

    ptr_np, col_np, val_np, _ = cfg3_powerlaw_spmm(sort_keys=gpu_sort, with_mat=False)
    m, e = ptr_np.shape[0] - 1, int(ptr_np[-1])
    ptr = torch.from_numpy(ptr_np).to(dev)
    row = ptr2ind_tensor(ptr, e)
    order = torch.randperm(e, device=dev, generator=torch.Generator(device=dev).manual_seed(3))
    index = torch.stack([row[order], torch.from_numpy(col_np).to(dev)[order]]).contiguous()
    value = torch.from_numpy(val_np).to(dev)[order].contiguous()
    del row, order
    # index and values in (20 B / edge), pointers, columns and values out
    # (8 B / row + 12 B / edge), the permutation kept for the layout cache (8 B / edge)
    nbytes = 40 * e + 8 * (m + 1)
    sort_bytes = 16 * e  # the radix sort proper: 32-bit keys and positions, in and out
    fn = lambda: tss.coo_to_csr(index, value, m)
    with torch.no_grad():
        ms = _timed(fn, args.steps, args.warmup)
        kms = _kernel_ms(fn, args.steps, ["sort_rows_pack", "sort_rows_radix", "sort_rows_unpack"])
    log(f"bench convert: {ms:.4f} ms, {nbytes / ms / 1e6:.1f} GB/s; sort kernels {kms}")
    ops = {"coo_to_csr": {"ms": round(ms, 4), "GB/s": round(nbytes / ms / 1e6, 1), "bytes": nbytes},
           "sort_rows": {k: round(v, 4) for k, v in kms.items()}}
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import oracle

        idx_np = index.cpu().numpy()
        val_h = value.cpu().numpy()

        def convert(r):
            perm = np.argsort(idx_np[0, :r], kind="stable")
            oracle.ind2ptr(idx_np[0, :r][perm], m)
            return idx_np[1, :r][perm], val_h[:r][perm]

        gbs, r, dt = _cpu_sample(convert, e, lambda r: 40 * r + 8 * (m + 1))
        cpu = {"value": round(gbs, 3), "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": f"numpy stable argsort + oracle_ind2ptr (C) + permutation on the first {r} edges "
                         f"of the same COO input, {dt:.2f} s"}
    return _line("COO -> CSR conversion effective GB/s (config 3 graph, random edge order)",
                 nbytes / ms / 1e6, "GB/s", ms, args, "int64", "configs[2] graph: coo_to_csr",
                 {"rows": m, "edges": e}, ops, "sort_rows_radix", sort_bytes, kms["sort_rows_radix"], cpu,
                 basis="32-bit keys and positions in and out of the radix sort")


def bench_coo(args):
    """Config 5: ind2ptr/ptr2ind round trip, scatter sum/mean/max,
    scatter_log_softmax and scatter_logsumexp over a sorted destination index
    (50 M edges, 1 M nodes, Zipf(1.8) in-degree), src [50 M, 32] fp32."""
    import numpy as np
    import torch

    import ops_gnn
    from ops_gnn.synthetic import cfg5_coo_scatter

    dev = torch.device("cuda:0")
    idx_np, src_np = cfg5_coo_scatter()
    e, f = src_np.shape
    nodes = 1_000_000
    index = torch.from_numpy(idx_np).to(dev)
    src = torch.from_numpy(src_np).to(dev)
    ptr = ops_gnn.ind2ptr(index, nodes)
    rt = ops_gnn.ptr2ind(ptr, e)
    assert torch.equal(rt, index), "ind2ptr/ptr2ind round trip differs"
    sb = 4 * e * f + 8 * e + 4 * nodes * f
    # ind2ptr reads what its lower_bound searches touch, not the whole index:
    # about one 64-byte line of the index per output boundary, plus the output
    cases = [("ind2ptr", lambda: ops_gnn.ind2ptr(index, nodes), 64 * (nodes + 1) + 8 * (nodes + 1)),
             ("ptr2ind", lambda: ops_gnn.ptr2ind(ptr, e), 8 * e + 8 * (nodes + 1)),
             ("scatter_sum", lambda: ops_gnn.scatter(src, index, 0, dim_size=nodes, reduce="sum"), sb),
             ("scatter_mean", lambda: ops_gnn.scatter(src, index, 0, dim_size=nodes, reduce="mean"), sb),
             ("scatter_max", lambda: ops_gnn.scatter(src, index, 0, dim_size=nodes, reduce="max"),
              sb + 8 * nodes * f),
             ("scatter_log_softmax", lambda: ops_gnn.scatter_log_softmax(src, index, 0, nodes),
              8 * e * f + 8 * e),
             ("scatter_logsumexp", lambda: ops_gnn.scatter_logsumexp(src, index, 0, nodes), sb),
             # the same edges in a random order: the unsorted path (index sort
             # cached after the first call, then the engine through the permutation)
             ("scatter_sum_unsorted", lambda: ops_gnn.scatter(src_sh, index_sh, 0, dim_size=nodes, reduce="sum"), sb),
             ("scatter_max_unsorted", lambda: ops_gnn.scatter(src_sh, index_sh, 0, dim_size=nodes, reduce="max"),
              sb + 8 * nodes * f)]
    order = torch.randperm(e, device=dev, generator=torch.Generator(device=dev).manual_seed(5))
    index_sh, src_sh = index[order].contiguous(), src[order].contiguous()
    del order
    ops = {}
    with torch.no_grad():
        for name, fn, nbytes in cases:
            ms = _timed(fn, args.steps, args.warmup)
            ops[name] = {"ms": round(ms, 4), "GB/s": round(nbytes / ms / 1e6, 1), "bytes": nbytes}
            log(f"bench coo {name}: {ms:.4f} ms, {nbytes / ms / 1e6:.1f} GB/s")
        kms = _kernel_ms(cases[2][1], args.steps, ["segment_main"])["segment_main"]
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import oracle

        ptr_np = ptr.cpu().numpy()

        def cpu_rows(r):
            oracle.scatter(src_np[: int(ptr_np[r])], idx_np[: ptr_np[r], None], 0, r, "sum")

        gbs, r, dt = _cpu_sample(cpu_rows, nodes, lambda r: 4 * int(ptr_np[r]) * f + 8 * int(ptr_np[r]) + 4 * r * f)
        cpu = {"value": round(gbs, 3), "unit": "GB/s", "cores": oracle.threads(), "kind": "port",
               "sample": f"oracle_scatter sum (C) on nodes [0, {r}) = {int(ptr_np[r])} edges, {dt:.2f} s"}
    s = ops["scatter_sum"]
    return _line("scatter sum (sorted COO) effective HBM GB/s (config 5)", s["GB/s"], "GB/s", s["ms"], args, "f32",
                 "configs[4]: COO scatter path", {"edges": e, "nodes": nodes, "k": f}, ops, "segment_main", sb,
                 kms, cpu)

if __name__ == "__main__":
    main()
