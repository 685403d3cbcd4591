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
    return {
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
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for {args.gpus}); the sparse "
              "hot path has no multi-GPU code here -- see DESIGN.md for how it would shard.",
              file=sys.stderr)
        sys.exit(2)

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
            src = torch.empty(1 << 28, dtype=torch.float32, device=dev).fill_(1.0)
            dst = torch.empty_like(src)
            for _ in range(3):
                dst.copy_(src)
            torch.cuda.synchronize()
            del src, dst

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
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
