"""Benchmark of the per-matrix quantization hot path on one MI355X.

A step is one pass of the hot path over one matrix of the workload: the input rotation X = W R_in^T with the row
scales S, the Hessian rotation R_in H R_in^T, the damped Cholesky-inverse U, the block-LDLQ sweep with the row
trellis (fused Viterbi + in-block refit kernel per 128-column block, fp64 MFMA trailing update between blocks) and
the packed codes. W and H are resident in HBM when the timed region starts (the calibration capture that produces
H is not part of a step).

    python bench.py [--steps K] [--warmup W] [--L 16|12] [--k 2] [--no-cpu]

The default is the benchmark configuration (config 2: 16-bit states, the fp16 quantile table); --L 12 runs the
reference's own production trellis (the fitted 12-bit tables).

Prints one JSON line: weights quantized per second (metric value), Viterbi rows/s, the roofline of the dominant
kernel (the fused trellis block kernel) measured with HIP events on its stream, and the CPU oracle timed on a
bounded row sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

METRIC = "weights quantized/sec (LDLQ+trellis) & Viterbi rows/sec; % MFMA/HBM roofline"
VALU_PEAK_TOPS = 256 * 4 * 16 * 2.4e9 / 1e12  # one non-packed fp32 VALU op per lane per clock at 2.4 GHz: 39.3 TOP/s


def viterbi_ops_per_row_step(L: int, k: int) -> int:
    """Algorithmic fp32 operations of one trellis step of one row: a subtraction, a square and an addition per state,
    and 2^k - 1 comparisons per group of 2^k predecessors."""
    return 3 * (1 << L) + ((1 << k) - 1) * (1 << (L - k))


def row_steps(n: int, width: int, look: int, lazy: int) -> list[int]:
    """Trellis positions searched per row in each lazy block (settled plus look-ahead columns of every call)."""
    out = []
    for b0 in range(0, n, lazy):
        b1 = min(b0 + lazy, n)
        tot = 0
        for j in range(b0, b1, width):
            w = min(width, b1 - j)
            tot += w + min(look, n - j - w)
        out.append(tot)
    return out


def cpu_baseline(W, H, table, L, k, in_seed, budget_s=12.0):
    """The C oracle (one core, BLAS limited to one thread) on the same workload: the rotation, Hessian rotation and
    factorization in full, the sweep on as many rows as fit in the budget, extrapolated by rows (rows are
    independent given U and S)."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import oracle as O

    m, n = W.shape
    with threadpool_limits(limits=1):
        t0 = time.perf_counter()
        R = O.rht(n, in_seed)
        X = np.asarray(W, dtype=np.float64) @ R.T
        S = O.row_scale(X)
        Hr = R @ H @ R.T
        _, U, dead = O.environment(Hr)
        t_fixed = time.perf_counter() - t0
        rows, t_rows = 0, 0.0
        chunk = 8
        while rows < m and t_rows < budget_s:
            r1 = min(rows + chunk, m)
            t1 = time.perf_counter()
            O.ldlq_trellis(X[rows:r1], U, S[rows:r1], table, L, k, dead=dead if dead.any() else None)
            t_rows += time.perf_counter() - t1
            rows = r1
    per_row = t_rows / rows
    total = t_fixed + per_row * m
    return {"value": m * n / total, "unit": "weights/s", "cores": 1, "kind": "port",
            "sample": f"C oracle: rotation, R H R^T and U (numpy LAPACK, 1 thread) in full ({t_fixed:.2f} s); "
                      f"sweep on the first {rows} of {m} rows ({t_rows:.2f} s), extrapolated by rows",
            "seconds_total_extrapolated": round(total, 3)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--L", type=int, default=16)
    ap.add_argument("--k", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the per-matrix hot path runs on one MI355X here (rows would shard across "
              "GPUs with no communication; see DESIGN.md). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from lookatmyquant_amd import engine as E
    from lookatmyquant_amd import synthetic
    from lookatmyquant_amd.tables import load_table, quantile_table

    torch.cuda.set_device(0)
    L, k = args.L, args.k
    width, look, lazy = 16, 8, 128
    in_seed = 201  # quantize.py:1492-1493 for layer 0's self_attn.q_proj
    W, H = synthetic.config12()
    table = load_table(12, k) if L == 12 else quantile_table(L, 0)
    m, n = W.shape
    dev = torch.device("cuda", 0)
    Wg = torch.from_numpy(W.astype(np.float64)).to(dev)
    Hg = torch.from_numpy(H).to(dev)
    tab64 = torch.from_numpy(np.array(table)).to(dev)
    tab32 = E.half_bits(tab64) if L >= E.BIG_L else tab64.to(torch.float32)

    def step(events=None):
        X, S = E.rht_rows(Wg, in_seed, want_rms=True)
        Hr = E.rotate_hessian(Hg, in_seed)
        _, U, dead, info = E.chol_inv_upper(Hr, raise_on_fail=False)
        st = E.ldlq_trellis(X, S, U, tab64, L, k, width, look, lazy, dead=dead, table32=tab32, events=events)
        codes, bad = E.pack_trellis(st, k, L, check_paths=False)
        return st, codes, info, bad

    for _ in range(args.warmup):
        st, codes, info, bad = step()
    torch.cuda.synchronize()
    assert int(info.item()) == 0 and int(bad.item()) == 0

    events: dict = {}
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        st, codes, info, bad = step(events)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms = (t1 - t0) * 1e3 / args.steps

    # the dominant kernel: the fused trellis block (search + in-block refit)
    blk = E.event_ms(events, "block")
    trl = E.event_ms(events, "trailing")
    per_block = row_steps(n, width, look, lazy)
    ops_step = m * sum(per_block) * viterbi_ops_per_row_step(L, k)
    blk_ms_step = sum(blk) / args.steps
    achieved = ops_step / (blk_ms_step * 1e-3) / 1e12
    value = m * n / (ms * 1e-3)
    rows_per_s = m / (ms * 1e-3)
    out = {
        "metric": METRIC, "value": round(value, 1), "unit": "weights/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f64/f32", "data": "synthetic",
        "config": {"workload": f"config 2: one 960x960 q_proj, row-trellis block LDLQ k={k} L={L} (width 16, look 8, lazy 128), "
                               "H from 16384 bf16 tokens, rotation + factor + sweep + packed codes per step",
                   "rows": m, "columns": n, "L": L, "k": k,
                   "table": "reference e-means L=12 table" if L == 12 else f"fp16 Gaussian quantiles, 2^{L} entries"},
        "viterbi_rows_per_s": round(rows_per_s, 1),
        "viterbi_row_steps_per_s": round(m * sum(per_block) / (ms * 1e-3), 1),
        "roofline": {"kernel": "ldlq_trellis_block_big_kernel" if L >= E.BIG_L else "ldlq_trellis_block_kernel", "bound": "valu", "achieved": round(achieved, 3),
                     "peak": round(VALU_PEAK_TOPS, 1), "unit": "TOP/s", "frac": round(achieved / VALU_PEAK_TOPS, 4),
                     "traffic": None, "launches_per_step": len(per_block),
                     "avg_launch_us": round(1e3 * sum(blk) / len(blk), 2),
                     "ops_per_row_step": viterbi_ops_per_row_step(L, k)},
        "phase_ms": {"block_kernels": round(blk_ms_step, 4), "trailing_updates": round(sum(trl) / args.steps, 4)},
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(W, H, table, L, k, in_seed)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
