"""Benchmark of the per-matrix quantization hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--L 16|12] [--no-cpu] [--workload c5|c1|c2|c3|c4|l2] [--copy-probe MiB]

The default workload is config 5, the build of a random-initialised Qwen3.5-4B-shaped stack (36 layers x 7 linears:
q/k/v/o [4096|1024|1024 x 2560, 2560 x 4096], gate/up [9728 x 2560], down [2560 x 9728]), and a step is one decoder
layer of that build: both calibration streams (32 x 2048 token ids) through the layer, per stage the Hessian with digit
token weights and the QEP cross-Gram, the QEP targets at alpha 0.5, the stage factor, the row-plan trellis sweeps
(bits 1-4, 2.3 bpw; width 16, look 8, lazy 128) and the packed codes. Every layer has the same shapes, so the 36-layer
build takes 36 steps; the line reports that build's seconds (36 x the per-step time) beside the north star's 3-minute
target. The trellis has 16-bit states by default (the fp16 Gaussian-quantile table of 2^16 entries); --L 12 runs the
reference's own production trellis (its four fitted 12-bit tables), whose per-layer time the default line also
reports from a few extra layers.

In the timed layers every kernel runs on one stream, each launch between HIP events on that stream, so that each
kernel's average launch duration is measured over the timed region; the line's "kernels" gives each kernel's
achieved rate and fraction of the published MI355X peak (bf16 MFMA 2.5 PFLOP/s, fp64 MFMA 78.6 TFLOP/s, fp32 vector
157.3 TFLOP/s, HBM 8 TB/s), and "roofline" the dominant kernel's (the trellis search). The production schedule (each
stage's bit widths swept on streams of their own, the stage factor next to the QEP targets) is timed on extra layers
after the timed region and reported as well.

The other workloads (one JSON line each):
  --workload c1  config 1, one 960x960 q_proj with the 3-bit Lloyd-Max code: rotation, factor, width-1 sweep and
                 packed codes per step
  --workload c2  config 2, one 960x960 q_proj: rotation, factor, row-trellis sweep and packed codes per step
  --workload c3  config 3, one Qwen3.5-4B-shaped MLP block: Hessians of [131072, 2560] and [131072, 9728] with digit
                 token weights, one factor per stage, the row-plan sweeps of gate/up and down, packed codes
  --workload c4  config 4, one KL evaluation over paired bf16 logits [8192, 151936] per step
  --workload l2  the Gram kernels' operand delivery beside the ceiling of their global->LDS load path (a measurement
                 for the profiles, not a config)
--copy-probe M ends the run with one device-to-device copy of M MiB, the known-size reference for the HBM byte
counters of a profiler run.
"""

from __future__ import annotations

import argparse
import gc
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

METRIC = "weights quantized/sec (LDLQ+trellis) & Viterbi rows/sec; % MFMA/HBM roofline"

# published MI355X peaks
MFMA_BF16_PEAK_TFLOPS = 2500.0
MFMA_F64_PEAK_TFLOPS = 78.6
FP32_VECTOR_PEAK_TFLOPS = 157.3
FP64_VECTOR_PEAK_TFLOPS = 78.6
HBM_PEAK_GBS = 8000.0
# the trellis search's own ceiling: one non-packed, non-fused fp32 VALU op per lane per clock (the search rounds after
# every subtraction, square and addition, and packed FP32 is disabled): 256 CUs x 4 SIMDs x 16 lanes x 2.4 GHz
VALU_ISSUE_TOPS = 256 * 4 * 16 * 2.4e9 / 1e12

# HBM bytes per launch of the dominant kernel from two rocprofv3 counter runs (FETCH_SIZE, WRITE_SIZE), scaled by a
# 1 GiB copy's readings; keyed by (workload, kernel, L)
MEASURED_TRAFFIC = {("c2", "ldlq_trellis_block_gx_kernel", 16): 423926181,
                    ("c5", "ldlq_trellis_groups_gx_kernel", 16): 1394276752,
                    ("c5", "ldlq_trellis_groups_kernel", 12): 21661290}


def kernel_line(ms: float, work: float, peak: float, unit: str, bound: str, scale: float, launches: int = 0) -> dict:
    """Roofline entry of one kernel: `work` algorithmic units (flops, ops or bytes) done in `ms` of summed launch
    durations, `scale` units per reported unit (1e12 for TFLOP/s, 1e9 for GB/s)."""
    achieved = work / (ms * 1e-3) / scale if ms > 0 else 0.0
    out = {"bound": bound, "ms": round(ms, 4), "launches": launches, "achieved": round(achieved, 3), "peak": peak,
           "unit": unit, "frac": round(achieved / peak, 4)}
    if launches:
        out["avg_launch_us"] = round(1e3 * ms / launches, 2)
    return out


def trellis_line(ms: float, ops: float, launches: int, full_ops: float) -> dict:
    """The search kernel's line. ops counts reachable states only (engine.viterbi_search_ops: the first positions of
    a search from a fixed start reach fewer than 2^L states); full_ops counts every state of every position, as the
    reference's full-array recurrence computes them, and is reported beside it, never as `achieved`."""
    line = kernel_line(ms, ops, FP32_VECTOR_PEAK_TFLOPS, "TFLOP/s", "valu", 1e12, launches)
    line["issue_ceiling"] = round(VALU_ISSUE_TOPS, 1)
    line["frac_of_issue_ceiling"] = round(line["achieved"] / VALU_ISSUE_TOPS, 4)
    line["ops_counted"] = "reachable states"
    line["achieved_full_array_formulation"] = round(full_ops / (ms * 1e-3) / 1e12, 3) if ms > 0 else None
    return line


def spin_cycles(us: float) -> int:
    """torch.cuda._sleep cycles that keep the stream busy for about `us` microseconds, measured once on this GPU."""
    import torch

    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(1000)
    a.record()
    torch.cuda._sleep(1_000_000)
    b.record()
    torch.cuda.synchronize()
    per_us = 1_000_000 / max(a.elapsed_time(b) * 1e3, 1e-3)
    return max(1, int(us * per_us))


# ----------------------------------------------------------------------------- the CPU baseline


def host_threads() -> tuple[int, int]:
    """(CPUs in this process's affinity mask, the CPUs its cgroup quota lets it use at once, at most the former)."""
    aff = len(os.sched_getaffinity(0))
    eff = aff
    try:
        q, p = Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
        if q != "max":
            eff = min(aff, max(1, int(-(-int(q) // int(p)))))
    except (OSError, ValueError):
        pass
    return aff, eff


def _rows_parallel(fn, rows: list, threads: int) -> float:
    """Seconds of wall time for fn(row_chunk) over `rows` split across `threads` host threads (the C oracle releases
    the interpreter lock for its whole call)."""
    from concurrent.futures import ThreadPoolExecutor

    chunks = [rows[i::threads] for i in range(threads)]
    chunks = [c for c in chunks if c]
    t0 = time.perf_counter()
    with ThreadPoolExecutor(max_workers=len(chunks)) as ex:
        list(ex.map(fn, chunks))
    return time.perf_counter() - t0


_FACTORS: dict = {}


def _sample_factor(n: int, seed: int):
    """U of a random positive definite H at width n (made once per width: the factor's cost is timed elsewhere)."""
    import numpy as np

    from oracle import oracle as O

    if (n, seed) not in _FACTORS:
        Xa = np.random.default_rng(seed + 7 * n).standard_normal((2 * n, n))
        _FACTORS[(n, seed)] = O.environment(Xa.T @ Xa / (2 * n))[1]
    return _FACTORS[(n, seed)]


def cpu_sweep_rows(n: int, L: int, k: int, table, threads: int, rows_per_thread: int = 1, seed: int = 0) -> float:
    """Seconds per row of the C oracle's row-trellis sweep (search + in-block refit + trailing updates) at width n with
    `threads` rows in flight at once: one row per thread (times rows_per_thread), wall time / rows."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import oracle as O

    rng = np.random.default_rng(seed + n)
    U = _sample_factor(n, seed)
    rows = threads * rows_per_thread
    X = rng.standard_normal((rows, n))
    S = O.row_scale(X)
    with threadpool_limits(limits=1):
        wall = _rows_parallel(lambda r: O.ldlq_trellis(X[r], U, S[r], table, L, k), list(range(rows)), threads)
    return wall / rows


def cpu_fixed_parts(n: int, threads: int, sample_tokens: int = 4096, seed: int = 0, qep: bool = True,
                    m: int | None = None) -> dict:
    """Seconds of a stage's per-matrix statistics and algebra on the CPU (numpy/LAPACK on `threads` threads) at width n,
    by how each part scales, as the reference computes them (quantize.py:1457-1470, 1330-1335, 1503; codes.py:129-132,
    430-439; frame.py:515-522): "stats" the weighted Hessian (and with qep the QEP cross-Gram) in float32 over
    `sample_tokens` tokens (N n^2), "cubic" the QEP solve (with qep), the dense rotation R H R^T and the damped
    Cholesky-inverse factor (n^3), "rows" the rows' rotation W R^T (with qep after the target product W M) for m rows
    (default n; m n^2), "rht" the dense rotation matrix itself (n^2)."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import oracle as O

    rng = np.random.default_rng(seed + n)
    X = rng.standard_normal((sample_tokens, n), dtype=np.float32)
    Xr = X + np.float32(0.01) * rng.standard_normal((sample_tokens, n), dtype=np.float32)
    w = rng.random(sample_tokens, dtype=np.float32) + np.float32(0.5)
    W = rng.standard_normal((n if m is None else m, n))
    out = {}
    with threadpool_limits(limits=threads):
        t = time.perf_counter()
        Xw = X * w[:, None]
        H = X.T @ Xw
        D = Xr.T @ Xw if qep else None
        out["stats"] = time.perf_counter() - t
        t = time.perf_counter()
        R = O.rht(n, 1)
        out["rht"] = time.perf_counter() - t
        H = H.astype(np.float64) / sample_tokens
        t = time.perf_counter()
        if qep:
            D = D.astype(np.float64) / sample_tokens
            M = np.eye(n) + 0.5 * np.linalg.solve(H + 0.1 * np.mean(np.diag(H)) * np.eye(n), (D - H).T).T
        Hr = R @ H @ R.T
        O.environment(Hr)
        out["cubic"] = time.perf_counter() - t
        t = time.perf_counter()
        target = W @ M if qep else W
        _ = target @ R.T
        out["rows"] = time.perf_counter() - t
    return out


def extrapolate_layer(per_row: dict, fx: dict, stages: list, plans_one_layer: dict, tokens: int, n0: int,
                      sample_tokens: int, row_steps) -> tuple[float, float]:
    """(fixed, sweep) seconds of one layer from the sampled figures: per_row {bits: seconds per row at width n0 with
    the host's threads all busy, i.e. wall time / rows of a batch of one row per thread}, fx cpu_fixed_parts(n0),
    stages [(n, {name: m})], plans_one_layer {name: row groups}, row_steps(n) the trellis row-steps of a row of width
    n. The sweep of a row of width n costs per_row[bits] * row_steps(n) / row_steps(n0); the statistics scale with
    tokens x n^2, the solve, R H R^T and the factor with n^3, the target and row rotation with m n^2 and the rotation
    matrix with n^2."""
    fixed = sweep = 0.0
    for n, ms in stages:
        m = sum(ms.values())
        r = n / n0
        fixed += (fx["stats"] * tokens / sample_tokens * r * r + fx["cubic"] * r ** 3 + fx["rows"] * (m / n0) * r * r
                  + fx["rht"] * r * r)
        ratio = row_steps(n) / row_steps(n0)
        for nm in ms:
            for g in plans_one_layer[nm]:
                sweep += len(g["rows"]) * per_row[int(g["bits"])] * ratio
    return fixed, sweep


def cpu_baseline_c5(L: int, threads: int, sh, plans_one_layer: dict, tokens: int) -> dict:
    """The CPU restatement's time for one layer of the config-5 build at `threads` threads, from a bounded sample
    extrapolated by shape: the row sweep's seconds per row measured at n = 2,560 for each width (one row per thread in
    flight) and carried to n = 4,096 and 9,728 by trellis row-steps; the stage statistics and algebra measured at
    n = 2,560 (cpu_fixed_parts, the statistics on 4,096 tokens) and carried to each stage by their own scaling (tokens
    x n^2, n^3, rows x n^2, n^2). The calibration forwards are not part of it (the reference runs them on the GPU)."""
    from lookatmyquant_amd import engine as E
    from lookatmyquant_amd import stack
    from lookatmyquant_amd.tables import load_table, quantile_table

    t0 = time.perf_counter()
    tables = {b: (quantile_table(16, 0) if L == 16 else load_table(12, b)) for b in (1, 2, 3, 4)}
    n0, sample_tokens = 2560, 4096
    per_row = {k: cpu_sweep_rows(n0, L, k, tables[k], threads, rows_per_thread=4) for k in (1, 2, 3, 4)}
    fx = cpu_fixed_parts(n0, threads, sample_tokens)
    shapes = stack.matrix_shapes(sh)
    stages = [(shapes[names[0]][1], {nm: shapes[nm][0] for nm in names}) for names in stack.STAGES]
    fixed, sweep = extrapolate_layer(per_row, fx, stages, plans_one_layer, tokens, n0, sample_tokens,
                                     lambda n: sum(E.trellis_row_steps(n)))
    weights = sum(shapes[nm][0] * shapes[nm][1] for names in stack.STAGES for nm in names)
    total = fixed + sweep
    return {"value": round(weights / total, 1), "unit": "weights/s", "cores": threads, "kind": "port",
            "seconds_per_layer_extrapolated": round(total, 2), "of_which_sweeps": round(sweep, 2),
            "sample_seconds": round(time.perf_counter() - t0, 1),
            "seconds_per_row_n2560": {str(k): round(v, 4) for k, v in per_row.items()},
            "fixed_parts_n2560": {k: round(v, 4) for k, v in fx.items()}}


# ----------------------------------------------------------------------------- config 5 (the default)


def run_c5(args):
    import torch

    from lookatmyquant_amd import engine as E
    from lookatmyquant_amd import stack

    torch.cuda.set_device(0)
    sh = stack.Shape()
    tokens, w = stack.calibration_tokens()
    ntok = tokens.numel()
    layers = args.warmup + args.steps
    print(f"bench c5: L={args.L}, {args.warmup} warmup + {args.steps} timed layers", file=sys.stderr, flush=True)
    kt = E.KernelTimer()
    timer = stack.Timer()
    b = stack.StackBuild(tokens, sh, w, L=args.L, layers=layers, redamp=True, timer=timer, kernels=kt)
    for _ in range(args.warmup):
        b.layer()
    torch.cuda.synchronize()
    kt.events.clear()
    kt.work.clear()
    timer.clear()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        b.layer()
        print(f"bench c5: layer {b.next_layer - 1} done", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    secs = time.perf_counter() - t0
    out = b.result()
    assert int(out["bad"].item()) == 0  # every packed row a trellis path from state 0
    per_layer = secs / args.steps
    shapes = stack.matrix_shapes(sh)
    layer_weights = sum(m * n for m, n in shapes.values())
    rows_per_layer = sum(m for m, _ in shapes.values())
    row_steps_per_layer = sum(m * sum(E.trellis_row_steps(n)) for m, n in shapes.values())
    kern = {
        "ldlq_trellis_block": trellis_line(kt.ms("block"), kt.work.get("block", 0.0), kt.launches("block"),
                                           kt.work.get("block_full", 0.0)),
        "trailing_update_f64": kernel_line(kt.ms("trailing"), kt.work.get("trailing", 0.0), MFMA_F64_PEAK_TFLOPS,
                                           "TFLOP/s", "mfma", 1e12, kt.launches("trailing")),
        "hessian_gram_bf16": kernel_line(kt.ms("hessian"), kt.work.get("hessian", 0.0), MFMA_BF16_PEAK_TFLOPS,
                                         "TFLOP/s", "mfma", 1e12, kt.launches("hessian")),
        "cross_gram_bf16": kernel_line(kt.ms("cross_gram"), kt.work.get("cross_gram", 0.0), MFMA_BF16_PEAK_TFLOPS,
                                       "TFLOP/s", "mfma", 1e12, kt.launches("cross_gram")),
        "chol_inv_upper": kernel_line(kt.ms("chol"), kt.work.get("chol", 0.0), MFMA_F64_PEAK_TFLOPS, "TFLOP/s", "mfma",
                                      1e12, kt.launches("chol")),
        "qep_gemm_f64": kernel_line(kt.ms("qep_gemm"), kt.work.get("qep_gemm", 0.0), MFMA_F64_PEAK_TFLOPS, "TFLOP/s",
                                    "mfma", 1e12, kt.launches("qep_gemm")),
        "rht": kernel_line(kt.ms("rht"), kt.work.get("rht", 0.0), MFMA_F64_PEAK_TFLOPS, "TFLOP/s", "mfma", 1e12,
                           kt.launches("rht")),
        "pack_codes": kernel_line(kt.ms("pack"), kt.work.get("pack", 0.0), HBM_PEAK_GBS, "GB/s", "hbm", 1e9,
                                  kt.launches("pack")),
    }
    for k, v in kern.items():
        v["ms_per_step"] = round(v["ms"] / args.steps, 3)
    blk = kern["ldlq_trellis_block"]
    # at L >= 13 and at L = 12 each lazy block of a stage is one launch over all its row groups (k = 1..4 by
    # workgroup); at other widths each group is its own launch
    kname = ("ldlq_trellis_groups_gx_kernel" if args.L >= E.BIG_L else
             "ldlq_trellis_groups_kernel" if args.L == E.MERGED_SMALL_L else "ldlq_trellis_block_kernel")
    roofline = {"kernel": kname + " (k = 1..4)", "bound": "valu", "achieved": blk["achieved"],
                "peak": FP32_VECTOR_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": blk["frac"],
                "traffic": MEASURED_TRAFFIC.get(("c5", kname, args.L)), "avg_launch_us": blk.get("avg_launch_us"),
                "launches_per_step": round(blk["launches"] / args.steps, 1), "issue_ceiling": blk["issue_ceiling"],
                "frac_of_issue_ceiling": blk["frac_of_issue_ceiling"], "ops_counted": blk["ops_counted"],
                "achieved_full_array_formulation": blk["achieved_full_array_formulation"],
                "ops_per_row_step": {str(k): E.viterbi_ops_per_row_step(args.L, k) for k in (1, 2, 3, 4)}}
    phases = {k: round(v / args.steps, 3) for k, v in timer.t.items()}
    redamped, bpw = dict(out["redamped"]), out["bits"] / out["weights"]
    del b, out
    torch.cuda.empty_cache()
    # the production schedule, and the reference's own 12-bit trellis, on a few more layers (untimed by events)
    extra = {}
    for L, n_l in () if args.no_extra else ((args.L, 3), (12 if args.L != 12 else 16, 3)):
        bb = stack.StackBuild(tokens, sh, w, L=L, layers=n_l, redamp=True)
        bb.layer()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        for _ in range(n_l - 1):
            bb.layer()
        torch.cuda.synchronize()
        s = (time.perf_counter() - t1) / (n_l - 1)
        extra[f"L{L}_production_schedule"] = {"seconds_per_layer": round(s, 3),
                                              "seconds_per_36_layer_build": round(36 * s, 1),
                                              "weights_per_s": round(layer_weights / s, 1), "layers_timed": n_l - 1,
                                              "stages_damped_more": bb.redamped}
        del bb
        torch.cuda.empty_cache()
    line = {
        "metric": METRIC, "value": round(layer_weights / per_layer, 1), "unit": "weights/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(per_layer * 1e3, 1), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32 (trellis search) / f64 (sweep, factor, QEP) / bf16->f32 "
                                                         "(statistics)",
        "data": "synthetic (random-initialised stack, token ids uniform over the vocabulary, seed 501)",
        "config": {"workload": f"config 5: build of a Qwen3.5-4B-shaped stack (36 layers x 7 linears, hidden 2560, "
                               f"GQA 32/8 x 128, MLP 9728), 32 x 2048 calibration tokens through both streams with "
                               f"digit weights, QEP alpha 0.5, row-plan trellis L={args.L} bits 1-4 at 2.3 bpw, packed "
                               f"codes; a step is one decoder layer (its 7 linears), every kernel on one stream with "
                               f"per-launch events", "L": args.L,
                   "table": "fp16 Gaussian quantiles, 2^16 entries" if args.L == 16 else "the reference's fitted "
                                                                                         "12-bit tables",
                   "weights_per_step": layer_weights, "layers_timed": args.steps,
                   "bits_per_weight": round(bpw, 4),
                   "seconds_per_36_layer_build": round(36 * per_layer, 1), "target_seconds": 180,
                   "reference_published": "LM2 build of Qwen3.5-4B (32 layers, L = 12): 37 min on 1 x H100 + 8 CPU "
                                          "cores (README.md:68)",
                   "stages_damped_more": redamped, "seconds_by_phase_per_step": phases},
        "viterbi_rows_per_s": round(rows_per_layer / per_layer, 1),
        "viterbi_row_steps_per_s": round(row_steps_per_layer / per_layer, 1),
        "roofline": roofline, "kernels": kern, "other_schedules": extra,
    }
    if not args.no_cpu:
        aff, eff = host_threads()
        row_plan = stack.synthetic_plans(sh, 1)[1]
        plans_one = {nm: row_plan[f"model.layers.0.{nm}.weight"] for nm in shapes}
        base = cpu_baseline_c5(args.L, eff, sh, plans_one, ntok)
        eight = base if eff == 8 else cpu_baseline_c5(args.L, 8, sh, plans_one, ntok)
        base["sample"] = (f"C oracle + numpy/LAPACK, one layer of the same build extrapolated from a bounded sample: the row "
                          f"sweep timed at n = 2560 for k = 1..4 (one row per thread in flight) and carried to n = 4096 "
                          f"and 9728 by trellis row-steps; the per-stage Hessian and cross-Gram (float32, 4096 of {ntok} "
                          f"tokens), QEP solve and target, dense rotations and the factor timed at n = 2560 and carried "
                          f"to each stage by their own scaling; forwards excluded. {eff} threads = the CPUs this "
                          f"process may use at once ({aff} in its affinity mask)")
        base["affinity_cpus"] = aff
        base["at_8_threads"] = {"value": eight["value"], "cores": 8,
                                "seconds_per_layer_extrapolated": eight["seconds_per_layer_extrapolated"]}
        line["cpu_baseline"] = base
    print(json.dumps(line))


# ----------------------------------------------------------------------------- config 2


def cpu_baseline_c2(W, H, table, L, k, in_seed, threads, budget_s=8.0):
    """The C oracle on config 2 at `threads` host threads: the rotation, Hessian rotation and factor (numpy/LAPACK on
    those threads) in full, the sweep on as many rows as fit in the budget (one row per thread at once), extrapolated by
    rows (rows are independent given U and S)."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import oracle as O

    m, n = W.shape
    with threadpool_limits(limits=threads):
        t0 = time.perf_counter()
        R = O.rht(n, in_seed)
        X = np.asarray(W, dtype=np.float64) @ R.T
        S = O.row_scale(X)
        Hr = R @ H @ R.T
        _, U, dead = O.environment(Hr)
        t_fixed = time.perf_counter() - t0
    rows, t_rows = 0, 0.0
    with threadpool_limits(limits=1):
        while rows < m and t_rows < budget_s:
            r = list(range(rows, min(rows + threads, m)))
            t_rows += _rows_parallel(lambda c: O.ldlq_trellis(X[c], U, S[c], table, L, k,
                                                              dead=dead if dead.any() else None), r, threads)
            rows += len(r)
    total = t_fixed + t_rows / rows * m
    return {"value": round(m * n / total, 1), "unit": "weights/s", "cores": threads, "kind": "port",
            "sample": f"C oracle: rotation, R H R^T and U (numpy LAPACK) in full ({t_fixed:.2f} s); sweep on the first "
                      f"{rows} of {m} rows, {threads} at once ({t_rows:.2f} s), extrapolated by rows",
            "seconds_total_extrapolated": round(total, 3)}


def scalar_ops_per_row(n: int, K: int, lazy: int = 128) -> float:
    """Algorithmic work of the width-1 sweep per row (syntax.py:106-121 with the search of nested.py:127-140): per
    entry the search's K subtractions, K squares and K - 1 comparisons and the division z = E / U_jj; per lazy block
    of w columns the in-block rank-1 refits, w (w - 1) / 2 fused multiply-adds of two flops each."""
    ops = 0.0
    for b0 in range(0, n, lazy):
        w = min(lazy, n - b0)
        ops += w * (3 * K) + w * (w - 1)
    return ops


def run_c1(args):
    """Config 1: one 960x960 q_proj with the 3-bit Lloyd-Max code (nested.py:127-140's one-rate sweep)."""
    import numpy as np
    import torch

    from lookatmyquant_amd import engine as E
    from lookatmyquant_amd import synthetic
    from lookatmyquant_amd.nested import lloyd_max

    torch.cuda.set_device(0)
    bits, lazy = 3, 128
    in_seed = 201
    W, H = synthetic.config12()
    m, n = W.shape
    dev = torch.device("cuda", 0)
    Wg = torch.from_numpy(W.astype(np.float64)).to(dev)
    Hg = torch.from_numpy(H).to(dev)
    levels = lloyd_max(bits).to(dev)
    K = levels.numel()

    def step(events=None):
        X, S = E.rht_rows(Wg, in_seed, want_rms=True)
        Hr = E.rotate_hessian(Hg, in_seed)
        _, U, dead, info = E.chol_inv_upper(Hr, raise_on_fail=False)
        idx = E.ldlq_scalar(X / S[:, None], U, levels, mode=0, lazy=lazy, dead=dead, events=events)
        codes, bad = E.pack_codes(idx, bits, trellis=False)
        return idx, codes, info, bad

    for _ in range(args.warmup):
        idx, codes, info, bad = step()
    torch.cuda.synchronize()
    assert int(info.item()) == 0 and int(bad.item()) == 0
    events = E.EventLog()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        idx, codes, info, bad = step(events)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    blk = E.event_ms(events, "block")
    trl = E.event_ms(events, "trailing")
    work = m * scalar_ops_per_row(n, K, lazy) * args.steps
    line = kernel_line(sum(blk), work, FP64_VECTOR_PEAK_TFLOPS, "TFLOP/s", "valu", 1e12, len(blk))
    out = {
        "metric": METRIC, "value": round(m * n / (ms * 1e-3), 1), "unit": "weights/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f64 (sweep and search)", "data": "synthetic",
        "config": {"workload": f"config 1: one 960x960 q_proj, width-1 block LDLQ onto the {bits}-bit Lloyd-Max levels "
                               f"(lazy {lazy}), H from 16384 bf16 tokens, rotation + factor + sweep + packed codes per "
                               "step", "rows": m, "columns": n, "bits": bits},
        "roofline": {"kernel": "ldlq_scalar_block_kernel", "bound": "valu", "achieved": line["achieved"],
                     "peak": FP64_VECTOR_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": line["frac"], "traffic": None,
                     "avg_launch_us": line.get("avg_launch_us"), "launches_per_step": len(blk) // args.steps,
                     "work": "per entry 3K search operations; per lazy block of w columns w (w - 1) flops of in-block "
                             "refits (fp64 FMAs)"},
        "phase_ms": {"block_kernels": round(sum(blk) / args.steps, 4),
                     "trailing_updates": round(sum(trl) / args.steps, 4)},
    }
    if not args.no_cpu:
        aff, eff = host_threads()
        base = cpu_baseline_c1(W, H, levels.cpu().numpy(), in_seed, lazy, eff)
        eight = base if eff == 8 else cpu_baseline_c1(W, H, levels.cpu().numpy(), in_seed, lazy, 8)
        base["affinity_cpus"] = aff
        base["at_8_threads"] = {"value": eight["value"], "cores": 8, "sample": eight["sample"]}
        out["cpu_baseline"] = base
    print(json.dumps(out))


def cpu_baseline_c1(W, H, levels, in_seed, lazy, threads, budget_s: float = 5.0):
    """The C oracle on config 1, all of it: rotation, Hessian rotation and factor (numpy/LAPACK on `threads` host
    threads), then the width-1 sweep of every row (one row per thread at once); the whole matrix again until about
    budget_s seconds have passed (one matrix takes a fraction of a second), the median repetition reported."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import oracle as O

    m, n = W.shape
    reps = []
    while not reps or (sum(t for t, _, _ in reps) < budget_s and len(reps) < 50):
        with threadpool_limits(limits=threads):
            t0 = time.perf_counter()
            R = O.rht(n, in_seed)
            X = np.asarray(W, dtype=np.float64) @ R.T
            S = O.row_scale(X)
            Hr = R @ H @ R.T
            _, U, dead = O.environment(Hr)
            t_fixed = time.perf_counter() - t0
        T0 = X / S[:, None]
        with threadpool_limits(limits=1):
            t_rows = _rows_parallel(lambda c: O.ldlq_scalar(T0[c], U, levels, 0, lazy=lazy,
                                                            dead=dead if dead.any() else None), list(range(m)), threads)
        reps.append((t_fixed + t_rows, t_fixed, t_rows))
    total, t_fixed, t_rows = sorted(reps)[len(reps) // 2]
    return {"value": round(m * n / total, 1), "unit": "weights/s", "cores": threads, "kind": "port",
            "sample": f"C oracle: rotation, R H R^T and U (numpy LAPACK) ({t_fixed:.3f} s) and the sweep of all {m} rows "
                      f"({t_rows:.3f} s), {threads} threads; the median of {len(reps)} repetitions of the whole matrix",
            "seconds_total": round(total, 4)}


def run_c2(args):
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
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    blk = E.event_ms(events, "block")
    trl = E.event_ms(events, "trailing")
    per_block = E.trellis_row_steps(n, width, look, lazy)
    ops = m * sum(E.trellis_block_ops(n, L, k, width, look, lazy)) * args.steps
    full_ops = m * sum(per_block) * E.viterbi_ops_per_row_step(L, k) * args.steps
    line = trellis_line(sum(blk), ops, len(blk), full_ops)
    if L < E.BIG_L:
        kname = "ldlq_trellis_block_kernel"
    else:
        kname = "ldlq_trellis_block_gx_kernel"
    out = {
        "metric": METRIC, "value": round(m * n / (ms * 1e-3), 1), "unit": "weights/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32 (trellis search) / f64 (sweep)", "data": "synthetic",
        "config": {"workload": f"config 2: one 960x960 q_proj, row-trellis block LDLQ k={k} L={L} (width 16, look 8, "
                               "lazy 128), H from 16384 bf16 tokens, rotation + factor + sweep + packed codes per step",
                   "rows": m, "columns": n, "L": L, "k": k,
                   "table": "reference e-means L=12 table" if L == 12 else f"fp16 Gaussian quantiles, 2^{L} entries"},
        "viterbi_rows_per_s": round(m / (ms * 1e-3), 1),
        "viterbi_row_steps_per_s": round(m * sum(per_block) / (ms * 1e-3), 1),
        "roofline": {"kernel": kname, "bound": "valu", "achieved": line["achieved"], "peak": FP32_VECTOR_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": line["frac"], "traffic": MEASURED_TRAFFIC.get(("c2", kname, L)),
                     "launches_per_step": len(per_block), "avg_launch_us": line["avg_launch_us"],
                     "issue_ceiling": line["issue_ceiling"], "frac_of_issue_ceiling": line["frac_of_issue_ceiling"],
                     "ops_counted": line["ops_counted"],
                     "achieved_full_array_formulation": line["achieved_full_array_formulation"],
                     "ops_per_row_step": E.viterbi_ops_per_row_step(L, k)},
        "phase_ms": {"block_kernels": round(sum(blk) / args.steps, 4),
                     "trailing_updates": round(sum(trl) / args.steps, 4)},
    }
    if not args.no_cpu:
        aff, eff = host_threads()
        base = cpu_baseline_c2(W, H, table, L, k, in_seed, eff)
        eight = base if eff == 8 else cpu_baseline_c2(W, H, table, L, k, in_seed, 8)
        base["affinity_cpus"] = aff
        base["at_8_threads"] = {"value": eight["value"], "cores": 8, "sample": eight["sample"]}
        out["cpu_baseline"] = base
    print(json.dumps(out))


# ----------------------------------------------------------------------------- config 3


def cpu_baseline_c3(L: int, threads: int, plans: dict, N: int, stage_rows: list, rows_per_thread: int = 1,
                    sample_tokens: int = 4096) -> dict:
    """The CPU restatement's time for config 3 at `threads` threads, each part measured at the stage's own width: per
    stage (n = 2,560: gate and up; n = 9,728: down) the weighted Hessian in float32 on `sample_tokens` of the N tokens
    (scaled by N / sample_tokens: its cost is linear in the tokens), the dense rotation matrix, R H R^T, the damped
    Cholesky-inverse factor and the rotation of the stage's rows W R^T in full (numpy/LAPACK), and the row sweep
    (the C oracle, one row per thread in flight) for each bit width on threads x rows_per_thread rows, extrapolated by
    the plan's row count of that width (rows are independent given U and S)."""
    from lookatmyquant_amd.tables import load_table, quantile_table

    t0 = time.perf_counter()
    tables = {b: (quantile_table(16, 0) if L == 16 else load_table(12, b)) for b in (1, 2, 3, 4)}
    fixed = sweep = 0.0
    parts = {}
    for n, names in stage_rows:
        m = sum(len(g["rows"]) for nm in names for g in plans[nm])
        fx = cpu_fixed_parts(n, threads, sample_tokens, qep=False, m=m)
        fixed += fx["stats"] * N / sample_tokens + fx["rht"] + fx["cubic"] + fx["rows"]
        per_row = {}
        for k in (1, 2, 3, 4):
            rows_k = sum(len(g["rows"]) for nm in names for g in plans[nm] if int(g["bits"]) == k)
            if rows_k:
                per_row[k] = cpu_sweep_rows(n, L, k, tables[k], threads, rows_per_thread)
                sweep += rows_k * per_row[k]
        parts[str(n)] = {"fixed": {p: round(v, 4) for p, v in fx.items()},
                         "seconds_per_row": {str(k): round(v, 5) for k, v in per_row.items()}}
    total = fixed + sweep
    weights = sum(len(g["rows"]) * n for n, names in stage_rows for nm in names for g in plans[nm])
    return {"value": round(weights / total, 1), "unit": "weights/s", "cores": threads, "kind": "port",
            "seconds_total_extrapolated": round(total, 3), "of_which_sweeps": round(sweep, 3),
            "sample_seconds": round(time.perf_counter() - t0, 1), "by_width": parts,
            "sample": f"C oracle + numpy/LAPACK on {threads} threads: per stage the weighted Hessian (float32) on "
                      f"{sample_tokens} of {N} tokens scaled by tokens, the dense rotation, R H R^T, the damped "
                      f"Cholesky-inverse factor and W R^T in full; the row sweep on {threads * rows_per_thread} rows "
                      f"per bit width (one row per thread in flight), extrapolated by the plan's rows"}


def run_c3(args):
    """Config 3: one MLP block (gate/up stage on the hidden input, down stage on the intermediate)."""
    import torch

    from lookatmyquant_amd import engine as E
    from lookatmyquant_amd import synthetic
    from lookatmyquant_amd.quantize import quantize_stage_row_groups
    from lookatmyquant_amd.tables import load_table, quantile_table

    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    L = args.L
    hid, inter, N = 2560, 9728, 131072
    t0 = time.perf_counter()
    Wg = torch.from_numpy(synthetic.weight(inter, hid, 0.015, 301)).to(dev).bfloat16()
    Wu = torch.from_numpy(synthetic.weight(inter, hid, 0.015, 302)).to(dev).bfloat16()
    Wd = torch.from_numpy(synthetic.weight(hid, inter, 0.015, 303)).to(dev).bfloat16()
    X1 = torch.from_numpy(synthetic.calibration(N, hid, 304, 305)).to(dev).bfloat16()
    # the down input is the block's intermediate: silu(X1 Wg^T) * (X1 Wu^T) in bf16, computed in slices
    X2 = torch.empty(N, inter, dtype=torch.bfloat16, device=dev)
    for b in range(0, N, 16384):
        x = X1[b : b + 16384]
        X2[b : b + 16384] = torch.nn.functional.silu(x @ Wg.t().contiguous()) * (x @ Wu.t().contiguous())
    w = torch.from_numpy(synthetic.digit_weights(N, 306)).to(dev)
    plans = {"gate": synthetic.row_plan(inter, 307), "up": synthetic.row_plan(inter, 308),
             "down": synthetic.row_plan(hid, 309)}
    tables = {b: (quantile_table(16, 0) if L == 16 else load_table(12, b)) for b in (1, 2, 3, 4)}
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t0
    stages = [({"gate": Wg, "up": Wu}, X1, 1301), ({"down": Wd}, X2, 3301)]  # in_seed of layer 0's stages
    plan_rows = {nm: E.device_rows(p, dev) for nm, p in plans.items()}

    def step(kt):
        """One build of the block. kt None: the production schedule (each row group's sweep on its own stream); a
        KernelTimer: every launch timed in turn on one stream."""
        out = {}
        for targets, X, in_seed in stages:
            n = X.shape[1]
            with E.span(kt, "hessian", float(N) * n * (n + 1)):
                H = E.hessian(X, w)
            sub = {nm: W.double() for nm, W in targets.items()}
            res = quantize_stage_row_groups(sub, {nm: plans[nm] for nm in sub}, H, in_seed, L=L, tables=tables,
                                            timer=kt)
            for nm, (st, S) in res.items():
                for g, rows in zip(plans[nm], plan_rows[nm]):
                    out[(nm, g["group"])] = E.pack_trellis(st.index_select(0, rows).contiguous(), g["bits"], L,
                                                           check_paths=False)
        return out

    for _ in range(args.warmup):
        step(None)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(args.steps):
        out = step(None)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t1) * 1e3 / args.steps
    bad = sum(int(b.item()) for _, b in out.values())
    assert bad == 0
    # the per-kernel lines: one more build with every launch timed in turn (row groups one after the other). The
    # host enqueues this build's short launches more slowly than the GPU runs them, so each span starts behind a GPU
    # spin of about 100 us (outside the span): the span then times its kernel, not the host's launch latency.
    kt = E.KernelTimer(lead_cycles=spin_cycles(100.0))
    step(kt)
    torch.cuda.synchronize()
    weights = 2 * inter * hid + hid * inter
    row_steps_total, ops_total, full_total, trail_total = 0.0, 0.0, 0.0, 0.0
    for targets, X, _ in stages:
        n = X.shape[1]
        for bits in (1, 2, 3, 4):
            m = sum(len(g["rows"]) for nm in targets for g in plans[nm] if g["bits"] == bits)
            if m == 0:
                continue
            rs = m * sum(E.trellis_row_steps(n))
            row_steps_total += rs
            ops_total += m * sum(E.trellis_block_ops(n, L, bits))
            full_total += rs * E.viterbi_ops_per_row_step(L, bits)
            trail_total += E.trailing_flops(m, n)
    kern = {"hessian_gram_bf16": kernel_line(kt.ms("hessian"), kt.work["hessian"], MFMA_BF16_PEAK_TFLOPS, "TFLOP/s",
                                             "mfma", 1e12, kt.launches("hessian")),
            "chol_inv_upper": kernel_line(kt.ms("chol"), kt.work["chol"], MFMA_F64_PEAK_TFLOPS, "TFLOP/s", "mfma",
                                          1e12, kt.launches("chol")),
            "ldlq_trellis_block": trellis_line(kt.ms("block"), ops_total, kt.launches("block"), full_total),
            "trailing_update_f64": kernel_line(kt.ms("trailing"), trail_total, MFMA_F64_PEAK_TFLOPS, "TFLOP/s",
                                               "mfma", 1e12, kt.launches("trailing")),
            "rht": kernel_line(kt.ms("rht"), kt.work["rht"], MFMA_F64_PEAK_TFLOPS, "TFLOP/s", "mfma", 1e12,
                               kt.launches("rht"))}
    line = {
        "metric": METRIC, "value": round(weights / (ms * 1e-3), 1), "unit": "weights/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16->f32 (Hessian), f64/f32 (sweep)", "data": "synthetic",
        "config": {"workload": f"config 3: Qwen3.5-4B-shaped MLP block, gate/up [9728, 2560] and down [2560, 9728], "
                               f"Hessians from {N} bf16 tokens (10% digit tokens weighted 10x), row plans 2.3 bpw "
                               f"bits 1-4, row trellis L={L}, one factor per stage, packed codes per group",
                   "L": L, "tokens": N, "weights": weights, "setup_s": round(setup_s, 1)},
        "viterbi_row_steps_per_s": round(row_steps_total / (ms * 1e-3), 1),
        "kernels": kern}
    if not args.no_cpu:
        aff, eff = host_threads()
        stage_rows = [(hid, ("gate", "up")), (inter, ("down",))]
        base = cpu_baseline_c3(L, eff, plans, N, stage_rows)
        eight = base if eff == 8 else cpu_baseline_c3(L, 8, plans, N, stage_rows)
        base["affinity_cpus"] = aff
        base["at_8_threads"] = {"value": eight["value"], "cores": 8,
                                "seconds_total_extrapolated": eight["seconds_total_extrapolated"]}
        line["cpu_baseline"] = base
    print(json.dumps(line))


# ----------------------------------------------------------------------------- L2-to-CU delivery


def run_l2(args):
    """The Gram kernels' operand delivery against the ceiling of their load path: lamq_probe_l2_delivery (one workgroup
    a CU streaming 32 KB stages global->LDS from L2-resident regions, nothing else) beside the unweighted Hessian and
    cross-Gram base passes at the config-5 widths over 65,536 tokens. A 256-tile Gram workgroup loads 32 KB of operands
    per 32-token stage (256 features x 32 tokens x 2 bytes, two operands), so its delivered bytes are tiles x splits x
    stages x 32 KB. Rates per CU per clock at the 2.4 GHz peak clock (the ratio does not depend on the clock)."""
    import torch

    from lookatmyquant_amd import engine as E
    from lookatmyquant_amd._abi import check, ld, lib, ptr, stream

    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    cus, clk = 256, 2.4e9

    def timed(fn, reps):
        fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps * 1e-3

    region, stages, wgs = 2 << 20, 4096, 256
    buf = torch.zeros(8 * region, dtype=torch.uint8, device=dev)
    st = stream(dev)
    t = timed(lambda: check(lib().lamq_probe_l2_delivery(ptr(buf), region, stages, wgs, st), "probe"), args.steps)
    probe = wgs * stages * 32768 / t
    out = {"probe": {"bytes_per_s": round(probe, 1), "bytes_per_clk_per_cu": round(probe / cus / clk, 2),
                     "workgroups": wgs, "stages": stages, "region_bytes_per_xcd": region}}
    del buf
    N = 65536
    for n in (2560, 9728):
        X = torch.randn(N, n, device=dev).bfloat16()
        Y = torch.randn(N, n, device=dev).bfloat16()
        H = torch.zeros(n, n, device=dev)
        nt = -(-n // 256)
        for sym in (1, 0):
            nb = lib().lamq_gram_workspace_size(N, n, sym)
            ws = E.workspace(nb, dev)
            if sym:
                fn = lambda: check(lib().lamq_hessian_accum(ptr(X), N, n, ld(X), None, 1.0, ptr(H), ld(H), ptr(ws), nb,
                                                            st), "hessian")
            else:
                fn = lambda: check(lib().lamq_cross_gram(ptr(Y), ptr(X), N, n, ld(X), None, 1.0, ptr(H), ld(H), ptr(ws),
                                                         nb, st), "cross_gram")
            t = timed(fn, args.steps)
            tiles = nt * (nt + 1) // 2 if sym else nt * nt
            delivered = tiles * -(-N // 32) * 32768 / t  # every split's workgroups cover the N tokens once per tile
            flops = N * n * (n + 1) if sym else 2.0 * N * n * n
            out[f"{'hessian' if sym else 'cross_gram'}_n{n}"] = {
                "bytes_per_s": round(delivered, 1), "bytes_per_clk_per_cu": round(delivered / cus / clk, 2),
                "of_probe": round(delivered / probe, 3), "ms": round(t * 1e3, 3),
                "frac_of_bf16_peak": round(flops / t / (MFMA_BF16_PEAK_TFLOPS * 1e12), 3)}
            del ws
        del X, Y, H
        torch.cuda.empty_cache()
    print(json.dumps({"metric": "L2-to-CU delivery of the Gram kernels' load path", "value": out["probe"][
        "bytes_per_clk_per_cu"], "unit": "bytes/clk/CU (at 2.4 GHz)", "n_gpus": 1, "steps": args.steps,
        "warmup": 1, "higher_is_better": True, "data": "synthetic", "config": {"workload": "l2 delivery probe"},
        "results": out}))


# ----------------------------------------------------------------------------- config 4


def run_c4(args):
    """Config 4: KL(p_ref || p_q) over paired bf16 logits [8192, 151936], one evaluation per step."""
    import torch

    from lookatmyquant_amd import engine as E

    torch.cuda.set_device(0)
    T, V = 8192, 151936
    g1 = torch.Generator(device="cuda").manual_seed(401)
    g2 = torch.Generator(device="cuda").manual_seed(402)
    ref = (torch.randn(T, V, generator=g1, device="cuda") * 3.0).bfloat16()
    q = (ref.float() + 0.3 * torch.randn(T, V, generator=g2, device="cuda")).bfloat16()
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        E.kl_rows(ref, q)
    torch.cuda.synchronize()
    kt = E.KernelTimer()
    nbytes = 2.0 * T * V * 2 + 4 * T
    t1 = time.perf_counter()
    for _ in range(args.steps):
        with kt.span("kl", nbytes):
            kl, sums = E.kl_rows(ref, q)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t1) * 1e3 / args.steps
    cpu = None
    if not args.no_cpu:
        aff, eff = host_threads()
        cpu = cpu_baseline_c4(ref, q, eff, T)
        eight = cpu if eff == 8 else cpu_baseline_c4(ref, q, 8, T)
        cpu["affinity_cpus"] = aff
        cpu["at_8_threads"] = {"value": eight["value"], "cores": 8, "sample": eight["sample"]}
    print(json.dumps({
        "metric": "KL evaluations/s (per-token KL over paired bf16 logits)", "value": round(1e3 / ms, 2),
        "unit": "evals/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16->f32", "data":
        "synthetic (torch CUDA generator, seeds 401/402; ref ~ N(0, 3^2), q = ref + N(0, 0.3^2))",
        "config": {"workload": "config 4: one KL evaluation over [8192, 151936] bf16 logit pairs per step",
                   "tokens": T, "vocab": V, "mean_kl": float(sums[0] / sums[1])},
        "kernels": {"kl_rows": kernel_line(kt.ms("kl"), kt.work["kl"], HBM_PEAK_GBS, "GB/s", "hbm", 1e9,
                                           kt.launches("kl"))},
        **({"cpu_baseline": cpu} if cpu else {})}))


def cpu_baseline_c4(ref, q, threads: int, T: int, sample_tokens: int = 1024) -> dict:
    """The C oracle's KL (compiler.py:177-188 in float64) on the first `sample_tokens` token rows of the same logits,
    the rows split across `threads` host threads, scaled to one evaluation of T tokens (tokens are independent)."""
    import numpy as np
    import torch

    from oracle import oracle as O

    r = ref[:sample_tokens].cpu().view(torch.int16).numpy().view(np.uint16)
    qq = q[:sample_tokens].cpu().view(torch.int16).numpy().view(np.uint16)
    from concurrent.futures import ThreadPoolExecutor

    cuts = [i * sample_tokens // threads for i in range(threads + 1)]  # contiguous token blocks, one per thread
    t0 = time.perf_counter()
    with ThreadPoolExecutor(max_workers=threads) as ex:
        list(ex.map(lambda i: O.kl_rows(r[cuts[i]:cuts[i + 1]], qq[cuts[i]:cuts[i + 1]]), range(threads)))
    wall = time.perf_counter() - t0
    per_eval = wall * T / sample_tokens
    return {"value": round(1.0 / per_eval, 4), "unit": "evals/s", "cores": threads, "kind": "port",
            "seconds_per_eval_extrapolated": round(per_eval, 3),
            "sample": f"C oracle (float64) on the first {sample_tokens} of {T} token rows, {threads} threads "
                      f"({wall:.2f} s), scaled by tokens"}


def copy_probe(mib: int):
    """One device-to-device copy of `mib` MiB: reads and writes that many bytes once."""
    import torch

    n = mib * (1 << 20) // 4
    a = torch.ones(n, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()
    print(f"copy probe: {mib} MiB device-to-device", file=sys.stderr)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (c5: decoder layers, default 12; c2 10; c3 5; c4 10)")
    ap.add_argument("--warmup", type=int, default=None, help="untimed steps first (default 2; c3 1; c2, c4 3)")
    ap.add_argument("--L", type=int, default=None,
                    help="trellis state bits: default 16 for c5 and c2 (the 2^16-entry fp16 table), 12 for c3 (the "
                         "reference's production trellis)")
    ap.add_argument("--k", type=int, default=2, help="c2: bits per weight")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--workload", choices=("c1", "c2", "c3", "c4", "c5", "l2"), default="c5")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MiB")
    ap.add_argument("--no-extra", action="store_true",
                    help="c5: skip the extra layers timed in the production schedule and at the other state width")
    args = ap.parse_args()
    if args.steps is None:
        args.steps = {"c5": 12, "c3": 5}.get(args.workload, 10)
    if args.warmup is None:
        args.warmup = {"c5": 2, "c3": 1}.get(args.workload, 3)
    if args.L is None:
        args.L = 12 if args.workload == "c3" else 16
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the per-matrix hot path runs on one MI355X here (rows would shard across "
              "GPUs with no communication). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    # no collector passes inside the timed regions: a generation-2 pass over the many event objects of a timed build
    # stalls the host for tens of ms, and where the GPU has drained its queue by then, the stall lands inside a span
    gc.collect()
    gc.disable()
    {"c1": run_c1, "c2": run_c2, "c3": run_c3, "c4": run_c4, "c5": run_c5, "l2": run_l2}[args.workload](args)
    if args.copy_probe:
        copy_probe(args.copy_probe)


if __name__ == "__main__":
    main()
