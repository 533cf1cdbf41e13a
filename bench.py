"""Benchmark of the per-matrix quantization hot path on one MI355X.

A step is one pass of the hot path over one matrix of the workload: the input rotation X = W R_in^T with the row
scales S, the Hessian rotation R_in H R_in^T, the damped Cholesky-inverse U, the block-LDLQ sweep with the row
trellis (fused Viterbi + in-block refit kernel per 128-column block, fp64 MFMA trailing update between blocks) and
the packed codes. W and H are resident in HBM when the timed region starts (the calibration capture that produces
H is not part of a step).

    python bench.py [--steps K] [--warmup W] [--L 16|12] [--k 2] [--no-cpu] [--workload c2|c3|c4|c5] [--copy-probe MiB]

The default is the benchmark configuration (config 2: 16-bit states, the fp16 quantile table); --L 12 runs the
reference's own production trellis (the fitted 12-bit tables), the default of the c3 and c5 workloads.

Prints one JSON line: weights quantized per second (metric value), Viterbi rows/s, the roofline of the dominant
kernel (the fused trellis block kernel) measured with HIP events on its stream, and the CPU oracle timed on a
bounded row sample of the same workload.

The other workloads measure the remaining kernels at their configurations' shapes (one JSON line each, with a
roofline per kernel from HIP events):
  --workload c3  config 3, one Qwen3.5-4B-shaped MLP block: Hessians of the gate/up input [131072, 2560] and of the
                 down input [131072, 9728] with digit token weights, one factor per stage, the row-plan sweeps of
                 gate/up [9728, 2560] and down [2560, 9728] (bits 1-4, 2.3 bpw) and the packed codes per group
  --workload c4  config 4, one KL evaluation over paired bf16 logits [8192, 151936] per step
  --workload c5  config 5, the end-to-end build of a random-initialised Qwen3.5-4B-shaped stack (36 layers x 7
                 linears, hidden 2560, GQA 32/8 x 128, MLP 9728): calibration forwards of 32 x 2048 token ids through
                 the reference and the quantized stream, per-stage Hessians and QEP cross terms (alpha 0.5), the
                 row-plan trellis codes (bits 1-4, 2.3 bpw) and the packed codes; one step is the whole build
                 (--layers N builds the first N layers)
--copy-probe M ends the run with one device-to-device copy of M MiB, the known-size reference for the HBM byte
counters of a profiler run.
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


# HBM bytes per launch of the dominant kernel, from two rocprofv3 counter runs (FETCH_SIZE, WRITE_SIZE) scaled by a
# 1 GiB copy's readings (profiles/ldlq_trellis_block_gx_config2_L16_k2.md); keyed by (kernel, L, k).
MEASURED_TRAFFIC = {("ldlq_trellis_block_gx_kernel", 16, 2): 10749602}

MFMA_F64_PEAK_TFLOPS = 78.6
MFMA_BF16_PEAK_TFLOPS = 2500.0
HBM_PEAK_GBS = 8000.0


def kernel_line(ms_per_step: float, work: float, peak: float, unit: str, bound: str, scale: float) -> dict:
    """Roofline entry of one kernel: `work` algorithmic units per step (flops, ops or bytes), `scale` units per
    reported unit (1e12 for TFLOP/s and TOP/s, 1e9 for GB/s)."""
    achieved = work / (ms_per_step * 1e-3) / scale if ms_per_step > 0 else 0.0
    return {"bound": bound, "ms_per_step": round(ms_per_step, 4), "achieved": round(achieved, 3), "peak": peak,
            "unit": unit, "frac": round(achieved / peak, 4)}


def timed(events: dict, key: str):
    """Context manager recording a torch.cuda.Event pair on the current stream under events[key]."""
    import contextlib

    import torch

    @contextlib.contextmanager
    def cm():
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        yield
        b.record()
        events.setdefault(key, []).append((a, b))

    return cm()


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


def trail_flops(m: int, n: int, lazy: int = 128) -> float:
    """Algorithmic flops of the trailing updates of one sweep: sum over blocks of 2 m (b1 - b0) (n - b1)."""
    return float(sum(2 * m * (min(b0 + lazy, n) - b0) * (n - min(b0 + lazy, n)) for b0 in range(0, n, lazy)))


def run_c3(args):
    """Config 3: one MLP block (gate/up stage on the hidden input, down stage on the intermediate)."""
    import numpy as np
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

    def step(events):
        """One build of the block. events=None: the production schedule (each row group's sweep on its own
        stream); a dict: every launch timed in turn on one stream, for the per-kernel lines."""
        import contextlib

        out = {}
        for targets, X, in_seed in stages:
            n = X.shape[1]
            with (timed(events, f"hessian_{n}") if events is not None else contextlib.nullcontext()):
                H = E.hessian(X, w)
            sub = {nm: W.double() for nm, W in targets.items()}
            res = quantize_stage_row_groups(sub, {nm: plans[nm] for nm in sub}, H, in_seed, L=L, tables=tables,
                                            events=events,
                                            chol_events=None if events is None else (events, f"chol_{n}"))
            for nm, (st, S) in res.items():
                for g in plans[nm]:
                    rows = torch.as_tensor(g["rows"], device=dev)
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
    # the per-kernel lines: one more build with every launch timed in turn (row groups one after the other)
    events: dict = {}
    step(events)
    torch.cuda.synchronize()
    weights = 2 * inter * hid + hid * inter
    per = lambda key: sum(E.event_ms(events, key))
    kern = {}
    for n in (hid, inter):
        kern[f"hessian_n{n}"] = kernel_line(per(f"hessian_{n}"), float(N) * n * (n + 1), MFMA_BF16_PEAK_TFLOPS,
                                            "TFLOP/s", "mfma", 1e12)
        kern[f"chol_inv_upper_n{n}"] = kernel_line(per(f"chol_{n}"), 4.0 * n ** 3 / 3, MFMA_F64_PEAK_TFLOPS,
                                                   "TFLOP/s", "mfma", 1e12)
    # trellis block kernels and trailing updates: every sweep is one width's rows of a stage
    row_steps_total, ops_total, trail_total = 0.0, 0.0, 0.0
    for targets, X, _ in stages:
        n = X.shape[1]
        for bits in (1, 2, 3, 4):
            m = sum(len(g["rows"]) for nm in targets for g in plans[nm] if g["bits"] == bits)
            if m == 0:
                continue
            rs = m * sum(row_steps(n, 16, 8, 128))
            row_steps_total += rs
            ops_total += rs * viterbi_ops_per_row_step(L, bits)
            trail_total += trail_flops(m, n)
    kern["trellis_block"] = kernel_line(per("block"), ops_total, round(VALU_PEAK_TOPS, 1), "TOP/s", "valu", 1e12)
    kern["trailing_update"] = kernel_line(per("trailing"), trail_total, MFMA_F64_PEAK_TFLOPS, "TFLOP/s", "mfma", 1e12)
    print(json.dumps({
        "metric": METRIC, "value": round(weights / (ms * 1e-3), 1), "unit": "weights/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16->f32 (Hessian), f64/f32 (sweep)", "data": "synthetic",
        "config": {"workload": f"config 3: Qwen3.5-4B-shaped MLP block, gate/up [9728, 2560] and down [2560, 9728], "
                               f"Hessians from {N} bf16 tokens (10% digit tokens weighted 10x), row plans 2.3 bpw "
                               f"bits 1-4, row trellis L={L}, one factor per stage, packed codes per group",
                   "L": L, "tokens": N, "weights": weights, "setup_s": round(setup_s, 1)},
        "viterbi_row_steps_per_s": round(row_steps_total / (ms * 1e-3), 1),
        "kernels": kern}))


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
    events: dict = {}
    t1 = time.perf_counter()
    for _ in range(args.steps):
        with timed(events, "kl"):
            kl, sums = E.kl_rows(ref, q)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t1) * 1e3 / args.steps
    per = sum(E.event_ms(events, "kl")) / args.steps
    nbytes = 2.0 * T * V * 2 + 4 * T
    print(json.dumps({
        "metric": "KL evaluations/s (per-token KL over paired bf16 logits)", "value": round(1e3 / ms, 2),
        "unit": "evals/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16->f32", "data":
        "synthetic (torch CUDA generator, seeds 401/402; ref ~ N(0, 3^2), q = ref + N(0, 0.3^2))",
        "config": {"workload": "config 4: one KL evaluation over [8192, 151936] bf16 logit pairs per step",
                   "tokens": T, "vocab": V, "mean_kl": float(sums[0] / sums[1])},
        "kernels": {"kl_rows": kernel_line(per, nbytes, HBM_PEAK_GBS, "GB/s", "hbm", 1e9)}}))


def run_c5(args):
    """Config 5: the whole build of a random-initialised Qwen3.5-4B-shaped stack, one build per step."""
    import torch

    from lookatmyquant_amd import stack

    torch.cuda.set_device(0)
    sh = stack.Shape()
    tokens, w = stack.calibration_tokens()
    # warmup: one layer (kernel and GEMM selection, table uploads)
    for _ in range(args.warmup):
        stack.build(tokens, sh, w, L=args.L, layers=1)
    torch.cuda.synchronize()
    timer = stack.Timer()
    t1 = time.perf_counter()
    for _ in range(args.steps):
        out = stack.build(tokens, sh, w, L=args.L, layers=args.layers, timer=timer)
    torch.cuda.synchronize()
    secs = (time.perf_counter() - t1) / args.steps
    assert int(out["bad"].item()) == 0  # every packed row a trellis path from state 0
    weights = out["weights"]
    export = None
    if args.artifact:
        t2 = time.perf_counter()
        receipt = stack.export_codes(out, args.artifact)
        export = {"seconds": round(time.perf_counter() - t2, 2), "total_bytes": receipt["total_bytes"],
                  "tensors": receipt["tensor_count"]}
    print(json.dumps({
        "metric": METRIC, "value": round(weights / secs, 1), "unit": "weights/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(secs * 1e3, 1), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16 (forwards, statistics) / f64 (factor, sweep) / f32 (search)",
        "data": "synthetic (random-initialised stack, token ids uniform over the vocabulary, seed 501)",
        "config": {"workload": f"config 5: end-to-end build of a Qwen3.5-4B-shaped stack, {args.layers} of 36 layers x 7 "
                               "linears, 32 x 2048 calibration tokens through both streams, QEP alpha 0.5, row-plan "
                               f"trellis L={args.L} bits 1-4 at 2.3 bpw, packed codes",
                   "layers": args.layers, "weights": weights, "bits_per_weight": round(out["bits"] / weights, 4),
                   "seconds_per_build": round(secs, 2), "target_seconds": 180,
                   "stages_damped_more": out["redamped"],
                   "seconds_by_phase": {k: round(v / args.steps, 2) for k, v in timer.t.items()},
                   **({"artifact_export": export} if export else {})}}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (default 10; c3 5; c5 1, a whole 36-layer build)")
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed steps first (default 3; c3 and c5 1, for c5 a one-layer build)")
    ap.add_argument("--L", type=int, default=None,
                    help="trellis state bits: default 16 for c2 (the benchmark table), 12 for c3 and c5 (the reference's "
                         "production trellis)")
    ap.add_argument("--k", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--workload", choices=("c2", "c3", "c4", "c5"), default="c2")
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MiB")
    ap.add_argument("--artifact", default=None, metavar="DIR",
                    help="c5: after the timed builds, write the last build's codes as an opgraph-packed-1 artifact "
                         "under DIR (a new directory) and report its size and the seconds it took, outside the "
                         "timed region")
    args = ap.parse_args()
    if args.steps is None:
        args.steps = {"c3": 5, "c5": 1}.get(args.workload, 10)
    if args.warmup is None:
        args.warmup = {"c3": 1, "c5": 1}.get(args.workload, 3)
    if args.L is None:
        args.L = 16 if args.workload == "c2" else 12
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the per-matrix hot path runs on one MI355X here (rows would shard across "
              "GPUs with no communication). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if args.workload == "c3":
        run_c3(args)
    elif args.workload == "c4":
        run_c4(args)
    elif args.workload == "c5":
        run_c5(args)
    else:
        run_c2(args)
    if args.copy_probe:
        copy_probe(args.copy_probe)


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
    if L < E.BIG_L:
        kname = "ldlq_trellis_block_kernel"
    else:  # the minima-exchange kernel up to 2^14 groups, the quarter-window one beyond (L = 16, k = 1)
        kname = "ldlq_trellis_block_gx_kernel" if L - k <= 14 else "ldlq_trellis_block_big_kernel"
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
        "roofline": {"kernel": kname, "bound": "valu", "achieved": round(achieved, 3),
                     "peak": round(VALU_PEAK_TOPS, 1), "unit": "TOP/s", "frac": round(achieved / VALU_PEAK_TOPS, 4),
                     "traffic": MEASURED_TRAFFIC.get((kname, L, k)), "launches_per_step": len(per_block),
                     "avg_launch_us": round(1e3 * sum(blk) / len(blk), 2),
                     "ops_per_row_step": viterbi_ops_per_row_step(L, k)},
        "phase_ms": {"block_kernels": round(blk_ms_step, 4), "trailing_updates": round(sum(trl) / args.steps, 4)},
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(W, H, table, L, k, in_seed)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
