"""The CPU baselines of bench.py: the extrapolation from sampled timings to a whole layer or block is checked with the
timings stubbed, against the sum written out by hand (rows x seconds per row x row-step ratio + the fixed parts);
the KL baseline runs for real on a tiny logit pair."""

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

REPO = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(REPO))

import bench  # noqa: E402

PER_ROW = {1: 0.5, 2: 0.25, 3: 0.125, 4: 2.0}
FIXED = {"stats": 0.3, "rht": 0.01, "cubic": 0.7, "rows": 0.2}


def _stub(monkeypatch):
    calls = []

    def sweep_rows(n, L, k, table, threads, rows_per_thread=1, seed=0):
        calls.append(("rows", n, k, threads))
        return PER_ROW[k] * n / 2560

    def fixed_parts(n, threads, sample_tokens=4096, seed=0, qep=True, m=None):
        calls.append(("fixed", n, threads, qep, m))
        return {p: v * n / 2560 for p, v in FIXED.items()}

    monkeypatch.setattr(bench, "cpu_sweep_rows", sweep_rows)
    monkeypatch.setattr(bench, "cpu_fixed_parts", fixed_parts)
    return calls


def test_c5_extrapolation_is_rows_times_seconds_per_row(monkeypatch):
    from lookatmyquant_amd import engine as E
    from lookatmyquant_amd import stack

    calls = _stub(monkeypatch)
    sh = stack.Shape()
    rp = stack.synthetic_plans(sh, 1)[1]
    shapes = stack.matrix_shapes(sh)
    plans = {nm: rp[f"model.layers.0.{nm}.weight"] for nm in shapes}
    tokens, threads = 65536, 8
    out = bench.cpu_baseline_c5(16, threads, sh, plans, tokens)
    # by hand: each stage's fixed parts from the n = 2,560 figures, each row's sweep from its width's seconds per row
    # carried by trellis row-steps; nothing divided by the thread count (the per-row figure is already wall / rows)
    steps0 = sum(E.trellis_row_steps(2560))
    fixed = sweep = 0.0
    for names in stack.STAGES:
        n = shapes[names[0]][1]
        m = sum(shapes[nm][0] for nm in names)
        r = n / 2560
        fixed += FIXED["stats"] * tokens / 4096 * r * r + FIXED["cubic"] * r ** 3 + FIXED["rows"] * m / 2560 * r * r
        fixed += FIXED["rht"] * r * r
        for nm in names:
            for g in plans[nm]:
                sweep += len(g["rows"]) * PER_ROW[int(g["bits"])] * sum(E.trellis_row_steps(n)) / steps0
    assert out["seconds_per_layer_extrapolated"] == pytest.approx(fixed + sweep, abs=0.01)
    assert out["of_which_sweeps"] == pytest.approx(sweep, abs=0.01)
    weights = sum(m * n for m, n in shapes.values())
    assert out["value"] == pytest.approx(weights / (fixed + sweep), rel=1e-3)
    assert out["cores"] == threads
    assert {c[2] for c in calls if c[0] == "rows"} == {1, 2, 3, 4}


def test_c3_baseline_sums_measured_parts(monkeypatch):
    from lookatmyquant_amd import synthetic

    calls = _stub(monkeypatch)
    plans = {"gate": synthetic.row_plan(9728, 307), "up": synthetic.row_plan(9728, 308),
             "down": synthetic.row_plan(2560, 309)}
    N = 131072
    stage_rows = [(2560, ("gate", "up")), (9728, ("down",))]
    out = bench.cpu_baseline_c3(12, 16, plans, N, stage_rows)
    total = 0.0
    for n, names in stage_rows:
        f = {p: v * n / 2560 for p, v in FIXED.items()}
        total += f["stats"] * N / 4096 + f["rht"] + f["cubic"] + f["rows"]
        for nm in names:
            for g in plans[nm]:
                total += len(g["rows"]) * PER_ROW[int(g["bits"])] * n / 2560
    assert out["seconds_total_extrapolated"] == pytest.approx(total, abs=1e-3)
    assert out["value"] == pytest.approx(3 * 9728 * 2560 / total, rel=1e-3)
    # the fixed parts measured at each stage's own width and row count, without the QEP terms
    assert [c for c in calls if c[0] == "fixed"] == [("fixed", 2560, 16, False, 19456), ("fixed", 9728, 16, False, 2560)]


def test_c4_baseline_runs_on_a_small_pair():
    rng = np.random.default_rng(0)
    ref = torch.from_numpy(rng.standard_normal((64, 1000)).astype(np.float32) * 3).bfloat16()
    q = (ref.float() + 0.3 * torch.from_numpy(rng.standard_normal((64, 1000)).astype(np.float32))).bfloat16()
    out = bench.cpu_baseline_c4(ref, q, 4, 8192, sample_tokens=64)
    assert out["value"] > 0 and out["cores"] == 4 and out["kind"] == "port"
    assert out["seconds_per_eval_extrapolated"] == pytest.approx(1.0 / out["value"], rel=1e-2)
