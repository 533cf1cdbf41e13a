"""The build harness's per-matrix entry points (quantize.py of the reference) on the gfx950 path.

    parse(program)                                                          quantize.py:276-285
    word(program, W, H, seed, trellis, in_seed=None, out_rot=True, G=None)  quantize.py:332-347
    trellis_states(values, table), trellis_code_entry(net, shape, bits, in_seed)    quantize.py:502-527
    quantize_row_groups(target, groups, round_group, in_seed, keep_codes)   quantize.py:530-565
    lamq_codes(values, levels)                                              quantize.py:491-493
    trellis_code(k, T, rows=(16, 8), L=12)                                  quantize.py:588-590
    token_weights_from_kinds(kinds, floor, ceiling, gamma)                  quantize.py:593-629 ("digits")
    cross_target(H, D, alpha, lam)                                          quantize.py:1330-1335
    block_seed(name), matrix_seeds(i, names, j, seed_set, first)            quantize.py:1492-1493, compiler_arch.py:33,75-77
    stage_statistics(...)                                                   quantize.py:1404-1470 (H and the QEP D)
    quantize_stage_row_groups(...)                                          the batched form of quantize_row_groups

quantize_stage_row_groups is the production form of the per-stage loop: every matrix of a stage shares H and the
input rotation, so R_in H R_in^T and U are computed once for all its matrices and row groups (the reference
recomputes them inside every ldlq_words call; the factor is the same) and all rows of one bit width go through
one sweep. The results are those of quantize_row_groups with the trellis word, row for row.
"""

from __future__ import annotations

import re
import zlib

import numpy as np
import torch

from . import codes as C
from . import engine as E
from . import nested as N
from .frame import Dense

PROGRAM = re.compile(r"orig|(rtn|gptq|gptaq|lm|tr|higgs|ter)(\d)(x?)")
LAM = 0.1
KNOWN_BLOCKS = {"linear_attn": 1, "self_attn": 2, "mlp": 3}


def parse(program: str):
    """(family, bits, cross-term target) of a program name (quantize.py:276-285)."""
    if program == "fp16":
        return "fp", 16, False
    if program in ("mean", "prng", "zero"):
        return program, 0, False
    m = PROGRAM.fullmatch(program)
    if not m or (m.group(1) in ("gptaq",) and m.group(3)) or (m.group(1) in ("rtn", "gptq", "higgs") and m.group(3)):
        raise ValueError(f"unknown program {program}")
    return m.group(1), int(m.group(2)), m.group(1) == "gptaq" or m.group(3) == "x"


def trellis_code(k: int, T: int = 256, rows: tuple | None = (16, 8), L: int = 12, values=None):
    """The code of a tr<k> program (quantize.py:588-590): the row trellis (width, look) = rows with --trellis-rows,
    else the column trellis over sequences of T outputs."""
    if rows is None:
        return C.TrellisCode(L, k, T=T, values=values)
    return C.RowTrellisCode(L, k, T=256, width=rows[0], look=rows[1], values=values)


def word(program, W, H, seed, trellis, in_seed=None, out_rot=True, G=None):
    """One matrix's quantized word for its target W and input statistics H (quantize.py:332-347): lm<b> and ter<b>
    are one-rate nested words on Lloyd-Max levels, tr<b> the trellis code trellis[b], fp16 the bf16 values."""
    fam, b, _ = parse(program)
    if fam == "fp":
        return Dense(torch.as_tensor(W).to(torch.bfloat16).double(), 16 * W.numel())
    if fam == "lm":
        return N.nested_words([W], H, [seed], b, [b], 0.4, [1.0], N.lloyd_max(b), in_seed=in_seed, out_rot=out_rot, G=G)[b][0]
    if fam == "ter":
        return N.nested_words([W], H, [seed], 2, [2], 0.4, [1.0], N.lloyd_max_levels(b), in_seed=in_seed, out_rot=out_rot)[2][0]
    if fam == "tr":
        return C.ldlq_words([W], H, trellis[b], [seed], in_seed=in_seed, out_rot=out_rot)[0]
    raise NotImplementedError(f"program family {fam!r} is not part of this path")


def lamq_codes(values: torch.Tensor, levels: torch.Tensor) -> torch.Tensor:
    """The index of the nearest level for each value (quantize.py:491-493)."""
    levels = torch.as_tensor(levels, dtype=torch.float64)
    return torch.searchsorted(((levels[1:] + levels[:-1]) / 2).contiguous(), torch.as_tensor(values).double().contiguous())


def trellis_states(values: torch.Tensor, table: torch.Tensor) -> torch.Tensor:
    """Each entry's state: the index of its value in the table (quantize.py:502-510). Ambiguous for tables with
    repeated values; words built here carry their states (net.codes) instead."""
    t = torch.as_tensor(table).double().flatten()
    st, order = t.sort()
    v = torch.as_tensor(values).double().contiguous()
    pos = torch.searchsorted(st, v).clamp(1, len(st) - 1)
    pos = torch.where((v - st[pos - 1]).abs() <= (st[pos] - v).abs(), pos - 1, pos)
    assert float((st[pos] - v).abs().max()) < 1e-9, "a trellis value not in its table"
    return order[pos].to(torch.int16)


def trellis_code_entry(net, shape, bits, in_seed):
    """A one-sided row-trellis word in the saved codes format (quantize.py:513-527): int16 states, f32 row scales,
    the input seed, the f32 table and one row group."""
    if in_seed is None or "I[u]" in net.cores:
        raise ValueError("saved trellis codes require an input-only rotation with a recorded seed")
    core = net.cores["W"]
    table = torch.as_tensor(core.domain.levels, dtype=torch.float64)
    if len(table) != 4096:
        raise ValueError("saved row-group codes require a 12-bit state table")
    states = net.codes.reshape(shape).to(torch.int16) if getattr(net, "codes", None) is not None else \
        trellis_states(core.data.reshape(shape), table)
    entry = {"states": states, "scales": net.cores["W.S"].data.float().flatten(), "in_seed": int(in_seed),
             "table": table.float(), "trellis_layout": "row" if core.domain.fixed_start else "column"}
    if core.domain.fixed_start:
        entry["row_groups"] = [{"rows": torch.arange(shape[0], dtype=torch.long), "bits": int(bits), "table_index": 0}]
    return entry


def quantize_row_groups(target, groups, round_group, in_seed, keep_codes):
    """Apply validated original-row groups (quantize.py:530-565): one to eight non-empty groups of widths 1-4 that
    cover every row exactly once; each group is round_group(rows, bits), a word; returns (W_hat, bits, entry)."""
    groups = [(torch.as_tensor(g["rows"], dtype=torch.long), int(g["bits"])) for g in groups]
    if not groups or len(groups) > 8 or any(not len(rows) or bits not in (1, 2, 3, 4) for rows, bits in groups):
        raise ValueError("row groups need one to eight nonempty groups at widths 1–4")
    all_rows = torch.cat([rows for rows, _ in groups])
    if not torch.equal(all_rows.sort().values, torch.arange(target.shape[0])):
        raise ValueError("row groups must cover every matrix row exactly once")
    Wq, rate = torch.empty(target.shape, dtype=torch.float64), 0.0
    states = torch.empty(target.shape, dtype=torch.int16) if keep_codes else None
    scales = torch.empty(target.shape[0], dtype=torch.float32) if keep_codes else None
    tables, saved_groups, layouts = [], [], set()
    for rows, bits in groups:
        net = round_group(rows, bits)
        Wq[rows] = net.matrix(dtype=torch.float64)
        rate += net.rate_bits()
        if keep_codes:
            entry = trellis_code_entry(net, (len(rows), target.shape[1]), bits, in_seed)
            table_index = len(tables)
            states[rows] = entry["states"] + table_index * 4096
            scales[rows] = entry["scales"]
            tables.append(entry["table"])
            layouts.add(entry["trellis_layout"])
            saved_groups.append({"rows": rows.clone(), "bits": bits, "table_index": table_index})
    if not keep_codes:
        return Wq, rate, None
    if len(layouts) != 1:
        raise ValueError("mixed trellis layouts are not a saved row-group representation")
    return Wq, rate, {"states": states, "scales": scales, "in_seed": int(in_seed), "table": torch.cat(tables),
                      "row_groups": saved_groups, "trellis_layout": next(iter(layouts))}


# ----------------------------------------------------------------------------- seeds, weights and statistics


def block_seed(path: str) -> int:
    """compiler_arch.block_seed (compiler_arch.py:75-77): the known blocks' fixed seeds, else 4 + crc32 % 5."""
    head = path.split(".")[0]
    return KNOWN_BLOCKS.get(head, 4 + zlib.crc32(head.encode()) % 5)


def matrix_seeds(layer: int, name: str, j: int, first: str, seed_set: int = 0, stage_j: int = 0):
    """(seed, in_seed) of a matrix (quantize.py:1492-1493 with --rot in-shared)."""
    shift = 100000 * seed_set
    seed = 1000 * layer + 100 * block_seed(name) + j + stage_j + shift
    in_seed = 1000 * layer + 100 * block_seed(first) + 1 + shift
    return seed, in_seed


def token_weights_from_kinds(kinds: torch.Tensor, floor: float = 0.1, ceiling: float = 100.0, gamma: float = 1.0):
    """Per-token weights of the "digits" rule (quantize.py:593-629) from the token kinds of the next position
    (0: a digit of a computed result, 1: another digit, else other; the last position of a window has none):
    2 / 1 / 0, over their mean, raised to gamma, kept within [floor, ceiling] times the mean, mean 1, float32."""
    k = torch.as_tensor(kinds)
    v = torch.zeros(k.shape, dtype=torch.float64)
    v[..., :-1] = 2.0 * (k[..., :-1] == 0) + 1.0 * (k[..., :-1] == 1)
    w = (v / v.mean()).clamp(min=1e-9) ** gamma
    w = (w / w.mean()).clamp(floor, ceiling)
    return (w / w.mean()).float()


def cross_target(H: torch.Tensor, D: torch.Tensor, alpha: float, lam: float = LAM) -> torch.Tensor:
    """M = I + alpha ((H + lam mean(diag H) I)^-1 D^T)^T (quantize.py:1330-1335), D = X_ref^T X_q / N - H. The
    damped H is symmetric positive definite, so the solve is the Cholesky solve of lamq_chol_inv_upper's factor:
    (H + d I)^-1 = U^T U. Returned on the CPU in float64."""
    return cross_map(H, D, alpha, lam).cpu()


def qep_factor(H: torch.Tensor, lam: float = LAM, timer: E.KernelTimer | None = None) -> tuple:
    """(U, info): the upper Cholesky factor of (H + lam mean(diag H) I)^-1, the QEP solve's factor, and the failing
    pivot as a device value (0 when positive definite; no host synchronisation), for a caller that checks info
    itself later. timer: span "chol" (4n^3/3 flops)."""
    dev = E._abi.device()
    Hg = torch.as_tensor(H).to(dev, torch.float64).contiguous()
    n = Hg.shape[0]
    with E.span(timer, "chol", 4.0 * n ** 3 / 3):
        _, U, _, info = E.chol_inv_upper(Hg, damp=lam, raise_on_fail=False)
    return U, info


def qep_check(info: torch.Tensor) -> None:
    """Raises LinAlgError, as the factorization does, when qep_factor's info names a failing pivot (one host
    synchronisation)."""
    bad = int(info.item())
    if bad:
        raise E.LinAlgError(f"linalg.cholesky: the leading minor of order {bad} is not positive-definite")


def _qep_u(H: torch.Tensor, lam: float, timer, U: torch.Tensor | None) -> torch.Tensor:
    """U as given (from qep_factor, its info checked by the caller), else the factor here, checked at once."""
    if U is not None:
        return U
    U, info = qep_factor(H, lam, timer)
    qep_check(info)
    return U


def cross_map(H: torch.Tensor, D: torch.Tensor, alpha: float, lam: float = LAM,
              timer: E.KernelTimer | None = None, U: torch.Tensor | None = None) -> torch.Tensor:
    """cross_target's M, float64 on the GPU. U: qep_factor(H, lam)[0], if the caller has it already. timer: spans
    "chol" (4n^3/3 flops) and "qep_gemm" (the products: 2 M N K flops for a full one, M N K for a triangular one)."""
    dev = E._abi.device()
    Dg = torch.as_tensor(D).to(dev, torch.float64).contiguous()
    n = Dg.shape[0]
    U = _qep_u(H, lam, timer, U)
    # (H + d I)^-1 = U^T U, so M = I + alpha ((H + d I)^-1 D^T)^T = I + alpha D U^T U: two triangular products
    with E.span(timer, "qep_gemm", 2.0 * n ** 3):
        P = torch.zeros(n, n, dtype=torch.float64, device=dev)
        E.gemm_sub(P, alpha * Dg, U, transb=True, tri=1)  # P = -alpha D U^T
        M = torch.eye(n, dtype=torch.float64, device=dev)
        return E.gemm_sub(M, P, U, tri=2)  # M = I + alpha D U^T U


def _product(A: torch.Tensor, B: torch.Tensor, scale: float = 1.0) -> torch.Tensor:
    """scale * A @ B on the fp64 MFMA GEMM (lamq_gemm_sub_f64 from a zero C: 0 - (-scale A) B, exact negations, so
    the products are summed once, as a plain product sums them)."""
    C = torch.zeros(A.shape[0], B.shape[1], dtype=torch.float64, device=A.device)
    return E.gemm_sub(C, (-scale * A).contiguous(), B.contiguous())


def qep_targets(H: torch.Tensor, D: torch.Tensor, alpha: float, Ws: dict, lam: float = LAM,
                timer: E.KernelTimer | None = None, U: torch.Tensor | None = None) -> dict:
    """W* = W M for every matrix of a stage (quantize.py:1505), M = cross_target(H, D, alpha, lam), float64 on the
    GPU. When the stage has fewer rows than inputs M is not formed: W M = W + alpha (W D) (H + d I)^-1 =
    W + alpha (W D) U^T U, one product and two triangular ones (4 m n^2 flops against 2 n^3 + 2 m n^2).
    U: qep_factor(H, lam)[0], if the caller has made it (and checks its info itself)."""
    dev = E._abi.device()
    n = H.shape[0]
    Wg = {nm: torch.as_tensor(W).to(dev, torch.float64) for nm, W in Ws.items()}
    m = sum(W.shape[0] for W in Wg.values())
    if m >= n:
        M = cross_map(H, D, alpha, lam, timer, U)
        with E.span(timer, "qep_gemm", 2.0 * m * n * n):
            return {nm: _product(W, M) for nm, W in Wg.items()}
    Dg = torch.as_tensor(D).to(dev, torch.float64).contiguous()
    U = _qep_u(H, lam, timer, U)
    out = {}
    with E.span(timer, "qep_gemm", 4.0 * m * n * n):
        for nm, W in Wg.items():
            Z = _product(W, Dg, alpha)
            P = torch.zeros(W.shape[0], n, dtype=torch.float64, device=dev)
            E.gemm_sub(P, Z, U, transb=True, tri=1)  # P = -alpha W D U^T
            out[nm] = E.gemm_sub(W.contiguous().clone(), P, U, tri=2)  # W + alpha W D U^T U
    return out


def stage_statistics(Xq_chunks, w_chunks=None, Xr_chunks=None):
    """H = (1/N) sum_t w_t x_t x_t^T and, for a cross-term stage, D = (1/N) sum_t w_t x_ref,t x_q,t^T, from bf16
    activation chunks [tokens, n] on the GPU (quantize.py:1416-1470). Returns float64 (H, D or None)."""
    dev = E._abi.device()
    n = Xq_chunks[0].shape[-1]
    H = torch.zeros(n, n, dtype=torch.float32, device=dev)
    D = torch.zeros(n, n, dtype=torch.float32, device=dev) if Xr_chunks is not None else None
    ntok = 0
    for c, xq in enumerate(Xq_chunks):
        xq = xq.reshape(-1, n).to(dev, torch.bfloat16).contiguous()
        w = None if w_chunks is None else w_chunks[c].reshape(-1).to(dev, torch.float32)
        E.hessian_accum(H, xq, w)
        if D is not None:
            xr = Xr_chunks[c].reshape(-1, n).to(dev, torch.bfloat16).contiguous()
            E.cross_gram_accum(D, xr, xq, w)
        ntok += xq.shape[0]
    H64 = E.hessian_finalize(H, float(ntok))
    D64 = None if D is None else (D / ntok).double()
    return H64, D64


# ----------------------------------------------------------------------------- the batched stage path


def stage_factor(H: torch.Tensor, in_seed: int, damp: float = 0.01, timer: E.KernelTimer | None = None):
    """The stage's factor as quantize_stage_row_groups makes it: (U, dead, info) of the rotated, damped H (no host
    synchronisation: info is a device value, 0 when positive definite). timer: spans "rht" (R H R^T: two
    passes of rht_rows, 2n(a + b) flops a row, and a transpose) and "chol" (4n^3/3 flops)."""
    dev = E._abi.device()
    Hg = torch.as_tensor(H).to(dev, torch.float64).contiguous()
    n = Hg.shape[0]
    with E.span(timer, "rht", 2.0 * E.rht_flops(n, n)):
        Hr = E.rotate_hessian(Hg, in_seed)
    with E.span(timer, "chol", 4.0 * n ** 3 / 3):
        _, U, dead, info = E.chol_inv_upper(Hr, damp=damp, raise_on_fail=False)
    return U, dead, info


def quantize_stage_row_groups(targets: dict, groups: dict, H: torch.Tensor, in_seed: int, L: int = 12,
                              width: int = 16, look: int = 8, tables: dict | None = None, events: dict | None = None,
                              chol_events: tuple | None = None, damp: float = 0.01, factor: tuple | None = None,
                              timer: E.KernelTimer | None = None, check: bool = True):
    """Every matrix of a stage, row group by row group, with the row trellis at the group's width: the same result
    as quantize_row_groups(target, groups, round_group) with round_group = the tr<bits> word of (target[rows], H,
    in_seed, out_rot=False), for each matrix. targets: {name: W [m, n]}; groups: {name: [{"rows", "bits"}]};
    tables: {bits: float64 table} (default: the cached L = 12 tables). Returns {name: (states int32 [m, n] on the
    GPU, S float64 [m] on the GPU)}; the codes entries and reconstructions follow from them. events / chol_events
    ((dict, key)): torch.cuda.Event pairs around the sweep kernels / the factorization, for timing. damp: the
    Environment's damping fraction (frame.py:521). factor: stage_factor(H, in_seed, damp), if the caller has made it
    already (for instance on another stream, next to other work); a non-positive-definite factor raises (with
    check=False the caller checks the factor's info itself, after the sweep is enqueued: no host synchronisation
    here, the results then to be discarded if it failed). timer: an
    engine.KernelTimer; every launch of the sweep is timed on this stream (one stream for all groups) under "block" and
    "trailing", the row rotations under "rht" (2n(a + b) flops a row), and the factor as in stage_factor."""
    names = list(targets)
    stage_tables = {}  # the table of each width, resolved before any device work
    for bits in sorted({int(g["bits"]) for nm in names for g in groups[nm]}):
        table = (tables or {}).get(bits)
        if table is None:
            if L != 12:
                raise ValueError(f"no trellis table given for {bits} bits at L = {L}: only the 12-bit tables are cached")
            table = C.load_table(12, bits)
        table = table if isinstance(table, torch.Tensor) else torch.from_numpy(np.array(table, dtype=np.float64))
        stage_tables[bits] = table.to(torch.float64)
    dev = E._abi.device()
    if timer is not None:
        events = timer.events
    if factor is None and timer is not None:
        factor = stage_factor(H, in_seed, damp, timer)
    if factor is not None:
        U, dead, info = factor
        if check and int(info.item()):
            raise E.LinAlgError(f"linalg.cholesky: the leading minor of order {int(info.item())} is not positive-definite")
    else:
        Hr = E.rotate_hessian(torch.as_tensor(H).to(dev, torch.float64).contiguous(), in_seed)
        ev = None
        if chol_events is not None:
            ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            ev[0].record()
        _, U, dead, info = E.chol_inv_upper(Hr, damp=damp, raise_on_fail=chol_events is None)
        if ev is not None:
            ev[1].record()
            chol_events[0].setdefault(chol_events[1], []).append(ev)
            if int(info.item()):
                raise E.LinAlgError(f"linalg.cholesky: the leading minor of order {int(info.item())} is not "
                                    "positive-definite")
    X_all, S_all = {}, {}
    for nm in names:
        W = torch.as_tensor(targets[nm]).to(dev, torch.float64).contiguous()
        with E.span(timer, "rht", E.rht_flops(W.shape[0], W.shape[1])):
            X_all[nm], S_all[nm] = E.rht_rows(W, in_seed, want_rms=True)
    # rows of one width across the stage's matrices go through one sweep
    by_bits: dict = {}
    for nm in names:
        for g, r in zip(groups[nm], E.device_rows(groups[nm], dev)):
            by_bits.setdefault(int(g["bits"]), []).append((nm, r))
    # all of the stage's rows go through one sweep: the block kernel runs width by width on consecutive row
    # groups, and each trailing update covers every row at once
    out = {nm: torch.empty(X_all[nm].shape, dtype=torch.int32, device=dev) for nm in names}
    idx, sweep_groups = [], []
    for bits, parts in sorted(by_bits.items()):
        table = stage_tables[bits]
        rows = 0
        for nm, r in parts:
            idx.append((nm, r))
            rows += len(r)
        sweep_groups.append((rows, bits, table.to(dev), None))
    X = torch.cat([X_all[nm].index_select(0, r) for nm, r in idx])
    S = torch.cat([S_all[nm].index_select(0, r) for nm, r in idx])
    st = E.ldlq_trellis_groups(X, S, U, sweep_groups, L, width, look, 128, dead=dead, events=events)
    r0 = 0
    for nm, r in idx:
        out[nm].index_copy_(0, r, st[r0 : r0 + len(r)])
        r0 += len(r)
    return {nm: (out[nm], S_all[nm]) for nm in names}


# ----------------------------------------------------------------------------- the command line


def main(argv=None):
    """quantize.py --program plan|<program> [--plan P.json] [--row-plan R.json] ... (quantize.py:923-989), on the
    random-initialised Qwen3.5-4B-shaped stack (hidden 2560, GQA 32/8 x 128, MLP 9728; model loading and the text
    data are not part of this path): synthetic calibration token ids, the stage statistics, QEP targets, codes and
    packed codes on the GPU. Writes a summary JSON (--out), the reference's --save-codes dictionary, and with
    --artifact an opgraph-packed-1 artifact."""
    import argparse
    import json
    import time
    from pathlib import Path

    from . import stack
    from .rowplan import load_row_plan

    ap = argparse.ArgumentParser(prog="python -m lookatmyquant_amd.quantize")
    ap.add_argument("--program", required=True, help="plan, or one program for every linear: tr3x, lm6x, fp16, ...")
    ap.add_argument("--plan", default="", help="with --program plan: a plan JSON ({\"linears\": {\"i.name\": program}})")
    ap.add_argument("--row-plan", default="", help="rowgroup-plan-1 JSON: original row ids and widths by full parameter "
                                                   "name; requires --rot in-shared and --trellis-rows")
    ap.add_argument("--trellis-rows", default="16,8", help="width,look of the row trellis (quantize.py's --trellis-rows): width 1-16 dividing 128, width + look <= 24")
    ap.add_argument("--rot", choices=["in-shared"], default="in-shared",
                    help="one input rotation per stage, none on the output (the only rotation of this path)")
    ap.add_argument("--cross-alpha", type=float, default=1.0, help="QEP's alpha for cross-term programs")
    ap.add_argument("--lam", type=float, default=LAM, help="the cross term's ridge penalty")
    ap.add_argument("--layers", type=int, default=0, help="quantize only the first n layers; 0 = all 36")
    ap.add_argument("--calib", type=int, default=32, help="calibration windows")
    ap.add_argument("--calib-len", type=int, default=2048)
    ap.add_argument("--chunk", type=int, default=32, help="sequences per calibration forward")
    ap.add_argument("--token-weights", choices=["", "digits"], default="digits",
                    help="digits: a random 10%% of tokens weighted 10x (normalised to mean 1), the synthetic stand-in "
                         "for the digit weights of quantize.py:593-629")
    ap.add_argument("--seed-set", type=int, default=0, help="moves every randomized Hadamard seed")
    ap.add_argument("--state-bits", type=int, choices=[12, 16], default=12,
                    help="trellis state bits: 12, the reference's fitted tables; 16, the fp16 Gaussian-quantile table")
    ap.add_argument("--redamp", action="store_true", help="damp a stage x10, x100 when its statistics are not positive "
                                                          "definite (ldlq_gpu.py:19-23) instead of raising")
    ap.add_argument("--save-codes", default="", help="write the codes, scales, tables and row groups here (torch.save)")
    ap.add_argument("--artifact", default="", help="write the codes as an opgraph-packed-1 artifact in this new directory")
    ap.add_argument("--out", required=True)
    args = ap.parse_args(argv)
    try:
        window = tuple(int(v) for v in args.trellis_rows.split(","))
    except ValueError:
        window = ()
    if len(window) != 2:
        ap.error("--trellis-rows takes width,look")
    stack.trellis_window(window)
    if not 1 <= args.calib_len <= 0x7FFFFF:
        raise NotImplementedError("the forwards' fused attention takes sequence lengths of 1 to 8388607 tokens")
    sh = stack.Shape()
    layers = args.layers or sh.layers
    if args.program == "plan":
        if not args.plan:
            ap.error("--program plan needs --plan")
        plan = json.loads(Path(args.plan).read_text())
    else:
        parse(args.program)
        plan = {"linears": {f"{i}.{nm}": args.program for i in range(layers) for nm in stack.matrix_shapes(sh)}}
    row_plan, manifest = {}, None
    if args.row_plan:
        row_plan, manifest = load_row_plan(args.row_plan, stack.active_shapes(sh, plan, layers))
    tokens, w = stack.calibration_tokens(args.calib, args.calib_len, sh.vocab)
    torch.cuda.set_device(0)
    t0 = time.perf_counter()
    timer = stack.Timer()
    out = stack.build(tokens, sh, w if args.token_weights else None, alpha=args.cross_alpha, L=args.state_bits,
                      plan=plan, row_plan=row_plan, chunk=args.chunk, layers=layers, timer=timer, redamp=args.redamp,
                      lam=args.lam, seed_set=args.seed_set, window=window)
    torch.cuda.synchronize()
    secs = time.perf_counter() - t0
    res = {"program": args.program, "layers": layers, "weights": out["weights"],
           "bits per weight": out["bits"] / out["weights"], "quantize seconds": round(secs, 2),
           "seconds per layer": round(secs / layers, 3), "seconds by phase": {k: round(v, 2) for k, v in timer.t.items()},
           "stages damped more": out["redamped"], "row plan": manifest}
    if args.save_codes:
        Path(args.save_codes).parent.mkdir(parents=True, exist_ok=True)
        calibration = {"windows": args.calib, "tokens per window": args.calib_len,
                       "token weights": args.token_weights or "none"}
        torch.save(stack.saved_codes(out, manifest if args.row_plan else None, calibration), args.save_codes)
    if args.artifact:
        res["artifact"] = {k: v for k, v in stack.export_codes(out, args.artifact).items()
                           if k in ("total_bytes", "tensor_count", "all_tensor_bytes_verified")}
    Path(args.out).parent.mkdir(parents=True, exist_ok=True)
    Path(args.out).write_text(json.dumps(res, indent=1))
    print(json.dumps(res))


if __name__ == "__main__":
    main()
