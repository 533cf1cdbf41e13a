"""Host-side logic of the product, CPU only: the C ABI library loads and binds every symbol include/lamq.h
declares (no compute calls), the host tables (Hadamard factors, rotation signs, Lloyd-Max levels) equal the
reference's, and the plan/row-plan/program validation behaves like the reference's."""

import ctypes
import json
import re
import subprocess
import sys

import numpy as np
import pytest
import torch

from conftest import REPO


def declared_symbols():
    text = (REPO / "include" / "lamq.h").read_text()
    return sorted(set(re.findall(r"^(?:int|size_t)\s+(lamq_\w+)\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    from lookatmyquant_amd import _abi

    names = declared_symbols()
    assert len(names) >= 20
    assert sorted(_abi.SIGNATURES) == names, "the ctypes bindings must be exactly the header's declarations"
    lib = _abi.lib()  # loads the gfx950 library; binding fails on a missing symbol
    for n in names:
        assert hasattr(lib, n)
    assert lib.lamq_abi_version() == 101


def test_library_symbols_are_c_abi():
    so = REPO / "lookatmyquant_amd" / "liblamq_hip.so"
    out = subprocess.run(["nm", "-D", "--defined-only", str(so)], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r" T (lamq_\w+)$", out, flags=re.M))
    assert set(declared_symbols()) <= exported


def test_argument_errors_are_reported_without_a_gpu():
    """Entry points validate their arguments before touching a device: NULL pointers and bad shapes return
    LAMQ_EINVAL, unsupported parameters LAMQ_EUNSUP."""
    from lookatmyquant_amd import _abi

    L = _abi.lib()
    assert L.lamq_viterbi_rows(None, 4, 8, 8, None, 12, 2, None, None, 8, None, 0, None) == -1
    assert L.lamq_trailing_update_f64(None, 1, 1, 1, None, 1, None, 1, 0, 1, None) == -1
    assert L.lamq_kl_rows(None, None, 1, 1, 1, 1, None, None, None, None, 0, None) == -1
    p = torch.empty(64, dtype=torch.float64)
    q = torch.empty(64, dtype=torch.int32)
    ptr = lambda t: t.data_ptr()
    # width + look beyond the fused search's limit: unsupported, not a crash
    assert L.lamq_ldlq_trellis_block(ptr(p), 1, 8, 8, ptr(p), 8, ptr(p), ptr(p), ptr(p), 12, 2, 0, 8, 30, 8, ptr(q), ptr(q),
                                     8, ptr(p), 8, 0, None) == -2
    # earlier run columns beyond the block's start, or a Z too narrow to hold them
    assert L.lamq_ldlq_trellis_block(ptr(p), 1, 8, 8, ptr(p), 8, ptr(p), ptr(p), ptr(p), 12, 2, 0, 8, 4, 4, ptr(q), ptr(q),
                                     8, ptr(p), 8, 1, None) == -1
    # row groups in one launch: overlapping rows, rows past m, a width the 16-bit trellis lacks, k = 1 at L = 16
    # without the workspace its back-pointers need, too many groups
    from ctypes import addressof

    def groups(*gs):
        arr = (_abi.TrellisGroup * len(gs))()
        for i, (r0, rows, k, wsb) in enumerate(gs):
            arr[i] = _abi.TrellisGroup(r0, rows, k, ptr(p), ptr(q), ptr(p) if wsb else None, wsb)
        return arr

    def call(arr, count=None, Lbits=16):
        return L.lamq_ldlq_trellis16_block_groups(ptr(p), 8, 8, 8, ptr(p), 8, ptr(p), Lbits, addressof(arr),
                                                  len(arr) if count is None else count, 0, 8, 4, 4, ptr(q), ptr(q), 8,
                                                  ptr(p), 8, 0, None)

    assert call(groups((0, 5, 2, 0), (4, 4, 3, 0))) == -1
    assert call(groups((0, 5, 2, 0), (5, 4, 3, 0))) == -1
    assert call(groups((0, 4, 5, 0))) == -2
    assert call(groups((0, 4, 3, 0)), Lbits=14) == -2
    assert call(groups((0, 4, 1, 0))) == -1
    assert call(groups((0, 4, 1, 8)), count=0) == -1
    assert call(groups(*[(i, 1, 2, 0) for i in range(9)])) == -1
    # the fused causal softmax: a length not a multiple of 8 or past 4096, a short stride, a bad scale, overlapping
    # output, a misaligned pointer
    b = torch.empty(4096, dtype=torch.int16)
    assert L.lamq_causal_softmax_bf16(ptr(b), ptr(b), 4, 12, 16, 16, 0.5, None) == -2
    assert L.lamq_causal_softmax_bf16(ptr(b), ptr(b), 1, 4104, 4104, 4104, 0.5, None) == -2
    assert L.lamq_causal_softmax_bf16(ptr(b), ptr(b), 4, 16, 8, 16, 0.5, None) == -1
    assert L.lamq_causal_softmax_bf16(ptr(b), ptr(b), 4, 16, 16, 16, 0.0, None) == -1
    assert L.lamq_causal_softmax_bf16(ptr(b), ptr(b) + 16, 4, 16, 16, 16, 0.5, None) == -1
    assert L.lamq_causal_softmax_bf16(ptr(b) + 2, ptr(b) + 2, 4, 16, 16, 16, 0.5, None) == -1
    # the multi-rate sweep: more than four rates, no levels, a refit without Z
    assert L.lamq_ldlq_multirate_block(ptr(p), 1, 8, 8, ptr(p), 8, ptr(p), 5, 2, ptr(p), 0, 8, ptr(q), 8, ptr(p), 8,
                                       None) == -2
    assert L.lamq_ldlq_multirate_block(ptr(p), 1, 8, 8, ptr(p), 8, ptr(p), 2, 0, ptr(p), 0, 8, ptr(q), 8, ptr(p), 8,
                                       None) == -1
    assert L.lamq_ldlq_multirate_block(ptr(p), 1, 8, 8, ptr(p), 8, ptr(p), 2, 4, ptr(p), 0, 8, ptr(q), 8, None, 8,
                                       None) == -1
    assert L.lamq_ldlq_trellis16_block(ptr(p), 1, 8, 8, ptr(p), 8, ptr(p), ptr(p), ptr(p), 16, 2, 4, 8, 4, 4, ptr(q),
                                       ptr(q), 8, ptr(p), 4, 4, None) == -1
    # widths past the reference's uint8 back-pointers, or more states than the wide search holds, are unsupported; a
    # wide search (k = 5..8) keeps a byte per group and position in its workspace and refuses to run without it
    assert L.lamq_viterbi_rows(ptr(p), 1, 4, 4, ptr(p), 12, 9, None, ptr(q), 4, None, 0, None) == -2
    assert L.lamq_viterbi_rows(ptr(p), 1, 4, 4, ptr(p), 15, 5, None, ptr(q), 4, None, 0, None) == -2
    assert L.lamq_viterbi_rows(ptr(p), 1, 4, 4, ptr(p), 12, 7, None, ptr(q), 4, None, 0, None) == -1
    assert L.lamq_viterbi_workspace_size(3, 10, 12, 7) == 3 * 10 * 32
    assert L.lamq_viterbi_workspace_size(3, 10, 5, 5) == 3 * 10
    assert L.lamq_viterbi_workspace_size(3, 10, 12, 2) == 0
    # packing: widths beyond 8, a trellis no wider than its symbols, too few code words, more rows than the source
    assert L.lamq_pack_codes(ptr(q), 8, 8, None, 8, 8, 0, 9, 12, 1, ptr(q), 8, ptr(q), None) == -1
    assert L.lamq_pack_codes(ptr(q), 8, 8, None, 8, 8, 0, 4, 4, 1, ptr(q), 8, ptr(q), None) == -1
    assert L.lamq_pack_codes(ptr(q), 8, 8, None, 8, 8, 0, 4, 12, 0, ptr(q), 3, ptr(q), None) == -1
    assert L.lamq_pack_codes(ptr(q), 8, 4, None, 8, 8, 0, 2, 12, 1, ptr(q), 8, ptr(q), None) == -1
    assert L.lamq_pack_codes(None, 8, 8, None, 8, 8, 0, 2, 12, 1, ptr(q), 8, ptr(q), None) == -1
    # many groups at once: each entry is checked as lamq_pack_codes checks its arguments, before any launch (the
    # valid first entry is not packed when a later one is refused)
    good = dict(src=ptr(q), ld=8, src_rows=8, rows=None, m=8, base=0, k=2, codes=ptr(q), ldc=8)
    for bad_fields in ({"k": 9}, {"k": 12}, {"ldc": 1}, {"src_rows": 4}, {"src": None}, {"codes": None}, {"ld": 4},
                       {"m": -1}):
        descs = (_abi.PackGroup * 2)(_abi.PackGroup(**good), _abi.PackGroup(**dict(good, **bad_fields)))
        assert L.lamq_pack_codes_groups(ctypes.addressof(descs), 2, 8, 12, 1, ptr(q), None) == -1, bad_fields
    assert L.lamq_pack_codes_groups(None, 1, 8, 12, 1, ptr(q), None) == -1
    descs = (_abi.PackGroup * 1)(_abi.PackGroup(**good))
    assert L.lamq_pack_codes_groups(ctypes.addressof(descs), 1, 8, 12, 1, None, None) == -1
    assert L.lamq_pack_codes_groups(ctypes.addressof(descs), 1, 0, 12, 1, ptr(q), None) == -1
    assert L.lamq_pack_codes_groups(ctypes.addressof(descs), -1, 8, 12, 1, ptr(q), None) == -1
    # output shaping: the packed feedback's size (blocks of 32 rows over 100: 32 x (68 + 36 + 4) doubles), a block
    # past 64 or a column past LDS unsupported, missing arrays invalid
    assert L.lamq_shaping_feedback_size(100, 32) == 32 * (68 + 36 + 4) * 8
    assert L.lamq_shaping_feedback_size(30, 32) == 0
    assert L.lamq_shaping_feedback(None, 100, 100, 32, ptr(p), None) == -1
    assert L.lamq_shaping_feedback(ptr(p), 100, 100, 65, ptr(p), None) == -2
    assert L.lamq_ldlq_shaped_column(None, 8, 8, 8, 0, ptr(p), 4, ptr(p), 4, ptr(q), 8, ptr(p), None) == -1
    assert L.lamq_ldlq_shaped_column(ptr(p), 8, 8, 8, 8, ptr(p), 4, ptr(p), 4, ptr(q), 8, ptr(p), None) == -1
    assert L.lamq_ldlq_shaped_column(ptr(p), 20000, 8, 8, 0, ptr(p), 4, ptr(p), 4, ptr(q), 8, ptr(p), None) == -2
    assert L.lamq_ldlq_shaped_column(ptr(p), 8, 8, 8, 0, ptr(p), 4, ptr(p), 300, ptr(q), 8, ptr(p), None) == -2
    assert L.lamq_chol_inv_upper_workspace_size(10) >= 800
    assert L.lamq_viterbi_workspace_size(3, 100, 12, 2) == 3 * 100 * 256
    # the fused 16-bit-state search keeps its back-pointers (23 steps x 1024 words a row) in a workspace where LDS
    # cannot hold them (k = 1, 2^15 groups) or where the LDS they would take holds a second buffer of group minima
    # instead (k = 2, 2^14 groups); k = 3, 4 keep them in LDS
    for k, words in ((1, 23 * 1024), (2, 23 * 1024), (3, 0), (4, 0)):
        assert L.lamq_ldlq_trellis16_block_workspace_size(5, 16, k) == 5 * 4 * words
    assert L.lamq_ldlq_trellis16_block_workspace_size(5, 15, 1) == 5 * 4 * 23 * 1024
    assert L.lamq_ldlq_trellis16_block_workspace_size(5, 14, 1) == 0


def test_hadamard_factors_and_signs_equal_the_reference(golden):
    from lookatmyquant_amd import hadamard as Hd

    g = golden("misc")
    for n in (960, 2560, 4096, 9728):
        A, B = Hd.hadamard_factors(n)
        assert np.array_equal(A.numpy().astype(np.int8), g[f"had_{n}_A"])
        assert np.array_equal(B.numpy().astype(np.int8), g[f"had_{n}_B"])
    for n, s in ((960, 201), (2560, 1301), (9728, 3301)):
        assert np.array_equal(Hd.rht_signs(n, s).numpy().astype(np.int8), g[f"signs_{n}_{s}"])
    for n in (2, 12, 20, 64, 1024):
        H = Hd.hadamard(n)
        assert float((H @ H.T - torch.eye(n, dtype=torch.float64)).abs().max()) < 1e-12


def test_lloyd_max_levels_equal_the_reference_bits(golden):
    from lookatmyquant_amd import nested as N

    for b in (1, 2, 3, 4):
        assert np.array_equal(N.lloyd_max(b).numpy(), golden("misc")[f"lloyd_max_{b}"])


def test_tables():
    from lookatmyquant_amd.tables import load_table, quantile_table

    t = load_table(12, 2)
    assert t.shape == (4096,) and abs(t[0] - 1.056634) < 1e-6 and len(set(t.tolist())) == 4096
    with pytest.raises(FileNotFoundError):
        load_table(12, 5)
    q = quantile_table(16, 0)
    assert q.shape == (65536,)
    assert np.array_equal(q.astype(np.float16).astype(np.float64), q)
    assert len(set(q.tolist())) < 65536  # fp16 collapses neighbouring quantiles: ties are decided by the tie rules


def test_program_parsing():
    from lookatmyquant_amd.quantize import parse

    assert parse("tr2") == ("tr", 2, False)
    assert parse("lm3x") == ("lm", 3, True)
    assert parse("fp16") == ("fp", 16, False)
    for bad in ("tr", "gptaq3x", "rtn4x", "q4"):
        with pytest.raises(ValueError):
            parse(bad)


def test_seeds_follow_the_reference_rule():
    from lookatmyquant_amd.quantize import block_seed, matrix_seeds

    assert block_seed("self_attn.q_proj") == 2 and block_seed("mlp.down_proj") == 3 and block_seed("linear_attn.x") == 1
    assert 4 <= block_seed("vision.proj") <= 8
    assert matrix_seeds(0, "self_attn.q_proj", 0, "self_attn.q_proj") == (200, 201)
    assert matrix_seeds(3, "mlp.up_proj", 1, "mlp.gate_proj", seed_set=1) == (100000 + 3301, 100000 + 3301)


def test_token_weights_digits():
    from lookatmyquant_amd.quantize import token_weights_from_kinds

    kinds = torch.tensor([[0, 1, 2, 2, 2, 2, 2, 2, 2, 0]])
    w = token_weights_from_kinds(kinds)
    assert abs(float(w.mean()) - 1.0) < 1e-6
    assert float(w[0, 0]) > float(w[0, 1]) > float(w[0, 2])
    assert float(w.min()) > 0  # the floor keeps every token's pull


def _plan(tmp_path, groups, name="model.layers.0.mlp.down_proj.weight", cols=128):
    p = tmp_path / "plan.json"
    p.write_text(json.dumps({"format": "rowgroup-plan-1", "groups": [dict(g, matrix=name, columns=cols) for g in groups]}))
    return p


def test_row_plan_validation(tmp_path):
    from lookatmyquant_amd.rowplan import load_row_plan, write_row_plan

    shape = {"model.layers.0.mlp.down_proj.weight": (128, 128)}
    ok = _plan(tmp_path, [{"group": 0, "rows": list(range(64)), "bits": 2}, {"group": 1, "rows": list(range(64, 128)), "bits": 3}])
    plan, manifest = load_row_plan(ok, shape)
    assert [g["bits"] for g in plan["model.layers.0.mlp.down_proj.weight"]] == [2, 3] and manifest["groups"] == 2
    bad_cases = [
        [{"group": 0, "rows": list(range(64)), "bits": 2}],                                     # rows not covered
        [{"group": 0, "rows": list(range(100)), "bits": 2}, {"group": 1, "rows": list(range(100, 128)), "bits": 2}],  # not x64
        [{"group": 0, "rows": list(range(128)), "bits": 5}],                                    # width
        [{"group": 1, "rows": list(range(128)), "bits": 2}],                                    # group ids
        [{"group": 0, "rows": list(range(64)), "bits": 2}, {"group": 1, "rows": list(range(64)), "bits": 2}],  # overlap
    ]
    for groups in bad_cases:
        with pytest.raises(ValueError):
            load_row_plan(_plan(tmp_path, groups), shape)
    with pytest.raises(ValueError):
        load_row_plan(_plan(tmp_path, [{"group": 0, "rows": list(range(128)), "bits": 2}], name="unknown"), shape)
    from lookatmyquant_amd import synthetic

    plans = {"m": synthetic.row_plan(960, 7)}
    write_row_plan(tmp_path / "w.json", plans, {"m": (960, 960)})
    back, _ = load_row_plan(tmp_path / "w.json", {"m": (960, 960)})
    bpw = sum(len(g["rows"]) * g["bits"] for g in back["m"]) / 960
    assert 1.0 <= bpw <= 4.0


def test_quantize_row_groups_rejects_bad_groups():
    from lookatmyquant_amd.quantize import quantize_row_groups

    W = torch.zeros(128, 8, dtype=torch.float64)
    never = lambda rows, bits: (_ for _ in ()).throw(AssertionError("must not be called"))
    with pytest.raises(ValueError):
        quantize_row_groups(W, [{"rows": list(range(64)), "bits": 2}], never, 1, False)
    with pytest.raises(ValueError):
        quantize_row_groups(W, [{"rows": list(range(128)), "bits": 6}], never, 1, False)
    with pytest.raises(ValueError):
        quantize_row_groups(W, [{"rows": list(range(16)), "bits": 2}] * 9, never, 1, False)


def test_trellis_states_recovers_distinct_values():
    from lookatmyquant_amd.quantize import trellis_states
    from lookatmyquant_amd.tables import load_table

    t = torch.from_numpy(load_table(12, 3).copy())
    st = torch.randint(0, 4096, (5, 7))
    assert torch.equal(trellis_states(t[st], t).long(), st)


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"], capture_output=True, text=True)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_workload_counts():
    from lookatmyquant_amd import engine as E

    assert sum(E.trellis_row_steps(960, 16, 8, 128)) == 1432  # (n/16 - 1) * 24 + 16
    assert sum(E.trellis_row_steps(9728, 16, 8, 128)) == 14584
    assert E.viterbi_ops_per_row_step(16, 2) == 245760
    assert E.viterbi_ops_per_row_step(12, 2) == 15360
    # sum over blocks of 2 m (b1 - b0) (n - b1), against the closed form for n a multiple of 128: 2 m 128^2 B(B-1)/2
    assert E.trailing_flops(7, 1280) == 2 * 7 * 128 * 128 * 10 * 9 / 2


@pytest.mark.parametrize("L,k,T,start", [(6, 1, 9, 0), (6, 2, 5, 0), (6, 2, 5, 45), (6, 3, 4, 7), (8, 2, 7, 0),
                                         (8, 4, 4, 200), (12, 2, 24, 0)])
def test_reachable_search_ops_match_brute_force(L, k, T, start):
    """The reachable-state operation count of one search against an enumeration of the trellis itself: states
    s_t = (s_{t-1} 2^k + b) mod 2^L from the given start; each reachable state costs 3 operations, and each
    predecessor group (states sharing their low L - k bits) holding c reachable states costs c - 1 comparisons."""
    from lookatmyquant_amd import engine as E

    mask, low = (1 << L) - 1, (1 << (L - k)) - 1
    prev = {start}
    ops = 0
    for t in range(T):
        cur = {((s << k) | b) & mask for s in prev for b in range(1 << k)}
        ops += 3 * len(cur)
        if t > 0:
            groups = {}
            for s in prev:
                groups[s & low] = groups.get(s & low, 0) + 1
            ops += sum(c - 1 for c in groups.values())
        prev = cur
    assert E.viterbi_search_ops(L, k, T) == ops
    # once every state is reachable, each further position costs the full per-step count
    full = -(-L // k) + 1
    if T > full:
        assert E.viterbi_search_ops(L, k, T) - E.viterbi_search_ops(L, k, T - 1) == E.viterbi_ops_per_row_step(L, k)


def test_trellis_block_ops_cover_every_call():
    from lookatmyquant_amd import engine as E

    calls = E.trellis_call_lengths(960, 16, 8, 128)
    assert [sum(c) for c in calls] == E.trellis_row_steps(960, 16, 8, 128)
    assert sum(len(c) for c in calls) == 960 // 16 and calls[-1][-1] == 16
    assert E.trellis_block_ops(960, 12, 2) == [sum(E.viterbi_search_ops(12, 2, T) for T in c) for c in calls]


def test_trellis_tables_must_have_two_to_the_L_entries():
    """A table shorter than 2^L would be read past its end by the search kernels: refused before any launch."""
    from lookatmyquant_amd import engine as E
    from lookatmyquant_amd.tables import load_table, quantile_table

    t12 = torch.from_numpy(load_table(12, 2).copy())
    X = torch.zeros(4, 64, dtype=torch.float64)
    for L, t64, t32 in ((16, t12, None), (12, t12[:100], None), (12, t12, t12[:4095].float()),
                        (16, torch.from_numpy(np.array(quantile_table(16, 0), dtype=np.float64)), t12.float())):
        with pytest.raises(ValueError, match="2\\^L"):
            E.ldlq_trellis_groups(X, torch.ones(4, dtype=torch.float64), torch.eye(64, dtype=torch.float64),
                                  [(4, 2, t64, t32)], L)
    with pytest.raises(ValueError):
        E.check_tables([(4, 2, t12, None)], 17)
    E.check_tables([(4, 2, t12, t12.float())], 12)  # the right sizes pass


def test_stage_without_tables_refuses_other_state_bits():
    from lookatmyquant_amd.quantize import quantize_stage_row_groups

    with pytest.raises(ValueError, match="12-bit tables"):
        quantize_stage_row_groups({"a": torch.zeros(64, 64)}, {"a": [{"rows": list(range(64)), "bits": 2}]},
                                  torch.eye(64), 1, L=16, factor=(None, None, torch.zeros(1, dtype=torch.int32)))


def test_synthetic_plans_are_valid_row_plans(tmp_path):
    """The synthetic build's row plan written as rowgroup-plan-1 reads back through the reference's validation rules
    (rowgroup_alloc.py:268-307) for the matrices its plan puts on a trellis, at 2.3 bpw."""
    from lookatmyquant_amd import stack
    from lookatmyquant_amd.rowplan import load_row_plan, write_row_plan

    sh = stack.Shape()
    plan, rp = stack.synthetic_plans(sh, 2)
    assert set(plan["linears"].values()) == {"tr2x"} and len(plan["linears"]) == 14
    shapes = stack.active_shapes(sh, plan, 2)
    write_row_plan(tmp_path / "r.json", rp, shapes)
    back, manifest = load_row_plan(tmp_path / "r.json", shapes)
    assert manifest["matrices"] == 14 and back.keys() == rp.keys()
    for name, groups in back.items():
        assert [g["rows"] for g in groups] == [g["rows"] for g in rp[name]]
    bits = sum(len(g["rows"]) * shapes[nm][1] * g["bits"] for nm, gs in back.items() for g in gs)
    assert abs(bits / sum(m * n for m, n in shapes.values()) - 2.3) < 0.06
    # a matrix on an fp16 program is not active for a row plan
    plan["linears"]["1.mlp.down_proj"] = "fp16"
    assert "model.layers.1.mlp.down_proj.weight" not in stack.active_shapes(sh, plan, 2)


def test_cli_checks_its_arguments(tmp_path):
    """quantize.py's entry point: a row-trellis window the fused kernels do not take, a malformed window, --program
    plan without --plan and unknown programs are refused before any work (no GPU is touched)."""
    from lookatmyquant_amd.quantize import main

    for window in ("16,12", "12,4", "0,8", "17,0"):
        with pytest.raises(NotImplementedError):
            main(["--program", "tr2x", "--trellis-rows", window, "--out", str(tmp_path / "o.json")])
    for window in ("8", "8,4,2", "a,b"):
        with pytest.raises(SystemExit):
            main(["--program", "tr2x", "--trellis-rows", window, "--out", str(tmp_path / "o.json")])
    with pytest.raises(SystemExit):
        main(["--program", "plan", "--out", str(tmp_path / "o.json")])
    with pytest.raises(ValueError):
        main(["--program", "tr9y", "--out", str(tmp_path / "o.json")])


def test_stack_trellis_windows():
    """The windows the stages' fused row-group sweep takes: width 1-16 dividing the 128-column block, width + look
    <= 24."""
    from lookatmyquant_amd.stack import trellis_window

    for w in (1, 2, 4, 8, 16):
        for look in (0, 4, 24 - w):
            assert trellis_window((w, look)) == (w, look)
    for bad in ((16, 9), (3, 8), (32, 0), (0, 0), (8, -1)):
        with pytest.raises(NotImplementedError):
            trellis_window(bad)


def test_trellis_fit_checks_its_arguments():
    """Fitting covers the float32 search's trellises (L <= 12) and the two fits of codes.py:187-220; a table the
    reference cached is served without a GPU."""
    from lookatmyquant_amd import codes, fit

    with pytest.raises(NotImplementedError):
        fit.fit_table(16, 2)
    with pytest.raises(ValueError):
        fit.fit_table(12, 2, fit="kmeans")
    assert codes.trellis_values(12, 2).shape == (4096,)
