"""The reference-compatible API on the GPU (lookatmyquant_amd.codes / nested / quantize / syntax / compiler /
artifact): the words the reference's callers build give the reference's codes and reconstructions."""

import sys

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert torch.cuda.is_available(), "the GPU tests need an MI355X"


def test_ldlq_words_row_trellis_config2(golden, config12):
    """quantize.word('tr2', ...) with the LM2 flags: ldlq_words([W], H, RowTrellisCode(12, 2), [seed],
    in_seed=201, out_rot=False) -- the reference's states, scales and reconstruction."""
    from lookatmyquant_amd import codes as C

    W, H = config12
    g = golden("ldlq_trellis_c2_L12_k2")
    say("ldlq_words tr2 config 2")
    net = C.ldlq_words([torch.from_numpy(W.astype(np.float64))], torch.from_numpy(H), C.RowTrellisCode(12, 2), [200],
                       in_seed=201, out_rot=False)[0]
    assert np.array_equal(net.codes.numpy(), g["states"])
    S = net.cores["W.S"].data.numpy()
    assert np.abs(S / g["S"] - 1).max() < 1e-13
    What = net.matrix(dtype=torch.float64)[:8].numpy()
    assert np.abs(What - g["what_rows"]).max() < 1e-4 * np.abs(g["what_rows"]).max()
    assert net.rate_bits() == 960 * 960 * 2 + 16 * 960 + 960
    assert net.cores["W"].domain.fixed_start and net.cores["W"].domain.state_bits == 12
    assert C.is_trellis_path(net.codes, 12, 2)


def test_word_lm3_config1(golden, config12):
    from lookatmyquant_amd import quantize as Q

    W, H = config12
    g = golden("nested_lm3_c1")
    say("word lm3 config 1")
    net = Q.word("lm3", torch.from_numpy(W.astype(np.float64)), torch.from_numpy(H), 200, None, in_seed=201, out_rot=False)
    assert np.array_equal(net.codes.numpy(), g["idx"].astype(np.int32))
    codes = Q.lamq_codes(net.cores["W"].data, torch.from_numpy(g["levels"]))
    assert np.array_equal(codes.numpy(), g["idx"])
    What = net.matrix(dtype=torch.float64)[:8].numpy()
    assert np.abs(What - g["what_rows"]).max() < 1e-4 * np.abs(g["what_rows"]).max()
    assert net.rate_bits() == 960 * 960 * 3 + 16 * 960 + 960


def test_row_trellis_16bit_states(golden, config12):
    from lookatmyquant_amd import codes as C

    W, H = config12
    g = golden("ldlq_trellis_L16_k2_rows32")
    say("ldlq_words L=16 k=2, 32 rows")
    code = C.RowTrellisCode(16, 2, values=C.trellis_init_values(16, 0, "float16"))
    net = C.ldlq_words([torch.from_numpy(W[:32].astype(np.float64))], torch.from_numpy(H), code, [200], in_seed=201,
                       out_rot=False)[0]
    assert np.array_equal(net.codes.numpy(), g["states"])


def test_quantize_row_groups_and_the_batched_stage(config12, tables):
    """A rowgroup plan over one matrix through quantize_row_groups (one word per group, as the reference) and
    through quantize_stage_row_groups (one factor, one sweep per width): the same states; each group's states
    equal the oracle's for that group's rows."""
    from lookatmyquant_amd import codes as C
    from lookatmyquant_amd import quantize as Q
    from lookatmyquant_amd import synthetic

    W, H = config12
    Wt, Ht = torch.from_numpy(W.astype(np.float64)), torch.from_numpy(H)
    groups = synthetic.row_plan(960, 11)
    trellis = {b: C.RowTrellisCode(12, b) for b in (1, 2, 3, 4)}
    say("quantize_row_groups config 2 with a 2.3 bpw row plan")

    def round_group(rows, bits):
        return Q.word(f"tr{bits}", Wt[rows], Ht, 200, trellis, in_seed=201, out_rot=False)

    Wq, rate, entry = Q.quantize_row_groups(Wt, groups, round_group, 201, True)
    assert rate == sum(len(g["rows"]) * 960 * g["bits"] + 16 * len(g["rows"]) + 960 for g in groups)
    states = entry["states"].numpy().astype(np.int64) % 4096
    for g in groups[:3]:
        rows = np.array(g["rows"])
        ref, _, _ = O.ldlq_words_trellis(W[rows[:16]], H, tables[g["bits"]], 12, g["bits"], 201)
        assert np.array_equal(states[rows[:16]], ref)
    say("quantize_stage_row_groups")
    out = Q.quantize_stage_row_groups({"q": Wt}, {"q": groups}, Ht, 201)
    st, S = out["q"]
    assert np.array_equal(st.cpu().numpy(), states)
    assert torch.equal(entry["scales"], S.cpu().float())


def test_viterbi_api(golden, tables):
    from lookatmyquant_amd import codes as C

    g = golden("viterbi")
    x = torch.from_numpy(g["L12_k3_x"])
    say("codes.viterbi")
    st = C.viterbi(x, torch.from_numpy(tables[3].copy()), 12, 3, start=torch.from_numpy(g["L12_k3_start"]))
    assert st.dtype == torch.int64 and st.device == x.device
    assert np.array_equal(st.numpy(), g["L12_k3_fixed"])


def test_generic_sweep_matches_the_fused_scalar_kernel(config12):
    """syntax.sweep with a Python projection (the ScalarCode project of ldlq_words) settles the same levels as the
    fused width-1 kernel."""
    from lookatmyquant_amd import engine as E
    from lookatmyquant_amd.frame import Environment
    from lookatmyquant_amd.syntax import sweep

    W, H = config12
    X = (torch.from_numpy(W[:64].astype(np.float64)) @ torch.from_numpy(O.rht(960, 201)).T).cuda()
    S = E.row_rms(X)
    env = Environment(E.rotate_hessian(torch.from_numpy(H).cuda(), 201))
    lv = torch.tensor([-1.5104, -0.4528, 0.4528, 1.5104], dtype=torch.float64, device="cuda")
    mids = (lv[1:] + lv[:-1]) / 2
    chosen = torch.empty(X.shape, dtype=torch.long, device="cuda")

    def project(j, col, T):
        i = torch.bucketize((col / S).contiguous(), mids)
        chosen[:, j] = i
        return lv[i] * S

    say("generic sweep, width 1")
    sweep(X, env, project)
    fused = E.ldlq_scalar(X, env.U, lv, mode=1, S=S, dead=env.dead)
    assert torch.equal(chosen.to(torch.int32), fused)


def test_kl_api():
    from lookatmyquant_amd import compiler
    from lookatmyquant_amd import synthetic

    r, q = synthetic.logits(12, 5000, 5, 6)
    w = np.linspace(0.5, 2.0, 12).astype(np.float32)
    ref, mean = O.kl_rows(r, q, w)
    rt = torch.from_numpy(r.view(np.int16)).view(torch.bfloat16).reshape(3, 4, 5000)
    qt = torch.from_numpy(q.view(np.int16)).view(torch.bfloat16).reshape(3, 4, 5000)
    say("compiler.kl")
    assert abs(compiler.kl(rt, qt, torch.from_numpy(w).reshape(3, 4)) - mean) < 1e-4 * mean
    per = compiler.kl_per_token(rt, qt)
    assert per.shape == (3, 4)
    assert np.abs(per.cpu().numpy().reshape(-1) - ref).max() < 1e-4 * ref.max()


def test_artifact_packing(golden):
    from lookatmyquant_amd import artifact

    g = golden("misc")
    for bits in (1, 3):
        st = g[f"pack_{bits}_states"]
        codes = artifact.pack_trellis(st, bits)
        assert np.array_equal(codes, g[f"pack_{bits}_codes"])
        assert np.array_equal(artifact.unpack_trellis(codes, bits, st.shape[1]), st)


def _golden_artifact_inputs():
    """The saved codes and state dict the reference's golden artifacts were exported from (the golden script's own
    construction, over its committed arrays)."""
    import importlib.util

    from conftest import GOLDEN

    spec = importlib.util.spec_from_file_location("artifact_saved", GOLDEN / "artifact_saved.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    a = dict(np.load(GOLDEN / "artifact_inputs.npz"))
    return mod.saved_and_state(a, torch)


def _same_files(a, b):
    names = sorted(p.name for p in a.iterdir())
    assert names == sorted(p.name for p in b.iterdir())
    for n in names:
        assert (a / n).read_bytes() == (b / n).read_bytes(), n


def test_export_saved_codes_matches_the_reference_artifact(tmp_path):
    """export_saved_codes over the golden saved codes (explicit row groups, inferred widths, scalar codes, embedding
    buckets, a tied head, bf16/f16/i64/empty state, model assets): artifact.json and weights.bin equal the files the
    reference wrote, byte for byte, and so does the receipt."""
    import json

    from conftest import GOLDEN
    from lookatmyquant_amd import artifact

    saved, state, alias = _golden_artifact_inputs()
    receipts = json.loads((GOLDEN / "artifact_receipts.json").read_text())
    say("export_saved_codes of the golden saved codes")
    r = artifact.export_saved_codes(saved, tmp_path / "x", dense_tensors=state, model_dir=GOLDEN / "artifact_model")
    _same_files(tmp_path / "x", GOLDEN / "artifact_export")
    assert {k: v for k, v in r.items() if k != "path"} == receipts["export"]
    say("encode_entry + write_artifact with shared tables")
    tensors, meta = artifact.encode_entry("m.weight", alias)
    semantic = {"matrices": {"m.weight": meta}}
    r = artifact.write_artifact(tmp_path / "y", tensors, semantic,
                                tensor_aliases=artifact.find_table_aliases(tensors, semantic))
    _same_files(tmp_path / "y", GOLDEN / "artifact_alias")
    assert {k: v for k, v in r.items() if k != "path"} == receipts["alias"]


def test_encode_entry_rejects_what_the_reference_rejects():
    from lookatmyquant_amd import artifact

    saved, _, alias = _golden_artifact_inputs()
    up = saved["matrices"]["model.layers.0.mlp.up_proj.weight"]

    def variant(**kw):
        e = dict(up)
        e.update(kw)
        return e

    cases = []
    st = up["states"].clone()
    st[5, 9] = (int(st[5, 9]) & ~0xFFF) | ((int(st[5, 9]) + 1) & 0xFFF)  # a broken transition inside a row
    cases.append((variant(states=st), "states are not a row trellis from zero"))
    st = up["states"].clone()
    r0 = int(up["row_groups"][0]["rows"][0])
    st[r0, 3] += 4096  # one state in another table
    cases.append((variant(states=st), "a row crosses table identities"))
    st = up["states"].clone()
    st[0, 0] = 3 * 4096  # beyond the concatenated tables
    cases.append((variant(states=st), "invalid saved trellis table or states"))
    groups = [dict(g) for g in up["row_groups"]]
    groups[0] = dict(groups[0], table_index=1)
    cases.append((variant(row_groups=groups), "invalid row group"))
    groups = [dict(g) for g in up["row_groups"]][:2]
    cases.append((variant(row_groups=groups), "row groups must cover every row exactly once"))
    cases.append((variant(scales=up["scales"].double()), "saved row scales must be fp32"))
    cases.append((variant(table=up["table"][:-1]), "invalid saved trellis table or states"))
    cases.append((variant(log_g=0), "unsupported trained transforms"))
    cases.append((variant(states=up["states"].float()), "saved entry must be a matrix"))
    o = saved["matrices"]["model.layers.0.self_attn.o_proj.weight"]
    codes = o["codes"].clone()
    codes[3, 4] = 8
    cases.append((dict(o, codes=codes), "scalar index outside table"))
    for i, (entry, msg) in enumerate(cases):
        say(f"encode_entry error case {i}: {msg}")
        with pytest.raises(ValueError, match=msg):
            artifact.encode_entry("x", entry)
    with pytest.raises(ValueError, match="invalid input signs"):
        artifact.encode_entry("x", up, signs=np.zeros(70, dtype=np.int8))


@pytest.mark.parametrize("n", [1, 31, 32, 33, 70, 129])
def test_pack_widths_and_layouts_match_the_oracle(n):
    """pack_symbols and pack_trellis at every width 1..8 against the oracle's bit-by-bit restatement; pack_codes
    reading a row group in place (rows gathered, a table offset subtracted) against the same rows packed alone."""
    from lookatmyquant_amd import artifact
    from lookatmyquant_amd import engine as E

    rng = np.random.default_rng(100 + n)
    m = 37
    for bits in range(1, 9):
        say(f"pack n={n} bits={bits}")
        q = rng.integers(0, 1 << bits, (m, n))
        assert np.array_equal(artifact.pack_symbols(q, bits), O.pack_symbols(q, bits))
        st = np.zeros((m, n), dtype=np.int64)
        s = np.zeros(m, dtype=np.int64)
        for c in range(n):
            s = ((s << bits) | rng.integers(0, 1 << bits, m)) & 4095
            st[:, c] = s
        words = artifact.pack_trellis(st, bits)
        assert np.array_equal(words, O.pack_trellis(st, bits))
        if n >= 32:  # long random paths are paths at one width only
            assert artifact.infer_path_bits(st) == bits
        # in place: every other row of a matrix whose states carry the offset 4096 * 2
        big = np.zeros((2 * m, n), dtype=np.int64)
        big[1::2] = st + 8192
        rows = torch.arange(1, 2 * m, 2, device="cuda")
        codes, bad = E.pack_codes(torch.from_numpy(big).int().cuda(), bits, rows=rows, base=8192, L=12)
        assert int(bad.item()) == 0
        assert np.array_equal(codes.cpu().numpy().view(np.uint32), words)
        if n > 1:
            bad_st = st.copy()
            bad_st[m // 2, n // 2] ^= 1 << 11  # a high bit that no shift produced
            if not artifact.valid_path(bad_st, bits):
                with pytest.raises(ValueError, match="not a row trellis"):
                    artifact.pack_trellis(bad_st, bits)
        with pytest.raises(ValueError, match="invalid symbols or width"):
            artifact.pack_symbols(np.full((2, n), 1 << bits), bits)


def test_pack_codes_flags_rows_outside_the_source():
    """A row index outside the code array is caught by the kernel's own bounds check: flagged, words zero, no read."""
    from lookatmyquant_amd import engine as E

    src = torch.zeros(4, 40, dtype=torch.int32, device="cuda")
    rows = torch.tensor([0, 4, -1, 3], dtype=torch.int64, device="cuda")
    codes, bad = E.pack_codes(src, 2, rows=rows)
    assert int(bad.item()) == 2
    assert int(codes.abs().sum().item()) == 0


def _paths(rng, ks, n, L):
    """Random row-trellis paths from state 0, row i at width ks[i], states in [0, 2^L)."""
    ks = np.asarray(ks, dtype=np.int64)
    st = np.zeros((ks.size, n), dtype=np.int64)
    s = np.zeros(ks.size, dtype=np.int64)
    for c in range(n):
        s = ((s << ks) | rng.integers(0, 1 << ks)) & ((1 << L) - 1)
        st[:, c] = s
    return st


@pytest.mark.parametrize("n,L", [(33, 12), (600, 16), (2560, 16)])
def test_pack_codes_groups_equal_each_group_alone(n, L):
    """lamq_pack_codes_groups: 37 row groups of three code arrays (more than one launch's 32), widths 1-4 at random,
    gathered row lists, an empty group, one source with a table offset: every group's words equal lamq_pack_codes on
    that group alone (and, for the first eight groups, the oracle's pack_trellis of its rows), with no flag raised;
    then a bad path in one group and a row outside its source in another raise both flags (1 and 2), the
    out-of-source row's words zero."""
    from lookatmyquant_amd import engine as E

    rng = np.random.default_rng(n + L)
    srcs = []  # each row of a source is a path at the width of the groups that read it
    for si, m in enumerate((200, 96, 130)):
        ks = rng.integers(1, 5, m)
        base = 8192 if si == 1 else 0
        st = _paths(rng, ks, n, L) + base
        srcs.append((torch.from_numpy(st).int().cuda(), st, ks, base))
    items, picked = [], []
    for gi in range(37):
        src_t, st, ks, base = srcs[gi % 3]
        k = int(rng.integers(1, 5))
        cand = np.flatnonzero(ks == k)
        r = 0 if gi == 5 else int(rng.integers(1, min(40, cand.size) + 1))
        rows = rng.choice(cand, r, replace=False) if r else cand[:0]
        items.append((src_t, k, torch.from_numpy(rows.astype(np.int64)).cuda(), base))
        picked.append((st, rows))
    say(f"pack_codes_groups n={n} L={L}: 37 groups")
    outs, bad = E.pack_codes_groups(items, L=L)
    assert int(bad.item()) == 0
    for gi, ((src_t, k, rows_t, base), out, (st, rows)) in enumerate(zip(items, outs, picked)):
        assert out.shape == (rows.size, (n + 31) // 32 * k)
        if rows.size == 0:  # the empty group: no words, nothing launched for it
            continue
        alone, bad1 = E.pack_codes(src_t, k, rows=rows_t, base=base, L=L)
        assert int(bad1.item()) == 0
        assert torch.equal(out, alone)
        if gi < 8 and rows.size:
            assert np.array_equal(out.cpu().numpy().view(np.uint32), O.pack_trellis(st[rows] - base, k, L))
    # the flags: a state whose high bit no shift made (a bad path) and a row index past its source
    src_t, st, ks, base = srcs[0]
    broken = st.copy()
    row = int(np.flatnonzero(ks == 2)[0])
    broken[row, n // 2] ^= 1 << (L - 1)
    b_t = torch.from_numpy(broken).int().cuda()
    rows_ok = torch.tensor([row], dtype=torch.int64, device="cuda")
    rows_out = torch.tensor([0, 200], dtype=torch.int64, device="cuda")
    outs, bad = E.pack_codes_groups([(b_t, 2, rows_ok, 0), (src_t, 1, rows_out, 0)], L=L)
    assert int(bad.item()) == 3
    assert int(outs[1][1].abs().sum().item()) == 0
    alone, bad1 = E.pack_codes(b_t, 2, rows=rows_ok, L=L)
    assert int(bad1.item()) == 1 and torch.equal(outs[0], alone)


def test_pack_codes_groups_scalar_symbols():
    """The scalar layout (column order, widths 5-8, no trellis check) through lamq_pack_codes_groups against
    lamq_pack_codes group by group and the oracle's pack_symbols."""
    from lookatmyquant_amd import engine as E

    rng = np.random.default_rng(9)
    n = 70
    q = rng.integers(0, 256, (60, n))
    for k in (5, 6, 7):  # a few rows whose symbols fit each narrower width
        q[4 * k : 4 * k + 3] %= 1 << k
    src = torch.from_numpy(q).int().cuda()
    rows = {k: np.flatnonzero(q.max(axis=1) < (1 << k)) for k in (5, 6, 7, 8)}
    items = [(src, k, torch.from_numpy(rows[k].astype(np.int64)).cuda(), 0) for k in (5, 6, 7, 8)]
    say("pack_codes_groups, scalar symbols at widths 5-8")
    outs, bad = E.pack_codes_groups(items, trellis=False)
    assert int(bad.item()) == 0
    for (_, k, rows_t, _), out in zip(items, outs):
        assert rows[k].size >= 3
        alone, _ = E.pack_codes(src, k, rows=rows_t, trellis=False)
        assert torch.equal(out, alone)
        assert np.array_equal(out.cpu().numpy().view(np.uint32), O.pack_symbols(q[rows[k]], k))


def test_environment_and_covariance(config12):
    from lookatmyquant_amd import synthetic
    from lookatmyquant_amd.frame import Environment, covariance

    X = synthetic.calibration(3000, 320, 31, 32)
    say("covariance and Environment")
    H = covariance(torch.from_numpy(X).to(torch.bfloat16))
    ref = O.hessian(X) * 3000
    assert (H.cpu().numpy() - ref).__abs__().max() < 1e-4 * np.abs(ref).max()
    env = Environment(H)
    _, U, _ = O.environment(H.cpu().numpy())
    assert np.abs(env.U.cpu().numpy() - U).max() < 1e-9 * np.abs(U).max()


def test_environment_output_sensitivity_weights_the_error():
    """Environment(H, G).error(D) = tr(G D H D^T) (opgraph/frame.py:534-537): G = I gives the unweighted error, a
    diagonal G the g-weighted sum of the rows' d_i Hd d_i^T, a full G numpy's trace, on the oracle's damped H."""
    from lookatmyquant_amd.frame import Environment

    rng = np.random.default_rng(41)
    X = rng.standard_normal((400, 24))
    H = X.T @ X / 400
    D = rng.standard_normal((10, 24))
    A = rng.standard_normal((10, 10))
    Hd, _, _ = O.environment(H)
    rows = np.einsum("ij,jk,ik->i", D, Hd, D)
    Ht, Dt = torch.from_numpy(H), torch.from_numpy(D)
    e0 = Environment(Ht).error(Dt)
    assert abs(e0 - rows.sum()) < 1e-12 * rows.sum()
    assert abs(Environment(Ht, G=torch.eye(10, dtype=torch.float64)).error(Dt) - e0) < 1e-12 * e0
    g = rng.uniform(0.5, 2.0, 10)
    eg = Environment(Ht, G=torch.from_numpy(np.diag(g))).error(Dt)
    assert abs(eg - (g * rows).sum()) < 1e-12 * (g * rows).sum()
    G = A @ A.T
    ref = np.trace(G @ D @ Hd @ D.T)
    assert abs(Environment(Ht, G=torch.from_numpy(G)).error(Dt) - ref) < 1e-12 * ref
    with pytest.raises(ValueError):
        Environment(Ht, G=torch.ones(3, 4, dtype=torch.float64))
    with pytest.raises(ValueError):
        Environment(Ht, G=torch.eye(9, dtype=torch.float64)).error(Dt)


def test_cross_target_is_the_damped_solve():
    from lookatmyquant_amd.quantize import cross_target

    rng = np.random.default_rng(12)
    Xa = rng.standard_normal((500, 48))
    H = Xa.T @ Xa / 500
    D = 0.01 * rng.standard_normal((48, 48))
    M = cross_target(torch.from_numpy(H), torch.from_numpy(D), 0.5).numpy()
    ref = np.eye(48) + 0.5 * np.linalg.solve(H + 0.1 * np.diag(H).mean() * np.eye(48), D.T).T
    assert np.abs(M - ref).max() < 1e-9


def test_ldlq_factor_and_round(golden, config12):
    """ldlq_gpu.ldlq_factor / ldlq_round (ldlq_gpu.py:15-49): the factor of the symmetrised, damped H (retrying with
    more damping, a zero diagonal kept zero) and the levels the reference's config-1 vectors hold."""
    from lookatmyquant_amd import ldlq_gpu

    n = 200
    rng = np.random.default_rng(21)
    A = rng.standard_normal((3 * n, n))
    H = A.T @ A / (3 * n)
    H[7, :] = 0
    H[:, 7] = 0
    Hr = H + 1e-4 * np.triu(rng.standard_normal((n, n)), 1)  # not symmetric: the factor symmetrises first
    say("ldlq_factor n=200 with a zero diagonal")
    U = ldlq_gpu.ldlq_factor(torch.from_numpy(Hr)).cpu().numpy()
    ref = O.ldlq_factor(Hr)
    assert np.abs(U - ref).max() < 1e-9 * np.abs(ref).max()
    Q, _ = np.linalg.qr(rng.standard_normal((96, 96)))
    lam = np.ones(96)
    lam[0] = -0.05
    Hn = Q @ np.diag(lam) @ Q.T
    say("ldlq_factor retry")
    Un = ldlq_gpu.ldlq_factor(torch.from_numpy(Hn)).cpu().numpy()
    assert np.abs(Un - O.ldlq_factor(Hn)).max() < 1e-8 * np.abs(Un).max()
    lam[0] = -5.0
    with pytest.raises(AssertionError):
        ldlq_gpu.ldlq_factor(torch.from_numpy(Q @ np.diag(lam) @ Q.T))

    W, H1 = config12
    g = golden("nested_lm3_c1")
    R = O.rht(960, 201)
    X = W.astype(np.float64) @ R.T
    S = O.row_scale(X)
    say("ldlq_round config 1")
    U1 = ldlq_gpu.ldlq_factor(torch.from_numpy(R @ H1 @ R.T))
    got = ldlq_gpu.ldlq_round(torch.from_numpy(X / S[:, None]), U1, torch.from_numpy(g["levels"]))
    assert got.dtype == torch.float64 and got.shape == (960, 960)
    assert np.array_equal(got.cpu().numpy(), g["levels"][g["idx"]])


@pytest.mark.parametrize("with_h", [True, False])
def test_column_trellis_words(tables, with_h):
    """ldlq_words with the column TrellisCode (codes.py:363-383): the generic sweep, each block's columns cut into
    sequences of T rows searched from a free first state -- the oracle's states, sequences on trellis paths, the
    reconstruction the states' values times the row scales, rotated back."""
    from lookatmyquant_amd import codes as C

    m, n, T = 320, 96, 160
    rng = np.random.default_rng(22)
    W = rng.standard_normal((m, n)) * np.abs(rng.standard_t(5, n))
    A = rng.standard_normal((400, n)) * np.abs(rng.standard_t(4, n))
    H = A.T @ A / 400 if with_h else None
    code = C.TrellisCode(12, 2, T=T, values=tables[2].copy())
    say(f"column trellis ldlq_words H={with_h}")
    net = C.ldlq_words([torch.from_numpy(W)], None if H is None else torch.from_numpy(H), code, [5], in_seed=6)[0]
    st, S = O.ldlq_words_column_trellis(W, H, tables[2], 12, 2, T, 5, 6)
    assert np.array_equal(net.codes.numpy(), st)
    assert np.abs(net.cores["W.S"].data.numpy() / S - 1).max() < 1e-13
    c = net.cores["W"]
    assert c.labels[:2] == ("s", "t") and c.data.shape == (m // T, T, n)
    seqs = st.reshape(m // T, T, n).transpose(0, 2, 1).reshape(-1, T)
    assert C.is_trellis_path(torch.from_numpy(seqs), 12, 2)
    What = net.matrix(dtype=torch.float64).numpy()
    ref = O.rht(m, 5).T @ (S[:, None] * tables[2][st]) @ O.rht(n, 6)
    assert np.abs(What - ref).max() < 1e-10 * np.abs(ref).max()
    with pytest.raises(ValueError):
        C.ldlq_words([torch.from_numpy(W[:100])], None, code, [5], in_seed=6)


def test_chol_keep_dead_flag():
    """lamq_chol_inv_upper_ex with LAMQ_CHOL_KEEP_DEAD: a zero diagonal is damped, not replaced by 1, and the mean
    counts it as zero; without the flag it is the Environment factor; an unknown flag is EINVAL."""
    from lookatmyquant_amd import engine as E

    n = 130
    rng = np.random.default_rng(23)
    A = rng.standard_normal((3 * n, n))
    H = A.T @ A / (3 * n)
    H[0, :] = 0
    H[:, 0] = 0
    Ht = torch.from_numpy(H).cuda()
    say("chol keep_dead n=130")
    Hd, U, dead, info = E.chol_inv_upper(Ht, keep_dead=True)
    assert int(info.item()) == 0 and bool(dead[0]) and int(dead.sum()) == 1
    ref = O.ldlq_factor(H)
    assert np.abs(U.cpu().numpy() - ref).max() < 1e-9 * np.abs(ref).max()
    assert abs(Hd[0, 0].item() - 0.01 * np.mean(np.diag(H))) < 1e-15
    Hd2, U2, _, _ = E.chol_inv_upper(Ht)
    _, Ue, _ = O.environment(H)
    assert np.abs(U2.cpu().numpy() - Ue).max() < 1e-9 * np.abs(Ue).max()
    assert Hd2[0, 0].item() > 1.0
    lib = E._abi.lib()
    ws = torch.empty(lib.lamq_chol_inv_upper_workspace_size(n), dtype=torch.uint8, device="cuda")
    out = torch.empty(n, n, dtype=torch.float64, device="cuda")
    inf = torch.zeros(1, dtype=torch.int32, device="cuda")
    rc = lib.lamq_chol_inv_upper_ex(Ht.data_ptr(), n, n, 0.01, 2, None, 0, out.data_ptr(), n, None, inf.data_ptr(),
                                    ws.data_ptr(), ws.numel(), None, None)
    assert rc == -1  # LAMQ_EINVAL


def test_error_paths():
    from lookatmyquant_amd import codes as C
    from lookatmyquant_amd import engine as E
    from lookatmyquant_amd.frame import Environment

    with pytest.raises(E.LinAlgError):
        Environment(-torch.eye(16, dtype=torch.float64))
    with pytest.raises(NotImplementedError):  # a 17-bit state is beyond the kernels
        C.viterbi(torch.zeros(2, 4), torch.zeros(1 << 17), 17, 2)
    with pytest.raises(NotImplementedError):  # a 16-bit table that fp16 cannot hold
        C.viterbi(torch.zeros(2, 4), torch.randn(1 << 16, dtype=torch.float64), 16, 2)


@pytest.mark.parametrize("L,k,width,look", [(12, 5, 16, 8), (10, 7, 8, 4), (12, 2, 16, 20), (12, 3, 32, 8)])
def test_row_trellis_outside_the_fused_kernels_matches_oracle(L, k, width, look):
    """Row trellises the fused block kernels do not take (k past 4, a window longer than 24, a block wider than 16)
    go through codes.ldlq_words on the generic sweep, each block settled by the standalone search from each row's
    state with the look-ahead as it stands (codes.py:397-404, 441-448): the oracle's states for the same factor and
    row scales, 3 rows x 200 columns (two lazy blocks and a partial one)."""
    from lookatmyquant_amd import codes as C
    from lookatmyquant_amd import engine as E
    from lookatmyquant_amd.frame import Environment

    rng = np.random.default_rng(40 * L + k + look)
    n = 200
    Xa = rng.standard_normal((600, n))
    H = Xa.T @ Xa / 600
    W = rng.standard_normal((3, n))
    tab = rng.standard_normal(1 << L)
    code = C.RowTrellisCode(L, k, width=width, look=look, values=tab)
    assert not E.fused_trellis(L, k, width, look, torch.from_numpy(tab))
    say(f"row trellis on the generic sweep: L={L} k={k} width={width} look={look}")
    net = C.ldlq_words([torch.from_numpy(W)], torch.from_numpy(H), code, [1], incoherent=False, out_rot=False)[0]
    env = Environment(torch.from_numpy(H).cuda())
    S = net.cores["W.S"].data.numpy()
    ref = O.ldlq_trellis(W, env.U.cpu().numpy(), S, tab, L, k, width=width, look=look,
                         dead=env.dead.cpu().numpy().astype(np.uint8))
    assert np.array_equal(net.codes.numpy(), ref)
    assert C.is_trellis_path(net.codes, L, k)


def test_ldlq_noise_matches_the_oracle():
    """compiler.ldlq_noise against oracle.ldlq_noise on the same CPU-generator draw: rotations, damped factor and the
    triangular product agree to float64 rounding; with and without the output rotation."""
    from lookatmyquant_amd import compiler

    rng = np.random.default_rng(43)
    m, n = 96, 320
    W = rng.standard_normal((m, n))
    X = rng.standard_normal((2000, n)) * np.linspace(0.5, 2.0, n)
    H = X.T @ X / 2000
    for row_rotation in (True, False):
        say(f"ldlq_noise row_rotation={row_rotation}")
        out = compiler.ldlq_noise(torch.from_numpy(W), torch.from_numpy(H), 0.015, 11,
                                  torch.Generator().manual_seed(3), row_rotation=row_rotation)
        eta = torch.randn(m, n, generator=torch.Generator().manual_seed(3), dtype=torch.float64).numpy()
        ref, _, _ = O.ldlq_noise(W, H, 0.015, 11, eta, row_rotation=row_rotation)
        assert out.dtype == torch.float64 and out.device.type == "cpu"
        err = np.abs(out.numpy() - ref).max() / np.abs(ref - W).max()
        say(f"  max |diff| / max |E| = {err:.2e}")
        assert err < 1e-10


def test_fast_rht_and_rotated_moment():
    from lookatmyquant_amd.finetune_lib import FastRHT, rotated_moment

    rng = np.random.default_rng(44)
    n = 2560
    R = FastRHT(n, 17)
    Rn = O.rht(n, 17)
    X = rng.standard_normal((3, 5, n)).astype(np.float32)
    say("FastRHT back/forward")
    Xt = torch.from_numpy(X)
    back = R.back(Xt)
    assert back.dtype == torch.float32 and back.shape == Xt.shape and back.device.type == "cpu"
    ref = X.astype(np.float64) @ Rn.T
    assert np.abs(back.numpy() - ref).max() < 1e-6 * np.abs(ref).max()
    fwd = R.forward(back)
    assert np.abs(fwd.numpy() - X).max() < 1e-6 * np.abs(X).max()
    A = rng.standard_normal((n, 64))
    H = A @ A.T / 64
    Hr = rotated_moment(torch.from_numpy(H), R)
    assert Hr.dtype == torch.float64 and torch.equal(Hr, Hr.T)
    ref = Rn @ H @ Rn.T
    assert np.abs(Hr.cpu().numpy() - ref).max() < 1e-5 * np.abs(ref).max()


def test_rounded_matches_the_oracle(config12, tables):
    """finetune_lib.rounded over a row plan: each group's states are the oracle's row-trellis LDLQ of the rotated rows
    at the given scales; the refitted scale satisfies its normal equation under env.H; W_hat is the rotated-back
    scale * table[states]; a subset of rows gives those rows' result; the generic sweep (a non-RowPath code) and the
    fused pass agree."""
    from lookatmyquant_amd import synthetic
    from lookatmyquant_amd.finetune_lib import FastRHT, RowPath, rotated_moment, rounded
    from lookatmyquant_amd.frame import Environment

    W, H = config12
    W = W[:192].astype(np.float32)
    n = W.shape[1]
    R = FastRHT(n, 301)
    Hr = rotated_moment(torch.from_numpy(H), R)
    env = Environment(Hr)
    plan = synthetic.row_plan(192, 5, groups=3)
    groups = [(torch.tensor(g["rows"]), g["bits"], RowPath(torch.from_numpy(tables[g["bits"]].copy()), g["bits"]))
              for g in plan]
    Xr = R.back(torch.from_numpy(W)).double().numpy()
    scale0 = torch.from_numpy(np.sqrt((Xr ** 2).mean(1)).astype(np.float32))
    scale = scale0.clone()
    say("rounded, fused")
    W_hat, states = rounded(torch.from_numpy(W), R, groups, scale, env)
    assert states.dtype == torch.int16 and states.shape == W.shape
    Hd = env.H.cpu().numpy()
    Ud = env.U.cpu().numpy()
    st = states.numpy().astype(np.int64)
    for g in plan[:4]:
        rows = np.asarray(g["rows"])
        ref = O.ldlq_trellis(Xr[rows], Ud, scale0.numpy()[rows].astype(np.float64), tables[g["bits"]], 12, g["bits"],
                             dead=env.dead.cpu().numpy())
        say(f"  group bits {g['bits']} rows {len(rows)}")
        assert np.array_equal(st[rows], ref)
        got = tables[g["bits"]][st[rows]]
        s = scale.numpy()[rows].astype(np.float64)
        resid = ((Xr[rows] - s[:, None] * got) @ Hd * got).sum(1)
        assert np.abs(resid).max() < 1e-5 * np.abs((Xr[rows] @ Hd * got).sum(1)).max()
    Q = np.empty(W.shape)
    for g in plan:
        rows = np.asarray(g["rows"])
        Q[rows] = tables[g["bits"]][st[rows]]
    ref = (scale.numpy()[:, None] * Q.astype(np.float32)).astype(np.float64) @ O.rht(n, 301)
    assert np.abs(W_hat.numpy() - ref).max() < 1e-5 * np.abs(ref).max()
    say("rounded, a subset of rows")
    sub = np.arange(0, 192, 3)
    scale_s = scale0.clone()
    groups_s = [(g, k, RowPath(c.values, k)) for g, k, c in groups]
    W_s, states_s = rounded(torch.from_numpy(W), R, groups_s, scale_s, env, rows=torch.from_numpy(sub))
    assert torch.equal(states_s, states[sub])
    assert torch.equal(scale_s[sub], scale[sub])
    rest = np.setdiff1d(np.arange(192), sub)
    assert torch.equal(scale_s[rest], scale0[rest])
    say("rounded, generic sweep")

    class Generic:
        def __init__(self, code):
            self.code, self.width, self.look, self.paths = code, code.width, code.look, []

        def step(self, j, X, ahead):
            q = self.code.step(j, X, ahead)
            self.paths = self.code.paths
            return q

    scale_g = scale0.clone()
    groups_g = [(g, k, Generic(RowPath(c.values, k))) for g, k, c in groups[:2]]
    rows_g = torch.cat([g for g, _, _ in groups[:2]])
    _, states_g = rounded(torch.from_numpy(W), R, groups_g, scale_g, env, rows=rows_g)
    assert torch.equal(states_g, states[rows_g])
    assert torch.allclose(scale_g[rows_g], scale[rows_g], rtol=1e-6, atol=0)


@pytest.mark.parametrize("case", ["r3", "r3_noH", "r4"])
def test_multirate_sweep_matches_the_reference(golden, case):
    """nested.multirate_sweep for several rates at once (nested.py:104-147) on the GPU: the reference's indices
    (three rates of a 3-bit nested code with and without H, four rates of a 4-bit code with a dead input)."""
    from lookatmyquant_amd import nested as N

    g = golden("multirate")
    H = None if case.endswith("noH") else torch.from_numpy(g[f"{case}_H"])
    say(f"multirate {case}")
    idx = N.multirate_sweep(torch.from_numpy(g[f"{case}_X"]), H, torch.from_numpy(g[f"{case}_tables"]),
                            torch.from_numpy(g[f"{case}_weights"]))
    assert np.array_equal(idx.numpy(), g[f"{case}_idx"])


@pytest.mark.parametrize("m,n,block,with_h", [(96, 160, 32, True), (100, 130, 8, True), (70, 40, 16, False),
                                              (300, 150, 32, True)])
def test_output_shaping_matches_the_oracle(m, n, block, with_h):
    """nested.multirate_sweep with G (one rate, nested.py:104-147): each column's rows settled `block` at a time and
    the later rows re-solved under G's damped factor (lamq_shaping_feedback, lamq_ldlq_shaped_column), inside the
    width-1 sweep under H (two lazy runs at n = 160 and 150) or every column alone: the oracle's indices, whose
    block rule the generic block sweep and the isotropic G pin; partial last row blocks at m = 100, 70 and 300."""
    from lookatmyquant_amd import nested as N

    rng = np.random.default_rng(m + n + block)
    X = rng.standard_normal((m, n))
    Xa = rng.standard_normal((2 * n, n))
    H = Xa.T @ Xa / (2 * n) if with_h else None
    Ga = rng.standard_normal((3 * m, m)) * np.abs(rng.standard_t(4, m))
    G = Ga.T @ Ga / (3 * m)
    lv = N.lloyd_max(3)
    say(f"output shaping {m} x {n}, block {block}, H {with_h}")
    idx = N.multirate_sweep(torch.from_numpy(X), None if H is None else torch.from_numpy(H), lv[None],
                            torch.tensor([1.0], dtype=torch.float64), G=torch.from_numpy(G), block=block)
    assert np.array_equal(idx.numpy(), O.shaped_sweep(X, H, lv.numpy(), G, block=block))


def test_lm_word_with_output_shaping_matches_the_oracle(config12):
    """quantize.word("lm3", ..., G=G) (quantize.py:332-344 -> nested_words with G, nested.py:155-192): the input
    rotation, the row scales, G in units of the row scale (S G S) and the shaped sweep under R H R^T, against the
    oracle's indices from the same rotated rows; one matrix, rows not rotated, as the reference requires."""
    from lookatmyquant_amd import nested as N
    from lookatmyquant_amd import quantize as Q

    W, H = config12
    W = W[:128].astype(np.float64)
    rng = np.random.default_rng(5)
    Ga = rng.standard_normal((400, 128))
    G = Ga.T @ Ga / 400
    say("lm3 word with output shaping, 128 x 960")
    net = Q.word("lm3", torch.from_numpy(W), torch.from_numpy(H), 200, None, in_seed=201, out_rot=False,
                 G=torch.from_numpy(G))
    S = net.cores["W.S"].data.numpy()
    X = W @ O.rht(960, 201).T
    Hr = O.rht(960, 201) @ H @ O.rht(960, 201).T
    ref = O.shaped_sweep(X / S[:, None], Hr, N.lloyd_max(3).numpy(), S[:, None] * G * S[None, :], block=32)
    assert np.array_equal(net.codes.numpy(), ref)
    with pytest.raises(ValueError, match="one matrix at one rate"):
        N.nested_words([torch.from_numpy(W)], torch.from_numpy(H), [200], 3, [3], 0.4, [1.0], N.lloyd_max(3),
                       in_seed=201, out_rot=True, G=torch.from_numpy(G))


def test_multirate_kernel_matches_the_oracle_across_runs():
    """lamq_ldlq_multirate_block over two outer runs and several workgroups (300 rows x 700 columns, two rates of a
    4-bit nested code with unequal weights) against the oracle, and nested_words' three rates reading the shared
    indices with their own levels."""
    from lookatmyquant_amd import engine as E
    from lookatmyquant_amd import nested as N

    rng = np.random.default_rng(9)
    m, n = 300, 700
    X = rng.standard_normal((m, n))
    Xa = rng.standard_normal((2 * n, n))
    H = Xa.T @ Xa / (2 * n)
    tables = N.nested_tables(4, [2, 4], 0.4)
    w = torch.tensor([0.7, 0.3], dtype=torch.float64)
    say("multirate 300 x 700, two rates")
    _, U, dead, _ = E.chol_inv_upper(torch.from_numpy(H).cuda())
    idx = E.ldlq_multirate(torch.from_numpy(X).cuda(), U, tables.cuda(), w.cuda(), dead=dead).cpu().numpy()
    ref = O.multirate_sweep(X, H, tables.numpy(), w.numpy())
    assert np.array_equal(idx, ref)
    W = torch.from_numpy(rng.standard_normal((64, 256)) * 0.02)
    Hs = torch.from_numpy(Xa[:, :256].T @ Xa[:, :256] / (2 * n))
    out = N.nested_words([W], Hs, [300], 3, [1, 2, 3], 0.4, [0.2, 0.3, 0.5], in_seed=301, out_rot=False)
    assert sorted(out) == [1, 2, 3]
    codes = out[3][0].codes
    for b, tab in zip([1, 2, 3], N.nested_tables(3, [1, 2, 3], 0.4)):
        net = out[b][0]
        assert torch.equal(net.codes, codes)  # one index per entry, read by every rate
        assert torch.allclose(net.cores["W"].data, tab[codes.long()].to(net.cores["W"].data))
