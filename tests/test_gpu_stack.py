"""The layer loop (lookatmyquant_amd.stack, the caller of quantize.py:1280-1314, 1416-1560, 1626-1690) on a small
stack: the statistics it forms are the closed forms of the activations it captured, and every row group's codes are
the oracle's row-trellis words of the stage's QEP target under those statistics, bit for bit."""

import sys

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def test_small_stack_build(tmp_path):
    from lookatmyquant_amd import stack
    from lookatmyquant_amd.tables import load_table

    assert torch.cuda.is_available()
    sh = stack.Shape(hidden=512, heads=8, kv_heads=4, head_dim=128, inter=1024, layers=2, vocab=1000)
    tok, w = stack.calibration_tokens(sequences=4, T=256, vocab=1000, seed=11)
    say("stack build: 2 layers, hidden 512, 1024 calibration tokens")
    out = stack.build(tok, sh, w, alpha=0.5, chunk=2, keep=2)
    shapes = stack.matrix_shapes(sh)
    assert out["weights"] == 2 * sum(m * n for m, n in shapes.values())
    assert 1.0 < out["bits"] / out["weights"] < 4.1
    assert int(out["bad"].item()) == 0  # every packed row a trellis path from state 0
    for key, rec in out["codes"].items():
        assert sorted(r for g in rec["groups"] for r in g["rows"]) == list(range(shapes[key.split(".", 1)[1]][0]))
    tables = {b: np.array(load_table(12, b)) for b in (1, 2, 3, 4)}
    wn = np.asarray(w, dtype=np.float64).reshape(-1)
    for (i, s), kept in out["stages"].items():
        H, D, in_seed, plans = kept["H"].cpu(), kept["D"].cpu(), kept["in_seed"], kept["plans"]
        targets = {nm: t.cpu() for nm, t in kept["targets"].items()}
        xq = kept["Xq"].float().cpu().numpy().astype(np.float64)
        xr = kept["Xr"].float().cpu().numpy().astype(np.float64)
        Hn = (xq * wn[:, None]).T @ xq / len(xq)
        Dn = (xr * wn[:, None]).T @ xq / len(xq)
        assert np.abs(H.numpy() - Hn).max() < 1e-4 * np.abs(Hn).max()
        assert np.abs(D.numpy() - Dn).max() < 1e-4 * np.abs(Dn).max()
        # the QEP map of quantize.py:1330-1335 from the statistics the build used (float32 sums, so the map is
        # compared on those, not on the closed forms)
        Hg, Dg = H.numpy(), D.numpy()
        Mn = np.eye(len(Hg)) + 0.5 * np.linalg.solve(Hg + 0.1 * np.mean(np.diag(Hg)) * np.eye(len(Hg)), (Dg - Hg).T).T
        Wl = stack.layer_weights(i, sh, torch.device("cuda"))
        for nm, groups in plans.items():
            Wn = Wl[nm].double().cpu().numpy()
            target = targets[nm].numpy()
            assert np.abs(target - Wn @ Mn).max() < 1e-9 * np.abs(Wn).max()  # both forms of qep_targets
            if (i, s) == (0, 0):  # both streams enter the first layer equal: no cross term yet
                assert np.abs(target - Wn).max() < 1e-3 * np.abs(Wn).max()
            elif s == 1:  # the o_proj input already sees the quantized q/k/v
                assert np.abs(target - Wn).max() > 1e-3 * np.abs(Wn).max()
            states = out["codes"][f"{i}.{nm}"]["states"].cpu().numpy()
            for g in groups[:2]:
                rows = np.asarray(g["rows"])[:32]
                ref, _, _ = O.ldlq_words_trellis(target[rows], H.numpy(), tables[g["bits"]], 12, g["bits"], in_seed)
                say(f"layer {i} stage {s} {nm} group {g['group']} bits {g['bits']}")
                assert np.array_equal(states[rows], ref)
    # the packed codes out: an opgraph-packed-1 artifact whose groups unpack to the build's states, row for row, and
    # whose words are the oracle's packing of those states
    from lookatmyquant_amd import artifact

    say("export_codes")
    receipt = stack.export_codes(out, tmp_path / "artifact")
    assert receipt["all_tensor_bytes_verified"]
    stored, meta = artifact.read_artifact(tmp_path / "artifact")
    assert len(meta["matrices"]) == len(out["codes"])
    for key, rec in out["codes"].items():
        i, nm = key.split(".", 1)
        name = f"model.layers.{i}.{nm}.weight"
        states = rec["states"].cpu().numpy()
        n = states.shape[1]
        assert np.array_equal(stored[name + ".signs"], O.rht_signs(n, rec["in_seed"]).astype(np.int8))
        for j, g in enumerate(rec["groups"]):
            k = f"{name}.g{j}"
            rows = stored[k + ".rows"].astype(np.int64)
            assert np.array_equal(rows, np.asarray(g["rows"]))
            assert np.array_equal(O.unpack_trellis(stored[k + ".codes"], g["bits"], n), states[rows])
            if j == 0:
                assert np.array_equal(stored[k + ".codes"][:8], O.pack_trellis(states[rows[:8]], g["bits"]))
            assert np.array_equal(stored[k + ".scales"], rec["scales"].float().cpu().numpy()[rows])


def test_small_stack_build_at_another_trellis_window():
    """The stages' row trellis at width 8, look 4 (quantize.py's --trellis-rows 8,4): sampled rows of two row groups
    of every matrix equal the oracle's row-trellis LDLQ at that window."""
    from lookatmyquant_amd import stack
    from lookatmyquant_amd.tables import load_table

    sh = stack.Shape(hidden=512, heads=8, kv_heads=4, head_dim=128, inter=1024, layers=1, vocab=1000)
    tok, w = stack.calibration_tokens(sequences=4, T=256, vocab=1000, seed=11)
    say("stack build: 1 layer, hidden 512, window (8, 4)")
    out = stack.build(tok, sh, w, alpha=0.5, chunk=2, keep=1, window=(8, 4))
    assert int(out["bad"].item()) == 0
    tables = {b: np.array(load_table(12, b)) for b in (1, 2, 3, 4)}
    for (i, s), kept in out["stages"].items():
        H = kept["H"].cpu().numpy()
        for nm, groups in kept["plans"].items():
            target = kept["targets"][nm].cpu().numpy()
            states = out["codes"][f"{i}.{nm}"]["states"].cpu().numpy()
            for g in groups[:2]:
                rows = np.asarray(g["rows"])[:16]
                ref, _, _ = O.ldlq_words_trellis(target[rows], H, tables[g["bits"]], 12, g["bits"], kept["in_seed"],
                                                 width=8, look=4)
                say(f"layer {i} stage {s} {nm} group {g['group']} bits {g['bits']}")
                assert np.array_equal(states[rows], ref)


@pytest.mark.parametrize("T", [8, 64, 520, 2048, 4096])
def test_causal_softmax_matches_a_float64_reference(T):
    """engine.causal_softmax on bf16 scores [2, 3, T, T]: every kept entry within one bf16 rounding (2^-8 relative)
    of the float64 softmax of float(score) * scale under the causal mask, every masked entry exactly 0; in place and
    out of place alike, bit for bit."""
    from lookatmyquant_amd import engine as E

    g = torch.Generator(device="cuda").manual_seed(T)
    sc = (torch.randn(2, 3, T, T, generator=g, device="cuda") * 4).to(torch.bfloat16)
    scale = 1.0 / 128 ** 0.5
    print(f"causal softmax T={T}", flush=True)
    p = E.causal_softmax(sc, scale)
    q = sc.clone()
    E.causal_softmax(q, scale, out=q)
    assert torch.equal(p, q)
    ref = sc.double().cpu() * scale
    mask = torch.ones(T, T, dtype=torch.bool).triu(1)
    ref = torch.softmax(ref.masked_fill(mask, float("-inf")), -1)
    got = p.double().cpu()
    assert torch.all(got[..., mask] == 0)
    err = (got - ref).abs()
    assert torch.all(err <= 2.0 ** -8 * ref + 1e-30), float((err / ref.clamp(min=1e-300)).max())


def test_swiglu_matches_the_unfused_chain():
    """engine.swiglu against torch's silu(a) * b in bf16 (each rounded to bf16): equal up to one bf16 rounding where
    the exponentials differ in their last bit, over the config-5 MLP width and large |a|."""
    from lookatmyquant_amd import engine as E

    g = torch.Generator(device="cuda").manual_seed(9)
    a = (torch.randn(300, 9728, generator=g, device="cuda") * 4).bfloat16()
    b = torch.randn(300, 9728, generator=g, device="cuda").bfloat16()
    say("swiglu 300 x 9728")
    got = E.swiglu(a, b).float()
    ref = (torch.nn.functional.silu(a) * b).float()
    rel = ((got - ref).abs() / ref.abs().clamp_min(1e-30)).max().item()
    assert rel <= 2 ** -7, rel
    assert (got == ref).float().mean().item() > 0.99


@pytest.mark.parametrize("shape", [(3, 77, 2560), (2, 5, 32, 128), (1000, 4096), (7, 9728), (1, 8)])
def test_rms_norm_matches_the_float32_chain(shape):
    """engine.rms_norm against the float32 chain it replaces, xf * rsqrt(mean(xf^2) + eps) rounded to bf16, times g in
    bf16: equal up to one bf16 rounding of the product (the sum of squares is reduced in another order), at the
    forward's widths (hidden 2,560, head dim 128, 4,096, 9,728) and a width of 8."""
    from lookatmyquant_amd import engine as E

    g0 = torch.Generator(device="cuda").manual_seed(sum(shape))
    x = (torch.randn(*shape, generator=g0, device="cuda") * 3).bfloat16()
    g = (1 + 0.1 * torch.randn(shape[-1], generator=g0, device="cuda")).bfloat16()
    say(f"rms_norm {shape}")
    got = E.rms_norm(x, g, 1e-6).float()
    xf = x.float()
    ref = ((xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)).bfloat16() * g).float()
    rel = ((got - ref).abs() / ref.abs().clamp_min(1e-30)).max().item()
    assert rel <= 2 ** -7, rel
    assert (got == ref).float().mean().item() > 0.99


@pytest.mark.parametrize("B,H,Hkv,T", [(2, 32, 8, 2048), (3, 4, 4, 33), (1, 8, 2, 1)])
def test_fused_attention_shapes_against_float64(B, H, Hkv, T):
    """The fused attention at the config-5 shape (GQA 32/8, T = 2,048), a ragged T with one query block partly past it
    and T = 1, from strided q and k (the layouts the forward hands over) against float64 on the CPU: each output
    within 2e-2 of |v| ~ 1 (the probabilities are rounded to bf16 before the product with v) and the output of query
    0, which sees only key 0, equal to v[0]."""
    from lookatmyquant_amd import engine as E

    g = torch.Generator(device="cuda").manual_seed(B * 1000 + T)
    q = torch.randn(B, T, H, 128, generator=g, device="cuda").bfloat16().transpose(1, 2)
    k = torch.randn(B, T, Hkv, 128, generator=g, device="cuda").bfloat16().transpose(1, 2)
    v = torch.randn(B, Hkv, T, 128, generator=g, device="cuda").bfloat16()
    say(f"fused attention B={B} H={H} Hkv={Hkv} T={T}")
    got = E.attention_causal(q, k, v, 128 ** -0.5).float().cpu().double()
    rep = H // Hkv
    for b in range(B):
        for h in range(0, H, max(1, H // 4)):
            qd, kd, vd = (t[b, hh].float().cpu().double() for t, hh in ((q, h), (k, h // rep), (v, h // rep)))
            sc = qd @ kd.T / 128 ** 0.5
            sc = sc.masked_fill(torch.ones(T, T, dtype=torch.bool).triu(1), float("-inf"))
            ref = torch.softmax(sc, -1) @ vd
            err = (got[b, h] - ref).abs().max().item()
            assert err < 2e-2, (b, h, err)
            assert torch.equal(got[b, h, 0], vd[0].float().bfloat16().double())
    assert torch.isfinite(got).all()


@pytest.mark.parametrize("B,T,heads,tables", [(2, 2048, 32, "model"), (2, 2048, 8, "model"), (3, 37, 8, "random"),
                                               (1, 1, 4, "random")])
def test_rms_norm_rope_matches_the_unfused_chain(B, T, heads, tables):
    """engine.rms_norm_rope (lamq_rms_norm_rope_bf16) against the chain it replaces, the per-head RMSNorm kernel and
    then y * cos + rotate_half(y) * sin in torch's bf16 operations (each product and the sum rounded to bf16): equal
    bit for bit, at the config-5 q and k shapes with the model's tables and at ragged shapes with random ones."""
    from lookatmyquant_amd import engine as E, stack

    g0 = torch.Generator(device="cuda").manual_seed(B * 100 + T + heads)
    x = (torch.randn(B, T, heads, 128, generator=g0, device="cuda") * 2).bfloat16()
    g = (1 + 0.1 * torch.randn(128, generator=g0, device="cuda")).bfloat16()
    if tables == "model":
        cos, sin = stack.rope_tables(T, stack.Shape(), torch.device("cuda"))
    else:
        cos = (2 * torch.rand(T, 128, generator=g0, device="cuda") - 1).bfloat16()
        sin = (2 * torch.rand(T, 128, generator=g0, device="cuda") - 1).bfloat16()
    say(f"rms_norm_rope B={B} T={T} heads={heads} {tables} tables")
    got = E.rms_norm_rope(x, g, 1e-6, cos, sin)
    y = E.rms_norm(x, g, 1e-6).transpose(1, 2)
    rot = torch.cat([-y[..., 64:], y[..., :64]], -1)
    ref = (y * cos + rot * sin).transpose(1, 2)
    assert got.shape == ref.shape
    assert torch.equal(got, ref), (got.float() - ref.float()).abs().max().item()


def test_fused_attention_repeats_bit_for_bit_at_config5_size():
    """The fused attention at the config-5 forward's full size (32 sequences of 2,048 tokens, GQA 32/8: 16,384
    workgroups, two to a CU, so the LDS is busy with both): five calls on the same inputs bit for bit equal, and
    two sampled heads within 2e-2 of float64. The kernel reduces in a fixed order, so calls that differ are a
    fragment read that took a wrong LDS address under contention (the paired transposing reads' asm once let the
    first read's destination share the second's address register: about 1% of outputs then went wrong now and then,
    at this size only)."""
    from lookatmyquant_amd import engine as E

    B, H, Hkv, T = 32, 32, 8, 2048
    g = torch.Generator(device="cuda").manual_seed(52)
    q = torch.randn(B, T, H, 128, generator=g, device="cuda").bfloat16().transpose(1, 2)
    k = torch.randn(B, T, Hkv, 128, generator=g, device="cuda").bfloat16().transpose(1, 2)
    v = torch.randn(B, T, Hkv, 128, generator=g, device="cuda").bfloat16().transpose(1, 2)
    say(f"fused attention repeated: B={B} H={H} Hkv={Hkv} T={T}")
    o0 = E.attention_causal(q, k, v, 128 ** -0.5).clone()
    for rep in range(4):
        assert torch.equal(E.attention_causal(q, k, v, 128 ** -0.5), o0), f"repeat {rep}"
    for b, h in ((31, 5), (17, 30)):
        qd, kd, vd = (t[b, hh].float().cpu().double() for t, hh in ((q, h), (k, h // 4), (v, h // 4)))
        sc = qd @ kd.T / 128 ** 0.5
        sc = sc.masked_fill(torch.ones(T, T, dtype=torch.bool).triu(1), float("-inf"))
        ref = torch.softmax(sc, -1) @ vd
        err = (o0[b, h].float().cpu().double() - ref).abs().max().item()
        assert err < 2e-2, (b, h, err)


def test_attention_matches_a_float64_reference():
    """The stack's one attention path (causal grouped-query, bf16 products, float32 softmax) against the same
    attention in float64 on the CPU from the same bf16 inputs, over a batch that spans two of its sequence groups
    (6 sequences). The probabilities are rounded to bf16 before the product with v, so the tolerance is a few bf16
    units of |v| ~ 1."""
    from lookatmyquant_amd import stack

    sh = stack.Shape(hidden=512, heads=8, kv_heads=4, head_dim=128, inter=1024, layers=1, vocab=1000)
    g = torch.Generator(device="cuda").manual_seed(11)
    q = torch.randn(6, 8, 200, 128, generator=g, device="cuda").bfloat16()
    k = torch.randn(6, 4, 200, 128, generator=g, device="cuda").bfloat16()
    v = torch.randn(6, 4, 200, 128, generator=g, device="cuda").bfloat16()
    say("attention 6 x 8 heads x 200 x 128 (GQA 8/4)")
    got = stack.attention(q, k, v, sh).float().cpu().double()
    qd, kd, vd = (t.float().cpu().double() for t in (q, k, v))
    kd = kd.repeat_interleave(2, dim=1)
    vd = vd.repeat_interleave(2, dim=1)
    sc = qd @ kd.transpose(-1, -2) / 128 ** 0.5
    sc = sc.masked_fill(torch.ones(200, 200, dtype=torch.bool).triu(1), float("-inf"))
    ref = torch.softmax(sc, -1) @ vd
    err = (got - ref).abs().max().item()
    say(f"  max |diff| against float64: {err:.3e}")
    assert err < 3e-2
    assert torch.equal(got[:, :, 0], vd[:, :, 0].float().bfloat16().double())  # the first position attends to itself


def test_cli_plan_driven_build(tmp_path):
    """python -m lookatmyquant_amd.quantize (quantize.py:923-989's arguments): one layer of the Qwen3.5-4B-shaped stack
    from a plan file and a rowgroup-plan-1 file, with the saved codes and the artifact written; then the same layer
    under one program for every linear."""
    import json

    from lookatmyquant_amd import stack
    from lookatmyquant_amd.quantize import main
    from lookatmyquant_amd.rowplan import write_row_plan

    sh = stack.Shape()
    plan, rp = stack.synthetic_plans(sh, 1)
    (tmp_path / "plan.json").write_text(json.dumps(plan))
    write_row_plan(tmp_path / "rows.json", rp, stack.active_shapes(sh, plan, 1))
    small = ["--layers", "1", "--calib", "4", "--calib-len", "256", "--redamp"]
    print("quantize --program plan, one layer", flush=True)
    main(["--program", "plan", "--plan", str(tmp_path / "plan.json"), "--row-plan", str(tmp_path / "rows.json"),
          *small, "--save-codes", str(tmp_path / "codes.pt"), "--artifact", str(tmp_path / "art"),
          "--out", str(tmp_path / "res.json")])
    res = json.loads((tmp_path / "res.json").read_text())
    shapes = stack.matrix_shapes(sh)
    assert res["layers"] == 1 and res["weights"] == sum(m * n for m, n in shapes.values())
    assert abs(res["bits per weight"] - 2.3) < 0.1
    assert res["row plan"]["matrices"] == 7
    assert res["artifact"]["all_tensor_bytes_verified"] and res["artifact"]["tensor_count"] > 7
    payload = torch.load(tmp_path / "codes.pt", weights_only=True)
    # the reference's --save-codes layout (quantize.py:1737-1739): its consumers read payload["matrices"]
    assert payload["row plan"]["matrices"] == 7 and payload["model"] and payload["evaluation"].startswith("skipped")
    saved = payload["matrices"]
    assert sorted(saved) == sorted(f"model.layers.0.{nm}.weight" for nm in shapes)
    for name, e in saved.items():
        m, n = shapes[name.split(".", 3)[3][: -len(".weight")]]
        assert e["states"].shape == (m, n) and e["trellis_layout"] == "row"
        rows = torch.cat([g["rows"] for g in e["row_groups"]])
        assert torch.equal(rows.sort().values, torch.arange(m))  # every row in exactly one group
        for g in e["row_groups"]:
            s = e["states"][g["rows"]].long() - 4096 * g["table_index"]
            assert int(s.min()) >= 0 and int(s.max()) < 4096
    # the saved file through the reference's consumer (compiler_artifact.export_saved_codes): the same packed words as
    # the artifact the build wrote from its own packed groups
    from lookatmyquant_amd import artifact

    dense = {name: np.zeros(tuple(e["states"].shape), dtype=np.float32) for name, e in saved.items()}
    artifact.export_saved_codes(payload, tmp_path / "art2", dense_tensors=dense)
    t1, m1 = artifact.read_artifact(tmp_path / "art")
    t2, m2 = artifact.read_artifact(tmp_path / "art2")
    assert sorted(m1["matrices"]) == sorted(m2["matrices"]) == sorted(saved)
    assert sorted(t1) == sorted(t2)
    for key in t1:
        if key.endswith((".codes", ".rows", ".scales", ".table", ".signs")):
            assert np.array_equal(np.asarray(t1[key]), np.asarray(t2[key])), key
    print("quantize --program tr3x, one layer", flush=True)
    main(["--program", "tr3x", *small, "--out", str(tmp_path / "res3.json")])
    res3 = json.loads((tmp_path / "res3.json").read_text())
    assert abs(res3["bits per weight"] - 3.0) < 0.01 and res3["row plan"] is None
