"""The caller of the per-matrix path: the layer loop of a post-training build (quantize.py:1280-1314, 1416-1560,
1626-1690) on a Qwen3-shaped decoder stack.

Per layer, two streams of calibration activations go through the layer: the reference stream through the
full-precision weights and the quantized stream through the weights quantized so far. Each stage (q/k/v, o,
gate/up, down: the matrices reading one input) takes its input from both streams, forms H = X_q^T W X_q / N with
the token weights and the QEP cross term D = X_ref^T W X_q / N, moves the target to W* = W M with
M = I + alpha ((H + lam mean(diag H) I)^-1 (D - H)^T)^T (quantize.py:1330-1335, 1505; qep_targets), quantizes every matrix of
the stage by its row groups (quantize_stage_row_groups: one factor, one sweep per width), and writes the
reconstruction back, so the next stage's input already sees it. Then both streams advance through the layer.

The stack is random-initialised (there are no checkpoints here): N(0, std^2) weights, unit RMSNorm gains, rotary
position embedding, grouped-query attention. Everything runs on the GPU: the forwards in bf16 on torch's GEMMs,
the statistics, factors, rotations and sweeps on this package's kernels.
"""

from __future__ import annotations

import time
from dataclasses import dataclass

import numpy as np
import torch

from . import artifact
from . import engine as E
from . import synthetic
from .quantize import matrix_seeds, qep_targets, quantize_stage_row_groups, stage_factor
from .tables import load_table, quantile_table


@dataclass(frozen=True)
class Shape:
    """Qwen3.5-4B-shaped stack (the benchmark's config 5): hidden 2560, 32 query and 8 key/value heads of 128,
    MLP 9728."""

    hidden: int = 2560
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    inter: int = 9728
    layers: int = 36
    vocab: int = 151936
    rope_theta: float = 1e6
    eps: float = 1e-6
    std: float = 0.015


# the stages of one decoder layer in execution order: (matrix names, the name whose input they read)
STAGES = (("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"), ("self_attn.o_proj",),
          ("mlp.gate_proj", "mlp.up_proj"), ("mlp.down_proj",))


def matrix_shapes(sh: Shape) -> dict:
    q = sh.heads * sh.head_dim
    kv = sh.kv_heads * sh.head_dim
    return {"self_attn.q_proj": (q, sh.hidden), "self_attn.k_proj": (kv, sh.hidden), "self_attn.v_proj": (kv, sh.hidden),
            "self_attn.o_proj": (sh.hidden, q), "mlp.gate_proj": (sh.inter, sh.hidden),
            "mlp.up_proj": (sh.inter, sh.hidden), "mlp.down_proj": (sh.hidden, sh.inter)}


def layer_weights(i: int, sh: Shape, dev, seed: int = 5000) -> dict:
    """Layer i's weights, bf16 on the GPU, drawn from a generator seeded by (seed, i)."""
    g = torch.Generator(device=dev).manual_seed(seed * 1000 + i)
    w = {nm: (torch.randn(*s, generator=g, device=dev, dtype=torch.float32) * sh.std).to(torch.bfloat16)
         for nm, s in matrix_shapes(sh).items()}
    one = lambda n: torch.ones(n, dtype=torch.bfloat16, device=dev)
    w |= {"input_layernorm": one(sh.hidden), "post_attention_layernorm": one(sh.hidden),
          "self_attn.q_norm": one(sh.head_dim), "self_attn.k_norm": one(sh.head_dim)}
    return w


def rms_norm(x: torch.Tensor, g: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype) * g


def rope_tables(T: int, sh: Shape, dev):
    inv = 1.0 / (sh.rope_theta ** (torch.arange(0, sh.head_dim, 2, device=dev, dtype=torch.float32) / sh.head_dim))
    f = torch.outer(torch.arange(T, device=dev, dtype=torch.float32), inv)
    emb = torch.cat([f, f], -1)
    return emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)


def _rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat([-x[..., h:], x[..., :h]], -1)


def _lin(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """x W^T with a contiguous right operand (x [.., n] bf16, W [m, n])."""
    return torch.matmul(x, w.t().contiguous())


def _attention_flash(q, k, v):
    """Causal grouped-query attention [B, H, T, D] bf16 on the fused flash kernel only (the backend is forced, so a
    build without it raises instead of falling back to the unfused math path)."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    with sdpa_kernel(SDPBackend.FLASH_ATTENTION):
        return torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)


def _attention_unfused(q, k, v, sh: Shape):
    """The same attention one sequence at a time: scores and softmax in float32, every batched product's right
    operand contiguous."""
    B, _, T, _ = q.shape
    rep = sh.heads // sh.kv_heads
    kT = k.repeat_interleave(rep, dim=1).transpose(-1, -2).contiguous()
    vv = v.repeat_interleave(rep, dim=1).contiguous()
    mask = torch.ones(T, T, dtype=torch.bool, device=q.device).triu(1)
    out = torch.empty(B, sh.heads, T, sh.head_dim, dtype=q.dtype, device=q.device)
    scale = 1.0 / float(sh.head_dim) ** 0.5
    for b in range(B):  # one sequence at a time bounds the score matrix
        sc = torch.matmul(q[b], kT[b]).float() * scale
        sc.masked_fill_(mask, float("-inf"))
        out[b] = torch.matmul(torch.softmax(sc, -1).to(q.dtype), vv[b])
    return out


_FLASH = [True]


def attention_input_to_o(x: torch.Tensor, w: dict, sh: Shape, rope) -> torch.Tensor:
    """The o_proj input of one chunk [B, T, hidden] (normed hidden states in): q/k/v, per-head RMSNorm of q and k,
    rotary embedding, causal grouped-query attention (the fused flash kernel where the build has it, else the
    unfused float32-softmax path)."""
    B, T, _ = x.shape
    q = _lin(x, w["self_attn.q_proj"]).view(B, T, sh.heads, sh.head_dim)
    k = _lin(x, w["self_attn.k_proj"]).view(B, T, sh.kv_heads, sh.head_dim)
    v = _lin(x, w["self_attn.v_proj"]).view(B, T, sh.kv_heads, sh.head_dim)
    q = rms_norm(q, w["self_attn.q_norm"], sh.eps).transpose(1, 2)
    k = rms_norm(k, w["self_attn.k_norm"], sh.eps).transpose(1, 2)
    v = v.transpose(1, 2).contiguous()
    cos, sin = rope
    q = (q * cos + _rotate_half(q) * sin).contiguous()
    k = (k * cos + _rotate_half(k) * sin).contiguous()
    out = None
    if _FLASH[0]:
        try:
            out = _attention_flash(q, k, v)
        except RuntimeError:
            _FLASH[0] = False
    if out is None:
        out = _attention_unfused(q, k, v, sh)
    return out.transpose(1, 2).reshape(B, T, sh.heads * sh.head_dim)


def _flat(x: torch.Tensor) -> torch.Tensor:
    return x.reshape(-1, x.shape[-1])


class Timer:
    def __init__(self):
        self.t = {}

    def add(self, key, s):
        self.t[key] = self.t.get(key, 0.0) + s


@torch.no_grad()
def build(tokens: torch.Tensor, sh: Shape = Shape(), token_w: torch.Tensor | None = None, alpha: float = 0.5,
          L: int = 12, plan_seed: int = 7000, chunk: int = 32, layers: int | None = None, weight_seed: int = 5000,
          timer: Timer | None = None, keep: int = 0) -> dict:
    """The build of a random-initialised stack on calibration token ids [S, T]: per layer and stage, the two streams'
    statistics, the QEP target, the row-group trellis codes (a 2.3 bpw row plan per matrix, bits 1-4) and the
    quantized weights written back. Returns {"codes": {"i.name": {"states": int32 [m, n], "scales": float64 [m],
    "in_seed", "groups": the row plan, "packed": per group the code words (engine.pack_codes, read in place)}},
    "weights": n, "bits": total rate bits, "redamped": {"i.first matrix": damping} for stages that needed more than
    0.01, "bad": a device flag set if any packed row was not a trellis path, "L", "tables"}; export_codes writes the
    codes as an opgraph-packed-1 artifact. chunk: calibration sequences per forward pass (the default takes config
    5's 32 x 2048 tokens in one, about 17 GB of activations at its peak: fewer, larger products). token_w: per-token weights [S, T] (mean 1), or None. keep: the first `keep` layers
    also return their stages' inputs and statistics under "stages" (for tests: {(i, s): (X_q, X_ref, H, D,
    {name: W*}, in_seed, plans)}, on the CPU)."""
    dev = E._abi.device()
    main = torch.cuda.current_stream(dev)
    side = torch.cuda.Stream(dev)  # default priority
    S_, T = tokens.shape
    nl = sh.layers if layers is None else layers
    timer = timer or Timer()
    tables = {b: (quantile_table(16, 0) if L == 16 else load_table(12, b)) for b in (1, 2, 3, 4)}
    rope = tuple(t.to(dev) for t in rope_tables(T, sh, dev))
    chunks = [slice(c, min(c + chunk, S_)) for c in range(0, S_, chunk)]
    wt = None if token_w is None else [token_w[cs].reshape(-1).to(dev, torch.float32) for cs in chunks]
    wcls = None if wt is None else [E.weight_classes(wc, include_zero=True) for wc in wt]
    # the embedding (shared by both streams: it is not quantized here)
    g = torch.Generator(device=dev).manual_seed(weight_seed * 1000 + 999)
    emb = (torch.randn(sh.vocab, sh.hidden, generator=g, device=dev, dtype=torch.float32) * sh.std).to(torch.bfloat16)
    hq = [emb[tokens[cs].to(dev)] for cs in chunks]
    hr = [h.clone() for h in hq]
    del emb
    codes, n_w, bits, kept, redamped = {}, 0, 0.0, {}, {}
    bad = torch.zeros(1, dtype=torch.int32, device=dev)  # set if any packed row is not a trellis path from state 0
    shapes = matrix_shapes(sh)
    for i in range(nl):
        t0 = time.perf_counter()
        wr = layer_weights(i, sh, dev, weight_seed)  # the reference layer
        wq = {k: v.clone() for k, v in wr.items()}  # quantized in place, stage by stage
        # the reference stream's stage inputs (its weights never change) and its output
        xr = {s: [] for s in range(4)}
        hr_next = []
        for c, h in enumerate(hr):
            x1 = rms_norm(h, wr["input_layernorm"], sh.eps)
            a = attention_input_to_o(x1, wr, sh, rope)
            h1 = h + _lin(a, wr["self_attn.o_proj"])
            x2 = rms_norm(h1, wr["post_attention_layernorm"], sh.eps)
            m = torch.nn.functional.silu(_lin(x2, wr["mlp.gate_proj"])) * _lin(x2, wr["mlp.up_proj"])
            hr_next.append(h1 + _lin(m, wr["mlp.down_proj"]))
            for s, x in enumerate((x1, a, x2, m)):
                xr[s].append(_flat(x))
        torch.cuda.synchronize()
        timer.add("forward", time.perf_counter() - t0)
        # the quantized stream, stage by stage
        h1q = [None] * len(hq)
        x2q = [None] * len(hq)
        for s, names in enumerate(STAGES):
            t1 = time.perf_counter()
            if s == 0:
                xq = [rms_norm(h, wq["input_layernorm"], sh.eps) for h in hq]
                x1q = xq
            elif s == 1:
                xq = [attention_input_to_o(x, wq, sh, rope) for x in x1q]
                aq = xq
            elif s == 2:
                h1q = [h + _lin(a, wq["self_attn.o_proj"]) for h, a in zip(hq, aq)]
                xq = x2q = [rms_norm(h, wq["post_attention_layernorm"], sh.eps) for h in h1q]
            else:
                xq = [torch.nn.functional.silu(_lin(x, wq["mlp.gate_proj"])) * _lin(x, wq["mlp.up_proj"]) for x in x2q]
            xqf = [_flat(x) for x in xq]
            torch.cuda.synchronize()
            t2 = time.perf_counter()
            timer.add("forward", t2 - t1)
            H, D = _stage_statistics(xqf, wt, xr[s], wcls)
            torch.cuda.synchronize()
            t25 = time.perf_counter()
            timer.add("statistics", t25 - t2)
            _, in_seed = matrix_seeds(i, names[0], 0, names[0])
            # the stage's factor (rotation of H, damped inverse factor) on a second stream, next to the QEP targets
            # (their own factor of H + lambda I and products) on this one: the two are independent
            side.wait_stream(main)
            with torch.cuda.stream(side):
                factor = stage_factor(H, in_seed, 0.01)
            targets = qep_targets(H, D - H, alpha, {nm: wr[nm] for nm in names})
            main.wait_stream(side)
            for t in factor:
                t.record_stream(main)
            torch.cuda.synchronize()
            t3 = time.perf_counter()
            timer.add("qep_targets", t3 - t25)
            plans = {nm: synthetic.row_plan(shapes[nm][0], plan_seed + 10 * i + STAGE_INDEX[nm]) for nm in names}
            # a stage whose statistics the damping of the reference's Environment cannot make positive definite (float32
            # sums of a nearly singular H, as the o_proj input of a random-initialised stack with near-uniform
            # attention gives) is damped more, as ldlq_gpu.ldlq_factor does (ldlq_gpu.py:19-23), and counted
            for d in (0.01, 0.1, 1.0):
                try:
                    res = quantize_stage_row_groups(targets, plans, H, in_seed, L=L, tables=tables, damp=d,
                                                    factor=factor if d == 0.01 else None)
                    break
                except E.LinAlgError:
                    if d == 1.0:
                        raise
                    redamped[f"{i}.{names[0]}"] = 10 * d
            if i < keep:
                kept[(i, s)] = (torch.cat(xqf).cpu(), torch.cat(xr[s]).cpu(), H.cpu(), D.cpu(),
                                {nm: t.cpu() for nm, t in targets.items()}, in_seed, plans)
            for nm, (st, Srow) in res.items():
                wq[nm] = _reconstruct(st, Srow, plans[nm], tables, in_seed).to(torch.bfloat16)
                packed = []
                for gp in plans[nm]:
                    rows = torch.as_tensor(gp["rows"], dtype=torch.int64, device=dev)
                    packed.append(E.pack_codes(st, gp["bits"], rows=rows, L=L, bad=bad)[0])
                    bits += len(gp["rows"]) * shapes[nm][1] * gp["bits"] + 16 * len(gp["rows"])
                codes[f"{i}.{nm}"] = {"states": st, "scales": Srow, "in_seed": in_seed, "groups": plans[nm],
                                      "packed": packed}
                n_w += shapes[nm][0] * shapes[nm][1]
            torch.cuda.synchronize()
            timer.add("quantize", time.perf_counter() - t3)
            del xq, xqf, targets, H, D
        # both streams through the layer (the quantized one with its last matrix now quantized)
        t4 = time.perf_counter()
        hq = [h1 + _lin(torch.nn.functional.silu(_lin(x, wq["mlp.gate_proj"])) * _lin(x, wq["mlp.up_proj"]),
                        wq["mlp.down_proj"]) for h1, x in zip(h1q, x2q)]
        hr = hr_next
        del xr, wr, wq, h1q, x2q
        torch.cuda.synchronize()
        timer.add("forward", time.perf_counter() - t4)
    return {"codes": codes, "weights": n_w, "bits": bits, "stages": kept, "redamped": redamped, "bad": bad, "L": L,
            "tables": tables}


STAGE_INDEX = {nm: j for j, nm in enumerate(n for st in STAGES for n in st)}


def export_codes(out: dict, path) -> dict:
    """The build's codes as an opgraph-packed-1 artifact at `path` (compiler_artifact.py:307-371, 491-531): per
    matrix model.layers.{i}.{name}.weight, its row groups in plan order with the words packed during the build, fp32
    row scales, the stage rotation's signs and each group's fp32 table; semantic metadata {"matrices": ...} only
    (the random-initialised stack has no dense state to store). Returns write_artifact's receipt."""
    if out["L"] != artifact.STATE_BITS:
        raise ValueError("opgraph-packed-1 stores 12-bit trellis states")
    if int(out["bad"].item()):
        raise ValueError("states are not a row trellis from zero")
    tables = {b: np.asarray(t, dtype=np.float64).astype(np.float32) for b, t in out["tables"].items()}
    tensors, matrices = {}, {}
    for key, rec in out["codes"].items():
        i, nm = key.split(".", 1)
        name = f"model.layers.{i}.{nm}.weight"
        m, n = rec["states"].shape
        groups = [(np.asarray(gp["rows"], dtype=np.int64), int(gp["bits"]), "trellis", tables[int(gp["bits"])], words)
                  for gp, words in zip(rec["groups"], rec["packed"])]
        t, matrices[name] = artifact.encode_groups(name, (m, n), groups, rec["scales"].float().cpu().numpy(),
                                                   artifact._input_signs(n, rec["in_seed"]))
        tensors.update(t)
    return artifact.write_artifact(path, tensors, {"matrices": matrices})


def _stage_statistics(xq: list, w: list | None, xr: list, classes: list | None = None):
    """H = X_q^T W X_q / N and D = X_ref^T W X_q / N over the chunks (quantize.py:1416-1470), float64 on the GPU.
    classes: per chunk, engine.weight_classes(w[c], include_zero=True) (computed once per build)."""
    dev = xq[0].device
    n = xq[0].shape[1]
    H = torch.zeros(n, n, dtype=torch.float32, device=dev)
    D = torch.zeros(n, n, dtype=torch.float32, device=dev)
    ntok = 0
    for c, (a, b) in enumerate(zip(xq, xr)):
        a = a.contiguous()
        b = b.contiguous()
        wc = None if w is None else w[c]
        cc = None if classes is None else classes[c]
        E.hessian_accum(H, a, wc, classes=cc)
        E.cross_gram_accum(D, b, a, wc, classes=cc)
        ntok += a.shape[0]
    return E.hessian_finalize(H, float(ntok)), (D / ntok).double()


def _reconstruct(states: torch.Tensor, S: torch.Tensor, groups: list, tables: dict, in_seed: int) -> torch.Tensor:
    """W_hat = diag(S) table[states] R_in (codes.py:413-462 with out_rot=False), row group by row group."""
    dev = states.device
    Q = torch.empty(states.shape, dtype=torch.float64, device=dev)
    for gp in groups:
        rows = torch.as_tensor(gp["rows"], device=dev)
        tab = torch.as_tensor(np.asarray(tables[gp["bits"]]), dtype=torch.float64, device=dev)
        Q.index_copy_(0, rows, tab[states.index_select(0, rows).long()] * S.index_select(0, rows)[:, None])
    return E.rht_rows(Q, in_seed, inverse=True)


def calibration_tokens(sequences: int = 32, T: int = 2048, vocab: int = 151936, seed: int = 501, digit_share: float = 0.1,
                       digit_factor: float = 10.0):
    """Config 5's calibration: token ids uniform over the vocabulary (seed 501) and the digit weighting of
    config 3 (a random 10% of tokens weighted 10x, normalised to mean 1)."""
    rng = np.random.default_rng(seed)
    tok = torch.from_numpy(rng.integers(0, vocab, size=(sequences, T), dtype=np.int64))
    w = torch.from_numpy(synthetic.digit_weights(sequences * T, seed + 5, digit_share, digit_factor)).reshape(sequences, T)
    return tok, w


def stack_weights(sh: Shape = Shape(), layers: int | None = None) -> int:
    return (sh.layers if layers is None else layers) * sum(m * n for m, n in matrix_shapes(sh).values())

