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

from dataclasses import dataclass

import numpy as np
import torch

from . import artifact
from . import engine as E
from . import synthetic
from .quantize import (LAM, matrix_seeds, parse, qep_check, qep_factor, qep_targets, quantize_stage_row_groups,
                       stage_factor)
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


def rms_norm(x: torch.Tensor, g: torch.Tensor, eps: float, pad: bool = False) -> torch.Tensor:
    """Qwen3's RMSNorm in float32 and back: bf16(bf16(x rsqrt(mean(x^2) + eps)) g), one kernel (engine.rms_norm).
    pad: a stage input, whose rows are laid out engine.row_pad(n) elements apart for the Gram kernels."""
    return E.rms_norm(x, g, eps, E.row_pad(x.shape[-1]) if pad else 0)


def rope_tables(T: int, sh: Shape, dev):
    inv = 1.0 / (sh.rope_theta ** (torch.arange(0, sh.head_dim, 2, device=dev, dtype=torch.float32) / sh.head_dim))
    f = torch.outer(torch.arange(T, device=dev, dtype=torch.float32), inv)
    emb = torch.cat([f, f], -1)
    return emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)


def _lin(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """x W^T (x [.., n] bf16, W [m, n]) as a linear layer computes it: one 2-d product with W read transposed in
    place (no batched product, no copy of W per call)."""
    return torch.nn.functional.linear(x, w)


def attention(q, k, v, sh: Shape):
    """Causal grouped-query attention of [B, heads, T, head_dim] bf16 q and [B, kv_heads, T, head_dim] k, v (any
    strides with the head dim contiguous), fused in one kernel (engine.attention_causal: scores in registers, an
    online float32 softmax, bf16 probabilities times v). The one path of every forward here (no other backend, no
    fallback). Returns [B, heads, T, head_dim], a view of a [B, T, heads, head_dim] buffer."""
    return E.attention_causal(q, k, v, 1.0 / float(sh.head_dim) ** 0.5)


def attention_input_to_o(x: torch.Tensor, w: dict, sh: Shape, rope) -> torch.Tensor:
    """The o_proj input of one chunk [B, T, hidden] (normed hidden states in): q/k/v, per-head RMSNorm of q and k
    with the rotary embedding after it (one kernel each, the roundings of q_norm then q * cos + rotate_half(q) * sin),
    causal grouped-query attention."""
    B, T, _ = x.shape
    q = _lin(x, w["self_attn.q_proj"]).view(B, T, sh.heads, sh.head_dim)
    k = _lin(x, w["self_attn.k_proj"]).view(B, T, sh.kv_heads, sh.head_dim)
    v = _lin(x, w["self_attn.v_proj"]).view(B, T, sh.kv_heads, sh.head_dim)
    cos, sin = rope
    q = E.rms_norm_rope(q, w["self_attn.q_norm"], sh.eps, cos, sin).transpose(1, 2)
    k = E.rms_norm_rope(k, w["self_attn.k_norm"], sh.eps, cos, sin).transpose(1, 2)
    v = v.transpose(1, 2)
    out = attention(q, k, v, sh)
    return out.transpose(1, 2).reshape(B, T, sh.heads * sh.head_dim)


def _flat(x: torch.Tensor) -> torch.Tensor:
    return x.reshape(-1, x.shape[-1])


class Timer:
    """Seconds per phase of the build, from events recorded on the current stream at the phase boundaries: the GPU
    time from one boundary to the next, with no host synchronisation in the build (the events are read when `t` is)."""

    def __init__(self):
        self._spans, self._t = [], {}

    @staticmethod
    def mark() -> torch.cuda.Event:
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        return e

    def add(self, key: str, start: torch.cuda.Event, end: torch.cuda.Event):
        self._spans.append((key, start, end))

    @property
    def t(self) -> dict:
        for key, a, b in self._spans:
            b.synchronize()
            self._t[key] = self._t.get(key, 0.0) + a.elapsed_time(b) / 1e3
        self._spans = []
        return self._t

    def clear(self):
        self._spans, self._t = [], {}


def synthetic_plans(sh: Shape, layers: int, plan_seed: int = 7000, program: str = "tr2x"):
    """The synthetic build's plan and row plan: every linear of `layers` layers on `program` (the LM2 recipe's
    row-trellis codes with the QEP cross term), and per matrix a seeded 2.3 bpw row plan (synthetic.row_plan: eight
    groups, bits 1-4 drawn with the LM2 histogram), keyed as load_row_plan keys them."""
    shapes = matrix_shapes(sh)
    plan = {"linears": {f"{i}.{nm}": program for i in range(layers) for nm in shapes}}
    row_plan = {f"model.layers.{i}.{nm}.weight": synthetic.row_plan(shapes[nm][0], plan_seed + 10 * i + STAGE_INDEX[nm])
                for i in range(layers) for nm in shapes}
    return plan, row_plan


def active_shapes(sh: Shape, plan: dict, layers: int) -> dict:
    """{full parameter name: shape} of the matrices a plan quantizes with a trellis program: the matrices a row plan
    may name (quantize.py:1196-1207)."""
    shapes = matrix_shapes(sh)
    return {f"model.layers.{i}.{nm}.weight": shapes[nm] for i in range(layers) for nm in shapes
            if parse(plan["linears"][f"{i}.{nm}"])[0] == "tr"}


def trellis_window(window) -> tuple:
    """(width, look) of the stages' row trellis (quantize.py's --trellis-rows) as the fused row-group sweep takes it:
    1 to 16 columns settled at a time, dividing the 128-column lazy block, and width + look <= 24."""
    width, look = (int(v) for v in window)
    if not (1 <= width <= E.FUSED_WMAX and look >= 0 and width + look <= E.FUSED_TV and 128 % width == 0):
        raise NotImplementedError(f"the fused row-trellis kernels settle 1 to {E.FUSED_WMAX} columns dividing the "
                                  f"128-column block, width + look at most {E.FUSED_TV}; not ({width}, {look})")
    return width, look


class StackBuild:
    """The build of a random-initialised stack on calibration token ids [S, T], one decoder layer per call of
    layer(): per stage, the two streams' statistics, the QEP target of the matrices whose program asks for it, the
    codes of every matrix (row-trellis programs by their row-plan groups, in one batched sweep per stage; Lloyd-Max
    programs by the width-1 sweep on the stage's factor; fp16 programs kept) and the reconstruction written back, so
    the next stage's input already sees it; then both streams advance through the layer.

    plan: {"linears": {"i.name": program}} (the plan JSON of quantize.py --program plan; programs tr<k>[x],
    lm<b>[x], fp16; x: the QEP cross-term target W M at `alpha`); row_plan: {full parameter name: [{"group", "rows",
    "bits"}]} as load_row_plan returns it, for trellis matrices (a trellis matrix without one is a single group at its
    program's width). Both None: synthetic_plans() for the layers built.

    chunk: calibration sequences per forward pass (the default takes config 5's 32 x 2048 tokens in one: fewer,
    larger products). token_w: per-token weights [S, T] (mean 1), or None. keep: the first `keep` layers also return
    their stages' inputs and statistics under "stages" (for tests: {(i, s): {"Xq", "Xr" (the stage inputs of both
    streams, bf16 [tokens, n]), "H", "D" (float64), "targets" ({name: W*}), "in_seed", "plans" (the trellis matrices'
    row groups), "U", "dead" (the stage factor)}}, on the GPU). redamp: a stage whose damped statistics are not positive definite is damped x10 and x100
    (as ldlq_gpu.ldlq_factor retries, ldlq_gpu.py:19-23) and listed under "redamped"; without it (the default) it
    raises LinAlgError, as the reference's Environment does (frame.py:521-522). kernels: an engine.KernelTimer; every
    kernel of the stages then runs on the caller's stream, one after the other, each span timed with events and
    credited with its algorithmic work ("hessian" N n (n + 1) flops, "cross_gram" 2 N n^2, "chol" 4 n^3 / 3, "rht"
    HBM bytes, "qep_gemm", "block" trellis ops, "trailing" flops, "pack" bytes); without it the stage factor runs on a
    second stream next to the QEP targets and each stage's row groups are swept on streams of their own."""

    def __init__(self, tokens: torch.Tensor, sh: Shape = Shape(), token_w: torch.Tensor | None = None,
                 alpha: float = 0.5, L: int = 12, plan: dict | None = None, row_plan: dict | None = None,
                 plan_seed: int = 7000, chunk: int = 32, layers: int | None = None, weight_seed: int = 5000,
                 timer: Timer | None = None, keep: int = 0, redamp: bool = False, lam: float = LAM,
                 seed_set: int = 0, kernels: E.KernelTimer | None = None, window: tuple = (16, 8)):
        self.width, self.look = trellis_window(window)
        dev = E._abi.device()
        self.dev, self.sh, self.alpha, self.L, self.keep, self.redamp = dev, sh, alpha, L, keep, redamp
        self.lam, self.seed_set, self.kernels = lam, seed_set, kernels
        self.weight_seed = weight_seed
        self.layers = sh.layers if layers is None else layers
        if plan is None and row_plan is None:
            plan, row_plan = synthetic_plans(sh, self.layers, plan_seed)
        elif plan is None:
            raise ValueError("a row plan needs the plan it refines")
        for i in range(self.layers):
            for nm in matrix_shapes(sh):
                fam = parse(plan["linears"][f"{i}.{nm}"])[0]
                if fam not in ("tr", "lm", "fp"):
                    raise NotImplementedError(f"program family {fam!r} is not part of this path")
        self.plan, self.row_plan = plan, row_plan or {}
        self.main = torch.cuda.current_stream(dev)
        self.side = torch.cuda.Stream(dev)  # default priority
        self.timer = timer or Timer()
        self.tables = {b: (quantile_table(16, 0) if L == 16 else load_table(12, b)) for b in (1, 2, 3, 4)}
        S_, T = tokens.shape
        self.rope = tuple(t.to(dev) for t in rope_tables(T, sh, dev))
        chunks = [slice(c, min(c + chunk, S_)) for c in range(0, S_, chunk)]
        self.wt = None if token_w is None else [token_w[cs].reshape(-1).to(dev, torch.float32) for cs in chunks]
        self.wcls = None if self.wt is None else [E.weight_classes(wc, include_zero=True) for wc in self.wt]
        # the embedding (shared by both streams: it is not quantized here)
        g = torch.Generator(device=dev).manual_seed(weight_seed * 1000 + 999)
        emb = (torch.randn(sh.vocab, sh.hidden, generator=g, device=dev, dtype=torch.float32) * sh.std).to(torch.bfloat16)
        self.hq = [emb[tokens[cs].to(dev)] for cs in chunks]
        self.hr = [h.clone() for h in self.hq]
        del emb
        self.codes, self.n_w, self.bits, self.kept, self.redamped = {}, 0, 0.0, {}, {}
        self.bad = torch.zeros(1, dtype=torch.int32, device=dev)  # set if a packed row is not a trellis path from 0
        self.next_layer = 0

    def program(self, i: int, nm: str) -> str:
        return self.plan["linears"][f"{i}.{nm}"]

    def device_tables(self) -> dict:
        """The trellis tables as float64 tensors on the device, made once."""
        if getattr(self, "_dtables", None) is None:
            # (np.array copies: the cached tables are read-only)
            self._dtables = {b: torch.from_numpy(np.array(t, dtype=np.float64)).to(self.dev)
                             for b, t in self.tables.items()}
        return self._dtables

    def groups(self, i: int, nm: str) -> list:
        """The row groups of a trellis matrix: its row-plan entry, else one group at its program's width."""
        g = self.row_plan.get(f"model.layers.{i}.{nm}.weight")
        if g is not None:
            return g
        m = matrix_shapes(self.sh)[nm][0]
        return [{"group": 0, "rows": list(range(m)), "bits": parse(self.program(i, nm))[1]}]

    @torch.no_grad()
    def layer(self) -> int:
        """Builds the next layer; returns its index."""
        i = self.next_layer
        if i >= self.layers:
            raise ValueError(f"the stack has {self.layers} layers")
        sh, dev, timer = self.sh, self.dev, self.timer
        t0 = timer.mark()
        wr = layer_weights(i, sh, dev, self.weight_seed)  # the reference layer
        wq = {k: v.clone() for k, v in wr.items()}  # quantized in place, stage by stage
        # the reference stream's stage inputs (its weights never change) and its output
        xr = {s: [] for s in range(4)}
        hr_next = []
        for h in self.hr:
            x1 = rms_norm(h, wr["input_layernorm"], sh.eps, pad=True)
            a = attention_input_to_o(x1, wr, sh, self.rope)
            h1 = h + _lin(a, wr["self_attn.o_proj"])
            x2 = rms_norm(h1, wr["post_attention_layernorm"], sh.eps, pad=True)
            m = E.swiglu(_lin(x2, wr["mlp.gate_proj"]), _lin(x2, wr["mlp.up_proj"]))
            hr_next.append(h1 + _lin(m, wr["mlp.down_proj"]))
            for s, x in enumerate((x1, a, x2, m)):
                xr[s].append(_flat(x))
        timer.add("forward", t0, timer.mark())
        # the quantized stream, stage by stage
        hq = self.hq
        h1q = [None] * len(hq)
        x2q = [None] * len(hq)
        for s, names in enumerate(STAGES):
            t1 = timer.mark()
            if s == 0:
                xq = x1q = [rms_norm(h, wq["input_layernorm"], sh.eps, pad=True) for h in hq]
            elif s == 1:
                xq = aq = [attention_input_to_o(x, wq, sh, self.rope) for x in x1q]
            elif s == 2:
                h1q = [h + _lin(a, wq["self_attn.o_proj"]) for h, a in zip(hq, aq)]
                xq = x2q = [rms_norm(h, wq["post_attention_layernorm"], sh.eps, pad=True) for h in h1q]
            else:
                xq = mq = [E.swiglu(_lin(x, wq["mlp.gate_proj"]), _lin(x, wq["mlp.up_proj"])) for x in x2q]
            xqf = [_flat(x) for x in xq]
            timer.add("forward", t1, timer.mark())
            self._stage(i, s, names, xqf, xr[s], wr, wq)
            del xq, xqf
        # both streams through the layer (the quantized one with its last matrix now quantized); the MLP's gate and up
        # were quantized before the down stage, so its input (the down stage's) is the quantized stream's MLP
        # activation as it stands
        t4 = timer.mark()
        self.hq = [h1 + _lin(m, wq["mlp.down_proj"]) for h1, m in zip(h1q, mq)]
        self.hr = hr_next
        del xr, wr, wq, h1q, x2q, mq
        timer.add("forward", t4, timer.mark())
        self.next_layer = i + 1
        return i

    def _stage(self, i, s, names, xqf, xrf, wr, wq):
        dev, timer, L = self.dev, self.timer, self.L
        shapes = matrix_shapes(self.sh)
        progs = {nm: self.program(i, nm) for nm in names}
        coded = [nm for nm in names if parse(progs[nm])[0] != "fp"]
        for nm in names:
            if nm not in coded:  # fp16: the bf16 weights stay as they are, at 16 bits per weight
                self.n_w += shapes[nm][0] * shapes[nm][1]
                self.bits += 16.0 * shapes[nm][0] * shapes[nm][1]
        if not coded:
            return
        t2 = timer.mark()
        kt = self.kernels
        cross = [nm for nm in coded if parse(progs[nm])[2]]
        H, D = _stage_statistics(xqf, self.wt, xrf if cross else None, self.wcls, kt)
        t25 = timer.mark()
        timer.add("statistics", t2, t25)
        _, in_seed = matrix_seeds(i, names[0], 0, names[0], self.seed_set)
        qf = None
        if kt is None:
            # the stage's factor (rotation of H, damped inverse factor) on a second stream, next to the QEP targets
            # (their own factor of H + lambda I and products) on this one: the two are independent. Neither factor
            # is checked until the sweep is enqueued, so the host does not wait for the stream before then.
            self.side.wait_stream(self.main)
            with torch.cuda.stream(self.side):
                factor = stage_factor(H, in_seed, 0.01)
                f_bad = _flag_later(factor[2])
            if cross:
                qf = qep_factor(H, self.lam)
                q_bad = _flag_later(qf[1])
        else:
            factor = stage_factor(H, in_seed, 0.01, kt)
        targets = {}
        if cross:
            targets = qep_targets(H, D - H, self.alpha, {nm: wr[nm] for nm in cross}, self.lam, kt,
                                  U=None if qf is None else qf[0])
        for nm in coded:
            if nm not in targets:
                targets[nm] = wr[nm].double()
        if kt is None:
            self.main.wait_stream(self.side)
            for t in factor:
                t.record_stream(self.main)
        t3 = timer.mark()
        timer.add("qep_targets", t25, t3)
        trellis = [nm for nm in coded if parse(progs[nm])[0] == "tr"]
        plans = {nm: self.groups(i, nm) for nm in trellis}
        key = f"{i}.{names[0]}"
        if kt is not None:
            factor = self._factor(H, in_seed, factor, key)
        sweep = lambda f: quantize_stage_row_groups({nm: targets[nm] for nm in trellis}, plans, H, in_seed, L=L,
                                                    width=self.width, look=self.look,
                                                    tables=self.device_tables(), factor=f, timer=kt,
                                                    check=kt is not None)
        res = sweep(factor) if trellis else {}
        if kt is None:
            # the factors' checks, the sweep already queued behind them: a failed QEP factor raises (as the
            # factorization does), a failed stage factor is damped more and the stage swept again before anything
            # reads the results
            if qf is not None and q_bad():
                qep_check(qf[1])
            checked = self._factor(H, in_seed, factor, key, f_bad())
            if checked is not factor:
                factor = checked
                res = sweep(factor) if trellis else {}
        if trellis:
            if kt is not None:  # the sweep's algorithmic work: trellis ops and trailing-update flops per width
                n = shapes[trellis[0]][1]
                steps = sum(E.trellis_row_steps(n))
                for bits in sorted({int(g["bits"]) for nm in trellis for g in plans[nm]}):
                    m = sum(len(g["rows"]) for nm in trellis for g in plans[nm] if int(g["bits"]) == bits)
                    kt.add_work("block", m * sum(E.trellis_block_ops(n, L, bits)))  # reachable states
                    kt.add_work("block_full", m * steps * E.viterbi_ops_per_row_step(L, bits))  # every state
                    kt.add_work("trailing", E.trailing_flops(m, n))
        if i < self.keep:
            self.kept[(i, s)] = {"Xq": torch.cat(xqf), "Xr": torch.cat(xrf), "H": H, "D": D, "targets": targets,
                                 "in_seed": in_seed, "plans": plans, "U": factor[0], "dead": factor[1]}
        pack_items, pack_work = [], 0.0  # every row group of the stage's matrices, packed in one launch below
        for nm in trellis:
            st, Srow = res[nm]
            m, n = st.shape
            Q = _decode(st, Srow, plans[nm], self.device_tables())
            with E.span(kt, "rht", E.rht_flops(m, n)):
                Wh = E.rht_rows(Q, in_seed, inverse=True)
            wq[nm] = Wh.to(torch.bfloat16)
            for gp, rows in zip(plans[nm], E.device_rows(plans[nm], dev)):
                r = len(gp["rows"])
                pack_items.append((st, gp["bits"], rows, 0))
                pack_work += 4.0 * r * n + 4.0 * r * ((n + 31) // 32) * gp["bits"]
                self.bits += r * n * gp["bits"] + 16 * r
            self.codes[f"{i}.{nm}"] = {"kind": "trellis", "states": st, "scales": Srow, "in_seed": in_seed,
                                       "groups": plans[nm], "packed": []}
            self.n_w += shapes[nm][0] * shapes[nm][1]
            if i < self.keep:  # the weights the quantized stream goes on with (bf16 of the decoded reconstruction)
                self.kept[(i, s)].setdefault("Wq", {})[nm] = wq[nm]
        if pack_items:
            with E.span(kt, "pack", pack_work):
                packed, _ = E.pack_codes_groups(pack_items, L=L, bad=self.bad)
            for nm in trellis:
                self.codes[f"{i}.{nm}"]["packed"] = packed[: len(plans[nm])]
                packed = packed[len(plans[nm]) :]
        for nm in coded:
            if parse(progs[nm])[0] != "lm":
                continue
            b = parse(progs[nm])[1]
            idx, Srow, levels = _lloyd_max_codes(targets[nm], factor, in_seed, b)
            Q = levels[idx.long()] * Srow[:, None]
            wq[nm] = E.rht_rows(Q, in_seed, inverse=True).to(torch.bfloat16)
            m, n = idx.shape
            self.codes[f"{i}.{nm}"] = {"kind": "scalar", "states": idx, "scales": Srow, "in_seed": in_seed,
                                       "groups": [{"group": 0, "rows": list(range(m)), "bits": b}],
                                       "levels": levels, "packed": [E.pack_codes(idx, b, trellis=False, bad=self.bad)[0]]}
            self.bits += m * n * b + 16 * m
            self.n_w += m * n
        timer.add("quantize", t3, timer.mark())

    def _factor(self, H, in_seed, factor, key, bad: int | None = None):
        """The stage factor at the Environment's damping; with redamp, x10 and x100 more where that is not positive
        definite (one host synchronisation reads the pivot flag, unless the caller has read it: bad)."""
        U, dead, info = factor
        if (int(info.item()) if bad is None else bad) == 0:
            return factor
        if not self.redamp:
            raise E.LinAlgError(f"stage {key}: linalg.cholesky: the leading minor of order {int(info.item())} is not "
                                "positive-definite")
        for d in (0.1, 1.0):
            f = stage_factor(H, in_seed, d)
            if int(f[2].item()) == 0:
                self.redamped[key] = d
                return f
        raise E.LinAlgError(f"stage {key}: not positive definite even at damping 1.0")

    def result(self) -> dict:
        return {"codes": self.codes, "weights": self.n_w, "bits": self.bits, "stages": self.kept,
                "redamped": self.redamped, "bad": self.bad, "L": self.L, "tables": self.tables,
                "layers": self.next_layer}


def build(tokens: torch.Tensor, sh: Shape = Shape(), token_w: torch.Tensor | None = None, alpha: float = 0.5,
          L: int = 12, plan: dict | None = None, row_plan: dict | None = None, plan_seed: int = 7000, chunk: int = 32,
          layers: int | None = None, weight_seed: int = 5000, timer: Timer | None = None, keep: int = 0,
          redamp: bool = False, lam: float = LAM, seed_set: int = 0, window: tuple = (16, 8)) -> dict:
    """The whole build of a random-initialised stack (StackBuild, layer after layer). Returns {"codes": {"i.name":
    {"kind": "trellis" | "scalar", "states": int32 [m, n] (trellis states, or Lloyd-Max level indices), "scales":
    float64 [m], "in_seed", "groups": the row groups, "packed": per group the code words (engine.pack_codes, read in
    place), "levels" (scalar)}}, "weights": n, "bits": total rate bits, "redamped": {"i.first matrix": damping} (with
    redamp), "bad": a device flag set if any packed row was not a trellis path, "L", "tables", "layers"};
    export_codes writes the codes as an opgraph-packed-1 artifact and saved_codes as the reference's --save-codes
    dictionary."""
    b = StackBuild(tokens, sh, token_w, alpha, L, plan, row_plan, plan_seed, chunk, layers, weight_seed, timer, keep,
                   redamp, lam, seed_set, window=window)
    for _ in range(b.layers):
        b.layer()
    return b.result()


def _lloyd_max_codes(target: torch.Tensor, factor: tuple, in_seed: int, b: int):
    """An lm<b> word of one matrix on the stage's factor (quantize.py:332-347, nested.py:155-192 with one rate and
    out_rot=False): the rotated rows X = W R_in^T, their RMS scales S, the width-1 LDLQ of X / S onto the Lloyd-Max
    levels (first minimum). Returns (indices int32 [m, n], S float64 [m], levels float64 [2^b]), on the GPU."""
    from . import nested as N

    U, dead, _ = factor
    X, S = E.rht_rows(torch.as_tensor(target).to(U.device, torch.float64).contiguous(), in_seed, want_rms=True)
    levels = torch.as_tensor(N.lloyd_max(b), dtype=torch.float64).to(U.device).contiguous()
    idx = E.ldlq_scalar((X / S[:, None]).contiguous(), U, levels, mode=0, dead=dead)
    return idx, S, levels


STAGE_INDEX = {nm: j for j, nm in enumerate(n for st in STAGES for n in st)}


def export_codes(out: dict, path) -> dict:
    """The build's codes as an opgraph-packed-1 artifact at `path` (compiler_artifact.py:307-371, 491-531): per
    matrix model.layers.{i}.{name}.weight, its row groups in plan order with the words packed during the build, fp32
    row scales, the stage rotation's signs and each group's fp32 table (trellis) or levels (scalar); semantic
    metadata {"matrices": ...} only (the random-initialised stack has no dense state to store). Returns
    write_artifact's receipt."""
    if int(out["bad"].item()):
        raise ValueError("states are not a row trellis from zero")
    if any(rec["kind"] == "trellis" for rec in out["codes"].values()) and out["L"] != artifact.STATE_BITS:
        raise ValueError("opgraph-packed-1 stores 12-bit trellis states")
    tables = {b: np.asarray(t, dtype=np.float64).astype(np.float32) for b, t in out["tables"].items()}
    tensors, matrices = {}, {}
    for key, rec in out["codes"].items():
        i, nm = key.split(".", 1)
        name = f"model.layers.{i}.{nm}.weight"
        m, n = rec["states"].shape
        if rec["kind"] == "trellis":
            groups = [(np.asarray(gp["rows"], dtype=np.int64), int(gp["bits"]), "trellis", tables[int(gp["bits"])],
                       words) for gp, words in zip(rec["groups"], rec["packed"])]
        else:
            lv = rec["levels"].float().cpu().numpy()
            groups = [(np.arange(m, dtype=np.int64), int(rec["groups"][0]["bits"]), "scalar", lv, rec["packed"][0])]
        t, matrices[name] = artifact.encode_groups(name, (m, n), groups, rec["scales"].float().cpu().numpy(),
                                                   artifact._input_signs(n, rec["in_seed"]))
        tensors.update(t)
    return artifact.write_artifact(path, tensors, {"matrices": matrices})


SOURCE_MODEL = "random-initialised Qwen3.5-4B-shaped stack (hidden 2560, GQA 32/8 x 128, MLP 9728)"


def saved_codes(out: dict, row_plan: dict | None = None, calibration: dict | None = None) -> dict:
    """The build's codes as the reference's --save-codes file (quantize.py:1737-1739): {"matrices": per full parameter
    name, a row-trellis entry {"states": int16 [m, n] (state + 4096 * table_index), "scales": float32 [m], "in_seed",
    "table": float32 [4096 * groups], "row_groups": [{"rows", "bits", "table_index"}], "trellis_layout": "row"} or a
    scalar entry {"codes": uint8 [m, n], "scales", "in_seed", "levels": float32} (quantize.py:513-565, 1541-1553), on
    the CPU; "model": the source model; the evaluation record of a run that skipped evaluation; "text weights";
    "calibration"; and "row plan" (the validated row plan's manifest) when the build followed one}. Its consumers read
    saved["matrices"] (compiler_artifact.export_saved_codes, finetune.py:114-115)."""
    saved = {}
    for key, rec in out["codes"].items():
        i, nm = key.split(".", 1)
        name = f"model.layers.{i}.{nm}.weight"
        if rec["kind"] == "scalar":
            saved[name] = {"codes": rec["states"].cpu().to(torch.uint8), "scales": rec["scales"].float().cpu(),
                           "in_seed": int(rec["in_seed"]), "levels": rec["levels"].float().cpu()}
            continue
        if out["L"] != 12:
            raise ValueError("saved row-group codes require a 12-bit state table")
        st = rec["states"].cpu()
        states = torch.empty(st.shape, dtype=torch.int16)
        tabs, groups = [], []
        for ti, gp in enumerate(rec["groups"]):
            rows = torch.as_tensor(gp["rows"], dtype=torch.long)
            states[rows] = (st[rows] + 4096 * ti).to(torch.int16)
            tabs.append(torch.tensor(np.asarray(out["tables"][int(gp["bits"])], dtype=np.float32)))
            groups.append({"rows": rows, "bits": int(gp["bits"]), "table_index": ti})
        saved[name] = {"states": states, "scales": rec["scales"].float().cpu(), "in_seed": int(rec["in_seed"]),
                       "table": torch.cat(tabs), "row_groups": groups, "trellis_layout": "row"}
    # (quantize.py:1734: a run without evaluation records it so; this path has no text data to evaluate on)
    payload = {"matrices": saved, "model": SOURCE_MODEL, "evaluation": "skipped: no evaluation on this path",
               "eval": 0, "ctx": None, "text weights": None, "calibration": calibration}
    if row_plan is not None:
        payload["row plan"] = row_plan
    return payload


def _flag_later(t: torch.Tensor):
    """A one-element int32 device flag copied to pinned host memory on the current stream, an event after the copy;
    the returned function waits for that event only (not for what the stream does later) and gives the value."""
    h = torch.empty(1, dtype=torch.int32, pin_memory=True)
    h.copy_(t, non_blocking=True)
    ev = torch.cuda.Event()
    ev.record()
    return lambda: (ev.synchronize(), int(h[0]))[1]


def _stage_statistics(xq: list, w: list | None, xr: list | None, classes: list | None = None,
                      kt: E.KernelTimer | None = None):
    """H = X_q^T W X_q / N and D = X_ref^T W X_q / N (None without xr) over the chunks (quantize.py:1416-1470),
    float64 on the GPU. classes: per chunk, engine.weight_classes(w[c], include_zero=True) (computed once per
    build). kt: spans "hessian" (N n (n + 1) flops, the unique entries) and "cross_gram" (2 N n^2 flops)."""
    dev = xq[0].device
    n = xq[0].shape[1]
    H = torch.zeros(n, n, dtype=torch.float32, device=dev)
    D = None if xr is None else torch.zeros(n, n, dtype=torch.float32, device=dev)
    ntok = 0
    for c, a in enumerate(xq):
        if a.stride(-1) != 1:
            a = a.contiguous()  # rows may stay strided (padded stage inputs), the elements of a row not
        N = a.shape[0]
        wc = None if w is None else w[c]
        cc = None if classes is None else classes[c]
        b = None
        if D is not None:
            b = xr[c]
            if b.stride(-1) != 1 or b.stride(0) != a.stride(0):  # the cross-Gram reads both with one row stride
                a, b = a.contiguous(), b.contiguous()
        with E.span(kt, "hessian", float(N) * n * (n + 1)):
            E.hessian_accum(H, a, wc, classes=cc)
        if D is not None:
            with E.span(kt, "cross_gram", 2.0 * N * n * n):
                E.cross_gram_accum(D, b, a, wc, classes=cc)
        ntok += N
    return E.hessian_finalize(H, float(ntok)), None if D is None else (D / ntok).double()


def _decode(states: torch.Tensor, S: torch.Tensor, groups: list, tables: dict) -> torch.Tensor:
    """diag(S) table[states], each row through its group's table: tables {bits: float64 table on the device}. The
    tables are read as one concatenation, each row's states offset to its width's table, in one gather."""
    dev = states.device
    widths = sorted(tables)
    cat = torch.cat([tables[b] for b in widths])
    size = tables[widths[0]].numel()
    m = states.shape[0]
    base = torch.empty(m, dtype=torch.int64, pin_memory=True)
    seen = np.zeros(m, dtype=np.int64)
    for gp in groups:
        rows = np.asarray(gp["rows"], dtype=np.int64)
        if rows.size and (rows.min() < 0 or rows.max() >= m):
            raise ValueError("row group names a row outside the matrix")
        np.add.at(seen, rows, 1)
        base.numpy()[rows] = widths.index(int(gp["bits"])) * size
    if not (seen == 1).all():  # (quantize.py:530-565: the groups cover every row exactly once)
        raise ValueError("row groups do not cover every row exactly once")
    base = base.to(dev, non_blocking=True)
    return cat[states.long() + base[:, None]] * S[:, None]


def _reconstruct(states: torch.Tensor, S: torch.Tensor, groups: list, tables: dict, in_seed: int) -> torch.Tensor:
    """W_hat = diag(S) table[states] R_in (codes.py:413-462 with out_rot=False)."""
    dev = states.device
    dt = {b: torch.from_numpy(np.array(t, dtype=np.float64)).to(dev) for b, t in tables.items()}
    return E.rht_rows(_decode(states, S, groups, dt), in_seed, inverse=True)


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

