"""The trellis and the LDLQ words with the reference's signatures (opgraph/codes.py), on the gfx950 kernels.

    viterbi(X, values, L, k, chunk=None, start=None)                      codes.py:151
    trellis_values(L, k, T=256, seed=0, refine=None, fit=None)             codes.py:187 (cached, else fitted)
    is_trellis_path(states, L, k)                                          codes.py:246
    ScalarCode(domain), RowTrellisCode(L, k, T=256, width=16, look=8, seed=0, values=None)   codes.py:322,386
    TrellisCode(L, k, T=320, width=16, seed=0, values=None)                codes.py:363
    ldlq_words(Ws, H, code, seeds, incoherent=True, in_seed=None, out_rot=True) -> list[Net] codes.py:413
    ldlq_word(W, H, code, seed, incoherent=True)                           codes.py:465
    hadamard, hadamard_factors, rht                                        codes.py:83-132

Differences a caller can see: results are computed on the GPU whatever device the inputs are on (Net cores are
returned on the CPU, as the reference returns them); a word also carries its integer codes (`net.codes`: trellis
states or level indices) so they need not be recovered from values (which is ambiguous for tables with repeated
values)."""

from __future__ import annotations

import math

from functools import lru_cache

import numpy as np
import torch

from . import engine as E
from .frame import REAL, RHT, Core, Domain, Net, Rotation
from .hadamard import hadamard, hadamard_factors, rht  # noqa: F401  (re-exported, codes.py:83-132)
from .tables import load_table, quantile_table

TRELLIS_FIT = "ema"


def SET(levels, name: str | None = None, bits: float | None = None) -> Domain:
    """A finite value set, sorted and without repeats (opgraph/verbs.py:36-38)."""
    lv = tuple(sorted({float(x) for x in levels}))
    return Domain("set", float(math.ceil(math.log2(len(lv)))) if bits is None else bits, lv[0], lv[-1], levels=lv)


GAUSS2 = SET([-1.5104, -0.4528, 0.4528, 1.5104])  # Lloyd-Max for N(0, 1) at 2 bits (Max, 1960)


def TRELLIS(values, L: int, k: int, axis: str = "t", fixed_start: bool = False) -> Domain:
    return Domain("trellis", float(k), levels=tuple(float(v) for v in values), axis=axis, state_bits=L,
                  fixed_start=fixed_start)


# ----------------------------------------------------------------------------- the trellis


def _rows_per_pass(T: int, L: int, k: int, big: bool) -> int:
    """Rows per kernel launch so that long paths' back-pointer workspace stays within 1 GiB (big: the 2^13..2^16-state
    kernels take the search)."""
    per = E.lib().lamq_viterbi16_workspace_size(1, T, L, k) if big else E.lib().lamq_viterbi_workspace_size(1, T, L, k)
    return max(1, (1 << 30) // per) if per else 1 << 20


def viterbi(X: torch.Tensor, values: torch.Tensor, L: int, k: int, chunk: int | None = None,
            start: torch.Tensor | None = None) -> torch.Tensor:
    """The path through a bitshift trellis nearest each row of X in squared error (codes.py:151-181): X and the
    values are cast to float32; ties go to the lowest predecessor and the lowest final state. Returns the states
    (rows, T) as int64 on X's device."""
    dev = E._abi.device()
    values = torch.as_tensor(values)
    C = values.to(dev, torch.float64).to(torch.float32).contiguous()
    C16 = E.half_bits(C) if E.search16(L, k, C) else None
    x = X.to(dev).to(torch.float32).contiguous()
    st = None if start is None else torch.as_tensor(start).to(dev, torch.int32).contiguous()
    B, T = x.shape
    out = torch.empty(B, T, dtype=torch.int64, device=X.device)
    step = min(chunk or (1 << 30), _rows_per_pass(T, L, k, C16 is not None))
    for b in range(0, B, step):
        e = min(b + step, B)
        s = E.viterbi_rows(x[b:e], C, L, k, None if st is None else st[b:e], C16=C16)
        out[b:e] = s.to(torch.int64).to(X.device)
    return out


def trellis_values(L: int, k: int, T: int = 256, seed: int = 0, refine: int | None = None, fit: str | None = None) -> torch.Tensor:
    """A value for each of the 2^L states (codes.py:187-220), float64. The tables the reference has fitted and
    cached (L = 12, k = 1..4, T = 256, seed 0, fit "ema") are served as stored; any other (L, k, T, seed, refine, fit)
    is fitted on the GPU (fit.fit_table, the reference's procedure; refitting a cached table reproduces it to within
    4 units in the last place) and kept for the life of the process (the reference writes it into its cache)."""
    fit = fit or TRELLIS_FIT
    if refine is None:
        try:
            return torch.from_numpy(np.array(load_table(L, k, T, seed, fit)))
        except FileNotFoundError:
            pass
    return torch.from_numpy(_fitted(L, k, T, seed, refine, fit).copy())


@lru_cache(maxsize=16)
def _fitted(L, k, T, seed, refine, fit):
    from .fit import fit_table

    v = fit_table(L, k, T, seed, refine, fit)
    v.setflags(write=False)
    return v


def trellis_init_values(L: int, seed: int = 0, dtype: str = "float64") -> torch.Tensor:
    """The initial table of codes.py:202-204: ndtri((randperm(2^L, Generator(seed)) + 0.5) / 2^L), cast to `dtype`
    (float16 gives the 16-bit configurations' table)."""
    if dtype == "float64":
        S = 1 << L
        g = torch.Generator().manual_seed(int(seed))
        return torch.special.ndtri((torch.randperm(S, generator=g).double() + 0.5) / S)
    return torch.from_numpy(np.array(quantile_table(L, seed, dtype)))


def is_trellis_path(states: torch.Tensor, L: int, k: int) -> bool:
    """Every step keeps the previous state's low L - k bits as its high bits (codes.py:246-248)."""
    s = torch.as_tensor(states)
    return bool(torch.all((s[..., 1:] >> k) == (s[..., :-1] & ((1 << (L - k)) - 1))))


# ----------------------------------------------------------------------------- codes


class ScalarCode:
    """Each entry onto a finite set, width 1 (codes.py:322-332): the nearest level of x/S, halfway to the lower."""

    def __init__(self, domain: Domain):
        self.domain, self.width = domain, 1

    def project(self, X: torch.Tensor) -> torch.Tensor:
        lv = torch.tensor(self.domain.levels, dtype=X.dtype, device=X.device)
        return lv[torch.bucketize(X.contiguous(), (lv[1:] + lv[:-1]) / 2)]


class RowTrellisCode:
    """Each row one trellis path along its columns from state 0 (codes.py:386-410): block LDLQ settles `width`
    columns at a time, each block's search looking `look` columns ahead at their targets as they stand.
    `values` overrides the cached table (e.g. trellis_init_values(16, 0, "float16") for 16-bit states)."""

    def __init__(self, L: int, k: int, T: int = 256, width: int = 16, look: int = 8, seed: int = 0, values=None):
        self.L, self.k, self.width, self.look = L, k, width, look
        self.values = trellis_values(L, k, T, seed) if values is None else torch.as_tensor(values, dtype=torch.float64)
        if len(self.values) != 1 << L:
            raise ValueError("a table needs 2^L values")
        self.domain = TRELLIS(self.values, L, k, fixed_start=True)
        self.state = None

    def step(self, j, X, ahead):
        """Column j onward, `width` columns: the block's settled values, continuing each row's path
        (codes.py:397-404)."""
        if j == 0:
            self.state = torch.zeros(len(X), dtype=torch.long, device=X.device)
        w = X.shape[1]
        path = viterbi(torch.cat([X, ahead], 1), self.values, self.L, self.k, start=self.state)[:, :w]
        self.state = path[:, -1]
        return self.values.to(X.device, X.dtype)[path]


class TrellisCode:
    """Sequences of T consecutive outputs (one column) onto trellis paths with a free first state (codes.py:363-383):
    block LDLQ settles `width` columns at a time, each column of the block cut into m/T sequences searched
    independently. The rows must come in whole sequences (m a multiple of T)."""

    def __init__(self, L: int, k: int, T: int = 320, width: int = 16, seed: int = 0, values=None):
        self.L, self.k, self.T, self.width = L, k, T, width
        self.values = trellis_values(L, k, T, seed) if values is None else torch.as_tensor(values, dtype=torch.float64)
        if len(self.values) != 1 << L:
            raise ValueError("a table needs 2^L values")
        self.domain = TRELLIS(self.values, L, k)

    def _seqs(self, X: torch.Tensor) -> torch.Tensor:
        o, w = X.shape
        if o % self.T:
            raise ValueError(f"{o} rows are not whole sequences of {self.T}")
        return X.reshape(o // self.T, self.T, w).permute(0, 2, 1).reshape(-1, self.T)

    def states(self, X: torch.Tensor) -> torch.Tensor:
        """The states of every column's sequences, in X's layout (rows x columns)."""
        o, w = X.shape
        st = viterbi(self._seqs(X), self.values, self.L, self.k)
        return st.reshape(o // self.T, w, self.T).permute(0, 2, 1).reshape(o, w)

    def project(self, X: torch.Tensor) -> torch.Tensor:
        return self.values.to(X.device, X.dtype)[self.states(X)]


# ----------------------------------------------------------------------------- words


def _levels_of(code) -> torch.Tensor:
    return torch.tensor(code.domain.levels, dtype=torch.float64)


def _prepare(Ws, seeds, incoherent, in_seed, out_rot):
    dev = E._abi.device()
    Ws = [torch.as_tensor(W).to(dev, torch.float64).contiguous() for W in Ws]
    n = Ws[0].shape[1]
    if any(W.shape[1] != n for W in Ws):
        raise ValueError("matrices of one word read the same input")
    rin = (seeds[0] + 1 if in_seed is None else in_seed) if incoherent else None
    Xs = []
    for W, s in zip(Ws, seeds):
        X = W
        if incoherent:
            X = E.rht_rows(X, rin)  # W R_in^T
            if out_rot:
                X = E.rotate_columns(X, s)  # R_out W R_in^T
        Xs.append(X)
    X = torch.cat(Xs) if len(Xs) > 1 else Xs[0]
    S = E.row_rms(X)
    return dev, X, S, rin


def _nets(Ws, seeds, X_codes, values, S, domain, rows_label, rin, out_rot, incoherent, codes):
    nets, r0 = [], 0
    for W, s in zip(Ws, seeds):
        m = W.shape[0]
        r1 = r0 + m
        cores = {"W": Core(values[r0:r1].clone(), (rows_label, "v" if incoherent else "i"), domain),
                 "W.S": Core(S[r0:r1].clone(), (rows_label,), REAL)}
        rot_in = rot_out = None
        if incoherent:
            rot_in = Rotation(W.shape[1], rin)
            cores["I[v]"] = Core(torch.ones(W.shape[1]), ("v", "i"), RHT)
            if out_rot:
                rot_out = Rotation(m, s)
                cores["I[u]"] = Core(torch.ones(m), ("o", "u"), RHT)
        nets.append(Net(cores, rows_label, rot_in, rot_out, codes[r0:r1].clone()))
        r0 = r1
    return nets


def _row_trellis_sweep(X: torch.Tensor, S: torch.Tensor, Hr: torch.Tensor, code, table: torch.Tensor) -> torch.Tensor:
    """States of a row trellis the fused kernels do not take (k = 5..8, other widths and look-aheads): the generic
    sweep (syntax.sweep: the refit and the lazy trailing update on the GPU), each block settled as
    RowTrellisCode.step settles it (codes.py:397-404, driven by the project of codes.py:441-448): the standalone search
    over the block's columns and the next `look` as they stand, divided by the row scale, from each row's state."""
    from .frame import Environment
    from .syntax import sweep

    m, n = X.shape
    codes = torch.empty(m, n, dtype=torch.int32, device=X.device)
    state = torch.zeros(m, dtype=torch.long, device=X.device)

    def project(j, x, T):
        xs = x[:, None] if x.dim() == 1 else x
        w = xs.shape[1]
        seq = torch.cat([xs, T[:, j + w : j + w + code.look]], 1) / S[:, None]
        path = viterbi(seq, code.values, code.L, code.k, start=state)[:, :w]
        state.copy_(path[:, -1])
        codes[:, j : j + w] = path.to(torch.int32)
        q = table[path] * S[:, None]
        return q[:, 0] if x.dim() == 1 else q

    sweep(X, Environment(Hr), project, width=code.width)
    return codes


def ldlq_words(Ws: list, H: torch.Tensor | None, code, seeds: list[int], incoherent: bool = True,
               in_seed: int | None = None, out_rot: bool = True) -> list[Net]:
    """(incoherence ->) per-row RMS scale -> (block LDLQ under H ->) the code, for matrices that read the same input
    (codes.py:413-462). With H the columns are settled code.width at a time and the later ones re-solved under U;
    without H the code is applied directly. Row trellis and scalar codes run on the fused GPU sweep kernels; row
    trellises those do not take (k = 5..8, other block widths and look-aheads) on the generic sweep with the standalone
    search (_row_trellis_sweep)."""
    if not isinstance(code, (RowTrellisCode, ScalarCode, TrellisCode)):
        raise NotImplementedError(f"{type(code).__name__} is not one of the codes this path implements")
    if isinstance(code, TrellisCode) and any(torch.as_tensor(W).shape[0] % code.T for W in Ws):
        raise ValueError(f"the column trellis needs whole sequences of {code.T} rows in every matrix")
    dev, X, S, rin = _prepare(Ws, seeds, incoherent, in_seed, out_rot)
    rows_label = ("u" if out_rot else "o") if incoherent else "o"
    cols_label = "v" if incoherent else "i"
    m, n = X.shape
    if isinstance(code, TrellisCode):
        # the generic sweep, each block's columns projected by the column-sequence search (codes.py:441-458)
        from .frame import Environment
        from .syntax import sweep

        if H is None:
            codes = code.states(X / S[:, None]).to(torch.int32)
        else:
            Hr = E.rotate_hessian(torch.as_tensor(H).to(dev, torch.float64).contiguous(), rin) if incoherent else \
                torch.as_tensor(H).to(dev, torch.float64).contiguous()
            codes = torch.empty(m, n, dtype=torch.int32, device=dev)
            table = code.values.to(dev, torch.float64)

            def project(j, x, T):
                st = code.states(x / S[:, None])
                codes[:, j : j + x.shape[1]] = st.to(torch.int32)
                return table[st] * S[:, None]

            sweep(X, Environment(Hr), project, width=code.width)
        codes = codes.cpu()
        values = code.values.double()[codes.long()]
        domain = Domain("trellis", float(code.k), levels=code.domain.levels, axis="t", state_bits=code.L)
        nets = _nets(Ws, seeds, X, values, S.cpu(), domain, rows_label, rin, out_rot, incoherent, codes)
        for net in nets:  # rows split into (sequence, position): the sequences' start bits are counted per column
            c = net.cores["W"]
            c.data = c.data.reshape(-1, code.T, c.data.shape[1])
            c.labels = ("s", "t", c.labels[1])
        return nets
    if isinstance(code, RowTrellisCode):
        table = code.values.to(dev, torch.float64).contiguous()
        if H is None:
            x = (X / S[:, None])
            codes = viterbi(x, code.values, code.L, code.k, start=torch.zeros(m, dtype=torch.long)).to(torch.int32)
        else:
            Hr = E.rotate_hessian(torch.as_tensor(H).to(dev, torch.float64).contiguous(), rin) if incoherent else \
                torch.as_tensor(H).to(dev, torch.float64).contiguous()
            if E.fused_trellis(code.L, code.k, code.width, code.look, table):
                _, U, dead, _ = E.chol_inv_upper(Hr)
                codes = E.ldlq_trellis(X, S, U, table, code.L, code.k, code.width, code.look, 128, dead=dead)
            else:
                codes = _row_trellis_sweep(X, S, Hr, code, table)
        codes = codes.cpu()
        values = code.values.double()[codes.long()]
        domain = Domain("trellis", float(code.k), levels=code.domain.levels, axis=cols_label, state_bits=code.L,
                        fixed_start=True)
    else:
        lv = _levels_of(code).to(dev)
        if H is None:
            x = X / S[:, None]
            codes = torch.bucketize(x.contiguous(), (lv[1:] + lv[:-1]) / 2).to(torch.int32)
        else:
            Hr = E.rotate_hessian(torch.as_tensor(H).to(dev, torch.float64).contiguous(), rin) if incoherent else \
                torch.as_tensor(H).to(dev, torch.float64).contiguous()
            _, U, dead, _ = E.chol_inv_upper(Hr)
            codes = E.ldlq_scalar(X, U, lv, mode=1, S=S, dead=dead)
        codes = codes.cpu()
        values = _levels_of(code)[codes.long()]
        domain = code.domain
    return _nets(Ws, seeds, X, values, S.cpu(), domain, rows_label, rin, out_rot, incoherent, codes)


def ldlq_word(W: torch.Tensor, H: torch.Tensor | None, code, seed: int, incoherent: bool = True) -> Net:
    """ldlq_words for a single matrix (codes.py:465-467)."""
    return ldlq_words([W], H, code, [seed], incoherent)[0]
