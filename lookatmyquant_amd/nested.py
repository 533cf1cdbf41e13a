"""Lloyd-Max and compander level sets, and the LDLQ onto them for one or several rates (opgraph/nested.py), on the
gfx950 kernels.

    gaussian_centroids, gaussian_mse, compander_bounds, compander_levels      nested.py:44-68
    lloyd_max(bits, iters=500), lloyd_max_levels(n, iters=500)                nested.py:71-82
    nested_tables(top, rates, alpha)                                          nested.py:150-152
    multirate_sweep(X, H, tables, weights, G=None, block=32)                  nested.py:104-147
    nested_words(Ws, H, seeds, top, rates, alpha, weights, levels=None, in_seed=None, out_rot=True, G=None)
                                                                              nested.py:155

The level tables are small host computations in float64 with torch's special functions, as the reference does
them (so the levels are the same bits). The sweep is the width-1 LDLQ kernel: each column's index is the first
minimum of (t - level)^2 over the levels (one rate at weight 1), or of sum_r w_r (t_r - tables[r, i])^2 over the
rates' copies of the row (several rates: lamq_ldlq_multirate_block), then the later columns are re-solved under U.
With output-side shaping (G: one matrix at one rate) each column's rows are settled a block at a time and the later
rows re-solved under G's damped factor (lamq_ldlq_shaped_column), inside the generic width-1 sweep under H."""

from __future__ import annotations

import math

import torch

from . import engine as E
from .codes import SET, _nets, _prepare
from .frame import Domain

OUTPUT_DAMP = 0.03


def _phi(x):
    return torch.exp(-0.5 * x * x) / math.sqrt(2 * math.pi)


def _Phi(x):
    return 0.5 * (1 + torch.erf(x / math.sqrt(2)))


def gaussian_centroids(bounds: torch.Tensor) -> torch.Tensor:
    """The mean of a unit Gaussian on each cell [bounds[j], bounds[j+1]]."""
    a, b = bounds[:-1], bounds[1:]
    pa = torch.where(torch.isinf(a), torch.zeros_like(a), _phi(a))
    pb = torch.where(torch.isinf(b), torch.zeros_like(b), _phi(b))
    return (pa - pb) / (_Phi(b) - _Phi(a))


def gaussian_mse(bounds: torch.Tensor, levels: torch.Tensor) -> float:
    """E[(x - q(x))^2] for x ~ N(0, 1) by the truncated-moment formulas."""
    a, b = bounds[:-1], bounds[1:]
    P = _Phi(b) - _Phi(a)
    fa = lambda t: torch.where(torch.isinf(t), torch.zeros_like(t), t * _phi(t))
    pa = lambda t: torch.where(torch.isinf(t), torch.zeros_like(t), _phi(t))
    m1 = pa(a) - pa(b)
    m2 = P + fa(a) - fa(b)
    return float((m2 - 2 * levels * m1 + levels**2 * P).sum())


def compander_bounds(bits: int, alpha: float) -> torch.Tensor:
    u = torch.arange(2**bits + 1, dtype=torch.float64) / 2**bits
    return torch.special.ndtri(u) / math.sqrt(alpha)


def compander_levels(bits: int, alpha: float) -> torch.Tensor:
    return gaussian_centroids(compander_bounds(bits, alpha))


def lloyd_max_levels(n: int, iters: int = 500) -> torch.Tensor:
    """The best n levels for a unit Gaussian: Lloyd iterations from the centroids of equal-probability cells
    widened by sqrt(3)."""
    lv = gaussian_centroids(torch.special.ndtri(torch.arange(n + 1, dtype=torch.float64) / n) * math.sqrt(3))
    inf = torch.tensor([math.inf], dtype=torch.float64)
    for _ in range(iters):
        mid = (lv[1:] + lv[:-1]) / 2
        lv = gaussian_centroids(torch.cat([-inf, mid, inf]))
    return lv


def lloyd_max(bits: int, iters: int = 500) -> torch.Tensor:
    return lloyd_max_levels(2**bits, iters)


def NESTED(bits: int, alpha: float) -> Domain:
    return SET(compander_levels(bits, alpha).tolist())


def nested_tables(top: int, rates: list[int], alpha: float) -> torch.Tensor:
    i = torch.arange(2**top)
    return torch.stack([compander_levels(b, alpha)[i >> (top - b)] for b in rates])


def multirate_sweep(X: torch.Tensor, H: torch.Tensor | None, tables: torch.Tensor, weights: torch.Tensor,
                    G: torch.Tensor | None = None, block: int = 32) -> torch.Tensor:
    """One index per entry of X (already in units of the row scale) for R rates at once (nested.py:104-147): the first
    minimum of sum_r w_r (t_r - tables[r, i])^2, each rate's copy of the row keeping its own running target; with H,
    the width-1 LDLQ sweep under U; without H, every column alone. With G (one rate), the output sensitivity in units
    of the row scale, each column's rows are settled `block` at a time and the later rows re-solved under G's damped
    factor (_shaped_sweep). Returns int64 indices on the CPU."""
    dev = E._abi.device()
    tables = torch.as_tensor(tables, dtype=torch.float64)
    if tables.dim() != 2:
        raise ValueError("tables must be [rates, levels]")
    if G is not None:
        if tables.shape[0] != 1:
            raise ValueError("output shaping takes one rate")
        Hg = None if H is None else torch.as_tensor(H).to(dev, torch.float64).contiguous()
        return _shaped_sweep(torch.as_tensor(X).to(dev, torch.float64), Hg, tables[0].to(dev),
                             torch.as_tensor(G).to(dev, torch.float64).contiguous(), block).to(torch.int64).cpu()
    x = torch.as_tensor(X).to(dev, torch.float64).contiguous()
    U = dead = None
    if H is not None:
        _, U, dead, _ = E.chol_inv_upper(torch.as_tensor(H).to(dev, torch.float64).contiguous())
    return _sweep(x, U, dead, tables.to(dev), torch.as_tensor(weights, dtype=torch.float64).to(dev)).to(torch.int64).cpu()


def _shaped_sweep(x: torch.Tensor, H: torch.Tensor | None, levels: torch.Tensor, G: torch.Tensor,
                  block: int) -> torch.Tensor:
    """The index array [m, n] int32 on the device of multirate_sweep with G (nested.py:121-144): V the upper factor of
    G damped by OUTPUT_DAMP (frame.Environment), its row blocks' feedback packed once (lamq_shaping_feedback); each
    column settled by lamq_ldlq_shaped_column, inside the width-1 generic sweep under H (syntax.sweep: the refit and
    the lazy trailing update) or, without H, every column alone."""
    from .frame import Environment
    from .syntax import sweep

    m, n = x.shape
    V = Environment(G, damp=OUTPUT_DAMP).U
    M = E.shaping_feedback(V, block)
    idx = torch.empty(m, n, dtype=torch.int32, device=x.device)
    Q = torch.empty(m, 1, dtype=torch.float64, device=x.device)

    def project(j, col, T):
        E.shaped_column(T, j, M, block, levels, idx, Q)
        return Q[:, 0]

    if H is None:
        X = x.contiguous()
        for j in range(n):
            project(j, None, X)
    else:
        sweep(x, Environment(H), project)
    return idx


def _sweep(x, U, dead, tables, weights):
    """The index array [m, n] int32 on the device: one rate at weight 1 through the width-1 kernel (the joint cost is
    then the squared distance), several rates (or another weight) through the multi-rate kernel."""
    if tables.shape[0] == 1 and float(weights[0]) == 1.0:
        lv = tables[0].contiguous()
        if U is None:
            # first minimum of (t - lv)^2 per entry: every column alone
            return ((x[:, :, None] - lv[None, None, :]) ** 2).argmin(-1).to(torch.int32)
        return E.ldlq_scalar(x, U, lv, mode=0, dead=dead)
    return E.ldlq_multirate(x, U, tables.contiguous(), weights.contiguous(), dead=dead)


def nested_words(Ws: list, H: torch.Tensor | None, seeds: list[int], top: int, rates: list[int], alpha: float,
                 weights: list[float], levels: torch.Tensor | None = None, in_seed: int | None = None,
                 out_rot: bool = True, G: torch.Tensor | None = None, block: int = 32) -> dict:
    """Incoherence (shared input transform) -> per-row RMS scale -> LDLQ onto a `top`-bit nested code for every rate in
    `rates` at once (weights price the rates' squared errors) -> {rate: [Net per matrix]}, each rate reading the shared
    indices with its own levels (nested.py:155-192). With `levels` (one rate only) the code is that set (a dedicated
    code, as quantize.word's lm<b>)."""
    if levels is not None and len(rates) != 1:
        raise ValueError("a dedicated code has one rate")
    if G is not None and (len(Ws) > 1 or len(rates) > 1 or out_rot):
        raise ValueError("output shaping is for one matrix at one rate, with its rows not rotated")
    dev, X, S, rin = _prepare(Ws, seeds, True, in_seed, out_rot)
    if levels is None:
        tables = nested_tables(top, rates, alpha)
    else:
        tables = torch.as_tensor(levels, dtype=torch.float64)[None]
    x = (X / S[:, None]).contiguous()
    Hr = None
    if H is not None:
        Hr = E.rotate_hessian(torch.as_tensor(H).to(dev, torch.float64).contiguous(), rin)
    if G is not None:
        # the output sensitivity in units of the row scale (nested.py:180): Gs = diag(S) G diag(S)
        Gs = (S[:, None] * torch.as_tensor(G).to(dev, torch.float64) * S[None, :]).contiguous()
        idx = _shaped_sweep(x, Hr, tables[0].to(dev), Gs, block).cpu()
    else:
        U = dead = None
        if Hr is not None:
            _, U, dead, _ = E.chol_inv_upper(Hr)
        idx = _sweep(x, U, dead, tables.to(dev), torch.as_tensor(weights, dtype=torch.float64).to(dev)).cpu()
    rows_label = "u" if out_rot else "o"
    out = {}
    for r, b in enumerate(rates):
        if levels is not None:
            dom = SET(tables[r].tolist(), bits=math.log2(tables.shape[1]))
        else:
            dom = NESTED(b, alpha)
        out[b] = _nets(Ws, seeds, X, tables[r][idx.long()], S.cpu(), dom, rows_label, rin, out_rot, True, idx)
    return out
