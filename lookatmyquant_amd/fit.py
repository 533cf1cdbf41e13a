"""Fitting trellis tables (opgraph/codes.py:187-220): the table starts as 2^L unit-Gaussian quantiles in the order of
torch.randperm(2^L, Generator(seed)), and each state's value then moves to the mean of the Gaussian samples that the
Viterbi search assigns to it.

    fit="ema":   16 * refine batches (refine 384 by default) of 256 fresh N(0, 1) sequences of T samples; after each
                 batch every state keeps a decaying sum and count, the batch's weight a = 0.01 + 0.245 (1 + cos(pi j /
                 (steps - 1))) falling from 0.5 to 0.01 (e-means' update), and takes sum / count where its count is
                 positive.
    fit="lloyd": refine (6) Lloyd steps over one set of 4096 sequences (a = 1).

The samples come from torch's CPU generator in the reference's order (the quantile permutation, then one
torch.randn(256, T, float64) per batch), the search is this package's Viterbi kernel (the reference's search bit for
bit: float32 samples and values, lowest index on ties), and the per-state sums run on the host in sample order, as
torch's index_add_ and bincount add them (numpy's bincount gives the same doubles). Refitting the reference's cached
12-bit table for k = 2 gives 4091 of its 4096 entries exactly and the other 5 within 4 units in the last place: one
sample searched onto another state in any of the last ~1,200 of the 6,144 batches would leave a larger difference,
so every late search agreed, and the residue is the tie-break of an earlier exact float32 tie in the reference's own
run (torch's min on the GPU does not promise the lowest index). The fitted tables are float64 and not exactly
representable in fp16, so fitting covers the 12-bit-and-below trellises that the float32 search kernels take
(L <= 12).
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import _abi
from . import engine as E


def fit_table(L: int, k: int, T: int = 256, seed: int = 0, refine: int | None = None, fit: str = "ema",
              batch: int = 256) -> np.ndarray:
    """The fitted table of (L, k, T, seed, refine, fit), float64 [2^L] (codes.py:187-220)."""
    if fit not in ("ema", "lloyd"):
        raise ValueError(f"unknown trellis fit {fit!r}")
    if not 1 <= k < L <= 12:
        raise NotImplementedError("tables are fitted for trellises of at most 12 state bits (the float32 search)")
    dev = _abi.device()
    S = 1 << L
    g = torch.Generator().manual_seed(int(seed))
    v = torch.special.ndtri((torch.randperm(S, generator=g).double() + 0.5) / S).numpy().copy()
    if fit == "lloyd":
        X = torch.randn(4096, T, generator=g, dtype=torch.float64)
        batches = ((X, 1.0) for _ in range(6 if refine is None else refine))
    else:
        steps = 16 * (384 if refine is None else refine)
        batches = ((torch.randn(batch, T, generator=g, dtype=torch.float64),
                    0.01 + 0.245 * (1 + math.cos(math.pi * j / max(steps - 1, 1)))) for j in range(steps))
    sums = np.zeros(S)
    cnt = np.zeros(S)
    for X, a in batches:
        x = X.to(dev, torch.float32)
        C = torch.from_numpy(v).to(dev, torch.float32)
        st = E.viterbi_rows(x, C, L, k).reshape(-1).cpu().numpy()
        xs = X.reshape(-1).numpy()
        # a fresh zero vector and the samples added in order (index_add_), the counts as doubles (bincount)
        bs = np.bincount(st, weights=xs, minlength=S)
        bc = np.bincount(st, minlength=S).astype(np.float64)
        sums = (1 - a) * sums + a * bs
        cnt = (1 - a) * cnt + a * bc
        v = np.where(cnt > 0, sums / np.maximum(cnt, 1e-300), v)
    return v
