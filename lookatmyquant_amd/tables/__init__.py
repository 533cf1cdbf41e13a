"""Trellis state tables.

The four L = 12 tables are the reference's fitted tables (opgraph/codes.py:187-220 with fit "ema", T = 256,
seed 0; cache/codes/trellis_L12_k{1..4}_T256_s0_ema.pt), stored here as raw little-endian float64 x 4096: they
are part of the code format (a saved matrix stores its states, and its values are these tables). The 16-bit
table of the benchmark configurations is the unrefined initial table of the same construction, 2^16 unit-
Gaussian quantiles in the order of torch.randperm(2^16, Generator(seed)), cast to float16."""

from __future__ import annotations

from functools import lru_cache
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


@lru_cache(maxsize=None)
def load_table(L: int, k: int, T: int = 256, seed: int = 0, fit: str = "ema") -> np.ndarray:
    """The cached fitted table for (L, k, T, seed, fit), float64 [2^L]; raises FileNotFoundError for tables the
    reference has not fitted (fitting new tables is not part of this package)."""
    path = HERE / f"trellis_L{L}_k{k}_T{T}_s{seed}{'' if fit == 'lloyd' else '_' + fit}.f64"
    if not path.exists():
        raise FileNotFoundError(f"no fitted trellis table for L={L} k={k} T={T} seed={seed} fit={fit}")
    v = np.fromfile(path, dtype="<f8")
    if v.size != 1 << L:
        raise ValueError(f"{path.name}: expected {1 << L} values")
    v.setflags(write=False)
    return v


@lru_cache(maxsize=None)
def quantile_table(L: int, seed: int = 0, dtype: str = "float16") -> np.ndarray:
    """2^L unit-Gaussian quantiles ndtri((randperm(2^L, Generator(seed)) + 0.5) / 2^L), cast to `dtype`, returned as
    float64 (opgraph/codes.py:202-204 without refinement)."""
    S = 1 << L
    g = torch.Generator().manual_seed(int(seed))
    v = torch.special.ndtri((torch.randperm(S, generator=g).double() + 0.5) / S)
    v = v.to(getattr(torch, dtype)).double().numpy()
    v.setflags(write=False)
    return v
