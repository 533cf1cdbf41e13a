"""The block-LDLQ sweep with a caller's projection (opgraph/syntax.py:86-124), on the GPU.

    sweep(W, env, project, block=None, on_block=None, width=1, lazy=128) -> before

The running core T lives on the GPU in float64. For each lazy run [b0, b1) and each step j of `width` columns,
project(j, T[:, j] or T[:, j:j+width], T) returns the settled columns (any torch ops the caller likes); the refit
of the rest of the run (E = T_cols - q, z = E U_BB^-1, T[:, j+w:b1] -= z U[cols, j+w:b1]) is lamq_refit_step and
the lazy update of the columns after the run is the fp64 MFMA trailing update. Returns each column as it stood
just before it was settled. The word builders (codes.ldlq_words, nested.nested_words) do not call back into Python
per step: they use the fused block kernels, with the same arithmetic.
"""

from __future__ import annotations

from typing import Callable

import torch

from . import engine as E


def sweep(W: torch.Tensor, env, project: Callable, block: int | None = None, on_block: Callable | None = None,
          width: int = 1, lazy: int = 128) -> torch.Tensor:
    dev = E._abi.device()
    T = torch.as_tensor(W).to(dev, torch.float64).clone().contiguous()
    m, n = T.shape
    if env is not None:
        if lazy % width or (block and lazy % block):
            raise ValueError("lazy must be a multiple of width and of block")
        E.zero_columns(T, env.dead)
        U = env.U
    before = torch.empty_like(T)
    Z = torch.empty(m, lazy, dtype=torch.float64, device=dev) if env is not None else None
    for b0 in range(0, n, lazy):
        b1 = min(b0 + lazy, n)
        for j in range(b0, b1, width):
            if on_block is not None and block and j % block == 0:
                on_block(j, T)
            w = min(width, b1 - j)
            before[:, j : j + w] = T[:, j : j + w]
            q = project(j, T[:, j], T) if width == 1 else project(j, T[:, j : j + w], T)
            if env is None:
                continue
            Q = q.to(dev, torch.float64).reshape(m, w).contiguous()
            E.refit_step(T, U, Q, j, b0, b1, Z)
        if env is not None and b1 < n:
            E.trailing_update(T, Z, U, b0, b1)
    return before
