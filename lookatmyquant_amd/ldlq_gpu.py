"""LDLQ with a fixed set of levels, the reference's GPU variant (opgraph/ldlq_gpu.py), on the gfx950 kernels.

    U = ldlq_factor(Hr)                 # once per input statistics (H in the rotated basis)        ldlq_gpu.py:15
    Q = ldlq_round(X, U, levels)        # X: rows in units of their RMS; returns the chosen levels   ldlq_gpu.py:28

Both run in float64 on the GPU, as the reference's do; the factor and the sweep are the same kernels as Environment
and the scalar ldlq_words (the damping here keeps zero diagonal entries as they are, like the reference's).
"""

from __future__ import annotations

import torch

from . import engine as E


def ldlq_factor(Hr: torch.Tensor, damp: float = 0.01) -> torch.Tensor:
    """The upper Cholesky factor of (H + d mean(diag H) I)^-1 for H = (Hr + Hr^T)/2, with d = damp, then 10 and 100
    times damp while the damped H does not factor (ldlq_gpu.py:15-25). Raises AssertionError when none does.
    Returns U float64 on the GPU."""
    dev = E._abi.device()
    H = torch.as_tensor(Hr).to(dev, torch.float64)
    H = (0.5 * (H + H.T)).contiguous()
    for d in (damp, 10 * damp, 100 * damp):
        _, U, _, info = E.chol_inv_upper(H, damp=d, raise_on_fail=False, keep_dead=True)
        if int(info.item()) == 0:
            return U
    raise AssertionError("H is not positive definite even with damping")


@torch.no_grad()
def ldlq_round(X: torch.Tensor, U: torch.Tensor, levels: torch.Tensor, block: int = 128) -> torch.Tensor:
    """Each entry of X (rows x inputs, in units of each row's RMS) to a level, inputs in order, each rounding error
    carried into the later inputs through U: the bucketize rule (an exact midpoint goes to the lower level), lazy
    blocks of `block` columns (ldlq_gpu.py:28-49). Returns the chosen levels (float64, X's shape, on the GPU)."""
    dev = E._abi.device()
    Xg = torch.as_tensor(X).to(dev, torch.float64).contiguous()
    Ug = torch.as_tensor(U).to(dev, torch.float64).contiguous()
    lv = torch.as_tensor(levels).to(dev, torch.float64).contiguous()
    ones = torch.ones(Xg.shape[0], dtype=torch.float64, device=dev)
    idx = E.ldlq_scalar(Xg, Ug, lv, mode=1, S=ones, lazy=block)
    return lv[idx.long()]
