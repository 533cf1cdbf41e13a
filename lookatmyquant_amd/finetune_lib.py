"""The quantizer that fine-tuning re-runs (finetune_lib.py:19-34, 201-263 of the reference), on the same kernels as
the build: real weights rounded back onto a build's row-trellis form.

    FastRHT(n, seed)           X R and X R^T for R = rht(n, seed), Kronecker-factored on the GPU (fp64 arithmetic,
                               the result in X's dtype; the reference multiplies in float32)
    RowPath(table, k, width, look)   the builds' row trellis with a stored table, as a sweep projection
    rotated_moment(H, R)       R H R^T, symmetrised, float64
    rounded(W, R, groups, scale, env, rows=None)
                               block LDLQ of W R^T under env with each row group through its row trellis in units of
                               `scale`, which is refitted under env.H in place; returns (W_hat, states)

rounded sweeps every RowPath group of one width and look-ahead in one fused pass (the block kernel group by group,
one trailing update over all rows), as the build does; rows do not interact, so this is the reference's group-by-group
sweep. A group whose code is not a RowPath goes through the generic sweep with the code's own step.
"""

from __future__ import annotations

import torch

from . import codes as C
from . import engine as E
from .hadamard import hadamard_factors
from .syntax import sweep

L_TRELLIS = 12  # state bits of every trellis in the builds (finetune_lib.py:79)


class FastRHT:
    """X R and X R^T for R = rht(n, seed) = H diag(s), H = (A kron B) / sqrt(n), in n (a + b) operations per row
    (finetune_lib.py:19-34): the rotation kernels' Kronecker-factored fp64 MFMA products; any leading shape."""

    def __init__(self, n: int, seed: int):
        A, B = hadamard_factors(n)
        self.n, self.seed, self.shape = int(n), int(seed), (len(A), len(B))

    def _rows(self, X: torch.Tensor, inverse: bool) -> torch.Tensor:
        if X.shape[-1] != self.n:
            raise ValueError(f"the last axis must have {self.n} entries")
        dev = E._abi.device()
        Y = E.rht_rows(X.reshape(-1, self.n).to(dev, torch.float64).contiguous(), self.seed, inverse=inverse)
        return Y.to(X.dtype).reshape(X.shape).to(X.device)

    def forward(self, X: torch.Tensor) -> torch.Tensor:
        """X R: from the rotated basis back to the weights' own."""
        return self._rows(X, True)

    def back(self, X: torch.Tensor) -> torch.Tensor:
        """X R^T: a matrix's rows into the rotated basis."""
        return self._rows(X, False)


class RowPath:
    """The builds' row trellis (RowTrellisCode with --trellis-rows 16,8: each row one path from state 0, `width`
    columns settled at a time with `look` ahead) over a stored table (finetune_lib.py:201-216). `paths` holds the
    states of the last generic sweep's blocks."""

    def __init__(self, table, k: int, width: int = 16, look: int = 8):
        self.values = torch.as_tensor(table).double().cpu()
        self.k, self.width, self.look = int(k), int(width), int(look)
        self.paths: list = []

    def step(self, j, X, ahead):
        if j == 0:
            self.state = torch.zeros(len(X), dtype=torch.long, device=X.device)
            self.paths = []
        path = C.viterbi(torch.cat([X, ahead], 1), self.values, L_TRELLIS, self.k, start=self.state)[:, : X.shape[1]]
        self.state = path[:, -1]
        self.paths.append(path)
        return self.values.to(X.device, X.dtype)[path]


row_code = RowPath


def rotated_moment(H: torch.Tensor, R: FastRHT) -> torch.Tensor:
    """R H R^T symmetrised, float64 (finetune_lib.py:222-227): the statistics in the basis R.back takes rows to."""
    Hr = R.back(R.back(torch.as_tensor(H).float()).T).double()
    return (Hr + Hr.T) / 2


def _refit_scale(x: torch.Tensor, got: torch.Tensor, H: torch.Tensor) -> torch.Tensor:
    """The least-squares row scale s = <x, got H> / <got, got H> (minimising (x - s got) H (x - s got)^T), clamped as
    the reference does, float32."""
    gH = got @ H
    return ((x * gH).sum(1) / (got * gH).sum(1).clamp_min(1e-30)).clamp_min(1e-12).float()


@torch.no_grad()
def rounded(W: torch.Tensor, R: FastRHT, groups, scale: torch.Tensor, env, rows=None):
    """(R.forward(scale * Q), states int16 [rows, n] on the CPU) of W rounded as a build rounds it
    (finetune_lib.py:230-263): X = W R^T (the selected `rows` of W only, in that order), each row group
    (g_rows, bits, code) swept by block LDLQ under env (env.H, env.U, env.dead of frame.Environment) through its
    trellis in units of scale[g_rows]; then scale[g_rows] is refitted under env.H in place."""
    dev = E._abi.device()
    Wd = torch.as_tensor(W)
    Wsel = Wd if rows is None else Wd[torch.as_tensor(rows, device=Wd.device)]
    X = R.back(Wsel).double().to(dev)
    where = None
    if rows is not None:
        rows_t = torch.as_tensor(rows, dtype=torch.long)
        where = torch.full((Wd.shape[0],), -1, dtype=torch.long)
        where[rows_t] = torch.arange(len(rows_t))
    scale_dev = scale.to(dev, torch.float64)
    Q = torch.empty_like(X)
    states = torch.empty(X.shape, dtype=torch.int16)
    H = env.H.to(dev, torch.float64)
    fused: dict = {}  # (width, look) -> [(mine, at, code)]
    for g_rows, k, code in groups:
        g_rows = torch.as_tensor(g_rows, dtype=torch.long).cpu()
        mine = g_rows if where is None else g_rows[where[g_rows] >= 0]
        if not len(mine):
            continue
        at = mine if where is None else where[mine]
        if isinstance(code, RowPath) and code.k == int(k):
            fused.setdefault((code.width, code.look), []).append((mine, at, code))
            continue
        x, S = X[at.to(dev)], scale_dev[mine.to(dev)]
        got = torch.empty_like(x)

        def project(j, cols, T, code=code, S=S, got=got):
            q = code.step(j, cols / S[:, None], T[:, j + cols.shape[1] : j + cols.shape[1] + code.look] / S[:, None])
            got[:, j : j + cols.shape[1]] = q
            return q * S[:, None]

        sweep(x, env, project, width=code.width)
        scale[mine] = _refit_scale(x, got, H).to(scale.device)
        Q[at.to(dev)] = got
        states[at] = torch.cat(code.paths, 1).to(torch.int16).cpu()
        code.paths = []
    for (width, look), parts in fused.items():
        at_all = torch.cat([at for _, at, _ in parts]).to(dev)
        x = X.index_select(0, at_all)
        S = torch.cat([scale_dev[mine.to(dev)] for mine, _, _ in parts])
        sweep_groups = [(len(mine), code.k, code.values.to(dev), None) for mine, _, code in parts]
        st = E.ldlq_trellis_groups(x, S, env.U, sweep_groups, L_TRELLIS, width, look, 128, dead=env.dead)
        r0 = 0
        for mine, at, code in parts:
            r1 = r0 + len(mine)
            got = code.values.to(dev)[st[r0:r1].long()]
            scale[mine] = _refit_scale(x[r0:r1], got, H).to(scale.device)
            Q[at.to(dev)] = got
            states[at] = st[r0:r1].to(torch.int16).cpu()
            code.paths = []
            r0 = r1
    units = scale if rows is None else scale[torch.as_tensor(rows, dtype=torch.long, device=scale.device)]
    W_hat = R.forward(units.to(dev)[:, None] * Q.float())
    return W_hat.to(Wd.device), states
