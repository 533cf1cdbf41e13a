"""Words as the reference's callers see them (opgraph/frame.py): a Net of cores with a domain each, its value as
a matrix and its storage price, and the Environment of a linear core's input bond (damped H and the upper
Cholesky factor U of its inverse). Only the parts of the grammar the quantization path produces are here: a
word is W (the quantized core, in units of its row scale), W.S (the row scales), I[v] (the shared input
rotation, priced as its random signs) and, with out_rot, I[u] (the output rotation)."""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from . import engine as E


@dataclass(frozen=True)
class Domain:
    """What a core's entries may be and what each costs to store (opgraph/frame.py:33-45)."""
    kind: str
    bits: float
    lo: float | None = None
    hi: float | None = None
    levels: tuple | None = None
    axis: str | None = None
    state_bits: int | None = None
    fixed_start: bool = False


REAL = Domain("real", 16.0)
RHT = Domain("rht", 0.0)


@dataclass
class Core:
    data: torch.Tensor
    labels: tuple
    domain: Domain = REAL
    free: bool = False

    def axis(self, label: str) -> int:
        return self.labels.index(label)


def core_bits(c: Core) -> float:
    """Storage of one core (opgraph/frame.py:136-151, the kinds a word has): a transform by its n signs, a trellis
    core by k bits per entry plus L - k bits per sequence unless every sequence starts from state 0, anything else
    by its entries times the domain's bits."""
    if c.free:
        return 0.0
    if c.domain.kind == "rht":
        return float(c.data.shape[0] if c.data.dim() == 1 else math.isqrt(c.data.numel()))
    if c.domain.kind == "trellis":
        ax = c.axis(c.domain.axis) if c.domain.axis in c.labels else c.data.dim() - 1
        seqs = c.data.numel() / c.data.shape[ax]
        extra = 0 if c.domain.fixed_start else seqs * (c.domain.state_bits - c.domain.bits)
        return c.data.numel() * c.domain.bits + extra
    return c.data.numel() * c.domain.bits


class Rotation:
    """The randomized Hadamard transform R = hadamard(n) diag(s) of a seed, stored as its signs (a core of domain
    RHT: what the runtime applies and what the price counts)."""

    def __init__(self, n: int, seed: int):
        self.n, self.seed = n, int(seed)

    def dense(self) -> torch.Tensor:
        from .hadamard import rht
        return rht(self.n, self.seed)


@dataclass
class Net:
    """A quantized matrix: W_hat = R_out^T diag(S) W R_in (R_out absent unless out_rot). `cores` holds W, W.S and
    the rotations' sign cores I[v] (and I[u]); `codes` the stored integers (trellis states or level indices)."""
    cores: dict
    rows: str
    rot_in: Rotation | None
    rot_out: Rotation | None = None
    codes: torch.Tensor | None = None
    _matrix: torch.Tensor | None = field(default=None, repr=False)

    def matrix(self, device=None, dtype=None) -> torch.Tensor:
        """The value as a dense matrix (computed once on the GPU: scale, then the inverse rotations)."""
        if self._matrix is None:
            dev = E._abi.device()
            Q = self.cores["W"].data.to(dev, torch.float64)
            Q = Q.reshape(-1, Q.shape[-1])  # a column trellis keeps its rows split into (sequence, position)
            S = self.cores["W.S"].data.to(dev, torch.float64)
            X = Q * S[:, None]
            if self.rot_in is not None:
                X = E.rht_rows(X.contiguous(), self.rot_in.seed, inverse=True)
            if self.rot_out is not None:
                X = E.unrotate_columns(X, self.rot_out.seed)
            self._matrix = X.cpu()
        m = self._matrix
        if device is None and dtype is None:
            return m
        return m.to(device=device or m.device, dtype=dtype or m.dtype)

    def rate_bits(self) -> float:
        return sum(core_bits(c) for c in self.cores.values())

    def dim(self, label: str) -> int:
        for c in self.cores.values():
            if label in c.labels:
                return c.data.shape[c.axis(label)]
        raise KeyError(label)


class Dense:
    """A matrix kept as its dense reconstruction with the bits its format stores (quantize.py:291-302)."""

    def __init__(self, W, bits):
        self.W, self.bits = W, bits

    def matrix(self, dtype=torch.float64, device=None):
        return self.W.to(dtype=dtype, device=device or self.W.device)

    def rate_bits(self):
        return self.bits


# ----------------------------------------------------------------------------- environments


def covariance(x: torch.Tensor, w: torch.Tensor | None = None) -> torch.Tensor:
    """Sum over tokens of w_t x_t x_t^T in float64 (opgraph/frame.py:498-505; quantize.py:1465 with token weights),
    on the bf16 MFMA Gram kernel with float32 accumulation. x: [..., n] bfloat16 activations (as a bf16 model
    produces them); other dtypes are rejected rather than rounded."""
    x = x.reshape(-1, x.shape[-1])
    if x.dtype != torch.bfloat16:
        raise NotImplementedError("covariance takes bfloat16 activations (the Gram kernel multiplies bf16 exactly)")
    dev = E._abi.device()
    x = x.to(dev).contiguous()
    n = x.shape[1]
    H = torch.zeros(n, n, dtype=torch.float32, device=dev)
    E.hessian_accum(H, x, w)
    return E.hessian_finalize(H, 1.0)


class Environment:
    """What the rest of the network sees through a linear core's input bond (opgraph/frame.py:508-522):
    dead columns (zero diagonal) get a unit diagonal, H += damp * mean(diag H) * I, and U is the upper Cholesky
    factor of H^-1. Computed on the GPU; .H, .U, .dead live there. G, the output-side sensitivity (a square matrix
    over the output rows, frame.py:516), is kept in float64 beside them and weights error()."""

    def __init__(self, H: torch.Tensor, damp: float = 0.01, G: torch.Tensor | None = None):
        dev = E._abi.device()
        if G is not None and (G.dim() != 2 or G.shape[0] != G.shape[1]):
            raise ValueError("G must be a square matrix over the output rows")
        self.G = None if G is None else G.to(dev, torch.float64).contiguous()
        Hd, U, dead, _ = E.chol_inv_upper(H.to(dev, torch.float64).contiguous(), damp)
        self.H, self.U, self.dead = Hd, U, dead

    def error(self, D: torch.Tensor) -> float:
        """tr(D H D^T), or tr(G D H D^T) with G, the local objective (opgraph/frame.py:534-537)."""
        D = D.to(self.H.device, torch.float64)
        DH = D @ self.H
        if self.G is None:
            return float((DH * D).sum())
        if self.G.shape[0] != D.shape[0]:
            raise ValueError("G and D must have the same number of rows")
        return float(((self.G @ DH) * D).sum())
