"""The measure step's kernels (compiler.py:110-190 of the reference): the KL sensitivity on the gfx950 streaming
kernel, and the LDLQ-shaped noise its noise method adds instead of quantizing.

    kl(ref_logits, q_logits, wpos=None) -> float      the weighted mean of per-position KL(p_ref || p_q)
    kl_per_token(ref_logits, q_logits) -> tensor       per-position KL, as quantize.evaluate / text_kl use it
    ldlq_noise(W, H, d, seed, gen, row_rotation=True)  W plus LDLQ-shaped rounding noise of level d

For each position, KL = sum_v softmax(ref)_v (log_softmax(ref)_v - log_softmax(q)_v) in float32 from bf16 or
float32 logits (the reference casts the model's logits with .float(); other float dtypes are cast to float32 the
same way), in one pass over both logit matrices; positions are
weighted by wpos (the digit weight of compiler.py:170-173) and the result is sum w KL / sum w.
"""

from __future__ import annotations

import torch

from . import engine as E


def _as_rows(x: torch.Tensor) -> torch.Tensor:
    """Logit rows on the device: bf16 as they are (the kernel widens them exactly); any other floating dtype as
    float32, as the reference's .logits.float() (compiler.py:180,185) takes them."""
    dev = E._abi.device()
    x = torch.as_tensor(x)
    if not x.is_floating_point():
        raise ValueError("logits must be a floating-point tensor")
    if x.dtype != torch.bfloat16:
        x = x.to(dev, torch.float32)
    return x.reshape(-1, x.shape[-1]).to(dev).contiguous()


def _pair(ref_logits, q_logits):
    """Both logit matrices as rows of one dtype: bf16 if both are, else float32 (bf16 widens exactly)."""
    r, q = _as_rows(ref_logits), _as_rows(q_logits)
    if r.dtype != q.dtype:
        r, q = r.float(), q.float()
    return r, q


def kl_per_token(ref_logits: torch.Tensor, q_logits: torch.Tensor) -> torch.Tensor:
    """KL(p_ref || p_q) for every position, float32, shaped like the logits without their last axis."""
    shape = ref_logits.shape[:-1]
    kl, _ = E.kl_rows(*_pair(ref_logits, q_logits))
    return kl.reshape(shape)


def kl(ref_logits: torch.Tensor, q_logits: torch.Tensor, wpos: torch.Tensor | None = None) -> float:
    """sum_pos w_pos KL_pos / sum_pos w_pos (compiler.py:180-188); w = 1 without wpos."""
    r, q = _pair(ref_logits, q_logits)
    w = None if wpos is None else torch.as_tensor(wpos).reshape(-1).to(r.device, torch.float32)
    _, sums = E.kl_rows(r, q, w)
    s = sums.cpu()
    return float(s[0] / s[1])


NOISE_D = 0.015  # the noise level the measure step uses (compiler.py:132)


@torch.no_grad()
def ldlq_noise(W: torch.Tensor, H: torch.Tensor, d: float, seed: int, gen: torch.Generator, row_rotation: bool = True):
    """W plus an error shaped as LDLQ's (compiler.py:110-129): in the incoherent basis (input rotation rht(n, seed + 1),
    output rotation rht(m, seed)), noise eta ~ N(0, d (row RMS)^2) carried through the damped rotated statistics
    H = A A^T (A upper triangular) as E = eta diag(A) A^-1, so that E H E^T has trace sum_j A_jj^2 eta_j^2 per row;
    then back to the original basis. A^-1 is the upper factor U of H^-1 that the Cholesky-inverse kernel makes (and
    diag A = 1 / diag U), so E = (eta / diag U) U is one triangular fp64 product on MFMA; the rotations run on the
    Kronecker kernels. eta is drawn from `gen` on its own device (a CPU generator gives the reference's draw); the
    result is W + E on W's device in W's dtype promoted with float64."""
    dev = E._abi.device()
    Wt = torch.as_tensor(W)
    W64 = Wt.to(dev, torch.float64).contiguous()
    m, n = W64.shape
    Wr = E.rht_rows(W64, seed + 1)
    if row_rotation:
        Wr = E.rotate_columns(Wr, seed)
    Hr = E.rotate_hessian(torch.as_tensor(H).to(dev, torch.float64).contiguous(), seed + 1)
    _, U, _, _ = E.chol_inv_upper(Hr, damp=0.01)
    S = Wr.pow(2).mean(1, keepdim=True).sqrt()
    eta = torch.randn(m, n, generator=gen, dtype=torch.float64, device=gen.device).to(dev) * S * d ** 0.5
    Er = torch.zeros(m, n, dtype=torch.float64, device=dev)
    E.gemm_sub(Er, (eta / torch.diagonal(U)[None, :]).contiguous(), U, tri=2)  # Er = -(eta diag A) A^-1
    Er.neg_()
    if row_rotation:
        Er = E.unrotate_columns(Er, seed)
    Eo = E.rht_rows(Er, seed + 1, inverse=True)
    return Wt + Eo.to(Wt.device)
