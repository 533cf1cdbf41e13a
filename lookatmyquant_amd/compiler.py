"""The KL sensitivity of the measure step (compiler.py:170-190 of the reference) on the gfx950 streaming kernel.

    kl(ref_logits, q_logits, wpos=None) -> float      the weighted mean of per-position KL(p_ref || p_q)
    kl_per_token(ref_logits, q_logits) -> tensor       per-position KL, as quantize.evaluate / text_kl use it

For each position, KL = sum_v softmax(ref)_v (log_softmax(ref)_v - log_softmax(q)_v) in float32 from bf16 logits
(the reference casts the model's logits with .float()), in one pass over both logit matrices; positions are
weighted by wpos (the digit weight of compiler.py:170-173) and the result is sum w KL / sum w.
"""

from __future__ import annotations

import torch

from . import engine as E


def _as_bf16_rows(x: torch.Tensor) -> torch.Tensor:
    dev = E._abi.device()
    x = torch.as_tensor(x)
    if x.dtype != torch.bfloat16:
        raise NotImplementedError("the KL kernel reads bfloat16 logits (the model's output dtype)")
    return x.reshape(-1, x.shape[-1]).to(dev).contiguous()


def kl_per_token(ref_logits: torch.Tensor, q_logits: torch.Tensor) -> torch.Tensor:
    """KL(p_ref || p_q) for every position, float32, shaped like the logits without their last axis."""
    shape = ref_logits.shape[:-1]
    kl, _ = E.kl_rows(_as_bf16_rows(ref_logits), _as_bf16_rows(q_logits))
    return kl.reshape(shape)


def kl(ref_logits: torch.Tensor, q_logits: torch.Tensor, wpos: torch.Tensor | None = None) -> float:
    """sum_pos w_pos KL_pos / sum_pos w_pos (compiler.py:180-188); w = 1 without wpos."""
    r, q = _as_bf16_rows(ref_logits), _as_bf16_rows(q_logits)
    w = None if wpos is None else torch.as_tensor(wpos).reshape(-1).to(r.device, torch.float32)
    _, sums = E.kl_rows(r, q, w)
    s = sums.cpu()
    return float(s[0] / s[1])
