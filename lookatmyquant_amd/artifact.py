"""Packed trellis codes of the opgraph-packed-1 format (compiler_artifact.py:225-297 of the reference).

pack_trellis runs on the GPU (lamq_pack_trellis): symbols = state & (2^k - 1), each row padded forward with zero
symbols to a multiple of 32, reversed, and packed little-endian, symbol i of a group of 32 in bits [i*k, i*k+k) of
the group's k 32-bit words; a row that is not a trellis path from state 0 raises ValueError. The readers
(unpack_symbols, unpack_trellis) and valid_path are host numpy, as a consumer of the format would have them.
"""

from __future__ import annotations

import numpy as np
import torch

from . import engine as E

STATE_BITS = 12


def valid_path(states, bits: int, state_bits: int = STATE_BITS) -> bool:
    s = np.asarray(states, dtype=np.int64)
    return bool(s.ndim == 2 and s.shape[1] > 0 and np.all((s >= 0) & (s < (1 << state_bits))) and np.all(s[:, 0] < (1 << bits))
                and np.all((s[:, 1:] >> bits) == (s[:, :-1] & ((1 << (state_bits - bits)) - 1))))


def pack_trellis(states, bits: int, state_bits: int = STATE_BITS) -> np.ndarray:
    """uint32 code words [m, ceil(n/32)*bits] of row-trellis states (an array or a tensor; packed on the GPU)."""
    dev = E._abi.device()
    st = torch.as_tensor(np.asarray(states) if not isinstance(states, torch.Tensor) else states)
    st = st.to(dev, torch.int32).contiguous()
    codes = E.pack_trellis(st, bits, state_bits)
    return codes.cpu().numpy().view(np.uint32)


def unpack_symbols(codes, bits: int, columns: int) -> np.ndarray:
    codes = np.asarray(codes, dtype=np.uint32)
    m = codes.shape[0]
    blocks = (columns + 31) // 32
    if codes.shape != (m, blocks * bits):
        raise ValueError("code dimensions disagree with width")
    words = codes.reshape(m, blocks, bits).astype(np.uint64)
    out = np.empty((m, blocks, 32), dtype=np.uint32)
    for i in range(32):
        word, shift = divmod(i * bits, 32)
        v = words[:, :, word] >> np.uint64(shift)
        if shift + bits > 32:
            v |= words[:, :, word + 1] << np.uint64(32 - shift)
        out[:, :, i] = (v & np.uint64((1 << bits) - 1)).astype(np.uint32)
    return out.reshape(m, -1)[:, :columns]


def unpack_trellis(codes, bits: int, columns: int, state_bits: int = STATE_BITS) -> np.ndarray:
    """The states of packed row-trellis codes: symbols un-reversed, then each state shifted in from state 0."""
    padded = (columns + 31) // 32 * 32
    sym = unpack_symbols(codes, bits, padded)[:, ::-1]
    state = np.zeros(len(sym), dtype=np.uint32)
    out = np.empty((len(sym), columns), dtype=np.uint32)
    mask = (1 << state_bits) - 1
    for i in range(columns):
        state = ((state << bits) | sym[:, i]) & mask
        out[:, i] = state
    return out
