"""Synthetic inputs of the benchmark configurations (seeded numpy PCG64 streams), shared by tests, the fixture
generator and bench.py. Nothing here touches a GPU.

config 1/2: W [960, 960] ~ N(0, 0.02^2) (seed 101); calibration X [16384, 960] ~ N(0, 1) (seed 102) times a
            per-channel |Student-t(4)| scale (seed 103), cast to bfloat16; H = X^T X / N.
config 3:   W_gate, W_up [9728, 2560], W_down [2560, 9728] ~ N(0, 0.015^2) (seeds 301-303); X1 [131072, 2560]
            (seeds 304/305); token weights: a random 10% "digit" subset (seed 306) weighted 10x, mean 1.
config 4:   ref logits [8192, 151936] ~ N(0, 3^2) (seed 401), q = ref + N(0, 0.3^2) (seed 402), bfloat16.
"""

from __future__ import annotations

import numpy as np


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 values rounded to the nearest bfloat16 (ties to even), returned as float32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16).astype(np.uint32)
    return r.view(np.float32)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def weight(m: int, n: int, std: float, seed: int) -> np.ndarray:
    return (np.random.default_rng(seed).standard_normal((m, n), dtype=np.float32) * np.float32(std)).astype(np.float32)


def calibration(N: int, n: int, seed_x: int, seed_scale: int) -> np.ndarray:
    """Channel-scaled Gaussian activations, rounded to bfloat16 (returned as float32 holding bfloat16 values)."""
    s = np.abs(np.random.default_rng(seed_scale).standard_t(4, size=n)).astype(np.float32)
    x = np.random.default_rng(seed_x).standard_normal((N, n), dtype=np.float32) * s[None, :]
    return bf16_round(x)


def digit_weights(N: int, seed: int, share: float = 0.1, factor: float = 10.0) -> np.ndarray:
    """Per-token weights: a random `share` of tokens weighted `factor` times the rest, normalised to mean 1."""
    pick = np.random.default_rng(seed).random(N) < share
    w = np.where(pick, factor, 1.0)
    return (w / w.mean()).astype(np.float32)


def hessian64(X: np.ndarray, w: np.ndarray | None = None, chunk: int = 8192) -> np.ndarray:
    """X^T diag(w) X / N in float64, accumulated in chunks of tokens."""
    N, n = X.shape
    H = np.zeros((n, n))
    for b in range(0, N, chunk):
        x = X[b : b + chunk].astype(np.float64)
        H += x.T @ (x if w is None else x * w[b : b + chunk, None].astype(np.float64))
    return H / N


def config12(rows: int | None = None):
    """(W [m, 960] float32, H [960, 960] float64) of configs 1 and 2. H is rounded through float32, as the
    reference's float32 accumulation hands it over (quantize.py:1470), which also makes it reproducible bit for
    bit whatever BLAS summed it."""
    W = weight(960, 960, 0.02, 101)
    X = calibration(16384, 960, 102, 103)
    H = hessian64(X).astype(np.float32).astype(np.float64)
    return (W if rows is None else W[:rows]), H


def logits(T: int, V: int, seed_ref: int = 401, seed_noise: int = 402, noise: float = 0.3):
    """(ref, q) bfloat16 bit patterns (uint16) of config 4's shape family."""
    r = np.random.default_rng(seed_ref).standard_normal((T, V), dtype=np.float32) * np.float32(3.0)
    rb = bf16_round(r)
    q = rb + np.random.default_rng(seed_noise).standard_normal((T, V), dtype=np.float32) * np.float32(noise)
    return bf16_bits(rb), bf16_bits(q)


def row_plan(m: int, seed: int, groups: int = 8, target_bpw: float = 2.30,
             probs=(0.122, 0.434, 0.378, 0.066)) -> list[dict]:
    """A rowgroup plan for one matrix: a random permutation of the rows cut into `groups` groups (multiples of 64
    rows), bits 1-4 drawn with the LM2 histogram and adjusted until the mean is within 0.125 of `target_bpw`; then
    64 rows at a time move between groups one bit apart until the mean bits per row is within 32 / m of it (2.3
    exactly at the configurations' row counts that are multiples of 320)."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(m)
    size = m // groups // 64 * 64
    sizes = [size] * (groups - 1) + [m - size * (groups - 1)]
    bits = rng.choice([1, 2, 3, 4], size=groups, p=np.asarray(probs) / np.sum(probs))
    for _ in range(64):
        mean = float(np.dot(bits, sizes) / m)
        if abs(mean - target_bpw) <= 0.125:
            break
        i = int(rng.integers(groups))
        if mean < target_bpw and bits[i] < 4:
            bits[i] += 1
        elif mean > target_bpw and bits[i] > 1:
            bits[i] -= 1
    for _ in range(4 * m // 64):
        d = target_bpw * m - float(np.dot(bits, sizes))
        if abs(d) <= 32:
            break
        up = 1 if d > 0 else -1
        pairs = [(i, j) for i in range(groups) for j in range(groups) if bits[j] - bits[i] == up and sizes[i] > 64]
        if not pairs:
            break
        i, j = pairs[int(rng.integers(len(pairs)))]
        sizes[i] -= 64
        sizes[j] += 64
    out, r0 = [], 0
    for g, (s, b) in enumerate(zip(sizes, bits)):
        out.append({"group": g, "rows": sorted(int(v) for v in perm[r0 : r0 + s]), "bits": int(b)})
        r0 += s
    return out
