"""TEST INFRASTRUCTURE, NOT PRODUCT CODE.

The CPU oracle for the per-matrix quantization hot path: a restatement of the reference's
algorithm (ShinMegamiBoson/lookatmyquant) in plain C (lamq_oracle.c, loaded here through ctypes)
and numpy. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import it,
and only as the checker or the timed CPU baseline; the product (lookatmyquant_amd) never does.

Parity status of each function (what pins it is listed in the test named beside it):
  viterbi            brute force over all paths incl. exact-arithmetic tie cases (tests/test_oracle.py)
                     and the reference's own vectors (tests/golden)
  ldlq_trellis       least-squares refit identity, H = c*I composition, reference vectors
  ldlq_scalar        least-squares refit identity, eager GPTQ identity, reference vectors
  environment        LAPACK closed form; U^T U = H_damped^-1
  ldlq_factor        U^T U = (H + d mean(diag H) I)^-1 at the first d that factors; the retry path
  ldlq_round         the eager GPTQ loop of ldlq_gpu.py (reference vectors of ldlq_scalar); lazy-block invariance
  sweep              equals the C sweeps (ldlq_scalar, ldlq_trellis) under their projections
  multirate_sweep    the reference's own vectors for three and four rates, with and without H (tests/golden/multirate.npz);
                     one rate at weight 1 equals ldlq_scalar
  column_trellis_*   per-sequence viterbi (pinned above) on the reshaped columns; brute force for tiny L
  hadamard / rht     orthogonality, |H_ij| = 1/sqrt(n), Kronecker closed forms
  rht_apply          equals the products with the dense rht(n, seed) both ways (tests/test_oracle.py)
  hessian            fp64 closed form X^T diag(w) X / N
  kl_rows            fp64 closed form; KL(p||p) = 0; Gaussian-logit closed form
  kl_rows_float      equals kl_rows on bf16-valued logits; the Bernoulli closed form; shift invariance
  shaped_sweep       isotropic G equals the one-rate multirate_sweep; one column's row pass equals sweep along the rows
  lloyd_max          Max (1960) MSE table; GAUSS2 levels; reference vectors
  pack_symbols etc.  round trip and the reference's byte layout spelled out bit by bit
  ldlq_noise         A A^T = Hr with A upper; tr(E_r Hr E_r^T) = sum diag(A)^2 eta^2 (QuIP Theorem 1's identity);
                     E_r A = eta diag(A) exactly; zero noise gives W
"""

from __future__ import annotations

import ctypes
import math
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
_LIB = None

_i64, _i32, _dbl = ctypes.c_int64, ctypes.c_int, ctypes.c_double
_p = ctypes.c_void_p


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def build():
    """Compile lamq_oracle.c with gcc (no reference sources are involved: the reference is Python)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib():
    global _LIB
    if _LIB is None:
        so = HERE / "liblamq_oracle.so"
        if not so.exists() or so.stat().st_mtime < (HERE / "lamq_oracle.c").stat().st_mtime:
            build()
        L = ctypes.CDLL(str(so))
        L.orc_viterbi.argtypes = [_p, _i64, _i32, _i64, _p, _i32, _i32, _p, _p]
        L.orc_ldlq_trellis.argtypes = [_p, _i64, _i64, _i64, _p, _i64, _p, _p, _i32, _i32, _i32, _i32, _i32, _p, _p, _p]
        L.orc_ldlq_scalar.argtypes = [_p, _i64, _i64, _i64, _p, _i64, _p, _p, _i32, _i32, _i32, _p, _p, _p]
        L.orc_kl_rows.argtypes = [_p, _p, _i64, _i64, _i64, _i64, _p, _p, _p, _p]
        for f in (L.orc_viterbi, L.orc_ldlq_trellis, L.orc_ldlq_scalar, L.orc_kl_rows):
            f.restype = _i32
        _LIB = L
    return _LIB


def _check(rc, what):
    if rc != 0:
        raise ValueError(f"{what}: oracle returned {rc}")


# ----------------------------------------------------------------------------- Viterbi (codes.py:151-181)


def viterbi(X, values, L: int, k: int, start=None) -> np.ndarray:
    """States (rows, T) of the nearest trellis path, as opgraph/codes.py:151-181: X and the values are cast to float32."""
    x = np.ascontiguousarray(np.asarray(X, dtype=np.float64).astype(np.float32))
    if x.ndim != 2:
        raise ValueError("X must be (rows, T)")
    C = np.ascontiguousarray(np.asarray(values, dtype=np.float64).astype(np.float32))
    if len(C) != 1 << L:
        raise ValueError("values must have 2^L entries")
    st = None if start is None else np.ascontiguousarray(np.asarray(start, dtype=np.int64))
    out = np.empty(x.shape, dtype=np.int32)
    _check(lib().orc_viterbi(_ptr(x), x.shape[0], x.shape[1], x.shape[1], _ptr(C), L, k, _ptr(st), _ptr(out)), "viterbi")
    return out.astype(np.int64)


# ----------------------------------------------------------------------------- sweeps (syntax.py:86-124)


def ldlq_trellis(X, U, S, table64, L: int, k: int, width: int = 16, look: int = 8, lazy: int = 128, dead=None,
                 want_before: bool = False):
    """Row-trellis block LDLQ of X (rows in the rotated basis, not yet divided by S): the states, and optionally
    each column as it stood before it was settled. opgraph/codes.py:397-404,442-452 inside syntax.py:86-124."""
    T = np.array(X, dtype=np.float64, order="C", copy=True)
    m, n = T.shape
    U = np.ascontiguousarray(U, dtype=np.float64)
    S = np.ascontiguousarray(S, dtype=np.float64)
    tb = np.ascontiguousarray(table64, dtype=np.float64)
    dd = None if dead is None else np.ascontiguousarray(dead, dtype=np.uint8)
    states = np.empty((m, n), dtype=np.int32)
    before = np.empty((m, n), dtype=np.float64) if want_before else None
    _check(lib().orc_ldlq_trellis(_ptr(T), m, n, n, _ptr(U), U.shape[1], _ptr(S), _ptr(tb), L, k, width, look, lazy,
                                  _ptr(dd), _ptr(states), _ptr(before)), "ldlq_trellis")
    return (states, before) if want_before else states


def ldlq_scalar(T0, U, levels, mode: int = 0, S=None, lazy: int = 128, dead=None, want_before: bool = False):
    """Width-1 LDLQ onto a scalar set. mode 0: nested.multirate_sweep with one rate (T0 already X/S, argmin with the
    first minimum); mode 1: ldlq_words with a ScalarCode (T0 = X, bucketize(t/S) on midpoints, q*S)."""
    T = np.array(T0, dtype=np.float64, order="C", copy=True)
    m, n = T.shape
    U = np.ascontiguousarray(U, dtype=np.float64)
    lv = np.ascontiguousarray(levels, dtype=np.float64)
    Sv = None if S is None else np.ascontiguousarray(S, dtype=np.float64)
    dd = None if dead is None else np.ascontiguousarray(dead, dtype=np.uint8)
    idx = np.empty((m, n), dtype=np.int32)
    before = np.empty((m, n), dtype=np.float64) if want_before else None
    _check(lib().orc_ldlq_scalar(_ptr(T), m, n, n, _ptr(U), U.shape[1], _ptr(Sv), _ptr(lv), len(lv), mode, lazy,
                                 _ptr(dd), _ptr(idx), _ptr(before)), "ldlq_scalar")
    return (idx, before) if want_before else idx


# ----------------------------------------------------------------------------- environment (frame.py:508-522)


def environment(H, damp: float = 0.01):
    """(H damped, U, dead): dead = diag(H) == 0 gets a unit diagonal, H += damp*mean(diag H)*I, and U is the upper
    Cholesky factor of H^-1 (torch.linalg.cholesky(torch.cholesky_inverse(torch.linalg.cholesky(H)), upper=True))."""
    H = np.array(H, dtype=np.float64, copy=True)
    dead = np.diag(H) == 0
    idx = np.nonzero(dead)[0]
    H[idx, idx] = 1.0
    H = H + damp * np.mean(np.diag(H)) * np.eye(len(H))
    Lc = np.linalg.cholesky(H)
    Li = np.linalg.inv(Lc)
    Hinv = Li.T @ Li
    U = np.linalg.cholesky(Hinv).T
    return H, U, dead


def ldlq_factor(Hr, damp: float = 0.01) -> np.ndarray:
    """U of opgraph/ldlq_gpu.py:15-25: H = (Hr + Hr^T)/2 damped by d*mean(diag H) for d = damp, 10 damp, 100 damp until
    it factors (a zero diagonal stays zero and counts in the mean); U = upper Cholesky factor of the damped H's inverse.
    Raises AssertionError when no damping factors."""
    H = np.asarray(Hr, dtype=np.float64)
    H = 0.5 * (H + H.T)
    for d in (damp, 10 * damp, 100 * damp):
        try:
            Lc = np.linalg.cholesky(H + d * np.mean(np.diag(H)) * np.eye(len(H)))
        except np.linalg.LinAlgError:
            continue
        Li = np.linalg.inv(Lc)
        return np.linalg.cholesky(Li.T @ Li).T
    raise AssertionError("H is not positive definite even with damping")


def ldlq_round(X, U, levels, block: int = 128) -> np.ndarray:
    """The levels opgraph/ldlq_gpu.py:28-49 chooses: the width-1 sweep of ldlq_scalar with unit row scales (bucketize
    on the midpoints, the rounding error carried through U, lazy blocks of `block`)."""
    lv = np.asarray(levels, dtype=np.float64)
    idx = ldlq_scalar(X, U, lv, 1, np.ones(np.shape(X)[0]), block)
    return lv[idx]


def sweep(W, U, project, width: int = 1, lazy: int = 128, dead=None) -> np.ndarray:
    """The generic block sweep of opgraph/syntax.py:86-124 in numpy: columns settled `width` at a time, project(j, cols, T)
    returns the settled block, E = cols - q, z = E U_BB^-1, the rest of the lazy run refit at once and the columns after
    it by one product per run. Returns each column as it stood before it was settled."""
    from scipy.linalg import solve_triangular

    T = np.array(W, dtype=np.float64, copy=True)
    U = np.asarray(U, dtype=np.float64)
    if dead is not None:
        T[:, np.asarray(dead, dtype=bool)] = 0.0
    if lazy % width:
        raise ValueError("lazy must be a multiple of width")
    m, n = T.shape
    before = np.empty_like(T)
    for b0 in range(0, n, lazy):
        b1 = min(b0 + lazy, n)
        Z = np.empty((m, b1 - b0))
        for j in range(b0, b1, width):
            w = min(width, b1 - j)
            before[:, j : j + w] = T[:, j : j + w]
            q = np.asarray(project(j, T[:, j : j + w].copy(), T), dtype=np.float64).reshape(m, w)
            E = T[:, j : j + w] - q
            z = solve_triangular(U[j : j + w, j : j + w].T, E.T, lower=True).T  # z U_BB = E
            T[:, j + w : b1] -= z @ U[j : j + w, j + w : b1]
            Z[:, j - b0 : j - b0 + w] = z
        if b1 < n:
            T[:, b1:] -= Z @ U[b0:b1, b1:]
    return before


def multirate_sweep(X, H, tables, weights, lazy: int = 128) -> np.ndarray:
    """opgraph/nested.py:104-147 without output shaping: one index per entry of X (units of the row scale) for R rates
    at once, idx = first argmin_i sum_r w_r (t_r - tables[r, i])^2 (w_r times the rounded square, the rates summed in
    order); with H the width-1 sweep of X.repeat(R, 1) (the rates' copies of each row, rate-major) under
    Environment(H)'s U, each copy refit for its own rate's value; without H every column alone."""
    X = np.asarray(X, dtype=np.float64)
    tables = np.asarray(tables, dtype=np.float64)
    w = np.asarray(weights, dtype=np.float64)
    R, m = tables.shape[0], X.shape[0]
    idx = np.empty(X.shape, dtype=np.int64)

    def project(j, col, T):
        t = np.asarray(col).reshape(R, m)
        cost = (w[:, None, None] * (t[:, :, None] - tables[:, None, :]) ** 2).sum(0)
        i = cost.argmin(1)
        idx[:, j] = i
        return tables[:, i].reshape(-1, 1)

    if H is None:
        for j in range(X.shape[1]):
            project(j, np.tile(X[:, j], R), None)
        return idx
    _, U, dead = environment(H)
    sweep(np.tile(X, (R, 1)), U, project, width=1, lazy=lazy, dead=dead if dead.any() else None)
    return idx


OUTPUT_DAMP = 0.03  # opgraph/nested.py:101


def shaped_sweep(X, H, levels, G, block: int = 32, lazy: int = 128) -> np.ndarray:
    """opgraph/nested.py:104-147 with output shaping (one rate; G the output sensitivity in units of the row scale):
    V = Environment(G, damp=0.03).U (:121); within each column the rows are settled `block` at a time, each entry on its
    nearest level (the first least |u - level|, :131), and the later rows re-solved, u[b:] -= (u[a:b] - q[a:b]) M with
    M = V[a:b, a:b]^-1 V[a:b, b:] (:123-133); with H the width-1 sweep under Environment(H)'s U (:144), without H every
    column alone (:140-143). Indices int64."""
    from scipy.linalg import solve_triangular

    X = np.asarray(X, dtype=np.float64)
    lv = np.asarray(levels, dtype=np.float64)
    m = X.shape[0]
    _, V, _ = environment(G, damp=OUTPUT_DAMP)
    rows = [(a, min(a + block, m)) for a in range(0, m, block)]
    feedback = [solve_triangular(V[a:b, a:b], V[a:b, b:]) for a, b in rows]  # upper V[a:b, a:b] M = V[a:b, b:]
    idx = np.empty(X.shape, dtype=np.int64)

    def project(j, col, T):
        u = np.array(col, dtype=np.float64).reshape(-1)
        i = np.empty(m, dtype=np.int64)
        for (a, b), M in zip(rows, feedback):
            i[a:b] = np.abs(u[a:b, None] - lv[None, :]).argmin(1)
            if b < m:
                u[b:] -= (u[a:b] - lv[i[a:b]]) @ M
        idx[:, j] = i
        return lv[i].reshape(-1, 1)

    if H is None:
        for j in range(X.shape[1]):
            project(j, X[:, j], None)
        return idx
    _, U, dead = environment(H)
    sweep(X, U, project, width=1, lazy=lazy, dead=dead if dead.any() else None)
    return idx


def column_trellis_states(X, table64, L: int, k: int, T: int) -> np.ndarray:
    """TrellisCode's search (opgraph/codes.py:371-378): each column cut into sequences of T consecutive rows, each
    sequence the nearest path from a free first state; the states in X's layout."""
    X = np.asarray(X, dtype=np.float64)
    o, w = X.shape
    seqs = X.reshape(o // T, T, w).transpose(0, 2, 1).reshape(-1, T)
    st = viterbi(seqs, table64, L, k)
    return st.reshape(o // T, w, T).transpose(0, 2, 1).reshape(o, w)


def ldlq_words_column_trellis(W, H, table64, L: int, k: int, T: int, seed: int, in_seed: int, width: int = 16):
    """ldlq_words([W], H, TrellisCode(L, k, T), [seed], in_seed=in_seed) (codes.py:413-462): rows rotated by R_out,
    columns by R_in, per-row RMS scale, the generic sweep with the column-sequence projection. The states and the row
    scales (H None: the code applied directly)."""
    W = np.asarray(W, dtype=np.float64)
    X = rht(W.shape[0], seed) @ W @ rht(W.shape[1], in_seed).T
    S = row_scale(X)
    tb = np.asarray(table64, dtype=np.float64)
    if H is None:
        return column_trellis_states(X / S[:, None], tb, L, k, T), S
    R = rht(W.shape[1], in_seed)
    _, U, dead = environment(R @ np.asarray(H, dtype=np.float64) @ R.T)
    states = np.empty(X.shape, dtype=np.int64)

    def project(j, x, _T):
        st = column_trellis_states(x / S[:, None], tb, L, k, T)
        states[:, j : j + x.shape[1]] = st
        return tb[st] * S[:, None]

    sweep(X, U, project, width, 128, dead if dead.any() else None)
    return states, S


# ----------------------------------------------------------------------------- Hadamard and RHT (codes.py:83-132)


def _is_prime(q: int) -> bool:
    return q > 1 and all(q % d for d in range(2, math.isqrt(q) + 1))


def _sylvester(a: int) -> np.ndarray:
    H = np.ones((1, 1))
    while H.shape[0] < 2**a:
        H = np.block([[H, H], [H, -H]])
    return H


def _paley(q: int) -> np.ndarray:
    """Paley's first construction, order q + 1, q prime and q = 3 mod 4 (codes.py:87-94)."""
    squares = {(x * x) % q for x in range(1, q)}
    chi = np.array([0.0] + [1.0 if a in squares else -1.0 for a in range(1, q)])
    Q = chi[(np.arange(q)[None, :] - np.arange(q)[:, None]) % q]
    S = np.zeros((q + 1, q + 1))
    S[0, 1:], S[1:, 0], S[1:, 1:] = 1, -1, Q
    return S + np.eye(q + 1)


def hadamard_factors(n: int):
    """A, B with hadamard(n) = kron(A, B)/sqrt(n) (codes.py:104-119)."""
    for a in range(int(math.log2(n)), -1, -1):
        if n % 2**a:
            continue
        p = n // 2**a
        if p in (1, 2) or (_is_prime(p - 1) and (p - 1) % 4 == 3):
            if p == 1 and a > 1:
                return _sylvester(a // 2), _sylvester(a - a // 2)
            P = np.array([[1.0, 1.0], [1.0, -1.0]]) if p == 2 else np.ones((1, 1)) if p == 1 else _paley(p - 1)
            return _sylvester(a), P
    raise ValueError(f"no Hadamard construction here for order {n}")


def hadamard(n: int) -> np.ndarray:
    A, B = hadamard_factors(n)
    return np.kron(A, B) / math.sqrt(n)


def rht_signs(n: int, seed: int) -> np.ndarray:
    """s = -1 where torch.rand(n, Generator(seed), float64) < 0.5 (codes.py:131): the library RNG the reference calls."""
    import torch
    u = torch.rand(n, generator=torch.Generator().manual_seed(int(seed)), dtype=torch.float64).numpy()
    return np.where(u < 0.5, -1.0, 1.0)


def rht(n: int, seed: int) -> np.ndarray:
    return hadamard(n) * rht_signs(n, seed)[None, :]


def rht_apply(X, seed: int, inverse: bool = False) -> np.ndarray:
    """X @ rht(n, seed).T (the incoherent rows, codes.py:430), or with inverse X @ rht(n, seed) (a reconstruction,
    codes.py:459-462), through the factors hadamard(n) = kron(A, B) / sqrt(n) instead of the dense matrix: for a row
    z of length a b laid out as an a x b matrix Z, z kron(A, B)^T = vec(A Z B^T) and z kron(A, B) = vec(A^T Z B)."""
    X = np.asarray(X, dtype=np.float64)
    m, n = X.shape
    A, B = hadamard_factors(n)
    s = rht_signs(n, seed)
    if not inverse:
        Z = (X * s[None, :]).reshape(m, len(A), len(B))
        return (A @ Z @ B.T).reshape(m, n) / math.sqrt(n)
    Z = X.reshape(m, len(A), len(B))
    return (A.T @ Z @ B).reshape(m, n) / math.sqrt(n) * s[None, :]


# ----------------------------------------------------------------------------- statistics and scales


def hessian(X, w=None) -> np.ndarray:
    """H = (1/N) sum_t w_t x_t x_t^T in float64 (quantize.py:1465,1470 with the token weights of :1389-1391)."""
    X = np.asarray(X, dtype=np.float64)
    Xw = X if w is None else X * np.asarray(w, dtype=np.float64)[:, None]
    return (X.T @ Xw) / X.shape[0]


def cross_gram(Xr, Xq, w=None) -> np.ndarray:
    """D = (1/N) X_ref^T (w * X_q) in float64 (quantize.py:1457)."""
    Xr = np.asarray(Xr, dtype=np.float64)
    Xq = np.asarray(Xq, dtype=np.float64)
    Xw = Xq if w is None else Xq * np.asarray(w, dtype=np.float64)[:, None]
    return (Xr.T @ Xw) / Xr.shape[0]


def row_scale(X) -> np.ndarray:
    """S_r = max(sqrt(mean_j X_rj^2), 1e-12) (codes.py:436; nested.py:168)."""
    X = np.asarray(X, dtype=np.float64)
    return np.maximum(np.sqrt((X * X).mean(1)), 1e-12)


# ----------------------------------------------------------------------------- Lloyd-Max (nested.py:36-82)


def _phi(x):
    return np.exp(-0.5 * x * x) / math.sqrt(2 * math.pi)


def _Phi(x):
    from scipy.special import erf
    return 0.5 * (1 + erf(x / math.sqrt(2)))


def gaussian_centroids(bounds) -> np.ndarray:
    a, b = bounds[:-1], bounds[1:]
    with np.errstate(invalid="ignore"):
        pa = np.where(np.isinf(a), 0.0, _phi(a))
        pb = np.where(np.isinf(b), 0.0, _phi(b))
    return (pa - pb) / (_Phi(b) - _Phi(a))


def lloyd_max_levels(n: int, iters: int = 500) -> np.ndarray:
    from scipy.special import ndtri
    lv = gaussian_centroids(ndtri(np.arange(n + 1, dtype=np.float64) / n) * math.sqrt(3))
    for _ in range(iters):
        mid = (lv[1:] + lv[:-1]) / 2
        lv = gaussian_centroids(np.concatenate([[-math.inf], mid, [math.inf]]))
    return lv


def lloyd_max(bits: int, iters: int = 500) -> np.ndarray:
    return lloyd_max_levels(2**bits, iters)


def gaussian_mse(bounds, levels) -> float:
    """E[(x - q(x))^2] for x ~ N(0,1) (nested.py:51-59)."""
    a, b = bounds[:-1], bounds[1:]
    P = _Phi(b) - _Phi(a)
    with np.errstate(invalid="ignore"):
        fa = lambda t: np.where(np.isinf(t), 0.0, t * _phi(t))
        pa = lambda t: np.where(np.isinf(t), 0.0, _phi(t))
        m1 = pa(a) - pa(b)
        m2 = P + fa(a) - fa(b)
    return float((m2 - 2 * levels * m1 + levels**2 * P).sum())


# ----------------------------------------------------------------------------- KL (compiler.py:177-188)


def kl_rows(ref_bf16, q_bf16, w=None):
    """Per-token KL(p_ref || p_q) in float64 from bfloat16 logits given as uint16 bit patterns; returns (kl per token,
    sum_t w_t kl_t / sum_t w_t)."""
    r = np.ascontiguousarray(ref_bf16, dtype=np.uint16)
    q = np.ascontiguousarray(q_bf16, dtype=np.uint16)
    T, V = r.shape
    ww = None if w is None else np.ascontiguousarray(w, dtype=np.float32)
    kl = np.empty(T, dtype=np.float64)
    sw, st = ctypes.c_double(), ctypes.c_double()
    _check(lib().orc_kl_rows(_ptr(r), _ptr(q), T, V, V, V, _ptr(ww), _ptr(kl), ctypes.byref(sw), ctypes.byref(st)), "kl")
    return kl, (sw.value / st.value if st.value else 0.0)


def kl_rows_float(ref, q, w=None):
    """kl_rows for float logits (the reference's .logits.float(), compiler.py:180,185): the float32 values taken
    exactly, KL(p_ref || p_q) per token in float64 through log-sum-exp; returns (kl per token, sum_t w_t kl_t /
    sum_t w_t)."""
    r = np.asarray(ref, dtype=np.float32).astype(np.float64)
    p = np.asarray(q, dtype=np.float32).astype(np.float64)
    mr, mq = r.max(axis=1, keepdims=True), p.max(axis=1, keepdims=True)
    er = np.exp(r - mr)
    sr = er.sum(axis=1)
    lse_r = mr[:, 0] + np.log(sr)
    lse_q = mq[:, 0] + np.log(np.exp(p - mq).sum(axis=1))
    kl = (er * (r - p)).sum(axis=1) / sr - lse_r + lse_q
    ww = np.ones(len(kl)) if w is None else np.asarray(w, dtype=np.float32).astype(np.float64)
    return kl, (float((ww * kl).sum() / ww.sum()) if ww.sum() else 0.0)


def bf16_bits(x) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round to nearest even (what torch's .to(bfloat16) does)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r


def bf16_to_f32(h) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ----------------------------------------------------------------------------- packing (compiler_artifact.py:225-297)


def pack_symbols(q, bits: int) -> np.ndarray:
    """Symbols (m, n) < 2^bits, each row padded to a multiple of 32 and packed little-endian: symbol i of a group of
    32 starts at bit i*bits of the group's `bits` 32-bit words (compiler_artifact.py:225-240)."""
    q = np.asarray(q)
    m, n = q.shape
    npad = (n + 31) // 32 * 32
    out = np.zeros((m, npad // 32 * bits), dtype=np.uint32)
    for r in range(m):
        for g in range(npad // 32):
            acc = 0
            for i in range(32):
                c = g * 32 + i
                v = int(q[r, c]) if c < n else 0
                acc |= v << (i * bits)
            for wd in range(bits):
                out[r, g * bits + wd] = (acc >> (32 * wd)) & 0xFFFFFFFF
    return out


def unpack_symbols(codes, bits: int, columns: int) -> np.ndarray:
    codes = np.asarray(codes, dtype=np.uint32)
    m = codes.shape[0]
    blocks = (columns + 31) // 32
    out = np.zeros((m, blocks * 32), dtype=np.uint32)
    for r in range(m):
        for g in range(blocks):
            acc = 0
            for wd in range(bits):
                acc |= int(codes[r, g * bits + wd]) << (32 * wd)
            for i in range(32):
                out[r, g * 32 + i] = (acc >> (i * bits)) & ((1 << bits) - 1)
    return out[:, :columns]


def valid_path(states, bits: int, state_bits: int = 12) -> bool:
    s = np.asarray(states, dtype=np.int64)
    return bool(s.ndim == 2 and s.shape[1] > 0 and np.all((s >= 0) & (s < (1 << state_bits))) and np.all(s[:, 0] < (1 << bits))
                and np.all((s[:, 1:] >> bits) == (s[:, :-1] & ((1 << (state_bits - bits)) - 1))))


def pack_trellis(states, bits: int, state_bits: int = 12) -> np.ndarray:
    """Symbols = state & (2^bits - 1), padded forward to 32, the row reversed, then packed (compiler_artifact.py:276-284)."""
    s = np.asarray(states, dtype=np.int64)
    if not valid_path(s, bits, state_bits):
        raise ValueError("states are not a row trellis from zero")
    sym = s & ((1 << bits) - 1)
    sym = np.pad(sym, ((0, 0), (0, (-sym.shape[1]) % 32)))
    return pack_symbols(sym[:, ::-1], bits)


def unpack_trellis(codes, bits: int, columns: int, state_bits: int = 12) -> np.ndarray:
    padded = (columns + 31) // 32 * 32
    sym = unpack_symbols(codes, bits, padded)[:, ::-1]
    state = np.zeros(len(sym), dtype=np.int64)
    out = np.empty((len(sym), columns), dtype=np.int64)
    for i in range(columns):
        state = ((state << bits) | sym[:, i]) & ((1 << state_bits) - 1)
        out[:, i] = state
    return out


# ----------------------------------------------------------------------------- LDLQ-shaped noise (compiler.py:110-129)


def ldlq_noise(W, H, d: float, seed: int, eta_unit, row_rotation: bool = True):
    """(W + E, E_r, A) of compiler.ldlq_noise: Wr = Ro W Ri^T (Ri = rht(n, seed+1), Ro = rht(m, seed)),
    Hr = Ri H Ri^T + 0.01 mean(diag) I = A A^T with A upper triangular (the flipped lower Cholesky factor of the
    flipped Hr), eta = eta_unit * RMS(Wr rows) * sqrt(d) (eta_unit: the standard normal draw), E_r A = eta diag(A) by
    a triangular solve, E = Ro^T E_r Ri. LAPACK (numpy cholesky, scipy solve_triangular) in float64."""
    from scipy.linalg import solve_triangular

    W = np.asarray(W, dtype=np.float64)
    m, n = W.shape
    Ri = rht(n, seed + 1)
    Ro = rht(m, seed) if row_rotation else None
    Wr = Ro @ W @ Ri.T if row_rotation else W @ Ri.T
    Hr = Ri @ np.asarray(H, dtype=np.float64) @ Ri.T
    Hr = Hr + 0.01 * np.mean(np.diag(Hr)) * np.eye(n)
    A = np.linalg.cholesky(Hr[::-1, ::-1])[::-1, ::-1]
    S = np.sqrt(np.mean(Wr ** 2, axis=1, keepdims=True))
    eta = np.asarray(eta_unit, dtype=np.float64) * S * d ** 0.5
    Er = solve_triangular(A.T, (eta * np.diag(A)[None, :]).T, lower=True).T  # E_r A = eta diag(A)
    E = Ro.T @ Er @ Ri if row_rotation else Er @ Ri
    return W + E, Er, A


# ----------------------------------------------------------------------------- end-to-end words


def ldlq_words_trellis(W, H, table64, L: int, k: int, in_seed: int, width: int = 16, look: int = 8, lazy: int = 128):
    """ldlq_words([W], H, RowTrellisCode(L, k), [seed], in_seed=in_seed, out_rot=False) (codes.py:413-462): the
    states, the row scales and the reconstruction diag(S) table[states] R_in."""
    W = np.asarray(W, dtype=np.float64)
    R = rht(W.shape[1], in_seed)
    X = W @ R.T
    S = row_scale(X)
    Hr = R @ np.asarray(H, dtype=np.float64) @ R.T
    _, U, dead = environment(Hr)
    st = ldlq_trellis(X, U, S, table64, L, k, width, look, lazy, dead if dead.any() else None)
    What = (S[:, None] * np.asarray(table64)[st]) @ R
    return st, S, What


def nested_lm(W, H, levels, in_seed: int, lazy: int = 128):
    """nested_words([W], H, [seed], b, [b], 0.4, [1.0], lloyd_max(b), in_seed=in_seed, out_rot=False)[b][0]
    (nested.py:155-192): the level indices, the row scales and the reconstruction."""
    W = np.asarray(W, dtype=np.float64)
    R = rht(W.shape[1], in_seed)
    X = W @ R.T
    S = row_scale(X)
    Hr = R @ np.asarray(H, dtype=np.float64) @ R.T
    _, U, dead = environment(Hr)
    idx = ldlq_scalar(X / S[:, None], U, levels, 0, None, lazy, dead if dead.any() else None)
    What = (S[:, None] * np.asarray(levels)[idx]) @ R
    return idx, S, What
