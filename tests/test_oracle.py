"""The CPU oracle pinned: against the reference's own vectors (tests/golden, written from the reference by
tests/golden/make_golden.py), against brute force on tiny trellises, and against identities the mathematics fixes
(least-squares refit, the H = c*I composition, closed-form KL, Max 1960). CPU only."""

import itertools
import math

import numpy as np
import pytest

from oracle import oracle as O


# ----------------------------------------------------------------------------- Viterbi


@pytest.mark.parametrize("k", [1, 2, 3, 4])
def test_viterbi_matches_reference_vectors(golden, tables, k):
    g = golden("viterbi")
    x = g[f"L12_k{k}_x"]
    assert np.array_equal(O.viterbi(x, tables[k], 12, k), g[f"L12_k{k}_free"])
    assert np.array_equal(O.viterbi(x, tables[k], 12, k, start=g[f"L12_k{k}_start"]), g[f"L12_k{k}_fixed"])


def test_viterbi_L16_fp16_table_matches_reference(golden):
    g = golden("viterbi")
    got = O.viterbi(g["L16_k2_x"], g["L16_k2_table"], 16, 2, start=g["L16_k2_start"])
    assert np.array_equal(got, g["L16_k2_fixed"])


@pytest.mark.parametrize("L,k", [(8, 2), (6, 1), (9, 3)])
def test_viterbi_tie_rules_match_reference(golden, L, k):
    g = golden("viterbi")
    p = f"ties_L{L}_k{k}_"
    assert np.array_equal(O.viterbi(g[p + "x"], g[p + "table"], L, k), g[p + "free"])
    assert np.array_equal(O.viterbi(g[p + "x"], g[p + "table"], L, k, start=g[p + "start"]), g[p + "fixed"])


def _paths(L, k, T, start=None):
    """Every path of T states (first state free, or continuing from `start`)."""
    firsts = range(1 << L) if start is None else [((start << k) | b) & ((1 << L) - 1) for b in range(1 << k)]
    for s0 in firsts:
        for bits in itertools.product(range(1 << k), repeat=T - 1):
            s, path = s0, [s0]
            for b in bits:
                s = ((s << k) | b) & ((1 << L) - 1)
                path.append(s)
            yield path


def test_viterbi_is_optimal_by_brute_force():
    """tests/test_codes.py:101-117 of the reference: the path cost equals the best over all paths."""
    rng = np.random.default_rng(0)
    L, k, T = 4, 1, 7
    v = rng.standard_normal(1 << L)
    X = rng.standard_normal((5, T))
    st = O.viterbi(X, v, L, k)
    v32, X32 = v.astype(np.float32), X.astype(np.float32)
    for r in range(len(X)):
        best = min(sum((float(X32[r, t]) - float(v32[s])) ** 2 for t, s in enumerate(p)) for p in _paths(L, k, T))
        got = sum((float(X32[r, t]) - float(v32[s])) ** 2 for t, s in enumerate(st[r]))
        assert abs(got - best) < 1e-5
        assert all((st[r][t] >> k) == (st[r][t - 1] & ((1 << (L - k)) - 1)) for t in range(1, T))


@pytest.mark.parametrize("L,k,start,T", [(4, 1, None, 6), (5, 2, None, 6), (4, 2, 9, 6), (6, 2, 17, 6),
                                         (6, 5, None, 3), (6, 5, 45, 3), (5, 5, None, 3), (7, 6, 100, 3)])
def test_viterbi_ties_by_brute_force(L, k, start, T):
    """With small-integer values every float32 sum is exact, so the path the search keeps is determined by its
    rules alone: among minimal-cost paths the lowest final state, then at each earlier step the predecessor with
    the lowest top bits (torch's min returns the first minimum). Brute force over all paths with that order; the
    widths past 4 (k up to 8 in the reference, its back-pointers uint8) and k = L (one group) on short paths."""
    rng = np.random.default_rng(L * 100 + k)
    v = rng.integers(-2, 3, 1 << L).astype(np.float64)
    R = 1 << (L - k)
    for _ in range(6):
        x = rng.integers(-3, 4, T).astype(np.float64)
        st = O.viterbi(x[None], v, L, k, start=None if start is None else [start])[0]

        def key(p):
            cost = sum((x[t] - v[s]) ** 2 for t, s in enumerate(p))
            tops = tuple(p[t - 1] // R for t in range(T - 1, 0, -1))  # h of each step, last step first
            return (cost, p[-1]) + tops

        want = min(_paths(L, k, T, start), key=key)
        assert list(st) == list(want), (list(st), want)


# ----------------------------------------------------------------------------- the sweeps


def _spd(n, seed, N=None):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((N or 3 * n, n)) * np.abs(rng.standard_t(4, n))
    return X.T @ X / len(X)


def test_ldlq_trellis_matches_reference_vectors(golden, tables, config12):
    """Config 2 rows (rows are independent given H): the reference's states, bit for bit."""
    W, H = config12
    g = golden("ldlq_trellis_c2_L12_k2")
    st, S, What = O.ldlq_words_trellis(W[:96], H, tables[2], 12, 2, 201)
    assert np.array_equal(st, g["states"][:96])
    assert np.allclose(S, g["S"][:96], rtol=1e-14, atol=0)
    assert np.abs(What[:8] - g["what_rows"]).max() < 1e-12 * np.abs(g["what_rows"]).max()


@pytest.mark.parametrize("k", [1, 3, 4])
def test_ldlq_trellis_widths_match_reference_vectors(golden, tables, config12, k):
    W, H = config12
    g = golden(f"ldlq_trellis_L12_k{k}_rows128")
    st, _, _ = O.ldlq_words_trellis(W[:32], H, tables[k], 12, k, 201)
    assert np.array_equal(st, g["states"][:32])


def test_nested_lm3_matches_reference_vectors(golden, config12):
    W, H = config12
    g = golden("nested_lm3_c1")
    idx, S, What = O.nested_lm(W, H, g["levels"], 201)
    assert np.array_equal(idx, g["idx"].astype(np.int32))
    assert np.abs(What[:8] - g["what_rows"]).max() < 1e-12 * np.abs(g["what_rows"]).max()


def _refit_exact(H, W, fixed_cols, values):
    """The least-squares form of the refit (opgraph/frame.py:539-546): given the fixed columns, the free columns
    minimising ||(W - W_hat) X||."""
    free = [j for j in range(W.shape[1]) if j not in set(fixed_cols)]
    out = W.copy()
    out[:, fixed_cols] = values
    out[:, free] = W[:, free] + (W[:, fixed_cols] - values) @ H[np.ix_(fixed_cols, free)] @ np.linalg.inv(H[np.ix_(free, free)])
    return out


@pytest.mark.parametrize("kind", ["scalar", "trellis"])
def test_sweep_is_the_least_squares_refit(kind, tables):
    """Each column just before it is settled equals the least-squares refit of W given the columns settled before
    it: the lazy block refit (in-block and trailing) is exact, whatever the projection chose."""
    n, m = 40, 6
    H = _spd(n, 1)
    Hd, U, _ = O.environment(H)
    rng = np.random.default_rng(2)
    W = rng.standard_normal((m, n))
    if kind == "scalar":
        width = 1
        lv = O.lloyd_max(2)
        idx, before = O.ldlq_scalar(W, U, lv, mode=0, lazy=16, want_before=True)
        Q = lv[idx]
    else:
        width = 4
        S = O.row_scale(W)
        st, before = O.ldlq_trellis(W, U, S, tables[2], 12, 2, width=width, look=2, lazy=16, want_before=True)
        Q = tables[2][st] * S[:, None]
    for j in (1, 7, 16, 23, 39):
        j0 = j - j % width  # a block of `width` columns is settled together
        ref = _refit_exact(Hd, W, list(range(j0)), Q[:, :j0])
        assert np.abs(before[:, j] - ref[:, j]).max() < 1e-9


def test_trellis_sweep_with_diagonal_H_is_the_chained_search(tables):
    """With H = c*I the refit moves nothing, so the sweep is the chain of searches: each step's path starts from
    the previous step's last state and sees `look` further targets, as RowTrellisCode.step does (codes.py:397-404)."""
    m, n, width, look, lazy = 4, 70, 16, 8, 32
    rng = np.random.default_rng(3)
    X = rng.standard_normal((m, n))
    S = O.row_scale(X)
    _, U, _ = O.environment(np.eye(n) * 2.0)
    st = O.ldlq_trellis(X, U, S, tables[2], 12, 2, width, look, lazy)
    want = np.empty((m, n), dtype=np.int64)
    state = np.zeros(m, dtype=np.int64)
    for b0 in range(0, n, lazy):
        b1 = min(b0 + lazy, n)
        for j in range(b0, b1, width):
            w = min(width, b1 - j)
            a = min(look, n - j - w)
            p = O.viterbi(X[:, j : j + w + a] / S[:, None], tables[2], 12, 2, start=state)[:, :w]
            want[:, j : j + w] = p
            state = p[:, -1]
    assert np.array_equal(st, want)


def test_sweep_lazy_equals_eager_for_scalar():
    """The lazy run only reorders floating-point work (tests/test_grammar.py:76-91): lazy 1 (eager) and lazy 128
    settle the same levels on a well-conditioned H."""
    n, m = 60, 10
    H = _spd(n, 5)
    _, U, _ = O.environment(H)
    W = np.random.default_rng(6).standard_normal((m, n))
    lv = O.lloyd_max(3)
    a = O.ldlq_scalar(W, U, lv, mode=0, lazy=1)
    b = O.ldlq_scalar(W, U, lv, mode=0, lazy=128)
    assert (a == b).mean() > 0.99


def test_numpy_sweep_equals_the_c_sweeps(tables):
    """The generic numpy sweep (syntax.py:86-124), given the scalar projection of ldlq_words and the row-trellis step
    of RowTrellisCode, settles what the two C sweeps settle (both pinned to the reference's vectors above), dead
    columns included; its `before` columns agree to rounding."""
    n, m = 72, 8
    H = _spd(n, 11)
    H[5, :] = 0
    H[:, 5] = 0
    _, U, dead = O.environment(H)
    rng = np.random.default_rng(12)
    W = rng.standard_normal((m, n))
    S = O.row_scale(W)
    lv = O.lloyd_max(2)
    mids = (lv[1:] + lv[:-1]) / 2
    got = np.empty((m, n), dtype=np.int64)

    def scalar(j, x, T):
        i = np.searchsorted(mids, x[:, 0] / S, side="left")  # torch.bucketize, right=False
        got[:, j] = i
        return lv[i] * S

    before = O.sweep(W, U, scalar, 1, 32, dead)
    idx, before_c = O.ldlq_scalar(W, U, lv, 1, S, 32, dead, want_before=True)
    assert np.array_equal(got, idx)
    assert np.abs(before - before_c).max() < 1e-11

    width, look = 8, 4
    state = np.zeros(m, dtype=np.int64)

    def step(j, x, T):
        nonlocal state
        ahead = T[:, j + width : j + width + look]
        p = O.viterbi(np.concatenate([x, ahead], 1) / S[:, None], tables[3], 12, 3, start=state)[:, : x.shape[1]]
        got[:, j : j + x.shape[1]] = p
        state = p[:, -1]
        return tables[3][p] * S[:, None]

    O.sweep(W, U, step, width, 32, dead)
    st = O.ldlq_trellis(W, U, S, tables[3], 12, 3, width, look, 32, dead)
    assert np.array_equal(got, st)


def test_column_trellis_states_are_per_sequence_searches(tables):
    """TrellisCode's reshape (codes.py:371-378): rows s*T .. s*T+T-1 of column c are one free-start sequence."""
    T, o, w = 24, 72, 5
    X = np.random.default_rng(13).standard_normal((o, w))
    st = O.column_trellis_states(X, tables[2], 12, 2, T)
    for s in range(o // T):
        for c in range(w):
            assert np.array_equal(st[s * T : (s + 1) * T, c], O.viterbi(X[s * T : (s + 1) * T, c][None], tables[2], 12, 2)[0])


def test_column_trellis_words_without_H_is_round_to_nearest_path(tables):
    """Without H, ldlq_words with the column trellis is the search on the rotated, scaled rows; the states of each
    sequence lie on one trellis path."""
    W = np.random.default_rng(14).standard_normal((48, 16))
    st, S = O.ldlq_words_column_trellis(W, None, tables[2], 12, 2, 24, 3, 4)
    X = O.rht(48, 3) @ W @ O.rht(16, 4).T
    assert np.allclose(S, np.sqrt((X**2).mean(1)), rtol=1e-14)
    seqs = st.reshape(2, 24, 16).transpose(0, 2, 1).reshape(-1, 24)
    assert np.all((seqs[:, 1:] >> 2) == (seqs[:, :-1] & 1023))


def test_ldlq_factor_damping_and_retries():
    """ldlq_gpu.py:15-25: U^T U inverts H + d mean(diag H) I at the first d in (damp, 10 damp, 100 damp) that factors;
    a zero diagonal stays zero and counts in the mean; none factoring raises AssertionError."""
    n = 24
    H = _spd(n, 15)
    A = np.random.default_rng(16).standard_normal((n, n)) * 1e-3
    U = O.ldlq_factor(H + (A - A.T))  # the antisymmetric part is dropped
    assert np.allclose(U, np.triu(U)) and np.all(np.diag(U) > 0)
    assert np.abs(U.T @ U @ (H + 0.01 * np.mean(np.diag(H)) * np.eye(n)) - np.eye(n)).max() < 1e-10
    H0 = H.copy()
    H0[3, :] = 0
    H0[:, 3] = 0
    U0 = O.ldlq_factor(H0)
    assert np.abs(U0.T @ U0 @ (H0 + 0.01 * np.mean(np.diag(H0)) * np.eye(n)) - np.eye(n)).max() < 1e-10
    Q, _ = np.linalg.qr(np.random.default_rng(17).standard_normal((n, n)))
    lam = np.ones(n)
    lam[0] = -0.05  # mean(diag) = mean(lam) ~ 0.96: fails at d = 0.01, factors at 0.1
    Hn = Q @ np.diag(lam) @ Q.T
    Un = O.ldlq_factor(Hn)
    assert np.abs(Un.T @ Un @ (Hn + 0.1 * np.mean(lam) * np.eye(n)) - np.eye(n)).max() < 1e-9
    lam[0] = -5.0
    with pytest.raises(AssertionError):
        O.ldlq_factor(Q @ np.diag(lam) @ Q.T)


def test_ldlq_round_is_the_one_rate_nested_sweep(golden, config12):
    """ldlq_gpu.py documents ldlq_round(X/S, ldlq_factor(Hr), levels) as nested.multirate_sweep with one rate: on
    config 1 it chooses the reference's levels (nested_lm3 vectors), whatever the lazy block."""
    W, H = config12
    g = golden("nested_lm3_c1")
    R = O.rht(960, 201)
    X = W.astype(np.float64) @ R.T
    S = O.row_scale(X)
    U = O.ldlq_factor(R @ H @ R.T)
    want = g["levels"][g["idx"]]
    assert np.array_equal(O.ldlq_round(X[:64] / S[:64, None], U, g["levels"]), want[:64])
    assert (O.ldlq_round(X[:16] / S[:16, None], U, g["levels"], block=64) == want[:16]).mean() > 0.99


def test_environment_is_the_cholesky_factor_of_the_inverse():
    H = _spd(30, 7)
    H[4, :] = 0
    H[:, 4] = 0
    Hd, U, dead = O.environment(H)
    assert dead[4] and dead.sum() == 1 and Hd[4, 4] > 1.0
    assert np.allclose(U, np.triu(U)) and np.all(np.diag(U) > 0)
    assert np.abs(U.T @ U @ Hd - np.eye(30)).max() < 1e-10


# ----------------------------------------------------------------------------- tables, transforms, statistics


def test_lloyd_max_matches_max_1960_and_reference_bits(golden):
    inf = np.array([math.inf])
    for b, mse in ((1, 0.3634), (2, 0.1175), (3, 0.03455), (4, 0.009497)):  # Max (1960)
        lv = O.lloyd_max(b)
        bounds = np.concatenate([-inf, (lv[1:] + lv[:-1]) / 2, inf])
        assert abs(O.gaussian_mse(bounds, lv) - mse) < 2e-4
        assert np.abs(lv - golden("misc")[f"lloyd_max_{b}"]).max() < 1e-12
    assert np.allclose(O.lloyd_max(2), [-1.5104, -0.4528, 0.4528, 1.5104], atol=1e-4)


@pytest.mark.parametrize("n", [64, 320, 960, 2560])
def test_hadamard_orders(n, golden):
    H = O.hadamard(n)
    assert np.abs(H @ H.T - np.eye(n)).max() < 1e-10
    assert np.abs(np.abs(H) - 1 / math.sqrt(n)).max() < 1e-12
    if n in (960, 2560):
        A, B = O.hadamard_factors(n)
        assert np.array_equal(A, golden("misc")[f"had_{n}_A"]) and np.array_equal(B, golden("misc")[f"had_{n}_B"])


@pytest.mark.parametrize("n", [64, 960, 2560])
def test_rht_apply_is_the_dense_rotation(n):
    """The factored rotation equals the products with the dense R = rht(n, seed) both ways, and the two undo each
    other (a transposed factor, a missing sign or a wrong 1/sqrt(n) breaks one of these)."""
    rng = np.random.default_rng(n)
    X = rng.standard_normal((5, n))
    R = O.rht(n, 1001)
    Y = O.rht_apply(X, 1001)
    assert np.abs(Y - X @ R.T).max() < 1e-12
    assert np.abs(O.rht_apply(X, 1001, inverse=True) - X @ R).max() < 1e-12
    assert np.abs(O.rht_apply(Y, 1001, inverse=True) - X).max() < 1e-12


def test_hessian_is_the_weighted_sum_of_outer_products():
    rng = np.random.default_rng(8)
    X = rng.standard_normal((9, 5))
    w = rng.uniform(0.1, 3, 9)
    ref = sum(w[t] * np.outer(X[t], X[t]) for t in range(9)) / 9
    assert np.abs(O.hessian(X, w) - ref).max() < 1e-14


def test_kl_closed_forms():
    """KL(p || p) = 0; for two logits the KL of two Bernoulli distributions; and KL >= 0."""
    rng = np.random.default_rng(9)
    r = O.bf16_bits(rng.standard_normal((4, 300)).astype(np.float32) * 3)
    kl, mean = O.kl_rows(r, r)
    assert np.abs(kl).max() < 1e-12
    a = np.array([[0.5, -1.25], [2.0, 0.0]], dtype=np.float32)
    b = np.array([[-0.75, 0.25], [1.0, 1.5]], dtype=np.float32)
    kl, _ = O.kl_rows(O.bf16_bits(a), O.bf16_bits(b))
    for t in range(2):
        p = 1 / (1 + math.exp(-(a[t, 0] - a[t, 1])))
        q = 1 / (1 + math.exp(-(b[t, 0] - b[t, 1])))
        assert abs(kl[t] - (p * math.log(p / q) + (1 - p) * math.log((1 - p) / (1 - q)))) < 1e-12
    q = O.bf16_bits(O.bf16_to_f32(r) + rng.standard_normal(r.shape).astype(np.float32))
    kl, _ = O.kl_rows(r, q)
    assert np.all(kl > 0)


def test_kl_float_restatement_matches_the_bf16_oracle():
    """kl_rows_float (float logits) equals the C bf16 oracle on logits bf16 holds exactly, weighted mean included; on
    two logits it is the Bernoulli KL; a shift of a row's logits leaves it unchanged."""
    rng = np.random.default_rng(19)
    r = O.bf16_bits(rng.standard_normal((6, 777)).astype(np.float32) * 3)
    q = O.bf16_bits(O.bf16_to_f32(r) + rng.standard_normal(r.shape).astype(np.float32) * 0.5)
    w = rng.uniform(0.5, 2.0, 6).astype(np.float32)
    k16, m16 = O.kl_rows(r, q, w)
    kf, mf = O.kl_rows_float(O.bf16_to_f32(r), O.bf16_to_f32(q), w)
    assert np.abs(kf - k16).max() < 1e-12 * np.abs(k16).max()
    assert abs(mf - m16) < 1e-12 * abs(m16)
    a = np.array([[0.3, -1.7]], dtype=np.float32)
    b = np.array([[-0.9, 0.4]], dtype=np.float32)
    p = 1 / (1 + math.exp(-(float(a[0, 0]) - float(a[0, 1]))))
    qq = 1 / (1 + math.exp(-(float(b[0, 0]) - float(b[0, 1]))))
    kf, _ = O.kl_rows_float(a, b)
    assert abs(kf[0] - (p * math.log(p / qq) + (1 - p) * math.log((1 - p) / (1 - qq)))) < 1e-12
    x = rng.standard_normal((3, 50)).astype(np.float32)
    y = rng.standard_normal((3, 50)).astype(np.float32)
    k0, _ = O.kl_rows_float(x, y)
    k1, _ = O.kl_rows_float(x + np.float32(4.0), y - np.float32(2.0))
    assert np.abs(k0 - k1).max() < 1e-5 * np.abs(k0).max()


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_pack_trellis_matches_reference_bytes(golden, bits):
    g = golden("misc")
    st = g[f"pack_{bits}_states"].astype(np.int64)
    codes = O.pack_trellis(st, bits)
    assert np.array_equal(codes, g[f"pack_{bits}_codes"])
    assert np.array_equal(O.unpack_trellis(codes, bits, st.shape[1]), st)
    bad = st.copy()
    bad[1, 5] ^= 1 << 11
    with pytest.raises(ValueError):
        O.pack_trellis(bad, bits)


def test_ldlq_noise_oracle_invariants():
    """oracle.ldlq_noise (compiler.py:110-129): A is the upper factor of the damped rotated H; the rotated error has
    LDLQ's energy, tr(E_r H E_r^T) = sum_j A_jj^2 eta_j^2 row by row (QuIP, Theorem 1); it is causal in column order
    (column j of E_r depends only on noise columns <= j, which fixes the triangle); the rotations are orthogonal and
    undone exactly; zero noise gives W."""
    import torch

    rng = np.random.default_rng(41)
    m, n = 24, 40
    W = rng.standard_normal((m, n))
    X = rng.standard_normal((300, n)) * np.linspace(0.5, 2.0, n)
    H = X.T @ X / 300
    eta = torch.randn(m, n, generator=torch.Generator().manual_seed(5), dtype=torch.float64).numpy()
    out, Er, A = O.ldlq_noise(W, H, 0.015, 7, eta)
    Ri, Ro = O.rht(n, 8), O.rht(m, 7)
    Hr = Ri @ H @ Ri.T
    Hr = Hr + 0.01 * np.mean(np.diag(Hr)) * np.eye(n)
    assert np.allclose(np.tril(A, -1), 0) and np.all(np.diag(A) > 0)
    assert np.abs(A @ A.T - Hr).max() < 1e-12 * np.abs(Hr).max()
    Wr = Ro @ W @ Ri.T
    e = eta * np.sqrt(np.mean(Wr ** 2, axis=1, keepdims=True)) * 0.015 ** 0.5
    energy = np.einsum("ij,jk,ik->i", Er, Hr, Er)
    assert np.abs(energy - (e ** 2 * np.diag(A) ** 2).sum(1)).max() < 1e-10 * energy.max()
    eta2 = eta.copy()
    eta2[:, -1] += 1.0
    _, Er2, _ = O.ldlq_noise(W, H, 0.015, 7, eta2)
    assert np.abs(Er2[:, :-1] - Er[:, :-1]).max() < 1e-14 and np.abs(Er2[:, -1] - Er[:, -1]).min() > 0
    eta3 = eta.copy()
    eta3[:, 0] += 1.0
    _, Er3, _ = O.ldlq_noise(W, H, 0.015, 7, eta3)
    assert np.abs(Er3[:, 1:] - Er[:, 1:]).max() > 1e-6  # the first column's noise is carried into the later ones
    E = out - W
    assert np.abs(Ro @ E @ Ri.T - Er).max() < 1e-12 * np.abs(Er).max()
    back, _, _ = O.ldlq_noise(W, H, 0.0, 7, eta)
    assert np.array_equal(back, W)
    out_in, Er_in, _ = O.ldlq_noise(W, H, 0.015, 7, eta, row_rotation=False)
    assert np.abs((out_in - W) @ Ri.T - Er_in).max() < 1e-12 * np.abs(Er_in).max()


@pytest.mark.parametrize("case", ["r3", "r3_noH", "r4"])
def test_multirate_sweep_matches_the_reference(golden, case):
    """nested.py:104-147 for several rates at once: the reference's indices (tests/golden/multirate.npz: three rates of
    a 3-bit nested code with and without H, four rates of a 4-bit code with a dead input)."""
    g = golden("multirate")
    H = g[f"{case}_H"] if not case.endswith("noH") else None
    idx = O.multirate_sweep(g[f"{case}_X"], H, g[f"{case}_tables"], g[f"{case}_weights"])
    assert np.array_equal(idx, g[f"{case}_idx"])


@pytest.mark.parametrize("with_h", [True, False])
def test_shaped_sweep_with_isotropic_g_is_plain_rounding(with_h):
    """Output shaping under G = c I: the damped factor V is diagonal, every block's feedback V[a:b, a:b]^-1 V[a:b, b:]
    is zero, and each entry takes its nearest level, so the sweep is the one-rate multirate sweep's."""
    rng = np.random.default_rng(11)
    m, n = 40, 90
    X = rng.standard_normal((m, n))
    Xa = rng.standard_normal((300, n))
    H = Xa.T @ Xa / 300 if with_h else None
    lv = np.sort(rng.standard_normal(8))
    got = O.shaped_sweep(X, H, lv, 2.5 * np.eye(m), block=8)
    assert np.array_equal(got, O.multirate_sweep(X, H, lv[None], [1.0]))


@pytest.mark.parametrize("block", [1, 4, 8, 16])
def test_shaped_rows_are_the_block_sweep_of_the_column(block):
    """Within a column, output shaping settles the rows `block` at a time on their nearest levels and re-solves the
    later rows through M = V[a:b, a:b]^-1 V[a:b, b:]: the generic block sweep (width = block, the triangular solve
    z U_BB = E and T -= z U) run along the column, the rows as its columns and V as its factor. Checked against that
    sweep, written separately, on 42 rows (a partial last block for 4, 8 and 16) with a dense G."""
    rng = np.random.default_rng(20 + block)
    m = 42
    Ga = rng.standard_normal((200, m))
    G = Ga.T @ Ga / 200
    u = rng.standard_normal(m)
    lv = np.sort(rng.standard_normal(16))
    got = O.shaped_sweep(u[:, None], None, lv, G, block=block)[:, 0]
    _, V, _ = O.environment(G, damp=O.OUTPUT_DAMP)
    want = np.empty(m, dtype=np.int64)

    def nearest(j, cols, T):
        i = np.abs(cols[0][:, None] - lv[None, :]).argmin(1)
        want[j : j + len(i)] = i
        return lv[i][None, :]

    O.sweep(u[None, :], V, nearest, width=block, lazy=block * (-(-m // block)))
    assert np.array_equal(got, want)


def test_one_rate_multirate_is_the_scalar_sweep():
    """One rate at weight 1: the joint cost is the squared distance, so the sweep is ldlq_scalar's (mode 0)."""
    rng = np.random.default_rng(3)
    m, n = 20, 150
    X = rng.standard_normal((m, n))
    Xa = rng.standard_normal((300, n))
    H = Xa.T @ Xa / 300
    lv = np.sort(rng.standard_normal(8))
    _, U, _ = O.environment(H)
    assert np.array_equal(O.multirate_sweep(X, H, lv[None], [1.0]), O.ldlq_scalar(X, U, lv, 0))
