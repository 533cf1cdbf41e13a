"""GPU parity of each kernel against the reference's own vectors (tests/golden) and the CPU oracle, through the
C ABI (lookatmyquant_amd.engine wraps include/lamq.h one to one). Codes and states must be bit-exact; floating
point results meet the tolerance written in each test."""

import math
import sys

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def E():
    from lookatmyquant_amd import engine

    assert torch.cuda.is_available(), "the GPU tests need an MI355X"
    return engine


def cuda(a, dtype=None):
    a = np.ascontiguousarray(a)
    t = torch.as_tensor(a if a.flags.writeable else a.copy())
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()


# ----------------------------------------------------------------------------- Viterbi


@pytest.mark.parametrize("k", [1, 2, 3, 4])
def test_viterbi_L12_matches_reference(E, golden, tables, k):
    g = golden("viterbi")
    x = g[f"L12_k{k}_x"].astype(np.float32)
    C = cuda(tables[k].astype(np.float32))
    say(f"viterbi L=12 k={k} rows={len(x)}")
    free = E.viterbi_rows(cuda(x), C, 12, k).cpu().numpy()
    fixed = E.viterbi_rows(cuda(x), C, 12, k, start=cuda(g[f"L12_k{k}_start"], torch.int32)).cpu().numpy()
    assert np.array_equal(free, g[f"L12_k{k}_free"])
    assert np.array_equal(fixed, g[f"L12_k{k}_fixed"])


@pytest.mark.parametrize("L,k", [(8, 2), (6, 1), (9, 3)])
def test_viterbi_ties_match_reference(E, golden, L, k):
    g = golden("viterbi")
    p = f"ties_L{L}_k{k}_"
    C = cuda(g[p + "table"].astype(np.float32))
    x = cuda(g[p + "x"].astype(np.float32))
    say(f"viterbi ties L={L} k={k}")
    assert np.array_equal(E.viterbi_rows(x, C, L, k).cpu().numpy(), g[p + "free"])
    st = cuda(g[p + "start"], torch.int32)
    assert np.array_equal(E.viterbi_rows(x, C, L, k, start=st).cpu().numpy(), g[p + "fixed"])


def test_viterbi_L16_matches_reference(E, golden):
    g = golden("viterbi")
    x = cuda(g["L16_k2_x"].astype(np.float32))
    C = cuda(g["L16_k2_table"].astype(np.float32))
    say("viterbi L=16 k=2 (fp16 quantile table, with duplicate values)")
    got = E.viterbi_rows(x, C, 16, 2, start=cuda(g["L16_k2_start"], torch.int32)).cpu().numpy()
    assert np.array_equal(got, g["L16_k2_fixed"])


@pytest.mark.parametrize("L,k", [(16, 1), (16, 3), (16, 4), (15, 3), (14, 2), (13, 1)])
def test_viterbi_big_tables_match_oracle(E, L, k):
    from lookatmyquant_amd.tables import quantile_table

    tab = quantile_table(L, 0)
    rng = np.random.default_rng(L * 10 + k)
    x = rng.standard_normal((5, 24)).astype(np.float32)
    st = rng.integers(0, 1 << L, 5)
    say(f"viterbi L={L} k={k}")
    got = E.viterbi_rows(cuda(x), cuda(tab.astype(np.float32)), L, k, start=cuda(st, torch.int32)).cpu().numpy()
    assert np.array_equal(got, O.viterbi(x, tab, L, k, start=st))
    free = E.viterbi_rows(cuda(x[:2]), cuda(tab.astype(np.float32)), L, k).cpu().numpy()
    assert np.array_equal(free, O.viterbi(x[:2], tab, L, k))


@pytest.mark.parametrize("k", [1, 2, 3, 4])
def test_viterbi_L16_ties_match_oracle(E, k):
    """A 16-bit-state table of three values (every state -1, 0 or 1) and targets on and between them: path costs
    tie at every step, so every group's winner is decided by the lowest-h rule (the tournaments of k = 2, 3, 4 and the
    strict compare of k = 1), against the oracle, whose tie rule brute force pins at small L. Fixed starts over 24
    positions (back-pointers in LDS) and free starts over 40 (in the workspace)."""
    rng = np.random.default_rng(160 + k)
    tab = rng.choice([-1.0, 0.0, 1.0], 1 << 16)
    x = rng.choice([-1.0, -0.5, 0.0, 0.25, 0.5, 1.0], (4, 40)).astype(np.float32)
    st = rng.integers(0, 1 << 16, 4)
    C = cuda(tab.astype(np.float32))
    say(f"viterbi L=16 k={k}, three-valued table")
    got = E.viterbi_rows(cuda(x[:, :24]), C, 16, k, start=cuda(st, torch.int32)).cpu().numpy()
    assert np.array_equal(got, O.viterbi(x[:, :24], tab, 16, k, start=st))
    free = E.viterbi_rows(cuda(x[:2]), C, 16, k).cpu().numpy()
    assert np.array_equal(free, O.viterbi(x[:2], tab, 16, k))


@pytest.mark.parametrize("k", [2, 3, 4])
def test_ldlq_trellis_L16_ties_match_oracle(E, k):
    """The fused 16-bit-state sweep with the three-valued table (ties at every step of every search), 3 rows x 160
    columns, against the C oracle."""
    rng = np.random.default_rng(170 + k)
    m, n = 3, 160
    Xa = rng.standard_normal((400, n))
    _, U, _ = O.environment(Xa.T @ Xa / 400)
    X = rng.standard_normal((m, n))
    S = O.row_scale(X)
    tab = rng.choice([-1.0, 0.0, 1.0], 1 << 16)
    say(f"ldlq trellis L=16 k={k}, three-valued table")
    st = E.ldlq_trellis(cuda(X), cuda(S), cuda(U), cuda(tab), 16, k).cpu().numpy()
    assert np.array_equal(st, O.ldlq_trellis(X, U, S, tab, 16, k))


def test_viterbi_L16_long_paths_use_workspace(E):
    from lookatmyquant_amd.tables import quantile_table

    tab = quantile_table(16, 0)
    x = np.random.default_rng(4).standard_normal((2, 40)).astype(np.float32)
    say("viterbi L=16 k=2 T=40")
    got = E.viterbi_rows(cuda(x), cuda(tab.astype(np.float32)), 16, 2).cpu().numpy()
    assert np.array_equal(got, O.viterbi(x, tab, 16, 2))


def test_viterbi_long_paths_use_workspace(E, tables):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((6, 200)).astype(np.float32)
    say("viterbi L=12 k=2 T=200")
    got = E.viterbi_rows(cuda(x), cuda(tables[2].astype(np.float32)), 12, 2).cpu().numpy()
    assert np.array_equal(got, O.viterbi(x, tables[2], 12, 2))


@pytest.mark.parametrize("L,k", [(12, 5), (12, 6), (12, 7), (12, 8), (8, 8), (6, 5), (4, 4), (13, 2), (14, 3),
                                 (13, 6)])
def test_viterbi_wide_widths_match_oracle(E, L, k):
    """The wide search (k = 5..8, k = L, and up to 2^14 states with a float32 table fp16 cannot hold) against the C
    oracle, whose rules brute force pins at these widths on short paths: random tables and targets, 5 rows of 40
    positions from given starts and 3 free rows, also through codes.viterbi (the reference's signature); then a
    table of three values with targets on and between them, where every group's winner and the final state are
    decided by the tie rules."""
    from lookatmyquant_amd import codes as Cd

    rng = np.random.default_rng(500 + 16 * L + k)
    tab = rng.standard_normal(1 << L)
    x = rng.standard_normal((5, 40)).astype(np.float32)
    st = rng.integers(0, 1 << L, 5)
    C = cuda(tab.astype(np.float32))
    say(f"viterbi wide L={L} k={k}")
    got = E.viterbi_rows(cuda(x), C, L, k, start=cuda(st, torch.int32)).cpu().numpy()
    assert np.array_equal(got, O.viterbi(x, tab, L, k, start=st))
    free = E.viterbi_rows(cuda(x[:3]), C, L, k).cpu().numpy()
    assert np.array_equal(free, O.viterbi(x[:3], tab, L, k))
    api = Cd.viterbi(torch.from_numpy(x[:3].astype(np.float64)), torch.from_numpy(tab), L, k)
    assert np.array_equal(api.cpu().numpy(), free)
    tab3 = rng.choice([-1.0, 0.0, 1.0], 1 << L)
    x3 = rng.choice([-1.0, -0.5, 0.0, 0.25, 0.5, 1.0], (4, 30)).astype(np.float32)
    say(f"viterbi wide L={L} k={k}, three-valued table")
    got3 = E.viterbi_rows(cuda(x3), cuda(tab3.astype(np.float32)), L, k).cpu().numpy()
    assert np.array_equal(got3, O.viterbi(x3, tab3, L, k))


# ----------------------------------------------------------------------------- fp64 building blocks


@pytest.mark.parametrize("m,n,b0,b1", [(200, 300, 64, 192), (2309, 2560, 128, 256), (1800, 1571, 0, 128),
                                       (2600, 3100, 0, 384)])
def test_trailing_update_matches_oracle_order(E, m, n, b0, b1):
    """Small shapes take the 64-tile kernel, large ones (>= 256 tiles of 128) the LDS-staged 128-tile kernel; ragged
    rows included."""
    rng = np.random.default_rng(5)
    T = rng.standard_normal((m, n))
    Z = rng.standard_normal((m, b1 - b0))
    U = np.triu(rng.standard_normal((n, n)))
    say(f"trailing update m={m} n={n}")
    got = E.trailing_update(cuda(T), cuda(Z), cuda(U), b0, b1).cpu().numpy()
    ref = T.copy()
    acc = np.zeros((m, n - b1))
    for c in range(b1 - b0):  # fma chain in c order, as the oracle spells it
        acc = acc + Z[:, c : c + 1] * U[b0 + c, b1:][None, :]
    ref[:, b1:] = T[:, b1:] - acc
    assert np.array_equal(got[:, :b1], T[:, :b1])
    err = np.abs(got - ref).max() / np.abs(ref).max()
    say(f"  max relative difference {err:.3e}")
    assert err < 1e-14


@pytest.mark.parametrize("M,N,K,transb,tri", [(1500, 1700, 1700, True, 1), (1500, 1700, 1700, False, 2),
                                               (1300, 2000, 900, False, 0), (200, 300, 300, True, 1),
                                               (200, 300, 300, False, 2)])
def test_gemm_sub_triangular(E, M, N, K, transb, tri):
    """C -= A op(B) with op(B) triangular (tri 1: lower, the QEP's Z U^T; tri 2: upper, the QEP's P U): the 128-tile
    kernel skips the zero stages, the 64-tile kernel reads them; against a float64 product on the GPU."""
    g = torch.Generator(device="cuda").manual_seed(M + N + K + tri)
    C = torch.randn(M, N, generator=g, device="cuda", dtype=torch.float64)
    A = torch.randn(M, K, generator=g, device="cuda", dtype=torch.float64)
    Bm = torch.randn(N, K, generator=g, device="cuda", dtype=torch.float64) if transb else \
        torch.randn(K, N, generator=g, device="cuda", dtype=torch.float64)
    opB = Bm.T if transb else Bm
    if tri == 1:
        opB = torch.tril(opB)
    elif tri == 2:
        opB = torch.triu(opB)
    Bm = (opB.T if transb else opB).contiguous()
    ref = C - A @ opB
    say(f"gemm_sub M={M} N={N} K={K} transb={transb} tri={tri}")
    got = E.gemm_sub(C.clone(), A, Bm, transb=transb, tri=tri)
    err = ((got - ref).abs().max() / ref.abs().max()).item()
    say(f"  max relative difference {err:.3e}")
    assert err < 1e-13


@pytest.mark.parametrize("M,N,K,transb", [(2560, 384, 128, False), (300, 136, 128, True), (77, 190, 64, False),
                                           (130, 70, 64, True), (65, 66, 2, False), (200, 128, 100, True),
                                           (203, 130, 100, False), (33, 31, 16, False), (19456, 256, 128, False)])
def test_gemm_sub_short_k(E, M, N, K, transb):
    """Short products (K <= 128): with B as [k][col] (the sweep's narrow refits) on the split-K kernel (four waves, a
    quarter of the k-range each, partial tiles summed in LDS), with B as [col][k] (the factor's panels) on the 64-tile
    kernel that loads a tile's whole k-range into LDS at once: ragged M, N and K (zeros past them), against a float64
    product on the GPU; columns outside [0, N) of a wider C untouched."""
    g = torch.Generator(device="cuda").manual_seed(M + 3 * N + 7 * K)
    Cw = torch.randn(M, N + 6, generator=g, device="cuda", dtype=torch.float64)
    C = Cw[:, 2 : 2 + N]
    A = torch.randn(M, K, generator=g, device="cuda", dtype=torch.float64)
    Bm = torch.randn(N, K, generator=g, device="cuda", dtype=torch.float64) if transb else \
        torch.randn(K, N, generator=g, device="cuda", dtype=torch.float64)
    ref = Cw.clone()
    ref[:, 2 : 2 + N] -= A @ (Bm.T if transb else Bm)
    say(f"gemm_sub short k: M={M} N={N} K={K} transb={transb}")
    E.gemm_sub(C, A, Bm, transb=transb)
    err = ((Cw - ref).abs().max() / ref.abs().max()).item()
    say(f"  max relative difference {err:.3e}")
    assert err < 1e-13


@pytest.mark.parametrize("M,N,K", [(2560, 9216, 512), (2560, 1536, 512), (6144, 1536, 512), (19456, 2048, 512),
                                   (300, 1000, 136), (2560, 3584, 512), (2500, 700, 512), (77, 130, 1024),
                                   (2560, 128, 512)])
def test_gemm_sub_deep_rounds(E, M, N, K):
    """The sweep's deep products (B as [k][col], K = 512 at the config-5 and config-3 stage shapes): on the LDS-staged
    128-tile kernel where its tiles fill the CUs' slots, on the split-K kernel where they would not (fewer than 384
    tiles of 128, or 512 + under 64: 2560 x 1536, 2560 x 3584, ragged 2500 x 700 and 77 x 130 at K = 1024, the last
    run's 2560 x 128); against a float64 product on the GPU."""
    g = torch.Generator(device="cuda").manual_seed(M + 5 * N + 11 * K)
    C = torch.randn(M, N, generator=g, device="cuda", dtype=torch.float64)
    A = torch.randn(M, K, generator=g, device="cuda", dtype=torch.float64)
    Bm = torch.randn(K, N, generator=g, device="cuda", dtype=torch.float64)
    ref = C - A @ Bm
    say(f"gemm_sub deep: M={M} N={N} K={K}")
    got = E.gemm_sub(C, A, Bm)
    err = ((got - ref).abs().max() / ref.abs().max()).item()
    say(f"  max relative difference {err:.3e}")
    assert err < 1e-13


@pytest.mark.parametrize("n", [16, 64, 100, 200, 960, 2500])
def test_chol_inv_upper(E, n):
    rng = np.random.default_rng(n)
    X = rng.standard_normal((2 * n + 50, n))
    H = X.T @ X / len(X)
    if n == 100:
        H[7, :] = 0
        H[:, 7] = 0  # a dead column
    say(f"chol_inv_upper n={n}")
    Hd, U, dead, info = E.chol_inv_upper(cuda(H))
    Hd_o, U_o, dead_o = O.environment(H)
    assert int(info.item()) == 0
    assert np.array_equal(dead.cpu().numpy(), dead_o)
    assert np.allclose(Hd.cpu().numpy(), Hd_o, rtol=0, atol=1e-12 * np.abs(Hd_o).max())
    Ug = U.cpu().numpy()
    assert np.all(np.tril(Ug, -1) == 0)
    assert np.all(np.diag(Ug) > 0)
    err = np.abs(Ug - U_o).max() / np.abs(U_o).max()
    say(f"  |U - U_lapack| / |U| = {err:.3e}")
    assert err < 1e-10
    # U^T U = Hd^-1
    assert np.abs(Ug.T @ Ug @ Hd_o - np.eye(n)).max() < 1e-9


@pytest.mark.parametrize("n", [6000, 9728])
def test_chol_inv_upper_large_inverse_identity(E, n):
    """At the stage widths of the benchmark (many workgroups per 64-column step, the side stream busy with the
    inverse) U^T U must invert Hd, on two calls in a row (the result may not depend on workgroup timing)."""
    g = torch.Generator(device="cuda").manual_seed(n)
    X = torch.randn(2 * n, n, generator=g, device="cuda", dtype=torch.float64)
    H = X.T @ X / (2 * n)
    eye = torch.eye(n, device="cuda", dtype=torch.float64)
    say(f"chol_inv_upper U^T U Hd = I, n={n}")
    first = None
    for rep in range(2):
        Hd, U, _, info = E.chol_inv_upper(H, damp=0.1)
        assert int(info.item()) == 0
        err = (U.T @ (U @ Hd) - eye).abs().max().item()
        say(f"  call {rep}: |U^T U Hd - I| = {err:.3e}")
        assert err < 1e-10
        assert float(torch.tril(U, -1).abs().max()) == 0.0
        if first is None:
            first = U
        else:
            assert torch.equal(first, U)


def test_chol_inv_upper_on_two_streams(E):
    """Two factorizations enqueued on two streams (each with its own side stream for the inverse) run side by side and
    give the factors they give one after the other, bit for bit."""
    g = torch.Generator(device="cuda").manual_seed(23)
    Hs = []
    for n in (2560, 1100):
        A = torch.randn(2 * n, n, generator=g, device="cuda", dtype=torch.float64)
        Hs.append((A.T @ A / (2 * n)).contiguous())
    say("chol_inv_upper: n = 2560 and 1100, one after the other, then on two streams")
    ref = [E.chol_inv_upper(H)[1] for H in Hs]
    torch.cuda.synchronize()
    main = torch.cuda.current_stream()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for _ in range(2):
        out = []
        for H, st in zip(Hs, streams):
            st.wait_stream(main)
            with torch.cuda.stream(st):
                out.append(E.chol_inv_upper(H, raise_on_fail=False))
        for st in streams:
            main.wait_stream(st)
        torch.cuda.synchronize()
        for (Hd, U, dead, info), r in zip(out, ref):
            assert int(info.item()) == 0
            assert torch.equal(U, r)


def test_chol_inv_upper_without_a_side_stream(E):
    """lamq_chol_inv_upper (no side stream: every step on the caller's stream) and lamq_chol_inv_upper_ex with a side
    stream for the inverse give the same factor bit for bit, and the damped H the same."""
    n = 1500
    g = torch.Generator(device="cuda").manual_seed(29)
    A = torch.randn(2 * n, n, generator=g, device="cuda", dtype=torch.float64)
    H = (A.T @ A / (2 * n)).contiguous()
    say("chol_inv_upper: n = 1500 with and without a side stream")
    Hd, U, _, info = E.chol_inv_upper(H)
    lib = E._abi.lib()
    nb = lib.lamq_chol_inv_upper_workspace_size(n)
    ws = torch.empty(nb, dtype=torch.uint8, device="cuda")
    U1 = torch.empty(n, n, dtype=torch.float64, device="cuda")
    Hd1 = torch.empty(n, n, dtype=torch.float64, device="cuda")
    info1 = torch.empty(1, dtype=torch.int32, device="cuda")
    rc = lib.lamq_chol_inv_upper(H.data_ptr(), n, n, 0.01, Hd1.data_ptr(), n, U1.data_ptr(), n, None, info1.data_ptr(),
                                 ws.data_ptr(), nb, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    assert int(info.item()) == 0 and int(info1.item()) == 0
    assert torch.equal(U1, U)
    assert torch.equal(Hd1, Hd)


@pytest.mark.parametrize("n,k", [(300, 3), (300, 37), (300, 250)])
def test_chol_inv_upper_reports_a_pivot_inside_a_block(E, n, k):
    """A negative diagonal entry at H[k][k] of an otherwise diagonal H is pivot n - k of the reversed
    factorization: inside a diagonal block, at a 16-column step boundary or not, and in a padded last block."""
    H = np.diag(np.linspace(1.0, 2.0, n))
    H[k, k] = -1.0
    say(f"chol_inv_upper pivot n={n} k={k}")
    _, U, _, info = E.chol_inv_upper(cuda(H), damp=0.0, raise_on_fail=False)
    assert int(info.item()) == n - k
    assert float(U.abs().max()) == 0.0


@pytest.mark.parametrize("n", [40, 130])
def test_chol_inv_upper_reports_non_pd(E, n):
    """H[0][0] < 0 is the last pivot of the reversed factorization (the last diagonal block when n > 64): info
    names it, as LAPACK's info names the first non-positive leading minor, and U comes back zero."""
    H = np.eye(n)
    H[0, 0] = -5.0
    say(f"chol_inv_upper not positive definite, n={n}")
    _, U, _, info = E.chol_inv_upper(cuda(H), damp=0.0, raise_on_fail=False)
    assert int(info.item()) == n
    assert float(U.abs().max()) == 0.0
    with pytest.raises(E.LinAlgError):
        E.chol_inv_upper(cuda(H), damp=0.0)


# shapes: the MFMA kernel's specialised layouts (960: a = 16, b = 60; 2560: 128 x 20; 4096: 64 x 64; 9728: 64 x 152;
# 3072: 256 x 12; 5120: 256 x 20), its generic layout (7680: 128 x 60) and more rows than workgroups (1030 x 960)
@pytest.mark.parametrize("m,n,seed", [(48, 960, 201), (20, 2560, 1301), (8, 4096, 7), (4, 9728, 3301), (5, 3072, 5),
                                      (3, 5120, 9), (6, 7680, 11), (1030, 960, 17)])
def test_rht_rows(E, m, n, seed):
    rng = np.random.default_rng(n)
    W = rng.standard_normal((m, n))
    R = O.rht(n, seed)
    say(f"rht rows m={m} n={n}")
    Xg, S = E.rht_rows(cuda(W), seed, want_rms=True)
    X = W @ R.T
    assert np.abs(Xg.cpu().numpy() - X).max() < 1e-12 * np.abs(X).max()
    assert np.allclose(S.cpu().numpy(), O.row_scale(X), rtol=1e-13, atol=0)
    back = E.rht_rows(Xg, seed, inverse=True).cpu().numpy()
    assert np.abs(back - W).max() < 1e-12 * np.abs(W).max()


def test_rotate_hessian(E, config12):
    _, H = config12
    say("rotate hessian n=960")
    Hr = E.rotate_hessian(cuda(H), 201).cpu().numpy()
    R = O.rht(960, 201)
    ref = R @ H @ R.T
    assert np.abs(Hr - ref).max() < 1e-12 * np.abs(ref).max()


# ----------------------------------------------------------------------------- the sweeps


def _rotated(W, H, seed):
    R = O.rht(W.shape[1], seed)
    X = np.asarray(W, dtype=np.float64) @ R.T
    S = O.row_scale(X)
    _, U, dead = O.environment(R @ H @ R.T)
    return X, S, U, dead


def test_ldlq_trellis_block_matches_reference_config2(E, golden, tables, config12):
    """Config 2 (960 x 960, L = 12, k = 2): the sweep kernels on the oracle's U reproduce the reference states."""
    W, H = config12
    g = golden("ldlq_trellis_c2_L12_k2")
    X, S, U, dead = _rotated(W, H, 201)
    say("ldlq trellis config 2 L=12 k=2 (960 rows)")
    st = E.ldlq_trellis(cuda(X), cuda(S), cuda(U), cuda(tables[2]), 12, 2).cpu().numpy()
    agree = (st == g["states"]).mean()
    say(f"  state agreement with the reference {agree:.6f}")
    assert np.array_equal(st, g["states"])


@pytest.mark.parametrize("k", [1, 3, 4])
def test_ldlq_trellis_other_widths_match_reference(E, golden, tables, config12, k):
    W, H = config12
    g = golden(f"ldlq_trellis_L12_k{k}_rows128")
    X, S, U, dead = _rotated(W[:128], H, 201)
    say(f"ldlq trellis L=12 k={k} (128 rows)")
    st = E.ldlq_trellis(cuda(X), cuda(S), cuda(U), cuda(tables[k]), 12, k).cpu().numpy()
    assert np.array_equal(st, g["states"])


def test_ldlq_trellis_L16_matches_reference(E, golden, config12):
    """The 16-bit-state configuration (fp16 quantile table with repeated values): states of the first 32 rows of
    config 2 equal the states the reference's sweep records."""
    W, H = config12
    g = golden("ldlq_trellis_L16_k2_rows32")
    tab = golden("viterbi")["L16_k2_table"]
    X, S, U, dead = _rotated(W[:32], H, 201)
    say("ldlq trellis L=16 k=2 (32 rows)")
    st = E.ldlq_trellis(cuda(X), cuda(S), cuda(U), cuda(tab), 16, 2).cpu().numpy()
    agree = (st == g["states"]).mean()
    say(f"  state agreement with the reference {agree:.6f}")
    assert np.array_equal(st, g["states"])


@pytest.mark.parametrize("k", [1, 3, 4])
def test_ldlq_trellis_L16_other_widths_match_oracle(E, k):
    """The 16-bit-state sweep at the widths a row plan also assigns (k = 1: the minima-exchange kernel with its
    back-pointers in a workspace; k = 3, 4: the minima-exchange kernel), 3 rows x 272 columns (two lazy blocks, the
    second ragged), against the C oracle."""
    from lookatmyquant_amd.tables import quantile_table

    rng = np.random.default_rng(40 + k)
    m, n = 3, 272
    Xa = rng.standard_normal((600, n))
    _, U, _ = O.environment(Xa.T @ Xa / 600)
    X = rng.standard_normal((m, n))
    S = O.row_scale(X)
    tab = np.asarray(quantile_table(16, 0), dtype=np.float64)
    say(f"ldlq trellis L=16 k={k}, 3 x 272")
    st = E.ldlq_trellis(cuda(X), cuda(S), cuda(U), cuda(tab), 16, k).cpu().numpy()
    ref = O.ldlq_trellis(X, U, S, tab, 16, k)
    assert np.array_equal(st, ref)


@pytest.mark.parametrize("k", [1, 2])
def test_ldlq_trellis16_without_workspace_matches_oracle(E, monkeypatch, k):
    """lamq_ldlq_trellis16_block at L = 16, the entry point without a workspace, for the widths whose fused search
    otherwise keeps its back-pointers in one (k = 1: the quarter-window kernel, full path costs exchanged through
    LDS; k = 2: the back-pointers in LDS beside one buffer of group minima instead of in the workspace beside two):
    the same states as the oracle and as the workspace kernel, 3 rows x 272 columns."""
    from lookatmyquant_amd.tables import quantile_table

    assert E._abi.lib().lamq_ldlq_trellis16_block_workspace_size(3, 16, k) > 0
    rng = np.random.default_rng(40 + k)
    m, n = 3, 272
    Xa = rng.standard_normal((600, n))
    _, U, _ = O.environment(Xa.T @ Xa / 600)
    X = rng.standard_normal((m, n))
    S = O.row_scale(X)
    tab = np.asarray(quantile_table(16, 0), dtype=np.float64)
    say(f"ldlq trellis L=16 k={k}, 3 x 272, workspace kernel")
    with_ws = E.ldlq_trellis(cuda(X), cuda(S), cuda(U), cuda(tab), 16, k).cpu().numpy()
    monkeypatch.setattr(E._abi.lib(), "lamq_ldlq_trellis16_block_workspace_size", lambda *a: 0)
    say(f"ldlq trellis L=16 k={k}, 3 x 272, no workspace (lamq_ldlq_trellis16_block)")
    without = E.ldlq_trellis(cuda(X), cuda(S), cuda(U), cuda(tab), 16, k).cpu().numpy()
    ref = O.ldlq_trellis(X, U, S, tab, 16, k)
    assert np.array_equal(with_ws, ref)
    assert np.array_equal(without, ref)


@pytest.mark.parametrize("L", [12, 16])
def test_ldlq_trellis_groups_in_one_launch_equal_each_group_alone(E, tables, L):
    """lamq_ldlq_trellis16_block_groups (L = 16) and lamq_ldlq_trellis_block_groups (L = 12): every row group of a stage
    in one launch per lazy block, each workgroup taking its group's width, against each group swept on its own through
    lamq_ldlq_trellis16_block(_ws) or lamq_ldlq_trellis_block: the same states, bit for bit, for groups at k = 4, 1, 3,
    2 (at L = 16, k = 1 with its back-pointers in a workspace) in that row order, with an empty group among them;
    n = 600 (two outer runs, the look-ahead past the first taken in the kernel)."""
    from lookatmyquant_amd.tables import quantile_table

    rng = np.random.default_rng(77 + L)
    n = 600
    sizes, widths = [37, 90, 0, 65, 130], [4, 1, 2, 3, 2]
    m = sum(sizes)
    Xa = rng.standard_normal((2 * n, n))
    _, U, _ = O.environment(Xa.T @ Xa / (2 * n))
    X = rng.standard_normal((m, n))
    S = O.row_scale(X)
    tabs = {k: cuda(np.array(quantile_table(16, 0) if L == 16 else tables[k])) for k in (1, 2, 3, 4)}
    say(f"ldlq_trellis_groups L={L}: {m} rows, groups in one launch")
    merged = E.ldlq_trellis_groups(cuda(X), cuda(S), cuda(U), [(r, k, tabs[k], None) for r, k in zip(sizes, widths)],
                                   L)
    torch.cuda.synchronize()
    r0 = 0
    for r, k in zip(sizes, widths):
        if r:
            say(f"  group of {r} rows at k={k} alone")
            alone = E.ldlq_trellis(cuda(X[r0 : r0 + r]), cuda(S[r0 : r0 + r]), cuda(U), tabs[k], L, k)
            assert torch.equal(merged[r0 : r0 + r], alone), k
        r0 += r
    for i, k in ((36, 4), (37, 1), (130, 3), (200, 2)):  # one row of each width against the oracle
        assert np.array_equal(merged[i].cpu().numpy(), O.ldlq_trellis(X[[i]], U, S[[i]], tabs[k].cpu().numpy(), L, k)[0])


@pytest.mark.parametrize("L", [12, 16])
def test_ldlq_trellis_nan_row_stays_in_range(E, tables, L):
    """A row whose target is NaN (every path cost NaN from its first position on) gets states inside the table, so the
    traceback, the next search's start and any later table lookup stay in bounds: the two-pass final argmin of the
    16-bit-state searches falls back to state 0, the reference's argmin of an all-NaN row. The other rows of the same
    launch (groups at k = 1..4, one launch per lazy block at L = 16) equal the oracle's states."""
    from lookatmyquant_amd.tables import quantile_table

    rng = np.random.default_rng(91)
    n = 272
    sizes, widths = [5, 4, 4, 5], [1, 2, 3, 4]
    m = sum(sizes)
    Xa = rng.standard_normal((2 * n, n))
    _, U, _ = O.environment(Xa.T @ Xa / (2 * n))
    X = rng.standard_normal((m, n))
    S = O.row_scale(X)
    nan_rows = [1, 6, 10, 17]  # one row of each width's group
    X[nan_rows] = np.nan
    S[nan_rows] = 1.0
    tabs = {k: (np.array(quantile_table(16, 0)) if L == 16 else np.array(tables[k])) for k in widths}
    say(f"ldlq trellis L={L}: {m} rows in groups k = 1..4, rows {nan_rows} NaN")
    if L == 16:
        tab = cuda(tabs[1])
        st = E.ldlq_trellis_groups(cuda(X), cuda(S), cuda(U), [(r, k, tab, None) for r, k in zip(sizes, widths)], 16)
    else:
        parts, r0 = [], 0
        for r, k in zip(sizes, widths):
            parts.append(E.ldlq_trellis(cuda(X[r0:r0 + r]), cuda(S[r0:r0 + r]), cuda(U), cuda(tabs[k]), 12, k))
            r0 += r
        st = torch.cat(parts)
    st = st.cpu().numpy()
    assert st.min() >= 0 and st.max() < (1 << L)
    r0 = 0
    for r, k in zip(sizes, widths):
        keep = [i for i in range(r0, r0 + r) if i not in nan_rows]
        ref = O.ldlq_trellis(X[keep], U, S[keep], tabs[k], L, k)
        assert np.array_equal(st[keep], ref), k
        r0 += r


def test_ldlq_trellis_ragged_matches_oracle(E, tables):
    """n not a multiple of the lazy block or of the width, m not a multiple of anything."""
    rng = np.random.default_rng(11)
    m, n = 37, 200
    Xa = rng.standard_normal((500, n))
    H = Xa.T @ Xa / 500
    _, U, _ = O.environment(H)
    X = rng.standard_normal((m, n))
    S = O.row_scale(X)
    say("ldlq trellis ragged 37 x 200, width 12, look 5, lazy 96")
    st = E.ldlq_trellis(cuda(X), cuda(S), cuda(U), cuda(tables[3]), 12, 3, width=12, look=5, lazy=96).cpu().numpy()
    ref = O.ldlq_trellis(X, U, S, tables[3], 12, 3, width=12, look=5, lazy=96)
    assert np.array_equal(st, ref)


def test_ldlq_trellis_full_width_matches_oracle(E, tables):
    """The down stage's width (n = 9,728: 76 lazy blocks, 19 runs of trailing updates on the 128-tile kernel, the
    factor's large-n path): 64 rows swept on the GPU, two of them against the C oracle with the same U."""
    n, m = 9728, 64
    g = torch.Generator(device="cuda").manual_seed(97)
    Xa = torch.randn(2 * n, n, generator=g, device="cuda", dtype=torch.float64)
    H = Xa.T @ Xa / (2 * n)
    del Xa
    _, U, _, _ = E.chol_inv_upper(H)
    X = torch.randn(m, n, generator=g, device="cuda", dtype=torch.float64)
    Xh = X.cpu().numpy()
    S = O.row_scale(Xh)
    say("ldlq trellis 64 x 9728, L = 12, k = 2")
    st = E.ldlq_trellis(X, cuda(S), U, cuda(tables[2]), 12, 2).cpu().numpy()
    rows = [0, 37]
    ref = O.ldlq_trellis(Xh[rows], U.cpu().numpy(), S[rows], tables[2], 12, 2)
    same = (st[rows] == ref).mean()
    say(f"  states equal to the oracle's: {same:.6f}")
    assert np.array_equal(st[rows], ref)


@pytest.mark.parametrize("L", [12, 16])
def test_ldlq_trellis_groups_concurrent_equals_serial_and_oracle(E, tables, L):
    """Four row groups of different widths (and a fifth, empty one) swept together (one launch per lazy block for all
    groups) in the production schedule and with every launch in turn on one stream give the same states, bit for bit, and each group's states are the oracle's for its rows alone (n = 1,100: three outer runs, a
    ragged last lazy block)."""
    rng = np.random.default_rng(12 + L)
    n = 1100
    sizes, widths = [70, 0, 301, 129, 64], [1, 2, 2, 3, 4]
    m = sum(sizes)
    Xa = rng.standard_normal((2 * n, n))
    H = Xa.T @ Xa / (2 * n)
    _, U, _ = O.environment(H)
    X = rng.standard_normal((m, n))
    S = O.row_scale(X)
    if L == 12:
        tabs = {k: tables[k] for k in (1, 2, 3, 4)}
    else:
        from lookatmyquant_amd.tables import quantile_table

        tabs = {k: np.array(quantile_table(16, 0)) for k in (1, 2, 3, 4)}
    groups = [(r, k, cuda(tabs[k]), None) for r, k in zip(sizes, widths)]
    say(f"ldlq_trellis_groups L={L}: {m} rows in 4 groups, concurrent and serial")
    a = E.ldlq_trellis_groups(cuda(X), cuda(S), cuda(U), groups, L, concurrent=True)
    b = E.ldlq_trellis_groups(cuda(X), cuda(S), cuda(U), groups, L, concurrent=False)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    st = a.cpu().numpy()
    r0 = 0
    for r, k in zip(sizes, widths):
        if r:
            pick = [r0 + r - 1] if L == 16 else list(range(r0, r0 + min(r, 8)))
            ref = O.ldlq_trellis(X[pick], U, S[pick], tabs[k], L, k)
            assert np.array_equal(st[pick], ref), (r0, k)
        r0 += r


def test_ldlq_scalar_matches_reference_config1(E, golden, config12):
    """Config 1 (960 x 960, 3-bit Lloyd-Max, nested_words path): indices equal the reference's."""
    W, H = config12
    g = golden("nested_lm3_c1")
    X, S, U, dead = _rotated(W, H, 201)
    say("ldlq scalar config 1 lm3")
    idx = E.ldlq_scalar(cuda(X / S[:, None]), cuda(U), cuda(g["levels"]), mode=0).cpu().numpy()
    assert np.array_equal(idx, g["idx"].astype(np.int32))


def test_ldlq_scalar_bucketize_mode_matches_oracle(E):
    rng = np.random.default_rng(2)
    m, n = 50, 170
    Xa = rng.standard_normal((400, n))
    _, U, _ = O.environment(Xa.T @ Xa / 400)
    X = rng.standard_normal((m, n)) * 0.02
    S = O.row_scale(X)
    lv = np.array([-1.5104, -0.4528, 0.4528, 1.5104])
    say("ldlq scalar bucketize mode")
    idx = E.ldlq_scalar(cuda(X), cuda(U), cuda(lv), mode=1, S=cuda(S)).cpu().numpy()
    assert np.array_equal(idx, O.ldlq_scalar(X, U, lv, 1, S))


@pytest.mark.parametrize("K,m", [(2, 40), (3, 40), (5, 40), (8, 40), (16, 40), (17, 40), (40, 40), (8, 2100),
                                 (5, 4200), (40, 4200)])
def test_ldlq_scalar_level_counts_match_oracle(E, K, m):
    """The width-1 sweep at every level count the kernel specialises (K <= 2, 4, 8, 16 searched from registers by a
    tournament, more from LDS by the scan) and every workgroup size (4, 8 and 16 rows sharing the staged U block),
    both searches (mode 0: first argmin; mode 1: bucketize on midpoints), against the oracle: m rows x 300 columns
    (two full lazy blocks and a ragged one)."""
    rng = np.random.default_rng(100 + K + m)
    n = 300
    Xa = rng.standard_normal((2 * n, n))
    _, U, _ = O.environment(Xa.T @ Xa / (2 * n))
    X = rng.standard_normal((m, n))
    S = O.row_scale(X)
    lv = np.sort(rng.standard_normal(K)) * 1.5
    lv[K // 2] = lv[K // 2 - 1] if K > 3 else lv[K // 2]  # a repeated level: ties go to the lower index
    say(f"ldlq scalar K={K} m={m}")
    T0 = X / S[:, None]
    assert np.array_equal(E.ldlq_scalar(cuda(T0), cuda(U), cuda(lv), mode=0).cpu().numpy(), O.ldlq_scalar(T0, U, lv, 0))
    assert np.array_equal(E.ldlq_scalar(cuda(X), cuda(U), cuda(lv), mode=1, S=cuda(S)).cpu().numpy(),
                          O.ldlq_scalar(X, U, lv, 1, S))


@pytest.mark.parametrize("K,m,bw", [(8, 40, 128), (8, 130, 100), (4, 40, 50), (16, 40, 128)])
def test_ldlq_scalar_block_z_is_the_ieee_quotient(E, K, m, bw):
    """One lazy block of the width-1 kernel (lamq_ldlq_scalar_block, the first block, before any trailing update) through
    the C ABI: its indices are the oracle's and each refit coefficient z = (t - q) / U[j][j] is numpy's IEEE quotient
    of the oracle's pre-settlement value t (syntax.py:117-118), bit for bit, including the columns whose residual is
    exactly zero (t on a level) and a row whose values lie far outside 2^-300 .. 2^300 (the plain division's cases)."""
    import ctypes

    rng = np.random.default_rng(200 + K + m + bw)
    n = 160
    Xa = rng.standard_normal((2 * n, n))
    _, U, _ = O.environment(Xa.T @ Xa / (2 * n))
    T0 = rng.standard_normal((m, n))
    lv = np.sort(rng.standard_normal(K)) * 1.5
    T0[1, :5] = lv[K // 2]  # t on a level: a zero residual in the first column
    T0[2, [0, 3, 7]] = lv[0]
    T0[3] *= 1e95  # residuals beyond 2^300
    T0[4, 0] = 1e-310  # a subnormal column value
    idx_ref, before = O.ldlq_scalar(T0, U, lv, 0, want_before=True)
    lib = E._abi.lib()
    Tg, Ug, lvg = cuda(T0), cuda(U), cuda(lv)
    idx = torch.zeros(m, n, dtype=torch.int32, device="cuda")
    Z = torch.zeros(m, 128, dtype=torch.float64, device="cuda")
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    say(f"lamq_ldlq_scalar_block K={K} m={m} bw={bw}")
    rc = lib.lamq_ldlq_scalar_block(p(Tg), m, n, n, p(Ug), n, None, p(lvg), K, 0, 0, bw, p(idx), n, p(Z), 128,
                                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0
    torch.cuda.synchronize()
    assert np.array_equal(idx.cpu().numpy()[:, :bw], idx_ref[:, :bw])
    zr = (before[:, :bw] - lv[idx_ref[:, :bw]]) / np.diag(U)[:bw]
    zg = Z.cpu().numpy()[:, :bw]
    assert np.array_equal(zg.view(np.int64), zr.view(np.int64))


def test_end_to_end_gpu_factor_config2(E, golden, tables, config12):
    """Hessian rotation and U on the GPU too: the reference states at config 2, bit for bit."""
    W, H = config12
    g = golden("ldlq_trellis_c2_L12_k2")
    say("end to end config 2 with GPU rotation and factor")
    X, S = E.rht_rows(cuda(W.astype(np.float64)), 201, want_rms=True)
    Hr = E.rotate_hessian(cuda(H), 201)
    _, U, dead, _ = E.chol_inv_upper(Hr)
    st = E.ldlq_trellis(X, S, U, cuda(tables[2]), 12, 2, dead=dead).cpu().numpy()
    agree = (st == g["states"]).mean()
    say(f"  state agreement with the reference {agree:.6f}")
    assert agree == 1.0


# ----------------------------------------------------------------------------- statistics and KL


@pytest.mark.parametrize("N,n,weighted", [(4096, 960, None), (3000, 256, "digits"), (2048, 2560, "digits"),
                                          (2000, 264, "uniform"), (1000, 250, None), (777, 200, "digits")])
def test_hessian(E, N, n, weighted):
    """Unweighted and few-valued weights (digit tokens) take the 256-tile kernel (class by class), continuous weights
    the hi/lo kernel, n not a multiple of 8 the 128-tile kernel; ragged token counts and partial tiles included."""
    from lookatmyquant_amd import synthetic

    X = synthetic.calibration(N, n, 12, 13)
    w = None
    if weighted == "digits":
        w = synthetic.digit_weights(N, 14)
    elif weighted == "uniform":
        w = np.random.default_rng(15).uniform(0.1, 3.0, N).astype(np.float32)
    say(f"hessian N={N} n={n} weights={weighted}")
    Xb = torch.from_numpy(X).to(torch.bfloat16).cuda()
    Hg = E.hessian(Xb, None if w is None else torch.from_numpy(w).cuda()).cpu().numpy()
    ref = O.hessian(X, w)
    err = np.abs(Hg - ref).max() / np.abs(ref).max()
    say(f"  max |H - H64| / max |H64| = {err:.3e}")
    assert err < 1e-4
    assert np.array_equal(Hg, Hg.T)


def test_hessian_zero_weight_class(E):
    """Token weights with a zero class: the most frequent weight runs over all tokens and the zero-weight tokens are
    taken back out by a correction of -w0 over their rows."""
    from lookatmyquant_amd import synthetic

    N, n = 3000, 264
    X = synthetic.calibration(N, n, 31, 32)
    rng = np.random.default_rng(33)
    w = np.ones(N, np.float32)
    w[rng.random(N) < 0.2] = 0.0
    w[rng.random(N) < 0.1] = 10.0
    say("hessian with zero-weight tokens")
    Hg = E.hessian(torch.from_numpy(X).to(torch.bfloat16).cuda(), torch.from_numpy(w).cuda()).cpu().numpy()
    ref = O.hessian(X, w)
    err = np.abs(Hg - ref).max() / np.abs(ref).max()
    say(f"  max |H - H64| / max |H64| = {err:.3e}")
    assert err < 1e-4


def test_hessian_classes_that_leave_tokens_out(E):
    """Classes made without the zero class (weight_classes(w, include_zero=False)) leave the zero-weight tokens out:
    those tokens count with weight 0, not at the most frequent weight (each class then runs over its own rows)."""
    from lookatmyquant_amd import synthetic

    N, n = 3000, 264
    X = synthetic.calibration(N, n, 34, 35)
    rng = np.random.default_rng(36)
    w = np.ones(N, np.float32)
    w[rng.random(N) < 0.3] = 0.0
    w[rng.random(N) < 0.1] = 4.0
    wg = torch.from_numpy(w).cuda()
    classes = E.weight_classes(wg, include_zero=False)
    assert sum(r.numel() for _, r in classes) < N
    say("hessian with classes that leave the zero-weight tokens out")
    H = torch.zeros(n, n, dtype=torch.float32, device="cuda")
    E.hessian_accum(H, torch.from_numpy(X).to(torch.bfloat16).cuda(), wg, classes=classes)
    Hg = E.hessian_finalize(H, float(N)).cpu().numpy()
    ref = O.hessian(X, w)
    err = np.abs(Hg - ref).max() / np.abs(ref).max()
    say(f"  max |H - H64| / max |H64| = {err:.3e}")
    assert err < 1e-4


@pytest.mark.parametrize("N,n,weighted", [(16384, 6000, True), (4096, 9728, False)])
def test_hessian_large_against_float32(E, N, n, weighted):
    """The 256-tile kernel at the widths of the benchmark (hundreds of tiles, workgroups renumbered XCD by XCD):
    against a float32 product of the same bf16 activations on the GPU."""
    g = torch.Generator(device="cuda").manual_seed(n)
    X = torch.randn(N, n, generator=g, device="cuda").bfloat16()
    w = None
    if weighted:
        w = torch.ones(N, device="cuda")
        w[torch.rand(N, generator=g, device="cuda") < 0.1] = 10.0
    say(f"hessian N={N} n={n} against float32")
    H = E.hessian(X, w)
    Xf = X.float()
    ref = (Xf.T @ (Xf * (w[:, None] if w is not None else 1.0))) / N
    err = ((H.float() - ref).abs().max() / ref.abs().max()).item()
    say(f"  max |H - ref| / max |ref| = {err:.3e}")
    assert err < 1e-4


@pytest.mark.parametrize("n", [2560, 9728])
def test_gram_kernels_repeat_bit_for_bit_under_load(E, n):
    """The Gram kernels at the config-5 statistics' size (65,536 tokens with digit weights, so the 256-tile kernel
    class by class; hundreds of tiles keep every CU's LDS busy): H and the cross-Gram four times over from the same
    inputs, bit for bit equal, and H within 1e-4 of a float32 product. The kernels reduce in a fixed order, so a
    repeat that differs is a fragment read that took a wrong LDS address under contention (the paired transposing
    reads' asm once let the first read's destination share the second's address register: runs then differed now
    and then, only at full size)."""
    from lookatmyquant_amd import synthetic

    N = 65536
    g = torch.Generator(device="cuda").manual_seed(n + 7)
    X = torch.randn(N, n, generator=g, device="cuda").bfloat16()
    Xq = (X.float() + 0.05 * torch.randn(N, n, generator=g, device="cuda")).bfloat16()
    w = torch.from_numpy(synthetic.digit_weights(N, 41)).cuda()
    say(f"gram kernels repeated: N={N} n={n}")
    H0 = E.hessian(X, w)
    D0 = E.cross_gram_accum(torch.zeros(n, n, dtype=torch.float32, device="cuda"), X, Xq, w, scale=1.0 / N)
    for rep in range(3):
        assert torch.equal(E.hessian(X, w), H0), f"hessian repeat {rep}"
        D = E.cross_gram_accum(torch.zeros(n, n, dtype=torch.float32, device="cuda"), X, Xq, w, scale=1.0 / N)
        assert torch.equal(D, D0), f"cross-Gram repeat {rep}"
    rows = torch.arange(0, n, max(1, n // 64), device="cuda")
    Xf = X.float()
    ref = (Xf[:, rows].T @ (Xf * w[:, None])) / N
    err = ((H0[rows].float() - ref).abs().max() / ref.abs().max()).item()
    say(f"  max |H - ref| / max |ref| over {rows.numel()} rows = {err:.3e}")
    assert err < 1e-4


def test_hessian_accum_rows(E):
    """lamq_hessian_accum_rows over a row list (repeats allowed, ragged count): scale * sum over the listed rows."""
    from lookatmyquant_amd import synthetic

    N, n = 3000, 520
    X = synthetic.calibration(N, n, 16, 17)
    rows = np.random.default_rng(18).integers(0, N, 1111).astype(np.int32)
    say("hessian_accum_rows")
    Xb = torch.from_numpy(X).to(torch.bfloat16).cuda()
    H = torch.zeros(n, n, dtype=torch.float32, device="cuda")
    rg = torch.from_numpy(rows).cuda()
    nbytes = E.lib().lamq_gram_workspace_size(len(rows), n, 1)
    ws = E.workspace(nbytes, Xb.device)
    E.check(E.lib().lamq_hessian_accum_rows(E.ptr(Xb), E.ptr(rg), len(rows), n, n, 0.5, E.ptr(H), n, E.ptr(ws), nbytes,
                                            E.stream(Xb.device)), "hessian_accum_rows")
    Hg = np.tril(H.cpu().numpy())
    ref = np.tril(0.5 * O.hessian(X[rows]) * len(rows))
    assert np.abs(Hg - ref).max() < 1e-5 * np.abs(ref).max()


@pytest.mark.parametrize("N,n,weighted", [(2500, 192, "digits"), (1500, 320, "uniform"), (900, 264, None)])
def test_cross_gram(E, N, n, weighted):
    from lookatmyquant_amd import synthetic

    Xr = synthetic.calibration(N, n, 21, 22)
    Xq = synthetic.bf16_round(Xr + 0.05 * np.random.default_rng(23).standard_normal(Xr.shape).astype(np.float32))
    if weighted == "digits":
        w = synthetic.digit_weights(N, 24)
    elif weighted == "uniform":
        w = np.random.default_rng(25).uniform(0.1, 3.0, N).astype(np.float32)
    else:
        w = np.ones(N, dtype=np.float32)
    say(f"cross gram N={N} n={n} weights={weighted}")
    D = torch.zeros(n, n, dtype=torch.float32, device="cuda")
    E.cross_gram_accum(D, torch.from_numpy(Xr).to(torch.bfloat16).cuda(), torch.from_numpy(Xq).to(torch.bfloat16).cuda(),
                       None if weighted is None else torch.from_numpy(w).cuda(), scale=1.0 / N)
    ref = O.cross_gram(Xr, Xq, w)
    err = np.abs(D.cpu().numpy() - ref).max() / np.abs(ref).max()
    assert err < 1e-4


@pytest.mark.parametrize("T,V", [(64, 151936), (33, 1000), (5, 77)])
def test_kl_rows(E, T, V):
    from lookatmyquant_amd import synthetic

    r, q = synthetic.logits(T, V, 401 + V, 402 + V)
    w = np.random.default_rng(V).uniform(0.5, 2.0, T).astype(np.float32)
    say(f"kl T={T} V={V}")
    kl, sums = E.kl_rows(cuda(r.view(np.int16)).view(torch.bfloat16), cuda(q.view(np.int16)).view(torch.bfloat16),
                         torch.from_numpy(w).cuda())
    ref, mean = O.kl_rows(r, q, w)
    kl = kl.cpu().numpy().astype(np.float64)
    # per token: float32 chunk sums against the float64 oracle
    err = (np.abs(kl - ref) / np.abs(ref)).max()
    say(f"  largest per-token relative KL error {err:.3e}")
    assert np.all(np.abs(kl - ref) <= 1e-4 * np.abs(ref) + 1e-9)
    s = sums.cpu().numpy()
    assert abs(s[0] / s[1] - mean) < 1e-4 * abs(mean)


@pytest.mark.parametrize("T,V", [(33, 1000), (7, 777), (64, 151936)])
def test_kl_rows_float32_logits(E, T, V):
    """lamq_kl_rows_f32: on logits bf16 holds exactly, the bf16 kernel's results bit for bit (the same float32
    arithmetic in the same order, both vector loads at V = 1,000 and 151,936, both scalar at 777); on general float32
    logits, and through a padded row stride, within 1e-4 of the float oracle."""
    from lookatmyquant_amd import synthetic

    r, q = synthetic.logits(T, V, 501 + V, 502 + V)
    w = torch.from_numpy(np.random.default_rng(V).uniform(0.5, 2.0, T).astype(np.float32)).cuda()
    rb, qb = cuda(r.view(np.int16)).view(torch.bfloat16), cuda(q.view(np.int16)).view(torch.bfloat16)
    say(f"kl float32 T={T} V={V}")
    kb, sb = E.kl_rows(rb, qb, w)
    kf, sf = E.kl_rows(rb.float(), qb.float(), w)
    assert torch.equal(kb, kf) and torch.equal(sb, sf)
    g = torch.Generator(device="cuda").manual_seed(V)
    rf = torch.randn(T, V, generator=g, device="cuda") * 3.0
    qf = rf + 0.3 * torch.randn(T, V, generator=g, device="cuda")
    for pad in (0, 3):
        if pad:
            rp = torch.zeros(T, V + pad, device="cuda")
            qp = torch.zeros(T, V + pad, device="cuda")
            rp[:, :V], qp[:, :V] = rf, qf
            a, b = rp[:, :V], qp[:, :V]
        else:
            a, b = rf, qf
        kl, sums = E.kl_rows(a, b, w)
        ref, mean = O.kl_rows_float(rf.cpu().numpy(), qf.cpu().numpy(), w.cpu().numpy())
        k64 = kl.cpu().numpy().astype(np.float64)
        assert np.all(np.abs(k64 - ref) <= 1e-4 * np.abs(ref) + 1e-9), pad
        s = sums.cpu().numpy()
        assert abs(s[0] / s[1] - mean) < 1e-4 * abs(mean)
    with pytest.raises(ValueError):
        E.kl_rows(rf, qf.bfloat16())


def test_compiler_kl_takes_any_float_logits():
    """compiler.kl and kl_per_token take float16, float32 and mixed logits as the reference's .logits.float() does:
    the float32 results of the cast tensors, exactly."""
    from lookatmyquant_amd import compiler

    g = torch.Generator(device="cuda").manual_seed(5)
    r = (torch.randn(2, 3, 500, generator=g, device="cuda") * 3.0).half()
    q = (r.float() + 0.3 * torch.randn(2, 3, 500, generator=g, device="cuda")).half()
    ref = compiler.kl_per_token(r.float(), q.float())
    assert ref.shape == (2, 3)
    assert torch.equal(compiler.kl_per_token(r, q), ref)
    assert torch.equal(compiler.kl_per_token(r.float(), q), ref)
    assert compiler.kl(r, q) == compiler.kl(r.float(), q.float())
    rb, qb = r.bfloat16(), q.bfloat16()
    assert torch.equal(compiler.kl_per_token(rb, qb.float()), compiler.kl_per_token(rb, qb))


def test_kl_rows_config4_full_size(E):
    """Config 4's shape, [8192, 151936] bf16 logit pairs with token weights: the launch's fixed-order sums over all
    8,192 tokens equal the float64 sums of its own per-token values, and 64 sampled tokens equal the oracle's KL."""
    T, V = 8192, 151936
    g1 = torch.Generator(device="cuda").manual_seed(401)
    g2 = torch.Generator(device="cuda").manual_seed(402)
    ref = (torch.randn(T, V, generator=g1, device="cuda") * 3.0).bfloat16()
    q = (ref.float() + 0.3 * torch.randn(T, V, generator=g2, device="cuda")).bfloat16()
    w = torch.rand(T, generator=g1, device="cuda") * 1.5 + 0.5
    say(f"kl T={T} V={V} (config 4), weighted")
    kl, sums = E.kl_rows(ref, q, w)
    k64 = kl.double().cpu().numpy()
    w64 = w.double().cpu().numpy()
    s = sums.double().cpu().numpy()
    assert abs(s[0] - (w64 * k64).sum()) <= 1e-5 * abs(s[0])
    assert abs(s[1] - w64.sum()) <= 1e-5 * abs(s[1])
    pick = np.sort(np.random.default_rng(4).choice(T, 64, replace=False))
    idx = torch.as_tensor(pick, device="cuda")
    r16 = ref[idx].view(torch.int16).cpu().numpy().view(np.uint16)
    q16 = q[idx].view(torch.int16).cpu().numpy().view(np.uint16)
    ref_kl, _ = O.kl_rows(r16, q16, None)
    err = (np.abs(k64[pick] - ref_kl) / np.abs(ref_kl)).max()
    say(f"  sampled tokens: largest relative KL error {err:.3e}; mean KL {s[0] / s[1]:.5f}")
    assert np.all(np.abs(k64[pick] - ref_kl) <= 1e-4 * np.abs(ref_kl) + 1e-9)


def test_pack_trellis_matches_reference(E, golden):
    g = golden("misc")
    for bits in (1, 2, 3, 4):
        st = g[f"pack_{bits}_states"].astype(np.int32)
        say(f"pack bits={bits}")
        codes = E.pack_trellis(cuda(st), bits).cpu().numpy().view(np.uint32)
        assert np.array_equal(codes, g[f"pack_{bits}_codes"])
    bad = g["pack_2_states"].astype(np.int32).copy()
    bad[3, 10] ^= 0x100
    with pytest.raises(ValueError):
        E.pack_trellis(cuda(bad), 2)
