"""Fitting trellis tables (opgraph/codes.py:187-220) with the Viterbi kernel doing the searches.

The reference's cached tables (cache/codes/trellis_L12_k*_T256_s0_ema.pt, kept here as tables/*.f64) are the output
of its own e-means fit: 6,144 batches of 256 fresh Gaussian sequences drawn from torch's CPU generator. Refitting the
k = 2 table here reproduces it to within 4 units in the last place (4091 of 4096 entries exactly): one sample searched
onto another state in any of the last ~1,200 batches would move its state's value by more, so that bound holds only
if every late search agreed. The Lloyd fit is checked against the same steps computed with the C oracle's search on a
small trellis, and both fits against the reference's own properties of them (tests/test_codes.py:139-165): an e-means
table leaves under 99% of a Lloyd table's error on held-out Gaussians, and a fitted 256-state trellis beats the
2-bit Lloyd-Max scalar code by more than 0.01 in mean squared error.
"""

import sys

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("k", [2])
def test_ema_fit_reproduces_the_reference_table(k):
    from lookatmyquant_amd import fit
    from lookatmyquant_amd.tables import load_table

    say(f"e-means fit L=12 k={k} T=256 seed 0 (6144 batches)")
    v = fit.fit_table(12, k, 256, 0)
    ref = load_table(12, k)
    ulp = np.abs(v - ref) / np.spacing(np.abs(ref))
    say(f"  entries equal {int((v == ref).sum())} of {v.size}; largest difference {float(ulp.max()):.1f} ulp")
    assert ulp.max() <= 4
    assert (v == ref).mean() >= 0.995


def test_lloyd_fit_is_the_mean_of_the_searched_samples():
    """Two Lloyd steps on L = 6, k = 2, T = 16: each step the oracle's search of the same 4096 sequences, then every
    visited state at the mean of its samples (the rest keep their values), against the GPU fit."""
    from lookatmyquant_amd import fit

    L, k, T, seed = 6, 2, 16, 3
    say("lloyd fit L=6 k=2 T=16, two steps")
    got = fit.fit_table(L, k, T, seed, refine=2, fit="lloyd")
    S = 1 << L
    g = torch.Generator().manual_seed(seed)
    v = torch.special.ndtri((torch.randperm(S, generator=g).double() + 0.5) / S).numpy()
    X = torch.randn(4096, T, generator=g, dtype=torch.float64).numpy()
    for _ in range(2):
        st = O.viterbi(X, v, L, k).reshape(-1)
        sums = np.zeros(S)
        cnt = np.zeros(S)
        for s, x in zip(st, X.reshape(-1)):  # in sample order
            sums[s] += x
            cnt[s] += 1
        v = np.where(cnt > 0, sums / np.maximum(cnt, 1e-300), v)
    assert np.array_equal(got, v)


def test_trellis_values_serves_cached_tables_and_fits_others():
    from lookatmyquant_amd import codes
    from lookatmyquant_amd.tables import load_table

    assert np.array_equal(codes.trellis_values(12, 3).numpy(), load_table(12, 3))
    say("trellis_values L=8 k=2 T=32 seed 1, refine 1 (fitted)")
    v = codes.trellis_values(8, 2, T=32, seed=1, refine=1)
    assert v.shape == (256,) and v.dtype == torch.float64 and torch.isfinite(v).all()
    assert torch.equal(v, codes.trellis_values(8, 2, T=32, seed=1, refine=1))  # kept for the process


def _held_out_error(v, L, k, X):
    from lookatmyquant_amd import codes

    st = codes.viterbi(X, v, L, k).cpu()
    return (X - v[st]).square().mean().item()


def test_ema_fit_beats_lloyd_on_held_out_gaussians():
    """tests/test_codes.py:147-165: L = 8, k = 2, T = 64, refine 6, 1024 held-out sequences from seed 1."""
    from lookatmyquant_amd import codes

    L, k, T = 8, 2, 64
    X = torch.randn(1024, T, generator=torch.Generator().manual_seed(1), dtype=torch.float64)
    err = {fit: _held_out_error(codes.trellis_values(L, k, T, refine=6, fit=fit), L, k, X) for fit in ("lloyd", "ema")}
    say(f"  2-bit distortion, 256-state trellis: Lloyd {err['lloyd']:.4f}, e-means {err['ema']:.4f}")
    assert err["ema"] < 0.99 * err["lloyd"], err


def test_fitted_trellis_beats_the_scalar_code():
    """tests/test_codes.py:139-144: a 256-state trellis (k = 2, T = 320, refine 2) against Lloyd-Max at 2 bits."""
    from lookatmyquant_amd import codes

    X = torch.randn(512, 320, generator=torch.Generator().manual_seed(5), dtype=torch.float64)
    levels = torch.tensor(codes.GAUSS2.levels, dtype=torch.float64)
    scalar = (X - levels[(X[..., None] - levels).abs().argmin(-1)]).square().mean().item()
    assert abs(scalar - 0.1175) < 0.005, scalar  # the Lloyd-Max distortion of N(0, 1) at 2 bits
    tcq = _held_out_error(codes.trellis_values(8, 2, 320, refine=2), 8, 2, X)
    say(f"  2-bit distortion: scalar {scalar:.4f}, 256-state trellis {tcq:.4f}")
    assert tcq < scalar - 0.01, (scalar, tcq)
