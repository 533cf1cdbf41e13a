"""lamq_kl_rows_noalloc, the allocation-free variant of lamq_kl_rows (its partials in a static per-device array),
called through the C ABI: the same per-token KL and sums as the entry point with a workspace, bit for bit, on two
calls in a row (the second with fewer tokens, so stale partials of the first would show), with and without token
weights; more tokens than the array holds are refused before any launch."""

import sys

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def test_kl_rows_noalloc_equals_kl_rows():
    from lookatmyquant_amd import engine as E

    assert torch.cuda.is_available()
    g = torch.Generator(device="cuda").manual_seed(77)
    V = 151936
    for T, weighted in ((48, True), (17, False)):
        ref = (torch.randn(T, V, generator=g, device="cuda") * 3.0).bfloat16()
        q = (ref.float() + 0.3 * torch.randn(T, V, generator=g, device="cuda")).bfloat16()
        w = torch.rand(T, generator=g, device="cuda") + 0.5 if weighted else None
        say(f"kl_rows_noalloc T={T} V={V} weighted={weighted}")
        kl_ws, sums_ws = E.kl_rows(ref, q, w)
        kl = torch.full((T,), float("nan"), dtype=torch.float32, device="cuda")
        sums = torch.full((2,), float("nan"), dtype=torch.float64, device="cuda")
        E.kl_rows_noalloc(ref, q, kl, sums, w)
        torch.cuda.synchronize()
        assert torch.equal(kl, kl_ws)
        assert torch.equal(sums, sums_ws)
        if not weighted:
            assert float(sums[1]) == float(T)
    with pytest.raises(ValueError, match="at most"):
        big = torch.zeros(E.KL_NOALLOC_MAX_T + 1, 8, dtype=torch.bfloat16, device="cuda")
        E.kl_rows_noalloc(big, big, torch.empty(E.KL_NOALLOC_MAX_T + 1, device="cuda"), None)
    # the C entry point refuses the size too, before any launch
    from lookatmyquant_amd._abi import lib, ptr, stream

    big = torch.zeros(E.KL_NOALLOC_MAX_T + 1, 8, dtype=torch.bfloat16, device="cuda")
    out = torch.empty(E.KL_NOALLOC_MAX_T + 1, device="cuda")
    assert lib().lamq_kl_rows_noalloc(ptr(big), ptr(big), big.shape[0], 8, 8, 8, None, ptr(out), None,
                                      stream(big.device)) == -1
