"""Writes the reference's own input/output vectors for the parts of the hot path that no closed form pins: the
tie-breaking of the trellis search, the end-to-end index arrays of ldlq_words / nested_words (fp64 order of
operations plus the float32 search), the exact bits of lloyd_max, the random signs of rht and the packed byte
layout of pack_trellis.

Runs only in the build container, where the reference is mounted read-only at /root/reference; it is never run by
the tests, smoke() or bench.py, and the reference never travels to the GPU box. The reference imports
opgraph/model.py, which reads a SmolLM2-360M config.json from the Hugging Face cache at import time only to size
its own model (none of the functions called here use those sizes); this script points HOME at a temporary
directory holding that public config so the import succeeds offline.

    python tests/golden/make_golden.py                    # rewrites tests/golden/*.npz
    python tests/golden/make_golden.py --only multirate   # rewrites tests/golden/multirate.npz alone
"""

from __future__ import annotations

import json
import os
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

REF = Path("/root/reference")
OUT = Path(__file__).resolve().parent
REPO = OUT.parents[1]
sys.path.insert(0, str(REPO))

from lookatmyquant_amd import synthetic  # noqa: E402  (numpy-only input generators)

SMOLLM2_360M = {"hidden_size": 960, "num_attention_heads": 15, "num_key_value_heads": 5, "intermediate_size": 2560,
                "num_hidden_layers": 32, "rms_norm_eps": 1e-05, "rope_theta": 100000.0, "model_type": "llama"}


def import_reference():
    home = Path(tempfile.mkdtemp(prefix="lamq_golden_home_"))
    snap = home / ".cache/huggingface/hub/models--HuggingFaceTB--SmolLM2-360M/snapshots/golden"
    snap.mkdir(parents=True)
    (snap / "config.json").write_text(json.dumps(SMOLLM2_360M))
    os.environ["HOME"] = str(home)
    os.environ["OPGRAPH_DEVICE"] = "cpu"
    sys.path.insert(0, str(REF))
    import torch
    torch.set_num_threads(8)
    from opgraph import codes as C
    from opgraph import nested as N
    import compiler_artifact as CA
    C.TRELLIS_FIT = "ema"
    C.GPU_SWEEP = False
    return torch, C, N, CA


def fp16_quantile_table(torch, L: int, seed: int = 0):
    """2^L unit-Gaussian quantiles in the order of torch.randperm(2^L, Generator(seed)), cast to float16: the
    initial table of codes.py:202-204 without refinement, the 16-bit-state table of the benchmark configurations."""
    S = 1 << L
    g = torch.Generator().manual_seed(seed)
    v = torch.special.ndtri((torch.randperm(S, generator=g).double() + 0.5) / S)
    return v.to(torch.float16).double()


def main():
    t0 = time.time()
    torch, C, N, CA = import_reference()
    rng = np.random.default_rng(7)

    # ---------------------------------------------------------------- Viterbi (codes.py:151-181)
    vit = {}
    for k in (1, 2, 3, 4):
        tab = C.trellis_values(12, k, 256, 0)
        X = rng.standard_normal((48, 24))
        start = rng.integers(0, 4096, 48)
        vit[f"L12_k{k}_x"] = X
        vit[f"L12_k{k}_start"] = start
        vit[f"L12_k{k}_free"] = C.viterbi(torch.from_numpy(X), tab, 12, k).numpy().astype(np.int32)
        vit[f"L12_k{k}_fixed"] = C.viterbi(torch.from_numpy(X), tab, 12, k, start=torch.from_numpy(start)).numpy().astype(np.int32)
    tab16 = fp16_quantile_table(torch, 16)
    X = rng.standard_normal((12, 24))
    start = rng.integers(0, 1 << 16, 12)
    vit["L16_k2_table"] = tab16.numpy()
    vit["L16_k2_x"] = X
    vit["L16_k2_start"] = start
    vit["L16_k2_fixed"] = C.viterbi(torch.from_numpy(X), tab16, 16, 2, start=torch.from_numpy(start)).numpy().astype(np.int32)
    # integer tables with many equal values: every comparison is exact, so ties decide the path
    for L, k in ((8, 2), (6, 1), (9, 3)):
        tab = torch.from_numpy(rng.integers(-3, 4, 1 << L).astype(np.float64))
        X = rng.integers(-4, 5, (32, 20)).astype(np.float64)
        vit[f"ties_L{L}_k{k}_table"] = tab.numpy()
        vit[f"ties_L{L}_k{k}_x"] = X
        vit[f"ties_L{L}_k{k}_free"] = C.viterbi(torch.from_numpy(X), tab, L, k).numpy().astype(np.int32)
        st = rng.integers(0, 1 << L, 32)
        vit[f"ties_L{L}_k{k}_start"] = st
        vit[f"ties_L{L}_k{k}_fixed"] = C.viterbi(torch.from_numpy(X), tab, L, k, start=torch.from_numpy(st)).numpy().astype(np.int32)
    np.savez_compressed(OUT / "viterbi.npz", **vit)
    print(f"viterbi cases written ({time.time() - t0:.0f}s)", flush=True)

    # ---------------------------------------------------------------- config 1/2 inputs
    W, H = synthetic.config12()
    Wt, Ht = torch.from_numpy(W.astype(np.float64)), torch.from_numpy(H)
    in_seed, seed = 201, 200  # quantize.py:1492-1493 for layer 0, self_attn.q_proj (block seed 2), no --seed-set

    # ---------------------------------------------------------------- rht signs and Hadamard factors
    misc = {}
    for n in (960, 2560, 4096, 9728):
        A, B = C.hadamard_factors(n)
        misc[f"had_{n}_A"] = A.numpy().astype(np.int8)
        misc[f"had_{n}_B"] = B.numpy().astype(np.int8)
    for n, s in ((960, 201), (2560, 1301), (9728, 3301)):
        R = C.rht(n, s)
        misc[f"signs_{n}_{s}"] = torch.sign(R[0] / C.hadamard(n)[0]).numpy().astype(np.int8)
    for b in (1, 2, 3, 4):
        misc[f"lloyd_max_{b}"] = N.lloyd_max(b).numpy()
    # pack_trellis (compiler_artifact.py:276-284) on random valid row paths from state 0
    for bits in (1, 2, 3, 4):
        m, n = 40, 77
        sym = rng.integers(0, 1 << bits, (m, n))
        st = np.zeros((m, n), dtype=np.int64)
        cur = np.zeros(m, dtype=np.int64)
        for c in range(n):
            cur = ((cur << bits) | sym[:, c]) & 4095
            st[:, c] = cur
        misc[f"pack_{bits}_states"] = st.astype(np.int16)
        misc[f"pack_{bits}_codes"] = CA.pack_trellis(st, bits)
    np.savez_compressed(OUT / "misc.npz", **misc)
    print(f"misc written ({time.time() - t0:.0f}s)", flush=True)

    # ---------------------------------------------------------------- ldlq_words, row trellis L = 12
    class Recording(C.RowTrellisCode):
        """RowTrellisCode whose steps also record the states (codes.py:397-404, step as written there)."""

        def __init__(self, L, k, values=None):
            if values is None:
                super().__init__(L, k)
            else:
                self.L, self.k, self.width, self.look = L, k, 16, 8
                self.values = values
                self.domain = C.TRELLIS(values, L, k, fixed_start=True)
                self.state = None
            self.rec = []

        def step(self, j, X, ahead):
            if j == 0:
                self.state = torch.zeros(len(X), dtype=torch.long, device=X.device)
            w = X.shape[1]
            path = C.viterbi(torch.cat([X, ahead], 1), self.values, self.L, self.k, start=self.state)[:, :w]
            self.state = path[:, -1]
            self.rec.append(path.clone())
            return self.values.to(X.device, X.dtype)[path]

    def trellis_case(rows, k, values=None, L=12):
        code = Recording(L, k, values)
        if values is not None:
            code.apply = lambda net, core, r_, c_, settled=None: net  # the value-to-state check is ambiguous here
        net = C.ldlq_words([Wt[:rows]], Ht, code, [seed], in_seed=in_seed, out_rot=False)[0]
        states = torch.cat(code.rec, 1).numpy()
        out = {"states": states.astype(np.int32), "S": net.cores["W.S"].data.numpy()}
        if values is None:
            out["what_rows"] = net.matrix(dtype=torch.float64)[:8].numpy()
            core = net.cores["W"].data
            out["values_match"] = np.array(bool(torch.equal(core, code.values[torch.from_numpy(states)])))
        return out

    t1 = time.time()
    c2 = trellis_case(960, 2)
    np.savez_compressed(OUT / "ldlq_trellis_c2_L12_k2.npz", **c2)
    print(f"config 2 L=12 k=2 written ({time.time() - t1:.0f}s)", flush=True)
    for k in (1, 3, 4):
        t1 = time.time()
        np.savez_compressed(OUT / f"ldlq_trellis_L12_k{k}_rows128.npz", **trellis_case(128, k))
        print(f"L=12 k={k} written ({time.time() - t1:.0f}s)", flush=True)
    t1 = time.time()
    c16 = trellis_case(32, 2, values=tab16, L=16)
    np.savez_compressed(OUT / "ldlq_trellis_L16_k2_rows32.npz", **c16)
    print(f"L=16 k=2 written ({time.time() - t1:.0f}s)", flush=True)

    # ---------------------------------------------------------------- nested_words lm3 (config 1)
    t1 = time.time()
    lv = N.lloyd_max(3)
    net = N.nested_words([Wt], Ht, [seed], 3, [3], 0.4, [1.0], lv, in_seed=in_seed, out_rot=False)[3][0]
    core = net.cores["W"].data
    idx = torch.searchsorted(((lv[1:] + lv[:-1]) / 2).contiguous(), core.contiguous())  # quantize.py:491-493
    np.savez_compressed(OUT / "nested_lm3_c1.npz", idx=idx.numpy().astype(np.uint8), S=net.cores["W.S"].data.numpy(),
                        what_rows=net.matrix(dtype=torch.float64)[:8].numpy(), levels=lv.numpy())
    print(f"config 1 lm3 written ({time.time() - t1:.0f}s)", flush=True)
    print(f"done in {time.time() - t0:.0f}s")


def multirate(torch, N):
    """multirate_sweep (nested.py:104-147) for several rates at once: the joint index of each entry minimises the
    weighted sum of the rates' squared errors, each rate's copy of the row keeping its own running target. Three cases
    on synthetic inputs: three rates of a 3-bit nested code with H, the same without H, and four rates of a 4-bit
    nested code with H holding a dead input."""
    t1 = time.time()
    out = {}
    rng = np.random.default_rng(31)
    cases = (("r3", 3, [1, 2, 3], [0.25, 0.5, 1.0], True, None), ("r3_noH", 3, [1, 2, 3], [0.25, 0.5, 1.0], False, None),
             ("r4", 4, [1, 2, 3, 4], [1.0, 0.5, 0.3, 0.2], True, 17))
    for name, top, rates, weights, with_h, dead in cases:
        m, n = 48, 200
        X = rng.standard_normal((m, n))
        Xa = rng.standard_normal((2 * n, n))
        if dead is not None:
            Xa[:, dead] = 0.0
        H = Xa.T @ Xa / (2 * n)
        tables = N.nested_tables(top, rates, 0.4)
        idx = N.multirate_sweep(torch.from_numpy(X), torch.from_numpy(H) if with_h else None, tables,
                                torch.tensor(weights, dtype=torch.float64))
        out[f"{name}_X"], out[f"{name}_H"] = X, H
        out[f"{name}_tables"], out[f"{name}_weights"] = tables.numpy(), np.array(weights)
        out[f"{name}_idx"] = idx.numpy().astype(np.int16)
    np.savez_compressed(OUT / "multirate.npz", **out)
    print(f"multirate written ({time.time() - t1:.0f}s)", flush=True)


if __name__ == "__main__":
    if sys.argv[1:] == ["--only", "multirate"]:
        torch_, _, N_, _ = import_reference()
        multirate(torch_, N_)
    else:
        main()
        torch_, _, N_, _ = import_reference()
        multirate(torch_, N_)
