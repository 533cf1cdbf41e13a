"""Writes the reference's own opgraph-packed-1 artifacts for small synthetic saved codes, so that the writer's files
can be compared byte for byte: the manifest's keys, order and canonical encoding, the blob's tensor order, the
sha256 fields, the packed code words, the stored signs, tied-state aliases, embedding buckets, checked assets and
shared-table aliases. The packed bit layout alone is also pinned by misc.npz; the rest of the file format is pinned
only here.

Runs only in the build container, where the reference is mounted read-only at /root/reference; it is never run by
the tests, smoke() or bench.py. compiler_artifact imports only the standard library, numpy and torch.

    python tests/golden/make_artifact_golden.py     # rewrites tests/golden/artifact_*
Outputs:
    artifact_inputs.npz            the saved entries and state tensors (arrays; how they combine is in the tests)
    artifact_model/                the model directory's asset files
    artifact_export/               export_saved_codes(saved, ..., dense_tensors, model_dir=artifact_model)
    artifact_alias/                write_artifact(..., tensor_aliases=find_table_aliases(...)) of one entry
    artifact_receipts.json         both receipts without their paths
"""

from __future__ import annotations

import json
import shutil
import sys
import tempfile
from pathlib import Path

import numpy as np

REF = Path("/root/reference")
OUT = Path(__file__).resolve().parent
sys.path.insert(0, str(OUT))
from artifact_saved import saved_and_state  # noqa: E402  (how the arrays combine, shared with the tests)


def trellis_rows(rng, rows: int, columns: int, bits: int) -> np.ndarray:
    """Random row paths from state 0: each state shifts a random symbol into the low bits of 12."""
    st = np.empty((rows, columns), dtype=np.int64)
    s = np.zeros(rows, dtype=np.int64)
    for c in range(columns):
        s = ((s << bits) | rng.integers(0, 1 << bits, rows)) & 4095
        st[:, c] = s
    return st


def inputs(seed: int = 2024) -> dict:
    """Every array the two artifacts are made of (names <matrix>__<field>)."""
    rng = np.random.default_rng(seed)
    a = {}
    # row-grouped trellis matrix with explicit row groups, n = 70 (not a multiple of 32)
    m, n = 96, 70
    perm = rng.permutation(m)
    sizes, widths = (40, 32, 24), (2, 1, 3)
    states = np.empty((m, n), dtype=np.int16)
    start = 0
    for ti, (size, bits) in enumerate(zip(sizes, widths)):
        rows = np.sort(perm[start:start + size])
        start += size
        states[rows] = trellis_rows(rng, size, n, bits) + 4096 * ti
        a[f"up__rows{ti}"] = rows
    a["up__states"] = states
    a["up__scales"] = rng.uniform(0.5, 2.0, m).astype(np.float32)
    a["up__table"] = rng.normal(size=3 * 4096).astype(np.float32)
    a["up__dense"] = rng.normal(size=(m, n)).astype(np.float32)
    # trellis matrix without row groups (the legacy form: groups and widths inferred from the paths)
    m, n = 64, 40
    states = np.empty((m, n), dtype=np.int16)
    states[0::2] = trellis_rows(rng, m // 2, n, 2)
    states[1::2] = trellis_rows(rng, m // 2, n, 4) + 4096
    a["gate__states"] = states
    a["gate__scales"] = rng.uniform(0.5, 2.0, m).astype(np.float32)
    a["gate__table"] = rng.normal(size=2 * 4096).astype(np.float32)
    a["gate__dense"] = rng.normal(size=(m, n)).astype(np.float32)
    # scalar codes over 8 levels (3 bits), n = 33
    m, n = 32, 33
    a["o__codes"] = rng.integers(0, 8, (m, n)).astype(np.uint8)
    a["o__scales"] = rng.uniform(0.5, 2.0, m).astype(np.float32)
    a["o__levels"] = np.sort(rng.normal(size=8)).astype(np.float32)
    a["o__dense"] = rng.normal(size=(m, n)).astype(np.float32)
    # embedding stored as two buckets (16 coded rows, 32 dense rows), tied to the output head
    vocab, hidden = 48, 64
    coded_rows = np.sort(rng.permutation(vocab)[:16])
    a["emb__dense"] = rng.normal(size=(vocab, hidden)).astype(np.float32)
    a["emb__rows0"] = coded_rows
    a["emb__rows1"] = np.setdiff1d(np.arange(vocab), coded_rows)
    a["emb__states"] = trellis_rows(rng, 16, hidden, 2).astype(np.int16)
    a["emb__scales"] = rng.uniform(0.5, 2.0, 16).astype(np.float32)
    a["emb__table"] = rng.normal(size=4096).astype(np.float32)
    # uncoded state in several storage types (bf16 as raw bits)
    a["norm_bf16_bits"] = (rng.normal(size=64).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    a["bias_f32"] = rng.normal(size=96).astype(np.float32)
    a["kn_f16"] = rng.normal(size=8).astype(np.float16)
    a["pos_i64"] = np.arange(10, dtype=np.int64)
    a["empty_f32"] = np.zeros(0, dtype=np.float32)
    # one entry whose first two tables are byte-identical (for shared-table aliases), n = 35
    m, n = 40, 35
    t0 = rng.normal(size=4096).astype(np.float32)
    states = np.empty((m, n), dtype=np.int16)
    states[:16] = trellis_rows(rng, 16, n, 1)
    states[16:28] = trellis_rows(rng, 12, n, 2) + 4096
    states[28:] = trellis_rows(rng, 12, n, 3) + 8192
    a["alias__states"] = states
    a["alias__scales"] = rng.uniform(0.5, 2.0, m).astype(np.float32)
    a["alias__table"] = np.concatenate([t0, t0, rng.normal(size=4096).astype(np.float32)])
    return a


MODEL_FILES = {"config.json": '{"model_type": "tiny", "hidden_size": 64}\n',
               "tokenizer.json": '{"version": "1.0", "model": {"type": "BPE"}}\n'}


def main():
    sys.path.insert(0, str(REF))
    import torch
    import compiler_artifact as CA

    a = inputs()
    np.savez_compressed(OUT / "artifact_inputs.npz", **a)
    model = OUT / "artifact_model"
    shutil.rmtree(model, ignore_errors=True)
    model.mkdir()
    for name, text in MODEL_FILES.items():
        (model / name).write_text(text)
    saved, state, alias = saved_and_state(a, torch)
    receipts = {}
    with tempfile.TemporaryDirectory() as tmp:
        r = CA.export_saved_codes(saved, Path(tmp) / "x", dense_tensors=state, model_dir=model)
        shutil.rmtree(OUT / "artifact_export", ignore_errors=True)
        shutil.copytree(Path(tmp) / "x", OUT / "artifact_export")
        receipts["export"] = {k: v for k, v in r.items() if k != "path"}
        tensors, meta = CA.encode_entry("m.weight", alias)
        semantic = {"matrices": {"m.weight": meta}}
        r = CA.write_artifact(Path(tmp) / "y", tensors, semantic, tensor_aliases=CA.find_table_aliases(tensors, semantic))
        shutil.rmtree(OUT / "artifact_alias", ignore_errors=True)
        shutil.copytree(Path(tmp) / "y", OUT / "artifact_alias")
        receipts["alias"] = {k: v for k, v in r.items() if k != "path"}
    (OUT / "artifact_receipts.json").write_text(json.dumps(receipts, indent=1, sort_keys=True) + "\n")
    print(json.dumps(receipts, indent=1))


if __name__ == "__main__":
    main()
