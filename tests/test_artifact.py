"""The opgraph-packed-1 files on the host, CPU only: the reference's own artifacts (tests/golden/artifact_*, written
by compiler_artifact.export_saved_codes and write_artifact on small synthetic saved codes) are read, checked and
written again byte for byte; the planned sizes, shared tables and layout checks behave like the reference's; and the
code words the reference packed decode to the saved states. The packing itself runs on the GPU
(tests/test_gpu_api.py compares a whole export with the same files)."""

import json
import shutil

import numpy as np
import pytest
import torch

from conftest import GOLDEN

EXPORT = GOLDEN / "artifact_export"
ALIAS = GOLDEN / "artifact_alias"
RECEIPTS = json.loads((GOLDEN / "artifact_receipts.json").read_text())
STORAGE_KEYS = ("format", "blob", "blob_bytes", "tensors")


@pytest.fixture(scope="module")
def A():
    from lookatmyquant_amd import artifact

    return artifact


@pytest.fixture(scope="module")
def inputs():
    return dict(np.load(GOLDEN / "artifact_inputs.npz"))


def semantic_of(meta):
    return {k: v for k, v in meta.items() if k not in STORAGE_KEYS}


def as_written(tensors, meta):
    """The tensors as a writer receives them: BF16 entries as torch bfloat16 (the blob keeps their raw bits)."""
    out = {}
    for name, a in tensors.items():
        if meta["tensors"][name]["dtype"] == "BF16":
            out[name] = torch.from_numpy(a.copy()).view(torch.bfloat16)
        elif "alias_of" not in meta["tensors"][name]:
            out[name] = a
        else:
            out[name] = a.copy()
    return out


def same_files(a, b):
    names = sorted(p.name for p in a.iterdir())
    assert names == sorted(p.name for p in b.iterdir())
    for n in names:
        assert (a / n).read_bytes() == (b / n).read_bytes(), n


def test_reads_the_reference_artifacts(A):
    for path in (EXPORT, ALIAS):
        tensors, meta = A.read_artifact(path)
        assert meta["format"] == "opgraph-packed-1" and meta["blob"] == "weights.bin"
        assert set(tensors) == set(meta["tensors"])
        raw = (path / "artifact.json").read_bytes()
        assert A.canonical_json(meta) == raw  # the manifest is the canonical encoding of itself
        specs = {n: {"dtype": s["dtype"], "shape": s["shape"]} for n, s in meta["tensors"].items()}
        aliases = {n: s["alias_of"] for n, s in meta["tensors"].items() if "alias_of" in s}
        total = (path / "weights.bin").stat().st_size + len(raw)
        assert A.artifact_serialized_bytes(specs, semantic_of(meta), tensor_aliases=aliases) == total


def test_rewrites_the_export_byte_for_byte(A, tmp_path):
    tensors, meta = A.read_artifact(EXPORT)
    assets = {n: GOLDEN / "artifact_model" / n for n in meta["assets"]}
    receipt = A.write_artifact(tmp_path / "out", as_written(tensors, meta), semantic_of(meta), assets=assets)
    same_files(tmp_path / "out", EXPORT)
    assert {k: v for k, v in receipt.items() if k != "path"} == RECEIPTS["export"]


def test_shared_tables(A, tmp_path):
    tensors, meta = A.read_artifact(ALIAS)
    aliases = {n: s["alias_of"] for n, s in meta["tensors"].items() if "alias_of" in s}
    assert aliases == {"m.weight.g1.table": "m.weight.g0.table"}
    assert A.find_table_aliases(tensors, semantic_of(meta)) == aliases
    assert A.manifest_table_aliases(meta) == aliases
    receipt = A.write_artifact(tmp_path / "out", as_written(tensors, meta), semantic_of(meta), tensor_aliases=aliases)
    same_files(tmp_path / "out", ALIAS)
    assert {k: v for k, v in receipt.items() if k != "path"} == RECEIPTS["alias"]
    # equal bytes under another shape or storage type are not shared; different bytes under an alias are refused
    t2 = as_written(tensors, meta)
    t2["m.weight.g1.table"] = t2["m.weight.g1.table"].copy()
    t2["m.weight.g1.table"][7] += 1.0
    assert A.find_table_aliases(t2, semantic_of(meta)) == {}
    with pytest.raises(ValueError, match="table alias bytes differ"):
        A.write_artifact(tmp_path / "bad", t2, semantic_of(meta), tensor_aliases=aliases)


def test_grouped_specs_match_the_manifest(A, inputs):
    _, meta = A.read_artifact(EXPORT)
    rec = meta["matrices"]["model.layers.0.mlp.up_proj.weight"]
    specs, got = A.grouped_matrix_specs("model.layers.0.mlp.up_proj.weight", [96, 70],
                                        [{"rows": 40, "bits": 2}, {"rows": 32, "bits": 1}, {"rows": 24, "bits": 3}])
    assert got == rec
    for name, spec in specs.items():
        assert {k: meta["tensors"][name][k] for k in ("dtype", "shape", "nbytes")} == spec
    # the scalar matrix: levels as the table, no state fields
    rec = meta["matrices"]["model.layers.0.self_attn.o_proj.weight"]
    _, got = A.grouped_matrix_specs("model.layers.0.self_attn.o_proj.weight", [32, 33],
                                    [{"rows": 32, "bits": 3, "kind": "scalar", "table_entries": 8}])
    assert got == rec
    with pytest.raises(ValueError, match="groups must cover the matrix"):
        A.grouped_matrix_specs("x", [10, 4], [{"rows": 9, "bits": 2}])
    with pytest.raises(ValueError, match="empty group or unsupported width"):
        A.grouped_matrix_specs("x", [10, 4], [{"rows": 10, "bits": 9}])
    # the payload price of one group equals its tensors' bytes
    price = A.row_group_payload_bytes(40, 70, 2)
    assert price == sum(specs[f"model.layers.0.mlp.up_proj.weight.g0.{t}"]["nbytes"] for t in ("rows", "codes", "scales", "table"))


def test_reference_code_words_decode_to_the_saved_states(A, inputs):
    """The reference's packed words, unpacked by this module's readers, give back the saved states and symbols."""
    tensors, meta = A.read_artifact(EXPORT)
    states = inputs["up__states"].astype(np.int64)
    for i, bits in enumerate((2, 1, 3)):
        key = f"model.layers.0.mlp.up_proj.weight.g{i}"
        rows = tensors[key + ".rows"].astype(np.int64)
        assert np.array_equal(rows, inputs[f"up__rows{i}"])
        got = A.unpack_trellis(tensors[key + ".codes"], bits, 70)
        assert np.array_equal(got, states[rows] - 4096 * i)
    # the legacy entry: one group per table, widths inferred (2 for the even rows, 4 for the odd ones)
    gate = meta["matrices"]["model.layers.0.mlp.gate_proj.weight"]
    assert [(g["rows"], g["bits"]) for g in gate["groups"]] == [(32, 2), (32, 4)]
    key = "model.layers.0.self_attn.o_proj.weight.g0"
    assert np.array_equal(A.unpack_symbols(tensors[key + ".codes"], 3, 33), inputs["o__codes"])
    # decode_rotated: table[index] * scale row by row
    W = A.decode_rotated(tensors, meta["matrices"]["model.layers.0.mlp.up_proj.weight"])
    table = inputs["up__table"]
    ref = table[states] * inputs["up__scales"][:, None]
    assert np.array_equal(W, ref.astype(np.float32))
    # stored signs are the rotation's signs of the entry's seed
    assert np.array_equal(tensors["model.layers.0.mlp.up_proj.weight.signs"], A._input_signs(70, 1201))


def test_export_metadata(A):
    _, meta = A.read_artifact(EXPORT)
    assert meta["aliases"] == {"lm_head.weight": "model.embed_tokens.weight"}
    assert meta["dense"] == ["model.layers.0.mlp.up_proj.bias", "model.layers.0.self_attn.k_norm.weight",
                             "model.norm.weight", "model.position_ids", "model.empty"]
    assert meta["tensors"]["model.norm.weight"]["dtype"] == "BF16"
    emb = meta["matrices"]["model.embed_tokens.weight"]
    assert emb["kind"] == "table" and [sorted(b) for b in emb["buckets"]] == [["matrix", "rows"], ["dense", "rows"]]


def test_layout_errors(A, tmp_path):
    _, meta = A.read_artifact(ALIAS)
    bad = json.loads(json.dumps(meta))
    bad["tensors"]["m.weight.g1.table"]["sha256"] = "1" * 64
    with pytest.raises(ValueError, match="table alias descriptor mismatch"):
        A.validate_artifact_layout(bad)
    bad = json.loads(json.dumps(meta))
    bad["tensors"]["m.weight.g0.rows"]["offset"] += 4
    with pytest.raises(ValueError, match="invalid tensor layout"):
        A.validate_artifact_layout(bad)
    bad = json.loads(json.dumps(meta))
    bad["blob_bytes"] += 1
    with pytest.raises(ValueError, match="unaccounted artifact payload"):
        A.validate_artifact_layout(bad)
    bad = json.loads(json.dumps(meta))
    bad["tensors"]["m.weight.g0.scales"]["alias_of"] = "m.weight.g0.rows"
    with pytest.raises(ValueError, match="invalid table alias owner"):
        A.validate_artifact_layout(bad)
    bad = json.loads(json.dumps(meta))
    bad["format"] = "opgraph-packed-0"
    with pytest.raises(ValueError, match="unsupported compiler artifact"):
        A.validate_artifact_layout(bad)
    with pytest.raises(ValueError, match="semantic metadata cannot override"):
        A.artifact_manifest({}, {"blob": "x"})
    with pytest.raises(ValueError, match="table alias owner must precede its alias"):
        A.artifact_manifest({"a.table": {"dtype": "F32", "shape": [1]}, "b.table": {"dtype": "F32", "shape": [1]}},
                            {}, tensor_aliases={"a.table": "b.table"})
    with pytest.raises(ValueError, match="invalid tensor specification"):
        A.tensor_spec("F8", [1])
    with pytest.raises(FileExistsError):
        A.write_artifact(tmp_path, {}, {})
    # a damaged blob fails its checksum; a truncated one its size
    copy = tmp_path / "copy"
    shutil.copytree(ALIAS, copy)
    blob = bytearray((copy / "weights.bin").read_bytes())
    blob[100] ^= 1
    (copy / "weights.bin").write_bytes(bytes(blob))
    with pytest.raises(ValueError, match="tensor checksum mismatch"):
        A.read_artifact(copy)
    A.read_artifact(copy, verify=False)
    (copy / "weights.bin").write_bytes(bytes(blob[:-1]))
    with pytest.raises(ValueError, match="artifact blob size mismatch"):
        A.read_artifact(copy)


def test_state_aliases(A):
    e = torch.zeros(4, 3)
    dense = {"embed": e, "head": e, "other": torch.zeros(4, 3), "empty1": torch.zeros(0), "empty2": torch.zeros(0)}
    assert A.state_aliases(dense, {}) == {"head": "embed"}
    assert A.state_aliases(dense, {"head": {"buckets": []}}) == {"embed": "head"}
    with pytest.raises(ValueError, match="limited to tied embedding"):
        A.state_aliases(dense, {"head": {"states": None}})
    with pytest.raises(ValueError, match="multiple coded aliases"):
        A.state_aliases(dense, {"head": {"buckets": []}, "embed": {"buckets": []}})
