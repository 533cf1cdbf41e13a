"""Packed codes out: the opgraph-packed-1 compiler artifact (compiler_artifact.py of the reference).

An artifact is a directory with two files (compiler_artifact.py:491-531):
  artifact.json  the manifest, canonical JSON (sorted keys, compact separators, no NaN, UTF-8, one newline);
  weights.bin    the bytes of every physical tensor, C order and little-endian, concatenated in the sorted order
                 of the tensor names with no padding.
The manifest holds "format": "opgraph-packed-1", "blob": "weights.bin", "blob_bytes" and "tensors": name ->
{dtype, shape, nbytes, offset, sha256} (+ "alias_of" for a codebook table stored once under an earlier name), and
the caller's semantic metadata next to them. A row-grouped matrix `name` of shape [rows, n] stores
(compiler_artifact.py:143-167)
  name.signs        I8  [n]                      the input rotation's signs
  name.g{i}.rows    U32 [m]                      the original row ids of group i
  name.g{i}.codes   U32 [m, ceil(n/32) * k]      the group's symbols, k bits each, packed
  name.g{i}.scales  F32 [m]
  name.g{i}.table   F32 [4096] (trellis) | [2^k] (scalar levels)
and its metadata record {"kind": "grouped", "shape", "signs", "groups": [{key, kind, bits, rows, columns,
padded_columns[, state_bits, start_state]}]}.

The code words are made on the GPU (lamq_pack_codes: each group's rows read in place from the matrix's code
array, with the table offset, the path and the range checks of encode_entry). Hashing, file IO and the manifest are
host work; sha256 runs over the tensors on a thread pool (hashlib releases the GIL on large buffers). The readers
(unpack_symbols, unpack_trellis, decode_rotated, read_artifact) are host numpy, as a consumer of the format has them.
"""

from __future__ import annotations

import concurrent.futures as cf
import hashlib
import json
import math
import os
import shutil
from pathlib import Path

import numpy as np
import torch

from . import engine as E
from .hadamard import rht_signs

FORMAT = "opgraph-packed-1"
BLOB = "weights.bin"
MANIFEST = "artifact.json"
STATE_BITS = 12
TABLE_ENTRIES = 1 << STATE_BITS
# the format's storage types: numpy dtype and bytes per element (BF16 is stored as its raw 16 bits)
_STORAGE = {"F64": ("<f8", 8), "F32": ("<f4", 4), "F16": ("<f2", 2), "BF16": ("<u2", 2), "U32": ("<u4", 4),
            "I32": ("<i4", 4), "I64": ("<i8", 8), "I16": ("<i2", 2), "U16": ("<u2", 2), "I8": ("i1", 1),
            "U8": ("u1", 1), "BOOL": ("?", 1)}
DTYPE_BYTES = {k: v[1] for k, v in _STORAGE.items()}
NP_DTYPES = {k: v[0] for k, v in _STORAGE.items()}
# numpy dtype -> storage type name (uint16 is U16; BF16 only comes from a torch bfloat16 tensor)
_FROM_NP = {np.dtype(v[0]): k for k, v in _STORAGE.items() if k != "BF16"}
_RESERVED = ("format", "blob", "blob_bytes", "tensors")
_ASSETS = ("config.json", "generation_config.json", "tokenizer.json", "tokenizer_config.json", "special_tokens_map.json",
           "chat_template.jinja", "tokenizer.model")


def _pool():
    return cf.ThreadPoolExecutor(max_workers=max(1, min(8, os.cpu_count() or 1)))


# ----------------------------------------------------------------------------- manifest (compiler_artifact.py:29-167)


def row_group_payload_bytes(rows, columns, bits, *, scale_bytes=4, table_entries=TABLE_ENTRIES, include_rows=True):
    """Payload bytes of one row group: codes, scales, row ids and its table (the matrix's signs are counted once
    per matrix, elsewhere) (compiler_artifact.py:29-33)."""
    if rows < 0 or columns < 1 or not 1 <= bits <= 8 or scale_bytes not in (2, 4, 8):
        raise ValueError("invalid row-group shape or precision")
    per_row = (columns + 31) // 32 * bits * 4 + scale_bytes + (4 if include_rows else 0)
    return rows * per_row + 4 * table_entries


def canonical_json(value) -> bytes:
    text = json.dumps(value, sort_keys=True, separators=(",", ":"), ensure_ascii=False, allow_nan=False)
    return (text + "\n").encode()


def file_sha256(path) -> str:
    h = hashlib.sha256()
    with Path(path).open("rb") as f:
        while True:
            block = f.read(8 << 20)
            if not block:
                return h.hexdigest()
            h.update(block)


def tensor_spec(dtype: str, shape) -> dict:
    dims = [int(d) for d in shape]
    if dtype not in DTYPE_BYTES or min(dims, default=0) < 0:
        raise ValueError("invalid tensor specification")
    return {"dtype": dtype, "shape": dims, "nbytes": math.prod(dims) * DTYPE_BYTES[dtype]}


def table_tensor_names(semantic: dict) -> set:
    """The codebook tensors the matrices' groups name, embedding buckets included (compiler_artifact.py:55-69)."""
    found = set()
    stack = list(semantic.get("matrices", {}).values())
    while stack:
        mat = stack.pop()
        if mat.get("kind") == "grouped":
            found.update(g["key"] + ".table" for g in mat["groups"])
        elif mat.get("kind") == "table":
            stack.extend(b["matrix"] for b in mat["buckets"] if "matrix" in b)
    return found


def _is_digest(d) -> bool:
    return isinstance(d, str) and len(d) == 64 and all(c in "0123456789abcdef" for c in d)


def validate_artifact_layout(meta: dict) -> dict:
    """name -> physical owner (itself, or the table it aliases), after checking the whole layout
    (compiler_artifact.py:72-109): every descriptor agrees with its dtype and shape and carries a sha256; an alias
    names a table whose owner is an earlier non-alias table with the same descriptor; the owners' payloads tile
    [0, blob_bytes) once, in name order."""
    if meta.get("format") != FORMAT or meta.get("blob") != BLOB:
        raise ValueError("unsupported compiler artifact")
    if type(meta.get("blob_bytes")) is not int or meta["blob_bytes"] < 0:
        raise ValueError("invalid blob size")
    tensors = meta["tensors"]
    tables = table_tensor_names(meta)
    owners, end = {}, 0
    for name in sorted(tensors):
        spec = tensors[name]
        if (tensor_spec(spec["dtype"], spec["shape"])["nbytes"] != spec["nbytes"] or type(spec["offset"]) is not int
                or not _is_digest(spec.get("sha256"))):
            raise ValueError(f"invalid tensor layout: {name}")
        if "alias_of" not in spec:
            if spec["offset"] != end:
                raise ValueError(f"invalid tensor layout: {name}")
            owners[name] = name
            end += spec["nbytes"]
            continue
        owner = spec["alias_of"]
        if not (isinstance(owner, str) and name in tables and owner in tables and owners.get(owner) == owner):
            raise ValueError(f"invalid table alias owner: {name}")
        if any(spec[f] != tensors[owner][f] for f in ("dtype", "shape", "nbytes", "sha256", "offset")):
            raise ValueError(f"table alias descriptor mismatch: {name}")
        owners[name] = owner
    if end != meta["blob_bytes"]:
        raise ValueError("unaccounted artifact payload")
    return owners


def artifact_manifest(specs: dict, semantic: dict, *, tensor_aliases: dict | None = None) -> dict:
    """The manifest of tensors `specs` (name -> {dtype, shape}) before any payload exists: offsets in name order,
    sha256 fields as 64 zeros (a hash has a fixed length, so the manifest's size is already exact)
    (compiler_artifact.py:112-134)."""
    if set(semantic) & set(_RESERVED):
        raise ValueError("semantic metadata cannot override the storage contract")
    aliases = dict(tensor_aliases or {})
    if not set(aliases) <= set(specs):
        raise ValueError("unknown table alias name")
    if not all(isinstance(o, str) for o in aliases.values()):
        raise ValueError("invalid table alias owner")
    tensors, offset = {}, 0
    for name in sorted(specs):
        spec = tensor_spec(specs[name]["dtype"], specs[name]["shape"])
        owner = aliases.get(name)
        if owner is None:
            tensors[name] = {**spec, "offset": offset, "sha256": "0" * 64}
            offset += spec["nbytes"]
        elif owner in tensors:
            tensors[name] = {**spec, "offset": tensors[owner]["offset"], "sha256": "0" * 64, "alias_of": owner}
        else:
            raise ValueError(f"table alias owner must precede its alias: {name}")
    meta = {"format": FORMAT, "blob": BLOB, "blob_bytes": offset, "tensors": tensors, **semantic}
    validate_artifact_layout(meta)
    return meta


def artifact_serialized_bytes(specs: dict, semantic: dict, *, tensor_aliases: dict | None = None) -> int:
    """Bytes of artifact.json + weights.bin (compiler_artifact.py:137-140)."""
    meta = artifact_manifest(specs, semantic, tensor_aliases=tensor_aliases)
    return meta["blob_bytes"] + len(canonical_json(meta))


def grouped_matrix_specs(name: str, shape, groups, *, state_bits: int = STATE_BITS):
    """(tensor specs, matrix record) of a row-grouped matrix from its group descriptors {rows, bits[, kind,
    table_entries]}, nothing allocated (compiler_artifact.py:143-167)."""
    rows, columns = (int(d) for d in shape)
    if sum(int(g["rows"]) for g in groups) != rows:
        raise ValueError("groups must cover the matrix")
    words = (columns + 31) // 32
    specs = {name + ".signs": tensor_spec("I8", [columns])}
    records = []
    for i, g in enumerate(groups):
        m, bits = int(g["rows"]), int(g["bits"])
        if m <= 0 or not 1 <= bits <= 8:
            raise ValueError("empty group or unsupported width")
        kind = g.get("kind", "trellis")
        entries = int(g.get("table_entries", 1 << (state_bits if kind == "trellis" else bits)))
        key = f"{name}.g{i}"
        specs[key + ".rows"] = tensor_spec("U32", [m])
        specs[key + ".codes"] = tensor_spec("U32", [m, words * bits])
        specs[key + ".scales"] = tensor_spec("F32", [m])
        specs[key + ".table"] = tensor_spec("F32", [entries])
        rec = {"key": key, "kind": kind, "bits": bits, "rows": m, "columns": columns, "padded_columns": words * 32}
        if kind == "trellis":
            rec.update(state_bits=state_bits, start_state=0)
        records.append(rec)
    return specs, {"kind": "grouped", "shape": [rows, columns], "signs": name + ".signs", "groups": records}


# ----------------------------------------------------------------------------- storage of values


def _host(value) -> np.ndarray:
    if isinstance(value, torch.Tensor):
        return value.detach().cpu().numpy()
    return np.asarray(value)


def _typed_array(value):
    """(C-contiguous little-endian numpy array, storage type name) of a tensor or array."""
    if isinstance(value, torch.Tensor) and value.dtype == torch.bfloat16:
        return value.detach().cpu().contiguous().view(torch.uint16).numpy(), "BF16"
    a = _host(value)
    code = _FROM_NP.get(a.dtype)
    if code is None:
        raise ValueError(f"unsupported storage dtype {a.dtype}")
    return np.ascontiguousarray(a.astype(NP_DTYPES[code], copy=False)), code


def _bytes_of(a: np.ndarray) -> memoryview:
    """The array's bytes, C order, without a copy (a is C-contiguous)."""
    return memoryview(a.reshape(-1).view(np.uint8))


def _storage_identity(value):
    """What makes two state entries the same stored tensor (never merely equal values)."""
    if isinstance(value, torch.Tensor):
        return ("torch", str(value.device), str(value.dtype), value.untyped_storage().data_ptr(), value.storage_offset(),
                tuple(value.shape), tuple(value.stride()))
    a = np.asarray(value)
    return ("numpy", a.dtype.str, a.__array_interface__["data"][0], tuple(a.shape), tuple(a.strides))


def state_aliases(dense_tensors: dict, coded: dict) -> dict:
    """alias name -> anchor name for state entries that are one stored tensor (tied weights); a coded entry is the
    anchor if there is one, so a tied head is not stored dense as well (compiler_artifact.py:204-222)."""
    same: dict = {}
    for name, value in dense_tensors.items():
        if math.prod(value.shape):  # empty tensors share ambiguous pointers and cost nothing
            same.setdefault(_storage_identity(value), []).append(name)
    aliases = {}
    for names in same.values():
        if len(names) < 2:
            continue
        anchors = [nm for nm in names if nm in coded]
        if len(anchors) > 1:
            raise ValueError("multiple coded aliases require an explicit untied selected state")
        if anchors and "buckets" not in coded[anchors[0]]:
            raise ValueError("packed alias support is currently limited to tied embedding/output tables")
        anchor = anchors[0] if anchors else min(names)
        aliases.update((nm, anchor) for nm in names if nm != anchor)
    return aliases


# ----------------------------------------------------------------------------- code words (compiler_artifact.py:225-297)


def _on_device(values, what: str) -> torch.Tensor:
    """An integer array or tensor on the GPU, in its own dtype (unsigned types widened to int64: an entry beyond
    int64 turns negative there and fails every range check)."""
    t = values if isinstance(values, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(np.asarray(values)))
    if t.dtype.is_floating_point or t.dtype.is_complex or t.dtype == torch.bool:
        raise ValueError(what)
    if t.dtype in (torch.uint16, torch.uint32, torch.uint64):
        t = t.to(torch.int64)
    return t.to(E._abi.device())


def _int32_in_range(t: torch.Tensor, limit: int, what: str) -> torch.Tensor:
    """t (integers on the GPU) as a contiguous int32 tensor, after checking in its own dtype that every entry lies
    in [0, limit), so that no value can wrap into range."""
    if t.numel() and (int(t.min()) < 0 or int(t.max()) >= limit):
        raise ValueError(what)
    return t.to(torch.int32).contiguous()


def _device_codes(values, limit: int, what: str) -> torch.Tensor:
    return _int32_in_range(_on_device(values, what), limit, what)


def _words(codes: torch.Tensor) -> np.ndarray:
    return codes.cpu().numpy().view(np.uint32)


def pack_symbols(symbols, bits: int) -> np.ndarray:
    """uint32 words [m, ceil(n/32)*bits] of scalar symbols [m, n] in [0, 2^bits): each row padded with zeros to a
    multiple of 32, symbol i of a group in bits [i*bits, i*bits+bits) of the group's words (compiler_artifact.py:
    225-240). Packed on the GPU."""
    shape = tuple(symbols.shape) if hasattr(symbols, "shape") else np.shape(symbols)
    if len(shape) != 2 or not 1 <= bits <= 8:
        raise ValueError("invalid symbols or width")
    q = _device_codes(symbols, 1 << bits, "invalid symbols or width")
    if shape[1] == 0:
        return np.zeros((shape[0], 0), dtype=np.uint32)
    codes, _ = E.pack_codes(q, bits, trellis=False)
    return _words(codes)


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


def valid_path(states, bits: int, state_bits: int = STATE_BITS) -> bool:
    s = np.asarray(states, dtype=np.int64)
    return bool(s.ndim == 2 and s.shape[1] > 0 and np.all((s >= 0) & (s < (1 << state_bits))) and np.all(s[:, 0] < (1 << bits))
                and np.all((s[:, 1:] >> bits) == (s[:, :-1] & ((1 << (state_bits - bits)) - 1))))


def _path_bits(st: torch.Tensor, state_bits: int, rows: torch.Tensor | None = None, base: int = 0):
    """The widths k (1 <= k <= min(8, state_bits-1)) at which rows `rows` of device states st (minus base) are paths
    from state 0, with each width's code words: one pack per candidate on the GPU, one host synchronisation."""
    found = []
    for k in range(1, min(8, state_bits - 1) + 1):
        codes, bad = E.pack_codes(st, k, rows=rows, base=base, L=state_bits)
        found.append((k, codes, bad))
    flags = torch.cat([b for _, _, b in found]).cpu().tolist()
    return [(k, c) for (k, c, _), f in zip(found, flags) if f == 0]


def infer_path_bits(states, state_bits: int = STATE_BITS) -> int:
    """The one width at which every row of `states` is a trellis path from zero (compiler_artifact.py:269-273)."""
    if np.ndim(states) != 2 or np.shape(states)[1] == 0:
        raise ValueError("trellis width is ambiguous or invalid ([]); save explicit row_groups metadata")
    st = _device_codes(states, 1 << state_bits, "trellis width is ambiguous or invalid ([]); save explicit row_groups "
                       "metadata")
    ks = [k for k, _ in _path_bits(st, state_bits)]
    if len(ks) != 1:
        raise ValueError(f"trellis width is ambiguous or invalid ({ks}); save explicit row_groups metadata")
    return ks[0]


def pack_trellis(states, bits: int, state_bits: int = STATE_BITS) -> np.ndarray:
    """uint32 words [m, ceil(n/32)*bits] of row-trellis states: symbols state & (2^bits-1), each row padded forward
    with zeros to a multiple of 32, reversed, then packed as pack_symbols; a row that is not a path from state 0
    raises ValueError (compiler_artifact.py:276-284). Packed and checked on the GPU."""
    shape = tuple(states.shape) if hasattr(states, "shape") else np.shape(states)
    msg = "states are not a row trellis from zero"
    if len(shape) != 2 or shape[1] == 0 or not 1 <= bits < state_bits or state_bits > 16 or bits > 8:
        raise ValueError(msg)
    st = _device_codes(states, 1 << state_bits, msg)
    codes, bad = E.pack_codes(st, bits, L=state_bits)
    if int(bad.item()):
        raise ValueError(msg)
    return _words(codes)


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


def _input_signs(columns: int, seed: int) -> np.ndarray:
    """The input rotation's signs as stored (compiler_artifact.py:300-304): -1 where torch.rand(columns,
    Generator(seed), float64) < 0.5, else +1, as int8 (the same draw the rotation kernels use)."""
    return rht_signs(int(columns), int(seed)).numpy().astype(np.int8)


# ----------------------------------------------------------------------------- saved entries (compiler_artifact.py:307-371)


def encode_entry(name: str, entry: dict, *, signs=None):
    """(tensors, matrix record) of one saved codes entry, values and paths unchanged (compiler_artifact.py:307-371).

    A trellis entry holds "states" [m, n] (each row's states offset by table_index * 4096 into the concatenated
    4096-entry "table"), "scales" fp32 [m], "in_seed" and, optionally, "row_groups" [{rows, bits, table_index}]
    (without them each table's rows form one group and the width is inferred from the paths). A scalar entry holds
    "codes" [m, n] and "levels". The checks and their messages are the reference's; the states are checked and
    packed on the GPU, each group's rows read in place."""
    unsupported = set(entry) & {"log_g", "group_scales", "log_c", "col_scales", "kron", "A", "B"}
    if unsupported:
        raise ValueError(f"unsupported trained transforms: {sorted(unsupported)}")
    trellis = "states" in entry
    enc = _on_device(entry["states"] if trellis else entry["codes"], "saved entry must be a matrix")
    if enc.dim() != 2:
        raise ValueError("saved entry must be a matrix")
    m, n = enc.shape
    scales = _host(entry["scales"])
    if scales.shape != (m,) or scales.dtype != np.float32:
        raise ValueError("saved row scales must be fp32, one per row")
    if not np.isfinite(scales).all():
        raise ValueError("nonfinite row scales")
    table = _host(entry["table" if trellis else "levels"])
    if table.ndim != 1 or table.dtype != np.float32 or not np.isfinite(table).all():
        raise ValueError("saved table must be a finite fp32 vector")
    signs = _input_signs(n, entry["in_seed"]) if signs is None else _host(signs).astype(np.int8)
    if signs.shape != (n,) or not np.isin(signs, [-1, 1]).all():
        raise ValueError("invalid input signs")
    dev = E._abi.device()
    if trellis:
        if len(table) % TABLE_ENTRIES:
            raise ValueError("invalid saved trellis table or states")
        st = _int32_in_range(enc, len(table), "invalid saved trellis table or states")
        gid = torch.div(st, TABLE_ENTRIES, rounding_mode="floor")
        if m and n and not bool((gid == gid[:, :1]).all()):
            raise ValueError("a row crosses table identities")
        row_gid = gid[:, 0].cpu().numpy() if n else np.zeros(m, dtype=np.int32)
        if entry.get("row_groups") is None:
            groups = []
            for ti in sorted(set(row_gid.tolist())):
                rows = np.flatnonzero(row_gid == ti)
                rows_d = torch.from_numpy(rows).to(dev)
                ks = _path_bits(st, STATE_BITS, rows_d, ti * TABLE_ENTRIES)
                if len(ks) != 1:
                    raise ValueError(f"trellis width is ambiguous or invalid ({[k for k, _ in ks]}); save explicit "
                                     "row_groups metadata")
                groups.append({"rows": rows, "bits": ks[0][0], "table_index": ti, "_codes": ks[0][1]})
        else:
            groups = entry["row_groups"]
        prepared, bad = [], torch.zeros(1, dtype=torch.int32, device=dev)
        for g in groups:
            rows = _host(g["rows"]).astype(np.int64)
            bits, ti = int(g["bits"]), int(g["table_index"])
            if rows.ndim != 1 or np.any(rows < 0) or np.any(rows >= m) or not np.all(row_gid[rows] == ti):
                raise ValueError("invalid row group")
            codes = g.get("_codes")
            if codes is None:
                if not 1 <= bits <= 8 or bits >= STATE_BITS:
                    raise ValueError("states are not a row trellis from zero")
                codes, _ = E.pack_codes(st, bits, rows=torch.from_numpy(rows).to(dev), base=ti * TABLE_ENTRIES,
                                        L=STATE_BITS, bad=bad)
            prepared.append((rows, bits, "trellis", table[ti * TABLE_ENTRIES:(ti + 1) * TABLE_ENTRIES], codes))
        if int(bad.item()):
            raise ValueError("states are not a row trellis from zero")
    else:
        bits = max(1, (len(table) - 1).bit_length())
        if enc.numel() and int(enc.max()) >= len(table):
            raise ValueError("scalar index outside table")
        if bits > 8:
            raise ValueError("invalid symbols or width")
        q = _int32_in_range(enc, 1 << bits, "invalid symbols or width")
        codes, _ = E.pack_codes(q, bits, trellis=False)
        prepared = [(np.arange(m), bits, "scalar", table, codes)]
    covered = np.sort(np.concatenate([p[0] for p in prepared])) if prepared else np.zeros(0, dtype=np.int64)
    if not np.array_equal(covered, np.arange(m)):
        raise ValueError("row groups must cover every row exactly once")
    return encode_groups(name, (m, n), prepared, scales, signs)


def encode_groups(name: str, shape, groups, scales: np.ndarray, signs: np.ndarray):
    """(tensors, matrix record) of a matrix whose groups are already packed: groups = [(rows int64 [m_i], bits,
    kind, table float32, code words)] in storage order (the words an int32 device tensor from engine.pack_codes, or
    uint32 host words); scales float32 [rows] of the whole matrix; signs int8 [n]. The tail of encode_entry, and the
    entry point of a caller whose codes were packed where they were made."""
    m, n = (int(d) for d in shape)
    specs, meta = grouped_matrix_specs(name, [m, n], [{"rows": len(r), "bits": b, "kind": kd, "table_entries": len(v)}
                                                      for r, b, kd, v, _ in groups])
    tensors = {name + ".signs": np.asarray(signs, dtype=np.int8)}
    for i, (rows, bits, kind, values, codes) in enumerate(groups):
        key = f"{name}.g{i}"
        tensors[key + ".rows"] = np.asarray(rows).astype(np.uint32)
        tensors[key + ".codes"] = _words(codes) if isinstance(codes, torch.Tensor) else np.asarray(codes, dtype=np.uint32)
        tensors[key + ".scales"] = scales[rows]
        tensors[key + ".table"] = values
    for key, value in tensors.items():
        if _typed_array(value)[0].nbytes != specs[key]["nbytes"]:
            raise AssertionError(f"encoded tensor disagrees with its specification: {key}")
    return tensors, meta


def export_saved_codes(saved: dict, out, *, dense_tensors: dict, model_dir=None) -> dict:
    """Pack a complete model state: every saved codes entry (saved["matrices"]) encoded, every other state tensor
    stored as it is, tied tensors once, the model directory's tokenizer and config files as checked assets
    (compiler_artifact.py:374-430). Returns write_artifact's receipt."""
    coded = saved["matrices"]
    if not set(coded) <= set(dense_tensors):
        raise ValueError("complete dense state is missing named coded matrices")
    aliases = state_aliases(dense_tensors, coded)
    tensors, matrices = {}, {}
    for name, entry in coded.items():
        if "buckets" not in entry:
            tensors_i, matrices[name] = encode_entry(name, entry)
            tensors.update(tensors_i)
            continue
        # an embedding table stored as row buckets: each bucket either coded or kept dense at its own dtype
        dense = dense_tensors[name]
        buckets, seen = [], []
        for i, bucket in enumerate(entry["buckets"]):
            key = f"{name}.b{i}"
            rows = _host(bucket["rows"]).astype(np.uint32)
            seen.extend(rows.tolist())
            tensors[key + ".rows"] = rows
            if "states" in bucket or "codes" in bucket:
                tensors_i, meta = encode_entry(key, bucket)
                tensors.update(tensors_i)
                buckets.append({"rows": key + ".rows", "matrix": meta})
            else:
                tensors[key + ".dense"] = dense[rows.astype(np.int64)]
                buckets.append({"rows": key + ".rows", "dense": key + ".dense"})
        if sorted(seen) != list(range(dense.shape[0])):
            raise ValueError(f"embedding buckets do not exactly cover {name}")
        matrices[name] = {"kind": "table", "shape": list(dense.shape), "buckets": buckets}
    dense_names = [nm for nm in dense_tensors if nm not in coded and nm not in aliases]
    tensors.update((nm, dense_tensors[nm]) for nm in dense_names)
    assets = {}
    if model_dir is not None:
        assets = {a: Path(model_dir) / a for a in _ASSETS if (Path(model_dir) / a).exists()}
    semantic = {"matrices": matrices, "dense": dense_names, "aliases": aliases, "self_contained_weights": True,
                "source_model": saved.get("model"), "scale_precision": "fp32 preserved",
                "assets": {a: {"bytes": p.stat().st_size, "sha256": file_sha256(p)} for a, p in assets.items()}}
    return write_artifact(out, tensors, semantic, assets=assets)


def decode_rotated(tensors: dict, meta: dict) -> np.ndarray:
    """table[symbol or state] * scale of a grouped matrix, in the rotated input basis (compiler_artifact.py:433-442)."""
    out = np.empty(meta["shape"], dtype=np.float32)
    for g in meta["groups"]:
        key, bits, n = g["key"], g["bits"], g["columns"]
        if g["kind"] == "trellis":
            idx = unpack_trellis(tensors[key + ".codes"], bits, n, g["state_bits"])
        else:
            idx = unpack_symbols(tensors[key + ".codes"], bits, n)
        out[tensors[key + ".rows"]] = tensors[key + ".table"][idx] * tensors[key + ".scales"][:, None]
    return out


# ----------------------------------------------------------------------------- shared tables (compiler_artifact.py:445-488)


def find_table_aliases(tensors: dict, semantic: dict) -> dict:
    """alias -> owner among the codebook tables that are byte-identical (same storage type and shape): the first
    in name order owns the bytes. Scales and dense state are never shared."""
    owners: dict = {}
    aliases = {}
    for name in sorted(table_tensor_names(semantic)):
        a, dtype = _typed_array(tensors[name])
        raw = bytes(_bytes_of(a))
        key = (dtype, a.shape, hashlib.sha256(raw).digest())
        for owner, owner_raw in owners.get(key, ()):
            if owner_raw == raw:
                aliases[name] = owner
                break
        else:
            owners.setdefault(key, []).append((name, raw))
    return aliases


def manifest_table_aliases(meta: dict) -> dict:
    """The sharing a manifest's table digests propose (for pricing; write_artifact compares the bytes)."""
    validate_artifact_layout(meta)
    first, aliases = {}, {}
    for name in sorted(table_tensor_names(meta)):
        spec = meta["tensors"][name]
        key = (spec["dtype"], tuple(spec["shape"]), spec["sha256"])
        if key in first:
            aliases[name] = first[key]
        else:
            first[key] = name
    return aliases


# ----------------------------------------------------------------------------- files (compiler_artifact.py:491-558)


def write_artifact(path, tensors: dict, semantic: dict, *, assets: dict | None = None,
                   tensor_aliases: dict | None = None) -> dict:
    """Write the artifact once (an existing path raises FileExistsError), read every byte back and check it, and
    return the receipt of what is stored (compiler_artifact.py:491-530)."""
    path = Path(path)
    if path.exists():
        raise FileExistsError(path)
    typed = {name: _typed_array(v) for name, v in tensors.items()}
    specs = {name: tensor_spec(dt, a.shape) for name, (a, dt) in typed.items()}
    meta = artifact_manifest(specs, semantic, tensor_aliases=tensor_aliases)
    owners = validate_artifact_layout(meta)
    for name, owner in owners.items():
        if owner != name and bytes(_bytes_of(typed[name][0])) != bytes(_bytes_of(typed[owner][0])):
            raise ValueError(f"table alias bytes differ: {name}")
    physical = [nm for nm in sorted(typed) if owners[nm] == nm]
    with _pool() as pool:
        digests = dict(zip(physical, pool.map(lambda nm: hashlib.sha256(_bytes_of(typed[nm][0])).hexdigest(), physical)))
    for name in sorted(typed):
        meta["tensors"][name]["sha256"] = digests[owners[name]]
    path.mkdir(parents=True)
    with (path / BLOB).open("xb") as f:
        for name in physical:
            f.write(_bytes_of(typed[name][0]))
    (path / MANIFEST).write_bytes(canonical_json(meta))
    for name, source in (assets or {}).items():
        if Path(name).name != name or name in (BLOB, MANIFEST):
            raise ValueError("invalid asset name")
        shutil.copyfile(source, path / name)
    loaded, checked = read_artifact(path)
    if checked != meta:
        raise RuntimeError("artifact manifest round-trip failed")
    for name, (a, _) in typed.items():
        if _bytes_of(loaded[name]) != _bytes_of(a):
            raise RuntimeError(f"artifact round-trip failed for {name}")
    payload = (path / BLOB).stat().st_size
    manifest_bytes = (path / MANIFEST).stat().st_size
    if payload + manifest_bytes != artifact_serialized_bytes(specs, semantic, tensor_aliases=tensor_aliases):
        raise RuntimeError("artifact size disagrees with its planned layout")
    files = list(path.iterdir())
    return {"path": str(path), "payload_bytes": payload, "manifest_bytes": manifest_bytes,
            "asset_bytes": sum(p.stat().st_size for p in files if p.name not in (BLOB, MANIFEST)),
            "total_bytes": sum(p.stat().st_size for p in files),
            "manifest_sha256": hashlib.sha256((path / MANIFEST).read_bytes()).hexdigest(),
            "tensor_count": len(tensors), "physical_tensor_count": len(physical),
            "table_alias_count": len(owners) - len(physical), "all_tensor_bytes_verified": True}


def read_artifact(path, *, verify: bool = True):
    """(tensors, manifest) of an artifact: read-only numpy views of one read of the blob, each tensor's sha256
    checked (with verify), and the assets' sizes and digests (compiler_artifact.py:533-558)."""
    path = Path(path)
    meta = json.loads((path / MANIFEST).read_text())
    owners = validate_artifact_layout(meta)
    blob_path = path / BLOB
    if blob_path.stat().st_size != meta["blob_bytes"]:
        raise ValueError("artifact blob size mismatch")
    blob = blob_path.read_bytes()
    if len(blob) != meta["blob_bytes"]:
        raise ValueError("artifact blob size mismatch")
    specs = meta["tensors"]
    physical = [nm for nm in sorted(specs) if owners[nm] == nm]
    view = memoryview(blob)
    if verify:
        def digest(nm):
            s = specs[nm]
            return hashlib.sha256(view[s["offset"]:s["offset"] + s["nbytes"]]).hexdigest()

        with _pool() as pool:
            for nm, d in zip(physical, pool.map(digest, physical)):
                if d != specs[nm]["sha256"]:
                    raise ValueError(f"tensor checksum mismatch: {nm}")
    tensors = {}
    for nm in sorted(specs):
        s = specs[owners[nm]]
        tensors[nm] = np.frombuffer(blob, dtype=NP_DTYPES[s["dtype"]], count=math.prod(s["shape"]),
                                    offset=s["offset"]).reshape(s["shape"])
    for name, spec in meta.get("assets", {}).items():
        if Path(name).name != name:
            raise ValueError("invalid asset path")
        asset = path / name
        if asset.stat().st_size != spec["bytes"] or (verify and file_sha256(asset) != spec["sha256"]):
            raise ValueError(f"asset checksum mismatch: {name}")
    return tensors, meta
