"""Row plans (rowgroup-plan-1 JSON) with the reference's validation (rowgroup_alloc.py:268-307): every listed
matrix is active, each group has a positive multiple of 64 rows inside the matrix, widths 1-4 and the matrix's
column count; a matrix has one to eight groups with consecutive ids from zero that cover every row exactly once."""

from __future__ import annotations

import hashlib
import json
from pathlib import Path
from typing import Mapping, Sequence


def _nonnegative_int(value, what):
    if isinstance(value, bool) or not isinstance(value, int) or value < 0:
        raise ValueError(f"{what} must be a nonnegative integer")
    return value


def load_row_plan(path, shapes: Mapping[str, Sequence[int]]):
    raw = Path(path).read_bytes()
    data = json.loads(raw)
    if data.get("format") != "rowgroup-plan-1" or not isinstance(data.get("groups"), list) or not data["groups"]:
        raise ValueError("row plan must be a nonempty rowgroup-plan-1 allocation")
    result: dict = {}
    for record in data["groups"]:
        name = record.get("matrix")
        if not isinstance(name, str) or name not in shapes:
            raise ValueError(f"row plan names an unknown or inactive matrix: {name!r}")
        rows, columns = map(int, shapes[name])
        bits = _nonnegative_int(record.get("bits"), "row-plan bits")
        index = _nonnegative_int(record.get("group"), "row-plan group")
        rids = record.get("rows")
        if bits not in (1, 2, 3, 4) or record.get("columns") != columns:
            raise ValueError(f"{name}: unsupported width or wrong column count")
        if not isinstance(rids, list) or not rids or len(rids) % 64:
            raise ValueError(f"{name}: each row group must have a positive multiple of 64 rows")
        if any(isinstance(r, bool) or not isinstance(r, int) or not 0 <= r < rows for r in rids):
            raise ValueError(f"{name}: row index outside the matrix")
        result.setdefault(name, []).append({"group": index, "rows": rids, "bits": bits})
    for name, records in result.items():
        records.sort(key=lambda r: r["group"])
        if len(records) > 8 or [r["group"] for r in records] != list(range(len(records))):
            raise ValueError(f"{name}: use one to eight consecutive group ids starting at zero")
        flat = [r for rec in records for r in rec["rows"]]
        if sorted(flat) != list(range(int(shapes[name][0]))):
            raise ValueError(f"{name}: row groups must cover every row exactly once")
    manifest = {"path": str(path), "sha256": hashlib.sha256(raw).hexdigest(), "matrices": len(result),
                "groups": len(data["groups"]),
                "allocation": {k: data[k] for k in ("budget_bytes", "total_bytes", "payload_bytes", "size_scope") if k in data}}
    return result, manifest


def write_row_plan(path, plans: Mapping[str, list], shapes: Mapping[str, Sequence[int]]):
    """Write {matrix: [{"group", "rows", "bits"}]} as a rowgroup-plan-1 file (the format load_row_plan reads)."""
    groups = [{"matrix": name, "group": int(g["group"]), "rows": [int(r) for r in g["rows"]], "bits": int(g["bits"]),
               "columns": int(shapes[name][1])} for name, gs in plans.items() for g in gs]
    Path(path).write_text(json.dumps({"format": "rowgroup-plan-1", "groups": groups}))
