"""How the arrays of artifact_inputs.npz combine into the saved-codes payload, the state dict and the shared-table
entry that the golden opgraph-packed-1 artifacts were exported from (make_artifact_golden.py wrote the arrays and
the reference's files from exactly this construction; the tests rebuild it to export the same codes)."""

from __future__ import annotations

import numpy as np


def saved_and_state(a: dict, torch):
    """The saved-codes payload and the complete state dict built from the arrays (the tests build the same)."""
    t = torch.from_numpy
    up = {"states": t(a["up__states"]), "scales": t(a["up__scales"]), "in_seed": 1201, "table": t(a["up__table"]),
          "row_groups": [{"rows": t(a[f"up__rows{i}"]), "bits": b, "table_index": i} for i, b in enumerate((2, 1, 3))]}
    gate = {"states": t(a["gate__states"]), "scales": t(a["gate__scales"]), "in_seed": 1202, "table": t(a["gate__table"])}
    o = {"codes": t(a["o__codes"]), "scales": t(a["o__scales"]), "in_seed": 1301, "levels": t(a["o__levels"])}
    emb = {"buckets": [{"rows": t(a["emb__rows0"]), "states": t(a["emb__states"]), "scales": t(a["emb__scales"]),
                        "in_seed": 1401, "table": t(a["emb__table"]),
                        "row_groups": [{"rows": torch.arange(16), "bits": 2, "table_index": 0}]},
                       {"rows": t(a["emb__rows1"])}]}
    embed = t(a["emb__dense"])
    state = {"model.embed_tokens.weight": embed,
             "model.layers.0.self_attn.o_proj.weight": t(a["o__dense"]),
             "model.layers.0.mlp.gate_proj.weight": t(a["gate__dense"]),
             "model.layers.0.mlp.up_proj.weight": t(a["up__dense"]),
             "model.layers.0.mlp.up_proj.bias": t(a["bias_f32"]),
             "model.layers.0.self_attn.k_norm.weight": t(a["kn_f16"]),
             "model.norm.weight": t(a["norm_bf16_bits"].astype(np.int16)).view(torch.bfloat16),
             "model.position_ids": t(a["pos_i64"]),
             "model.empty": t(a["empty_f32"]),
             "lm_head.weight": embed}
    saved = {"model": "synthetic/tiny", "matrices": {"model.embed_tokens.weight": emb,
                                                     "model.layers.0.self_attn.o_proj.weight": o,
                                                     "model.layers.0.mlp.gate_proj.weight": gate,
                                                     "model.layers.0.mlp.up_proj.weight": up}}
    alias = {"states": t(a["alias__states"]), "scales": t(a["alias__scales"]), "in_seed": 1501,
             "table": t(a["alias__table"]),
             "row_groups": [{"rows": torch.arange(0, 16), "bits": 1, "table_index": 0},
                            {"rows": torch.arange(16, 28), "bits": 2, "table_index": 1},
                            {"rows": torch.arange(28, 40), "bits": 3, "table_index": 2}]}
    return saved, state, alias
