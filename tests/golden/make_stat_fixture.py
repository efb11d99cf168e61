"""Writes tests/golden/stat_counts.json from the reference's statistical plan
and its recorded CUDA counts (data only: cells, keys and counts).

    python tests/golden/make_stat_fixture.py /root/reference

Sources: tests/stat_plan.json (the ten cells, the RNG keys) and
results/stat-cuda.json / results/stat-cuda-predicate.json (2,000,000 draws per
cell on the reference's fused path with list_max 256 / 0).
"""
import json
import sys
from pathlib import Path

root = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
plan = json.loads((root / "tests" / "stat_plan.json").read_text())
runs = {256: json.loads((root / "results" / "stat-cuda.json").read_text()),
        0: json.loads((root / "results" / "stat-cuda-predicate.json").read_text())}
out = {
    "source": "reference tests/stat_plan.json, results/stat-cuda.json (list_max 256), "
              "results/stat-cuda-predicate.json (list_max 0)",
    "samples_per_cell": plan["samples_per_cell"],
    "seed_start": plan["seed_start"],
    "stream_id": plan["stream_id"],
    "position": plan["position"],
    "proposal_rng": plan["proposal_rng"],
    "cells": [],
}
for cell in plan["cells"]:
    counts = {str(lm): next(c["counts"] for c in run["cells"] if c["cell"] == cell["name"]) for lm, run in runs.items()}
    out["cells"].append({**{k: cell[k] for k in ("name", "kind", "weights", "expected")},
                         "params": cell.get("params", {}), "counts": counts})
path = Path(__file__).with_name("stat_counts.json")
path.write_text(json.dumps(out, indent=1) + "\n")
print(path)
