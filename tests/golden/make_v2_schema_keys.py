"""Writes v2_schema_keys.json: the key sets of the reference's published v2
benchmark record (bench_results/v2/h200.json, the output schema of
scripts/bench_matrix.py:767-792), read as JSON data.  Run in the build
container, where /root/reference exists:

    python tests/golden/make_v2_schema_keys.py
"""

from __future__ import annotations

import json
from pathlib import Path

SRC = Path("/root/reference/bench_results/v2/h200.json")
OUT = Path(__file__).resolve().parent / "v2_schema_keys.json"


def main() -> None:
    rec = json.loads(SRC.read_text())
    keys = {
        "top": sorted(rec),
        "kernel": sorted(rec["kernel"]),
        "machine": sorted(rec["machine"]),
        "bench": sorted(rec["bench"]),
        "result": sorted(set().union(*(r.keys() for r in rec["results"]))),
        "variance": sorted(set().union(*(r["variance"].keys() for r in rec["results"]))),
        "surfaces": sorted({r["surface"] for r in rec["results"]}),
        "presets": sorted({r["preset"] for r in rec["results"]}),
        "shape": {r["surface"]: sorted(r["shape"]) for r in rec["results"]},
    }
    OUT.write_text(json.dumps(keys, indent=1) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
