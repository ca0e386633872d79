"""bench.py --matrix writes the reference's v2 benchmark record: the same
key sets at every level as the reference's published H200 record
(bench_results/v2/h200.json, schema of scripts/bench_matrix.py:767-792,
committed as tests/golden/v2_schema_keys.json), the same presets and
surfaces, and the commit the libraries were built from."""

from __future__ import annotations

import json
import re
from pathlib import Path

import bench

KEYS = json.loads((Path(__file__).resolve().parent / "golden" / "v2_schema_keys.json").read_text())


def _fake_runs(repeats=3):
    runs = []
    for r in range(repeats):
        rs = []
        for name, shape in bench.MATRIX_CONTRASTIVE:
            rs.append(dict(surface="contrastive_train", preset=name,
                           shape={"Nq": shape["Nq"], "Nb": shape["Nb"], "Lq": shape["Lq"],
                                  "Ld": shape["Ld"], "D": shape["dim"]},
                           dtype="bf16", k=0.1 + r * 0.01, n=1.0, kf=0.04, nf=0.4, padded=None,
                           kmb=10.0, nmb=20.0, red=float(shape["Ld"]), correct=True))
        for surface, table in (("padded_infer", bench.MATRIX_PADDED),
                               ("packed_infer", bench.MATRIX_PACKED)):
            for name, shape in table:
                rs.append(dict(surface=surface, preset=name,
                               shape={"B": shape["B"], "K": shape["C"], "Lq": shape["Lq"],
                                      "Ld": shape["Ld"], "D": shape["dim"]},
                               dtype="bf16", k=0.08, n=0.3 + r * 0.01, kf=None, nf=None,
                               padded=0.07 if surface == "packed_infer" else None,
                               kmb=5.0, nmb=9.0, red=None, correct=True))
        runs.append(rs)
    return runs


def test_matrix_record_has_the_reference_key_sets():
    machine = {"gpu_name": "x", "compute_capability": "gfx950", "torch_version": "t",
               "cuda_version": "h"}
    rec = bench.matrix_payload(_fake_runs(), machine=machine, n_iter=30, n_warm=5, repeats=3,
                               started="2026-01-01T00:00:00Z", wall=1.0)
    assert sorted(rec) == KEYS["top"]
    assert sorted(rec["kernel"]) == KEYS["kernel"]
    assert sorted(rec["machine"]) == KEYS["machine"]
    assert sorted(rec["bench"]) == KEYS["bench"]
    for r in rec["results"]:
        assert sorted(r) == KEYS["result"]
        assert sorted(r["variance"]) == KEYS["variance"]
        assert sorted(r["shape"]) == KEYS["shape"][r["surface"]]
    assert sorted({r["surface"] for r in rec["results"]}) == KEYS["surfaces"]
    assert sorted({r["preset"] for r in rec["results"]}) == KEYS["presets"]
    json.dumps(rec)  # serialisable
    # backward = step - forward; speedups from the medians
    r0 = rec["results"][0]
    assert abs(r0["maxsim_bwd_ms"] - (r0["maxsim_step_ms"] - r0["maxsim_fwd_ms"])) < 1e-12
    assert abs(r0["step_speedup"] - r0["naive_step_ms"] / r0["maxsim_step_ms"]) < 1e-12


def test_matrix_record_names_the_commit():
    state = bench.git_state()
    assert re.fullmatch(r"[0-9a-f]{40}", state["git_commit"]), state
    assert isinstance(state["git_dirty"], bool)
