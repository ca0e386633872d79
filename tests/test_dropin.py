"""The reference's import path resolves to this build (CPU only).

The reference's callers write ``import maxsim`` and ``from maxsim._ops import
ops`` (reference tests/conftest.py:129-145, tests/test_backward.py:15-16);
``maxsim`` here is a thin package over ``maxsim_amd``.  Also checks that the
ABI version the integration guide at the repository root states is the one
the library reports."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent

# torch-ext/torch_binding.cpp:7-90
REFERENCE_OPS = [
    "maxsim_forward",
    "maxsim_padded_forward",
    "maxsim_padded_forward_with_argmax",
    "maxsim_padded_backward",
    "maxsim_packed_forward_with_argmax",
    "maxsim_packed_backward",
    "maxsim_contrastive_forward",
    "maxsim_contrastive_forward_with_argmax",
    "maxsim_contrastive_backward",
]

# torch-ext/maxsim/__init__.py:38-56
REFERENCE_ALL = [
    "score_pairs_packed",
    "score_pairs_packed_with_argmax",
    "score_pairs_packed_train",
    "score_candidates_padded",
    "score_candidates_padded_with_argmax",
    "score_candidates_padded_train",
    "score_contrastive",
    "score_contrastive_with_argmax",
    "score_contrastive_train",
    "maxsim_reference",
    "maxsim_reference_with_argmax",
    "score_pairs_packed_reference",
    "score_pairs_packed_with_argmax_reference",
    "score_candidates_padded_reference",
    "score_candidates_padded_with_argmax_reference",
    "score_contrastive_reference",
    "score_contrastive_with_argmax_reference",
]


def test_import_maxsim_finds_the_ops():
    import maxsim
    from maxsim._ops import ops

    import maxsim_amd

    for name in REFERENCE_OPS:
        assert hasattr(ops, name), name
        # the very operator the maxsim_amd package calls
        assert getattr(ops, name) is getattr(maxsim_amd._ops.ops, name)
    assert maxsim._ops.ops is ops


def test_import_maxsim_public_surface():
    import maxsim

    import maxsim_amd

    assert sorted(maxsim.__all__) == sorted(REFERENCE_ALL)
    for name in REFERENCE_ALL + ["_pack_padded"]:
        assert getattr(maxsim, name) is getattr(maxsim_amd, name), name
    from maxsim.reference import score_contrastive_reference

    assert score_contrastive_reference is maxsim_amd.score_contrastive_reference


def test_integration_doc_states_the_library_abi_version():
    text = (ROOT / "INTEGRATION.md").read_text()
    documented = re.findall(r"maxsim_amd_abi_version\(\)` returns (\d+)", text)
    assert documented, "INTEGRATION.md must state the ABI version"
    lib = ctypes.CDLL(str(ROOT / "maxsim_amd" / "libmaxsim_amd.so"))
    assert {int(x) for x in documented} == {lib.maxsim_amd_abi_version()}
