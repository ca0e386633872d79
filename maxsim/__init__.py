"""``import maxsim`` for callers of the reference package.

The reference's callers and tests import ``maxsim`` and ``from maxsim._ops
import ops`` (reference tests/conftest.py:129-145, tests/test_backward.py:15-16,
torch-ext/maxsim/__init__.py:24).  This package answers to those names with
this build: every public function, the reference functions and
``_pack_padded`` are those of :mod:`maxsim_amd` (same objects), and
:mod:`maxsim._ops` exposes the operator namespace ``ops``.  Nothing here
computes; there is no fallback if the native libraries are missing (the
import of :mod:`maxsim_amd` then fails).
"""

from __future__ import annotations

import maxsim_amd as _impl
from maxsim_amd import (  # noqa: F401  (re-exported)
    __all__,
    __version__,
    _pack_padded,
    host_checks,
    maxsim_reference,
    maxsim_reference_with_argmax,
    pack_documents,
    score_candidates_padded,
    score_candidates_padded_backward_reference,
    score_candidates_padded_reference,
    score_candidates_padded_train,
    score_candidates_padded_with_argmax,
    score_candidates_padded_with_argmax_reference,
    score_contrastive,
    score_contrastive_backward_reference,
    score_contrastive_cross_entropy,
    score_contrastive_cross_entropy_value_and_grad,
    score_contrastive_reference,
    score_contrastive_train,
    score_contrastive_with_argmax,
    score_contrastive_with_argmax_reference,
    score_pairs_packed,
    score_pairs_packed_backward_reference,
    score_pairs_packed_reference,
    score_pairs_packed_train,
    score_pairs_packed_with_argmax,
    score_pairs_packed_with_argmax_reference,
    set_host_checks,
)

from . import _ops, reference  # noqa: F401,E402

__all__ = list(_impl.__all__)
