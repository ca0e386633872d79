"""Every public entry point rejects inputs spread over two devices.

The reference checks that all tensors of a call share one device and raises
RuntimeError naming the devices (torch-ext/maxsim/__init__.py:75-84,
tests/test_invalid_inputs.py:273-280).  Each case here moves one tensor
argument of a GPU call to the CPU, in every position, for the nine public
functions, and for the fused cross-entropy's targets."""

from __future__ import annotations

import pytest
import torch

import maxsim_amd

from ._helpers import make_contrastive, make_packed, make_padded

pytestmark = pytest.mark.gpu


def _padded():
    q, d, ql, dl = make_padded(2, 3, 16, 20, 32, torch.bfloat16, seed=1)
    return [q, d, ql, dl]


def _packed():
    return list(make_packed(3, 4, 6, 32, (4, 12), (5, 20), torch.bfloat16, seed=2))


def _contrastive():
    q, d, off = make_contrastive(3, 16, 32, [7, 9, 12, 5], torch.bfloat16, seed=3)
    return [q, d, off]


CASES = [
    ("score_candidates_padded", _padded),
    ("score_candidates_padded_with_argmax", _padded),
    ("score_candidates_padded_train", _padded),
    ("score_pairs_packed", _packed),
    ("score_pairs_packed_with_argmax", _packed),
    ("score_pairs_packed_train", _packed),
    ("score_contrastive", _contrastive),
    ("score_contrastive_with_argmax", _contrastive),
    ("score_contrastive_train", _contrastive),
]


@pytest.mark.parametrize("name,make", CASES, ids=[c[0] for c in CASES])
def test_one_cpu_tensor_among_gpu_inputs_raises(name, make):
    fn = getattr(maxsim_amd, name)
    args = make()
    fn(*args)  # all on the GPU: accepted
    for pos in range(len(args)):
        moved = list(args)
        moved[pos] = moved[pos].cpu()
        with pytest.raises(RuntimeError, match="device"):
            fn(*moved)


def test_cross_entropy_cpu_targets_raise():
    q, d, off = _contrastive()
    targets = torch.tensor([0, 1, 2])
    for fn in (maxsim_amd.score_contrastive_cross_entropy,
               maxsim_amd.score_contrastive_cross_entropy_value_and_grad):
        with pytest.raises(RuntimeError, match="device"):
            fn(q, d, off, targets)
