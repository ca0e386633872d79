"""``maxsim._ops.ops``: the operator namespace the reference's Python layer
and tests use (reference torch-ext/maxsim/__init__.py:24,
tests/test_backward.py:16).  It is ``torch.ops.maxsim_amd``, whose nine
operators have the reference's names and schemas
(torch-ext/torch_binding.cpp:7-90)."""

from maxsim_amd._ops import ops  # noqa: F401

__all__ = ["ops"]
