"""Operator namespace of the native binding.

``ops`` is ``torch.ops.maxsim_amd``: the nine operators of the reference's
torch extension (torch-ext/torch_binding.cpp:7-90) with identical names,
argument order and return arity, implemented by hand-written HIP kernels for
gfx950 behind the C ABI in ``include/maxsim_amd.h``.  Two more operators,
``maxsim_contrastive_backward_typed`` and ``maxsim_packed_backward_typed``,
are the contrastive and packed backwards with the gradients in the inputs'
dtype; the autograd Functions use them so that torch does not cast fp32
gradients in a separate pass.  ``maxsim_pack_padded_rows`` is the device
copy behind :func:`maxsim_amd._pack_padded` (padded -> packed rows), and
``maxsim_cross_entropy_forward`` / ``maxsim_contrastive_cross_entropy_backward``
are the fused training loss behind
:func:`maxsim_amd.score_contrastive_cross_entropy`.

Importing this module loads ``_maxsim_amd_torch.so`` (which pulls in
``libmaxsim_amd.so``).  There is no fallback: if the native build is missing
the import fails with instructions, so nothing can silently run elsewhere.
"""

from __future__ import annotations

from pathlib import Path

import torch

_HERE = Path(__file__).resolve().parent
NATIVE_LIB = _HERE / "libmaxsim_amd.so"
TORCH_BINDING = _HERE / "_maxsim_amd_torch.so"

if not TORCH_BINDING.exists() or not NATIVE_LIB.exists():
    raise ImportError(
        "maxsim_amd native libraries are not built "
        f"({TORCH_BINDING.name}, {NATIVE_LIB.name} missing in {_HERE}); "
        "run `python maxsim_amd/_build.py` (needs hipcc for gfx950)"
    )

if not hasattr(torch.ops.maxsim_amd, "maxsim_contrastive_forward"):
    torch.ops.load_library(str(TORCH_BINDING))

ops = torch.ops.maxsim_amd


# ---------------------------------------------------------------------------
# Shape functions so the operators trace under torch.compile / FakeTensor.
# ---------------------------------------------------------------------------
def _f32(t: torch.Tensor, shape) -> torch.Tensor:
    return t.new_empty(shape, dtype=torch.float32)


def _i32(t: torch.Tensor, shape) -> torch.Tensor:
    return t.new_empty(shape, dtype=torch.int32)


@torch.library.register_fake("maxsim_amd::maxsim_forward")
def _(queries, query_offsets, documents, document_offsets, pair_query_ids,
      pair_document_ids, max_q_len):
    return _f32(queries, (pair_query_ids.shape[0],))


@torch.library.register_fake("maxsim_amd::maxsim_packed_forward_with_argmax")
def _(queries, query_offsets, documents, document_offsets, pair_query_ids,
      pair_document_ids, max_q_len):
    n = pair_query_ids.shape[0]
    return _f32(queries, (n,)), _i32(queries, (n, max_q_len))


@torch.library.register_fake("maxsim_amd::maxsim_packed_backward")
def _(dscore, queries, query_offsets, documents, document_offsets,
      pair_query_ids, pair_document_ids, argmax, max_q_len):
    return _f32(queries, queries.shape), _f32(documents, documents.shape)


@torch.library.register_fake("maxsim_amd::maxsim_padded_forward")
def _(queries, query_lengths, documents, doc_lengths, Lq_max, Ld_max,
      num_candidates):
    return _f32(queries, (doc_lengths.shape[0],))


@torch.library.register_fake("maxsim_amd::maxsim_padded_forward_with_argmax")
def _(queries, query_lengths, documents, doc_lengths, Lq_max, Ld_max,
      num_candidates):
    n = doc_lengths.shape[0]
    return _f32(queries, (n,)), _i32(queries, (n, Lq_max))


@torch.library.register_fake("maxsim_amd::maxsim_padded_backward")
def _(dscore, queries, documents, query_lengths, doc_lengths, argmax, Lq_max,
      Ld_max, num_candidates):
    return _f32(queries, queries.shape), _f32(documents, documents.shape)


@torch.library.register_fake("maxsim_amd::maxsim_contrastive_forward")
def _(queries, documents, document_offsets):
    return _f32(queries, (queries.shape[0], document_offsets.shape[0] - 1))


@torch.library.register_fake("maxsim_amd::maxsim_contrastive_forward_with_argmax")
def _(queries, documents, document_offsets):
    nq, lq = queries.shape[0], queries.shape[1]
    nb = document_offsets.shape[0] - 1
    return _f32(queries, (nq, nb)), _i32(queries, (nq, nb, lq))


@torch.library.register_fake("maxsim_amd::maxsim_contrastive_backward")
def _(dscore, queries, documents, document_offsets, argmax):
    return _f32(queries, queries.shape), _f32(documents, documents.shape)


@torch.library.register_fake("maxsim_amd::maxsim_packed_backward_typed")
def _(dscore, queries, query_offsets, documents, document_offsets,
      pair_query_ids, pair_document_ids, argmax, max_q_len):
    return queries.new_empty(queries.shape), documents.new_empty(documents.shape)


@torch.library.register_fake("maxsim_amd::maxsim_padded_backward_typed")
def _(dscore, queries, documents, query_lengths, doc_lengths, argmax, Lq_max,
      Ld_max, num_candidates):
    return queries.new_empty(queries.shape), documents.new_empty(documents.shape)


@torch.library.register_fake("maxsim_amd::maxsim_pack_padded_rows")
def _(padded, lengths, offsets, max_len, packed_rows):
    return padded.new_empty((packed_rows, padded.shape[1]))


@torch.library.register_fake("maxsim_amd::maxsim_contrastive_backward_typed")
def _(dscore, queries, documents, document_offsets, argmax):
    return queries.new_empty(queries.shape), documents.new_empty(documents.shape)


@torch.library.register_fake("maxsim_amd::maxsim_cross_entropy_forward")
def _(scores, targets, inv_temperature, reduction):
    nq = scores.shape[0]
    return _f32(scores, (nq,)), _f32(scores, (nq,) if reduction == 0 else ())


@torch.library.register_fake("maxsim_amd::maxsim_contrastive_cross_entropy_backward")
def _(grad_loss, scores, lse, targets, inv_temperature, reduction, queries, documents,
      document_offsets, argmax):
    return queries.new_empty(queries.shape), documents.new_empty(documents.shape)


__all__ = ["ops", "NATIVE_LIB", "TORCH_BINDING"]
