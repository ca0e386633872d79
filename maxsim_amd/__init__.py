"""MaxSim on AMD Instinct MI355X (gfx950): ``score(q, d) = sum_i max_j <q_i, d_j>``.

Drop-in for the Python surface of the reference package
(torch-ext/maxsim/__init__.py, ``__all__`` at :38-56):

* :func:`score_candidates_padded` (+ ``_with_argmax``, ``_train``) -- padded
  reranking of ``[B, K, Ld, D]`` candidates per query.
* :func:`score_contrastive` (+ ``_with_argmax``, ``_train``) -- all-pairs
  ``[Nq, Nb]`` scores against packed documents; in-batch contrastive training.
* :func:`score_pairs_packed` (+ ``_with_argmax``, ``_train``) -- arbitrary
  ``(query, document)`` pair lists over ragged packed inputs.

Every function validates its inputs on the host with the reference's error
types and messages, then calls an operator of :mod:`maxsim_amd._ops`, which
runs hand-written HIP kernels (fused MFMA forward with an in-register
max/argmax epilogue; argmax-driven gather/scatter backward).  Scores are fp32;
gradients are summed in fp32.  ``.grad`` has the input dtype: the kernels
round the fp32 sums to nearest even on the way out, the bits autograd's cast
of fp32 gradients would give, without the separate cast pass.

The pure-PyTorch ``*_reference`` functions of the reference package are
exported too (:mod:`maxsim_amd.reference`) for benchmarks and comparisons;
they are never used by the operators.
"""

from __future__ import annotations

import contextlib
import os
from typing import Tuple

import numpy as np
import torch

from ._ops import ops
from .reference import (
    maxsim_reference,
    maxsim_reference_with_argmax,
    score_candidates_padded_backward_reference,
    score_candidates_padded_reference,
    score_candidates_padded_with_argmax_reference,
    score_contrastive_backward_reference,
    score_contrastive_reference,
    score_contrastive_with_argmax_reference,
    score_pairs_packed_backward_reference,
    score_pairs_packed_reference,
    score_pairs_packed_with_argmax_reference,
)

__version__ = "0.1.0"

__all__ = [
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

_FLOATS = (torch.float32, torch.float16, torch.bfloat16)
_INDEXES = (torch.int32, torch.int64)


# ---------------------------------------------------------------------------
# Host checks of device data (offsets, ids, lengths, targets)
# ---------------------------------------------------------------------------
_HOST_CHECKS = os.environ.get("MAXSIM_AMD_HOST_CHECKS", "1") != "0"


def set_host_checks(enabled: bool) -> bool:
    """Turn the host-side checks of device-resident layout data on (the
    default) or off, process-wide; returns the previous setting.  The
    environment variable ``MAXSIM_AMD_HOST_CHECKS=0`` sets it off at import.

    On, every call copies its offsets / ids / lengths to the host and raises
    the reference's errors for invalid values, which makes the host wait for
    that copy once per call (overlapped with the kernels, but a wait).

    Off, a call on device tensors never waits for the device: only the checks
    that need no device data run (shapes, dtypes, devices), and the kernels'
    own handling of invalid layouts is the contract:

    * a contrastive document with an invalid range (end <= start, start < 0,
      end beyond the documents), a packed pair with an out-of-range id, an
      invalid segment or a query longer than ``max_q_len``, a padded
      candidate or query with a length outside ``(0, padded extent]``: NaN
      score (argmax 0), no gradient from it, nothing read out of range;
    * a cross-entropy target outside ``[0, Nb)``: NaN loss for its row;
    * offsets that are valid ranges but break the CSR convention (not
      starting at 0, not ending at the row count, overlapping) are scored as
      they say; gradient rows that no valid segment covers are unspecified.

    The packed ``_with_argmax`` / ``_train`` functions size the argmax by the
    longest query: without ``max_q_len`` they still read that one integer
    back.  Everything else is capturable in a HIP graph with checks off."""
    global _HOST_CHECKS
    previous = _HOST_CHECKS
    _HOST_CHECKS = bool(enabled)
    return previous


@contextlib.contextmanager
def host_checks(enabled: bool):
    """Context manager form of :func:`set_host_checks` (process-wide while
    the block runs)."""
    previous = set_host_checks(enabled)
    try:
        yield
    finally:
        set_host_checks(previous)


# ---------------------------------------------------------------------------
# Validation helpers (reference __init__.py:59-223, 812-877).  Host work is
# vectorised: each call copies its layout metadata to the host once and checks
# it with numpy instead of per-element Python loops.
# ---------------------------------------------------------------------------
def _require_float(name: str, t: torch.Tensor) -> None:
    if t.dtype not in _FLOATS:
        raise TypeError(f"{name} must be float32, float16, or bfloat16; got {t.dtype}")


def _require_index(name: str, t: torch.Tensor) -> None:
    if t.dtype not in _INDEXES:
        raise TypeError(f"{name} must be int32 or int64; got {t.dtype}")


def _require_one_device(**tensors: torch.Tensor) -> None:
    items = list(tensors.items())
    first_name, first = items[0]
    for name, t in items[1:]:
        if t.device != first.device:
            raise RuntimeError(
                "all tensors must be on the same device; "
                f"{first_name} is on {first.device} but {name} is on {t.device}"
            )


def _to_host(*tensors: torch.Tensor) -> list[np.ndarray]:
    """One device->host copy for several small int tensors, as int64 arrays.

    Tensors of one dtype are joined on the device in their own dtype (no
    join for a single tensor) and widened on the host, so a single int32
    offsets tensor costs one copy and no device kernel."""
    if not tensors:
        return []
    flat = [t.detach().reshape(-1) for t in tensors]
    if len({f.dtype for f in flat}) > 1:
        flat = [f.to(torch.int64) for f in flat]
    joined = (flat[0] if len(flat) == 1 else torch.cat(flat)).cpu().numpy().astype(np.int64)
    out, pos = [], 0
    for f in flat:
        out.append(joined[pos:pos + f.numel()])
        pos += f.numel()
    return out


_COPY_STREAMS: dict = {}


def _host_copies_async(*tensors: torch.Tensor):
    """Queue device->host copies of small int tensors into pinned memory on a
    side stream (default priority, one per device) and return the host
    tensors and an event that marks their completion.

    The side stream first waits for the work already queued on the current
    stream, so the copies see every earlier write of their sources.  Kernels
    queued on the current stream afterwards do not wait for the copies: the
    validation copies stay off the compute stream.  Used where the kernels
    run many small workgroups (padded, packed), so the copies' blit kernels
    find a free CU at once."""
    device = tensors[0].device
    cur = torch.cuda.current_stream(device)
    side = _COPY_STREAMS.get(device.index)
    if side is None:
        side = _COPY_STREAMS[device.index] = torch.cuda.Stream(device)
    side.wait_stream(cur)
    hosts = []
    with torch.cuda.stream(side):
        for t in tensors:
            flat = t.detach().reshape(-1)
            host = torch.empty(flat.shape, dtype=flat.dtype, pin_memory=True)
            host.copy_(flat, non_blocking=True)
            hosts.append(host)
        done = torch.cuda.Event()
        done.record(side)
    return hosts, done


def _check_lengths(values: np.ndarray, max_len: int, name: str) -> None:
    if (values <= 0).any():
        raise ValueError(f"{name} must contain values > 0")
    if (values > max_len).any():
        raise ValueError(f"{name} values must be <= padded length {max_len}")


def _check_padded_meta(queries, documents, query_lengths, doc_lengths):
    """Shapes, dtypes and devices of a padded call (no device data read)."""
    if queries.dim() != 3:
        raise ValueError(f"queries must be 3-D [B, Lq, D]; got shape {tuple(queries.shape)}")
    if documents.dim() != 4:
        raise ValueError(
            f"documents must be 4-D [B, C, Ld, D]; got shape {tuple(documents.shape)}"
        )
    B, Lq, D = queries.shape
    Bd, C, Ld, Dd = documents.shape
    if B != Bd:
        raise ValueError(f"batch dim mismatch: queries B={B} but documents B={Bd}")
    if D != Dd:
        raise ValueError(f"embedding dim mismatch: queries D={D} but documents D={Dd}")
    if tuple(query_lengths.shape) != (B,):
        raise ValueError(
            f"query_lengths must have shape [B={B}]; got {tuple(query_lengths.shape)}"
        )
    if tuple(doc_lengths.shape) != (B, C):
        raise ValueError(
            f"doc_lengths must have shape [B={B}, C={C}]; got {tuple(doc_lengths.shape)}"
        )
    if queries.dtype != documents.dtype:
        raise TypeError(
            "queries and documents must have the same dtype; got "
            f"{queries.dtype} vs {documents.dtype}"
        )
    _require_float("queries", queries)
    _require_float("documents", documents)
    _require_index("query_lengths", query_lengths)
    _require_index("doc_lengths", doc_lengths)
    _require_one_device(queries=queries, documents=documents,
                        query_lengths=query_lengths, doc_lengths=doc_lengths)
    return B, C, Lq, Ld, D


# The _checked_* wrappers are host code (pinned copies, events, numpy checks);
# torch.compile runs them eagerly at a graph break, as it does the
# reference's host-side checks.  The operators they launch have fake
# implementations and trace on their own.
@torch.compiler.disable
def _checked_padded(queries, documents, query_lengths, doc_lengths, launch):
    """Validate a padded call and return ``launch(B, C, Lq, Ld)``.

    The lengths travel to pinned host memory by asynchronous copies on a side
    stream (:func:`_host_copies_async`), ``launch`` queues the kernels, and
    only then does the host wait for the copies and check the values, with the same errors
    as a check made before the launch.  The padded kernels are safe with any
    lengths (a candidate with a length outside ``(0, Ld]`` or a query length
    outside ``(0, Lq]`` gives a NaN score, nothing is read out of range), so
    work queued before a failing check is harmless and its result is
    dropped."""
    B, C, Lq, Ld, _ = _check_padded_meta(queries, documents, query_lengths, doc_lengths)
    if not _HOST_CHECKS and query_lengths.is_cuda:
        return launch(B, C, Lq, Ld)
    if not query_lengths.is_cuda:  # host tensors: check first (the operators reject them anyway)
        qlen, dlen = _to_host(query_lengths, doc_lengths)
        _check_lengths(qlen, Lq, "query_lengths")
        _check_lengths(dlen, Ld, "doc_lengths")
        return launch(B, C, Lq, Ld)
    hosts, copied = _host_copies_async(query_lengths, doc_lengths)
    result = launch(B, C, Lq, Ld)
    copied.synchronize()
    qlen, dlen = (h.numpy().astype(np.int64) for h in hosts)
    _check_lengths(qlen, Lq, "query_lengths")
    _check_lengths(dlen, Ld, "doc_lengths")
    return result


def _check_pair_ids(pair_query_ids, pair_document_ids) -> None:
    if pair_query_ids.shape != pair_document_ids.shape:
        raise ValueError(
            "pair_query_ids and pair_document_ids must have the same shape; got "
            f"{tuple(pair_query_ids.shape)} vs {tuple(pair_document_ids.shape)}"
        )
    if pair_query_ids.dim() != 1:
        raise ValueError(f"pair_query_ids must be 1-D; got shape {tuple(pair_query_ids.shape)}")


def _check_csr(values: np.ndarray, total: int, name: str) -> int:
    """Offsets must start at 0, end at ``total`` and have no empty segment.
    Returns the longest segment (reference __init__.py:178-196)."""
    if values.size < 2:
        raise RuntimeError(f"{name} must have length >= 2")
    if values[0] != 0:
        raise RuntimeError(f"{name}[0] must equal 0, got {int(values[0])}")
    if values[-1] != total:
        raise RuntimeError(
            f"{name}[-1] ({int(values[-1])}) must equal total token count ({total})"
        )
    seg = np.diff(values)
    bad = np.flatnonzero(seg <= 0)
    if bad.size:
        raise RuntimeError(f"empty segment in {name} at index {int(bad[0])}")
    return int(seg.max())


def _check_ids(values: np.ndarray, upper: int, name: str) -> None:
    bad = np.flatnonzero((values < 0) | (values >= upper))
    if bad.size:
        i = int(bad[0])
        raise RuntimeError(f"{name}[{i}] = {int(values[i])} out of range [0, {upper})")


def _packed_layout(queries, query_offsets, documents, document_offsets,
                   pair_query_ids, pair_document_ids) -> int:
    qoff, doff, qids, dids = _to_host(query_offsets, document_offsets,
                                      pair_query_ids, pair_document_ids)
    max_q = _check_csr(qoff, queries.shape[0], "query_offsets")
    _check_csr(doff, documents.shape[0], "document_offsets")
    _check_ids(qids, qoff.size - 1, "pair_query_ids")
    _check_ids(dids, doff.size - 1, "pair_document_ids")
    return max_q


def _device_max_segment(offsets: torch.Tensor, total: int):
    """Longest segment of device CSR offsets, read back as one integer (a
    small reduction and a one-element copy instead of all the offsets), or
    None when the offsets cannot be well formed (the host checks then give
    the error)."""
    flat = offsets.detach().reshape(-1)
    if flat.numel() < 2:
        return None
    m = int(torch.diff(flat).max())
    return m if 0 < m <= total else None


@torch.compiler.disable
def _checked_packed(queries, query_offsets, documents, document_offsets,
                    pair_query_ids, pair_document_ids, max_q_len, launch, *,
                    shape_needs_max=True):
    """Validate a packed call and return ``launch(max_q_len)``.

    The offsets and ids travel to pinned host memory by asynchronous copies
    on a side stream (:func:`_host_copies_async`), ``launch`` queues the
    kernels, and only then does the host wait for the copies and run the
    reference's checks with its errors.  The packed kernels are safe with
    any offsets and ids (an invalid pair gives a NaN score, nothing is read
    out of range), so work queued before a failing check is harmless and its
    result is dropped.

    Without ``max_q_len`` the launch needs a bound of the query lengths.  A
    score-only call (``shape_needs_max=False``) uses the number of query
    rows, which bounds every valid segment and gives the same scores.  Where
    the argmax shape is the longest query, that length is computed on the
    device and read back as one integer; offsets that cannot be well formed
    take the synchronous checks first."""
    if not query_offsets.is_cuda:  # host tensors: check first (the operators reject them)
        return launch(_resolve_max_q_len(max_q_len, _packed_layout(
            queries, query_offsets, documents, document_offsets,
            pair_query_ids, pair_document_ids)))
    if max_q_len is not None and max_q_len <= 0:
        raise ValueError(f"max_q_len must be > 0; got {max_q_len}")
    if not _HOST_CHECKS:
        if max_q_len is not None:
            return launch(int(max_q_len))
        if not shape_needs_max:
            return launch(max(int(queries.shape[0]), 1))
        mql = _device_max_segment(query_offsets, int(queries.shape[0]))
        # offsets that cannot be well formed: every pair is invalid anyway
        return launch(mql if mql is not None else 1)
    # queued before the read-back below, so that only the launch sits
    # between the host's wait for the longest query and the kernels
    hosts, copied = _host_copies_async(query_offsets, document_offsets, pair_query_ids,
                                       pair_document_ids)
    if max_q_len is not None:
        mql = int(max_q_len)
    elif not shape_needs_max:
        mql = max(int(queries.shape[0]), 1)
    else:
        mql = _device_max_segment(query_offsets, int(queries.shape[0]))
        if mql is None:
            return launch(_packed_layout(queries, query_offsets, documents, document_offsets,
                                         pair_query_ids, pair_document_ids))
    result = launch(mql)
    copied.synchronize()
    qoff, doff, qids, dids = (h.numpy().astype(np.int64) for h in hosts)
    max_q = _check_csr(qoff, queries.shape[0], "query_offsets")
    _check_csr(doff, documents.shape[0], "document_offsets")
    _check_ids(qids, qoff.size - 1, "pair_query_ids")
    _check_ids(dids, doff.size - 1, "pair_document_ids")
    if max_q_len is not None:
        _resolve_max_q_len(max_q_len, max_q)
    return result


def _resolve_max_q_len(max_q_len, actual: int) -> int:
    if max_q_len is None:
        return actual
    if max_q_len <= 0:
        raise ValueError(f"max_q_len must be > 0; got {max_q_len}")
    if max_q_len < actual:
        raise ValueError(
            f"max_q_len ({max_q_len}) must be >= actual max query segment length ({actual})"
        )
    return int(max_q_len)


def _check_packed_common(queries, query_offsets, documents, document_offsets,
                         pair_query_ids, pair_document_ids, *, argmax_wording: bool):
    if queries.dim() != 2:
        suffix = "" if argmax_wording else " [total_q_tokens, dim]"
        raise ValueError(f"queries must be 2-D{suffix}; got shape {tuple(queries.shape)}")
    if documents.dim() != 2:
        suffix = "" if argmax_wording else " [total_d_tokens, dim]"
        raise ValueError(f"documents must be 2-D{suffix}; got shape {tuple(documents.shape)}")
    if queries.shape[1] != documents.shape[1]:
        raise ValueError(
            f"queries.dim ({queries.shape[1]}) and documents.dim ({documents.shape[1]}) "
            "must match"
        )
    if queries.dtype != documents.dtype:
        raise TypeError(
            "queries and documents must have the same dtype; got "
            f"{queries.dtype} vs {documents.dtype}"
        )
    _require_float("queries", queries)
    _require_float("documents", documents)
    _require_index("query_offsets", query_offsets)
    _require_index("document_offsets", document_offsets)
    _require_index("pair_query_ids", pair_query_ids)
    _require_index("pair_document_ids", pair_document_ids)
    _require_one_device(queries=queries, query_offsets=query_offsets,
                        documents=documents, document_offsets=document_offsets,
                        pair_query_ids=pair_query_ids,
                        pair_document_ids=pair_document_ids)
    _check_pair_ids(pair_query_ids, pair_document_ids)


def _check_contrastive(queries, documents, document_offsets) -> None:
    _require_float("queries", queries)
    _require_float("documents", documents)
    _require_index("document_offsets", document_offsets)
    if queries.dtype != documents.dtype:
        raise TypeError(
            f"queries and documents must share dtype; got {queries.dtype} and {documents.dtype}"
        )
    if queries.dim() != 3:
        raise ValueError(f"queries must be 3-D [Nq, Lq, D]; got shape {tuple(queries.shape)}")
    if documents.dim() != 2:
        raise ValueError(
            "documents must be 2-D [total_d_tokens, D] (packed); got shape "
            f"{tuple(documents.shape)}"
        )
    if document_offsets.dim() != 1:
        raise ValueError(
            f"document_offsets must be 1-D [Nb+1]; got shape {tuple(document_offsets.shape)}"
        )
    if queries.shape[2] != documents.shape[1]:
        raise ValueError(
            f"queries.D ({queries.shape[2]}) must match documents.D ({documents.shape[1]})"
        )
    if queries.shape[1] <= 0:
        raise ValueError(f"Lq must be > 0; got {queries.shape[1]}")
    if queries.shape[2] <= 0:
        raise ValueError(f"dim must be > 0; got {queries.shape[2]}")
    if document_offsets.numel() < 2:
        raise ValueError(
            "document_offsets must have length >= 2 (at least one doc); "
            f"got {document_offsets.numel()}"
        )
    _require_one_device(queries=queries, documents=documents,
                        document_offsets=document_offsets)


def _check_offsets(offs: np.ndarray, total: int) -> None:
    """The host-side offset checks of the contrastive surface (reference
    __init__.py:880-905): CSR convention, total length, strictly increasing."""
    if offs[0] != 0:
        raise ValueError(
            f"document_offsets[0] must equal 0 (CSR offset convention); got {int(offs[0])}"
        )
    if offs[-1] != total:
        raise ValueError(
            f"document_offsets[-1] ({int(offs[-1])}) must equal total doc tokens ({total}); "
            "the packed documents tensor and the offsets must agree on the total length"
        )
    bad = np.flatnonzero(np.diff(offs) <= 0)
    if bad.size:
        i = int(bad[0])
        raise ValueError(
            "document_offsets must be strictly increasing; got "
            f"document_offsets[{i + 1}] ({int(offs[i + 1])}) <= "
            f"document_offsets[{i}] ({int(offs[i])})"
        )


# ---------------------------------------------------------------------------
# Packed pairs
# ---------------------------------------------------------------------------
def score_pairs_packed(queries, query_offsets, documents, document_offsets,
                       pair_query_ids, pair_document_ids, *, max_q_len=None) -> torch.Tensor:
    """MaxSim scores for a packed ragged list of (query, document) pairs.

    Args:
        queries: ``[total_q_tokens, dim]`` fp32 / fp16 / bf16.
        query_offsets: ``[num_queries + 1]`` int32/int64 CSR offsets (start at
            0, end at ``total_q_tokens``, no empty segment).
        documents: ``[total_d_tokens, dim]``, same dtype as ``queries``.
        document_offsets: ``[num_documents + 1]``, same rules.
        pair_query_ids / pair_document_ids: ``[num_pairs]`` ids.
        max_q_len: optional bound on query segment length (checked).

    Returns:
        ``[num_pairs]`` fp32 scores.
    """
    _check_packed_common(queries, query_offsets, documents, document_offsets,
                         pair_query_ids, pair_document_ids, argmax_wording=False)
    return _checked_packed(
        queries, query_offsets, documents, document_offsets, pair_query_ids,
        pair_document_ids, max_q_len,
        lambda mql: ops.maxsim_forward(
            queries.contiguous(), query_offsets.contiguous(), documents.contiguous(),
            document_offsets.contiguous(), pair_query_ids.contiguous(),
            pair_document_ids.contiguous(), mql),
        shape_needs_max=False)


def score_pairs_packed_with_argmax(queries, query_offsets, documents, document_offsets,
                                   pair_query_ids, pair_document_ids, *,
                                   max_q_len=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """As :func:`score_pairs_packed`, plus the winning document-token index per
    query token: int32 ``[num_pairs, max_q_len]`` (0 beyond a pair's length)."""
    _check_packed_common(queries, query_offsets, documents, document_offsets,
                         pair_query_ids, pair_document_ids, argmax_wording=True)
    return _checked_packed(
        queries, query_offsets, documents, document_offsets, pair_query_ids,
        pair_document_ids, max_q_len,
        lambda mql: ops.maxsim_packed_forward_with_argmax(
            queries.contiguous(), query_offsets.contiguous(), documents.contiguous(),
            document_offsets.contiguous(), pair_query_ids.contiguous(),
            pair_document_ids.contiguous(), mql))


class _PackedFn(torch.autograd.Function):
    """Packed forward+argmax / backward pair (reference __init__.py:414-454)."""

    @staticmethod
    def forward(ctx, queries, query_offsets, documents, document_offsets,
                pair_query_ids, pair_document_ids, max_q_len):
        q, d = queries.contiguous(), documents.contiguous()
        qoff, doff = query_offsets.contiguous(), document_offsets.contiguous()
        qids, dids = pair_query_ids.contiguous(), pair_document_ids.contiguous()
        scores, argmax = ops.maxsim_packed_forward_with_argmax(
            q, qoff, d, doff, qids, dids, int(max_q_len))
        ctx.save_for_backward(q, qoff, d, doff, qids, dids, argmax)
        ctx.max_q_len = int(max_q_len)
        return scores

    @staticmethod
    def backward(ctx, dscore):
        q, qoff, d, doff, qids, dids, argmax = ctx.saved_tensors
        # gradients in the inputs' dtype, written by the kernels (the fp32
        # sums rounded to nearest even: what autograd's cast of the reference's
        # fp32 gradients gives, without the separate cast pass)
        dq, dd = ops.maxsim_packed_backward_typed(
            dscore.contiguous().to(torch.float32), q, qoff, d, doff, qids, dids,
            argmax, ctx.max_q_len)
        return dq, None, dd, None, None, None, None


def score_pairs_packed_train(queries, query_offsets, documents, document_offsets,
                             pair_query_ids, pair_document_ids, *,
                             max_q_len=None) -> torch.Tensor:
    """Differentiable :func:`score_pairs_packed` (gradients accumulated in fp32)."""
    _check_packed_common(queries, query_offsets, documents, document_offsets,
                         pair_query_ids, pair_document_ids, argmax_wording=True)
    return _checked_packed(
        queries, query_offsets, documents, document_offsets, pair_query_ids,
        pair_document_ids, max_q_len,
        lambda mql: _PackedFn.apply(queries, query_offsets, documents, document_offsets,
                                    pair_query_ids, pair_document_ids, mql))


# ---------------------------------------------------------------------------
# Padded candidates
# ---------------------------------------------------------------------------
def _padded_flat(queries, documents, query_lengths, doc_lengths):
    B, Lq, D = queries.shape
    _, C, Ld, _ = documents.shape
    return (
        queries.reshape(B * Lq, D).contiguous(),
        documents.reshape(B * C * Ld, D).contiguous(),
        query_lengths.to(torch.int32).contiguous(),
        doc_lengths.reshape(B * C).to(torch.int32).contiguous(),
    )


def score_candidates_padded(queries, documents, query_lengths, doc_lengths) -> torch.Tensor:
    """MaxSim of each query against its own ``C`` padded candidates.

    Args:
        queries: ``[B, Lq, dim]``; documents: ``[B, C, Ld, dim]``;
        query_lengths: ``[B]`` in ``(0, Lq]``; doc_lengths: ``[B, C]`` in ``(0, Ld]``.
        Rows beyond the lengths are never read.

    Returns:
        ``[B, C]`` fp32 scores.
    """
    def launch(B, C, Lq, Ld):
        q, d, ql, dl = _padded_flat(queries, documents, query_lengths, doc_lengths)
        return ops.maxsim_padded_forward(q, ql, d, dl, int(Lq), int(Ld), int(C)).view(B, C)

    return _checked_padded(queries, documents, query_lengths, doc_lengths, launch)


def score_candidates_padded_with_argmax(queries, documents, query_lengths,
                                        doc_lengths) -> Tuple[torch.Tensor, torch.Tensor]:
    """As :func:`score_candidates_padded`, plus int32 argmax ``[B, C, Lq]``
    (first index wins ties; 0 beyond ``query_lengths[b]``)."""
    def launch(B, C, Lq, Ld):
        q, d, ql, dl = _padded_flat(queries, documents, query_lengths, doc_lengths)
        s, a = ops.maxsim_padded_forward_with_argmax(q, ql, d, dl, int(Lq), int(Ld), int(C))
        return s.view(B, C), a.view(B, C, Lq)

    return _checked_padded(queries, documents, query_lengths, doc_lengths, launch)


class _PaddedFn(torch.autograd.Function):
    """Padded forward+argmax / backward pair (reference __init__.py:716-771)."""

    @staticmethod
    def forward(ctx, queries, documents, query_lengths, doc_lengths):
        B, Lq, D = queries.shape
        _, C, Ld, _ = documents.shape
        q, d, ql, dl = _padded_flat(queries, documents, query_lengths, doc_lengths)
        scores, argmax = ops.maxsim_padded_forward_with_argmax(
            q, ql, d, dl, int(Lq), int(Ld), int(C))
        ctx.save_for_backward(q, d, ql, dl, argmax)
        ctx.shapes = (B, C, Lq, Ld, D)
        return scores.view(B, C)

    @staticmethod
    def backward(ctx, dscore):
        B, C, Lq, Ld, D = ctx.shapes
        q, d, ql, dl, argmax = ctx.saved_tensors
        # gradients in the inputs' dtype, rounded from the fp32 sums
        dq, dd = ops.maxsim_padded_backward_typed(
            dscore.reshape(B * C).contiguous().to(torch.float32), q, d, ql, dl,
            argmax, int(Lq), int(Ld), int(C))
        return dq.view(B, Lq, D), dd.view(B, C, Ld, D), None, None


def score_candidates_padded_train(queries, documents, query_lengths,
                                  doc_lengths) -> torch.Tensor:
    """Differentiable :func:`score_candidates_padded` (gradients accumulated in fp32)."""
    return _checked_padded(
        queries, documents, query_lengths, doc_lengths,
        lambda *_: _PaddedFn.apply(queries, documents, query_lengths, doc_lengths))


# ---------------------------------------------------------------------------
# Padded -> packed
# ---------------------------------------------------------------------------
def _pack_padded(queries, documents, query_lengths, doc_lengths, *, validate: bool = False):
    """Convert padded ``[B, Lq, D]`` / ``[B, C, Ld, D]`` inputs to the packed
    inputs of :func:`score_pairs_packed` (reference __init__.py:516-620).

    Returns ``(queries_packed, query_offsets, documents_packed,
    document_offsets, pair_query_ids, pair_document_ids, max_q_len)``; pairs
    are in row-major ``(batch, candidate)`` order, so the packed scores
    reshape to ``[B, C]``, and ``max_q_len`` is a Python int.  The valid rows
    of each query and candidate are one contiguous block of the padded
    tensor; a HIP kernel copies each block to its packed offset, and one
    device-to-host copy brings back the two row totals and the longest query
    (the reference gathers with boolean masks, which sync as well).
    ``validate=True`` adds the reference's length checks.  Without them,
    lengths outside ``[0, padded extent]`` are clamped for both the copy and
    the offsets, so the outputs stay consistent."""
    if queries.dim() != 3:
        raise ValueError(f"queries must be 3-D [B, Lq, D]; got shape {tuple(queries.shape)}")
    if documents.dim() != 4:
        raise ValueError(
            f"documents must be 4-D [B, C, Ld, D]; got shape {tuple(documents.shape)}"
        )
    B, Lq_max, D = queries.shape
    Bd, C, Ld_max, Dd = documents.shape
    if B != Bd:
        raise ValueError(f"batch dim mismatch: queries B={B} but documents B={Bd}")
    if D != Dd:
        raise ValueError(f"embedding dim mismatch: queries D={D} but documents D={Dd}")
    if query_lengths.shape != (B,):
        raise ValueError(
            f"query_lengths must have shape [B={B}]; got {tuple(query_lengths.shape)}"
        )
    if doc_lengths.shape != (B, C):
        raise ValueError(
            f"doc_lengths must have shape [B={B}, C={C}]; got {tuple(doc_lengths.shape)}"
        )
    device = queries.device
    qlen = query_lengths.to(device=device, dtype=torch.int32)
    dlen = doc_lengths.to(device=device, dtype=torch.int32)
    if validate:
        if (qlen <= 0).any().item():
            raise ValueError("query_lengths must all be > 0")
        if (dlen <= 0).any().item():
            raise ValueError("doc_lengths must all be > 0")
        if (qlen > Lq_max).any().item() or (dlen > Ld_max).any().item():
            raise ValueError("a length exceeds the padded extent")
    qc = qlen.clamp(0, Lq_max)
    dc = dlen.reshape(-1).clamp(0, Ld_max)
    query_offsets = torch.zeros(B + 1, dtype=torch.int32, device=device)
    query_offsets[1:] = qc.cumsum(0)
    document_offsets = torch.zeros(B * C + 1, dtype=torch.int32, device=device)
    document_offsets[1:] = dc.cumsum(0)
    longest = qc.max() if B > 0 else query_offsets[0]
    total_q, total_d, max_q = (int(x) for x in torch.stack(
        [query_offsets[-1], document_offsets[-1], longest.to(torch.int32)]).cpu())
    queries_packed = ops.maxsim_pack_padded_rows(
        queries.reshape(B * Lq_max, D), qc, query_offsets, Lq_max, total_q)
    documents_packed = ops.maxsim_pack_padded_rows(
        documents.reshape(B * C * Ld_max, D), dc, document_offsets, Ld_max, total_d)
    pair_indices = torch.arange(B * C, dtype=torch.int32, device=device)
    return (queries_packed, query_offsets, documents_packed, document_offsets,
            (pair_indices // C).contiguous(), pair_indices.contiguous(), max_q)


def pack_documents(doc_emb, doc_lengths):
    """Pack padded documents ``[Nb, Ld, D]`` with lengths ``[Nb]`` into the
    ``(documents [total, D], document_offsets [Nb + 1] int32)`` inputs of the
    contrastive functions: the device form of the ``torch.cat`` of valid rows
    and offset prefix sum that callers write before a contrastive call
    (reference README.md:184-191).  Not in ``__all__``, which stays the
    reference's list.  One HIP copy per document; lengths are
    clamped to ``[0, Ld]`` and one device-to-host copy brings back the total
    row count (the output size)."""
    if doc_emb.dim() != 3:
        raise ValueError(f"doc_emb must be 3-D [Nb, Ld, D]; got shape {tuple(doc_emb.shape)}")
    Nb, Ld, D = doc_emb.shape
    if doc_lengths.shape != (Nb,):
        raise ValueError(f"doc_lengths must have shape [Nb={Nb}]; got {tuple(doc_lengths.shape)}")
    lens = doc_lengths.to(device=doc_emb.device, dtype=torch.int32).clamp(0, Ld)
    offsets = torch.zeros(Nb + 1, dtype=torch.int32, device=doc_emb.device)
    offsets[1:] = lens.cumsum(0)
    total = int(offsets[-1])
    packed = ops.maxsim_pack_padded_rows(doc_emb.reshape(Nb * Ld, D), lens, offsets, Ld, total)
    return packed, offsets


# ---------------------------------------------------------------------------
# Contrastive (all pairs)
# ---------------------------------------------------------------------------
def _check_targets(t: np.ndarray, nb: int) -> None:
    bad = np.flatnonzero((t < 0) | (t >= nb))
    if bad.size:
        i = int(bad[0])
        raise ValueError(f"targets[{i}] = {int(t[i])} out of range [0, {nb})")


@torch.compiler.disable
def _checked_contrastive(queries, documents, document_offsets, launch, targets=None):
    """Validate a contrastive call and return ``launch()``.

    The offsets (and the cross-entropy targets, when given) travel to pinned
    host memory by asynchronous copies queued ahead of the kernels, and
    ``launch()`` queues the kernels before the host waits for those copies,
    so the GPU is never idle while the host checks them.  Invalid offsets or
    targets raise the same errors as before; the kernels already queued are
    safe with any offsets and targets (documents with an invalid range give
    NaN, a target outside ``[0, Nb)`` a NaN loss, nothing is read out of
    range) and their results are dropped."""
    _check_contrastive(queries, documents, document_offsets)
    flat = document_offsets.detach().reshape(-1)
    nb = flat.numel() - 1
    if not _HOST_CHECKS and flat.is_cuda:
        if documents.shape[0] == 0:
            raise ValueError("documents must not be empty (document_offsets has >= 1 document)")
        return launch()
    if not flat.is_cuda:  # host tensors: check first (the operators reject them anyway)
        _check_offsets(flat.numpy().astype(np.int64), documents.shape[0])
        if targets is not None:
            _check_targets(_to_host(targets)[0], nb)
        return launch()
    # The copy stays on the current stream: a small copy runs as a blit
    # kernel, and on a side stream it would wait for a free CU until the
    # contrastive forward (one large workgroup per CU) ends, keeping the host
    # from queueing the next launches in time.  In the stream it costs a few
    # microseconds between the previous step's work and the forward.
    host = torch.empty(flat.shape, dtype=flat.dtype, pin_memory=True)
    host.copy_(flat, non_blocking=True)
    host_t = None
    if targets is not None:
        tflat = targets.detach().reshape(-1)
        host_t = torch.empty(tflat.shape, dtype=tflat.dtype, pin_memory=True)
        host_t.copy_(tflat, non_blocking=True)
    copied = torch.cuda.Event()
    copied.record()
    result = launch()
    copied.synchronize()
    _check_offsets(host.numpy().astype(np.int64), documents.shape[0])
    if host_t is not None:
        _check_targets(host_t.numpy().astype(np.int64), nb)
    return result


def score_contrastive(queries, documents, document_offsets) -> torch.Tensor:
    """Score every query against every packed document.

    Args:
        queries: ``[Nq, Lq, dim]``; documents: ``[total_d_tokens, dim]`` packed;
        document_offsets: ``[Nb + 1]`` CSR offsets.

    Returns:
        ``[Nq, Nb]`` fp32 scores.
    """
    return _checked_contrastive(
        queries, documents, document_offsets,
        lambda: ops.maxsim_contrastive_forward(queries.contiguous(), documents.contiguous(),
                                               document_offsets.to(torch.int32).contiguous()))


def score_contrastive_with_argmax(queries, documents,
                                  document_offsets) -> Tuple[torch.Tensor, torch.Tensor]:
    """As :func:`score_contrastive`, plus int32 argmax ``[Nq, Nb, Lq]``."""
    return _checked_contrastive(
        queries, documents, document_offsets,
        lambda: ops.maxsim_contrastive_forward_with_argmax(
            queries.contiguous(), documents.contiguous(),
            document_offsets.to(torch.int32).contiguous()))


class _ContrastiveFn(torch.autograd.Function):
    """Contrastive forward+argmax / backward pair (reference __init__.py:925-954)."""

    @staticmethod
    def forward(ctx, queries, documents, document_offsets):
        q, d = queries.contiguous(), documents.contiguous()
        offs = document_offsets.to(torch.int32).contiguous()
        scores, argmax = ops.maxsim_contrastive_forward_with_argmax(q, d, offs)
        ctx.save_for_backward(q, d, offs, argmax)
        return scores

    @staticmethod
    def backward(ctx, dscore):
        # The reference returns the fp32 gradients and autograd casts them to
        # the input dtype; the typed operator writes that rounding directly.
        q, d, offs, argmax = ctx.saved_tensors
        dq, dd = ops.maxsim_contrastive_backward_typed(
            dscore.contiguous().to(torch.float32), q, d, offs, argmax)
        return dq, dd, None


def score_contrastive_train(queries, documents, document_offsets) -> torch.Tensor:
    """Differentiable :func:`score_contrastive` (gradients accumulated in fp32)."""
    return _checked_contrastive(
        queries, documents, document_offsets,
        lambda: _ContrastiveFn.apply(queries, documents, document_offsets))


# ---------------------------------------------------------------------------
# Fused contrastive cross-entropy (the training loss of the reference's README)
# ---------------------------------------------------------------------------
_REDUCTIONS = {"none": 0, "mean": 1, "sum": 2}


class _ContrastiveCEFn(torch.autograd.Function):
    """score_contrastive_train + F.cross_entropy(scores / temperature, targets)
    in one autograd node: the forward writes the scores, their argmax and each
    row's log-sum-exp; the backward computes the score gradients inside the
    dQ/dD kernels from those (no dscore tensor, no separate softmax pass)."""

    @staticmethod
    def forward(ctx, queries, documents, document_offsets, targets, inv_t, reduction):
        q, d = queries.contiguous(), documents.contiguous()
        offs = document_offsets.to(torch.int32).contiguous()
        scores, argmax = ops.maxsim_contrastive_forward_with_argmax(q, d, offs)
        tgt = _targets_i32(targets, offs.numel() - 1)
        lse, loss = ops.maxsim_cross_entropy_forward(scores, tgt, inv_t, reduction)
        if tgt is None:
            ctx.save_for_backward(q, d, offs, argmax, scores, lse)
        else:
            ctx.save_for_backward(q, d, offs, argmax, scores, lse, tgt)
        ctx.inv_t = inv_t
        ctx.reduction = reduction
        ctx.mark_non_differentiable(scores)
        return loss

    @staticmethod
    def backward(ctx, grad_loss):
        saved = ctx.saved_tensors
        q, d, offs, argmax, scores, lse = saved[:6]
        tgt = saved[6] if len(saved) > 6 else None
        dq, dd = ops.maxsim_contrastive_cross_entropy_backward(
            grad_loss.contiguous().to(torch.float32), scores, lse, tgt, ctx.inv_t,
            ctx.reduction, q, d, offs, argmax)
        return dq, dd, None, None, None, None


def _check_cross_entropy(queries, documents, document_offsets, targets, temperature,
                         reduction):
    """Argument checks of the fused contrastive cross-entropy; returns
    ``(1 / temperature, reduction code)``."""
    _check_contrastive(queries, documents, document_offsets)
    if reduction not in _REDUCTIONS:
        raise ValueError(f"reduction must be 'mean', 'sum' or 'none'; got {reduction!r}")
    temperature = float(temperature)
    if not (temperature > 0.0 and np.isfinite(temperature)):
        raise ValueError(f"temperature must be finite and > 0; got {temperature}")
    Nq, Nb = queries.shape[0], document_offsets.numel() - 1
    if targets is None:
        if Nq > Nb:
            raise ValueError(
                f"diagonal targets need Nq <= Nb; got Nq={Nq}, Nb={Nb} (pass targets)")
    else:
        _require_index("targets", targets)
        if targets.dim() != 1 or targets.shape[0] != Nq:
            raise ValueError(f"targets must have shape [Nq={Nq}]; got {tuple(targets.shape)}")
        _require_one_device(queries=queries, targets=targets)
        # the values are checked by _checked_contrastive, overlapped with
        # the kernels (host checks on) or by the kernels (NaN loss, off)
    return 1.0 / temperature, _REDUCTIONS[reduction]


def _targets_i32(targets, nb: int):
    """int32 targets for the kernels.  int64 values outside ``[0, Nb)`` become
    -1 on the device before the narrowing, so that with host checks off a
    value such as 2**32 + 1 gives the documented NaN loss instead of wrapping
    to a valid class (no host wait: capturable)."""
    if targets is None:
        return None
    if targets.dtype == torch.int64:
        targets = torch.where((targets >= 0) & (targets < nb), targets,
                              torch.full_like(targets, -1))
    return targets.to(torch.int32).contiguous()


def score_contrastive_cross_entropy(queries, documents, document_offsets, targets=None, *,
                                    temperature: float = 1.0,
                                    reduction: str = "mean") -> torch.Tensor:
    """The contrastive training loss in one call:
    ``F.cross_entropy(score_contrastive_train(queries, documents,
    document_offsets) / temperature, targets, reduction=reduction)``, the
    recipe of the reference's README (README.md:193-205), with the softmax
    gradient fused into the backward kernels.

    Args:
        queries, documents, document_offsets: as :func:`score_contrastive`.
        targets: ``[Nq]`` int32/int64 class (document) per query, or None for
            the diagonal (query i's positive is document i; needs Nq <= Nb).
        temperature: the scores are divided by it (> 0).
        reduction: ``"mean"`` (default), ``"sum"`` or ``"none"`` (``[Nq]``).

    Returns:
        fp32 loss (0-dim, or ``[Nq]`` for ``"none"``); differentiable with
        respect to queries and documents (gradients in their dtype).  Not in
        the reference's ``__all__``; its users call torch's cross-entropy.
    """
    inv_t, red = _check_cross_entropy(queries, documents, document_offsets, targets,
                                      temperature, reduction)
    return _checked_contrastive(
        queries, documents, document_offsets,
        lambda: _ContrastiveCEFn.apply(queries, documents, document_offsets, targets, inv_t, red),
        targets=targets)


def score_contrastive_cross_entropy_value_and_grad(queries, documents, document_offsets,
                                                   targets=None, *, temperature: float = 1.0,
                                                   reduction: str = "mean", grad_loss=None):
    """:func:`score_contrastive_cross_entropy` and its gradients in one call,
    without autograd: returns ``(loss, dqueries, ddocuments)``.

    The same kernels as ``score_contrastive_cross_entropy(...).backward()``
    (forward with argmax, the loss with each row's log-sum-exp, the fused
    backward), launched back to back.  The autograd engine's per-backward
    host cost (a thread hand-off and graph walk, tens of microseconds) is
    larger than all the kernels of a small batch; training loops that apply
    the gradients themselves avoid it here.

    Args:
        queries, documents, document_offsets, targets, temperature,
            reduction: as :func:`score_contrastive_cross_entropy`
            (``requires_grad`` is ignored; nothing is recorded).
        grad_loss: upstream gradient of the loss, fp32 on the inputs' device:
            one value (``"mean"``/``"sum"``) or ``[Nq]`` (``"none"``); None
            means 1 (``[Nq]`` ones for ``"none"``).

    Returns:
        ``loss`` (fp32, 0-dim or ``[Nq]``) and the gradients of
        ``(loss * grad_loss).sum()`` with respect to queries and documents,
        in their dtype (fp32 sums rounded once).
    """
    inv_t, red = _check_cross_entropy(queries, documents, document_offsets, targets,
                                      temperature, reduction)
    nq = queries.shape[0]
    if grad_loss is not None:
        if not isinstance(grad_loss, torch.Tensor) or grad_loss.dtype != torch.float32:
            raise TypeError("grad_loss must be a float32 tensor")
        _require_one_device(queries=queries, grad_loss=grad_loss)
        want = nq if reduction == "none" else 1
        if grad_loss.numel() != want:
            raise ValueError(f"grad_loss must hold {want} value(s); got {grad_loss.numel()}")

    def launch():
        q, d = queries.detach().contiguous(), documents.detach().contiguous()
        offs = document_offsets.to(torch.int32).contiguous()
        scores, argmax = ops.maxsim_contrastive_forward_with_argmax(q, d, offs)
        tgt = _targets_i32(targets, offs.numel() - 1)
        lse, loss = ops.maxsim_cross_entropy_forward(scores, tgt, inv_t, red)
        g = grad_loss
        if g is None:
            g = torch.ones(loss.shape, dtype=torch.float32, device=loss.device)
        dq, dd = ops.maxsim_contrastive_cross_entropy_backward(
            g.detach().reshape(loss.shape).contiguous(), scores, lse, tgt, inv_t, red, q, d,
            offs, argmax)
        return loss, dq, dd

    with torch.no_grad():
        return _checked_contrastive(queries, documents, document_offsets, launch,
                                    targets=targets)
