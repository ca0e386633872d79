"""Pure-PyTorch MaxSim baselines exported for API parity with the reference
package (torch-ext/maxsim/reference.py; exported from __init__.py:24-35).

They materialise the full similarity matrix in fp32 with ordinary torch ops
(matmul / einsum + max), so they are slow and memory hungry by design -- the
"naive PyTorch" a user would write, and the baseline the reference's
benchmarks compare against (scripts/bench_matrix.py:302-313, 402-413).
They follow ``torch.max`` semantics (first index on ties; NaN propagates),
run on whatever device their inputs live on, and are NOT used by the HIP
operators in :mod:`maxsim_amd._ops`.
"""

from __future__ import annotations

from typing import Tuple

import torch

__all__ = [
    "maxsim_reference",
    "maxsim_reference_with_argmax",
    "score_pairs_packed_reference",
    "score_pairs_packed_with_argmax_reference",
    "score_pairs_packed_backward_reference",
    "score_candidates_padded_reference",
    "score_candidates_padded_with_argmax_reference",
    "score_candidates_padded_backward_reference",
    "score_contrastive_reference",
    "score_contrastive_with_argmax_reference",
    "score_contrastive_backward_reference",
]


def _host_ints(t: torch.Tensor) -> list:
    return t.detach().to("cpu", torch.int64).tolist()


def maxsim_reference_with_argmax(q: torch.Tensor, d: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """One pair: ``q [Lq, dim]``, ``d [Ld, dim]`` -> (fp32 scalar score,
    int32 ``[Lq]`` argmax)."""
    best, where = torch.max(q.float() @ d.float().t(), dim=-1)
    return best.sum(), where.to(torch.int32)


def maxsim_reference(q: torch.Tensor, d: torch.Tensor) -> torch.Tensor:
    """One pair: fp32 scalar ``sum_i max_j <q_i, d_j>``."""
    return maxsim_reference_with_argmax(q, d)[0]


# ---- packed ---------------------------------------------------------------
def score_pairs_packed_with_argmax_reference(queries, query_offsets, documents,
                                             document_offsets, pair_query_ids,
                                             pair_document_ids, max_q_len: int):
    qo, do = _host_ints(query_offsets), _host_ints(document_offsets)
    qi, di = _host_ints(pair_query_ids), _host_ints(pair_document_ids)
    scores = torch.empty(len(qi), dtype=torch.float32, device=queries.device)
    argmax = torch.zeros(len(qi), max_q_len, dtype=torch.int32, device=queries.device)
    for k, (a, b) in enumerate(zip(qi, di)):
        s, am = maxsim_reference_with_argmax(queries[qo[a]:qo[a + 1]], documents[do[b]:do[b + 1]])
        scores[k] = s
        argmax[k, :am.numel()] = am
    return scores, argmax


def score_pairs_packed_reference(queries, query_offsets, documents, document_offsets,
                                 pair_query_ids, pair_document_ids) -> torch.Tensor:
    qo = _host_ints(query_offsets)
    mql = max([b - a for a, b in zip(qo, qo[1:])] or [1])
    return score_pairs_packed_with_argmax_reference(
        queries, query_offsets, documents, document_offsets, pair_query_ids,
        pair_document_ids, mql)[0]


def score_pairs_packed_backward_reference(dscore, queries, query_offsets, documents,
                                          document_offsets, pair_query_ids,
                                          pair_document_ids, argmax):
    """Route ``dscore[k]`` through the saved argmax; fp32 grads."""
    qo, do = _host_ints(query_offsets), _host_ints(document_offsets)
    qi, di = _host_ints(pair_query_ids), _host_ints(pair_document_ids)
    qf, df, g = queries.float(), documents.float(), dscore.float()
    dq, dd = torch.zeros_like(qf), torch.zeros_like(df)
    for k, (a, b) in enumerate(zip(qi, di)):
        lq, ld = qo[a + 1] - qo[a], do[b + 1] - do[b]
        j = argmax[k, :lq].to(torch.int64)
        ok = (j >= 0) & (j < ld)
        rows_q = torch.arange(qo[a], qo[a + 1], device=qf.device)[ok]
        rows_d = do[b] + j[ok]
        dq.index_add_(0, rows_q, g[k] * df[rows_d])
        dd.index_add_(0, rows_d, g[k] * qf[rows_q])
    return dq, dd


# ---- padded ---------------------------------------------------------------
def _padded_sim(queries, documents, doc_lengths):
    Ld = documents.shape[2]
    sim = torch.einsum("bid,bcjd->bcij", queries.float(), documents.float())
    pad = torch.arange(Ld, device=sim.device)[None, None, :] >= doc_lengths.to(sim.device)[:, :, None]
    return sim.masked_fill(pad[:, :, None, :], float("-inf"))


def score_candidates_padded_with_argmax_reference(queries, documents, query_lengths,
                                                  doc_lengths):
    """``[B, Lq, D]`` x ``[B, C, Ld, D]`` -> (``[B, C]`` fp32, ``[B, C, Lq]`` int32)."""
    best, where = _padded_sim(queries, documents, doc_lengths).max(dim=-1)
    Lq = queries.shape[1]
    qpad = torch.arange(Lq, device=best.device)[None, :] >= query_lengths.to(best.device)[:, None]
    best = best.masked_fill(qpad[:, None, :], 0.0)
    where = where.masked_fill(qpad[:, None, :], 0)
    return best.sum(dim=-1), where.to(torch.int32)


def score_candidates_padded_reference(queries, documents, query_lengths, doc_lengths):
    return score_candidates_padded_with_argmax_reference(
        queries, documents, query_lengths, doc_lengths)[0]


def score_candidates_padded_backward_reference(dscore, queries, documents, query_lengths,
                                               doc_lengths, argmax):
    """Route ``dscore[b, c]`` through ``argmax [B, C, Lq]``; fp32 grads."""
    B, C, Ld, D = documents.shape
    Lq = queries.shape[1]
    qf, df, g = queries.float(), documents.float(), dscore.float()
    j = argmax.to(torch.int64)
    valid = (torch.arange(Lq, device=j.device)[None, None, :] < query_lengths.to(j.device)[:, None, None])
    valid &= (j >= 0) & (j < doc_lengths.to(j.device)[:, :, None])
    w = g[:, :, None] * valid.float()                                   # [B, C, Lq]
    jc = j.clamp(0, Ld - 1)
    picked = torch.gather(df, 2, jc[..., None].expand(B, C, Lq, D))      # [B, C, Lq, D]
    dq = (w[..., None] * picked).sum(dim=1)
    dd = torch.zeros_like(df)
    dd.scatter_add_(2, jc[..., None].expand(B, C, Lq, D), w[..., None] * qf[:, None])
    return dq, dd


# ---- contrastive ----------------------------------------------------------
def score_contrastive_with_argmax_reference(queries, documents, document_offsets):
    """``[Nq, Lq, D]`` x packed docs -> (``[Nq, Nb]`` fp32, ``[Nq, Nb, Lq]`` int32)."""
    offs = _host_ints(document_offsets)
    Nq, Lq, _ = queries.shape
    nb = len(offs) - 1
    scores = torch.empty(Nq, nb, dtype=torch.float32, device=queries.device)
    argmax = torch.zeros(Nq, nb, Lq, dtype=torch.int32, device=queries.device)
    qf = queries.float()
    for b in range(nb):
        best, where = torch.einsum("qid,jd->qij", qf, documents[offs[b]:offs[b + 1]].float()).max(dim=-1)
        scores[:, b] = best.sum(dim=-1)
        argmax[:, b] = where.to(torch.int32)
    return scores, argmax


def score_contrastive_reference(queries, documents, document_offsets):
    return score_contrastive_with_argmax_reference(queries, documents, document_offsets)[0]


def score_contrastive_backward_reference(dscore, queries, documents, document_offsets, argmax):
    """Route ``dscore[q, b]`` through ``argmax [Nq, Nb, Lq]``; fp32 grads."""
    offs = torch.tensor(_host_ints(document_offsets), device=documents.device)
    qf, df, g = queries.float(), documents.float(), dscore.float()
    Nq, Lq, D = qf.shape
    lens = (offs[1:] - offs[:-1])[None, :, None]
    j = argmax.to(torch.int64)
    ok = (j >= 0) & (j < lens)
    rows = (offs[:-1][None, :, None] + j.clamp(min=0)).clamp(max=max(df.shape[0] - 1, 0))
    w = g[:, :, None] * ok.float()                                       # [Nq, Nb, Lq]
    dq = torch.einsum("qbi,qbid->qid", w, df[rows])
    dd = torch.zeros_like(df)
    contrib = (w[..., None] * qf[:, None, :, :]).reshape(-1, D)
    dd.index_add_(0, rows.reshape(-1), contrib)
    return dq, dd
