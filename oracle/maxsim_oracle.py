"""CPU oracle for MaxSim -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this module, and only as the checker; the product
(``maxsim_amd``) never imports or calls it.

It restates, in numpy float64, the semantics the reference's kernels and
tests fix for the operator family:

* score(q, d) = sum over valid query tokens i of max over valid document
  tokens j of <q_i, d_j>                     (reference.py:20-32, README.md:26-36)
* argmax: ascending j with a strict ``>`` -> the FIRST maximal index wins
  ties                                        (reference.py:35-47, maxsim.cu:412-443)
* a NaN similarity never wins; a query token whose similarities are all NaN
  contributes -inf and argmax 0               (maxsim.cu `v > max`, test_nan_inf.py:33-92)
* argmax slots beyond a pair's query length are 0 (maxsim.cu:543-547, 2005-2009)
* backward routes g = dscore[pair] to dq[i] += g * d[j], dd[j] += g * q[i]
  with j = argmax[pair, i], skipping j outside [0, Ld)
                                              (reference.py:141-183, 186-229, 284-323)
* gradients and scores are fp32              (torch_binding.h:83-85, 157-159)

Inputs may be any float arrays (bf16/fp16 values should be passed already
rounded to that precision, as the kernel sees them); all arithmetic is float64
and results are rounded to fp32 at the end.

How each function is pinned (tests/test_oracle.py): the known-answer cases
of the reference's tests (single pair, all-identical rows -> argmax 0, pad
garbage ignored, zero dscore, empty pair list), closed forms (score(q, q) =
Lq for distinct unit rows), torch's own einsum + max(dim) and its autograd on
finite inputs, NaN/inf contracts, cross-surface identities, and planted
mistakes that those checks must catch.
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "pair_forward",
    "contrastive_forward",
    "padded_forward",
    "packed_forward",
    "contrastive_backward",
    "padded_backward",
    "packed_backward",
    "pack_padded",
    "cross_entropy",
]


def _as64(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float64)


def _sim(q: np.ndarray, d: np.ndarray) -> np.ndarray:
    """q @ d.T in float64 such that bitwise-identical document rows get
    bitwise-identical similarities.  A BLAS gemm does not promise that (rows
    that land in different micro-kernel tiles are summed in different
    orders), and exact ties must be broken by index, so the rows are
    de-duplicated first and the products mapped back."""
    if d.shape[0] == 0:
        return np.zeros((q.shape[0], 0))
    uniq, inv = np.unique(d, axis=0, return_inverse=True)
    return (q @ uniq.T)[:, inv.reshape(-1)]


def _row_max_first(sim: np.ndarray):
    """Per-row (max, first argmax) with NaN treated as never winning."""
    clean = np.where(np.isnan(sim), -np.inf, sim)
    idx = np.argmax(clean, axis=1) if clean.shape[1] else np.zeros(clean.shape[0], np.int64)
    best = clean[np.arange(clean.shape[0]), idx]
    return best, idx


def pair_forward(q, d):
    """One pair (reference.py:20-47): ``q [Lq, D]``, ``d [Ld, D]`` ->
    (float score, int32 argmax [Lq])."""
    q, d = _as64(q), _as64(d)
    best, idx = _row_max_first(_sim(q, d))
    return float(np.float32(best.sum())), idx.astype(np.int32)


def contrastive_forward(queries, documents, offsets):
    """All pairs (reference.py:232-281): ``[Nq, Lq, D]`` x packed ``[T, D]``
    with CSR ``offsets [Nb+1]`` -> (fp32 ``[Nq, Nb]``, int32 ``[Nq, Nb, Lq]``)."""
    q = _as64(queries)
    d = _as64(documents)
    offs = np.asarray(offsets, dtype=np.int64)
    Nq, Lq, D = q.shape
    Nb = offs.size - 1
    flat = q.reshape(Nq * Lq, D)
    scores = np.empty((Nq, Nb), np.float64)
    argmax = np.zeros((Nq, Nb, Lq), np.int32)
    for b in range(Nb):
        best, idx = _row_max_first(_sim(flat, d[offs[b]:offs[b + 1]]))
        scores[:, b] = best.reshape(Nq, Lq).sum(axis=1)
        argmax[:, b, :] = idx.reshape(Nq, Lq)
    return scores.astype(np.float32), argmax


def padded_forward(queries, documents, query_lengths, doc_lengths):
    """Padded rerank (reference.py:112-138, 326-361): ``[B, Lq, D]`` x
    ``[B, C, Ld, D]`` -> (fp32 ``[B, C]``, int32 ``[B, C, Lq]``).  Rows past
    the lengths are never read; argmax slots past ``query_lengths[b]`` are 0."""
    q = _as64(queries)
    d = _as64(documents)
    ql = np.asarray(query_lengths, dtype=np.int64)
    dl = np.asarray(doc_lengths, dtype=np.int64)
    B, Lq, _ = q.shape
    C = d.shape[1]
    scores = np.empty((B, C), np.float64)
    argmax = np.zeros((B, C, Lq), np.int32)
    for b in range(B):
        qb = q[b, :ql[b]]
        for c in range(C):
            best, idx = _row_max_first(_sim(qb, d[b, c, :dl[b, c]]))
            scores[b, c] = best.sum()
            argmax[b, c, :ql[b]] = idx
    return scores.astype(np.float32), argmax


def packed_forward(queries, query_offsets, documents, document_offsets,
                   pair_query_ids, pair_document_ids, max_q_len):
    """Packed pairs (reference.py:50-109) -> (fp32 ``[P]``, int32 ``[P, max_q_len]``)."""
    q = _as64(queries)
    d = _as64(documents)
    qo = np.asarray(query_offsets, dtype=np.int64)
    do = np.asarray(document_offsets, dtype=np.int64)
    qi = np.asarray(pair_query_ids, dtype=np.int64)
    di = np.asarray(pair_document_ids, dtype=np.int64)
    P = qi.size
    scores = np.empty(P, np.float64)
    argmax = np.zeros((P, max_q_len), np.int32)
    for k in range(P):
        qs, qe = qo[qi[k]], qo[qi[k] + 1]
        best, idx = _row_max_first(_sim(q[qs:qe], d[do[di[k]]:do[di[k] + 1]]))
        scores[k] = best.sum()
        argmax[k, :qe - qs] = idx
    return scores.astype(np.float32), argmax


def contrastive_backward(dscore, queries, documents, offsets, argmax):
    """reference.py:284-323 -> (fp32 dq ``[Nq, Lq, D]``, fp32 dd ``[T, D]``)."""
    g = _as64(dscore)
    q = _as64(queries)
    d = _as64(documents)
    offs = np.asarray(offsets, dtype=np.int64)
    am = np.asarray(argmax, dtype=np.int64)
    Nq, Lq, D = q.shape
    Nb = offs.size - 1
    dq = np.zeros_like(q)
    dd = np.zeros_like(d)
    lens = (offs[1:] - offs[:-1])[None, :, None]
    ok = (am >= 0) & (am < lens)
    rows = offs[:-1][None, :, None] + np.where(ok, am, 0)
    w = np.where(ok, g[:, :, None], 0.0)                       # [Nq, Nb, Lq]
    dq += np.einsum("qbi,qbid->qid", w, d[rows])
    np.add.at(dd, rows.reshape(-1), (w[..., None] * q[:, None, :, :]).reshape(-1, D))
    return dq.astype(np.float32), dd.astype(np.float32)


def padded_backward(dscore, queries, documents, query_lengths, doc_lengths, argmax):
    """reference.py:141-183 -> (fp32 dq ``[B, Lq, D]``, fp32 dd ``[B, C, Ld, D]``)."""
    g = _as64(dscore)
    q = _as64(queries)
    d = _as64(documents)
    ql = np.asarray(query_lengths, dtype=np.int64)
    dl = np.asarray(doc_lengths, dtype=np.int64)
    am = np.asarray(argmax, dtype=np.int64)
    B, C, Ld, D = d.shape
    dq = np.zeros_like(q)
    dd = np.zeros_like(d)
    for b in range(B):
        for c in range(C):
            for i in range(ql[b]):
                j = am[b, c, i]
                if j < 0 or j >= dl[b, c]:
                    continue
                dq[b, i] += g[b, c] * d[b, c, j]
                dd[b, c, j] += g[b, c] * q[b, i]
    return dq.astype(np.float32), dd.astype(np.float32)


def packed_backward(dscore, queries, query_offsets, documents, document_offsets,
                    pair_query_ids, pair_document_ids, argmax):
    """reference.py:186-229 -> (fp32 dq ``[Tq, D]``, fp32 dd ``[Td, D]``)."""
    g = _as64(dscore)
    q = _as64(queries)
    d = _as64(documents)
    qo = np.asarray(query_offsets, dtype=np.int64)
    do = np.asarray(document_offsets, dtype=np.int64)
    qi = np.asarray(pair_query_ids, dtype=np.int64)
    di = np.asarray(pair_document_ids, dtype=np.int64)
    am = np.asarray(argmax, dtype=np.int64)
    dq = np.zeros_like(q)
    dd = np.zeros_like(d)
    for k in range(qi.size):
        qs, qe = qo[qi[k]], qo[qi[k] + 1]
        ds, de = do[di[k]], do[di[k] + 1]
        j = am[k, :qe - qs]
        ok = (j >= 0) & (j < de - ds)
        rq = np.arange(qs, qe)[ok]
        rd = ds + j[ok]
        np.add.at(dq, rq, g[k] * d[rd])
        np.add.at(dd, rd, g[k] * q[rq])
    return dq.astype(np.float32), dd.astype(np.float32)


def pack_padded(queries, documents, query_lengths, doc_lengths):
    """_pack_padded (torch-ext/maxsim/__init__.py:516-620): padded ``[B, Lq, D]``
    / ``[B, C, Ld, D]`` -> (queries_packed, query_offsets, documents_packed,
    document_offsets, pair_query_ids, pair_document_ids, max_q_len).  Rows
    keep their values (no arithmetic); the valid rows of each query and each
    candidate, in row-major (b, c) order; offsets are the prefix sums of the
    lengths; pair k = (b, c) = (k // C, k)."""
    q = np.asarray(queries)
    d = np.asarray(documents)
    ql = np.asarray(query_lengths, dtype=np.int64)
    dl = np.asarray(doc_lengths, dtype=np.int64)
    B, Lq, D = q.shape
    _, C, Ld, _ = d.shape
    qmask = np.arange(Lq)[None, :] < ql[:, None]
    dmask = np.arange(Ld)[None, None, :] < dl[:, :, None]
    qp = q.reshape(B * Lq, D)[qmask.reshape(-1)]
    dp = d.reshape(B * C * Ld, D)[dmask.reshape(-1)]
    qo = np.concatenate([[0], np.cumsum(ql)]).astype(np.int64)
    do = np.concatenate([[0], np.cumsum(dl.reshape(-1))]).astype(np.int64)
    pairs = np.arange(B * C, dtype=np.int64)
    return qp, qo, dp, do, pairs // max(C, 1), pairs, int(ql.max()) if B else 0


def cross_entropy(scores, targets=None, inv_temperature=1.0, reduction="mean"):
    """The loss of the reference's training recipe, F.cross_entropy(scores /
    temperature, targets) (README.md:193-205), and its gradient with respect
    to the scores: ``(loss, dscore)`` in float64, with ``targets`` None for
    the diagonal.  dscore[q, b] = w_q * (softmax(s * inv_t)[q, b] - [b == t_q])
    * inv_t, w_q = 1 / Nq (mean), 1 (sum) or the row's upstream 1 (none,
    where the loss is per row and dscore is for a sum of the row losses)."""
    s = _as64(scores) * float(inv_temperature)
    Nq, Nb = s.shape
    t = np.arange(Nq) if targets is None else np.asarray(targets, dtype=np.int64)
    m = s.max(axis=1, keepdims=True)
    lse = (m + np.log(np.exp(s - m).sum(axis=1, keepdims=True)))[:, 0]
    rows = lse - s[np.arange(Nq), t]
    p = np.exp(s - lse[:, None])
    onehot = np.zeros_like(p)
    onehot[np.arange(Nq), t] = 1.0
    w = 1.0 / Nq if reduction == "mean" else 1.0
    dscore = (p - onehot) * (w * float(inv_temperature))
    loss = rows if reduction == "none" else (rows.mean() if reduction == "mean" else rows.sum())
    return loss, dscore
