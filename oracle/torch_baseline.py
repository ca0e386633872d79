"""CPU baseline for bench.py -- TEST/MEASUREMENT INFRASTRUCTURE ONLY.

A restatement of the reference's naive PyTorch MaxSim, the formulation its
benchmarks compare against (scripts/bench_matrix.py:302-313 contrastive,
:402-413 padded): materialise the similarity with ``einsum`` in fp32, take
``max`` over document tokens, sum over query tokens; backward through
autograd.  Padded document slots are masked to -inf (the correct semantics;
the reference's contrastive baseline zero-pads, which only changes results
when every real similarity is negative).

Only bench.py's ``cpu_baseline`` leg uses this module.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def pad_documents(documents: torch.Tensor, lengths: list[int]) -> tuple[torch.Tensor, torch.Tensor]:
    """Packed ``[T, D]`` -> padded ``[Nb, Ld_max, D]`` plus a validity mask."""
    nb, ld = len(lengths), max(lengths)
    out = documents.new_zeros((nb, ld, documents.shape[1]))
    mask = torch.zeros(nb, ld, dtype=torch.bool)
    pos = 0
    for b, n in enumerate(lengths):
        out[b, :n] = documents[pos:pos + n]
        mask[b, :n] = True
        pos += n
    return out, mask


def contrastive_scores(q: torch.Tensor, docs_padded: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
    """``[nq, Lq, D]`` x ``[Nb, Ld, D]`` -> ``[nq, Nb]`` fp32."""
    sim = torch.einsum("qid,njd->qnij", q, docs_padded)
    sim = sim.masked_fill(~mask[None, :, None, :], float("-inf"))
    return sim.max(dim=-1).values.sum(dim=-1)


def contrastive_step(q_rows: torch.Tensor, row_ids: torch.Tensor, docs_padded: torch.Tensor,
                     mask: torch.Tensor, nq_total: int) -> float:
    """One fwd + CE(diagonal) + bwd over a subset of query rows (CE is
    row-separable, so a row subset is exact for those rows).  Returns the
    partial loss."""
    q = q_rows.detach().clone().requires_grad_(True)
    d = docs_padded.detach().clone().requires_grad_(True)
    scores = contrastive_scores(q, d, mask)
    loss = F.cross_entropy(scores, row_ids, reduction="sum") / nq_total
    loss.backward()
    return float(loss.detach())


def padded_scores(q: torch.Tensor, d: torch.Tensor, qlen: torch.Tensor, dlen: torch.Tensor) -> torch.Tensor:
    """Reference padded baseline: ``[B, Lq, D]`` x ``[B, C, Ld, D]`` -> ``[B, C]``."""
    Lq, Ld = q.shape[1], d.shape[2]
    sim = torch.einsum("bid,bcjd->bcij", q, d)
    dmask = torch.arange(Ld)[None, None, :] < dlen[:, :, None]
    sim = sim.masked_fill(~dmask[:, :, None, :], float("-inf"))
    best = sim.max(dim=-1).values
    qmask = torch.arange(Lq)[None, :] < qlen[:, None]
    return best.masked_fill(~qmask[:, None, :], 0.0).sum(dim=-1)


def padded_scores_with_argmax(q: torch.Tensor, d: torch.Tensor, qlen: torch.Tensor,
                              dlen: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """As :func:`padded_scores`, plus the argmax ``[B, C, Lq]`` (0 beyond a
    query's length)."""
    Lq, Ld = q.shape[1], d.shape[2]
    sim = torch.einsum("bid,bcjd->bcij", q, d)
    dmask = torch.arange(Ld)[None, None, :] < dlen[:, :, None]
    sim = sim.masked_fill(~dmask[:, :, None, :], float("-inf"))
    best, idx = sim.max(dim=-1)
    qmask = torch.arange(Lq)[None, :] < qlen[:, None]
    return (best.masked_fill(~qmask[:, None, :], 0.0).sum(dim=-1),
            idx.masked_fill(~qmask[:, None, :], 0).to(torch.int32))


def packed_step(q: torch.Tensor, qoff: torch.Tensor, d: torch.Tensor, doff: torch.Tensor,
                qids: torch.Tensor, dids: torch.Tensor, dscore: torch.Tensor,
                budget: int = 1 << 25) -> tuple[torch.Tensor, torch.Tensor]:
    """Packed pairs forward + backward with upstream ``dscore [P]``: pairs in
    order of document length, gathered into padded chunks of at most
    ``budget`` similarity entries (-inf past a document, 0 past a query),
    einsum + max + sum, autograd accumulating dQ and dD over the chunks.
    Returns ``(dq, dd)``."""
    qg = q.detach().clone().requires_grad_(True)
    dg = d.detach().clone().requires_grad_(True)
    ql = (qoff[1:] - qoff[:-1]).long()
    dl = (doff[1:] - doff[:-1]).long()
    qids, dids = qids.long(), dids.long()
    order = torch.argsort(dl[dids], stable=True)
    lq_max = int(ql.max())
    P, c = order.numel(), 0
    while c < P:
        # the chunk grows while n * Lq_max * Ld (Ld of its last, longest pair) fits the budget
        ld_last = int(dl[dids[order[min(P - 1, c)]]])
        n = max(1, min(P - c, budget // max(1, lq_max * ld_last)))
        idx = order[c:c + n]
        qi, di = qids[idx], dids[idx]
        Lq, Ld = int(ql[qi].max()), int(dl[di].max())
        qmask = torch.arange(Lq)[None, :] < ql[qi][:, None]
        dmask = torch.arange(Ld)[None, :] < dl[di][:, None]
        qrow = torch.where(qmask, qoff[qi].long()[:, None] + torch.arange(Lq)[None, :], 0)
        drow = torch.where(dmask, doff[di].long()[:, None] + torch.arange(Ld)[None, :], 0)
        sim = torch.einsum("nid,njd->nij", qg[qrow], dg[drow])
        sim = sim.masked_fill(~dmask[:, None, :], float("-inf"))
        s = sim.max(dim=-1).values.masked_fill(~qmask, 0.0).sum(dim=-1)
        (s * dscore[idx]).sum().backward()
        c += n
    return qg.grad, dg.grad
