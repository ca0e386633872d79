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
