"""Padded -> packed conversion on the GPU (reference torch-ext/maxsim/__init__.py
:516-620, ``_pack_padded``) against the CPU oracle's restatement: the packed
rows are bit-identical copies, the offsets and pair ids match, and scoring the
packed pairs gives the padded scores."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import maxsim_amd
from maxsim_amd._ops import ops
from oracle import maxsim_oracle as oracle

from ._helpers import DEVICE, npi

pytestmark = pytest.mark.gpu

CASES = [
    # B, C, Lq, Ld, dim, dtype  (row bytes -> copy unit)
    pytest.param(3, 5, 32, 100, 64, torch.bfloat16, id="bf16-dim64-16B"),
    pytest.param(2, 4, 40, 33, 20, torch.bfloat16, id="bf16-dim20-8B"),
    pytest.param(2, 3, 9, 17, 3, torch.float16, id="fp16-dim3-2B"),
    pytest.param(2, 3, 12, 21, 7, torch.float32, id="fp32-dim7-4B"),
    pytest.param(4, 6, 16, 300, 128, torch.float16, id="fp16-dim128-long"),
    pytest.param(1, 1, 1, 1, 16, torch.float32, id="smallest"),
]


def _inputs(B, C, Lq, Ld, dim, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Lq, dim, generator=g).to(dtype)
    d = torch.randn(B, C, Ld, dim, generator=g).to(dtype)
    ql = torch.randint(1, Lq + 1, (B,), generator=g, dtype=torch.int32)
    dl = torch.randint(1, Ld + 1, (B, C), generator=g, dtype=torch.int32)
    return q, d, ql, dl


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    return t.view(torch.int16 if t.element_size() == 2 else torch.int32).numpy()


@pytest.mark.parametrize("B,C,Lq,Ld,dim,dtype", CASES)
def test_pack_padded_matches_oracle(B, C, Lq, Ld, dim, dtype):
    q, d, ql, dl = _inputs(B, C, Lq, Ld, dim, dtype, seed=B * 31 + Ld)
    out = maxsim_amd._pack_padded(q.to(DEVICE), d.to(DEVICE), ql.to(DEVICE), dl.to(DEVICE))
    qp, qo, dp, do, qi, di, mql = out
    # the oracle indexes the same tensors (on the host), so the packed rows
    # must be the same bits
    idx_q = oracle.pack_padded(np.arange(B * Lq).reshape(B, Lq, 1),
                               np.arange(B * C * Ld).reshape(B, C, Ld, 1), ql.numpy(), dl.numpy())
    rows_q, rows_d = idx_q[0][:, 0], idx_q[2][:, 0]
    assert np.array_equal(_bits(qp), _bits(q.reshape(-1, dim)[torch.from_numpy(rows_q)]))
    assert np.array_equal(_bits(dp), _bits(d.reshape(-1, dim)[torch.from_numpy(rows_d)]))
    assert qp.dtype == dtype and dp.dtype == dtype
    assert np.array_equal(npi(qo), idx_q[1]) and np.array_equal(npi(do), idx_q[3])
    assert np.array_equal(npi(qi), idx_q[4]) and np.array_equal(npi(di), idx_q[5])
    assert qo.dtype == torch.int32 and qi.dtype == torch.int32 and mql == idx_q[6]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_packed_scores_of_packed_padded_equal_padded_scores(dtype):
    """score_pairs_packed over _pack_padded's output, reshaped to [B, C], is
    score_candidates_padded bit for bit (the same per-pair kernel work), and
    so is the argmax."""
    B, C, Lq, Ld, dim = 4, 7, 40, 90, 128
    q, d, ql, dl = (t.to(DEVICE) for t in _inputs(B, C, Lq, Ld, dim, dtype, seed=5))
    qp, qo, dp, do, qi, di, mql = maxsim_amd._pack_padded(q, d, ql, dl)
    s_packed, a_packed = maxsim_amd.score_pairs_packed_with_argmax(qp, qo, dp, do, qi, di,
                                                                   max_q_len=mql)
    s_pad, a_pad = maxsim_amd.score_candidates_padded_with_argmax(q, d, ql, dl)
    assert torch.equal(s_packed.view(B, C), s_pad)
    assert torch.equal(a_packed.view(B, C, mql), a_pad[..., :mql])


def test_pack_padded_clamps_lengths_without_validation():
    """validate=False: lengths of 0 or beyond the padded extent are clamped for
    the copy and the offsets alike, so the outputs stay consistent and nothing
    is read or written out of range."""
    B, C, Lq, Ld, dim = 3, 2, 8, 10, 16
    q, d, _, _ = _inputs(B, C, Lq, Ld, dim, torch.float32, seed=9)
    ql = torch.tensor([0, 12, 5], dtype=torch.int32)
    dl = torch.tensor([[3, 0], [25, 10], [-4, 1]], dtype=torch.int32)
    qp, qo, dp, do, qi, di, mql = maxsim_amd._pack_padded(q.to(DEVICE), d.to(DEVICE),
                                                          ql.to(DEVICE), dl.to(DEVICE))
    ref = oracle.pack_padded(q.numpy(), d.numpy(), ql.clamp(0, Lq).numpy(), dl.clamp(0, Ld).numpy())
    assert np.array_equal(qp.cpu().numpy(), ref[0]) and np.array_equal(dp.cpu().numpy(), ref[2])
    assert np.array_equal(npi(qo), ref[1]) and np.array_equal(npi(do), ref[3])
    assert mql == Lq


def test_pack_padded_validate_raises_reference_errors():
    q, d, ql, dl = (t.to(DEVICE) for t in _inputs(2, 3, 8, 10, 16, torch.float16, seed=2))
    with pytest.raises(ValueError, match="query_lengths must all be > 0"):
        maxsim_amd._pack_padded(q, d, torch.zeros_like(ql), dl, validate=True)
    with pytest.raises(ValueError, match="doc_lengths must all be > 0"):
        maxsim_amd._pack_padded(q, d, ql, torch.zeros_like(dl), validate=True)
    with pytest.raises(ValueError, match="exceeds the padded extent"):
        maxsim_amd._pack_padded(q, d, ql, dl + 20, validate=True)
    with pytest.raises(ValueError, match="batch dim mismatch"):
        maxsim_amd._pack_padded(q[:1], d, ql[:1], dl)
    with pytest.raises(ValueError, match="doc_lengths must have shape"):
        maxsim_amd._pack_padded(q, d, ql, dl[:, :2])


def test_pack_operator_respects_packed_capacity():
    """Called directly with a capacity smaller than the lengths need, the
    operator writes only the rows that fit (here the first segment and the
    start of the second) and nothing beyond."""
    dim, max_len = 8, 5
    padded = torch.arange(3 * max_len * dim, dtype=torch.float32, device=DEVICE).view(-1, dim)
    lengths = torch.tensor([2, 4, 3], dtype=torch.int32, device=DEVICE)
    offsets = torch.tensor([0, 2, 6], dtype=torch.int32, device=DEVICE)
    out = ops.maxsim_pack_padded_rows(padded, lengths, offsets, max_len, 4)
    torch.cuda.synchronize()
    assert out.shape == (4, dim)
    assert torch.equal(out[:2], padded[0:2]) and torch.equal(out[2:4], padded[5:7])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_pack_documents_matches_cat_and_feeds_contrastive(dtype):
    """pack_documents equals the torch.cat of valid rows plus the prefix-sum
    offsets that callers build by hand (reference README.md:184-191), bit for
    bit, and scoring against it equals scoring against the hand-packed form."""
    g = torch.Generator().manual_seed(17)
    Nb, Ld, D = 9, 70, 64
    emb = torch.randn(Nb, Ld, D, generator=g).to(dtype).to(DEVICE)
    lens = torch.randint(1, Ld + 1, (Nb,), generator=g).to(DEVICE)
    docs, offs = maxsim_amd.pack_documents(emb, lens)
    ref_docs = torch.cat([emb[i, :int(lens[i])] for i in range(Nb)], dim=0)
    ref_offs = torch.zeros(Nb + 1, dtype=torch.int32, device=DEVICE)
    ref_offs[1:] = lens.cumsum(0)
    assert torch.equal(docs, ref_docs) and torch.equal(offs, ref_offs)
    q = torch.randn(5, 32, D, generator=g).to(dtype).to(DEVICE)
    assert torch.equal(maxsim_amd.score_contrastive(q, docs, offs),
                       maxsim_amd.score_contrastive(q, ref_docs, ref_offs))
