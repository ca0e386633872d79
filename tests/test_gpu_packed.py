"""Packed surface on the GPU vs the CPU oracle (reference tests:
tests/test_correctness.py, test_dtypes.py, test_ragged.py, test_packed_train.py,
test_edge_shapes.py:118-154)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import maxsim_amd
from maxsim_amd._ops import ops
from oracle import maxsim_oracle as oracle

from ._helpers import (DEVICE, DTYPES, GRAD_TOL, SCORE_TOL, assert_close, assert_rounded_from,
                       check_argmax, make_packed, np64, npi, offsets_from_lengths)

pytestmark = pytest.mark.gpu

CASES = [
    # nq, nd, npairs, dim, q range, d range
    pytest.param(6, 11, 17, 64, (4, 32), (8, 200), id="basic-d64"),
    pytest.param(6, 11, 17, 96, (4, 32), (8, 200), id="d96"),
    pytest.param(5, 7, 13, 64, (1, 1), (1, 1), id="len1"),
    pytest.param(5, 7, 13, 64, (1, 64), (1, 64), id="ragged-short"),
    pytest.param(5, 7, 13, 64, (4, 32), (16, 1024), id="long-docs"),
    pytest.param(3, 4, 6, 128, (8, 24), (16, 96), id="train-shape"),
    pytest.param(4, 9, 40, 128, (8, 100), (16, 300), id="Lq-up-to-100"),
    pytest.param(2, 3, 5, 24, (3, 9), (5, 40), id="d24"),
    pytest.param(3, 4, 9, 64, (4, 40), (1100, 2600), id="docs-over-two-row-passes"),
]


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda t: str(t).split(".")[-1])
@pytest.mark.parametrize("nq,nd,npairs,dim,qr,dr", CASES)
def test_packed_forward_argmax_backward(nq, nd, npairs, dim, qr, dr, dtype):
    q, qoff, d, doff, qids, dids = make_packed(nq, nd, npairs, dim, qr, dr, dtype, seed=npairs + dim)
    qn, dn, qo, do = np64(q), np64(d), npi(qoff), npi(doff)
    mql = int(np.diff(qo).max())
    s_ref, a_ref = oracle.packed_forward(qn, qo, dn, do, npi(qids), npi(dids), mql)

    s = maxsim_amd.score_pairs_packed(q, qoff, d, doff, qids, dids)
    assert s.shape == (npairs,) and s.dtype == torch.float32
    assert_close(s, s_ref, **SCORE_TOL[dtype])

    s2, am = maxsim_amd.score_pairs_packed_with_argmax(q, qoff, d, doff, qids, dids)
    assert torch.equal(s, s2)
    assert tuple(am.shape) == (npairs, mql)
    qi, di = npi(qids), npi(dids)
    check_argmax(npi(am), a_ref, lambda idx: qn[qo[qi[idx[0]]] + idx[1]],
                 lambda idx, j: dn[do[di[idx[0]]] + j])

    g = torch.randn(npairs, generator=torch.Generator().manual_seed(5)).to(DEVICE)
    dq, dd = ops.maxsim_packed_backward(g, q, qoff, d, doff, qids, dids, am, mql)
    dq_ref, dd_ref = oracle.packed_backward(np64(g), qn, qo, dn, do, qi, di, npi(am))
    assert_close(dq, dq_ref, **GRAD_TOL[dtype])
    assert_close(dd, dd_ref, **GRAD_TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_packed_backward_hot_query_and_document(dtype):
    """One query and one document in 600 pairs each (more than one LDS stage
    of the grouped backward), plus repeated identical pairs."""
    q, qoff, d, doff, qids, dids = make_packed(7, 13, 900, 64, (4, 40), (8, 300), dtype, seed=77)
    qids[:600] = 2
    dids[300:900] = 5
    qids[890:] = 1
    dids[890:] = 1
    qn, dn, qo, do = np64(q), np64(d), npi(qoff), npi(doff)
    mql = int(np.diff(qo).max())
    _, am = maxsim_amd.score_pairs_packed_with_argmax(q, qoff, d, doff, qids, dids)
    g = torch.randn(900, generator=torch.Generator().manual_seed(6)).to(DEVICE)
    dq, dd = ops.maxsim_packed_backward(g, q, qoff, d, doff, qids, dids, am, mql)
    dq_ref, dd_ref = oracle.packed_backward(np64(g), qn, qo, dn, do, npi(qids), npi(dids), npi(am))
    assert_close(dq, dq_ref, **GRAD_TOL[dtype])
    assert_close(dd, dd_ref, **GRAD_TOL[dtype])


def test_packed_backward_op_zeroes_rows_outside_segments():
    """The op called directly (no Python validation) with offsets that leave
    rows before the first and after the last segment: those gradient rows are
    zero, as with the reference's zero-filled outputs."""
    gen = torch.Generator().manual_seed(3)
    q = torch.randn(12, 32, generator=gen).to(DEVICE)
    d = torch.randn(20, 32, generator=gen).to(DEVICE)
    qoff = torch.tensor([2, 5, 9], dtype=torch.int32, device=DEVICE)
    doff = torch.tensor([3, 10, 16], dtype=torch.int32, device=DEVICE)
    qids = torch.tensor([0, 1, 1, 0], dtype=torch.int32, device=DEVICE)
    dids = torch.tensor([1, 0, 1, 0], dtype=torch.int32, device=DEVICE)
    s, am = ops.maxsim_packed_forward_with_argmax(q, qoff, d, doff, qids, dids, 4)
    g = torch.randn(4, generator=gen).to(DEVICE)
    dq, dd = ops.maxsim_packed_backward(g, q, qoff, d, doff, qids, dids, am, 4)
    dq_ref, dd_ref = oracle.packed_backward(np64(g), np64(q), npi(qoff), np64(d), npi(doff),
                                            npi(qids), npi(dids), npi(am))
    assert_close(dq, dq_ref, **GRAD_TOL[torch.float32])
    assert_close(dd, dd_ref, **GRAD_TOL[torch.float32])
    assert torch.all(dq[:2] == 0) and torch.all(dq[9:] == 0)
    assert torch.all(dd[:3] == 0) and torch.all(dd[16:] == 0)


def test_packed_single_pair_single_token_closed_form():
    """test_correctness.py:39-50: 1 x 1 tokens -> score is the dot product."""
    q = torch.randn(1, 16, device=DEVICE)
    d = torch.randn(1, 16, device=DEVICE)
    one = torch.tensor([0, 1], dtype=torch.int32, device=DEVICE)
    z = torch.tensor([0], dtype=torch.int32, device=DEVICE)
    s = maxsim_amd.score_pairs_packed(q, one, d, one, z, z)
    expected = float(np.dot(np64(q)[0], np64(d)[0]))
    assert abs(float(s[0]) - expected) <= 1e-5 * max(1.0, abs(expected))


def test_packed_empty_pairs():
    q, qoff, d, doff, qids, dids = make_packed(2, 3, 0, 32, (2, 8), (2, 16), torch.float32, seed=0)
    s = maxsim_amd.score_pairs_packed(q, qoff, d, doff, qids, dids)
    assert s.shape == (0,) and s.dtype == torch.float32


def test_packed_max_q_len_larger_than_needed():
    q, qoff, d, doff, qids, dids = make_packed(3, 4, 6, 64, (8, 24), (16, 96), torch.bfloat16, seed=2)
    s, am = maxsim_amd.score_pairs_packed_with_argmax(q, qoff, d, doff, qids, dids, max_q_len=40)
    assert am.shape == (6, 40)
    qo = npi(qoff)
    lens = np.diff(qo)[npi(qids)]
    for k in range(6):
        assert np.all(npi(am)[k, lens[k]:] == 0)


def test_packed_nan_gives_neg_inf():
    Lq, Ld, D = 16, 32, 64
    q = torch.randn(2 * Lq, D, device=DEVICE, dtype=torch.float16)
    d = torch.randn(3 * Ld, D, device=DEVICE, dtype=torch.float16)
    qoff = torch.arange(0, 3 * Lq, Lq, dtype=torch.int32, device=DEVICE)
    doff = torch.arange(0, 4 * Ld, Ld, dtype=torch.int32, device=DEVICE)
    qids = torch.tensor([0, 1], dtype=torch.int32, device=DEVICE)
    dids = torch.tensor([0, 0], dtype=torch.int32, device=DEVICE)
    q[Lq] = float("nan")
    s = maxsim_amd.score_pairs_packed(q, qoff, d, doff, qids, dids, max_q_len=Lq)
    assert torch.isfinite(s[0]) and torch.isinf(s[1]) and s[1] < 0


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda t: str(t).split(".")[-1])
def test_packed_ties_first_index(dtype):
    base = torch.randn(32, dtype=dtype)
    d = base.expand(47, 32).contiguous().to(DEVICE)
    q = torch.randn(12, 32, dtype=dtype, device=DEVICE)
    qo = torch.tensor([0, 12], dtype=torch.int32, device=DEVICE)
    do = torch.tensor([0, 47], dtype=torch.int32, device=DEVICE)
    z = torch.zeros(1, dtype=torch.int32, device=DEVICE)
    _, am = maxsim_amd.score_pairs_packed_with_argmax(q, qo, d, do, z, z)
    assert torch.all(am == 0)


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda t: str(t).split(".")[-1])
def test_packed_train_end_to_end(dtype):
    q, qoff, d, doff, qids, dids = make_packed(3, 4, 6, 64, (8, 24), (16, 96), dtype, seed=2)
    q.requires_grad_(True)
    d.requires_grad_(True)
    s = maxsim_amd.score_pairs_packed_train(q, qoff, d, doff, qids, dids)
    w = torch.randn(6, generator=torch.Generator().manual_seed(1)).to(DEVICE)
    (s * w).sum().backward()
    qo, do = npi(qoff), npi(doff)
    mql = int(np.diff(qo).max())
    _, a_ref = oracle.packed_forward(np64(q), qo, np64(d), do, npi(qids), npi(dids), mql)
    dq_ref, dd_ref = oracle.packed_backward(np64(w), np64(q), qo, np64(d), do, npi(qids),
                                            npi(dids), a_ref)
    tol = GRAD_TOL[dtype] if dtype == torch.float32 else dict(rtol=1e-2, atol=1e-2)
    assert_close(q.grad, dq_ref, **tol)
    assert_close(d.grad, dd_ref, **tol)


PACKED_FNS = [maxsim_amd.score_pairs_packed, maxsim_amd.score_pairs_packed_with_argmax,
              maxsim_amd.score_pairs_packed_train]


def _packed_dev():
    gen = torch.Generator().manual_seed(5)
    q = torch.randn(13, 64, generator=gen).to(torch.float16).to(DEVICE)
    d = torch.randn(20, 64, generator=gen).to(torch.float16).to(DEVICE)
    i32 = dict(dtype=torch.int32, device=DEVICE)
    return q, torch.tensor([0, 5, 13], **i32), d, torch.tensor([0, 20], **i32), i32


@pytest.mark.parametrize("fn", PACKED_FNS, ids=lambda f: f.__name__)
def test_packed_bad_device_inputs_with_max_q_len_raise_after_queueing(fn):
    """With max_q_len given, the offsets and ids are checked on the host while
    the kernels already run: every bad input still raises the reference's
    error, and the queued kernels are safe with it."""
    q, qo, d, do, i32 = _packed_dev()
    one = torch.tensor([1], **i32)
    zero = torch.tensor([0], **i32)
    with pytest.raises(RuntimeError, match="0|offset|start"):
        fn(q, torch.tensor([1, 5, 13], **i32), d, do, one, zero, max_q_len=8)
    with pytest.raises(RuntimeError, match="total|equal|offset"):
        fn(q, qo, d, torch.tensor([0, 30], **i32), one, zero, max_q_len=8)
    with pytest.raises(RuntimeError, match="out of range"):
        fn(q, qo, d, do, torch.tensor([-1], **i32), zero, max_q_len=8)
    with pytest.raises(RuntimeError, match="out of range"):
        fn(q, qo, d, do, one, torch.tensor([7], **i32), max_q_len=8)
    with pytest.raises(ValueError, match="max_q_len"):
        fn(q, qo, d, do, one, zero, max_q_len=5)   # query 1 has 8 tokens
    torch.cuda.synchronize()
    # the device is fine and a good call gives the oracle's answer
    s = maxsim_amd.score_pairs_packed(q, qo, d, do, one, zero, max_q_len=8)
    s_ref, _ = oracle.packed_forward(np64(q), npi(qo), np64(d), npi(do), npi(one), npi(zero), 8)
    assert_close(s, s_ref, **SCORE_TOL[torch.float16])


@pytest.mark.parametrize("fn", PACKED_FNS, ids=lambda f: f.__name__)
def test_packed_bad_device_inputs_without_max_q_len(fn):
    """Without max_q_len the score-only call launches with the number of
    query rows as the length bound and the others read back only the longest
    query length; the checks then run while the kernels execute, or first
    when the offsets cannot be well formed.  Every bad input still raises the
    reference's error."""
    q, qo, d, do, i32 = _packed_dev()
    one = torch.tensor([1], **i32)
    zero = torch.tensor([0], **i32)
    with pytest.raises(RuntimeError, match="0|offset|start"):
        fn(q, torch.tensor([1, 5, 13], **i32), d, do, one, zero)
    with pytest.raises(RuntimeError, match="total|equal|offset"):
        fn(q, torch.tensor([0, 5, 12], **i32), d, do, one, zero)
    with pytest.raises(RuntimeError, match="total|equal|offset|decreas|order"):
        fn(q, torch.tensor([0, 9, 5, 13], **i32), d, do, one, zero)  # a negative segment
    with pytest.raises(RuntimeError, match="total|equal|offset"):
        fn(q, qo, d, torch.tensor([0, 30], **i32), one, zero)
    with pytest.raises(RuntimeError, match="out of range"):
        fn(q, qo, d, do, torch.tensor([-1], **i32), zero)
    with pytest.raises(RuntimeError, match="out of range"):
        fn(q, qo, d, do, one, torch.tensor([7], **i32))
    torch.cuda.synchronize()
    s_ref, a_ref = oracle.packed_forward(np64(q), npi(qo), np64(d), npi(do), npi(one), npi(zero), 8)
    out = fn(q, qo, d, do, one, zero)
    s = out[0] if isinstance(out, tuple) else out
    assert_close(s.detach(), s_ref, **SCORE_TOL[torch.float16])
    if isinstance(out, tuple):
        assert tuple(out[1].shape) == (1, 8)


def test_packed_score_only_bound_gives_identical_scores():
    """The score-only call without max_q_len launches with the number of
    query rows as the length bound (two query blocks in registers for every
    pair); the scores are bit-identical to a launch with the exact longest
    query length, including queries of at most 32 tokens."""
    for qr in [(4, 32), (4, 64), (30, 100)]:
        q, qoff, d, doff, qids, dids = make_packed(9, 13, 60, 128, qr, (8, 300), torch.bfloat16,
                                                   seed=qr[1])
        mql = int(np.diff(npi(qoff)).max())
        exact = ops.maxsim_forward(q, qoff, d, doff, qids, dids, mql)
        assert torch.equal(maxsim_amd.score_pairs_packed(q, qoff, d, doff, qids, dids), exact)


def _typed_vs_fp32(q, qoff, d, doff, qids, dids, seed):
    """Typed packed backward against the fp32 operator cast to the input
    dtype (round to nearest even), up to fp32 summation-order noise; both
    gradients are also checked against the oracle."""
    dtype = q.dtype
    _, am = maxsim_amd.score_pairs_packed_with_argmax(q, qoff, d, doff, qids, dids)
    mql = am.shape[1]
    g = torch.randn(qids.numel(), generator=torch.Generator().manual_seed(seed)).to(DEVICE)
    dq32, dd32 = ops.maxsim_packed_backward(g, q, qoff, d, doff, qids, dids, am, mql)
    dq, dd = ops.maxsim_packed_backward_typed(g, q, qoff, d, doff, qids, dids, am, mql)
    assert dq.dtype == dtype and dd.dtype == dtype
    assert dq.shape == dq32.shape and dd.shape == dd32.shape
    # absolute term sums: the same routing with |g| and |d| (dq), |g| and |q| (dd)
    mag_q, _ = ops.maxsim_packed_backward(g.abs(), q, qoff, d.abs(), doff, qids, dids, am, mql)
    _, mag_d = ops.maxsim_packed_backward(g.abs(), q.abs(), qoff, d, doff, qids, dids, am, mql)
    assert_rounded_from(dq, dq32, mag_q)
    assert_rounded_from(dd, dd32, mag_d)
    dq_ref, dd_ref = oracle.packed_backward(np64(g), np64(q), npi(qoff), np64(d), npi(doff),
                                            npi(qids), npi(dids), npi(am))
    assert_close(dq, dq_ref, rtol=1e-2, atol=1e-2)
    assert_close(dd, dd_ref, rtol=1e-2, atol=1e-2)


TYPED = [
    # nq, nd, npairs, dim, q range, d range, hot query / document
    pytest.param(6, 11, 17, 64, (4, 32), (8, 200), False, id="basic"),
    pytest.param(5, 7, 13, 20, (1, 64), (1, 64), False, id="dim20-element-wise"),
    pytest.param(7, 13, 900, 64, (4, 40), (8, 300), True, id="hot-document-multi-stage"),
    pytest.param(5, 6, 400, 128, (8, 64), (300, 1000), True, id="hot-long-documents-row-passes"),
    pytest.param(5, 6, 300, 20, (4, 40), (100, 900), True, id="hot-dim20-element-wise"),
    pytest.param(4, 5, 300, 256, (4, 48), (70, 200), True, id="hot-dim256-64-row-passes"),
    pytest.param(3, 4, 9, 64, (4, 40), (1100, 2600), False, id="docs-over-two-row-passes"),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bfloat16", "float16"])
@pytest.mark.parametrize("nq,nd,npairs,dim,qr,dr,hot", TYPED)
def test_packed_backward_typed_equals_cast_fp32(nq, nd, npairs, dim, qr, dr, hot, dtype):
    """The autograd path's operator writes the gradients in the input dtype.
    Documents whose entries fit one LDS stage are written by the grouped dD
    kernel; a document in hundreds of pairs takes the LDS-accumulator kernel
    (several row passes when longer than its 128 rows at dim 128)."""
    q, qoff, d, doff, qids, dids = make_packed(nq, nd, npairs, dim, qr, dr, dtype,
                                               seed=npairs + dim)
    if hot:
        qids[: npairs // 2] = 2
        dids[npairs // 3:] = 1
    _typed_vs_fp32(q, qoff, d, doff, qids, dids, seed=8)


def test_packed_backward_typed_query_longer_than_a_stage():
    """A query of 4100 tokens (more than the 4096 entries of one LDS stage):
    every document takes the LDS-accumulator kernel."""
    gen = torch.Generator().manual_seed(12)
    ql = torch.tensor([4100, 30])
    dl = torch.tensor([50, 7, 200])
    q = torch.randn(int(ql.sum()), 32, generator=gen).to(torch.bfloat16).to(DEVICE)
    d = torch.randn(int(dl.sum()), 32, generator=gen).to(torch.bfloat16).to(DEVICE)
    qoff, doff = offsets_from_lengths(ql).to(DEVICE), offsets_from_lengths(dl).to(DEVICE)
    qids = torch.tensor([0, 1, 0, 0, 1], dtype=torch.int32, device=DEVICE)
    dids = torch.tensor([0, 0, 2, 0, 2], dtype=torch.int32, device=DEVICE)
    _typed_vs_fp32(q, qoff, d, doff, qids, dids, seed=9)


def test_packed_backward_typed_zeroes_rows_outside_segments():
    """16-bit gradients of rows before the first and after the last segment
    are zero; document 2 is in no pair and gets zero rows."""
    gen = torch.Generator().manual_seed(4)
    q = torch.randn(12, 32, generator=gen).to(torch.bfloat16).to(DEVICE)
    d = torch.randn(24, 32, generator=gen).to(torch.bfloat16).to(DEVICE)
    qoff = torch.tensor([2, 5, 9], dtype=torch.int32, device=DEVICE)
    doff = torch.tensor([3, 10, 16, 20], dtype=torch.int32, device=DEVICE)
    qids = torch.tensor([0, 1, 1, 0], dtype=torch.int32, device=DEVICE)
    dids = torch.tensor([1, 0, 1, 0], dtype=torch.int32, device=DEVICE)
    _, am = ops.maxsim_packed_forward_with_argmax(q, qoff, d, doff, qids, dids, 4)
    g = torch.randn(4, generator=gen).to(DEVICE)
    dq32, dd32 = ops.maxsim_packed_backward(g, q, qoff, d, doff, qids, dids, am, 4)
    dq, dd = ops.maxsim_packed_backward_typed(g, q, qoff, d, doff, qids, dids, am, 4)
    assert dq.dtype == torch.bfloat16 and dd.dtype == torch.bfloat16
    assert torch.all(dq[:2] == 0) and torch.all(dq[9:] == 0)
    assert torch.all(dd[:3] == 0) and torch.all(dd[16:] == 0)
    torch.testing.assert_close(dq.float(), dq32.to(torch.bfloat16).float(), rtol=2 ** -7, atol=1e-6)
    torch.testing.assert_close(dd.float(), dd32.to(torch.bfloat16).float(), rtol=2 ** -7, atol=1e-6)


def test_packed_backward_typed_fp32_inputs_are_fp32():
    q, qoff, d, doff, qids, dids = make_packed(4, 5, 9, 32, (2, 20), (4, 50), torch.float32, seed=3)
    _, am = maxsim_amd.score_pairs_packed_with_argmax(q, qoff, d, doff, qids, dids)
    g = torch.randn(9, generator=torch.Generator().manual_seed(1)).to(DEVICE)
    dq, dd = ops.maxsim_packed_backward_typed(g, q, qoff, d, doff, qids, dids, am, am.shape[1])
    dq32, dd32 = ops.maxsim_packed_backward(g, q, qoff, d, doff, qids, dids, am, am.shape[1])
    assert dq.dtype == torch.float32 and dd.dtype == torch.float32
    torch.testing.assert_close(dq, dq32, rtol=1e-6, atol=1e-7)
    torch.testing.assert_close(dd, dd32, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bfloat16", "float16"])
def test_packed_train_grads_in_input_dtype(dtype):
    """score_pairs_packed_train: .grad has the input dtype and is the fp32
    operator's gradient rounded, as autograd's cast would give."""
    q, qoff, d, doff, qids, dids = make_packed(5, 9, 40, 64, (4, 40), (8, 200), dtype, seed=15)
    qg, dg = q.clone().requires_grad_(True), d.clone().requires_grad_(True)
    w = torch.randn(40, generator=torch.Generator().manual_seed(2)).to(DEVICE)
    (maxsim_amd.score_pairs_packed_train(qg, qoff, dg, doff, qids, dids) * w).sum().backward()
    assert qg.grad.dtype == dtype and dg.grad.dtype == dtype
    _, am = maxsim_amd.score_pairs_packed_with_argmax(q, qoff, d, doff, qids, dids)
    mql = am.shape[1]
    dq32, dd32 = ops.maxsim_packed_backward(w, q, qoff, d, doff, qids, dids, am, mql)
    mag_q, _ = ops.maxsim_packed_backward(w.abs(), q, qoff, d.abs(), doff, qids, dids, am, mql)
    _, mag_d = ops.maxsim_packed_backward(w.abs(), q.abs(), qoff, d, doff, qids, dids, am, mql)
    assert_rounded_from(qg.grad, dq32, mag_q)
    assert_rounded_from(dg.grad, dd32, mag_d)


def test_packed_validation_sees_writes_queued_just_before():
    """As for the contrastive path: with max_q_len the ids are copied on a
    side stream that waits for the current one, so an id made invalid just
    before the call, behind a long kernel, is rejected."""
    q, qoff, d, doff, qids, dids = make_packed(4, 5, 9, 32, (2, 20), (4, 50), torch.float32, seed=8)
    torch.cuda.synchronize()
    a = torch.randn(4096, 4096, device=DEVICE)
    for _ in range(4):
        a = a @ a / 64.0
    dids[3] = 99
    with pytest.raises(RuntimeError, match="pair_document_ids"):
        maxsim_amd.score_pairs_packed(q, qoff, d, doff, qids, dids, max_q_len=20)
    torch.cuda.synchronize()


@pytest.mark.parametrize("host_checks", [True, False], ids=["checks", "no-checks"])
def test_score_only_beyond_2pow20_query_rows(host_checks):
    """A score-only call without max_q_len over more than 2^20 query rows
    (four segments of 250k-300k tokens, fp32, dim 8) gives the oracle's
    scores: its query-length bound is the row count, and only the argmax
    shape is capped at 2^20 slots."""
    gen = torch.Generator().manual_seed(21)
    q_lens, d_lens, dim = [300_000, 250_000, 275_000, 275_000], [3, 17, 40, 8, 25], 8
    q = torch.randn(sum(q_lens), dim, generator=gen)
    q = (q / q.norm(dim=1, keepdim=True)).to(DEVICE)
    d = torch.randn(sum(d_lens), dim, generator=gen)
    d = (d / d.norm(dim=1, keepdim=True)).to(DEVICE)
    qoff = offsets_from_lengths(q_lens).to(DEVICE)
    doff = offsets_from_lengths(d_lens).to(DEVICE)
    qids = torch.tensor([0, 1, 2, 3, 0, 3], dtype=torch.int32, device=DEVICE)
    dids = torch.tensor([0, 2, 4, 1, 3, 3], dtype=torch.int32, device=DEVICE)
    assert q.shape[0] > (1 << 20)
    with maxsim_amd.host_checks(host_checks):
        s = maxsim_amd.score_pairs_packed(q, qoff, d, doff, qids, dids)
    s_ref, _ = oracle.packed_forward(np64(q), npi(qoff), np64(d), npi(doff), npi(qids),
                                     npi(dids), max(q_lens))
    # sums of 250k-300k token maxima in fp32 (a few 1e-6 relative)
    assert_close(s, s_ref, rtol=5e-5, atol=1e-2)
