"""The five benchmark configurations (C1-C5) on the GPU, at their real sizes.

C1 against the committed golden fixture; C2 and C4 against the oracle in
full; C3 on a slice of queries (any slice of the chunk-seeded set is
bit-identical to the bench's data); C5 forward against the oracle in full,
its backward at full size through the oracle on a query subset (dscore zero
elsewhere) and through properties that do not depend on size: the split and
single-pass dq gathers agree, the gradients are linear in dscore, and exact
duplicate tokens never win over their first copy."""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import bench
import maxsim_amd
from maxsim_amd._ops import ops
from oracle import maxsim_oracle as oracle

from ._helpers import DEVICE, GRAD_TOL, SCORE_TOL, assert_close, check_argmax, np64, npi
from .golden.c1_inputs import digest, make_c1
from .test_gpu_contrastive import assert_rounded_from

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "c1_expected.npz"


def test_c1_padded_fp32_matches_golden_fixture():
    q, d, qlen, dlen = make_c1(0)
    gold = np.load(GOLDEN)
    assert digest(q, d, qlen, dlen) == str(gold["input_sha256"])
    scores, argmax = maxsim_amd.score_candidates_padded_with_argmax(
        q.to(DEVICE), d.to(DEVICE), qlen.to(DEVICE), dlen.to(DEVICE))
    assert_close(scores, gold["scores"], **SCORE_TOL[torch.float32])
    qn, dn = np64(q), np64(d)
    check_argmax(npi(argmax), gold["argmax"], lambda idx: qn[idx[0], idx[2]],
                 lambda idx, j: dn[idx[0], idx[1], j])


def test_c2_contrastive_training_step():
    q, d, off, _ = bench.make_c5(torch, DEVICE, seed=1, nq=64, nb=64, lo=64, hi=512, dup=0.0)
    qg, dg = q.clone().requires_grad_(True), d.clone().requires_grad_(True)
    scores = maxsim_amd.score_contrastive_train(qg, dg, off)
    loss = F.cross_entropy(scores, torch.arange(64, device=DEVICE))
    loss.backward()
    s_ref, a_ref = oracle.contrastive_forward(np64(q), np64(d), npi(off))
    assert_close(scores, s_ref, **SCORE_TOL[torch.bfloat16])
    # the CE gradient w.r.t. the scores, from the kernel's own scores
    g = ((torch.softmax(scores.detach(), 1) - torch.eye(64, device=DEVICE)) / 64).cpu().numpy()
    dq_ref, dd_ref = oracle.contrastive_backward(g, np64(q), np64(d), npi(off), a_ref)
    # .grad is bf16 (autograd casts the fp32 gradient to the input dtype)
    assert_close(qg.grad.float(), dq_ref, rtol=1e-2, atol=1e-4)
    assert_close(dg.grad.float(), dd_ref, rtol=1e-2, atol=1e-4)


def test_c3_padded_rerank_query_slice():
    only = [0, 97, 255]
    q, d, qlen, dlen = bench.make_c3(torch, DEVICE, only=only)
    B, C, Ld, D = d.shape
    scores = maxsim_amd.score_candidates_padded(q, d, qlen, dlen)
    s2, argmax = maxsim_amd.score_candidates_padded_with_argmax(q, d, qlen, dlen)
    assert torch.equal(scores, s2)
    qn, dn = np64(q), np64(d)
    s_ref, a_ref = oracle.padded_forward(qn, dn, npi(qlen), npi(dlen))
    assert_close(scores, s_ref, **SCORE_TOL[torch.float16])
    check_argmax(npi(argmax), a_ref, lambda idx: qn[idx[0], idx[2]],
                 lambda idx, j: dn[idx[0], idx[1], j])


def test_c3_full_size_rows_equal_the_checked_slice():
    """C3 at full size (256 x 1000 x 300 x 128 fp16, 9.8e9 elements, well
    past 2^31): rows 0, 97 and 255 of the scores and argmax equal, bit for
    bit, those of the 3-query slice that the test above checks against the
    oracle (each (query, candidate) is computed independently of the batch,
    and the chunk-seeded inputs are identical), so addressing beyond 2^31
    elements is pinned."""
    only = [0, 97, 255]
    qs, ds, qls, dls = bench.make_c3(torch, DEVICE, only=only)
    s_slice, a_slice = maxsim_amd.score_candidates_padded_with_argmax(qs, ds, qls, dls)
    del qs, ds
    q, d, qlen, dlen = bench.make_c3(torch, DEVICE)
    assert d.numel() > 2**33
    try:
        scores = maxsim_amd.score_candidates_padded(q, d, qlen, dlen)
        s_full, a_full = maxsim_amd.score_candidates_padded_with_argmax(q, d, qlen, dlen)
        torch.cuda.synchronize()
        assert torch.equal(scores, s_full)
        assert torch.isfinite(s_full).all()
        rows = torch.tensor(only, device=DEVICE)
        assert torch.equal(s_full[rows], s_slice)
        assert torch.equal(a_full[rows], a_slice)
    finally:
        del q, d
        torch.cuda.empty_cache()


def test_c4_packed_forward_and_backward_full():
    (q, qo, d, do, qi, di, mql, g, *_r) = bench.make_c4(torch, DEVICE)
    scores, argmax = maxsim_amd.score_pairs_packed_with_argmax(q, qo, d, do, qi, di)
    assert argmax.shape[1] == mql
    qn, dn, qon, don, qin, din = np64(q), np64(d), npi(qo), npi(do), npi(qi), npi(di)
    s_ref, a_ref = oracle.packed_forward(qn, qon, dn, don, qin, din, mql)
    assert_close(scores, s_ref, **SCORE_TOL[torch.bfloat16])
    check_argmax(npi(argmax), a_ref, lambda idx: qn[qon[qin[idx[0]]] + idx[1]],
                 lambda idx, j: dn[don[din[idx[0]]] + j])
    dq, dd = ops.maxsim_packed_backward(g, q, qo, d, do, qi, di, argmax, mql)
    dq_ref, dd_ref = oracle.packed_backward(np64(g), qn, qon, dn, don, qin, din, npi(argmax))
    assert_close(dq, dq_ref, **GRAD_TOL[torch.bfloat16])
    assert_close(dd, dd_ref, **GRAD_TOL[torch.bfloat16])


@pytest.fixture(scope="module")
def c5():
    q, d, off, lens = bench.make_c5(torch, DEVICE)
    scores, argmax = ops.maxsim_contrastive_forward_with_argmax(q, d, off)
    return q, d, off, lens, scores, argmax


def test_c5_forward_full_against_oracle(c5):
    q, d, off, _, scores, argmax = c5
    qn, dn, on = np64(q), np64(d), npi(off)
    s_ref, a_ref = oracle.contrastive_forward(qn, dn, on)
    assert_close(scores, s_ref, **SCORE_TOL[torch.bfloat16])
    check_argmax(npi(argmax), a_ref, lambda idx: qn[idx[0], idx[2]],
                 lambda idx, j: dn[on[idx[1]] + j])
    # the score-only kernel gives the same scores bit for bit
    assert torch.equal(ops.maxsim_contrastive_forward(q, d, off), scores)


def test_c5_duplicate_tokens_never_beat_their_first_copy(c5):
    """1% of the document tokens are copies of an earlier token of the same
    document; whenever the winning row has an identical earlier row in its
    document, the kernel must have picked the earliest one."""
    _, d, off, lens, _, argmax = c5
    dn = d.view(torch.int16).cpu().numpy()
    on = npi(off)
    am = npi(argmax)
    checked = 0
    for b in range(0, len(lens), 7):
        rows = dn[on[b]:on[b + 1]]
        _, first, inv = np.unique(rows, axis=0, return_index=True, return_inverse=True)
        first_of = first[inv.reshape(-1)]            # earliest identical row for each row
        picked = am[:, b, :].reshape(-1)
        assert np.array_equal(first_of[picked], picked), f"document {b}: a later duplicate won"
        checked += int((first_of != np.arange(rows.shape[0])).sum())
    assert checked > 0  # the sample contains duplicates


def test_c5_backward_full_size(c5):
    q, d, off, _, _, argmax = c5
    nq, nb = q.shape[0], off.numel() - 1
    gen = torch.Generator().manual_seed(11)
    sub = torch.randperm(nq, generator=gen)[:16]
    g = torch.zeros(nq, nb)
    g[sub] = torch.randn(16, nb, generator=gen) / nb
    g = g.to(DEVICE)
    dq, dd = ops.maxsim_contrastive_backward(g, q, d, off, argmax)
    # oracle on the 16 queries with a non-zero dscore
    subn = sub.numpy()
    dq_ref, dd_ref = oracle.contrastive_backward(g.cpu().numpy()[subn], np64(q)[subn], np64(d),
                                                 npi(off), npi(argmax)[subn])
    assert_close(dq[sub], dq_ref, **GRAD_TOL[torch.bfloat16])
    assert_close(dd, dd_ref, **GRAD_TOL[torch.bfloat16])
    mask = torch.ones(nq, dtype=torch.bool)
    mask[sub] = False
    assert torch.all(dq[mask.to(DEVICE)] == 0)
    # linearity in dscore: scaling by a power of two is exact for dq (its
    # summation order is fixed); dd sums each bucket in an order set by LDS
    # atomics, so only to rounding
    dq2, dd2 = ops.maxsim_contrastive_backward(g * 4, q, d, off, argmax)
    assert torch.equal(dq2, dq * 4)
    torch.testing.assert_close(dd2, dd * 4, rtol=1e-5, atol=1e-7)


def test_c5_backward_split_and_single_pass_agree(c5):
    """The workspace (one document range per XCD) and single-pass dq gathers
    are different algorithms; at full size they agree to fp32 rounding."""
    q, d, off, _, scores, argmax = c5
    nq, lq, dim = q.shape
    nb = off.numel() - 1
    g = ((torch.softmax(scores, 1) - torch.eye(nq, device=DEVICE)) / nq).contiguous()
    lib = ctypes.CDLL(str(Path(maxsim_amd.__file__).resolve().parent / "libmaxsim_amd.so"))
    I64, P, SZ = ctypes.c_int64, ctypes.c_void_p, ctypes.c_size_t
    fn = lib.maxsim_amd_contrastive_backward
    fn.argtypes = [ctypes.c_int, P, P, I64, I64, P, I64, P, I64, P, I64, P, P, P, SZ, P]
    lib.maxsim_amd_contrastive_backward_workspace_size.restype = SZ
    lib.maxsim_amd_contrastive_backward_workspace_size.argtypes = [I64, I64, I64]
    need = lib.maxsim_amd_contrastive_backward_workspace_size(nq, lq, dim)
    ws = torch.empty(need // 4, device=DEVICE)
    outs = []
    for w, nbytes in [(None, 0), (ws, need)]:
        dq = torch.empty(nq, lq, dim, device=DEVICE)
        dd = torch.empty(d.shape[0], dim, device=DEVICE)
        rc = fn(2, g.data_ptr(), q.data_ptr(), nq, lq, d.data_ptr(), d.shape[0], off.data_ptr(),
                nb, argmax.data_ptr(), dim, dq.data_ptr(), dd.data_ptr(),
                w.data_ptr() if w is not None else None, nbytes,
                torch.cuda.current_stream().cuda_stream)
        assert rc == 0
        torch.cuda.synchronize()
        outs.append((dq, dd))
    torch.testing.assert_close(outs[0][0], outs[1][0], rtol=1e-5, atol=1e-7)
    torch.testing.assert_close(outs[0][1], outs[1][1], rtol=1e-5, atol=1e-7)


def test_c5_backward_in_input_dtype_equals_cast_fp32(c5):
    """The training step's backward writes bf16 gradients directly; at full
    size they equal the fp32 operator's gradients cast by torch: dq bit for
    bit, dd up to the fp32 bucket-order noise (CE's dscore has both signs, so
    some row sums cancel to far below their terms)."""
    q, d, off, _, scores, argmax = c5
    nq = q.shape[0]
    g = ((torch.softmax(scores, 1) - torch.eye(nq, device=DEVICE)) / nq).contiguous()
    dq32, dd32 = ops.maxsim_contrastive_backward(g, q, d, off, argmax)
    dq, dd = ops.maxsim_contrastive_backward_typed(g, q, d, off, argmax)
    assert dq.dtype == torch.bfloat16 and dd.dtype == torch.bfloat16
    assert torch.equal(dq, dq32.to(torch.bfloat16))
    _, mag = ops.maxsim_contrastive_backward(g.abs(), q.abs(), d, off, argmax)
    assert_rounded_from(dd, dd32, mag)


def test_c5_shard_of_8_forward_and_backward(c5):
    """One GPU's shard of C5 split by query rows over 8 GPUs: 64 queries
    against all 512 documents, the per-rank shape of the multi-GPU design
    (its backward takes the small-batch dQ path).  Forward, fp32 backward and
    the typed backward against the oracle."""
    q, d, off, _, _, _ = c5
    qs = q[:64].contiguous()
    nb = off.numel() - 1
    scores, argmax = ops.maxsim_contrastive_forward_with_argmax(qs, d, off)
    qn, dn, on = np64(qs), np64(d), npi(off)
    s_ref, a_ref = oracle.contrastive_forward(qn, dn, on)
    assert_close(scores, s_ref, **SCORE_TOL[torch.bfloat16])
    check_argmax(npi(argmax), a_ref, lambda idx: qn[idx[0], idx[2]],
                 lambda idx, j: dn[on[idx[1]] + j])
    g = ((torch.softmax(scores, 1) - torch.eye(64, nb, device=DEVICE)) / 64).contiguous()
    dq, dd = ops.maxsim_contrastive_backward(g, qs, d, off, argmax)
    dq_ref, dd_ref = oracle.contrastive_backward(g.double().cpu().numpy(), qn, dn, on,
                                                 npi(argmax))
    assert_close(dq, dq_ref, **GRAD_TOL[torch.bfloat16])
    assert_close(dd, dd_ref, **GRAD_TOL[torch.bfloat16])
    dqt, ddt = ops.maxsim_contrastive_backward_typed(g, qs, d, off, argmax)
    assert torch.equal(dqt, dq.to(torch.bfloat16))
    _, mag = ops.maxsim_contrastive_backward(g.abs(), qs.abs(), d, off, argmax)
    assert_rounded_from(ddt, dd, mag)
