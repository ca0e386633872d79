"""Embedding dims above 256 on all three surfaces, forward and backward, vs
the CPU oracle.

The reference accepts any dim on its scalar paths (README.md:537-539,
maxsim_cuda/maxsim.cu:59-126, 647-698).  Here dims up to 256 keep the query
blocks in registers; wider rows take wide_pair_kernel (operands streamed in
K-chunks) in the forward and slice-chunk loops in the backward.  The cases
cover a dim that is not a multiple of 16 (element-wise loads), the dims of
common embedding models, dims above 2048, where the contrastive dQ takes
the single-pass gather and the packed dQ covers a row in several rounds, and
the largest accepted dim (16384, MAXSIM_AMD_MAX_DIM: a 64 KiB fp32 row)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import maxsim_amd
from maxsim_amd._ops import ops
from oracle import maxsim_oracle as oracle

from ._helpers import (DEVICE, DTYPES, GRAD_TOL, SCORE_TOL, assert_close, assert_rounded_from,
                       check_argmax, make_contrastive, make_packed, make_padded, np64, npi)

pytestmark = pytest.mark.gpu

DIMS = [pytest.param(300, id="d300"), pytest.param(384, id="d384"),
        pytest.param(768, id="d768"), pytest.param(2560, id="d2560"),
        pytest.param(4096, id="d4096"), pytest.param(16384, id="d16384")]
_ids = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}


def _normalize(t):
    return torch.nn.functional.normalize(t.float(), dim=-1).to(t.dtype)


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda t: _ids[t])
@pytest.mark.parametrize("dim", DIMS)
def test_contrastive_wide(dim, dtype):
    Nq, Lq, d_lens = 3, 40, [37, 1, 90, 64, 5, 33, 120, 17, 9]
    q, d, off = make_contrastive(Nq, Lq, dim, d_lens, dtype, seed=dim, unit=True)
    qn, dn, on = np64(q), np64(d), npi(off)
    s_ref, a_ref = oracle.contrastive_forward(qn, dn, on)
    s = maxsim_amd.score_contrastive(q, d, off)
    assert_close(s, s_ref, **SCORE_TOL[dtype])
    s2, am = maxsim_amd.score_contrastive_with_argmax(q, d, off)
    assert torch.equal(s, s2)
    check_argmax(npi(am), a_ref, lambda idx: qn[idx[0], idx[2]], lambda idx, j: dn[on[idx[1]] + j])

    g = torch.randn(Nq, len(d_lens), generator=torch.Generator().manual_seed(dim)).to(DEVICE)
    dq, dd = ops.maxsim_contrastive_backward(g, q, d, off, am)
    dq_ref, dd_ref = oracle.contrastive_backward(np64(g), qn, dn, on, npi(am))
    assert_close(dq, dq_ref, **GRAD_TOL[dtype])
    assert_close(dd, dd_ref, **GRAD_TOL[dtype])

    # autograd path: gradients in the input dtype
    qg, dg = q.clone().requires_grad_(True), d.clone().requires_grad_(True)
    (maxsim_amd.score_contrastive_train(qg, dg, off) * g).sum().backward()
    assert qg.grad.dtype == dtype and dg.grad.dtype == dtype
    if dtype == torch.float32:
        assert_close(qg.grad, dq_ref, **GRAD_TOL[dtype])
        assert_close(dg.grad, dd_ref, **GRAD_TOL[dtype])
    else:
        mag_q = torch.as_tensor(oracle.contrastive_backward(
            np.abs(np64(g)), np.abs(qn), np.abs(dn), on, npi(am))[0], dtype=torch.float32)
        assert_rounded_from(qg.grad.cpu(), dq.cpu(), mag_q)
        assert_close(dg.grad, dd_ref, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda t: _ids[t])
@pytest.mark.parametrize("dim", DIMS)
def test_padded_wide(dim, dtype):
    B, C, Lq, Ld = 2, 5, 40, 70
    q, d, qlen, dlen = make_padded(B, C, Lq, Ld, dim, dtype, seed=dim + 1)
    q, d = _normalize(q), _normalize(d)
    qn, dn = np64(q), np64(d)
    s_ref, a_ref = oracle.padded_forward(qn, dn, npi(qlen), npi(dlen))
    s = maxsim_amd.score_candidates_padded(q, d, qlen, dlen)
    assert_close(s, s_ref, **SCORE_TOL[dtype])
    s2, am = maxsim_amd.score_candidates_padded_with_argmax(q, d, qlen, dlen)
    assert torch.equal(s, s2)
    check_argmax(npi(am), a_ref, lambda idx: qn[idx[0], idx[2]],
                 lambda idx, j: dn[idx[0], idx[1], j])

    g = torch.randn(B, C, generator=torch.Generator().manual_seed(dim)).to(DEVICE)
    dq, dd = ops.maxsim_padded_backward(
        g.reshape(-1).contiguous(), q.reshape(B * Lq, dim).contiguous(),
        d.reshape(B * C * Ld, dim).contiguous(), qlen, dlen.reshape(-1).contiguous(),
        am.reshape(B * C, Lq).contiguous(), Lq, Ld, C)
    dq_ref, dd_ref = oracle.padded_backward(np64(g), qn, dn, npi(qlen), npi(dlen), npi(am))
    assert_close(dq.view(B, Lq, dim), dq_ref, **GRAD_TOL[dtype])
    assert_close(dd.view(B, C, Ld, dim), dd_ref, **GRAD_TOL[dtype])

    qg, dg = q.clone().requires_grad_(True), d.clone().requires_grad_(True)
    (maxsim_amd.score_candidates_padded_train(qg, dg, qlen, dlen) * g).sum().backward()
    assert qg.grad.dtype == dtype and dg.grad.dtype == dtype
    # the padded typed gradients are the fp32 operator's rounded, bit for bit
    assert torch.equal(qg.grad, dq.view(B, Lq, dim).to(dtype))
    assert torch.equal(dg.grad, dd.view(B, C, Ld, dim).to(dtype))


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda t: _ids[t])
@pytest.mark.parametrize("dim", DIMS)
def test_packed_wide(dim, dtype):
    nq, nd, npairs = 5, 9, 23
    q, qoff, d, doff, qids, dids = make_packed(nq, nd, npairs, dim, (3, 45), (4, 150), dtype,
                                               seed=dim + 2)
    q, d = _normalize(q), _normalize(d)
    qn, dn, qo, do = np64(q), np64(d), npi(qoff), npi(doff)
    mql = int(np.diff(qo).max())
    s_ref, a_ref = oracle.packed_forward(qn, qo, dn, do, npi(qids), npi(dids), mql)
    s = maxsim_amd.score_pairs_packed(q, qoff, d, doff, qids, dids)
    assert_close(s, s_ref, **SCORE_TOL[dtype])
    s2, am = maxsim_amd.score_pairs_packed_with_argmax(q, qoff, d, doff, qids, dids)
    assert torch.equal(s, s2)
    qi, di = npi(qids), npi(dids)
    check_argmax(npi(am), a_ref, lambda idx: qn[qo[qi[idx[0]]] + idx[1]],
                 lambda idx, j: dn[do[di[idx[0]]] + j])

    g = torch.randn(npairs, generator=torch.Generator().manual_seed(dim)).to(DEVICE)
    dq, dd = ops.maxsim_packed_backward(g, q, qoff, d, doff, qids, dids, am, mql)
    dq_ref, dd_ref = oracle.packed_backward(np64(g), qn, qo, dn, do, qi, di, npi(am))
    assert_close(dq, dq_ref, **GRAD_TOL[dtype])
    assert_close(dd, dd_ref, **GRAD_TOL[dtype])

    qg, dg = q.clone().requires_grad_(True), d.clone().requires_grad_(True)
    (maxsim_amd.score_pairs_packed_train(qg, qoff, dg, doff, qids, dids) * g).sum().backward()
    assert qg.grad.dtype == dtype and dg.grad.dtype == dtype
    tol = GRAD_TOL[dtype] if dtype == torch.float32 else dict(rtol=1e-2, atol=1e-2)
    assert_close(qg.grad, dq_ref, **tol)
    assert_close(dg.grad, dd_ref, **tol)


def test_dim_limit():
    q = torch.randn(1, 4, 16385, device=DEVICE, dtype=torch.bfloat16)
    d = torch.randn(8, 16385, device=DEVICE, dtype=torch.bfloat16)
    off = torch.tensor([0, 8], dtype=torch.int32, device=DEVICE)
    with pytest.raises(RuntimeError, match="16384"):
        maxsim_amd.score_contrastive(q, d, off)
