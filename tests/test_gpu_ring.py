"""pair_ring_kernel (padded and packed forwards, 16-bit rows of 32/64/128
elements, queries of at most 64 tokens: document tiles through two
wave-private LDS slots) against pair_kernel on the same inputs, bit for bit,
and against the oracle.  A launch whose query bound exceeds 64 tokens takes
pair_kernel: packed with max_q_len 65 instead of 64, padded with one more
(padding) query row."""

from __future__ import annotations

import pytest
import torch

from maxsim_amd._ops import ops
from oracle import maxsim_oracle as oracle

from ._helpers import (DEVICE, SCORE_TOL, assert_close, check_argmax, make_packed, make_padded,
                       np64, npi)

pytestmark = pytest.mark.gpu

DT16 = [torch.bfloat16, torch.float16]


@pytest.mark.parametrize("dtype", DT16, ids=["bf16", "fp16"])
@pytest.mark.parametrize("dim", [32, 64, 128])
def test_packed_ring_equals_pair_kernel(dim, dtype):
    q, qo, d, do, qi, di = make_packed(9, 14, 120, dim, (1, 64), (1, 150), dtype, seed=dim)
    qi[3] = 9        # an invalid pair
    s_ring, a_ring = ops.maxsim_packed_forward_with_argmax(q, qo, d, do, qi, di, 64)
    s_pair, a_pair = ops.maxsim_packed_forward_with_argmax(q, qo, d, do, qi, di, 65)
    torch.testing.assert_close(s_ring, s_pair, rtol=0, atol=0, equal_nan=True)
    assert torch.equal(a_ring, a_pair[:, :64]) and torch.all(a_pair[:, 64] == 0)
    assert torch.isnan(s_ring[3]) and torch.all(a_ring[3] == 0)
    torch.testing.assert_close(ops.maxsim_forward(q, qo, d, do, qi, di, 64), s_ring, rtol=0, atol=0,
                               equal_nan=True)
    ok = torch.ones(120, dtype=torch.bool)
    ok[3] = False
    qn, dn, qon, don = np64(q), np64(d), npi(qo), npi(do)
    qin, din = npi(qi[ok.to(DEVICE)]), npi(di[ok.to(DEVICE)])
    s_ref, a_ref = oracle.packed_forward(qn, qon, dn, don, qin, din, 64)
    assert_close(s_ring[ok.to(DEVICE)], s_ref, **SCORE_TOL[dtype])
    check_argmax(npi(a_ring[ok.to(DEVICE)]), a_ref, lambda idx: qn[qon[qin[idx[0]]] + idx[1]],
                 lambda idx, j: dn[don[din[idx[0]]] + j])


@pytest.mark.parametrize("dtype", DT16, ids=["bf16", "fp16"])
@pytest.mark.parametrize("dim", [32, 64, 128])
def test_padded_ring_equals_pair_kernel(dim, dtype):
    B, C, Lq, Ld = 3, 7, 64, 90
    q, d, ql, dl = make_padded(B, C, Lq, Ld, dim, dtype, seed=dim + 1)
    dl[1, 2] = Ld + 1  # an invalid candidate
    qf, df, dlf = q.reshape(B * Lq, dim), d.reshape(B * C * Ld, dim), dl.reshape(-1)
    s_ring, a_ring = ops.maxsim_padded_forward_with_argmax(qf, ql, df, dlf, Lq, Ld, C)
    q65 = torch.cat([q, q[:, :1]], dim=1).contiguous()  # one more padding row: Lq_max 65
    s_pair, a_pair = ops.maxsim_padded_forward_with_argmax(q65.reshape(B * 65, dim), ql, df, dlf,
                                                           65, Ld, C)
    torch.testing.assert_close(s_ring, s_pair, rtol=0, atol=0, equal_nan=True)
    assert torch.equal(a_ring.view(B * C, Lq), a_pair.view(B * C, 65)[:, :Lq])
    assert torch.isnan(s_ring.view(B, C)[1, 2])
    valid = torch.ones(B, C, dtype=torch.bool)
    valid[1, 2] = False
    dl_ok = dl.clone()
    dl_ok[1, 2] = Ld
    s_ref, a_ref = oracle.padded_forward(np64(q), np64(d), npi(ql), npi(dl_ok))
    sv = s_ring.view(B, C).cpu()[valid]
    assert_close(sv, s_ref[valid.numpy()], **SCORE_TOL[dtype])
