"""Padded surface on the GPU vs the CPU oracle (reference tests:
tests/test_padded.py, test_argmax.py, test_backward.py, test_edge_shapes.py:37-110)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import maxsim_amd
from maxsim_amd._ops import ops
from oracle import maxsim_oracle as oracle

from ._helpers import (DEVICE, DTYPES, GRAD_TOL, SCORE_TOL, assert_close, check_argmax,
                       make_padded, np64, npi)

pytestmark = pytest.mark.gpu

SHAPES = [
    # B, C, Lq, Ld, dim, full lengths?
    pytest.param(4, 5, 32, 128, 64, False, id="random-lengths"),
    pytest.param(1, 1, 1, 1, 16, True, id="smallest"),
    pytest.param(1, 1, 16, 17, 16, True, id="Ld17"),
    pytest.param(1, 1, 16, 65, 16, True, id="Ld65"),
    pytest.param(2, 2, 8, 24, 24, True, id="dim24"),
    pytest.param(1, 1, 32, 100, 96, True, id="dim96"),
    pytest.param(4, 1, 16, 32, 64, True, id="C1"),
    pytest.param(1, 8, 16, 32, 64, True, id="B1"),
    pytest.param(3, 4, 64, 50, 128, False, id="Lq64"),
    pytest.param(2, 3, 130, 40, 32, False, id="Lq130-three-block-groups"),
    pytest.param(2, 2, 32, 300, 128, False, id="Ld300"),
    pytest.param(2, 37, 16, 40, 64, False, id="C37-dq-candidates-over-4-lanes"),
]


def _full_or_random(B, C, Lq, Ld, full):
    if full:
        return torch.full((B,), Lq, dtype=torch.int32), torch.full((B, C), Ld, dtype=torch.int32)
    return None, None


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda t: str(t).split(".")[-1])
@pytest.mark.parametrize("B,C,Lq,Ld,dim,full", SHAPES)
def test_padded_forward_argmax_backward(B, C, Lq, Ld, dim, full, dtype):
    ql, dl = _full_or_random(B, C, Lq, Ld, full)
    q, d, qlen, dlen = make_padded(B, C, Lq, Ld, dim, dtype, seed=B * 7 + Ld, qlen=ql, dlen=dl)
    qn, dn = np64(q), np64(d)
    s_ref, a_ref = oracle.padded_forward(qn, dn, npi(qlen), npi(dlen))

    s = maxsim_amd.score_candidates_padded(q, d, qlen, dlen)
    assert s.shape == (B, C) and s.dtype == torch.float32
    assert_close(s, s_ref, **SCORE_TOL[dtype])

    s2, am = maxsim_amd.score_candidates_padded_with_argmax(q, d, qlen, dlen)
    assert torch.equal(s, s2)
    assert tuple(am.shape) == (B, C, Lq) and am.dtype == torch.int32
    check_argmax(npi(am), a_ref, lambda idx: qn[idx[0], idx[2]],
                 lambda idx, j: dn[idx[0], idx[1], j])
    # pad slots are 0
    qlc = npi(qlen)
    for b in range(B):
        assert np.all(npi(am)[b, :, qlc[b]:] == 0)

    g = torch.randn(B, C, generator=torch.Generator().manual_seed(9)).to(DEVICE)
    dq, dd = ops.maxsim_padded_backward(
        g.reshape(-1).contiguous(), q.reshape(B * Lq, dim).contiguous(),
        d.reshape(B * C * Ld, dim).contiguous(), qlen, dlen.reshape(-1).contiguous(),
        am.reshape(B * C, Lq).contiguous(), Lq, Ld, C)
    dq_ref, dd_ref = oracle.padded_backward(np64(g), qn, dn, npi(qlen), npi(dlen), npi(am))
    assert_close(dq.view(B, Lq, dim), dq_ref, **GRAD_TOL[dtype])
    assert_close(dd.view(B, C, Ld, dim), dd_ref, **GRAD_TOL[dtype])


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda t: str(t).split(".")[-1])
def test_padded_ignores_pad_positions(dtype):
    """Garbage -- even NaN -- past the declared lengths never changes results
    (test_padded.py:38-61)."""
    B, C, Lq, Ld, D = 2, 3, 8, 40, 32
    q, d, _, _ = make_padded(B, C, Lq, Ld, D, dtype, seed=1)
    qlen = torch.tensor([4, 6], dtype=torch.int32, device=DEVICE)
    dlen = torch.tensor([[10, 8, 4], [40, 1, 33]], dtype=torch.int32, device=DEVICE)
    base_s, base_a = maxsim_amd.score_candidates_padded_with_argmax(q, d, qlen, dlen)
    qc, dc = q.clone(), d.clone()
    qc[0, 4:] = 1e4
    qc[1, 6:] = float("nan")
    dc[0, 0, 10:] = 1e4
    dc[1, 1, 1:] = float("nan")
    dc[1, 2, 33:] = -1e4
    s, a = maxsim_amd.score_candidates_padded_with_argmax(qc, dc, qlen, dlen)
    assert torch.equal(s, base_s) and torch.equal(a, base_a)


def test_padded_first_index_wins_on_ties():
    base = torch.randn(16, dtype=torch.float16)
    d = base.view(1, 1, 1, 16).expand(1, 1, 37, 16).contiguous().to(DEVICE)
    q = torch.randn(1, 16, 16, dtype=torch.float16, device=DEVICE)
    _, a = maxsim_amd.score_candidates_padded_with_argmax(
        q, d, torch.tensor([16], dtype=torch.int32, device=DEVICE),
        torch.tensor([[37]], dtype=torch.int32, device=DEVICE))
    assert torch.all(a == 0)


def test_padded_nan_gives_neg_inf():
    torch.manual_seed(0)
    q = torch.randn(2, 16, 64, device=DEVICE, dtype=torch.float16)
    d = torch.randn(2, 3, 32, 64, device=DEVICE, dtype=torch.float16)
    qlen = torch.full((2,), 16, dtype=torch.int32, device=DEVICE)
    dlen = torch.full((2, 3), 32, dtype=torch.int32, device=DEVICE)
    q[1, 0, 0] = float("nan")
    s = maxsim_amd.score_candidates_padded(q, d, qlen, dlen)
    assert torch.isinf(s[1]).all() and (s[1] < 0).all()
    assert torch.isfinite(s[0]).all()


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda t: str(t).split(".")[-1])
def test_padded_train_end_to_end(dtype):
    B, C, Lq, Ld, D = 2, 4, 16, 32, 64
    q, d, qlen, dlen = make_padded(B, C, Lq, Ld, D, dtype, seed=2)
    q.requires_grad_(True)
    d.requires_grad_(True)
    scores = maxsim_amd.score_candidates_padded_train(q, d, qlen, dlen)
    w = torch.randn(B, C, generator=torch.Generator().manual_seed(4)).to(DEVICE)
    (scores * w).sum().backward()
    _, a_ref = oracle.padded_forward(np64(q), np64(d), npi(qlen), npi(dlen))
    dq_ref, dd_ref = oracle.padded_backward(np64(w), np64(q), np64(d), npi(qlen), npi(dlen), a_ref)
    tol = GRAD_TOL[dtype] if dtype == torch.float32 else dict(rtol=1e-2, atol=1e-2)
    assert_close(q.grad, dq_ref, **tol)
    assert_close(d.grad, dd_ref, **tol)


def test_padded_operator_invalid_lengths_give_nan_only_there():
    """The padded kernels range-check every length they read: a candidate or
    query whose length is outside (0, Ld] / (0, Lq] scores NaN with argmax 0,
    every other candidate is unchanged, and nothing is read out of range."""
    B, C, Lq, Ld, D = 3, 4, 16, 24, 32
    q, d, qlen, dlen = make_padded(B, C, Lq, Ld, D, torch.bfloat16, seed=31)
    args = (q.reshape(B * Lq, D).contiguous(), None, d.reshape(B * C * Ld, D).contiguous())
    s_good, a_good = ops.maxsim_padded_forward_with_argmax(
        args[0], qlen, args[2], dlen.reshape(-1).contiguous(), Lq, Ld, C)
    bad_q = qlen.clone()
    bad_q[2] = Lq + 1
    bad_d = dlen.clone()
    bad_d[0, 1] = 0
    bad_d[1, 3] = Ld + 5
    bad_d[1, 0] = -7
    s, a = ops.maxsim_padded_forward_with_argmax(
        args[0], bad_q, args[2], bad_d.reshape(-1).contiguous(), Lq, Ld, C)
    torch.cuda.synchronize()
    s, a = s.view(B, C), a.view(B, C, Lq)
    invalid = torch.zeros(B, C, dtype=torch.bool)
    invalid[2, :] = True
    invalid[0, 1] = invalid[1, 3] = invalid[1, 0] = True
    invalid = invalid.to(DEVICE)
    assert torch.isnan(s[invalid]).all()
    assert torch.all(a[invalid] == 0)
    assert torch.equal(s[~invalid], s_good.view(B, C)[~invalid])
    assert torch.equal(a[~invalid], a_good.view(B, C, Lq)[~invalid])


PADDED_FNS = [maxsim_amd.score_candidates_padded, maxsim_amd.score_candidates_padded_with_argmax,
              maxsim_amd.score_candidates_padded_train]


@pytest.mark.parametrize("fn", PADDED_FNS, ids=lambda f: f.__name__)
@pytest.mark.parametrize("which,value,pattern", [
    ("q", 0, "query_lengths must contain values > 0"),
    ("q", 17, "query_lengths values must be <= padded length 16"),
    ("d", 0, "doc_lengths must contain values > 0"),
    ("d", -3, "doc_lengths must contain values > 0"),
    ("d", 25, "doc_lengths values must be <= padded length 24"),
])
def test_padded_bad_device_lengths_raise_after_queueing(fn, which, value, pattern):
    """Device lengths are checked on the host while the kernels already run
    (the check waits only for their copy): bad lengths still raise the
    reference's ValueError, the queued kernels are safe with them, and the
    device is in a good state afterwards."""
    B, C, Lq, Ld, D = 2, 3, 16, 24, 32
    q, d, qlen, dlen = make_padded(B, C, Lq, Ld, D, torch.float16, seed=37)
    bq, bd = qlen.clone(), dlen.clone()
    if which == "q":
        bq[1] = value
    else:
        bd[1, 2] = value
    with pytest.raises(ValueError, match=pattern):
        fn(q, d, bq, bd)
    torch.cuda.synchronize()
    s_ref, _ = oracle.padded_forward(np64(q), np64(d), npi(qlen), npi(dlen))
    assert_close(maxsim_amd.score_candidates_padded(q, d, qlen, dlen), s_ref,
                 **SCORE_TOL[torch.float16])


# ---------------------------------------------------------------------------
# gradients in the input dtype (the autograd path's operator)
# ---------------------------------------------------------------------------
def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.contiguous().view(torch.int16 if t.element_size() == 2 else torch.int32)


TYPED = [
    # B, C, Lq, Ld, dim
    pytest.param(3, 4, 32, 100, 64, id="basic"),
    pytest.param(2, 3, 40, 33, 20, id="dim20-element-wise"),
    pytest.param(2, 2, 48, 70, 256, id="dim256"),
    pytest.param(2, 3, 50, 70, 8, id="dim8-one-lane-per-row"),
    pytest.param(2, 2, 24, 40, 96, id="dim96-element-pairs"),
    pytest.param(2, 37, 24, 30, 64, id="C37-dq-candidates-over-4-lanes"),
    pytest.param(2, 3, 200, 3, 32, id="three-rows-many-tokens-each"),
    pytest.param(2, 2, 330, 40, 64, id="Lq330-argmax-in-lds"),
    pytest.param(1, 2, 4352, 20, 16, id="Lq4352-argmax-lds-at-its-64KB-cap"),
    pytest.param(1, 2, 4400, 20, 16, id="Lq4400-argmax-from-global"),
    pytest.param(2, 2, 30, 25, 7, id="dim7-odd-element-wise"),
    pytest.param(1, 1, 1, 1, 16, id="smallest"),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bfloat16", "float16"])
@pytest.mark.parametrize("B,C,Lq,Ld,dim", TYPED)
def test_padded_backward_typed_is_cast_fp32_bit_for_bit(B, C, Lq, Ld, dim, dtype):
    """The typed operator sums each gradient element in the same fp32 order
    as the fp32 one and rounds to nearest even, so it is the cast of the
    fp32 gradients bit for bit (padding rows included), and close to the
    oracle."""
    # the first query uses all Lq tokens (past the 256 kept in registers when
    # Lq > 256), the others about half, which leaves padding rows
    qlen = [Lq] + [max(1, Lq // 2 + b) for b in range(1, B)]
    q, d, qlen, dlen = make_padded(B, C, Lq, Ld, dim, dtype, seed=B * Lq + dim, qlen=qlen)
    _, am = maxsim_amd.score_candidates_padded_with_argmax(q, d, qlen, dlen)
    g = torch.randn(B * C, generator=torch.Generator().manual_seed(Ld)).to(DEVICE)
    qf, df = q.reshape(B * Lq, dim), d.reshape(B * C * Ld, dim)
    args = (g, qf, df, qlen.to(torch.int32), dlen.reshape(-1).to(torch.int32),
            am.reshape(B * C, Lq).contiguous(), Lq, Ld, C)
    dq32, dd32 = ops.maxsim_padded_backward(*args)
    dq, dd = ops.maxsim_padded_backward_typed(*args)
    assert dq.dtype == dtype and dd.dtype == dtype
    assert torch.equal(_bits(dq), _bits(dq32.to(dtype)))
    assert torch.equal(_bits(dd), _bits(dd32.to(dtype)))
    dq_ref, dd_ref = oracle.padded_backward(np64(g.view(B, C)), np64(q), np64(d), npi(qlen),
                                            npi(dlen), npi(am))
    assert_close(dq.view(B, Lq, dim), dq_ref, rtol=1e-2, atol=1e-2)
    assert_close(dd.view(B, C, Ld, dim), dd_ref, rtol=1e-2, atol=1e-2)


def test_padded_backward_typed_misaligned_views_match_fp32():
    """16-bit views that start 2 bytes into their storage take the 16-bit
    element path instead of 32-bit accesses; same bits as the cast."""
    B, C, Lq, Ld, dim = 2, 3, 20, 30, 32
    q, d, qlen, dlen = make_padded(B, C, Lq, Ld, dim, torch.float16, seed=23)
    _, am = maxsim_amd.score_candidates_padded_with_argmax(q, d, qlen, dlen)
    qbuf = torch.empty(B * Lq * dim + 1, dtype=torch.float16, device=DEVICE)
    qbuf[1:].copy_(q.reshape(-1))
    qv = qbuf[1:].view(B * Lq, dim)
    assert qv.data_ptr() % 4 == 2
    g = torch.randn(B * C, generator=torch.Generator().manual_seed(8)).to(DEVICE)
    args = (g, qv, d.reshape(B * C * Ld, dim), qlen, dlen.reshape(-1),
            am.reshape(B * C, Lq).contiguous(), Lq, Ld, C)
    dq32, dd32 = ops.maxsim_padded_backward(*args)
    dq, dd = ops.maxsim_padded_backward_typed(*args)
    assert torch.equal(_bits(dq), _bits(dq32.to(torch.float16)))
    assert torch.equal(_bits(dd), _bits(dd32.to(torch.float16)))


def test_padded_backward_typed_invalid_lengths_match_fp32():
    """Lengths the operator does not validate (0, beyond the padding): the
    typed gradients are still the cast of the fp32 ones, zero for the
    invalid query and candidates."""
    B, C, Lq, Ld, dim = 3, 3, 16, 24, 32
    q, d, qlen, dlen = make_padded(B, C, Lq, Ld, dim, torch.bfloat16, seed=41)
    _, am = maxsim_amd.score_candidates_padded_with_argmax(q, d, qlen, dlen)
    bq, bd = qlen.clone().to(torch.int32), dlen.clone().reshape(-1).to(torch.int32)
    bq[2] = 0
    bd[1] = 0
    bd[4] = Ld + 5
    g = torch.randn(B * C, generator=torch.Generator().manual_seed(3)).to(DEVICE)
    args = (g, q.reshape(B * Lq, dim), d.reshape(B * C * Ld, dim), bq, bd,
            am.reshape(B * C, Lq).contiguous(), Lq, Ld, C)
    dq32, dd32 = ops.maxsim_padded_backward(*args)
    dq, dd = ops.maxsim_padded_backward_typed(*args)
    assert torch.equal(_bits(dq), _bits(dq32.to(torch.bfloat16)))
    assert torch.equal(_bits(dd), _bits(dd32.to(torch.bfloat16)))
    assert torch.all(dq.view(B, Lq, dim)[2] == 0)
    assert torch.all(dd.view(B * C, Ld, dim)[[1, 4, 6, 7, 8]] == 0)


def test_padded_backward_typed_fp32_inputs_are_fp32():
    q, d, qlen, dlen = make_padded(2, 3, 16, 40, 32, torch.float32, seed=6)
    _, am = maxsim_amd.score_candidates_padded_with_argmax(q, d, qlen, dlen)
    g = torch.randn(6, generator=torch.Generator().manual_seed(1)).to(DEVICE)
    args = (g, q.reshape(32, 32), d.reshape(240, 32), qlen.to(torch.int32),
            dlen.reshape(-1).to(torch.int32), am.reshape(6, 16).contiguous(), 16, 40, 3)
    dq, dd = ops.maxsim_padded_backward_typed(*args)
    dq32, dd32 = ops.maxsim_padded_backward(*args)
    assert dq.dtype == torch.float32 and dd.dtype == torch.float32
    assert torch.equal(dq, dq32) and torch.equal(dd, dd32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bfloat16", "float16"])
def test_padded_train_grads_in_input_dtype(dtype):
    """score_candidates_padded_train: .grad has the input dtype and equals
    the fp32 operator's gradient cast, bit for bit."""
    B, C, Lq, Ld, D = 2, 4, 24, 60, 64
    q, d, qlen, dlen = make_padded(B, C, Lq, Ld, D, dtype, seed=19)
    qg, dg = q.clone().requires_grad_(True), d.clone().requires_grad_(True)
    w = torch.randn(B, C, generator=torch.Generator().manual_seed(5)).to(DEVICE)
    (maxsim_amd.score_candidates_padded_train(qg, dg, qlen, dlen) * w).sum().backward()
    assert qg.grad.dtype == dtype and dg.grad.dtype == dtype
    _, am = maxsim_amd.score_candidates_padded_with_argmax(q, d, qlen, dlen)
    dq32, dd32 = ops.maxsim_padded_backward(
        w.reshape(-1).contiguous(), q.reshape(B * Lq, D), d.reshape(B * C * Ld, D),
        qlen.to(torch.int32), dlen.reshape(-1).to(torch.int32),
        am.reshape(B * C, Lq).contiguous(), Lq, Ld, C)
    assert torch.equal(_bits(qg.grad.reshape(B * Lq, D)), _bits(dq32.to(dtype)))
    assert torch.equal(_bits(dg.grad.reshape(B * C * Ld, D)), _bits(dd32.to(dtype)))


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=["fp16", "fp32"])
@pytest.mark.parametrize("Lq,dim", [(40, 128), (300, 64), (24, 8)], ids=["Lq40-dim128", "Lq300-dim64",
                                                                       "Lq24-dim8"])
def test_padded_backward_row_paths_agree_bit_for_bit(Lq, dim, dtype):
    """16-byte-aligned queries with dim/8 dividing 64 take the path that
    writes each dD row once from its in-order sum; a view 2 or 4 bytes into
    its storage takes the zero-then-add path.  Both operators (fp32 and typed
    gradients) give the same bits on either path."""
    B, C, Ld = 2, 3, 50
    q, d, qlen, dlen = make_padded(B, C, Lq, Ld, dim, dtype, seed=Lq + dim, qlen=[Lq, Lq // 2])
    _, am = maxsim_amd.score_candidates_padded_with_argmax(q, d, qlen, dlen)
    qbuf = torch.empty(B * Lq * dim + 1, dtype=dtype, device=DEVICE)
    qbuf[1:].copy_(q.reshape(-1))
    q_off = qbuf[1:].view(B * Lq, dim)
    assert q_off.data_ptr() % 16 != 0
    g = torch.randn(B * C, generator=torch.Generator().manual_seed(2)).to(DEVICE)
    rest = (d.reshape(B * C * Ld, dim), qlen, dlen.reshape(-1), am.reshape(B * C, Lq).contiguous(),
            Lq, Ld, C)
    for op in (ops.maxsim_padded_backward, ops.maxsim_padded_backward_typed):
        dq_a, dd_a = op(g, q.reshape(B * Lq, dim), *rest)
        dq_b, dd_b = op(g, q_off, *rest)
        assert torch.equal(_bits(dq_a), _bits(dq_b))
        assert torch.equal(_bits(dd_a), _bits(dd_b))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_padded_small_batch_split_kernel_bits(dtype):
    """Below one pair per SIMD the forward spreads each pair's tiles over the
    waves of a workgroup and merges their maxima; from one pair per SIMD on,
    a wave walks a pair's tiles in order.  The first 8 queries of a 64-query
    batch (1024 pairs) and the same 8 queries alone (128 pairs) get the same
    score and argmax bits, ties, NaN rows and -inf rows included, and match
    the oracle."""
    gen = torch.Generator().manual_seed(61)
    B, C, Lq, Ld, dim = 64, 16, 40, 300, 128
    q = torch.randn(B, Lq, dim, generator=gen).to(dtype)
    d = torch.randn(B, C, Ld, dim, generator=gen).to(dtype)
    d[0, 1, 7] = d[0, 1, 200]          # an exact tie across tiles
    d[0, 2, 40] = float("nan")         # a NaN row never wins
    d[1, 3, :] = float("-inf")         # every similarity -inf or NaN
    qlen = torch.randint(1, Lq + 1, (B,), generator=gen, dtype=torch.int32)
    dlen = torch.randint(1, Ld + 1, (B, C), generator=gen, dtype=torch.int32)
    dlen[0, 1] = Ld
    q, d, qlen, dlen = q.to(DEVICE), d.to(DEVICE), qlen.to(DEVICE), dlen.to(DEVICE)
    s_all, a_all = maxsim_amd.score_candidates_padded_with_argmax(q, d, qlen, dlen)
    s8, a8 = maxsim_amd.score_candidates_padded_with_argmax(q[:8].contiguous(), d[:8].contiguous(),
                                                            qlen[:8].contiguous(),
                                                            dlen[:8].contiguous())
    torch.cuda.synchronize()
    same = (s8.view(torch.int32) == s_all[:8].view(torch.int32))
    assert bool(same.all())
    assert torch.equal(a8, a_all[:8])
    with np.errstate(invalid="ignore"):  # the -inf row's products are NaN
        s_ref, a_ref = oracle.padded_forward(np64(q[:8]), np64(d[:8]), npi(qlen[:8]),
                                             npi(dlen[:8]))
    finite = np.isfinite(s_ref)
    assert_close(s8[torch.as_tensor(finite, device=DEVICE)], s_ref[finite], **SCORE_TOL[dtype])
