"""Packed forward scored document by document (group_docs_kernel +
doc_chunk_kernel, taken with a workspace for 16-bit rows of 64 or 128
elements, max_q_len <= 64 and at least 4096 pairs) against pair_kernel on
the same inputs, bit for bit, and against the oracle.  The torch ops pass a
workspace; a max_q_len of 65 selects pair_kernel on the same pairs.  Cases
the grouping must route: pairs with an out-of-range query or document id,
empty document segments, a document named by hundreds of pairs (many
chunks of four), documents named by no pair, both query block counts, and
sparse pairs (partly filled chunks)."""

from __future__ import annotations

import ctypes

import pytest
import torch

from maxsim_amd._ops import ops
from oracle import maxsim_oracle as oracle

from ._helpers import (DEVICE, SCORE_TOL, assert_close, check_argmax, np64, npi,
                       offsets_from_lengths)

pytestmark = pytest.mark.gpu

DT16 = [torch.bfloat16, torch.float16]


def make_case(dim, dtype, seed, nq=37, nd=700, npairs=6000):
    gen = torch.Generator().manual_seed(seed)
    ql = torch.randint(1, 65, (nq,), generator=gen)
    dl = torch.randint(1, 300, (nd,), generator=gen)
    dl[[5, 17]] = 0                      # empty segments: invalid documents
    dl[40] = 2048                        # one long document (64 tiles)
    q = torch.randn(int(ql.sum()), dim, generator=gen).to(dtype)
    d = torch.randn(int(dl.sum()), dim, generator=gen).to(dtype)
    qids = torch.randint(0, nq, (npairs,), generator=gen, dtype=torch.int32)
    dids = torch.randint(0, nd - 50, (npairs,), generator=gen, dtype=torch.int32)  # 50 unused docs
    dids[100:400] = 3                    # a hot document: 75 chunks of four
    dids[[7, 8]] = torch.tensor([nd, -1], dtype=torch.int32)   # out-of-range documents
    qids[[9, 10]] = torch.tensor([nq, -5], dtype=torch.int32)  # out-of-range queries
    dids[11] = 5                         # an empty document
    dids[12] = 40
    bad = torch.zeros(npairs, dtype=torch.bool)
    bad[[7, 8, 9, 10, 11]] = True
    bad |= (dids == 5) | (dids == 17)
    return (q.to(DEVICE), offsets_from_lengths(ql).to(DEVICE), d.to(DEVICE),
            offsets_from_lengths(dl).to(DEVICE), qids.to(DEVICE), dids.to(DEVICE), bad)


@pytest.mark.parametrize("dtype", DT16, ids=["bf16", "fp16"])
@pytest.mark.parametrize("dim", [64, 128])
def test_doc_major_equals_pair_kernel_and_oracle(dim, dtype):
    q, qo, d, do, qi, di, bad = make_case(dim, dtype, seed=dim)
    s_doc, a_doc = ops.maxsim_packed_forward_with_argmax(q, qo, d, do, qi, di, 64)
    s_pair, a_pair = ops.maxsim_packed_forward_with_argmax(q, qo, d, do, qi, di, 65)
    torch.testing.assert_close(s_doc, s_pair, rtol=0, atol=0, equal_nan=True)
    assert torch.equal(a_doc, a_pair[:, :64]) and torch.all(a_pair[:, 64] == 0)
    badd = bad.to(DEVICE)
    assert torch.all(torch.isnan(s_doc[badd])) and torch.all(a_doc[badd] == 0)
    assert not torch.any(torch.isnan(s_doc[~badd]))
    # scores only (op maxsim_forward) through the same path
    torch.testing.assert_close(ops.maxsim_forward(q, qo, d, do, qi, di, 64), s_doc, rtol=0,
                               atol=0, equal_nan=True)
    ok = ~badd
    qn, dn, qon, don = np64(q), np64(d), npi(qo), npi(do)
    qin, din = npi(qi[ok]), npi(di[ok])
    s_ref, a_ref = oracle.packed_forward(qn, qon, dn, don, qin, din, 64)
    assert_close(s_doc[ok], s_ref, **SCORE_TOL[dtype])
    check_argmax(npi(a_doc[ok]), a_ref, lambda idx: qn[qon[qin[idx[0]]] + idx[1]],
                 lambda idx, j: dn[don[din[idx[0]]] + j])


def test_doc_major_repeatable_and_order_free():
    """Same bits on a second call (the grouping's atomics order the pairs
    differently from run to run) and with the pairs given in another order."""
    q, qo, d, do, qi, di, _ = make_case(128, torch.bfloat16, seed=3)
    s1, a1 = ops.maxsim_packed_forward_with_argmax(q, qo, d, do, qi, di, 64)
    s2, a2 = ops.maxsim_packed_forward_with_argmax(q, qo, d, do, qi, di, 64)
    torch.testing.assert_close(s1, s2, rtol=0, atol=0, equal_nan=True)
    assert torch.equal(a1, a2)
    perm = torch.randperm(qi.numel(), generator=torch.Generator().manual_seed(1)).to(DEVICE)
    s3, a3 = ops.maxsim_packed_forward_with_argmax(q, qo, d, do, qi[perm], di[perm], 64)
    torch.testing.assert_close(s3, s1[perm], rtol=0, atol=0, equal_nan=True)
    assert torch.equal(a3, a1[perm])


@pytest.mark.parametrize("qlen", [(1, 65), (33, 65)], ids=["mixed_blocks", "two_blocks"])
@pytest.mark.parametrize("seed,shift", [(0, 0), (1, 1)], ids=["aligned", "ids_offsets_unaligned"])
def test_doc_major_sparse_pairs(qlen, seed, shift):
    """C4-like sparsity (about 2.3 pairs per document): most chunks are
    partly filled (empty pair slots), with one or two query blocks per pair;
    documents whose pairs all name invalid queries give chunks with no tile
    among the others.  With shift 1 the document ids and offsets start 4
    bytes past a 16-byte boundary (the grouping's element-wise loads)."""
    gen = torch.Generator().manual_seed(100 + seed)
    nq, nd, npairs, dim = 61, 3000, 7000, 128
    ql = torch.randint(qlen[0], qlen[1], (nq,), generator=gen)
    dl = torch.randint(1, 400, (nd,), generator=gen)
    q = torch.randn(int(ql.sum()), dim, generator=gen).to(torch.bfloat16)
    d = torch.randn(int(dl.sum()), dim, generator=gen).to(torch.bfloat16)
    qids = torch.randint(0, nq, (npairs,), generator=gen, dtype=torch.int32)
    dids = torch.randint(0, nd, (npairs,), generator=gen, dtype=torch.int32)
    dead = torch.arange(7, nd, 97)       # documents named only by invalid queries
    qids[torch.isin(dids, dead)] = nq
    bad = torch.isin(dids, dead)
    def shifted(t):
        return torch.cat([t.new_zeros(shift), t]).to(DEVICE)[shift:]
    q, qo, d = q.to(DEVICE), offsets_from_lengths(ql).to(DEVICE), d.to(DEVICE)
    do, qi, di = shifted(offsets_from_lengths(dl)), qids.to(DEVICE), shifted(dids)
    assert (di.data_ptr() % 16 == 0) == (shift == 0) and (do.data_ptr() % 16 == 0) == (shift == 0)
    s_doc, a_doc = ops.maxsim_packed_forward_with_argmax(q, qo, d, do, qi, di, 64)
    s_pair, a_pair = ops.maxsim_packed_forward_with_argmax(q, qo, d, do, qi, di, 65)
    torch.testing.assert_close(s_doc, s_pair, rtol=0, atol=0, equal_nan=True)
    assert torch.equal(a_doc, a_pair[:, :64])
    badd = bad.to(DEVICE)
    assert torch.all(torch.isnan(s_doc[badd])) and torch.all(a_doc[badd] == 0)
    assert not torch.any(torch.isnan(s_doc[~badd]))
    ok = ~badd
    qn, dn, qon, don = np64(q), np64(d), npi(qo), npi(do)
    s_ref, _ = oracle.packed_forward(qn, qon, dn, don, npi(qi[ok]), npi(di[ok]), 64)
    assert_close(s_doc[ok], s_ref, **SCORE_TOL[torch.bfloat16])


@pytest.mark.parametrize("nd", [16384, 16381])
def test_doc_major_at_the_document_cap(nd):
    """The most documents the grouping takes (16 ranges of 1024) and a count
    that leaves the last range ragged: the document-major path against
    pair_kernel (max_q_len 65), bit for bit."""
    gen = torch.Generator().manual_seed(nd)
    nq, npairs, dim = 97, 40000, 64
    ql = torch.randint(1, 65, (nq,), generator=gen)
    dl = torch.randint(1, 40, (nd,), generator=gen)
    q = torch.randn(int(ql.sum()), dim, generator=gen).to(torch.bfloat16).to(DEVICE)
    d = torch.randn(int(dl.sum()), dim, generator=gen).to(torch.bfloat16).to(DEVICE)
    qo, do = offsets_from_lengths(ql).to(DEVICE), offsets_from_lengths(dl).to(DEVICE)
    qi = torch.randint(0, nq, (npairs,), generator=gen, dtype=torch.int32).to(DEVICE)
    di = torch.randint(0, nd, (npairs,), generator=gen, dtype=torch.int32).to(DEVICE)
    di[:3] = torch.tensor([nd - 1, nd - 1, 0], dtype=torch.int32)
    s_doc, a_doc = ops.maxsim_packed_forward_with_argmax(q, qo, d, do, qi, di, 64)
    s_pair, a_pair = ops.maxsim_packed_forward_with_argmax(q, qo, d, do, qi, di, 65)
    torch.testing.assert_close(s_doc, s_pair, rtol=0, atol=0, equal_nan=True)
    assert torch.equal(a_doc, a_pair[:, :64])
    assert not torch.any(torch.isnan(s_doc))


def test_c_abi_workspace_fallbacks():
    """Through the C ABI: a NULL, short or misaligned workspace takes the
    pair kernels; all three give the grouped path's bits."""
    from maxsim_amd._ops import NATIVE_LIB
    lib = ctypes.CDLL(str(NATIVE_LIB))
    P, I64, SZ = ctypes.c_void_p, ctypes.c_int64, ctypes.c_size_t
    fn = lib.maxsim_amd_packed_forward_with_argmax_ws
    fn.argtypes = [ctypes.c_int, P, I64, P, I64, P, I64, P, I64, P, P, I64, I64, I64, P, P, P,
                   SZ, P]
    wsz = lib.maxsim_amd_packed_forward_workspace_size
    wsz.restype, wsz.argtypes = SZ, [I64, I64]
    q, qo, d, do, qi, di, _ = make_case(128, torch.bfloat16, seed=11, npairs=4096)
    nq, nd, npairs = qo.numel() - 1, do.numel() - 1, qi.numel()
    need = wsz(nd, npairs)
    ws = torch.empty(need + 16, dtype=torch.uint8, device=DEVICE)
    outs = []
    for ptr, size in [(ws.data_ptr(), need), (None, 0), (ws.data_ptr(), need - 1),
                      (ws.data_ptr() + 4, need)]:
        s = torch.empty(npairs, device=DEVICE)
        a = torch.empty(npairs, 64, dtype=torch.int32, device=DEVICE)
        rc = fn(2, q.data_ptr(), q.shape[0], qo.data_ptr(), nq, d.data_ptr(), d.shape[0],
                do.data_ptr(), nd, qi.data_ptr(), di.data_ptr(), npairs, 128, 64, s.data_ptr(),
                a.data_ptr(), ptr, size, torch.cuda.current_stream().cuda_stream)
        assert rc == 0
        outs.append((s, a))
    torch.cuda.synchronize()
    for s, a in outs[1:]:
        torch.testing.assert_close(s, outs[0][0], rtol=0, atol=0, equal_nan=True)
        assert torch.equal(a, outs[0][1])
