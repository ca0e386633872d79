"""Contrastive surface on the GPU vs the CPU oracle (reference tests:
tests/test_contrastive.py, test_edge_shapes.py:165-190, test_nan_inf.py)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import maxsim_amd
from maxsim_amd._ops import ops
from oracle import maxsim_oracle as oracle

from ._helpers import (DEVICE, DTYPES, GRAD_TOL, SCORE_TOL, assert_close, assert_rounded_from,
                       check_argmax, make_contrastive, np64, npi)

pytestmark = pytest.mark.gpu


def _check_forward(q, d, off, scores, argmax):
    qn, dn, on = np64(q), np64(d), npi(off)
    s_ref, a_ref = oracle.contrastive_forward(qn, dn, on)
    assert scores.shape == s_ref.shape and scores.dtype == torch.float32
    assert_close(scores, s_ref, **SCORE_TOL[q.dtype])
    if argmax is not None:
        assert argmax.dtype == torch.int32 and tuple(argmax.shape) == a_ref.shape
        check_argmax(npi(argmax), a_ref,
                     lambda idx: qn[idx[0], idx[2]],
                     lambda idx, j: dn[on[idx[1]] + j])
    return a_ref


SHAPES = [
    # Nq, Lq, dim, doc lengths
    pytest.param(3, 16, 64, [37, 64, 200, 17, 81], id="ragged-Lq16-d64"),
    pytest.param(5, 32, 128, [128, 300, 33, 1, 64, 512, 7], id="Lq32-d128"),
    pytest.param(17, 32, 128, [40] * 9, id="Nq17-partial-group"),
    pytest.param(2, 40, 128, [50, 90, 31], id="Lq40-two-blocks"),
    pytest.param(2, 100, 64, [50, 90], id="Lq100-pair-kernel"),
    pytest.param(1, 16, 16, [16], id="single"),
    pytest.param(1, 16, 16, [1], id="Ld1"),
    pytest.param(1, 16, 16, [17], id="Ld17"),
    pytest.param(1, 16, 32, [16, 32, 48, 64], id="tile-boundaries"),
    pytest.param(2, 16, 32, [7, 8, 100], id="mixed-ragged"),
    pytest.param(1, 16, 96, [1], id="dim96"),
    pytest.param(3, 8, 24, [5, 70], id="dim24"),
    pytest.param(2, 7, 20, [9, 33], id="dim20-odd"),
    pytest.param(2, 32, 256, [65, 129], id="dim256"),
    pytest.param(1, 1, 128, [1000], id="Lq1-long-doc"),
]


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda t: str(t).split(".")[-1])
@pytest.mark.parametrize("Nq,Lq,dim,d_lens", SHAPES)
def test_contrastive_forward_and_argmax(Nq, Lq, dim, d_lens, dtype):
    q, d, off = make_contrastive(Nq, Lq, dim, d_lens, dtype, seed=Nq * 131 + dim)
    scores = maxsim_amd.score_contrastive(q, d, off)
    _check_forward(q, d, off, scores, None)
    scores2, argmax = maxsim_amd.score_contrastive_with_argmax(q, d, off)
    _check_forward(q, d, off, scores2, argmax)
    # score-only and with-argmax kernels agree bit for bit
    assert torch.equal(scores, scores2)


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda t: str(t).split(".")[-1])
@pytest.mark.parametrize("Nq,Lq,dim,d_lens", SHAPES[:6] + SHAPES[11:14])
def test_contrastive_backward(Nq, Lq, dim, d_lens, dtype):
    q, d, off = make_contrastive(Nq, Lq, dim, d_lens, dtype, seed=7 + dim)
    gen = torch.Generator().manual_seed(3)
    dscore = torch.randn(Nq, len(d_lens), generator=gen).to(DEVICE)
    _, argmax = maxsim_amd.score_contrastive_with_argmax(q, d, off)
    dq, dd = ops.maxsim_contrastive_backward(dscore, q, d, off, argmax)
    assert dq.dtype == torch.float32 and dd.dtype == torch.float32
    dq_ref, dd_ref = oracle.contrastive_backward(np64(dscore), np64(q), np64(d), npi(off), npi(argmax))
    assert_close(dq, dq_ref, **GRAD_TOL[dtype])
    assert_close(dd, dd_ref, **GRAD_TOL[dtype])


# Backward cases for the split dq pass (Nb >= 8: one document range per
# XCD, eight partial sums) and for the dd kernel's dimension parts (Q larger
# than 4 MiB: at 600 x 32 x 128, two parts for 16-bit and four for fp32).
BWD_SPLIT = [
    pytest.param(4, 32, 128, [40] * 8, id="Nb8-split"),
    pytest.param(3, 16, 20, [5, 70, 1, 33, 9, 64, 17, 2, 40, 8, 3, 90, 12], id="Nb13-dim20"),
    pytest.param(2, 32, 256, [65, 129, 7, 1, 300, 31, 16, 48, 90, 2, 77], id="Nb11-dim256"),
    pytest.param(600, 32, 128, [64, 10, 200, 33, 1, 128, 90, 47, 300, 5], id="Nq600-dim-parts"),
    # more query tokens than one dd entry pass holds: passes over token chunks
    pytest.param(1, 20000, 8, [3, 17, 1, 40, 9, 2, 5, 11], id="Lq20000-token-chunks"),
]


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda t: str(t).split(".")[-1])
@pytest.mark.parametrize("Nq,Lq,dim,d_lens", BWD_SPLIT)
def test_contrastive_backward_split(Nq, Lq, dim, d_lens, dtype):
    q, d, off = make_contrastive(Nq, Lq, dim, d_lens, dtype, seed=Nq + dim)
    gen = torch.Generator().manual_seed(9)
    dscore = torch.randn(Nq, len(d_lens), generator=gen).to(DEVICE)
    _, argmax = maxsim_amd.score_contrastive_with_argmax(q, d, off)
    dq, dd = ops.maxsim_contrastive_backward(dscore, q, d, off, argmax)
    dq_ref, dd_ref = oracle.contrastive_backward(np64(dscore), np64(q), np64(d), npi(off), npi(argmax))
    assert_close(dq, dq_ref, **GRAD_TOL[dtype])
    assert_close(dd, dd_ref, **GRAD_TOL[dtype])


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda t: str(t).split(".")[-1])
@pytest.mark.parametrize("d_lens", [[48, 48, 48], [47, 5, 33]])
def test_contrastive_first_index_wins_on_ties(dtype, d_lens):
    """All document rows identical -> every argmax is 0 (test_contrastive.py:70-95),
    here for any Ld (no tile-size restriction: one MFMA path, no scalar tail)."""
    gen = torch.Generator().manual_seed(7)
    q = torch.randn(2, 16, 32, generator=gen).to(dtype).to(DEVICE)
    base = torch.randn(32, generator=gen).to(dtype)
    d = base.expand(sum(d_lens), 32).contiguous().to(DEVICE)
    off = torch.zeros(len(d_lens) + 1, dtype=torch.int32)
    off[1:] = torch.tensor(d_lens).cumsum(0)
    _, argmax = maxsim_amd.score_contrastive_with_argmax(q, d, off.to(DEVICE))
    assert torch.all(argmax == 0)


def test_contrastive_duplicate_rows_pick_first_copy():
    """Exact duplicates later in a document never win (C5's tie rule)."""
    gen = torch.Generator().manual_seed(11)
    lens = [300, 129, 64]
    q = torch.nn.functional.normalize(torch.randn(4, 32, 128, generator=gen), dim=-1)
    d = torch.nn.functional.normalize(torch.randn(sum(lens), 128, generator=gen), dim=-1)
    off = torch.zeros(4, dtype=torch.int32)
    off[1:] = torch.tensor(lens).cumsum(0)
    # duplicate: rows 100..299 of doc 0 are copies of rows 0..99
    d[100:200] = d[0:100]
    d[200:300] = d[0:100]
    q, d, off = q.to(torch.bfloat16).to(DEVICE), d.to(torch.bfloat16).to(DEVICE), off.to(DEVICE)
    _, argmax = maxsim_amd.score_contrastive_with_argmax(q, d, off)
    assert int(argmax[:, 0].max()) < 100
    _, a_ref = oracle.contrastive_forward(np64(q), np64(d), npi(off))
    assert np.array_equal(npi(argmax)[:, 0], a_ref[:, 0])


def test_contrastive_nan_gives_neg_inf():
    """NaN in a query -> -inf for that query, finite elsewhere (test_nan_inf.py:33-92)."""
    torch.manual_seed(0)
    q = torch.randn(2, 16, 64, device=DEVICE, dtype=torch.float16)
    d = torch.randn(3 * 32, 64, device=DEVICE, dtype=torch.float16)
    cu = torch.arange(0, 4 * 32, 32, dtype=torch.int32, device=DEVICE)
    q[1, 0, 0] = float("nan")
    s = maxsim_amd.score_contrastive(q, d, cu)
    assert torch.isinf(s[1]).all() and (s[1] < 0).all()
    assert torch.isfinite(s[0]).all()
    s2, a2 = maxsim_amd.score_contrastive_with_argmax(q, d, cu)
    assert torch.equal(a2[1, :, 0], torch.zeros_like(a2[1, :, 0]))


def test_contrastive_inf_propagates():
    torch.manual_seed(1)
    q = torch.randn(1, 16, 64, device=DEVICE, dtype=torch.float16)
    d = torch.randn(2 * 32, 64, device=DEVICE, dtype=torch.float16).abs()
    cu = torch.arange(0, 3 * 32, 32, dtype=torch.int32, device=DEVICE)
    q[0, 0] = float("inf")
    s = maxsim_amd.score_contrastive(q, d, cu)
    assert torch.isinf(s).all() and (s > 0).all()


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda t: str(t).split(".")[-1])
def test_contrastive_zero_dscore(dtype):
    q, d, off = make_contrastive(1, 16, 32, [16, 16], dtype, seed=3)
    _, argmax = maxsim_amd.score_contrastive_with_argmax(q, d, off)
    dq, dd = ops.maxsim_contrastive_backward(torch.zeros(1, 2, device=DEVICE), q, d, off, argmax)
    assert torch.all(dq == 0) and torch.all(dd == 0)


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda t: str(t).split(".")[-1])
def test_contrastive_train_end_to_end(dtype):
    q, d, off = make_contrastive(2, 16, 64, [40, 64, 20, 80], dtype, seed=4)
    q.requires_grad_(True)
    d.requires_grad_(True)
    scores = maxsim_amd.score_contrastive_train(q, d, off)
    w = torch.randn(2, 4, generator=torch.Generator().manual_seed(5)).to(DEVICE)
    (scores * w).sum().backward()
    s_ref, a_ref = oracle.contrastive_forward(np64(q), np64(d), npi(off))
    dq_ref, dd_ref = oracle.contrastive_backward(np64(w), np64(q), np64(d), npi(off), a_ref)
    assert q.grad.dtype == dtype
    tol = GRAD_TOL[dtype] if dtype == torch.float32 else dict(rtol=1e-2, atol=1e-2)
    assert_close(q.grad, dq_ref, **tol)
    assert_close(d.grad, dd_ref, **tol)


TYPED = [
    pytest.param(3, 16, 64, [37, 64, 200, 17, 81], id="Nb5-gather"),
    pytest.param(4, 32, 128, [40, 1, 300, 33, 90, 64, 7, 129, 2], id="Nb9-split"),
    pytest.param(2, 7, 20, [9, 33, 5, 1, 2, 70, 3, 8], id="dim20-element-wise"),
    pytest.param(600, 32, 128, [64, 10, 200, 33, 1, 128, 90, 47, 300, 5], id="Nq600-lds-pass"),
    pytest.param(1200, 32, 64, [64, 10, 200, 33, 1, 28, 9], id="Nq1200-fp32-fallback"),
    pytest.param(1, 20000, 8, [3, 17, 1, 40, 9, 2, 5, 11], id="Lq20000-fp32-fallback"),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bfloat16", "float16"])
@pytest.mark.parametrize("Nq,Lq,dim,d_lens", TYPED)
def test_contrastive_backward_typed_equals_cast_fp32(Nq, Lq, dim, d_lens, dtype):
    """The autograd path's operator writes the gradients in the input dtype;
    they must be the fp32 operator's gradients cast by torch (round to
    nearest even).  dq is summed in a fixed order, so it is bit-identical;
    dd's bucket order can differ between runs, which changes fp32 last bits
    (by far more than a last bit, relative to the sum, where terms of both
    signs cancel)."""
    q, d, off = make_contrastive(Nq, Lq, dim, d_lens, dtype, seed=Nq * 7 + dim)
    gen = torch.Generator().manual_seed(21)
    dscore = torch.randn(Nq, len(d_lens), generator=gen).to(DEVICE)
    _, argmax = maxsim_amd.score_contrastive_with_argmax(q, d, off)
    dq32, dd32 = ops.maxsim_contrastive_backward(dscore, q, d, off, argmax)
    dq, dd = ops.maxsim_contrastive_backward_typed(dscore, q, d, off, argmax)
    assert dq.dtype == dtype and dd.dtype == dtype
    assert dq.shape == dq32.shape and dd.shape == dd32.shape
    assert torch.equal(dq, dq32.to(dtype))
    # absolute term sums of dd: the same routing with |dscore| and |q|
    _, mag = ops.maxsim_contrastive_backward(dscore.abs(), q.abs(), d, off, argmax)
    assert_rounded_from(dd, dd32, mag)


def test_contrastive_backward_typed_special_values_bits():
    """16-bit gradients of score gradients with +NaN, -NaN, +-inf, signed
    zeros and values whose products are fp32 denormals: the bits of the fp32
    gradients cast by torch (every NaN becomes 0x7FC0, denormals round to
    nearest even).  dq is summed in a fixed order; dd rows that receive one
    entry have no order to differ in."""
    q, d, off = make_contrastive(3, 8, 64, [40, 50, 33, 64, 100], torch.bfloat16, seed=41)
    nan = float("nan")
    dscore = torch.tensor([[nan, 0.5, -1e-39, 2.0, -0.0],
                           [-1e-39, 3e-41, 1e-40, -7e-40, 2e-41],
                           [1.0, -float("inf"), 0.0, -nan, 0.125]], device=DEVICE)
    assert torch.signbit(dscore[2, 3])
    _, argmax = maxsim_amd.score_contrastive_with_argmax(q, d, off)
    dq32, dd32 = ops.maxsim_contrastive_backward(dscore, q, d, off, argmax)
    dq, dd = ops.maxsim_contrastive_backward_typed(dscore, q, d, off, argmax)
    assert torch.isnan(dq32).any() and torch.isnan(dq).any()
    assert (dq32.abs() < 1.1754944e-38).logical_and(dq32 != 0).any()   # fp32 denormals
    assert torch.equal(dq.view(torch.int16), dq32.to(torch.bfloat16).view(torch.int16))
    on, am = npi(off), npi(argmax)
    hits = np.zeros(d.shape[0], dtype=np.int64)
    for b in range(len(on) - 1):
        np.add.at(hits, on[b] + am[:, b, :].reshape(-1), 1)
    single = torch.from_numpy(hits == 1).to(DEVICE)
    assert single.sum() >= 40
    assert torch.equal(dd[single].view(torch.int16), dd32[single].to(torch.bfloat16).view(torch.int16))
    assert torch.all(dd[torch.from_numpy(hits == 0).to(DEVICE)].view(torch.int16) == 0)


def test_contrastive_backward_typed_single_pass_limit():
    """Through the C ABI: 16-bit gradients for Nq * (Lq + 1) = 19,800 entries
    (beyond an 80 KB LDS pass, within the 160 KB a workgroup may use) are
    written directly; 39,600 entries return MAXSIM_ERR_UNSUPPORTED before
    any launch (the operator then takes the fp32 kernels and a cast)."""
    import ctypes
    from pathlib import Path

    lib = ctypes.CDLL(str(Path(maxsim_amd.__file__).resolve().parent / "libmaxsim_amd.so"))
    lib.maxsim_amd_last_error.restype = ctypes.c_char_p
    I64, P = ctypes.c_int64, ctypes.c_void_p
    fn = lib.maxsim_amd_contrastive_backward_typed
    fn.argtypes = [ctypes.c_int, ctypes.c_int, P, P, I64, I64, P, I64, P, I64, P, I64, P, P, P,
                   ctypes.c_size_t, P]
    BF16 = 2
    for nq, ok in ((600, True), (1200, False)):
        q, d, off = make_contrastive(nq, 32, 64, [64, 10, 200, 33], torch.bfloat16, seed=nq)
        _, argmax = ops.maxsim_contrastive_forward_with_argmax(q, d, off)
        dscore = torch.randn(nq, 4, generator=torch.Generator().manual_seed(1)).to(DEVICE)
        dq = torch.empty_like(q)
        dd = torch.empty_like(d)
        rc = fn(BF16, BF16, dscore.data_ptr(), q.data_ptr(), nq, 32, d.data_ptr(), d.shape[0],
                off.data_ptr(), 4, argmax.data_ptr(), 64, dq.data_ptr(), dd.data_ptr(), None, 0,
                torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        if ok:
            assert rc == 0, lib.maxsim_amd_last_error()
            dq32, dd32 = ops.maxsim_contrastive_backward(dscore, q, d, off, argmax)
            _, mag = ops.maxsim_contrastive_backward(dscore.abs(), q.abs(), d, off, argmax)
            assert_rounded_from(dd, dd32, mag)
        else:
            assert rc != 0 and b"16-bit" in lib.maxsim_amd_last_error()


def test_contrastive_backward_typed_fp32_inputs_are_fp32():
    q, d, off = make_contrastive(2, 16, 32, [16, 40], torch.float32, seed=5)
    dscore = torch.randn(2, 2, generator=torch.Generator().manual_seed(2)).to(DEVICE)
    _, argmax = maxsim_amd.score_contrastive_with_argmax(q, d, off)
    dq, dd = ops.maxsim_contrastive_backward_typed(dscore, q, d, off, argmax)
    dq32, dd32 = ops.maxsim_contrastive_backward(dscore, q, d, off, argmax)
    assert dq.dtype == torch.float32 and torch.equal(dq, dq32)
    torch.testing.assert_close(dd, dd32, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("grad_dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_contrastive_backward_zeroes_rows_outside_the_documents(grad_dtype):
    """With offsets that start after row 0 and end before the last row, the
    rows outside every document get a zero gradient (the reference zero-fills
    its gradient buffers), and the rows inside match the oracle.  Called
    through the C ABI into NaN-filled buffers, so an unwritten row shows."""
    import ctypes
    from pathlib import Path

    dtype = torch.bfloat16
    q, d_in, off_in = make_contrastive(3, 16, 64, [20, 33, 9], dtype, seed=13)
    pad_head, pad_tail = 5, 7
    d = torch.cat([torch.full((pad_head, 64), 3.0, dtype=dtype, device=DEVICE), d_in,
                   torch.full((pad_tail, 64), -2.0, dtype=dtype, device=DEVICE)])
    off = off_in + pad_head
    nq, lq, dim = q.shape
    nb, n = off.numel() - 1, d.shape[0]
    dscore = torch.randn(nq, nb, generator=torch.Generator().manual_seed(4)).to(DEVICE)
    _, argmax = ops.maxsim_contrastive_forward_with_argmax(q, d, off)
    dq = torch.full((nq, lq, dim), float("nan"), dtype=grad_dtype, device=DEVICE)
    dd = torch.full((n, dim), float("nan"), dtype=grad_dtype, device=DEVICE)
    lib = ctypes.CDLL(str(Path(maxsim_amd.__file__).resolve().parent / "libmaxsim_amd.so"))
    I64, P = ctypes.c_int64, ctypes.c_void_p
    fn = lib.maxsim_amd_contrastive_backward_typed
    fn.argtypes = [ctypes.c_int, ctypes.c_int, P, P, I64, I64, P, I64, P, I64, P, I64, P, P, P,
                   ctypes.c_size_t, P]
    BF16, F32 = 2, 0
    rc = fn(BF16, F32 if grad_dtype == torch.float32 else BF16, dscore.data_ptr(), q.data_ptr(),
            nq, lq, d.data_ptr(), n, off.data_ptr(), nb, argmax.data_ptr(), dim, dq.data_ptr(),
            dd.data_ptr(), None, 0, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.all(dd[:pad_head] == 0) and torch.all(dd[n - pad_tail:] == 0)
    dq_ref, dd_ref = oracle.contrastive_backward(np64(dscore), np64(q), np64(d_in), npi(off_in),
                                                 npi(argmax))
    assert_close(dd[pad_head:n - pad_tail].float(), dd_ref, rtol=1e-2, atol=1e-3)
    assert_close(dq.float(), dq_ref, rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("nb,lo,hi", [(5000, 1, 24), (2, 300, 700), (40, 1, 3000)],
                         ids=["5000-small-docs", "2-docs", "40-docs-skewed"])
def test_contrastive_work_balanced_chunks(nb, lo, hi):
    """The tiled forward splits the documents into chunks of equal work (rows
    plus a per-document share), found on the device: many small documents
    (more chunks than one per CU, to respect the offset table), fewer
    documents than chunks (empty chunks), and skewed lengths."""
    gen = torch.Generator().manual_seed(nb)
    lens = torch.randint(lo, hi + 1, (nb,), generator=gen).tolist()
    q, d, off = make_contrastive(3, 32, 128, lens, torch.bfloat16, seed=nb + 1, unit=True)
    scores, argmax = maxsim_amd.score_contrastive_with_argmax(q, d, off)
    _check_forward(q, d, off, scores, argmax)


@pytest.mark.parametrize("nq,nb,lo,hi,n_long", [
    (64, 300, 1, 1500, 0), (1, 511, 1, 700, 0), (16, 512, 100, 1100, 5), (64, 65, 1, 40, 0)],
    ids=["64q-300-skewed", "1q-511", "16q-512-long", "64q-65-short"])
def test_contrastive_dealt_chunks(nq, nb, lo, hi, n_long):
    """At most 512 documents and more chunks than one: the documents are
    ranked by tile count on the device (every workgroup the same ranks;
    counts past 127 tiles share one key, ties by index) and dealt to the
    chunks in snake order.  Every (query, document) score comes from exactly
    one workgroup: checked against the oracle, with documents longer than
    127 tiles and documents of one row."""
    gen = torch.Generator().manual_seed(nb * 7 + nq)
    lens = torch.randint(lo, hi + 1, (nb,), generator=gen)
    lens[torch.randperm(nb, generator=gen)[:n_long]] = torch.randint(4100, 6000, (n_long,),
                                                                      generator=gen)
    lens[nb // 2] = 1
    q, d, off = make_contrastive(nq, 32, 128, lens.tolist(), torch.bfloat16, seed=nb + 5,
                                 unit=True)
    scores, argmax = maxsim_amd.score_contrastive_with_argmax(q, d, off)
    _check_forward(q, d, off, scores, argmax)
    assert torch.equal(maxsim_amd.score_contrastive(q, d, off), scores)


@pytest.mark.parametrize("dim,dtype", [(32, torch.bfloat16), (64, torch.float32), (128, torch.float16)],
                         ids=["d32-bf16", "d64-fp32", "d128-fp16"])
def test_contrastive_dealt_chunks_other_shapes(dim, dtype):
    """The dealt chunks at the other tile shapes the tiled kernel takes: the
    ranking's scratch sits in the tile ring, smallest at dim 32 in bf16."""
    gen = torch.Generator().manual_seed(dim)
    lens = torch.randint(1, 900, (257,), generator=gen)
    q, d, off = make_contrastive(64, 32, dim, lens.tolist(), dtype, seed=dim + 3, unit=True)
    scores, argmax = maxsim_amd.score_contrastive_with_argmax(q, d, off)
    _check_forward(q, d, off, scores, argmax)


def test_contrastive_dealt_chunks_invalid_offsets_at_the_operator_level():
    """The dealt chunks with offsets that decrease at a few documents (called
    past the Python checks): those documents rank last (no tiles), get a NaN
    score and argmax 0; the others their MaxSim."""
    nb = 300
    gen = torch.Generator().manual_seed(5)
    lens = torch.randint(20, 400, (nb,), generator=gen)
    q, d, off = make_contrastive(64, 32, 64, lens.tolist(), torch.bfloat16, seed=9, unit=True)
    off = off.clone()
    bad_docs = [10, 11, 150]
    off_h = off.cpu()
    for b in bad_docs:
        off_h[b + 1] = off_h[b] - 1          # end before start: document b invalid
    off = off_h.to(DEVICE)
    scores, argmax = ops.maxsim_contrastive_forward_with_argmax(q, d, off)
    invalid = set()
    on = npi(off)
    for b in range(nb):
        if not (on[b] >= 0 and on[b + 1] > on[b] and on[b + 1] <= d.shape[0]):
            invalid.add(b)
    assert invalid >= set(bad_docs)
    bad = torch.tensor(sorted(invalid), device=DEVICE)
    assert torch.isnan(scores[:, bad]).all() and torch.all(argmax[:, bad] == 0)
    good = [b for b in range(nb) if b not in invalid]
    qn, dn = np64(q), np64(d)
    for b in good[::37]:
        s_ref, _ = oracle.contrastive_forward(qn, dn[on[b]:on[b + 1]],
                                              np.array([0, on[b + 1] - on[b]], dtype=np.int64))
        assert_close(scores[:, b:b + 1], s_ref, **SCORE_TOL[torch.bfloat16])


def test_contrastive_malformed_offsets_at_the_operator_level():
    """Offsets that decrease (the Python layer rejects them; the operator is
    called directly): documents with an invalid range get a NaN score and
    argmax 0, the valid ones their MaxSim, and nothing is read out of range."""
    q, d, _ = make_contrastive(2, 32, 64, [20, 20], torch.bfloat16, seed=17)
    off = torch.tensor([0, 10, 5, 20], dtype=torch.int32, device=DEVICE)
    scores, argmax = ops.maxsim_contrastive_forward_with_argmax(q, d, off)
    assert torch.isnan(scores[:, 1]).all()
    assert torch.all(argmax[:, 1] == 0)
    qn, dn = np64(q), np64(d)
    for b, (s0, e0) in [(0, (0, 10)), (2, (5, 20))]:
        s_ref, a_ref = oracle.contrastive_forward(qn, dn[s0:e0], np.array([0, e0 - s0], dtype=np.int64))
        assert_close(scores[:, b:b + 1], s_ref, **SCORE_TOL[torch.bfloat16])
        check_argmax(npi(argmax[:, b:b + 1]), a_ref, lambda idx: qn[idx[0], idx[2]],
                     lambda idx, j, s0=s0: dn[s0 + j])


CONTRASTIVE_FNS = [maxsim_amd.score_contrastive, maxsim_amd.score_contrastive_with_argmax,
                   maxsim_amd.score_contrastive_train]


@pytest.mark.parametrize("fn", CONTRASTIVE_FNS, ids=lambda f: f.__name__)
@pytest.mark.parametrize("bad,pattern", [
    ([1, 33, 65, 97, 129], "0|start|offset"),
    ([0, 32, 16, 96, 128], "monoton|decreas|order|offset"),
    ([0, 25, 50, 75, 100], "total|match|offset"),
    ([0, 0, 64, 96, 128], "strictly|empty|offset"),
    ([-5, 32, 64, 96, 140], "0|start|offset"),
])
def test_contrastive_bad_device_offsets_raise_after_queueing(fn, bad, pattern):
    """Device offsets are checked on the host while the kernels already run
    (the check waits only for their copy): bad offsets still raise the
    reference's ValueError, the queued kernels are safe with them, and the
    device is in a good state afterwards."""
    q, d, _ = make_contrastive(2, 16, 32, [32, 32, 32, 32], torch.float16, seed=3)
    with pytest.raises(ValueError, match=pattern):
        fn(q, d, torch.tensor(bad, dtype=torch.int32, device=DEVICE))
    torch.cuda.synchronize()
    good = torch.tensor([0, 32, 64, 96, 128], dtype=torch.int32, device=DEVICE)
    _check_forward(q, d, good, maxsim_amd.score_contrastive(q, d, good), None)


def test_contrastive_decreasing_offsets_overflowing_a_chunk():
    """3000 documents whose offsets decrease so that the work measure puts all
    of them in one chunk, more than the 2048-entry offset table holds: the
    chunk is reported like invalid documents (NaN score, argmax 0), with no
    out-of-range access.  (Every document here has end < start anyway.)"""
    nb = 3000
    q, d, _ = make_contrastive(2, 32, 128, [4096], torch.bfloat16, seed=23)
    off = (100000 - 32 * torch.arange(nb + 1, dtype=torch.int64)).to(torch.int32).to(DEVICE)
    scores, argmax = ops.maxsim_contrastive_forward_with_argmax(q, d, off)
    torch.cuda.synchronize()
    assert torch.isnan(scores).all()
    assert torch.all(argmax == 0)


def test_contrastive_validation_sees_writes_queued_just_before():
    """Offsets made invalid by a device write queued right before the call,
    behind a long kernel, are seen by the overlapped validation and
    rejected."""
    q, d, _ = make_contrastive(2, 16, 32, [32, 32, 32, 32], torch.float16, seed=4)
    off = torch.tensor([0, 32, 64, 96, 128], dtype=torch.int32, device=DEVICE)
    torch.cuda.synchronize()
    a = torch.randn(4096, 4096, device=DEVICE)
    for _ in range(4):
        a = a @ a / 64.0  # keeps the current stream busy for a while
    off[2] = -5
    with pytest.raises(ValueError):
        maxsim_amd.score_contrastive(q, d, off)
    torch.cuda.synchronize()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_contrastive_backward_skewed_buckets(dtype):
    """Document 0 holds a large row v and its negation -v: nearly every
    query token picks one of the two (|<v, q>| dominates), so two rows of
    document 0 receive almost all of its 5120 entries (far above the largest row size class
    of the dD row order, which documents of >= 4096 entries use) and its
    other rows none.  fp32 and typed gradients against the oracle; the typed
    ones are the fp32 ones rounded."""
    Nq, Lq, dim, d_lens = 160, 32, 128, [300, 40, 128, 700]
    q, d, off = make_contrastive(Nq, Lq, dim, d_lens, dtype, seed=29)
    v = torch.randn(dim, generator=torch.Generator().manual_seed(30)) * 100
    d[5] = v.to(dtype).to(DEVICE)
    d[6] = (-v).to(dtype).to(DEVICE)
    gen = torch.Generator().manual_seed(31)
    dscore = torch.randn(Nq, len(d_lens), generator=gen).to(DEVICE)
    _, argmax = maxsim_amd.score_contrastive_with_argmax(q, d, off)
    a0 = argmax[:, 0, :]
    assert float(((a0 == 5) | (a0 == 6)).float().mean()) > 0.9  # tokens almost orthogonal to v
    picked = torch.zeros(d_lens[0], dtype=torch.bool, device=DEVICE)
    picked[a0.reshape(-1).long()] = True
    dq, dd = ops.maxsim_contrastive_backward(dscore, q, d, off, argmax)
    dq_ref, dd_ref = oracle.contrastive_backward(np64(dscore), np64(q), np64(d), npi(off),
                                                 npi(argmax))
    tol = GRAD_TOL[dtype]
    assert_close(dq, dq_ref, **tol)
    # the two hot rows sum ~2560 terms each: tolerance scaled by their size
    assert_close(dd, dd_ref, rtol=tol["rtol"], atol=tol["atol"] * 50)
    assert bool((dd[:d_lens[0]][~picked] == 0).all())  # rows no entry picked
    if dtype != torch.float32:
        dqt, ddt = ops.maxsim_contrastive_backward_typed(dscore, q, d, off, argmax)
        assert torch.equal(dqt, dq.to(dtype))
        _, mag = ops.maxsim_contrastive_backward(dscore.abs(), q.abs(), d, off, argmax)
        assert_rounded_from(ddt, dd, mag)


DEALT_DD = {
    "ragged": lambda g: torch.randint(1, 401, (512,), generator=g).tolist(),
    "equal-lengths": lambda g: [50] * 512,
    "long-tail": lambda g: [5000 if i % 43 == 7 else 1 + i % 13 for i in range(512)],
}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("lens", list(DEALT_DD), ids=list(DEALT_DD))
def test_contrastive_backward_dealt_documents(lens, dtype):
    """512 documents at dim 128 with 16-bit inputs: one dimension part and
    two workgroups per CU on a 256-CU device, so the dD kernel ranks the
    documents by rows and deals them (rank c and 511 - c to the workgroups
    of one CU).  Ragged lengths, all lengths equal (every rank decided by
    the document index) and a long tail past the largest key; fp32 and
    typed gradients against the oracle."""
    gen = torch.Generator().manual_seed(41)
    d_lens = DEALT_DD[lens](gen)
    Nq, Lq, dim = 8, 32, 128
    q, d, off = make_contrastive(Nq, Lq, dim, d_lens, dtype, seed=43)
    dscore = torch.randn(Nq, len(d_lens), generator=gen).to(DEVICE)
    _, argmax = maxsim_amd.score_contrastive_with_argmax(q, d, off)
    dq, dd = ops.maxsim_contrastive_backward(dscore, q, d, off, argmax)
    dq_ref, dd_ref = oracle.contrastive_backward(np64(dscore), np64(q), np64(d), npi(off),
                                                 npi(argmax))
    assert_close(dq, dq_ref, **GRAD_TOL[dtype])
    assert_close(dd, dd_ref, **GRAD_TOL[dtype])
    dqt, ddt = ops.maxsim_contrastive_backward_typed(dscore, q, d, off, argmax)
    assert torch.equal(dqt, dq.to(dtype))
    _, mag = ops.maxsim_contrastive_backward(dscore.abs(), q.abs(), d, off, argmax)
    assert_rounded_from(ddt, dd, mag)


@pytest.mark.parametrize("grad_dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_contrastive_backward_dealt_documents_with_empty_ones_and_padding(grad_dtype):
    """The dealt dD at 512 documents, called through the C ABI (no host
    checks) into NaN-filled buffers: one document in ten is empty (its rank
    is the lowest key's, its workgroup writes nothing), and rows before the
    first and after the last document are padding.  Every row of every
    document is written once -- a document dealt to no workgroup would keep
    its NaNs -- and matches the oracle; padding rows are zero."""
    import ctypes
    from pathlib import Path

    gen = torch.Generator().manual_seed(51)
    lens = torch.randint(1, 121, (512,), generator=gen)
    lens[torch.arange(512) % 10 == 3] = 0
    nq, lq, dim = 8, 32, 128
    pad_head, pad_tail = 3, 5
    total = int(lens.sum())
    q = torch.randn(nq, lq, dim, generator=gen).to(torch.bfloat16).to(DEVICE)
    d = torch.randn(pad_head + total + pad_tail, dim, generator=gen).to(torch.bfloat16).to(DEVICE)
    off_in = torch.zeros(513, dtype=torch.int32)
    off_in[1:] = lens.cumsum(0)
    off = (off_in + pad_head).to(DEVICE)
    # argmax rows drawn inside each document (0 for the empty ones)
    am = (torch.rand(nq, 512, lq, generator=gen) * lens.clamp(min=1)[None, :, None]).to(torch.int32)
    am = am.to(DEVICE)
    dscore = torch.randn(nq, 512, generator=gen).to(DEVICE)
    n = d.shape[0]
    dq = torch.full((nq, lq, dim), float("nan"), dtype=grad_dtype, device=DEVICE)
    dd = torch.full((n, dim), float("nan"), dtype=grad_dtype, device=DEVICE)
    lib = ctypes.CDLL(str(Path(maxsim_amd.__file__).resolve().parent / "libmaxsim_amd.so"))
    I64, P = ctypes.c_int64, ctypes.c_void_p
    fn = lib.maxsim_amd_contrastive_backward_typed
    fn.argtypes = [ctypes.c_int, ctypes.c_int, P, P, I64, I64, P, I64, P, I64, P, I64, P, P, P,
                   ctypes.c_size_t, P]
    BF16, F32 = 2, 0
    rc = fn(BF16, F32 if grad_dtype == torch.float32 else BF16, dscore.data_ptr(), q.data_ptr(),
            nq, lq, d.data_ptr(), n, off.data_ptr(), 512, am.data_ptr(), dim, dq.data_ptr(),
            dd.data_ptr(), None, 0, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.all(dd[:pad_head] == 0) and torch.all(dd[n - pad_tail:] == 0)
    dq_ref, dd_ref = oracle.contrastive_backward(np64(dscore), np64(q),
                                                 np64(d[pad_head:n - pad_tail]), npi(off_in),
                                                 npi(am))
    body = dd[pad_head:n - pad_tail].float()
    assert not torch.isnan(body).any()
    assert_close(body, dd_ref, rtol=1e-2, atol=1e-3)
    assert_close(dq.float(), dq_ref, rtol=1e-2, atol=1e-3)
