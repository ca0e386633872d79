"""The C ABI called directly (ctypes) on device buffers.

The torch operators are one caller of libmaxsim_amd.so; these tests drive the
same entry points the way a non-torch host would (raw device pointers, sizes,
a stream handle) and check the choices the ABI leaves to its caller."""

from __future__ import annotations

import ctypes
from pathlib import Path

import pytest
import torch

import maxsim_amd
from oracle import maxsim_oracle as oracle

from ._helpers import DEVICE, GRAD_TOL, assert_close, make_contrastive, np64, npi

pytestmark = pytest.mark.gpu

LIB = Path(maxsim_amd.__file__).resolve().parent / "libmaxsim_amd.so"
DT = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
I64, P, SZ = ctypes.c_int64, ctypes.c_void_p, ctypes.c_size_t


@pytest.fixture(scope="module")
def lib():
    h = ctypes.CDLL(str(LIB))
    h.maxsim_amd_last_error.restype = ctypes.c_char_p
    h.maxsim_amd_contrastive_backward_workspace_size.restype = SZ
    h.maxsim_amd_contrastive_backward_workspace_size.argtypes = [I64, I64, I64]
    h.maxsim_amd_contrastive_backward.argtypes = [
        ctypes.c_int, P, P, I64, I64, P, I64, P, I64, P, I64, P, P, P, SZ, P]
    return h


def _backward(lib, dscore, q, d, off, argmax, ws, ws_bytes):
    Nq, Lq, dim = q.shape
    dq = torch.full((Nq, Lq, dim), float("nan"), device=DEVICE)
    dd = torch.full((d.shape[0], dim), float("nan"), device=DEVICE)
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.maxsim_amd_contrastive_backward(
        DT[q.dtype], dscore.data_ptr(), q.data_ptr(), Nq, Lq, d.data_ptr(), d.shape[0],
        off.data_ptr(), off.numel() - 1, argmax.data_ptr(), dim, dq.data_ptr(), dd.data_ptr(),
        ws.data_ptr() if ws is not None else None, ws_bytes, stream)
    assert rc == 0, lib.maxsim_amd_last_error()
    torch.cuda.synchronize()
    return dq, dd


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("d_lens", [[40] * 9, [3, 200, 1, 64, 17, 90, 5, 128, 33, 2, 70, 8, 16, 9]],
                         ids=["Nb9", "Nb14-ragged"])
def test_contrastive_backward_with_and_without_workspace(lib, dtype, d_lens):
    """NULL workspace -> single-pass gather; a large enough workspace -> split
    pass; a workspace one byte short -> single pass.  All match the oracle,
    and the two dq paths differ only by fp32 summation order."""
    Nq, Lq, dim = 6, 32, 128
    q, d, off = make_contrastive(Nq, Lq, dim, d_lens, dtype, seed=21)
    _, argmax = maxsim_amd.score_contrastive_with_argmax(q, d, off)
    dscore = torch.randn(Nq, len(d_lens), generator=torch.Generator().manual_seed(2)).to(DEVICE)
    need = lib.maxsim_amd_contrastive_backward_workspace_size(Nq, Lq, dim)
    assert need == 8 * Nq * Lq * dim * 4
    ws = torch.full((need // 4,), float("nan"), device=DEVICE)
    dq0, dd0 = _backward(lib, dscore, q, d, off, argmax, None, 0)
    dq1, dd1 = _backward(lib, dscore, q, d, off, argmax, ws, need)
    dq2, dd2 = _backward(lib, dscore, q, d, off, argmax, ws, need - 1)
    dq_ref, dd_ref = oracle.contrastive_backward(np64(dscore), np64(q), np64(d), npi(off), npi(argmax))
    for dq, dd in [(dq0, dd0), (dq1, dd1), (dq2, dd2)]:
        assert_close(dq, dq_ref, **GRAD_TOL[dtype])
        assert_close(dd, dd_ref, **GRAD_TOL[dtype])
    torch.testing.assert_close(dq0, dq1, rtol=1e-6, atol=1e-6)
    # the single-pass gather is bitwise reproducible
    assert torch.equal(dq0, dq2)


@pytest.mark.parametrize("grad_dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_contrastive_backward_unaligned_dq_takes_the_scalar_reduce(lib, grad_dtype):
    """With a workspace, dD's workgroups also add dQ's eight partial sums;
    a dQ pointer that is not 16-byte aligned makes that reduce go element by
    element instead of by 16-byte groups.  Same bits either way."""
    fn = lib.maxsim_amd_contrastive_backward_typed
    fn.argtypes = [ctypes.c_int, ctypes.c_int, P, P, I64, I64, P, I64, P, I64, P, I64, P, P, P,
                   SZ, P]
    Nq, Lq, dim = 5, 32, 128
    d_lens = [40, 3, 77, 12, 64, 9, 128, 31, 50]
    q, d, off = make_contrastive(Nq, Lq, dim, d_lens, torch.bfloat16, seed=31)
    _, argmax = maxsim_amd.score_contrastive_with_argmax(q, d, off)
    dscore = torch.randn(Nq, len(d_lens), generator=torch.Generator().manual_seed(4)).to(DEVICE)
    need = lib.maxsim_amd_contrastive_backward_workspace_size(Nq, Lq, dim)
    ws = torch.empty(need // 4, device=DEVICE)
    n = Nq * Lq * dim
    es = torch.tensor([], dtype=grad_dtype).element_size()
    outs = []
    for shift in (0, 1):  # elements: 0 keeps 16-byte alignment, 1 breaks it
        buf = torch.full((n + 16,), float("nan"), device=DEVICE, dtype=grad_dtype)
        dd = torch.empty(d.shape[0], dim, device=DEVICE, dtype=grad_dtype)
        rc = fn(DT[torch.bfloat16], DT[grad_dtype], dscore.data_ptr(), q.data_ptr(), Nq, Lq,
                d.data_ptr(), d.shape[0], off.data_ptr(), len(d_lens), argmax.data_ptr(), dim,
                buf.data_ptr() + shift * es, dd.data_ptr(), ws.data_ptr(), need,
                torch.cuda.current_stream().cuda_stream)
        assert rc == 0, lib.maxsim_amd_last_error()
        torch.cuda.synchronize()
        outs.append(buf[shift:shift + n].reshape(Nq, Lq, dim).clone())
        # nothing written outside dQ's n elements
        assert torch.isnan(buf[:shift].float()).all() and torch.isnan(buf[shift + n:].float()).all()
    assert torch.equal(outs[0], outs[1])
    dq_ref, _ = oracle.contrastive_backward(np64(dscore), np64(q), np64(d), npi(off), npi(argmax))
    tol = GRAD_TOL[torch.float32] if grad_dtype == torch.float32 else dict(rtol=1e-2, atol=1e-2)
    assert_close(outs[0], dq_ref, **tol)


def test_contrastive_backward_split_is_reproducible(lib):
    q, d, off = make_contrastive(4, 32, 128, [50] * 16, torch.bfloat16, seed=5)
    _, argmax = maxsim_amd.score_contrastive_with_argmax(q, d, off)
    dscore = torch.randn(4, 16, generator=torch.Generator().manual_seed(8)).to(DEVICE)
    need = lib.maxsim_amd_contrastive_backward_workspace_size(4, 32, 128)
    ws = torch.empty(need // 4, device=DEVICE)
    dq_a, _ = _backward(lib, dscore, q, d, off, argmax, ws, need)
    ws.fill_(float("nan"))
    dq_b, _ = _backward(lib, dscore, q, d, off, argmax, ws, need)
    assert torch.equal(dq_a, dq_b)


def test_packed_backward_with_and_without_workspace(lib):
    """The grouped (workspace) and atomic (no workspace) packed backward paths
    agree with the oracle and with each other."""
    from ._helpers import make_packed

    q, qoff, d, doff, qids, dids = make_packed(9, 17, 120, 128, (4, 40), (8, 400),
                                               torch.bfloat16, seed=12)
    _, am = maxsim_amd.score_pairs_packed_with_argmax(q, qoff, d, doff, qids, dids)
    mql = am.shape[1]
    g = torch.randn(120, generator=torch.Generator().manual_seed(4)).to(DEVICE)
    fn = lib.maxsim_amd_packed_backward
    fn.argtypes = [ctypes.c_int, P, P, I64, P, I64, P, I64, P, I64, P, P, I64, P, I64, I64,
                   P, P, P, SZ, P]
    lib.maxsim_amd_packed_backward_workspace_size.restype = SZ
    lib.maxsim_amd_packed_backward_workspace_size.argtypes = [I64, I64, I64]
    need = lib.maxsim_amd_packed_backward_workspace_size(9, 17, 120)
    ws = torch.full((need // 4 + 1,), -7, dtype=torch.int32, device=DEVICE)
    out = []
    for w, nbytes in [(None, 0), (ws, need), (ws, need - 1)]:
        dq = torch.full((q.shape[0], 128), float("nan"), device=DEVICE)
        dd = torch.full((d.shape[0], 128), float("nan"), device=DEVICE)
        rc = fn(DT[q.dtype], g.data_ptr(), q.data_ptr(), q.shape[0], qoff.data_ptr(), 9,
                d.data_ptr(), d.shape[0], doff.data_ptr(), 17, qids.data_ptr(), dids.data_ptr(), 120,
                am.data_ptr(), mql, 128, dq.data_ptr(), dd.data_ptr(),
                w.data_ptr() if w is not None else None, nbytes,
                torch.cuda.current_stream().cuda_stream)
        assert rc == 0, lib.maxsim_amd_last_error()
        torch.cuda.synchronize()
        out.append((dq, dd))
    dq_ref, dd_ref = oracle.packed_backward(np64(g), np64(q), npi(qoff), np64(d), npi(doff),
                                            npi(qids), npi(dids), npi(am))
    for dq, dd in out:
        assert_close(dq, dq_ref, **GRAD_TOL[torch.bfloat16])
        assert_close(dd, dd_ref, **GRAD_TOL[torch.bfloat16])
    torch.testing.assert_close(out[0][0], out[1][0], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(out[0][1], out[1][1], rtol=1e-5, atol=1e-5)


def test_packed_backward_typed_through_the_abi(lib):
    """maxsim_amd_packed_backward_typed with bf16 gradients writes every row
    of NaN-filled buffers with the oracle's gradients (to bf16 rounding);
    without a workspace it returns ERR_UNSUPPORTED before writing anything."""
    from ._helpers import make_packed

    q, qoff, d, doff, qids, dids = make_packed(7, 11, 90, 128, (4, 40), (8, 300),
                                               torch.bfloat16, seed=21)
    _, am = maxsim_amd.score_pairs_packed_with_argmax(q, qoff, d, doff, qids, dids)
    mql = am.shape[1]
    g = torch.randn(90, generator=torch.Generator().manual_seed(5)).to(DEVICE)
    fn = lib.maxsim_amd_packed_backward_typed
    fn.argtypes = [ctypes.c_int, ctypes.c_int, P, P, I64, P, I64, P, I64, P, I64, P, P, I64, P,
                   I64, I64, P, P, P, SZ, P]
    lib.maxsim_amd_packed_backward_workspace_size.restype = SZ
    lib.maxsim_amd_packed_backward_workspace_size.argtypes = [I64, I64, I64]
    need = lib.maxsim_amd_packed_backward_workspace_size(7, 11, 90)
    ws = torch.empty(need // 4 + 1, dtype=torch.int32, device=DEVICE)

    def call(w, nbytes):
        dq = torch.full((q.shape[0], 128), float("nan"), dtype=torch.bfloat16, device=DEVICE)
        dd = torch.full((d.shape[0], 128), float("nan"), dtype=torch.bfloat16, device=DEVICE)
        rc = fn(DT[q.dtype], DT[torch.bfloat16], g.data_ptr(), q.data_ptr(), q.shape[0],
                qoff.data_ptr(), 7, d.data_ptr(), d.shape[0], doff.data_ptr(), 11,
                qids.data_ptr(), dids.data_ptr(), 90, am.data_ptr(), mql, 128, dq.data_ptr(),
                dd.data_ptr(), w, nbytes, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        return rc, dq, dd

    rc, dq, dd = call(None, 0)
    assert rc == 2 and b"fp32" in lib.maxsim_amd_last_error()
    assert torch.isnan(dq.float()).all() and torch.isnan(dd.float()).all()
    rc, dq, dd = call(ws.data_ptr(), need)
    assert rc == 0, lib.maxsim_amd_last_error()
    dq_ref, dd_ref = oracle.packed_backward(np64(g), np64(q), npi(qoff), np64(d), npi(doff),
                                            npi(qids), npi(dids), npi(am))
    assert_close(dq, dq_ref, rtol=1e-2, atol=1e-2)
    assert_close(dd, dd_ref, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_padded_backward_typed_through_the_abi(lib, dtype):
    """maxsim_amd_padded_backward_typed in the input dtype fills NaN-filled
    buffers, padding rows included, with exactly the bits of
    maxsim_amd_padded_backward's fp32 gradients cast to that dtype."""
    from ._helpers import make_padded

    B, C, Lq, Ld, D = 3, 5, 40, 90, 128
    q, d, qlen, dlen = make_padded(B, C, Lq, Ld, D, dtype, seed=27)
    _, am = maxsim_amd.score_candidates_padded_with_argmax(q, d, qlen, dlen)
    am = am.contiguous()
    g = torch.randn(B * C, generator=torch.Generator().manual_seed(6)).to(DEVICE)
    dl = dlen.reshape(-1).contiguous()
    typed = lib.maxsim_amd_padded_backward_typed
    typed.argtypes = [ctypes.c_int, ctypes.c_int, P, P, P, P, P, P, I64, I64, I64, I64, I64, P,
                      P, P]
    fp32 = lib.maxsim_amd_padded_backward
    fp32.argtypes = [ctypes.c_int, P, P, P, P, P, P, I64, I64, I64, I64, I64, P, P, P]
    stream = torch.cuda.current_stream().cuda_stream
    dq = torch.full((B * Lq, D), float("nan"), dtype=dtype, device=DEVICE)
    dd = torch.full((B * C * Ld, D), float("nan"), dtype=dtype, device=DEVICE)
    rc = typed(DT[dtype], DT[dtype], g.data_ptr(), q.data_ptr(), d.data_ptr(), qlen.data_ptr(),
               dl.data_ptr(), am.data_ptr(), B, C, Lq, Ld, D, dq.data_ptr(), dd.data_ptr(),
               stream)
    assert rc == 0, lib.maxsim_amd_last_error()
    dq32 = torch.full((B * Lq, D), float("nan"), device=DEVICE)
    dd32 = torch.full((B * C * Ld, D), float("nan"), device=DEVICE)
    rc = fp32(DT[dtype], g.data_ptr(), q.data_ptr(), d.data_ptr(), qlen.data_ptr(), dl.data_ptr(),
              am.data_ptr(), B, C, Lq, Ld, D, dq32.data_ptr(), dd32.data_ptr(), stream)
    assert rc == 0, lib.maxsim_amd_last_error()
    torch.cuda.synchronize()
    assert not torch.isnan(dq32).any() and not torch.isnan(dd32).any()
    assert torch.equal(dq.view(torch.int16), dq32.to(dtype).view(torch.int16))
    assert torch.equal(dd.view(torch.int16), dd32.to(dtype).view(torch.int16))


def test_pack_padded_rows_through_the_abi(lib):
    """maxsim_amd_pack_padded_rows copies each segment's first rows to its
    offset, bit for bit, and leaves rows past the written ones untouched."""
    fn = lib.maxsim_amd_pack_padded_rows
    fn.argtypes = [ctypes.c_int, P, I64, I64, P, P, I64, P, I64, P]
    nseg, max_len, dim = 6, 9, 24
    padded = torch.randn(nseg * max_len, dim, generator=torch.Generator().manual_seed(3)).to(
        torch.bfloat16).to(DEVICE)
    lens = torch.tensor([9, 1, 4, 7, 2, 5], dtype=torch.int32, device=DEVICE)
    offs = torch.zeros(nseg, dtype=torch.int32, device=DEVICE)
    offs[1:] = lens.cumsum(0)[:-1]
    total = int(lens.sum())
    out = torch.full((total + 3, dim), float("nan"), dtype=torch.bfloat16, device=DEVICE)
    rc = fn(DT[torch.bfloat16], padded.data_ptr(), nseg, max_len, lens.data_ptr(),
            offs.data_ptr(), dim, out.data_ptr(), total + 3,
            torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.maxsim_amd_last_error()
    torch.cuda.synchronize()
    rows = torch.cat([torch.arange(s * max_len, s * max_len + int(n))
                      for s, n in enumerate(lens.tolist())]).to(DEVICE)
    assert torch.equal(out[:total].view(torch.int16), padded[rows].view(torch.int16))
    assert torch.isnan(out[total:].float()).all()
