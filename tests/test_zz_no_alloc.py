"""The allocation-free packed backward (maxsim_amd_packed_backward_typed_noalloc).

Called through the C ABI (ctypes) on device buffers and compared with
maxsim_amd_packed_backward_typed given a caller-allocated workspace, on two
calls in a row, the second with a smaller input (the shared device scratch
keeps the first call's contents, so the second call must clear what it
needs).  Also checked against the oracle, and a size beyond the scratch is
rejected before anything is launched."""

from __future__ import annotations

import ctypes
from pathlib import Path

import pytest
import torch

import maxsim_amd
from oracle import maxsim_oracle as oracle

from ._helpers import DEVICE, GRAD_TOL, assert_close, make_packed, np64, npi

pytestmark = pytest.mark.gpu

LIB = Path(maxsim_amd.__file__).resolve().parent / "libmaxsim_amd.so"
DT = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
I64, P, SZ = ctypes.c_int64, ctypes.c_void_p, ctypes.c_size_t
COMMON = [ctypes.c_int, ctypes.c_int, P, P, I64, P, I64, P, I64, P, I64, P, P, I64, P, I64, I64,
          P, P]
SCRATCH_INTS = 4 << 20


@pytest.fixture(scope="module")
def lib():
    h = ctypes.CDLL(str(LIB))
    h.maxsim_amd_last_error.restype = ctypes.c_char_p
    h.maxsim_amd_packed_backward_workspace_size.restype = SZ
    h.maxsim_amd_packed_backward_workspace_size.argtypes = [I64, I64, I64]
    h.maxsim_amd_packed_backward_typed.argtypes = COMMON + [P, SZ, P]
    h.maxsim_amd_packed_backward_typed_noalloc.argtypes = COMMON + [P]
    return h


def _grads(lib, inputs, am, g, grad_dtype, *, noalloc):
    q, qoff, d, doff, qids, dids = inputs
    nq, nd, npairs, dim = qoff.numel() - 1, doff.numel() - 1, qids.numel(), q.shape[1]
    dq = torch.full((q.shape[0], dim), float("nan"), dtype=grad_dtype, device=DEVICE)
    dd = torch.full((d.shape[0], dim), float("nan"), dtype=grad_dtype, device=DEVICE)
    args = [DT[q.dtype], DT[grad_dtype], g.data_ptr(), q.data_ptr(), q.shape[0], qoff.data_ptr(),
            nq, d.data_ptr(), d.shape[0], doff.data_ptr(), nd, qids.data_ptr(), dids.data_ptr(),
            npairs, am.data_ptr(), am.shape[1], dim, dq.data_ptr(), dd.data_ptr()]
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        rc = lib.maxsim_amd_packed_backward_typed_noalloc(*args, stream)
    else:
        need = lib.maxsim_amd_packed_backward_workspace_size(nq, nd, npairs)
        ws = torch.full((need // 4,), -3, dtype=torch.int32, device=DEVICE)
        rc = lib.maxsim_amd_packed_backward_typed(*args, ws.data_ptr(), need, stream)
    assert rc == 0, lib.maxsim_amd_last_error()
    torch.cuda.synchronize()
    return dq, dd


@pytest.mark.parametrize("dtype,grad_dtype", [(torch.bfloat16, torch.bfloat16),
                                              (torch.bfloat16, torch.float32),
                                              (torch.float32, torch.float32)],
                         ids=["bf16-bf16grad", "bf16-fp32grad", "fp32"])
def test_noalloc_matches_workspace_entry_point(lib, dtype, grad_dtype):
    # second call smaller: fewer queries, documents and pairs
    for seed, (nq, nd, npairs) in [(31, (40, 300, 2000)), (32, (7, 23, 90))]:
        inputs = make_packed(nq, nd, npairs, 128, (4, 70), (8, 300), dtype, seed=seed)
        q, qoff, d, doff, qids, dids = inputs
        _, am = maxsim_amd.score_pairs_packed_with_argmax(q, qoff, d, doff, qids, dids)
        g = torch.randn(npairs, generator=torch.Generator().manual_seed(seed)).to(DEVICE)
        dq_n, dd_n = _grads(lib, inputs, am, g, grad_dtype, noalloc=True)
        dq_w, dd_w = _grads(lib, inputs, am, g, grad_dtype, noalloc=False)
        assert not torch.isnan(dq_n.float()).any() and not torch.isnan(dd_n.float()).any()
        # the pair lists are filled by integer atomics, so both gradients sum
        # in an order that can vary between calls: equal up to fp32 order
        tol = GRAD_TOL[torch.float32] if grad_dtype == torch.float32 else dict(rtol=1e-2, atol=1e-2)
        torch.testing.assert_close(dq_n.float(), dq_w.float(), **tol)
        torch.testing.assert_close(dd_n.float(), dd_w.float(), **tol)
        dq_ref, dd_ref = oracle.packed_backward(np64(g), np64(q), npi(qoff), np64(d), npi(doff),
                                                npi(qids), npi(dids), npi(am))
        if grad_dtype == torch.float32:
            assert_close(dq_n, dq_ref, **GRAD_TOL[dtype])
            assert_close(dd_n, dd_ref, **GRAD_TOL[dtype])
        else:
            assert_close(dq_n, dq_ref, rtol=1e-2, atol=1e-2)
            assert_close(dd_n, dd_ref, rtol=1e-2, atol=1e-2)


def test_noalloc_rejects_sizes_beyond_the_scratch(lib):
    q, qoff, d, doff, qids, dids = make_packed(3, 5, 10, 64, (2, 5), (2, 5), torch.bfloat16, seed=1)
    _, am = maxsim_amd.score_pairs_packed_with_argmax(q, qoff, d, doff, qids, dids)
    g = torch.zeros(10, device=DEVICE)
    dq = torch.empty(q.shape[0], 64, dtype=torch.bfloat16, device=DEVICE)
    dd = torch.empty(d.shape[0], 64, dtype=torch.bfloat16, device=DEVICE)
    too_many = SCRATCH_INTS // 2  # 2 * num_pairs alone exceeds the scratch
    rc = lib.maxsim_amd_packed_backward_typed_noalloc(
        DT[q.dtype], DT[q.dtype], g.data_ptr(), q.data_ptr(), q.shape[0], qoff.data_ptr(), 3,
        d.data_ptr(), d.shape[0], doff.data_ptr(), 5, qids.data_ptr(), dids.data_ptr(), too_many,
        am.data_ptr(), am.shape[1], 64, dq.data_ptr(), dd.data_ptr(),
        torch.cuda.current_stream().cuda_stream)
    assert rc == 2
    assert b"no-allocation" in lib.maxsim_amd_last_error()
