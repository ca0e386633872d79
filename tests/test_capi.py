"""The C ABI library (CPU only: loading and argument checking, no kernels).

Checks that libmaxsim_amd.so loads with ctypes, exports every function that
include/maxsim_amd.h declares, and rejects bad arguments with the documented
status codes before touching the GPU."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "maxsim_amd.h"
LIB = ROOT / "maxsim_amd" / "libmaxsim_amd.so"

OK, INVALID, UNSUPPORTED = 0, 1, 2
F32, F16, BF16 = 0, 1, 2


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(maxsim_amd_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    if not LIB.exists():
        pytest.fail(f"{LIB} is not built; run python maxsim_amd/_build.py")
    handle = ctypes.CDLL(str(LIB))
    handle.maxsim_amd_last_error.restype = ctypes.c_char_p
    return handle


def test_header_declares_the_nine_ops_plus_helpers():
    names = declared_functions()
    assert len(names) == 22, names
    for op in ["forward", "packed_forward_with_argmax", "packed_backward", "padded_forward",
               "padded_forward_with_argmax", "padded_backward", "contrastive_forward",
               "contrastive_forward_with_argmax", "contrastive_backward"]:
        assert f"maxsim_amd_{op}" in names


def test_every_declared_symbol_is_exported(lib):
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in the header but not exported"


def test_abi_version(lib):
    assert lib.maxsim_amd_abi_version() == 10


def test_contrastive_backward_workspace_size(lib):
    fn = lib.maxsim_amd_contrastive_backward_workspace_size
    fn.restype = ctypes.c_size_t
    fn.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64]
    # eight fp32 partial copies of dq [Nq, Lq, dim]
    assert fn(512, 32, 128) == 8 * 512 * 32 * 128 * 4
    assert fn(3, 5, 7) == 8 * 3 * 5 * 7 * 4
    assert fn(4, 32, 2048) == 8 * 4 * 32 * 2048 * 4
    # above 2048 the backward always takes the single-pass gather
    for bad in [(0, 32, 128), (4, 0, 128), (4, 32, 0), (4, 32, 2049), (-1, 32, 128)]:
        assert fn(*bad) == 0


def test_packed_backward_workspace_size(lib):
    fn = lib.maxsim_amd_packed_backward_workspace_size
    fn.restype = ctypes.c_size_t
    fn.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64]
    # group starts + cursors for queries and documents, two pair lists (int32)
    assert fn(512, 8192, 20000) == 4 * (2 * 512 + 1 + 2 * 8192 + 1 + 2 * 20000)
    assert fn(0, 0, 0) == 8
    assert fn(-1, 4, 4) == 0


def test_packed_forward_workspace_size(lib):
    fn = lib.maxsim_amd_packed_forward_workspace_size
    fn.restype = ctypes.c_size_t
    fn.argtypes = [ctypes.c_int64, ctypes.c_int64]
    # 64-byte chunk records for ceil(P / 4) + min(nd, P) chunks, the chunk
    # count (16 bytes), int32 per document (pairs, first chunk) and per pair
    # (place in its document), to a 16-byte boundary; then 16 x 256 int32
    # chunk counts per (document range, length class) and one class byte per
    # document
    def r16(x):
        return (x + 15) // 16 * 16
    assert fn(8192, 20000) == r16(64 * (5000 + 8192) + 16 + 8 * 8192 + 4 * 20000) + 16384 + 8192
    assert fn(3, 4097) == r16(64 * (1025 + 3) + 16 + 8 * 3 + 4 * 4097) + 16384 + 3
    assert fn(3, 4097) % 16 == 3 and fn(0, 0) == 16 + 16384
    assert fn(-1, 4) == 0 and fn(4, -1) == 0


I64 = ctypes.c_int64
P = ctypes.c_void_p


def _contrastive(lib, dtype=BF16, nq=2, lq=16, total=64, nb=2, dim=64, ptr=1, argmax=True):
    fn = lib.maxsim_amd_contrastive_forward_with_argmax
    fn.argtypes = [ctypes.c_int, P, I64, I64, P, I64, P, I64, I64, P, P, P]
    p = P(ptr) if ptr else None
    return fn(dtype, p, nq, lq, p, total, p, nb, dim, p, p if argmax else None, None)


def test_rejects_unknown_dtype(lib):
    assert _contrastive(lib, dtype=7) == INVALID
    assert b"dtype" in lib.maxsim_amd_last_error()


def test_rejects_bad_dims(lib):
    assert _contrastive(lib, dim=0) == INVALID
    assert b"dim" in lib.maxsim_amd_last_error()
    assert _contrastive(lib, dim=16385) == UNSUPPORTED
    assert b"16384" in lib.maxsim_amd_last_error()


def test_rejects_nonpositive_lq_and_negative_sizes(lib):
    assert _contrastive(lib, lq=0) == INVALID
    assert b"Lq" in lib.maxsim_amd_last_error()
    assert _contrastive(lib, nq=-1) == INVALID


def test_rejects_null_pointers(lib):
    assert _contrastive(lib, ptr=0) == INVALID
    assert b"null" in lib.maxsim_amd_last_error()


def test_empty_problem_is_a_noop(lib):
    # zero queries: nothing to do, no device work, success
    assert _contrastive(lib, nq=0, ptr=0) == OK
    assert lib.maxsim_amd_last_error() == b""


def test_packed_rejects_bad_max_q_len(lib):
    fn = lib.maxsim_amd_packed_forward_with_argmax
    fn.argtypes = [ctypes.c_int, P, I64, P, I64, P, I64, P, I64, P, P, I64, I64, I64, P, P, P]
    one = P(1)
    assert fn(F32, one, 4, one, 1, one, 4, one, 1, one, one, 1, 8, 0, one, one, None) == INVALID
    assert b"max_q_len" in lib.maxsim_amd_last_error()


def test_padded_rejects_bad_extents(lib):
    fn = lib.maxsim_amd_padded_forward_with_argmax
    fn.argtypes = [ctypes.c_int, P, P, P, P, I64, I64, I64, I64, I64, P, P, P]
    one = P(1)
    assert fn(F16, one, one, one, one, 2, 3, 0, 8, 64, one, one, None) == INVALID
    assert fn(F16, one, one, one, one, 2, -3, 4, 8, 64, one, one, None) == INVALID


def test_backward_rejects_null_grads(lib):
    fn = lib.maxsim_amd_padded_backward
    fn.argtypes = [ctypes.c_int, P, P, P, P, P, P, I64, I64, I64, I64, I64, P, P, P]
    one = P(1)
    assert fn(BF16, one, one, one, one, one, one, 2, 3, 4, 8, 64, None, one, None) == INVALID
    assert b"null" in lib.maxsim_amd_last_error()


def _typed_backward(lib, dtype=BF16, grad_dtype=BF16, nq=2, lq=16, nb=2, dim=64):
    fn = lib.maxsim_amd_contrastive_backward_typed
    fn.argtypes = [ctypes.c_int, ctypes.c_int, P, P, I64, I64, P, I64, P, I64, P, I64, P, P, P,
                   ctypes.c_size_t, P]
    one = P(16)
    return fn(dtype, grad_dtype, one, one, nq, lq, one, 64, one, nb, one, dim, one, one, None, 0,
              None)


def test_typed_backward_rejects_a_third_grad_dtype(lib):
    # gradients are fp32 or the input dtype, nothing else
    assert _typed_backward(lib, dtype=BF16, grad_dtype=F16) == INVALID
    assert b"grad_dtype" in lib.maxsim_amd_last_error()


def test_typed_backward_16bit_needs_one_entry_pass(lib):
    # 1300 x 33 entries exceed one LDS pass of the document gradient (even
    # with all 160 KB of a gfx950 workgroup): refused before any launch, so
    # the caller can take the fp32 path
    assert _typed_backward(lib, nq=1300, lq=32) == UNSUPPORTED
    assert b"fp32" in lib.maxsim_amd_last_error()
    # one query whose tokens alone exceed a pass (token chunks): refused too
    assert _typed_backward(lib, nq=1, lq=40000) == UNSUPPORTED


def _typed_packed_backward(lib, dtype=BF16, grad_dtype=BF16, npairs=3, mql=8, ws=None, ws_bytes=0):
    fn = lib.maxsim_amd_packed_backward_typed
    fn.argtypes = [ctypes.c_int, ctypes.c_int, P, P, I64, P, I64, P, I64, P, I64, P, P, I64, P,
                   I64, I64, P, P, P, ctypes.c_size_t, P]
    one = P(16)
    return fn(dtype, grad_dtype, one, one, 10, one, 2, one, 20, one, 3, one, one, npairs, one, mql,
              64, one, one, ws, ws_bytes, None)


def test_typed_packed_backward_rejects_a_third_grad_dtype(lib):
    assert _typed_packed_backward(lib, dtype=BF16, grad_dtype=F16) == INVALID
    assert b"grad_dtype" in lib.maxsim_amd_last_error()


def test_typed_packed_backward_16bit_needs_the_grouped_path(lib):
    # without the workspace the gradients would be fp32 atomics: refused
    # before any launch, so the caller can take the fp32 path
    assert _typed_packed_backward(lib) == UNSUPPORTED
    assert b"fp32" in lib.maxsim_amd_last_error()
    # max_q_len beyond the 16-bit entry ids of the grouped kernels: refused too
    assert _typed_packed_backward(lib, mql=70000, ws=P(16), ws_bytes=1 << 20) == UNSUPPORTED


def test_typed_padded_backward_rejects_a_third_grad_dtype(lib):
    fn = lib.maxsim_amd_padded_backward_typed
    fn.argtypes = [ctypes.c_int, ctypes.c_int, P, P, P, P, P, P, I64, I64, I64, I64, I64, P, P,
                   P]
    one = P(16)
    assert fn(BF16, F16, one, one, one, one, one, one, 2, 3, 8, 16, 64, one, one, None) == INVALID
    assert b"grad_dtype" in lib.maxsim_amd_last_error()
    assert fn(F16, F16, one, one, one, one, one, one, 2, 3, 8, 16, 300, one, one, None) != OK
    # no queries: nothing to write, success without a launch
    assert fn(BF16, BF16, None, None, None, None, None, None, 0, 3, 8, 16, 64, None, None,
              None) == OK


def test_pack_rejects_bad_arguments(lib):
    fn = lib.maxsim_amd_pack_padded_rows
    fn.argtypes = [ctypes.c_int, P, I64, I64, P, P, I64, P, I64, P]
    one = P(16)
    assert fn(7, one, 2, 4, one, one, 8, one, 8, None) == INVALID
    assert fn(F32, one, -1, 4, one, one, 8, one, 8, None) == INVALID
    assert fn(F32, one, 2, 4, one, one, 0, one, 8, None) == INVALID
    assert b"dim" in lib.maxsim_amd_last_error()
    assert fn(F32, None, 2, 4, one, one, 8, one, 8, None) == INVALID
    assert b"null" in lib.maxsim_amd_last_error()
    # nothing to copy: success without touching the pointers
    assert fn(F32, None, 0, 4, None, None, 8, None, 0, None) == OK
    # more padded bytes per segment than one launch covers
    assert fn(F32, one, 2, 1 << 28, one, one, 256, one, 8, None) == UNSUPPORTED


def test_cross_entropy_entry_points_reject_bad_arguments(lib):
    """The fused loss's forward and backward check their arguments before
    touching the device."""
    fwd = lib.maxsim_amd_cross_entropy_forward
    fwd.argtypes = [P, I64, I64, P, ctypes.c_float, ctypes.c_int, P, P, P]
    one = P(16)
    assert fwd(one, 4, 8, None, 1.0, 3, one, one, None) == INVALID      # reduction
    assert b"reduction" in lib.maxsim_amd_last_error()
    assert fwd(one, 4, 8, None, 0.0, 1, one, one, None) == INVALID      # temperature
    assert fwd(one, 4, 8, None, float("inf"), 1, one, one, None) == INVALID
    assert fwd(one, 9, 8, None, 1.0, 1, one, one, None) == INVALID      # diagonal needs Nq <= Nb
    assert b"diagonal" in lib.maxsim_amd_last_error()
    assert fwd(one, -1, 8, None, 1.0, 1, one, one, None) == INVALID
    assert fwd(None, 4, 8, None, 1.0, 1, one, one, None) == INVALID
    bwd = lib.maxsim_amd_contrastive_ce_backward_typed
    bwd.argtypes = [ctypes.c_int, ctypes.c_int, P, P, P, P, ctypes.c_int, ctypes.c_float,
                    P, I64, I64, P, I64, P, I64, P, I64, P, P, P, ctypes.c_size_t, P]
    args = [BF16, BF16, one, one, None, one, 1, 1.0, one, 2, 16, one, 64, one, 2, one, 64,
            one, one, None, 0, None]
    bad = list(args); bad[6] = 5
    assert bwd(*bad) == INVALID
    bad = list(args); bad[7] = -1.0
    assert bwd(*bad) == INVALID
    bad = list(args); bad[2] = None
    assert bwd(*bad) == INVALID
    bad = list(args); bad[9] = 3                                           # Nq > Nb, diagonal
    assert bwd(*bad) == INVALID
