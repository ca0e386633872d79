"""Shared input generators, tolerances and comparison helpers for the tests.

Tolerances.  The oracle consumes exactly the (rounded) values the kernel
reads and accumulates in float64, so the only difference left is the
kernel's fp32 accumulation order.  The bars below are therefore tighter than
the north-star bounds (1e-5 relative for fp32, 2e-2 for bf16/fp16).
"""

from __future__ import annotations

import numpy as np
import torch

DEVICE = torch.device("cuda")

# Scores: relative 1e-5 (fp32) / 2e-2 (16-bit) is the contract; we test at
# 1e-5 / 1e-4 relative with a small absolute floor for near-zero scores.
SCORE_TOL = {
    torch.float32: dict(rtol=1e-5, atol=1e-4),
    torch.float16: dict(rtol=1e-4, atol=1e-3),
    torch.bfloat16: dict(rtol=1e-4, atol=1e-3),
}
# Gradients are sums of many fp32 products; same relative bars.
GRAD_TOL = {
    torch.float32: dict(rtol=1e-5, atol=1e-4),
    torch.float16: dict(rtol=1e-4, atol=1e-3),
    torch.bfloat16: dict(rtol=1e-4, atol=1e-3),
}
# Two similarities closer than this may legitimately pick different argmax
# (fp32 accumulation order); anything else must match exactly.
SIM_TIE_TOL = 1e-4

DTYPES = [torch.bfloat16, torch.float16, torch.float32]


def np64(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def npi(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy().astype(np.int64)


def normalized(gen: torch.Generator, shape, dtype) -> torch.Tensor:
    x = torch.randn(*shape, generator=gen, dtype=torch.float32)
    return torch.nn.functional.normalize(x, dim=-1).to(dtype)


def offsets_from_lengths(lengths) -> torch.Tensor:
    lens = torch.as_tensor(lengths, dtype=torch.int64)
    off = torch.zeros(lens.numel() + 1, dtype=torch.int32)
    off[1:] = lens.cumsum(0).to(torch.int32)
    return off


def make_contrastive(Nq, Lq, dim, d_lens, dtype, seed, *, unit=False, device=DEVICE):
    gen = torch.Generator().manual_seed(seed)
    total = int(sum(d_lens))
    if unit:
        q = normalized(gen, (Nq, Lq, dim), dtype)
        d = normalized(gen, (total, dim), dtype)
    else:
        q = torch.randn(Nq, Lq, dim, generator=gen).to(dtype)
        d = torch.randn(total, dim, generator=gen).to(dtype)
    return q.to(device), d.to(device), offsets_from_lengths(d_lens).to(device)


def make_padded(B, C, Lq, Ld, dim, dtype, seed, *, qlen=None, dlen=None, device=DEVICE):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Lq, dim, generator=gen).to(dtype)
    d = torch.randn(B, C, Ld, dim, generator=gen).to(dtype)
    if qlen is None:
        qlen = torch.randint(1, Lq + 1, (B,), generator=gen, dtype=torch.int32)
    if dlen is None:
        dlen = torch.randint(1, Ld + 1, (B, C), generator=gen, dtype=torch.int32)
    return (q.to(device), d.to(device), torch.as_tensor(qlen, dtype=torch.int32).to(device),
            torch.as_tensor(dlen, dtype=torch.int32).to(device))


def make_packed(nq, nd, npairs, dim, q_range, d_range, dtype, seed, device=DEVICE):
    gen = torch.Generator().manual_seed(seed)
    ql = torch.randint(q_range[0], q_range[1] + 1, (nq,), generator=gen)
    dl = torch.randint(d_range[0], d_range[1] + 1, (nd,), generator=gen)
    q = torch.randn(int(ql.sum()), dim, generator=gen).to(dtype)
    d = torch.randn(int(dl.sum()), dim, generator=gen).to(dtype)
    qids = torch.randint(0, nq, (npairs,), generator=gen, dtype=torch.int32)
    dids = torch.randint(0, nd, (npairs,), generator=gen, dtype=torch.int32)
    return (q.to(device), offsets_from_lengths(ql).to(device), d.to(device),
            offsets_from_lengths(dl).to(device), qids.to(device), dids.to(device))


def assert_close(actual: torch.Tensor, expected, **tol) -> None:
    exp = torch.as_tensor(np.asarray(expected, dtype=np.float32))
    torch.testing.assert_close(actual.detach().float().cpu(), exp, **tol)


def check_argmax(kernel_am: np.ndarray, oracle_am: np.ndarray, qvec, dvec,
                 tol: float = SIM_TIE_TOL) -> None:
    """Exact argmax equality, except where the two candidate document rows
    differ and their similarities are within ``tol`` (an fp32 near-tie).
    ``qvec(idx)`` / ``dvec(idx, j)`` return the float64 query row and document
    row for a multi-index ``idx`` of the argmax array."""
    bad = np.argwhere(kernel_am != oracle_am)
    for idx in bad:
        idx = tuple(int(x) for x in idx)
        jk, jo = int(kernel_am[idx]), int(oracle_am[idx])
        qv = qvec(idx)
        dk, do = dvec(idx, jk), dvec(idx, jo)
        assert not np.array_equal(dk, do), f"tie broken differently at {idx}: kernel {jk}, oracle {jo}"
        gap = abs(float(qv @ dk) - float(qv @ do))
        assert gap <= tol * max(1.0, abs(float(qv @ do))), (
            f"argmax mismatch at {idx}: kernel {jk}, oracle {jo}, similarity gap {gap}"
        )
    assert bad.shape[0] <= max(4, kernel_am.size // 1000), f"{bad.shape[0]} argmax mismatches"


def assert_rounded_from(typed: torch.Tensor, ref32: torch.Tensor, mag: torch.Tensor) -> None:
    """`typed` (16-bit) is `ref32` rounded to nearest, up to the fp32
    summation-order noise of a gradient whose terms have absolute sum `mag`:
    most elements are bit-identical to the cast, and every element is within
    1.5 units of the 16-bit format of ref32 plus 2^-16 * mag (far above the
    fp32 reordering error of the bucket sums, far below any real mistake)."""
    dtype = typed.dtype
    cast = ref32.to(dtype)
    same = (typed.view(torch.int16) == cast.view(torch.int16)) | ((typed == 0) & (cast == 0))
    assert float(same.float().mean()) > 0.99
    rel = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10
    atol = 0.0 if dtype == torch.bfloat16 else 2.0 ** -24  # fp16 subnormal spacing
    err = (typed.float() - ref32).abs()
    bound = rel * ref32.abs() + 2.0 ** -16 * mag + atol
    assert bool(torch.all(err <= bound)), float((err - bound).max())
