"""Contrastive backward with an argmax above 2^30 entries (over 4 GiB).

The dD kernel that holds a whole document's entries in registers addresses
the argmax with 32-bit byte offsets, so it may only take batches whose argmax
is below 2^31 bytes; larger batches must take the kernels that address it in
64 bits.  This test sits just above 2^30 entries (16 queries x 32 tokens
against 2,100,000 one-token documents, Nq * Nb * Lq = 1.075e9), where 32-bit
byte offsets would wrap and read other entries of the same buffer.

With one-token documents every argmax entry is 0, so the gradients have a
closed form that needs no oracle run over a billion entries:
    dQ[q, i] = sum_b g[q, b] * D[b]            (the same for every token i)
    dD[b]    = sum_q g[q, b] * sum_i Q[q, i]
computed here in float64 on the device."""

from __future__ import annotations

import pytest
import torch

from maxsim_amd._ops import ops

from ._helpers import DEVICE

pytestmark = pytest.mark.gpu

NQ, LQ, NB, DIM = 16, 32, 2_100_000, 128


def test_backward_above_2pow30_argmax_entries():
    assert NQ * NB * LQ > 2**30
    print(f"case: Nq={NQ} Lq={LQ} Nb={NB} dim={DIM} bf16", flush=True)
    gen = torch.Generator(device=DEVICE).manual_seed(7)
    q = torch.nn.functional.normalize(
        torch.randn(NQ, LQ, DIM, device=DEVICE, generator=gen), dim=-1).to(torch.bfloat16)
    d = torch.nn.functional.normalize(
        torch.randn(NB, DIM, device=DEVICE, generator=gen), dim=-1).to(torch.bfloat16)
    off = torch.arange(NB + 1, device=DEVICE, dtype=torch.int32)
    am = torch.zeros(NQ, NB, LQ, device=DEVICE, dtype=torch.int32)
    g = torch.randn(NQ, NB, device=DEVICE, generator=gen) * 0.01

    g64 = g.double()
    dq_ref = (g64 @ d.double()).unsqueeze(1).expand(NQ, LQ, DIM)
    dd_ref = g64.t() @ q.double().sum(dim=1)

    dq, dd = ops.maxsim_contrastive_backward(g, q, d, off, am)
    torch.cuda.synchronize()
    assert dq.dtype == torch.float32 and dd.dtype == torch.float32
    torch.testing.assert_close(dq.double(), dq_ref, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(dd.double(), dd_ref, rtol=1e-4, atol=1e-4)
    del dq, dd

    # gradients in the input dtype (the autograd path's operator)
    dq16, dd16 = ops.maxsim_contrastive_backward_typed(g, q, d, off, am)
    torch.cuda.synchronize()
    assert dq16.dtype == torch.bfloat16 and dd16.dtype == torch.bfloat16
    torch.testing.assert_close(dq16.double(), dq_ref, rtol=1e-2, atol=1e-3)
    torch.testing.assert_close(dd16.double(), dd_ref, rtol=1e-2, atol=1e-3)
