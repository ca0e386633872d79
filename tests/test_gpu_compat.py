"""Training-loop compatibility on the GPU (reference tests/test_compat.py):
``torch.autocast`` around the training entry points, ``torch.compile`` of a
training step, and non-contiguous inputs."""

from __future__ import annotations

import pytest
import torch

import maxsim_amd
from oracle import maxsim_oracle as oracle

from ._helpers import DEVICE, SCORE_TOL, assert_close, np64, npi

pytestmark = pytest.mark.gpu


def _padded(dt, seed, B=2, C=4, Lq=16, Ld=32, D=64):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Lq, D, generator=g).to(dt).to(DEVICE)
    d = torch.randn(B, C, Ld, D, generator=g).to(dt).to(DEVICE)
    qlen = torch.tensor([Lq - 5 * (b % 2) for b in range(B)], dtype=torch.int32, device=DEVICE)
    dlen = torch.randint(1, Ld + 1, (B, C), generator=g, dtype=torch.int32).to(DEVICE)
    return q, d, qlen, dlen


def _contrastive(dt, seed, Nq=4, Nb=4, Lq=16, Ld=32, D=64):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(Nq, Lq, D, generator=g).to(dt).to(DEVICE)
    d = torch.randn(Nb * Ld, D, generator=g).to(dt).to(DEVICE)
    cu = torch.arange(0, (Nb + 1) * Ld, Ld, dtype=torch.int32, device=DEVICE)
    return q, d, cu


def _packed(dt, seed, Nq=3, Nb=4, Lq=12, Ld=24, D=64):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(Nq * Lq, D, generator=g).to(dt).to(DEVICE)
    d = torch.randn(Nb * Ld, D, generator=g).to(dt).to(DEVICE)
    qoff = torch.arange(0, (Nq + 1) * Lq, Lq, dtype=torch.int32, device=DEVICE)
    doff = torch.arange(0, (Nb + 1) * Ld, Ld, dtype=torch.int32, device=DEVICE)
    qids = torch.tensor([0, 1, 2, 0, 1, 2], dtype=torch.int32, device=DEVICE)
    dids = torch.tensor([0, 1, 2, 3, 0, 1], dtype=torch.int32, device=DEVICE)
    return q, qoff, d, doff, qids, dids


@pytest.mark.parametrize("api", ["padded", "contrastive", "packed"])
def test_training_entry_points_inside_autocast(api):
    """Inputs at the kernels' dtype inside a bf16 autocast region: the custom
    operators have no autocast policy, so autocast must leave them alone;
    loss and gradients are finite and the gradients match the oracle."""
    dt = torch.bfloat16
    if api == "padded":
        q, d, qlen, dlen = _padded(dt, 0)
        q.requires_grad_(True)
        d.requires_grad_(True)
        with torch.autocast(device_type="cuda", dtype=dt):
            loss = maxsim_amd.score_candidates_padded_train(q, d, qlen, dlen).sum()
        loss.backward()
        _, a_ref = oracle.padded_forward(np64(q), np64(d), npi(qlen), npi(dlen))
        g = torch.ones(q.shape[0], d.shape[1], dtype=torch.float64).numpy()
        dq_ref, dd_ref = oracle.padded_backward(g, np64(q), np64(d), npi(qlen), npi(dlen), a_ref)
    elif api == "contrastive":
        q, d, cu = _contrastive(dt, 1)
        q.requires_grad_(True)
        d.requires_grad_(True)
        with torch.autocast(device_type="cuda", dtype=dt):
            loss = maxsim_amd.score_contrastive_train(q, d, cu).sum()
        loss.backward()
        _, a_ref = oracle.contrastive_forward(np64(q), np64(d), npi(cu))
        g = torch.ones(q.shape[0], cu.numel() - 1, dtype=torch.float64).numpy()
        dq_ref, dd_ref = oracle.contrastive_backward(g, np64(q), np64(d), npi(cu), a_ref)
    else:
        q, qoff, d, doff, qids, dids = _packed(dt, 2)
        q.requires_grad_(True)
        d.requires_grad_(True)
        with torch.autocast(device_type="cuda", dtype=dt):
            loss = maxsim_amd.score_pairs_packed_train(q, qoff, d, doff, qids, dids,
                                                       max_q_len=12).sum()
        loss.backward()
        _, a_ref = oracle.packed_forward(np64(q), npi(qoff), np64(d), npi(doff), npi(qids),
                                         npi(dids), 12)
        g = torch.ones(qids.numel(), dtype=torch.float64).numpy()
        dq_ref, dd_ref = oracle.packed_backward(g, np64(q), npi(qoff), np64(d), npi(doff),
                                                npi(qids), npi(dids), a_ref)
    assert torch.isfinite(loss).item()
    assert q.grad.dtype == dt and d.grad.dtype == dt
    assert_close(q.grad, dq_ref, rtol=1e-2, atol=1e-2)
    assert_close(d.grad, dd_ref, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("api", ["padded", "contrastive", "packed"])
def test_training_step_under_torch_compile(api):
    """A training step wrapped in torch.compile (default backend,
    fullgraph=False) gives the eager result: the operators are visible to
    the dispatcher with fake implementations, and the host-side checks
    become graph breaks."""
    dt = torch.float16
    if api == "padded":
        q, d, qlen, dlen = _padded(dt, 3)

        def step(q, d):
            return maxsim_amd.score_candidates_padded_train(q, d, qlen, dlen).sum()
    elif api == "contrastive":
        q, d, cu = _contrastive(dt, 4)

        def step(q, d):
            return maxsim_amd.score_contrastive_train(q, d, cu).sum()
    else:
        q, qoff, d, doff, qids, dids = _packed(dt, 5)

        def step(q, d):
            return maxsim_amd.score_pairs_packed_train(q, qoff, d, doff, qids, dids,
                                                       max_q_len=12).sum()

    eager = step(q, d)
    out = torch.compile(step, fullgraph=False)(q, d)
    torch.testing.assert_close(out, eager, rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("api", ["padded", "contrastive", "packed"])
def test_non_contiguous_inputs(api):
    """Stride-2 slices give the same scores as their contiguous copies, and
    the oracle's."""
    dt = torch.float16
    if api == "padded":
        q, d, qlen, dlen = _padded(dt, 6, B=4)
        q_nc, d_nc, ql, dl = q[::2], d[::2], qlen[::2], dlen[::2]
        assert not q_nc.is_contiguous() and not d_nc.is_contiguous()
        s_nc = maxsim_amd.score_candidates_padded(q_nc, d_nc, ql, dl)
        s_c = maxsim_amd.score_candidates_padded(q_nc.contiguous(), d_nc.contiguous(),
                                                 ql.contiguous(), dl.contiguous())
        s_ref, _ = oracle.padded_forward(np64(q_nc), np64(d_nc), npi(ql), npi(dl))
    elif api == "contrastive":
        q, _, cu = _contrastive(dt, 7, Nq=8)
        big_d = torch.randn(2 * 4 * 32, 64, generator=torch.Generator().manual_seed(8))
        q_nc, d_nc = q[::2], big_d.to(dt).to(DEVICE)[::2]
        assert not q_nc.is_contiguous() and not d_nc.is_contiguous()
        s_nc = maxsim_amd.score_contrastive(q_nc, d_nc, cu)
        s_c = maxsim_amd.score_contrastive(q_nc.contiguous(), d_nc.contiguous(), cu)
        s_ref, _ = oracle.contrastive_forward(np64(q_nc), np64(d_nc), npi(cu))
    else:
        q, qoff, d, doff, qids, dids = _packed(dt, 9)
        big_q = torch.randn(2 * q.shape[0], 64, generator=torch.Generator().manual_seed(10))
        q_nc = big_q.to(dt).to(DEVICE)[::2]
        ids_q = torch.stack([qids, qids]).t().reshape(-1)[::2]
        assert not q_nc.is_contiguous() and not ids_q.is_contiguous()
        s_nc = maxsim_amd.score_pairs_packed(q_nc, qoff, d, doff, ids_q, dids)
        s_c = maxsim_amd.score_pairs_packed(q_nc.contiguous(), qoff, d, doff,
                                           ids_q.contiguous(), dids)
        s_ref, _ = oracle.packed_forward(np64(q_nc), npi(qoff), np64(d), npi(doff),
                                         npi(ids_q), npi(dids), 12)
    assert torch.equal(s_nc, s_c)
    assert_close(s_nc, s_ref, **SCORE_TOL[dt])


def test_operators_compile_in_one_graph():
    """The operators themselves trace with their fake implementations: a
    forward, its argmax and the backward compile with fullgraph=True and
    match eager."""
    from maxsim_amd._ops import ops

    q, d, cu = _contrastive(torch.bfloat16, 11)

    def fn(q, d, cu):
        s, a = ops.maxsim_contrastive_forward_with_argmax(q, d, cu)
        dq, dd = ops.maxsim_contrastive_backward(torch.ones_like(s), q, d, cu, a)
        return s.sum() + dq.float().sum() + dd.float().sum(), a

    eager = fn(q, d, cu)
    out = torch.compile(fn, fullgraph=True)(q, d, cu)
    torch.testing.assert_close(out[0], eager[0], rtol=1e-4, atol=1e-3)
    assert torch.equal(out[1], eager[1])
