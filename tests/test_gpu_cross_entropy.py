"""The fused contrastive cross-entropy (score_contrastive_cross_entropy) on
the GPU against the oracle and against the unfused recipe of the reference's
README (score_contrastive_train, then F.cross_entropy; README.md:193-205)."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

import maxsim_amd
from oracle import maxsim_oracle as oracle

from ._helpers import DEVICE, GRAD_TOL, assert_close, make_contrastive, np64, npi

pytestmark = pytest.mark.gpu

_ids = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}

CASES = [
    # Nq, Lq, dim, doc lengths
    pytest.param(8, 32, 128, [40, 300, 17, 64, 128, 9, 255, 77, 31, 500], id="Nq8-Nb10"),
    pytest.param(5, 16, 64, [3, 90, 40, 12, 66], id="Nq5-Nb5-square"),
    pytest.param(6, 40, 96, [33, 70, 1, 120, 8, 45, 200], id="Lq40-dim96"),
]


def _oracle(q, d, off, targets, inv_t, reduction, upstream=None):
    qn, dn, on = np64(q), np64(d), npi(off)
    s_ref, a_ref = oracle.contrastive_forward(qn, dn, on)
    loss, dscore = oracle.cross_entropy(s_ref, None if targets is None else npi(targets), inv_t,
                                        reduction)
    if upstream is not None:
        dscore = dscore * np64(upstream)[:, None]
    dq, dd = oracle.contrastive_backward(dscore, qn, dn, on, a_ref)
    return loss, dq, dd


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=lambda t: _ids[t])
@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
@pytest.mark.parametrize("Nq,Lq,dim,d_lens", CASES)
def test_fused_cross_entropy_vs_oracle(Nq, Lq, dim, d_lens, reduction, dtype):
    q, d, off = make_contrastive(Nq, Lq, dim, d_lens, dtype, seed=Nq + dim, unit=True)
    gen = torch.Generator().manual_seed(3)
    targets = torch.randint(0, len(d_lens), (Nq,), generator=gen).to(DEVICE)
    temperature = 0.05
    qg, dg = q.clone().requires_grad_(True), d.clone().requires_grad_(True)
    loss = maxsim_amd.score_contrastive_cross_entropy(qg, dg, off, targets,
                                                      temperature=temperature,
                                                      reduction=reduction)
    upstream = None
    if reduction == "none":
        assert loss.shape == (Nq,)
        upstream = torch.randn(Nq, generator=gen).to(DEVICE)
        loss.backward(upstream)
    else:
        assert loss.shape == ()
        loss.backward()
    assert loss.dtype == torch.float32
    assert qg.grad.dtype == dtype and dg.grad.dtype == dtype
    l_ref, dq_ref, dd_ref = _oracle(q, d, off, targets, 1 / temperature, reduction, upstream)
    # scores / 0.05 are ~20x the scores: relative tolerance on the loss
    assert_close(loss, l_ref, rtol=1e-4 if dtype == torch.float32 else 2e-4, atol=1e-4)
    tol = GRAD_TOL[dtype] if dtype == torch.float32 else dict(rtol=1e-2, atol=2e-3)
    assert_close(qg.grad, dq_ref, **tol)
    assert_close(dg.grad, dd_ref, **tol)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=lambda t: _ids[t])
def test_fused_matches_unfused_recipe(dtype):
    """Diagonal targets, default temperature: the fused loss and gradients
    equal the README's two-step recipe run through this build."""
    Nq, Lq, dim = 16, 32, 128
    d_lens = [int(x) for x in torch.randint(64, 513, (Nq,), generator=torch.Generator().manual_seed(1))]
    q, d, off = make_contrastive(Nq, Lq, dim, d_lens, dtype, seed=7, unit=True)
    q1, d1 = q.clone().requires_grad_(True), d.clone().requires_grad_(True)
    loss1 = maxsim_amd.score_contrastive_cross_entropy(q1, d1, off)
    loss1.backward()
    q2, d2 = q.clone().requires_grad_(True), d.clone().requires_grad_(True)
    scores = maxsim_amd.score_contrastive_train(q2, d2, off)
    loss2 = F.cross_entropy(scores, torch.arange(Nq, device=DEVICE))
    loss2.backward()
    torch.testing.assert_close(loss1, loss2, rtol=1e-6, atol=1e-6)
    # the same fp32 sums up to the softmax's last bits, then one rounding
    torch.testing.assert_close(q1.grad.float(), q2.grad.float(), rtol=1e-2, atol=1e-4)
    torch.testing.assert_close(d1.grad.float(), d2.grad.float(), rtol=1e-2, atol=1e-4)


def test_fused_cross_entropy_c2_vs_oracle():
    """C2 (Nq = Nb = 64, Lq = 32, Ld ~ U[64, 512], bf16), diagonal targets,
    mean: loss and gradients against the oracle's forward, cross-entropy and
    backward in float64."""
    import bench

    q, d, off, _ = bench.make_c5(torch, DEVICE, seed=1, nq=64, nb=64, lo=64, hi=512, dup=0.0)
    qg, dg = q.clone().requires_grad_(True), d.clone().requires_grad_(True)
    loss = maxsim_amd.score_contrastive_cross_entropy(qg, dg, off)
    loss.backward()
    l_ref, dq_ref, dd_ref = _oracle(q, d, off, None, 1.0, "mean")
    assert_close(loss, l_ref, rtol=1e-5, atol=1e-5)
    assert_close(qg.grad, dq_ref, rtol=1e-2, atol=1e-4)
    assert_close(dg.grad, dd_ref, rtol=1e-2, atol=1e-4)


def test_fused_cross_entropy_c5():
    """C5 (Nq = Nb = 512, Lq = 32, Ld ~ U[128, 1024], bf16): fused loss and
    gradients against the unfused recipe through this build."""
    import bench

    q, d, off, _ = bench.make_c5(torch, DEVICE)
    q1, d1 = q.clone().requires_grad_(True), d.clone().requires_grad_(True)
    loss1 = maxsim_amd.score_contrastive_cross_entropy(q1, d1, off)
    loss1.backward()
    q2, d2 = q.clone().requires_grad_(True), d.clone().requires_grad_(True)
    loss2 = F.cross_entropy(maxsim_amd.score_contrastive_train(q2, d2, off),
                            torch.arange(q.shape[0], device=DEVICE))
    loss2.backward()
    torch.testing.assert_close(loss1, loss2, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(q1.grad.float(), q2.grad.float(), rtol=1e-2, atol=1e-5)
    torch.testing.assert_close(d1.grad.float(), d2.grad.float(), rtol=1e-2, atol=1e-5)
    assert torch.isfinite(q1.grad.float()).all() and torch.isfinite(d1.grad.float()).all()


def test_fused_ops_match_dscore_path():
    """The two operators of the fused loss (row log-sum-exp forward, fused
    backward) give the gradients of the plain contrastive backward fed the
    oracle's softmax gradient, here at temperature 0.5."""
    from maxsim_amd._ops import ops

    q, d, off = make_contrastive(6, 32, 64, [40, 13, 90, 200, 7, 66, 31, 18, 5], torch.bfloat16,
                                 seed=4, unit=True)
    scores, argmax = ops.maxsim_contrastive_forward_with_argmax(q, d, off)
    lse, loss = ops.maxsim_cross_entropy_forward(scores, None, 2.0, 1)
    _, dscore = oracle.cross_entropy(np64(scores), None, 2.0, "mean")
    dq_ref, dd_ref = ops.maxsim_contrastive_backward(
        torch.as_tensor(dscore, dtype=torch.float32).to(DEVICE), q, d, off, argmax)
    one = torch.ones((), device=DEVICE)
    dq, dd = ops.maxsim_contrastive_cross_entropy_backward(one, scores, lse, None, 2.0, 1, q, d,
                                                           off, argmax)
    assert_close(dq, dq_ref.cpu().numpy(), rtol=1e-2, atol=1e-5)
    assert_close(dd, dd_ref.cpu().numpy(), rtol=1e-2, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=lambda t: _ids[t])
@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
def test_value_and_grad_vs_autograd_and_oracle(reduction, dtype):
    """score_contrastive_cross_entropy_value_and_grad gives the autograd
    path's loss and gradients (the same kernels: loss and dQ bit for bit, dD
    up to the order of its bucket sums) and the oracle's."""
    Nq, Lq, dim, d_lens = 8, 32, 128, [40, 300, 17, 64, 128, 9, 255, 77, 31, 500]
    q, d, off = make_contrastive(Nq, Lq, dim, d_lens, dtype, seed=11, unit=True)
    gen = torch.Generator().manual_seed(5)
    targets = torch.randint(0, len(d_lens), (Nq,), generator=gen).to(DEVICE)
    upstream = torch.randn(Nq, generator=gen).to(DEVICE) if reduction == "none" else None
    kw = dict(temperature=0.1, reduction=reduction)
    loss, dq, dd = maxsim_amd.score_contrastive_cross_entropy_value_and_grad(
        q, d, off, targets, grad_loss=upstream, **kw)
    assert loss.shape == ((Nq,) if reduction == "none" else ())
    assert dq.dtype == dtype and dd.dtype == dtype and dq.shape == q.shape
    qg, dg = q.clone().requires_grad_(True), d.clone().requires_grad_(True)
    ref = maxsim_amd.score_contrastive_cross_entropy(qg, dg, off, targets, **kw)
    ref.backward(upstream)
    assert torch.equal(loss, ref.detach())
    assert torch.equal(dq, qg.grad)
    # dD rows add their bucket in LDS-atomic order: fp32 rounding apart
    # (or one bfloat16 step after rounding)
    scale = float(dg.grad.float().abs().max())
    torch.testing.assert_close(dd, dg.grad, rtol=1e-5 if dtype == torch.float32 else 8e-3,
                               atol=1e-6 * scale)
    l_ref, dq_ref, dd_ref = _oracle(q, d, off, targets, 10.0, reduction, upstream)
    assert_close(loss, l_ref, rtol=1e-4 if dtype == torch.float32 else 2e-4, atol=1e-4)
    tol = GRAD_TOL[dtype] if dtype == torch.float32 else dict(rtol=1e-2, atol=2e-3)
    assert_close(dq, dq_ref, **tol)
    assert_close(dd, dd_ref, **tol)


def test_value_and_grad_default_diagonal_and_no_graph():
    """Diagonal targets and grad_loss None (= 1); inputs that require grad
    get no autograd graph and no .grad."""
    q, d, off = make_contrastive(6, 32, 64, [50, 20, 90, 33, 70, 12, 8], torch.bfloat16, seed=2,
                                 unit=True)
    qg, dg = q.clone().requires_grad_(True), d.clone().requires_grad_(True)
    loss, dq, dd = maxsim_amd.score_contrastive_cross_entropy_value_and_grad(qg, dg, off)
    assert loss.grad_fn is None and not dq.requires_grad and qg.grad is None
    l2, dq2, dd2 = maxsim_amd.score_contrastive_cross_entropy_value_and_grad(
        q, d, off, grad_loss=torch.full((), 2.0, device=DEVICE))
    assert torch.equal(l2, loss)
    l_ref, dq_ref, dd_ref = _oracle(q, d, off, None, 1.0, "mean")
    assert_close(loss, l_ref, rtol=2e-4, atol=1e-4)
    assert_close(dq, dq_ref, rtol=1e-2, atol=2e-3)
    assert_close(dd, dd_ref, rtol=1e-2, atol=2e-3)
    assert_close(dq2, 2 * dq_ref, rtol=1e-2, atol=4e-3)
