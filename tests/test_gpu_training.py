"""Training loops and random shapes on the GPU (reference tests:
test_stability.py, test_train_convergence.py, test_fuzz.py).

* many fwd+bwd iterations of each training surface: loss and gradients stay
  finite and allocated memory stays flat;
* in-batch InfoNCE training with the contrastive kernel: the loss falls, and
  the loss curve tracks a float32 autograd run of the pure-PyTorch
  reference functions (``maxsim_amd.reference``) from the same start;
* seeded random shapes of all three surfaces against the CPU oracle."""

from __future__ import annotations

import math
import random

import pytest
import torch
import torch.nn.functional as F

import maxsim_amd
from maxsim_amd.reference import score_contrastive_reference
from oracle import maxsim_oracle as oracle

from ._helpers import DEVICE, SCORE_TOL, assert_close, np64, npi, offsets_from_lengths

pytestmark = pytest.mark.gpu


# ---------------------------------------------------------------------------
# stability
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("api", ["padded", "contrastive", "packed"])
def test_no_leak_or_nan_over_many_iterations(api):
    """200 fwd+bwd+SGD iterations: finite loss and gradients at every tenth
    step, and allocated memory within 20 MB of where it started."""
    g = torch.Generator().manual_seed(0)
    dt = torch.float16
    if api == "padded":
        B, C, Lq, Ld, D = 2, 4, 16, 32, 64
        q0 = torch.randn(B, Lq, D, generator=g).to(dt).to(DEVICE)
        d0 = torch.randn(B, C, Ld, D, generator=g).to(dt).to(DEVICE)
        qlen = torch.full((B,), Lq, dtype=torch.int32, device=DEVICE)
        dlen = torch.full((B, C), Ld, dtype=torch.int32, device=DEVICE)

        def step(q, d):
            return maxsim_amd.score_candidates_padded_train(q, d, qlen, dlen).mean()
    elif api == "contrastive":
        Nq, Nb, Lq, Ld, D = 4, 4, 16, 32, 64
        q0 = torch.randn(Nq, Lq, D, generator=g).to(dt).to(DEVICE)
        d0 = torch.randn(Nb * Ld, D, generator=g).to(dt).to(DEVICE)
        cu = torch.arange(0, (Nb + 1) * Ld, Ld, dtype=torch.int32, device=DEVICE)

        def step(q, d):
            return maxsim_amd.score_contrastive_train(q, d, cu).mean()
    else:
        Nq, Nb, Lq, Ld, D = 3, 4, 12, 24, 64
        q0 = torch.randn(Nq * Lq, D, generator=g).to(dt).to(DEVICE)
        d0 = torch.randn(Nb * Ld, D, generator=g).to(dt).to(DEVICE)
        qoff = torch.arange(0, (Nq + 1) * Lq, Lq, dtype=torch.int32, device=DEVICE)
        doff = torch.arange(0, (Nb + 1) * Ld, Ld, dtype=torch.int32, device=DEVICE)
        qids = torch.tensor([0, 1, 2, 0, 1, 2], dtype=torch.int32, device=DEVICE)
        dids = torch.tensor([0, 1, 2, 3, 0, 1], dtype=torch.int32, device=DEVICE)

        def step(q, d):
            return maxsim_amd.score_pairs_packed_train(q, qoff, d, doff, qids, dids,
                                                       max_q_len=Lq).mean()

    def iterate():
        q = q0.detach().clone().requires_grad_(True)
        d = d0.detach().clone().requires_grad_(True)
        loss = step(q, d)
        loss.backward()
        with torch.no_grad():
            q.sub_(0.01 * q.grad)
            d.sub_(0.01 * d.grad)
        return loss, q, d

    for _ in range(5):
        iterate()
    torch.cuda.synchronize()
    mem_start = torch.cuda.memory_allocated() / 2**20
    for i in range(200):
        loss, q, d = iterate()
        if i % 20 == 0:
            assert math.isfinite(float(loss.detach())), f"non-finite loss at step {i}"
            assert bool(torch.isfinite(q.grad).all()) and bool(torch.isfinite(d.grad).all())
    torch.cuda.synchronize()
    grown = torch.cuda.memory_allocated() / 2**20 - mem_start
    assert grown < 20.0, f"{api}: allocated memory grew by {grown:.1f} MB over 200 steps"


# ---------------------------------------------------------------------------
# convergence
# ---------------------------------------------------------------------------
def _initial(Nq, Nb, Lq, Ld, dim, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(Nq, Lq, dim, generator=g).to(dtype).to(DEVICE)
    d = torch.randn(Nb * Ld, dim, generator=g).to(dtype).to(DEVICE)
    cu = torch.arange(0, (Nb + 1) * Ld, Ld, dtype=torch.int32, device=DEVICE)
    return q, d, cu


def _info_nce(scores):
    targets = torch.arange(scores.shape[0], device=scores.device)
    return F.cross_entropy(scores / scores.shape[1] ** 0.5, targets)


def _train(q0, d0, cu, score_fn, steps, lr, cast=None):
    q = (q0 if cast is None else q0.to(cast)).detach().clone().requires_grad_(True)
    d = (d0 if cast is None else d0.to(cast)).detach().clone().requires_grad_(True)
    losses = []
    for _ in range(steps):
        loss = _info_nce(score_fn(q, d, cu))
        loss.backward()
        with torch.no_grad():
            q.sub_(lr * q.grad)
            d.sub_(lr * d.grad)
            q.grad = None
            d.grad = None
        losses.append(float(loss.detach()))
    return losses


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_contrastive_loss_decreases(dtype):
    """50 SGD steps of in-batch InfoNCE through the kernels: the final loss
    is well below the first and every loss is finite."""
    q0, d0, cu = _initial(8, 8, 16, 32, 64, dtype, seed=0)
    losses = _train(q0, d0, cu, maxsim_amd.score_contrastive_train, steps=50, lr=0.05)
    assert all(math.isfinite(x) for x in losses), losses
    assert losses[0] > 1.3 * losses[-1], losses


def test_kernel_training_tracks_fp32_autograd_reference():
    """30 steps from the same fp16 start: the kernel run (fp16 weights) and a
    float32 autograd run of the pure-PyTorch reference stay within the
    reference test's bars at every step, and both train."""
    q0, d0, cu = _initial(6, 6, 16, 32, 64, torch.float16, seed=1)
    loss_k = _train(q0, d0, cu, maxsim_amd.score_contrastive_train, steps=30, lr=0.05)
    loss_r = _train(q0, d0, cu, score_contrastive_reference, steps=30, lr=0.05,
                    cast=torch.float32)
    for i, (lk, lr_) in enumerate(zip(loss_k, loss_r)):
        gap = abs(lk - lr_)
        assert gap < 0.05 or gap / max(abs(lr_), 1e-6) < 0.3, (i, lk, lr_)
    assert loss_k[-1] < 0.5 * loss_k[0] and loss_r[-1] < 0.5 * loss_r[0]


# ---------------------------------------------------------------------------
# random shapes
# ---------------------------------------------------------------------------
N_FUZZ = 30
DIMS = [16, 24, 32, 64, 96, 128]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_padded_random_shapes(dtype):
    rng = random.Random(123)
    for i in range(N_FUZZ):
        B, C, Lq, Ld, dim = (rng.randint(1, 4), rng.randint(1, 8), rng.randint(1, 64),
                             rng.randint(1, 200), rng.choice(DIMS))
        g = torch.Generator().manual_seed(i * 7919 + 1)
        q = torch.randn(B, Lq, dim, generator=g).to(dtype).to(DEVICE)
        d = torch.randn(B, C, Ld, dim, generator=g).to(dtype).to(DEVICE)
        qlen = torch.randint(1, Lq + 1, (B,), generator=g, dtype=torch.int32).to(DEVICE)
        dlen = torch.randint(1, Ld + 1, (B, C), generator=g, dtype=torch.int32).to(DEVICE)
        s = maxsim_amd.score_candidates_padded(q, d, qlen, dlen)
        s_ref, _ = oracle.padded_forward(np64(q), np64(d), npi(qlen), npi(dlen))
        assert_close(s, s_ref, **SCORE_TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_packed_random_shapes(dtype):
    rng = random.Random(7777)
    for i in range(N_FUZZ):
        nq, nd, npairs, dim = (rng.randint(1, 6), rng.randint(1, 8), rng.randint(1, 16),
                               rng.choice(DIMS))
        ql = [rng.randint(1, 70) for _ in range(nq)]
        dl = [rng.randint(1, 128) for _ in range(nd)]
        g = torch.Generator().manual_seed(i * 4283 + 1)
        q = torch.randn(sum(ql), dim, generator=g).to(dtype).to(DEVICE)
        d = torch.randn(sum(dl), dim, generator=g).to(dtype).to(DEVICE)
        qoff = offsets_from_lengths(torch.tensor(ql)).to(DEVICE)
        doff = offsets_from_lengths(torch.tensor(dl)).to(DEVICE)
        qids = torch.tensor([rng.randint(0, nq - 1) for _ in range(npairs)],
                            dtype=torch.int32, device=DEVICE)
        dids = torch.tensor([rng.randint(0, nd - 1) for _ in range(npairs)],
                            dtype=torch.int32, device=DEVICE)
        mql = max(ql) if i % 2 else None  # both the given and the derived length bound
        s = maxsim_amd.score_pairs_packed(q, qoff, d, doff, qids, dids, max_q_len=mql)
        s_ref, _ = oracle.packed_forward(np64(q), npi(qoff), np64(d), npi(doff), npi(qids),
                                         npi(dids), max(ql))
        assert_close(s, s_ref, **SCORE_TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_contrastive_random_shapes(dtype):
    rng = random.Random(4242)
    for i in range(N_FUZZ):
        nq, nb, lq, dim = rng.randint(1, 6), rng.randint(1, 10), rng.randint(1, 48), rng.choice(DIMS)
        lens = [rng.randint(1, 150) for _ in range(nb)]
        g = torch.Generator().manual_seed(i * 131 + 5)
        q = torch.randn(nq, lq, dim, generator=g).to(dtype).to(DEVICE)
        d = torch.randn(sum(lens), dim, generator=g).to(dtype).to(DEVICE)
        off = offsets_from_lengths(torch.tensor(lens)).to(DEVICE)
        s = maxsim_amd.score_contrastive(q, d, off)
        s_ref, _ = oracle.contrastive_forward(np64(q), np64(d), npi(off))
        assert_close(s, s_ref, **SCORE_TOL[dtype])
