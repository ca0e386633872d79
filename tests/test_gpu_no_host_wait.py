"""Host checks off (maxsim_amd.set_host_checks(False)): no call waits for the
device, invalid layouts give NaN scores where they are invalid and nothing
else changes, and a whole training step can be captured in a HIP graph (a
host wait inside the capture would make it fail)."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

import maxsim_amd
from oracle import maxsim_oracle as oracle

from ._helpers import (DEVICE, SCORE_TOL, assert_close, make_contrastive, make_packed, make_padded,
                       np64, npi)

pytestmark = pytest.mark.gpu


@pytest.fixture
def no_checks():
    previous = maxsim_amd.set_host_checks(False)
    yield
    maxsim_amd.set_host_checks(previous)


def _same(a, b):
    torch.testing.assert_close(a, b, rtol=0, atol=0, equal_nan=True)


def test_contrastive_valid_inputs_identical(no_checks):
    q, d, off = make_contrastive(6, 32, 128, [40, 300, 17, 64, 9, 200, 31], torch.bfloat16,
                                 seed=5, unit=True)
    s1, a1 = maxsim_amd.score_contrastive_with_argmax(q, d, off)
    with maxsim_amd.host_checks(True):
        s2, a2 = maxsim_amd.score_contrastive_with_argmax(q, d, off)
    _same(s1, s2)
    _same(a1, a2)


def test_contrastive_invalid_document_is_nan_only_there(no_checks):
    """Document 1 is empty (offsets 8, 8): its column is NaN with argmax 0, the
    others equal the oracle, and the training backward runs: with a loss over
    the valid columns, the gradients equal the oracle's."""
    q, d, _ = make_contrastive(4, 32, 64, [20], torch.bfloat16, seed=9, unit=True)
    off = torch.tensor([0, 8, 8, 20], dtype=torch.int32, device=DEVICE)
    scores, argmax = maxsim_amd.score_contrastive_with_argmax(q, d, off)
    assert torch.isnan(scores[:, 1]).all() and torch.all(argmax[:, 1] == 0)
    valid = torch.tensor([0, 2], device=DEVICE)
    qn, dn = np64(q), np64(d)
    s_ref, a_ref = oracle.contrastive_forward(qn, dn, [0, 8, 20])
    assert_close(scores[:, valid], s_ref, **SCORE_TOL[torch.bfloat16])
    qg, dg = q.clone().requires_grad_(True), d.clone().requires_grad_(True)
    s = maxsim_amd.score_contrastive_train(qg, dg, off)
    w = torch.randn(4, 2, generator=torch.Generator().manual_seed(2)).to(DEVICE)
    (s[:, valid] * w).sum().backward()
    dq_ref, dd_ref = oracle.contrastive_backward(np64(w), qn, dn, [0, 8, 20], a_ref)
    assert_close(qg.grad.float(), dq_ref, rtol=1e-2, atol=1e-3)
    assert_close(dg.grad.float(), dd_ref, rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("bad", [[0, 10, 5, 20], [0, 10, 40, 20], [-5, 10, 15, 20]],
                         ids=["decreasing", "past-end", "negative-start"])
def test_contrastive_malformed_offsets_no_error(no_checks, bad):
    """Offsets the checked mode rejects: no error, NaN for each invalid range,
    the training step runs (NaN loss), and the device stays usable."""
    q, d, _ = make_contrastive(3, 16, 64, [20], torch.float16, seed=11)
    off = torch.tensor(bad, dtype=torch.int32, device=DEVICE)
    scores = maxsim_amd.score_contrastive(q, d, off)
    torch.cuda.synchronize()
    for b in range(3):
        s0, s1 = bad[b], bad[b + 1]
        ok = s0 >= 0 and s1 > s0 and s1 <= 20
        assert bool(torch.isnan(scores[:, b]).all()) == (not ok)
    qg, dg = q.clone().requires_grad_(True), d.clone().requires_grad_(True)
    loss = F.cross_entropy(maxsim_amd.score_contrastive_train(qg, dg, off),
                           torch.arange(3, device=DEVICE))
    loss.backward()
    torch.cuda.synchronize()
    assert torch.isnan(loss)
    good = torch.tensor([0, 5, 12, 20], dtype=torch.int32, device=DEVICE)
    s_ref, _ = oracle.contrastive_forward(np64(q), np64(d), npi(good))
    assert_close(maxsim_amd.score_contrastive(q, d, good), s_ref, **SCORE_TOL[torch.float16])


def test_cross_entropy_target_out_of_range_is_nan_row(no_checks):
    q, d, off = make_contrastive(4, 16, 64, [20, 30, 12, 9, 40], torch.bfloat16, seed=3,
                                 unit=True)
    targets = torch.tensor([0, 7, 2, 4], device=DEVICE)  # 7 is out of range
    loss = maxsim_amd.score_contrastive_cross_entropy(q, d, off, targets, reduction="none")
    torch.cuda.synchronize()
    assert torch.isnan(loss[1]) and torch.isfinite(loss[[0, 2, 3]]).all()
    with maxsim_amd.host_checks(True):
        ok = torch.tensor([0, 1, 2, 4], device=DEVICE)
        ref = maxsim_amd.score_contrastive_cross_entropy(q, d, off, ok, reduction="none")
    _same(loss[[0, 2, 3]], ref[[0, 2, 3]])


def test_cross_entropy_int64_target_beyond_int32_is_nan_row(no_checks):
    """An int64 target that would wrap to a valid class when narrowed to
    int32 (2**32 + 1 -> 1) still gives the NaN loss of an invalid target."""
    q, d, off = make_contrastive(4, 16, 64, [20, 30, 12, 9, 40], torch.bfloat16, seed=3,
                                 unit=True)
    targets = torch.tensor([0, 2**32 + 1, 2, -(2**32) + 3], dtype=torch.int64, device=DEVICE)
    loss = maxsim_amd.score_contrastive_cross_entropy(q, d, off, targets, reduction="none")
    torch.cuda.synchronize()
    assert torch.isnan(loss[1]) and torch.isnan(loss[3])
    assert torch.isfinite(loss[[0, 2]]).all()
    vloss, _, _ = maxsim_amd.score_contrastive_cross_entropy_value_and_grad(
        q, d, off, targets, reduction="none")
    torch.cuda.synchronize()
    assert torch.isnan(vloss[1]) and torch.isnan(vloss[3])
    _same(vloss[[0, 2]], loss[[0, 2]])


def test_cross_entropy_device_targets_checked_after_launch():
    """With host checks on, device targets are copied with the offsets and
    checked while the kernels run; an out-of-range one still raises."""
    q, d, off = make_contrastive(4, 16, 64, [20, 30, 12, 9, 40], torch.bfloat16, seed=3,
                                 unit=True)
    for bad in (torch.tensor([0, 7, 2, 4], device=DEVICE),
                torch.tensor([0, 1, -1, 4], dtype=torch.int32, device=DEVICE),
                torch.tensor([0, 2**32 + 1, 2, 4], device=DEVICE)):
        with pytest.raises(ValueError, match="out of range"):
            maxsim_amd.score_contrastive_cross_entropy(q, d, off, bad)
        with pytest.raises(ValueError, match="out of range"):
            maxsim_amd.score_contrastive_cross_entropy_value_and_grad(q, d, off, bad)
    ok = torch.tensor([0, 1, 2, 4], device=DEVICE)
    loss = maxsim_amd.score_contrastive_cross_entropy(q, d, off, ok, reduction="none")
    assert torch.isfinite(loss).all()


def test_padded_invalid_lengths_nan_only_there(no_checks):
    q, d, ql, dl = make_padded(3, 5, 16, 40, 64, torch.bfloat16, seed=4)
    with maxsim_amd.host_checks(True):
        ref = maxsim_amd.score_candidates_padded(q, d, ql, dl)
    dl_bad = dl.clone()
    dl_bad[1, 2] = 41      # beyond Ld
    dl_bad[2, 0] = 0       # empty
    s = maxsim_amd.score_candidates_padded(q, d, ql, dl_bad)
    torch.cuda.synchronize()
    bad = torch.zeros(3, 5, dtype=torch.bool, device=DEVICE)
    bad[1, 2] = bad[2, 0] = True
    assert torch.isnan(s[bad]).all()
    _same(s[~bad], ref[~bad])
    ql_bad = ql.clone()
    ql_bad[0] = 17         # beyond Lq: the whole query is invalid
    s = maxsim_amd.score_candidates_padded(q, d, ql_bad, dl)
    torch.cuda.synchronize()
    assert torch.isnan(s[0]).all()
    _same(s[1:], ref[1:])


def test_packed_invalid_pairs_nan_only_there(no_checks):
    q, qoff, d, doff, qids, dids = make_packed(6, 9, 40, 64, (4, 24), (10, 80), torch.bfloat16,
                                               seed=8)
    with maxsim_amd.host_checks(True):
        ref = maxsim_amd.score_pairs_packed(q, qoff, d, doff, qids, dids)
        ref_am, _ = maxsim_amd.score_pairs_packed_with_argmax(q, qoff, d, doff, qids, dids)
        mql = int((qoff[1:] - qoff[:-1]).max())
    qb, db = qids.clone(), dids.clone()
    qb[3] = 6              # query id out of range
    db[7] = -1             # document id out of range
    s = maxsim_amd.score_pairs_packed(q, qoff, d, doff, qb, db)
    torch.cuda.synchronize()
    bad = torch.zeros(40, dtype=torch.bool, device=DEVICE)
    bad[3] = bad[7] = True
    assert torch.isnan(s[bad]).all()
    _same(s[~bad], ref[~bad])
    # a max_q_len below the longest query: the pairs of longer queries are NaN
    lens = (qoff[1:] - qoff[:-1])[qids.long()]
    s, _ = maxsim_amd.score_pairs_packed_with_argmax(q, qoff, d, doff, qids, dids,
                                                     max_q_len=mql - 1)
    torch.cuda.synchronize()
    long = lens > mql - 1
    assert long.any()
    assert torch.isnan(s[long]).all()
    _same(s[~long], ref_am[~long])


def _c2_inputs():
    import bench

    return bench.make_c5(torch, DEVICE, seed=1, nq=64, nb=64, lo=64, hi=512, dup=0.0)


@pytest.mark.parametrize("fused", [False, True], ids=["F.cross_entropy", "fused"])
def test_c2_training_step_captured_in_a_graph(no_checks, fused):
    """A C2 training step (forward, loss, backward) captured in a HIP graph:
    a host wait anywhere in it would fail the capture.  Each replay, with
    eager work and synchronisations between replays, gives the eager step's
    loss and gradients bit for bit (the contrastive dQ is reproducible; dD
    sums in bucket order, so its last bits may differ)."""
    q, d, off, _ = _c2_inputs()
    target = torch.arange(64, device=DEVICE)
    qg, dg = q.clone().requires_grad_(True), d.clone().requires_grad_(True)

    def step():
        if fused:
            loss = maxsim_amd.score_contrastive_cross_entropy(qg, dg, off)
        else:
            loss = F.cross_entropy(maxsim_amd.score_contrastive_train(qg, dg, off), target)
        loss.backward()
        return loss

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            qg.grad = dg.grad = None
            step()
    torch.cuda.current_stream().wait_stream(side)
    qg.grad = dg.grad = None
    eager_loss = step().detach().clone()
    eager_dq, eager_dd = qg.grad.clone(), dg.grad.clone()

    graph = torch.cuda.CUDAGraph()
    qg.grad = dg.grad = None
    with torch.cuda.graph(graph):
        static_loss = step()
    static_dq, static_dd = qg.grad, dg.grad
    for r in range(4):
        static_dq.fill_(float("nan"))
        static_dd.fill_(float("nan"))
        static_loss.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        _same(static_loss, eager_loss)
        _same(static_dq, eager_dq)
        torch.testing.assert_close(static_dd.float(), eager_dd.float(), rtol=1e-2, atol=1e-6)
        # eager work between replays
        maxsim_amd.score_contrastive(q, d, off).sum().item()


def test_c2_value_and_grad_captured_in_a_graph(no_checks):
    """score_contrastive_cross_entropy_value_and_grad (no autograd) captured
    in a HIP graph at C2: each replay, with eager work and synchronisations
    between replays, gives the eager call's loss and dQ bit for bit and dD
    up to its bucket-sum order."""
    q, d, off, _ = _c2_inputs()
    vg = maxsim_amd.score_contrastive_cross_entropy_value_and_grad
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            vg(q, d, off)
    torch.cuda.current_stream().wait_stream(side)
    eager = [t.clone() for t in vg(q, d, off)]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static = vg(q, d, off)
    for r in range(4):
        for t in static:
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        _same(static[0], eager[0])
        _same(static[1], eager[1])
        torch.testing.assert_close(static[2].float(), eager[2].float(), rtol=1e-2, atol=1e-6)
        # eager work between replays
        maxsim_amd.score_contrastive(q, d, off).sum().item()
