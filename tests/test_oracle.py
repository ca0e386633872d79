"""Pins the CPU oracle (CPU only).

Each oracle function is checked against something that is not a retyping of
its own formula:
  * known answers from the reference's tests (single pair/token, all-identical
    rows -> argmax 0, pad garbage ignored, zero dscore, empty pair list);
  * closed forms: for distinct unit rows, score(q, q) = Lq with argmax = i;
  * torch's own einsum + ``max(dim)`` (first index on ties) and its autograd
    on finite inputs -- a library routine, not our code;
  * the NaN / inf contract of the reference kernels (test_nan_inf.py);
  * identities between the three surfaces;
  * the golden fixture for config C1 (tests/golden/c1_expected.npz);
  * planted mistakes (last-index ties, NaN-propagating max, a dropped query
    token, an off-by-one document offset) that these checks must catch.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import maxsim_oracle as oracle

from .golden.c1_inputs import digest, make_c1


def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


def _unit(shape, seed):
    x = _rand(shape, seed)
    return x / np.linalg.norm(x, axis=-1, keepdims=True)


# ---------------------------------------------------------------------------
# Individual pins, written as functions so the planted-mistake test can run
# them against a deliberately broken oracle.
# ---------------------------------------------------------------------------
def pin_single_token():
    q, d = _rand((1, 16), 0), _rand((1, 16), 1)
    s, a = oracle.pair_forward(q, d)
    assert abs(s - float(q[0] @ d[0])) <= 1e-6 * max(1, abs(s)) and a.tolist() == [0]


def pin_identical_rows_argmax_zero():
    base = _rand((32,), 2)
    d = np.tile(base, (47, 1))
    q = _rand((3, 12, 32), 3)
    off = np.array([0, 20, 47])
    _, a = oracle.contrastive_forward(q, d, off)
    assert np.all(a == 0)
    _, ap = oracle.padded_forward(q, np.tile(base, (3, 2, 20, 1)), [12, 5, 1], [[20, 3], [1, 20]] + [[7, 7]])
    assert np.all(ap == 0)


def pin_self_similarity():
    q = _unit((4, 24, 64), 4)
    for k in range(4):
        s, a = oracle.pair_forward(q[k], q[k])
        assert abs(s - 24.0) < 1e-5
        assert np.array_equal(a, np.arange(24))


def pin_torch_einsum_max():
    q = _rand((3, 16, 32), 5)
    lens = [37, 64, 5, 81]
    d = _rand((sum(lens), 32), 6)
    off = np.concatenate([[0], np.cumsum(lens)])
    s, a = oracle.contrastive_forward(q, d, off)
    qt = torch.from_numpy(q)
    for b in range(len(lens)):
        sim = torch.einsum("qid,jd->qij", qt, torch.from_numpy(d[off[b]:off[b + 1]]))
        best, idx = sim.max(dim=-1)
        np.testing.assert_allclose(s[:, b], best.sum(-1).numpy(), rtol=1e-6)
        assert np.array_equal(a[:, b], idx.numpy())


def pin_torch_autograd():
    q = _rand((2, 8, 16), 7)
    lens = [9, 20, 4]
    d = _rand((sum(lens), 16), 8)
    off = np.concatenate([[0], np.cumsum(lens)])
    g = _rand((2, 3), 9)
    _, a = oracle.contrastive_forward(q, d, off)
    dq, dd = oracle.contrastive_backward(g, q, d, off, a)
    qt = torch.from_numpy(q).requires_grad_(True)
    dt = torch.from_numpy(d).requires_grad_(True)
    scores = torch.stack([
        torch.einsum("qid,jd->qij", qt, dt[off[b]:off[b + 1]]).max(dim=-1).values.sum(-1)
        for b in range(len(lens))], dim=1)
    (scores * torch.from_numpy(g)).sum().backward()
    np.testing.assert_allclose(dq, qt.grad.numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(dd, dt.grad.numpy(), rtol=1e-5, atol=1e-6)


def pin_nan_contract():
    q = _rand((2, 16, 64), 10)
    d = _rand((96, 64), 11)
    off = np.array([0, 32, 64, 96])
    q[1, 0, 0] = np.nan
    s, a = oracle.contrastive_forward(q, d, off)
    assert np.all(np.isneginf(s[1])) and np.all(np.isfinite(s[0]))
    assert np.all(a[1, :, 0] == 0)
    # a NaN document row never wins; the others still do
    d2 = d.copy()
    d2[0] = np.nan
    _, a2 = oracle.contrastive_forward(q[:1], d2, off)
    assert np.all(a2[0, 0] != 0)


def pin_inf_contract():
    q = _rand((1, 16, 64), 12)
    d = np.abs(_rand((64, 64), 13)) + 0.1
    q[0, 0] = np.inf
    s, _ = oracle.contrastive_forward(q, d, np.array([0, 32, 64]))
    assert np.all(np.isposinf(s))


def pin_surfaces_agree():
    rng = np.random.default_rng(14)
    Nq, Lq, D = 3, 10, 24
    lens = [5, 17, 9, 30]
    q = rng.standard_normal((Nq, Lq, D))
    d = rng.standard_normal((sum(lens), D))
    off = np.concatenate([[0], np.cumsum(lens)])
    s_c, a_c = oracle.contrastive_forward(q, d, off)
    qids = np.repeat(np.arange(Nq), len(lens))
    dids = np.tile(np.arange(len(lens)), Nq)
    s_p, a_p = oracle.packed_forward(q.reshape(-1, D), np.arange(0, (Nq + 1) * Lq, Lq), d, off,
                                     qids, dids, Lq)
    np.testing.assert_allclose(s_p.reshape(Nq, -1), s_c, rtol=1e-6)
    assert np.array_equal(a_p.reshape(Nq, len(lens), Lq), a_c)
    # padded: every query gets all documents as its candidates
    dp = np.zeros((Nq, len(lens), max(lens), D))
    for b, n in enumerate(lens):
        dp[:, b, :n] = d[off[b]:off[b + 1]]
    s_d, a_d = oracle.padded_forward(q, dp, np.full(Nq, Lq), np.tile(lens, (Nq, 1)))
    np.testing.assert_allclose(s_d, s_c, rtol=1e-6)
    assert np.array_equal(a_d, a_c)


def pin_pad_garbage_ignored():
    q = _rand((2, 8, 32), 15)
    d = _rand((2, 3, 16, 32), 16)
    ql, dl = np.array([4, 6]), np.array([[10, 8, 4], [16, 1, 12]])
    s0, a0 = oracle.padded_forward(q, d, ql, dl)
    q2, d2 = q.copy(), d.copy()
    q2[0, 4:] = 1e4
    q2[1, 6:] = np.nan
    d2[0, 0, 10:] = 1e4
    d2[1, 1, 1:] = -1e4
    s1, a1 = oracle.padded_forward(q2, d2, ql, dl)
    assert np.array_equal(s0, s1) and np.array_equal(a0, a1)
    assert np.all(a1[0, :, 4:] == 0)


def pin_backward_zero_and_padded_packed():
    rng = np.random.default_rng(17)
    B, C, Lq, Ld, D = 2, 3, 6, 9, 8
    q = rng.standard_normal((B, Lq, D))
    d = rng.standard_normal((B, C, Ld, D))
    ql, dl = np.array([6, 3]), np.array([[9, 2, 5], [1, 9, 7]])
    _, a = oracle.padded_forward(q, d, ql, dl)
    dq, dd = oracle.padded_backward(np.zeros((B, C)), q, d, ql, dl, a)
    assert not dq.any() and not dd.any()
    g = rng.standard_normal((B, C))
    dq, dd = oracle.padded_backward(g, q, d, ql, dl, a)
    qt = torch.from_numpy(q).requires_grad_(True)
    dt = torch.from_numpy(d).requires_grad_(True)
    tot = 0
    for b in range(B):
        for c in range(C):
            sim = qt[b, :ql[b]] @ dt[b, c, :dl[b, c]].T
            tot = tot + g[b, c] * sim.max(dim=-1).values.sum()
    tot.backward()
    np.testing.assert_allclose(dq, qt.grad.numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(dd, dt.grad.numpy(), rtol=1e-5, atol=1e-6)
    # packed backward = padded backward on the same pairs
    qp = np.concatenate([q[b, :ql[b]] for b in range(B)])
    qo = np.concatenate([[0], np.cumsum(ql)])
    dpk = np.concatenate([d[b, c, :dl[b, c]] for b in range(B) for c in range(C)])
    do = np.concatenate([[0], np.cumsum(dl.reshape(-1))])
    qids, dids = np.repeat(np.arange(B), C), np.arange(B * C)
    _, ap = oracle.packed_forward(qp, qo, dpk, do, qids, dids, Lq)
    dqp, ddp = oracle.packed_backward(g.reshape(-1), qp, qo, dpk, do, qids, dids, ap)
    np.testing.assert_allclose(dqp, np.concatenate([dq[b, :ql[b]] for b in range(B)]), rtol=1e-6)
    np.testing.assert_allclose(ddp, np.concatenate([dd[b, c, :dl[b, c]] for b in range(B) for c in range(C)]),
                               rtol=1e-6)


def pin_empty_pairs():
    s, a = oracle.packed_forward(_rand((4, 8), 18), [0, 4], _rand((6, 8), 19), [0, 6],
                                 np.zeros(0, int), np.zeros(0, int), 4)
    assert s.shape == (0,) and s.dtype == np.float32 and a.shape == (0, 4)


def pin_golden_c1():
    q, d, qlen, dlen = make_c1(0)
    gold = np.load(__import__("pathlib").Path(__file__).parent / "golden" / "c1_expected.npz")
    assert str(gold["input_sha256"]) == digest(q, d, qlen, dlen), "C1 input generator drifted"
    s, a = oracle.padded_forward(q.numpy(), d.numpy(), qlen.numpy(), dlen.numpy())
    np.testing.assert_allclose(s, gold["scores"], rtol=1e-6)
    assert np.array_equal(a, gold["argmax"])


def pin_pack_padded():
    """Packing against a row-by-row construction, and scoring the packed pairs
    against scoring the padded candidates."""
    rng = np.random.default_rng(23)
    B, C, Lq, Ld, D = 3, 4, 7, 11, 5
    q = rng.standard_normal((B, Lq, D))
    d = rng.standard_normal((B, C, Ld, D))
    ql = np.array([7, 1, 4])
    dl = rng.integers(1, Ld + 1, (B, C))
    qp, qo, dp, do, qi, di, mql = oracle.pack_padded(q, d, ql, dl)
    assert np.array_equal(qp, np.array([q[b, i] for b in range(B) for i in range(ql[b])]))
    assert np.array_equal(dp, np.array([d[b, c, j] for b in range(B) for c in range(C)
                                        for j in range(dl[b, c])]))
    assert qo.tolist() == [0, 7, 8, 12]
    lens = [int(dl[b, c]) for b in range(B) for c in range(C)]
    assert do.tolist() == [sum(lens[:k]) for k in range(B * C + 1)]
    assert qi.tolist() == [b for b in range(B) for _ in range(C)]
    assert di.tolist() == list(range(B * C)) and mql == 7
    sp, ap = oracle.packed_forward(qp, qo, dp, do, qi, di, mql)
    s, a = oracle.padded_forward(q, d, ql, dl)
    assert np.array_equal(sp.reshape(B, C), s)
    assert np.array_equal(ap.reshape(B, C, mql), a)


PINS = [pin_single_token, pin_identical_rows_argmax_zero, pin_self_similarity,
        pin_torch_einsum_max, pin_torch_autograd, pin_nan_contract, pin_inf_contract,
        pin_surfaces_agree, pin_pad_garbage_ignored, pin_backward_zero_and_padded_packed,
        pin_empty_pairs, pin_golden_c1, pin_pack_padded]


@pytest.mark.parametrize("pin", PINS, ids=lambda f: f.__name__)
def test_oracle_pin(pin):
    pin()


# ---------------------------------------------------------------------------
# Planted mistakes: each broken oracle must fail at least one pin.
# ---------------------------------------------------------------------------
def _last_index(sim):
    clean = np.where(np.isnan(sim), -np.inf, sim)
    rev = clean[:, ::-1]
    idx = clean.shape[1] - 1 - np.argmax(rev, axis=1)
    return clean[np.arange(clean.shape[0]), idx], idx


def _nan_propagates(sim):
    idx = np.argmax(np.where(np.isnan(sim), np.inf, sim), axis=1)
    return sim[np.arange(sim.shape[0]), idx], idx


def _drops_last_token(sim):
    clean = np.where(np.isnan(sim), -np.inf, sim)
    idx = np.argmax(clean, axis=1)
    best = clean[np.arange(clean.shape[0]), idx].copy()
    best[-1] = 0.0
    return best, idx


def _off_by_one_doc(sim):
    clean = np.where(np.isnan(sim), -np.inf, sim)[:, :-1] if sim.shape[1] > 1 else sim
    idx = np.argmax(clean, axis=1)
    return clean[np.arange(clean.shape[0]), idx], idx


@pytest.mark.parametrize("mutant", [_last_index, _nan_propagates, _drops_last_token, _off_by_one_doc],
                         ids=lambda f: f.__name__)
def test_planted_mistake_is_caught(monkeypatch, mutant):
    monkeypatch.setattr(oracle, "_row_max_first", mutant)
    failures = 0
    for pin in PINS:
        try:
            with np.errstate(all="ignore"):
                pin()
        except (AssertionError, ValueError, IndexError):
            failures += 1
    assert failures > 0, f"no pin caught {mutant.__name__}"


def test_backward_mutant_is_caught(monkeypatch):
    """A backward that routes to the wrong row (j + 1) must fail the autograd pin."""
    real = oracle.contrastive_backward

    def shifted(dscore, queries, documents, offsets, argmax):
        return real(dscore, queries, documents, offsets, np.asarray(argmax) + 1)

    monkeypatch.setattr(oracle, "contrastive_backward", shifted)
    with pytest.raises(AssertionError):
        pin_torch_autograd()


@pytest.mark.parametrize("mutant", ["candidate_major_pairs", "offsets_shifted", "one_row_short"])
def test_pack_padded_mutant_is_caught(monkeypatch, mutant):
    """A packing that orders the pairs candidate-major, shifts the offsets by
    one segment, or drops a segment's last row must fail the packing pin."""
    real = oracle.pack_padded

    def broken(q, d, ql, dl):
        qp, qo, dp, do, qi, di, mql = real(q, d, ql, dl)
        B, C = np.asarray(dl).shape
        if mutant == "candidate_major_pairs":
            k = np.arange(B * C)
            qi, di = k % B, (k % B) * C + k // B
        elif mutant == "offsets_shifted":
            do = np.concatenate([[0], do[:-1]])
        else:
            return real(q, d, np.maximum(np.asarray(ql) - 1, 1), dl)
        return qp, qo, dp, do, qi, di, mql

    monkeypatch.setattr(oracle, "pack_padded", broken)
    with pytest.raises(AssertionError):
        pin_pack_padded()


@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
@pytest.mark.parametrize("with_targets", [False, True])
def test_cross_entropy_matches_torch(reduction, with_targets):
    """oracle.cross_entropy is F.cross_entropy(scores / T, targets) and its
    autograd gradient (the library routine the reference's README calls)."""
    gen = torch.Generator().manual_seed(11)
    s = torch.randn(6, 9, generator=gen, dtype=torch.float64) * 5
    t = torch.randint(0, 9, (6,), generator=gen) if with_targets else None
    inv_t = 1 / 0.3
    sr = s.clone().requires_grad_(True)
    ref = torch.nn.functional.cross_entropy(sr * inv_t, t if t is not None else torch.arange(6),
                                            reduction=reduction)
    ref.backward(torch.ones_like(ref))
    loss, dscore = oracle.cross_entropy(s.numpy(), None if t is None else t.numpy(), inv_t,
                                        reduction)
    np.testing.assert_allclose(loss, ref.detach().numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(dscore, sr.grad.numpy(), rtol=1e-12, atol=1e-12)


def test_cross_entropy_catches_planted_mistakes():
    """A softmax without the max shift overflows, a dropped temperature or a
    wrong target both change the gradient: the torch pin above would fail."""
    s = np.array([[1000.0, 999.0, 0.0], [0.0, 1.0, 2.0]])
    loss, dscore = oracle.cross_entropy(s, None, 1.0, "mean")
    assert np.isfinite(loss) and np.all(np.isfinite(dscore))
    # rows of the gradient sum to zero (softmax sums to one)
    np.testing.assert_allclose(dscore.sum(axis=1), 0.0, atol=1e-12)
    _, d2 = oracle.cross_entropy(s, None, 0.5, "mean")
    assert not np.allclose(dscore, d2)
    _, d3 = oracle.cross_entropy(s, np.array([1, 1]), 1.0, "mean")
    assert not np.allclose(dscore, d3)
