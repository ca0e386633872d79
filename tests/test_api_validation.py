"""Input-validation contract of the Python API (CPU only).

Mirrors the reference's tests/test_invalid_inputs.py and test_ragged.py:
every bad input raises before any kernel runs, with the reference's
exception type and a message containing the same keywords.  Tensors live on
the CPU here; validation never reaches the operators."""

from __future__ import annotations

import pytest
import torch

import maxsim_amd


def _padded(B=2, C=3, Lq=16, Ld=32, dim=64, dtype=torch.float16):
    return (torch.randn(B, Lq, dim, dtype=dtype), torch.randn(B, C, Ld, dim, dtype=dtype),
            torch.full((B,), Lq, dtype=torch.int32), torch.full((B, C), Ld, dtype=torch.int32))


def _contrastive(Nq=2, Nb=4, Lq=16, Ld=32, dim=64, dtype=torch.float16):
    return (torch.randn(Nq, Lq, dim, dtype=dtype), torch.randn(Nb * Ld, dim, dtype=dtype),
            torch.arange(0, (Nb + 1) * Ld, Ld, dtype=torch.int32))


PADDED = [maxsim_amd.score_candidates_padded, maxsim_amd.score_candidates_padded_with_argmax,
          maxsim_amd.score_candidates_padded_train]
PACKED = [maxsim_amd.score_pairs_packed, maxsim_amd.score_pairs_packed_with_argmax,
          maxsim_amd.score_pairs_packed_train]
CONTRASTIVE = [maxsim_amd.score_contrastive, maxsim_amd.score_contrastive_with_argmax,
               maxsim_amd.score_contrastive_train]


# ---- padded ---------------------------------------------------------------
@pytest.mark.parametrize("fn", PADDED)
def test_padded_dim_mismatch(fn):
    q, _, ql, dl = _padded()
    with pytest.raises(ValueError, match="dim"):
        fn(q, torch.randn(2, 3, 32, 32, dtype=q.dtype), ql, dl)


@pytest.mark.parametrize("fn", PADDED)
def test_padded_dtype_mismatch(fn):
    q, d, ql, dl = _padded()
    with pytest.raises(TypeError, match="dtype"):
        fn(q, d.to(torch.bfloat16), ql, dl)


def test_padded_int_queries():
    _, d, ql, dl = _padded()
    with pytest.raises((TypeError, RuntimeError), match="float|dtype"):
        maxsim_amd.score_candidates_padded(torch.randint(0, 5, (2, 16, 64), dtype=torch.int32), d, ql, dl)


def test_padded_both_int_rejected_as_non_float():
    q = torch.randint(0, 5, (2, 16, 64), dtype=torch.int32)
    d = torch.randint(0, 5, (2, 3, 32, 64), dtype=torch.int32)
    with pytest.raises(TypeError, match="float32, float16, or bfloat16"):
        maxsim_amd.score_candidates_padded(q, d, torch.full((2,), 16), torch.full((2, 3), 32))


@pytest.mark.parametrize("fn", PADDED)
@pytest.mark.parametrize("case,msg", [("query_zero", "query_lengths"), ("query_too_long", "query_lengths"),
                                      ("doc_zero", "doc_lengths"), ("doc_too_long", "doc_lengths")])
def test_padded_lengths_out_of_bounds(fn, case, msg):
    q, d, ql, dl = _padded()
    if case == "query_zero":
        ql[0] = 0
    elif case == "query_too_long":
        ql[0] = q.shape[1] + 1
    elif case == "doc_zero":
        dl[0, 0] = 0
    else:
        dl[0, 0] = d.shape[2] + 1
    with pytest.raises(ValueError, match=msg):
        fn(q, d, ql, dl)


def test_padded_shape_errors():
    q, d, ql, dl = _padded()
    with pytest.raises(ValueError, match="3-D"):
        maxsim_amd.score_candidates_padded(q[0], d, ql, dl)
    with pytest.raises(ValueError, match="4-D"):
        maxsim_amd.score_candidates_padded(q, d[0], ql, dl)
    with pytest.raises(ValueError, match="batch"):
        maxsim_amd.score_candidates_padded(q[:1], d, ql[:1], dl)
    with pytest.raises(ValueError, match="query_lengths"):
        maxsim_amd.score_candidates_padded(q, d, ql[:1], dl)
    with pytest.raises(ValueError, match="doc_lengths"):
        maxsim_amd.score_candidates_padded(q, d, ql, dl[:, :2])
    with pytest.raises(TypeError, match="int32 or int64"):
        maxsim_amd.score_candidates_padded(q, d, ql.float(), dl)


# ---- packed ---------------------------------------------------------------
def _packed():
    return (torch.randn(10, 64, dtype=torch.float16), torch.tensor([0, 10], dtype=torch.int32),
            torch.randn(20, 64, dtype=torch.float16), torch.tensor([0, 20], dtype=torch.int32),
            torch.tensor([0], dtype=torch.int32), torch.tensor([0], dtype=torch.int32))


@pytest.mark.parametrize("fn", PACKED)
def test_packed_dim_mismatch(fn):
    q, qo, _, do, qi, di = _packed()
    with pytest.raises(ValueError, match="dim|match"):
        fn(q, qo, torch.randn(20, 32, dtype=torch.float16), do, qi, di)


@pytest.mark.parametrize("fn", PACKED)
def test_packed_offsets_not_starting_at_zero(fn):
    q, _, d, do, qi, di = _packed()
    with pytest.raises(RuntimeError, match="0|offset|start"):
        fn(q, torch.tensor([1, 10], dtype=torch.int32), d, do, qi, di)


@pytest.mark.parametrize("fn", PACKED)
def test_packed_offsets_not_ending_at_total(fn):
    q, _, d, do, qi, di = _packed()
    with pytest.raises(RuntimeError, match="total|equal|offset"):
        fn(q, torch.tensor([0, 5], dtype=torch.int32), d, do, qi, di)


@pytest.mark.parametrize("fn", PACKED)
def test_packed_negative_and_out_of_range_ids(fn):
    q, qo, d, do, _, di = _packed()
    with pytest.raises(RuntimeError, match="out of range"):
        fn(q, qo, d, do, torch.tensor([-1], dtype=torch.int32), di)
    with pytest.raises(RuntimeError, match="out of range"):
        fn(q, qo, d, do, torch.tensor([0], dtype=torch.int32), torch.tensor([5], dtype=torch.int32))


@pytest.mark.parametrize("fn", PACKED)
def test_packed_max_q_len_too_small(fn):
    q = torch.randn(13, 64, dtype=torch.float16)
    qo = torch.tensor([0, 5, 13], dtype=torch.int32)
    _, _, d, do, _, di = _packed()
    with pytest.raises(ValueError, match="max_q_len"):
        fn(q, qo, d, do, torch.tensor([1], dtype=torch.int32), di, max_q_len=5)
    with pytest.raises(ValueError, match="max_q_len"):
        fn(q, qo, d, do, torch.tensor([1], dtype=torch.int32), di, max_q_len=0)


def test_packed_empty_segment_and_dtype():
    q = torch.randn(4, 32)
    qo = torch.tensor([0, 1, 1, 4], dtype=torch.int32)
    d = torch.randn(8, 32)
    do = torch.tensor([0, 4, 8], dtype=torch.int32)
    z = torch.tensor([0], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="empty segment"):
        maxsim_amd.score_pairs_packed(q, qo, d, do, z, z)
    with pytest.raises(TypeError, match="same dtype"):
        maxsim_amd.score_pairs_packed(q, torch.tensor([0, 4]), d.half(), do, z, z)
    with pytest.raises(ValueError, match="same shape"):
        maxsim_amd.score_pairs_packed(q, torch.tensor([0, 4]), d, do, z, torch.zeros(2, dtype=torch.int32))


# ---- contrastive ----------------------------------------------------------
@pytest.mark.parametrize("fn", CONTRASTIVE)
def test_contrastive_rank_errors(fn):
    q, d, cu = _contrastive()
    with pytest.raises(ValueError, match="3-D|3D|Nq, Lq"):
        fn(q[..., None], d, cu)
    with pytest.raises(ValueError, match="2-D|2D|packed"):
        fn(q, d[..., None], cu)
    with pytest.raises(ValueError, match="dim|D|match"):
        fn(q, torch.randn(128, 32, dtype=q.dtype), cu)
    with pytest.raises(TypeError, match="dtype"):
        fn(q, d.to(torch.bfloat16), cu)


@pytest.mark.parametrize("fn", CONTRASTIVE)
@pytest.mark.parametrize("bad,pattern", [
    ([1, 33, 65, 97, 129], "0|start|offset"),
    ([0, 32, 16, 96, 128], "monoton|decreas|order|offset"),
    ([0, 25, 50, 75, 100], "total|match|offset"),
    ([0, 0, 64, 96, 128], "strictly|empty|offset"),
])
def test_contrastive_bad_offsets(fn, bad, pattern):
    q, d, _ = _contrastive()
    with pytest.raises(ValueError, match=pattern):
        fn(q, d, torch.tensor(bad, dtype=torch.int32))


@pytest.mark.parametrize("fn", CONTRASTIVE)
def test_contrastive_zero_lq_and_dim(fn):
    q, d, cu = _contrastive()
    with pytest.raises(ValueError, match="Lq"):
        fn(q[:, :0], d, cu)
    with pytest.raises(ValueError, match="dim"):
        fn(q[:, :, :0], d[:, :0], cu)
    with pytest.raises(ValueError, match="length >= 2"):
        fn(q, d, cu[:1])


def test_contrastive_offsets_dtype():
    q, d, cu = _contrastive()
    with pytest.raises(TypeError, match="int32 or int64"):
        maxsim_amd.score_contrastive(q, d, cu.float())


def test_exports_match_reference_all():
    expected = {
        "score_pairs_packed", "score_pairs_packed_with_argmax", "score_pairs_packed_train",
        "score_candidates_padded", "score_candidates_padded_with_argmax",
        "score_candidates_padded_train", "score_contrastive", "score_contrastive_with_argmax",
        "score_contrastive_train", "maxsim_reference", "maxsim_reference_with_argmax",
        "score_pairs_packed_reference", "score_pairs_packed_with_argmax_reference",
        "score_candidates_padded_reference", "score_candidates_padded_with_argmax_reference",
        "score_contrastive_reference", "score_contrastive_with_argmax_reference",
    }
    assert set(maxsim_amd.__all__) == expected
    for name in expected:
        assert callable(getattr(maxsim_amd, name))


def test_ops_namespace_has_the_nine_reference_ops():
    from maxsim_amd._ops import ops

    for name in ["maxsim_forward", "maxsim_padded_forward", "maxsim_padded_forward_with_argmax",
                 "maxsim_padded_backward", "maxsim_packed_forward_with_argmax",
                 "maxsim_packed_backward", "maxsim_contrastive_forward",
                 "maxsim_contrastive_forward_with_argmax", "maxsim_contrastive_backward"]:
        assert hasattr(ops, name)


def test_cpu_tensors_never_fall_back():
    """A valid call on CPU tensors must fail loudly: there is no CPU path."""
    q, d, cu = _contrastive()
    with pytest.raises(NotImplementedError):
        maxsim_amd.score_contrastive(q, d, cu)


def test_cross_entropy_validation():
    """score_contrastive_cross_entropy rejects bad reductions, temperatures
    and targets before anything runs (CPU tensors: the checks come first)."""
    q, d, off = _contrastive(Nq=3, Nb=4)
    with pytest.raises(ValueError, match="reduction"):
        maxsim_amd.score_contrastive_cross_entropy(q, d, off, reduction="avg")
    with pytest.raises(ValueError, match="temperature"):
        maxsim_amd.score_contrastive_cross_entropy(q, d, off, temperature=0.0)
    with pytest.raises(ValueError, match="temperature"):
        maxsim_amd.score_contrastive_cross_entropy(q, d, off, temperature=float("nan"))
    with pytest.raises(ValueError, match="targets"):
        maxsim_amd.score_contrastive_cross_entropy(q, d, off, torch.tensor([0, 1]))
    with pytest.raises(ValueError, match="out of range"):
        maxsim_amd.score_contrastive_cross_entropy(q, d, off, torch.tensor([0, 1, 4]))
    with pytest.raises(TypeError, match="int32 or int64"):
        maxsim_amd.score_contrastive_cross_entropy(q, d, off, torch.tensor([0.0, 1.0, 2.0]))
    q5, d5, off5 = _contrastive(Nq=5, Nb=4)
    with pytest.raises(ValueError, match="diagonal"):
        maxsim_amd.score_contrastive_cross_entropy(q5, d5, off5)


def test_value_and_grad_validation():
    """score_contrastive_cross_entropy_value_and_grad shares the loss's
    argument checks and checks grad_loss; CPU tensors fail loudly."""
    q, d, off = _contrastive(Nq=3, Nb=4)
    vg = maxsim_amd.score_contrastive_cross_entropy_value_and_grad
    with pytest.raises(ValueError, match="reduction"):
        vg(q, d, off, reduction="avg")
    with pytest.raises(ValueError, match="out of range"):
        vg(q, d, off, torch.tensor([0, 1, 4]))
    with pytest.raises(TypeError, match="grad_loss"):
        vg(q, d, off, grad_loss=torch.ones((), dtype=torch.float64))
    with pytest.raises(ValueError, match="grad_loss"):
        vg(q, d, off, grad_loss=torch.ones(3))
    with pytest.raises(ValueError, match="grad_loss"):
        vg(q, d, off, reduction="none", grad_loss=torch.ones(()))
    with pytest.raises(NotImplementedError):
        vg(q, d, off)
    import maxsim
    assert maxsim.score_contrastive_cross_entropy_value_and_grad is vg


def test_host_checks_switch():
    """set_host_checks / host_checks toggle the process-wide setting and
    restore it; with checks off, shape and dtype errors still raise, and
    layout data on the host is still checked (only device-resident data is
    left to the kernels)."""
    assert maxsim_amd.set_host_checks(False) is True
    try:
        q, d, _ = _contrastive()
        with pytest.raises(ValueError, match="Lq"):
            maxsim_amd.score_contrastive(q[:, :0], d, torch.tensor([0, 8], dtype=torch.int32))
        with pytest.raises(ValueError, match="0|start|offset"):
            maxsim_amd.score_contrastive(q, d, torch.tensor([1, 33, 65, 97, 129],
                                                            dtype=torch.int32))
        with pytest.raises(TypeError, match="int32 or int64"):
            maxsim_amd.score_contrastive(q, d, torch.tensor([0.0, 8.0]))
    finally:
        assert maxsim_amd.set_host_checks(True) is False
    with maxsim_amd.host_checks(False):
        assert maxsim_amd._HOST_CHECKS is False
        with maxsim_amd.host_checks(True):
            assert maxsim_amd._HOST_CHECKS is True
        assert maxsim_amd._HOST_CHECKS is False
    assert maxsim_amd._HOST_CHECKS is True
    import maxsim
    assert maxsim.set_host_checks is maxsim_amd.set_host_checks
