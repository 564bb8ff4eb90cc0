"""Pins of the logit comparison diagnostics (mslim_attn.conformance,
restating src/conformance.rs:75-155 and the BF16 neighbour test of
src/bin/mslim-adapter-parity.rs:38-57) against closed forms."""
import math

import numpy as np
import pytest

from mslim_attn.conformance import (ConformanceError, compare_logit_distributions, ordered_bf16, top_two,
                                    within_one_bf16_ulp)


def test_identical_rows_are_exact_with_zero_divergence():
    x = np.random.default_rng(1).standard_normal(1000).astype(np.float32)
    r = compare_logit_distributions(x, x.copy())
    assert r["exact"] and r["top1_equal"]
    assert r["max_abs_difference"] == r["mean_abs_difference"] == r["p95_abs_difference"] == 0.0
    assert r["kl_reference_to_candidate"] == 0.0
    assert r["reference_top1_top2_margin"] == r["candidate_top1_top2_margin"]


def test_constant_shift_changes_values_not_the_distribution():
    # softmax is shift-invariant: KL 0 while every logit moves by 0.5
    x = np.float32([0.25, -1.0, 3.0, 2.5])
    r = compare_logit_distributions(x, x + np.float32(0.5))
    assert not r["exact"]
    assert r["max_abs_difference"] == r["mean_abs_difference"] == r["p95_abs_difference"] == 0.5
    assert r["kl_reference_to_candidate"] == pytest.approx(0.0, abs=1e-15)
    assert r["reference_top1"] == r["candidate_top1"] == 2
    assert r["reference_top1_top2_margin"] == 0.5


def test_two_token_kl_closed_form():
    # p = (1/2, 1/2), q = (3/4, 1/4): KL(p || q) = 1/2 ln(4/3)
    r = compare_logit_distributions(np.float32([0.0, 0.0]), np.float32([math.log(3.0), 0.0]))
    assert r["kl_reference_to_candidate"] == pytest.approx(0.5 * math.log(4.0 / 3.0), rel=1e-6)
    # the reference's top-1 is the first of two equal maxima, margin 0
    assert r["reference_top1"] == 0 and r["reference_top1_top2_margin"] == 0.0


def test_p95_index_rule_and_mean():
    # 21 differences 0..20: sorted index (20 * 95) // 100 = 19
    ref = np.zeros(21, np.float32)
    cand = np.arange(21, dtype=np.float32)
    r = compare_logit_distributions(ref, cand)
    assert r["p95_abs_difference"] == 19.0
    assert r["max_abs_difference"] == 20.0 and r["mean_abs_difference"] == 10.0


def test_top_two_ties_and_single_value():
    assert top_two(np.float32([1, 3, 3, 2])) == (1, 3.0, 3.0)
    assert top_two(np.float32([5, 1, 4])) == (0, 5.0, 4.0)
    index, first, second = top_two(np.float32([7]))
    assert (index, first) == (0, 7.0) and second == -math.inf


def test_rejections():
    with pytest.raises(ConformanceError, match="empty"):
        compare_logit_distributions([], [])
    with pytest.raises(ConformanceError, match="vocabularies differ"):
        compare_logit_distributions([1.0], [1.0, 2.0])
    with pytest.raises(ConformanceError, match="finite"):
        compare_logit_distributions([1.0, np.nan], [1.0, 2.0])


def test_bf16_neighbours():
    one, next_up, two_up = np.float32(1.0), np.float32(1.0078125), np.float32(1.015625)
    assert within_one_bf16_ulp([one], [next_up])
    assert not within_one_bf16_ulp([one], [two_up])
    # both zeros are one value; the smallest subnormals of either sign are two apart
    assert ordered_bf16(0x0000) == ordered_bf16(0x8000)
    tiny = np.uint32(0x00010000).view(np.float32)
    assert within_one_bf16_ulp([0.0], [tiny]) and within_one_bf16_ulp([-0.0], [-tiny])
    assert not within_one_bf16_ulp([tiny], [-tiny])
    # values inside one BF16 rounding interval compare equal
    assert within_one_bf16_ulp([np.float32(1.001)], [np.float32(1.002)])
    # non-finite values must match bit for bit
    assert within_one_bf16_ulp([np.inf, 1.0], [np.inf, 1.0])
    assert not within_one_bf16_ulp([np.inf], [np.float32(3e38)])
    assert not within_one_bf16_ulp([1.0, 2.0], [1.0])


def test_token_gate_catches_a_wrong_token_on_a_near_tie():
    """The greedy-token gate of the model tests.  A near tie (top-1 / top-2
    margin below twice the step's logit error) excuses equality with the
    oracle's token but not a token other than the runner's own first maximum,
    so a runner that picks a clearly wrong token fails on a near tie as on a
    clear margin.  (With the runner's own maximum and the max logit error, the
    near-tie bound and equality on clear margins both follow; the gate states
    them too.)"""
    import oracle
    from _data import TokenGate

    want = np.zeros(64, np.float32)
    want[10], want[20], want[30] = 5.0, 4.96875, 1.0  # top-2 margin 0.03125
    got = want.copy()
    got[20] += 0.0625  # the runner's logits move by 0.0625: its maximum is now 20
    wb, gb = oracle.write_bf16(want), oracle.write_bf16(got)
    gate = TokenGate("planted")
    gate.check(20, gb, wb, "near tie, runner picks the runner-up")  # excused: 4.97 >= 5 - 0.125
    assert gate.excused == ["near tie, runner picks the runner-up"]
    with pytest.raises(AssertionError, match="not its logits' argmax"):
        gate.check(30, gb, wb, "near tie, runner picks a token 4 below the maximum")
    clear = want.copy()
    clear[20] = 3.0
    with pytest.raises(AssertionError, match="not its logits' argmax"):
        gate.check(20, oracle.write_bf16(clear), oracle.write_bf16(clear), "clear margin, wrong token")
    gate.check(10, oracle.write_bf16(clear), oracle.write_bf16(clear), "clear margin")
    assert gate.checked == 1
    with pytest.raises(AssertionError):
        gate.finish(max_excused=0)
