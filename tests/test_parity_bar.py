"""CPU checks of the parity bar itself (tests/_cases.py): the O bound is 2e-2 below |O| = 4
and one bf16 step at and above it; a planted error of 0.025 at |O| = 1, or of two steps at
|O| = 5, fails; the LSE bound is the reference's rtol = atol = 1e-3."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from _cases import assert_parity, bf16_step, o_bound


def test_bf16_step_closed_form():
    assert bf16_step(np.array([1.0]))[0] == 2.0 ** -7
    assert bf16_step(np.array([3.99]))[0] == 2.0 ** -6
    assert bf16_step(np.array([4.0]))[0] == 2.0 ** -5
    assert bf16_step(np.array([-6.5]))[0] == 2.0 ** -5
    assert np.all(o_bound(np.array([0.0, 0.5, 3.9, -3.99])) == 2e-2)
    assert o_bound(np.array([4.0]))[0] == 2.0 ** -5
    # consecutive bf16 values really are one step apart
    for x in (1.0, 4.0, 5.5, 100.0):
        b = oracle.bf16_bits(np.array([x], np.float32))
        nxt = oracle.bf16_to_f32(b + 1)[0]
        assert nxt - x == bf16_step(np.array([x]))[0]


def _o(vals):
    return oracle.bf16_bits(np.array(vals, np.float32))


def test_assert_parity_accepts_one_step_at_large_o():
    ref = _o([5.0, 1.0, -4.5])
    got = _o([5.0 + 2 ** -5, 1.0 + 2 ** -7, -4.5])
    lse = np.zeros(1, np.float32)
    assert_parity(got, lse, ref, lse, "one step")


@pytest.mark.parametrize("ref_v,got_v", [(5.0, 5.0 + 2 * 2 ** -5),     # two steps at |O| = 5
                                          (1.0, 1.0 + 0.025),          # 0.025 at |O| = 1
                                          (3.5, 3.5 + 2 * 2 ** -6)])   # 0.031 at |O| = 3.5
def test_assert_parity_rejects_planted_errors(ref_v, got_v):
    lse = np.zeros(1, np.float32)
    with pytest.raises(AssertionError):
        assert_parity(_o([got_v, -4.5]), lse, _o([ref_v, -4.5]), lse, "planted")


def test_lse_bar():
    o = _o([0.0])
    ref = np.array([10.0, 0.0], np.float32)
    assert_parity(o, np.array([10.0 + 0.0109, 0.00099], np.float32), o, ref, "lse ok")
    with pytest.raises(AssertionError):
        assert_parity(o, np.array([10.0 + 0.0111, 0.0], np.float32), o, ref, "lse off")


@pytest.mark.parametrize("ref_v,got_v", [(float("nan"), 1.0),        # NaN in the reference
                                          (1.0, float("nan")),        # NaN in the result
                                          (float("inf"), 3.0e38)])    # inf reference, finite result
def test_assert_parity_rejects_non_finite(ref_v, got_v):
    lse = np.zeros(1, np.float32)
    with pytest.raises(AssertionError):
        assert_parity(_o([got_v, 0.5]), lse, _o([ref_v, 0.5]), lse, "non-finite")
