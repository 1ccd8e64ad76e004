"""CPU: the argmax check the lm_head GPU tests use, against planted mistakes: a kernel argmax
outside the reference's top two, a gap wider than one bf16 step, and more near-tie rows than
allowed must each fail; an exact match and one genuine near tie pass."""
import numpy as np
import pytest

from conftest import check_argmax


def _logits(rows=4, n=1000, seed=0):
    ref = np.random.default_rng(seed).standard_normal((rows, n))
    return ref, ref.copy()


def test_exact_argmax_passes():
    ref, got = _logits()
    assert check_argmax(got, ref, "exact") == 0


def test_one_near_tie_passes_and_is_counted():
    ref, got = _logits()
    a = ref[1].argmax()
    b = np.argsort(ref[1])[-2]
    ref[1, b] = ref[1, a] * (1 - 2 ** -9)      # reference top two within one bf16 step
    got[1] = ref[1]
    got[1, b] = ref[1, a] * (1 + 2 ** -9)      # the kernel orders them the other way
    assert check_argmax(got, ref, "near tie") == 1


def test_argmax_outside_top_two_fails():
    ref, got = _logits()
    third = np.argsort(ref[0])[-3]
    got[0, third] = ref[0].max() + 1.0
    with pytest.raises(AssertionError, match="top two"):
        check_argmax(got, ref, "third")


def test_gap_wider_than_one_bf16_step_fails():
    ref, got = _logits()
    a, b = ref[2].argmax(), np.argsort(ref[2])[-2]
    ref[2, b] = ref[2, a] * (1 - 2 ** -5)
    got[2, b] = ref[2, a] * 1.5
    with pytest.raises(AssertionError, match="gap"):
        check_argmax(got, ref, "wide gap")


def test_too_many_near_ties_fail():
    ref, got = _logits()
    for r in (0, 3):
        a, b = ref[r].argmax(), np.argsort(ref[r])[-2]
        ref[r, b] = ref[r, a] * (1 - 2 ** -9)
        got[r] = ref[r]
        got[r, b] = ref[r, a] * (1 + 2 ** -9)
    with pytest.raises(AssertionError, match="near-tie rows"):
        check_argmax(got, ref, "two ties")
    assert check_argmax(got, ref, "two ties allowed", max_ties=2) == 2
