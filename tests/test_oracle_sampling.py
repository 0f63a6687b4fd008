"""Pins the sampler's restatement (oracle/sampling_ref.py) with closed forms: the kept set of
top-k and top-p on hand-made rows, the renormalised distribution, inverse-CDF draws at known
uniforms, and ties kept at both thresholds."""
import numpy as np
import pytest

from oracle import sampling_ref as sr


def test_top_k_keeps_the_k_largest():
    x = np.array([0.5, 3.0, -1.0, 2.0, 1.0])
    assert sr.kept_set(x, 2, 1.0).tolist() == [False, True, False, True, False]
    assert sr.kept_set(x, 0, 1.0).all() and sr.kept_set(x, 5, 1.0).all() and sr.kept_set(x, 9, 1.0).all()
    # ties at the k-th value are kept
    assert sr.kept_set(np.array([1.0, 2.0, 2.0, 0.0]), 1, 1.0).tolist() == [False, True, True, False]


def test_top_p_is_the_smallest_nucleus():
    # probabilities 0.5, 0.25, 0.125, 0.125 (logits log2-spaced)
    x = np.log(np.array([0.5, 0.25, 0.125, 0.125]))
    assert sr.kept_set(x, 0, 0.5).tolist() == [True, False, False, False]
    assert sr.kept_set(x, 0, 0.51).tolist() == [True, True, False, False]
    assert sr.kept_set(x, 0, 0.75).tolist() == [True, True, False, False]
    assert sr.kept_set(x, 0, 0.76).tolist() == [True, True, True, True]  # the 0.125 tie is kept whole
    # top-p measured on the renormalised top-k set: top-2 = {0.5, 0.25} -> 2/3, 1/3
    assert sr.kept_set(x, 2, 0.6).tolist() == [True, False, False, False]
    assert sr.kept_set(x, 2, 0.7).tolist() == [True, True, False, False]


def test_distribution_and_inverse_cdf():
    x = np.log(np.array([0.1, 0.2, 0.3, 0.4]))
    p = sr.probabilities(x, 3, 1.0)  # drops 0.1, renormalises 0.2 / 0.3 / 0.4 over 0.9
    np.testing.assert_allclose(p, [0.0, 2 / 9, 3 / 9, 4 / 9])
    # the cumulative boundaries 2/9, 5/9 in vocabulary order
    assert sr.sample(x, 3, 1.0, 0.0) == 1
    assert sr.sample(x, 3, 1.0, 2 / 9 - 1e-9) == 1
    assert sr.sample(x, 3, 1.0, 2 / 9 + 1e-9) == 2
    assert sr.sample(x, 3, 1.0, 5 / 9 + 1e-9) == 3
    assert sr.sample(x, 3, 1.0, 0.999999) == 3
    # top_k = 1 is the argmax whatever u is
    assert {sr.sample(x, 1, 1.0, u) for u in (0.0, 0.3, 0.99)} == {3}


def test_nan_and_masked_logits_are_never_drawn():
    x = np.array([np.nan, -np.inf, 1.0, 2.0])
    p = sr.probabilities(x, 0, 1.0)
    assert p[0] == 0 and p[1] == 0
    assert pytest.approx(p[2] + p[3]) == 1.0
