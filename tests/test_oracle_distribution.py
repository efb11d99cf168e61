"""Pins the oracle's target distribution (python/exactsample/reference.py:30-86).

Checks are hand-calculated closed forms (the reference's own examples in
tests/exact/test_hand_examples.py and tests/edge/test_contract_edges.py),
an exhaustive enumeration of uniform rows with a closed-form support
(tests/exact/test_exhaustive_oracle.py:12-27), and the exact-fsum prefix
search against math.fsum on every prefix.
"""
import math

import numpy as np
import pytest

from oracle import Status, distribution
from oracle.reference import shortest_prefix, unpack_mask


def check(weights, expected, **kw):
    p, status = distribution(np.log(np.asarray(weights, dtype=np.float64)), **kw)
    assert status == Status.OK
    np.testing.assert_allclose(p, expected, rtol=1e-13, atol=1e-15)


def test_hand_examples():
    check([1, 1, 1, 1], [0.25] * 4)
    check([97, 1, 1, 1], [.97, .01, .01, .01])
    check([8, 4, 2, 1], [1, 0, 0, 0], min_p=.75)
    check([1, 1, 1, 1], [.5, .5, 0, 0], top_p=.5)                       # equality includes the token
    check([1, 1, 1, 1], [1 / 3] * 3 + [0], top_p=np.nextafter(.5, 1))   # one ulp more needs a third
    check([4, 2, 2, 1], [2 / 3, 1 / 3, 0, 0], top_k=2)                   # tie: lower ID kept
    check([8, 4, 2, 1], [2 / 3, 1 / 3, 0, 0], min_p=.2, top_k=2, top_p=.7)  # min-p, top-k, top-p order
    check([16, 4, 1], [4 / 7, 2 / 7, 1 / 7], temperature=2)


def test_exhaustive_uniform_rows():
    # Uniform allowed tokens: the support is the first ceil(n * top_p) allowed
    # IDs, each with mass 1/n; any leak through a filter or tie-order error shows.
    for vocab in range(1, 9):
        for bits in range(1, 1 << vocab):
            allowed = [i for i in range(vocab) if bits & (1 << i)]
            for k in [0, 1, vocab]:
                retained = len(allowed) if k == 0 else min(k, len(allowed))
                for top_p in [.25, .5, .75, 1.]:
                    n = math.ceil(retained * top_p)
                    expected = np.zeros(vocab)
                    expected[allowed[:n]] = 1 / n
                    actual, status = distribution(np.zeros(vocab), top_k=k, top_p=top_p,
                                                  mask=np.array([bits], np.int32))
                    assert status == Status.OK
                    np.testing.assert_array_equal(actual, expected)


def test_contract_edges():
    p, s = distribution([1., 3., 2.], top_k=1)
    assert s == Status.OK and p.tolist() == [0, 1, 0]
    np.testing.assert_array_equal(distribution([1., 3., 2.], top_k=3)[0], distribution([1., 3., 2.])[0])
    assert distribution([2., 2., 1.], temperature=0)[0].tolist() == [1, 0, 0]
    assert distribution([2., 2., 1.], temperature=0, mask=np.array([6], np.int32))[0].tolist() == [0, 1, 0]
    for bad in [math.nan, math.inf]:
        p, s = distribution([0., bad], mask=np.array([1], np.int32))   # masked, still invalid
        assert s == Status.INVALID_INPUT and p.tolist() == [0, 0]
    assert distribution([-math.inf] * 3)[1] == Status.NO_VALID_TOKEN
    p, s = distribution([0., 0., -10.], min_p=1)                          # min-p keeps equality
    assert s == Status.OK and p.tolist() == [.5, .5, 0]
    p, s = distribution(np.zeros(35), mask=np.array([-2147483648, 1], np.int32))
    assert np.flatnonzero(p).tolist() == [31, 32] and p[[31, 32]].tolist() == [.5, .5]
    for params in [dict(temperature=-1), dict(temperature=math.nan), dict(top_p=0), dict(top_p=1.1),
                   dict(min_p=-.1), dict(min_p=1.1), dict(top_k=-1), dict(top_k=1.5), dict(top_k=True),
                   dict(top_k=3)]:
        assert distribution([0., 1.], **params)[1] == Status.INVALID_INPUT, params
    assert distribution([0., 1.], mask=np.array([0], np.int32))[1] == Status.NO_VALID_TOKEN


def test_negative_zero_equals_positive_zero():
    # -0 and +0 are equal logits, so top-k keeps the lower ID.
    p, _ = distribution(np.array([-0.0, 0.0, -1.0]), top_k=1)
    assert p.tolist() == [1, 0, 0]
    p, _ = distribution(np.array([0.0, -0.0, -1.0]), top_k=1)
    assert p.tolist() == [1, 0, 0]


def test_underflowing_weights_leave_the_support():
    # exp((l - max) / T) underflows to 0 far below the maximum: zero mass, not kept.
    p, s = distribution(np.array([0., -800., -1.]), temperature=1.0)
    assert s == Status.OK and p[1] == 0 and p[0] > 0 and p[2] > 0
    p, s = distribution(np.array([0., -8., -1.]), temperature=0.001)
    assert s == Status.OK and p.tolist() == [1, 0, 0]


def test_mask_unpacking_bit_order():
    words = np.array([0b1011, -2147483648], np.int32)
    bits = unpack_mask(words, 64)
    assert np.flatnonzero(bits).tolist() == [0, 1, 3, 63]


def fsum_loop(weights, target):
    prefix = []
    for count, w in enumerate(weights, 1):
        prefix.append(float(w))
        if math.fsum(prefix) >= target:
            return count
    return len(weights)


def test_shortest_prefix_equals_the_fsum_loop():
    g = np.random.default_rng(1)
    for trial in range(300):
        n = int(g.integers(1, 60))
        kind = trial % 3
        if kind == 0:
            w = np.exp(-np.sort(g.exponential(2.0, size=n)))
        elif kind == 1:
            w = np.ones(n)                                     # integer prefix sums: exact boundaries
        else:
            w = np.exp(-np.sort(g.exponential(40.0, size=n)))  # wide dynamic range
        total = math.fsum(w)
        for p in [g.random(), 0.5, count / n if (count := int(g.integers(1, n + 1))) else 1, 1.0,
                  np.nextafter(0.5, 1)]:
            target = float(p) * total
            assert shortest_prefix(w, target) == fsum_loop(w, target)
            for t in [np.nextafter(target, 0), np.nextafter(target, 2)]:
                assert shortest_prefix(w, t) == fsum_loop(w, t)


def test_shortest_prefix_rounding_boundary():
    # 1 + 2^-53 rounds to 1 (ties to even), 1 + 2^-53 + 2^-105 rounds up: the
    # prefix search must see the correctly rounded sum, not a naive one.
    w = [1.0, 2.0**-53, 2.0**-105]
    assert shortest_prefix(w, np.nextafter(1.0, 2)) == 3 == fsum_loop(w, np.nextafter(1.0, 2))
    assert shortest_prefix(w, 1.0) == 1
