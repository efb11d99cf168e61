"""Pins the oracle's verification walk (python/exactsample/reference.py:125-255).

* hand-worked rejections (reference tests/exact/test_hand_examples.py:33-45)
* contract edges (reference tests/edge/test_contract_edges.py:52-112)
* identities that hold for any correct implementation: slot permutation,
  coupled == ordinary sampling up to the first mismatch for every draft
  triple, replay (reference tests/invariance/test_identity.py)
* the reference's golden outputs on captured Qwen3-8B logits
"""
import math
from itertools import product
from unittest.mock import patch

import numpy as np
import pytest

from oracle import RequestParams, RngKey, Status, verify_reference
from tests.golden import capture as cap


def ordinary(rows, seed, stream, positions, params=None):
    return verify_reference(rows, np.arange(len(rows) + 1), np.empty((len(rows), 0), np.int64),
                            rng=RngKey([seed] * len(rows), [stream] * len(rows), positions),
                            params=params).tokens[:, 0]


def test_reject_first_and_middle_draft():
    out = verify_reference([[0., -math.inf], [0., 0.]], [0, 2], [[1]], rng=RngKey(123, 0, [4, 5]))
    assert out.status.tolist() == [0] and out.tokens.tolist() == [[0, -1]] and out.accepted_len.tolist() == [0]
    out = verify_reference([[0., -math.inf], [-math.inf, 0.], [0., 0.]], [0, 3], [[0, 0]],
                           rng=RngKey(456, 0, [4, 5, 6]))
    assert out.tokens.tolist() == [[0, 1, -1]] and out.accepted_len.tolist() == [1]


def test_status_edges():
    out = verify_reference(np.zeros((1, 2)), [0, 0, 1], np.empty((2, 0), np.int64), rng=RngKey([2, 3], [0, 0], [0]))
    assert out.status.tolist() == [Status.INVALID_INPUT, Status.OK] and out.tokens[0].tolist() == [-1]
    out = verify_reference([[0., 0.], [0., 0.]], [0, 2], [[1]], draft_logits=[[0., -math.inf], [0., 0.]],
                           params=RequestParams(draft_kind="full"), rng=RngKey(3, 0, [0, 1]))
    assert out.status.tolist() == [Status.DRAFT_ZERO_PROB] and out.tokens.tolist() == [[-1, -1]]
    out = verify_reference([[0., -math.inf], [math.nan, 0.]], [0, 2], [[1]], rng=RngKey(5, 0, [0, 1]))
    assert out.status.tolist() == [Status.INVALID_INPUT] and out.tokens.tolist() == [[-1, -1]]
    for draft in [-1, 2]:
        out = verify_reference(np.zeros((2, 2)), [0, 2], [[draft]], rng=RngKey(3, 0, [0, 1]))
        assert out.status.tolist() == [Status.INVALID_INPUT]
    out = verify_reference(np.zeros((2, 2)), [0, 1, 2], np.empty((2, 0), np.int64),
                           rng=RngKey([2**64 - 1, 0], [2**32 - 1, 0], [2**32 - 1, 0]))
    assert out.status.tolist() == [0, 0]
    out = verify_reference([[-math.inf] * 2] * 2, [0, 2], [[2]], rng=RngKey(0, 0, [0, 1]))
    assert out.status.tolist() == [Status.INVALID_INPUT]  # metadata before NO_VALID_TOKEN
    # A later target failure outranks an earlier q failure.
    out = verify_reference([[0., 0.], [math.nan, 0.]], [0, 2], [[1]], params=RequestParams(draft_kind="full"),
                           draft_logits=[[0., -math.inf], [0., 0.]], rng=RngKey(1, 0, [0, 1]))
    assert out.status.tolist() == [Status.INVALID_INPUT]
    for bad in [dict(seed=2**64), dict(stream_id=2**32), dict(positions=[-1, 0])]:
        key = dict(seed=1, stream_id=0, positions=[0, 1])
        key.update(bad)
        out = verify_reference(np.zeros((2, 2)), [0, 2], [[0]], rng=RngKey(**key))
        assert out.status.tolist() == [Status.INVALID_INPUT]
    with pytest.raises(ValueError):
        verify_reference(np.zeros((2, 2)), [0, 2, 1], np.empty((2, 0), np.int64), rng=RngKey(1, 0, [0, 1]))


def test_acceptance_threshold_is_strict():
    with patch("oracle.reference.uniform", return_value=.5):
        out = verify_reference(np.zeros((2, 2)), [0, 2], [[0]], rng=RngKey(1, 0, [0, 1]))
    assert out.accepted_len.tolist() == [0] and out.tokens.tolist() == [[1, -1]]
    with patch("oracle.reference.uniform", return_value=np.nextafter(.5, 0)):
        out = verify_reference(np.zeros((2, 2)), [0, 2], [[0]], rng=RngKey(1, 0, [0, 1]))
    assert out.accepted_len.tolist() == [1]


def test_slot_permutation_and_insertion():
    rows = np.array([[1., 2., 3., 0.], [4., 0., 1., 2.], [0., 0., 0., 0.]])
    seeds, streams, positions = [12, 99, 123], [0, 1, 3], [100, 5, 12]
    original = verify_reference(rows, [0, 1, 2, 3], np.empty((3, 0), np.int64), rng=RngKey(seeds, streams, positions))
    order = np.array([2, 0, 1])
    permuted = verify_reference(rows[order], [0, 1, 2, 3], np.empty((3, 0), np.int64),
                                rng=RngKey(np.array(seeds)[order], np.array(streams)[order], np.array(positions)[order]))
    np.testing.assert_array_equal(original.tokens[order], permuted.tokens)
    for r in range(3):
        np.testing.assert_array_equal(ordinary(rows[r:r + 1], seeds[r], streams[r], [positions[r]]), original.tokens[r])


def test_coupled_equals_ordinary_for_every_draft_triple():
    rows = np.array([[0., 1., -1.], [1., 1., 0.], [2., -1., 0.], [-2., 0., 1.]])
    for seed in [0, 1, 0xFFFFFFFFFFFFFFFF]:
        target = ordinary(rows, seed, 17, [10, 11, 12, 13])
        for drafts in product(range(3), repeat=3):
            out = verify_reference(rows, [0, 4], [drafts], rng=RngKey(seed, 17, [10, 11, 12, 13]), mode="coupled")
            accepted = next((i for i, (x, y) in enumerate(zip(drafts, target)) if x != y), 3)
            assert out.accepted_len.tolist() == [accepted] and out.status.tolist() == [0]
            assert out.tokens[0, :accepted + 1].tolist() == target[:accepted + 1].tolist()
            assert np.all(out.tokens[0, accepted + 1:] == -1)


def test_scalar_and_vectorised_rng_agree():
    g = np.random.default_rng(4)
    rows = g.normal(scale=2.0, size=(6, 300))
    kw = dict(params=RequestParams(temperature=[1.0, 0.7], top_k=[0, 40], top_p=[1.0, 0.9]),
              rng=RngKey([5, 2**64 - 3], [1, 2**32 - 1], g.integers(0, 2**32, size=6)))
    a = verify_reference(rows, [0, 3, 6], [[4, 9], [1, 2]], **kw)
    b = verify_reference(rows, [0, 3, 6], [[4, 9], [1, 2]], vectorized_rng=False, **kw)
    for field in ("tokens", "accepted_len", "status"):
        np.testing.assert_array_equal(getattr(a, field), getattr(b, field))


def test_statistics_of_the_ratio_chain():
    # The verification marginal of the first emitted token equals p (the
    # speculative-sampling law), and one-hot acceptance happens with
    # probability p[x]. Both are checked with a 6-sigma binomial bound.
    p_logits = np.log([[1., 3.], [1., 1.]])
    n, zero, accepted = 4000, 0, 0
    for seed in range(n):
        out = verify_reference(p_logits, [0, 2], [[1]], rng=RngKey(seed, 7, [3, 4]))
        zero += out.tokens[0, 0] == 0
        accepted += out.accepted_len[0]
    for count, prob in [(zero, .25), (accepted, .75)]:
        assert abs(count - n * prob) < 6 * math.sqrt(n * prob * (1 - prob))


@pytest.mark.parametrize("name,requests,drafts", cap.CELLS)
def test_reference_golden_outputs_on_captured_logits(name, requests, drafts):
    capture = cap.load_capture()
    rows, offsets, ids, seeds, streams, positions = cap.workload(capture, requests, drafts)
    logits = cap.bf16_bits_to_float32(capture["logits_bf16"][rows]).astype(np.float64)
    out = verify_reference(logits, offsets, ids, params=RequestParams(**cap.PARAMS[name]),
                           rng=RngKey(seeds.astype(np.uint64), streams, positions))
    expected = cap.expected_outputs(name, requests, drafts)
    for field in ("tokens", "accepted_len", "status"):
        np.testing.assert_array_equal(getattr(out, field), expected[field], err_msg=field)
