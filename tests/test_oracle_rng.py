"""Pins the oracle's Philox4x32-10 and its counter layout.

Known answers come from outside this repository: the Random123 KAT vectors
(github.com/DEShawResearch/random123, tests/kat_vectors; also quoted by the
reference at tests/exact/test_philox.py:9-14) and the zero-key vector of
docs/rng.md:26-27.
"""
import math

import numpy as np
import pytest

from oracle import gumbel, philox4x32, random_word, uniform, words_for_tokens
from oracle.rng import gumbel_from_word, philox4x32_np

KATS = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("counter,key,expected", KATS)
def test_random123_known_answers(counter, key, expected):
    assert tuple(philox4x32(counter, key)) == expected
    out = philox4x32_np(*[np.array([c]) for c in counter], key[0], key[1])
    assert tuple(int(x[0]) for x in out) == expected


def test_lane_addressing_and_open_interval():
    # Counter (stream, position, substream, token // 4) = 0 and key 0 give the
    # zero KAT; token t picks word t % 4 (docs/rng.md:6-9).
    expected = KATS[0][2]
    for token in range(8):
        word = expected[token % 4] if token < 4 else None
        u = uniform(0, 0, 0, 0, token)
        assert 0 < u < 1
        if word is not None:
            assert random_word(0, 0, 0, 0, token) == word
            assert u == (word + 0.5) / 4294967296


def test_counter_words_follow_the_address():
    # Each address component lands in its own counter/key word.
    seed, stream, position, sub, token = 0x0123456789ABCDEF, 77, 4242, 2, 4 * 1000 + 3
    words = philox4x32((stream, position, sub, token // 4), (seed & 0xFFFFFFFF, seed >> 32))
    assert random_word(seed, stream, position, sub, token) == words[3]
    # A different seed half changes the key, not the counter.
    assert random_word(seed ^ (1 << 40), stream, position, sub, token) != words[3]


def test_vectorised_words_equal_scalar_words():
    g = np.random.default_rng(0)
    for _ in range(20):
        seed = int(g.integers(0, 2**63)) * 2 + int(g.integers(0, 2))
        stream, position = int(g.integers(0, 2**32)), int(g.integers(0, 2**32))
        sub = int(g.integers(0, 4))
        tokens = g.integers(0, 200000, size=17)
        vec = words_for_tokens(seed, stream, position, sub, tokens)
        assert [int(x) for x in vec] == [random_word(seed, stream, position, sub, int(t)) for t in tokens]


def test_domain_is_checked():
    for bad in [dict(seed=-1), dict(seed=2**64), dict(stream_id=2**32), dict(position=-1), dict(substream=True)]:
        args = dict(seed=1, stream_id=0, position=0, substream=0, token=0)
        args.update(bad)
        with pytest.raises(ValueError):
            random_word(**args)


def test_gumbel_closed_form_and_range():
    # G = -log(-log u); u in [(0.5)/2^32, (2^32-0.5)/2^32] bounds the noise to
    # [-3.1300, 22.8739] (the extreme words 0 and 2^32-1).
    lo, hi = gumbel_from_word(0), gumbel_from_word(2**32 - 1)
    assert lo == pytest.approx(-math.log(-math.log(0.5 / 2**32)))
    assert -3.1301 < lo < -3.1299
    assert 22.8738 < hi < 22.8740
    for word in [1, 2**31 - 1, 2**31, 2**32 - 2, 123456789]:
        assert lo <= gumbel_from_word(word) <= hi
    assert gumbel(5, 6, 7, 1, 9) == gumbel_from_word(random_word(5, 6, 7, 1, 9))
