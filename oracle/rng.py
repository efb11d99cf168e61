"""Philox4x32-10 with exactsample's v1 counter layout, in Python and NumPy.

Restates python/exactsample/rng.py:22-65 and docs/rng.md:1-28:

* key     = (seed & 0xffffffff, seed >> 32)
* counter = (stream_id, position, substream, token // 4); lane = token % 4
* uniform = (word + 0.5) / 2**32, an exactly representable double in (0, 1)
* gumbel  = -log(-log(uniform)) with CPython's ``math.log``

``philox4x32`` is the scalar Python-integer form the reference uses;
``philox4x32_np`` evaluates many counters at once in uint64 NumPy arithmetic
(every product of two 32-bit words fits in 64 bits, so it is exact) and gives
bit-identical words. Both are pinned by the Random123 known-answer vectors.
"""
import math
import operator

import numpy as np

_U32 = (1 << 32) - 1
_U64 = (1 << 64) - 1
_M0, _M1 = 0xD2511F53, 0xCD9E8D57      # Philox multipliers (docs/rng.md:3)
_W0, _W1 = 0x9E3779B9, 0xBB67AE85      # Weyl key increments (docs/rng.md:4)


def _uint(value, maximum, name):
    """Integer in [0, maximum], rejecting bools (rng.py:10-17)."""
    try:
        result = operator.index(value)
    except TypeError as exc:
        raise ValueError(f"{name} must be an integer") from exc
    if isinstance(value, bool) or not 0 <= result <= maximum:
        raise ValueError(f"{name} outside [0, {maximum}]")
    return result


def philox4x32(counter, key):
    """Four uint32 output words for four counter words and two key words (rng.py:20-41)."""
    if len(counter) != 4 or len(key) != 2:
        raise ValueError("Philox requires 4 counter and 2 key words")
    c0, c1, c2, c3 = [_uint(x, _U32, "counter") for x in counter]
    k0, k1 = [_uint(x, _U32, "key") for x in key]
    for _ in range(10):
        hi0, lo0 = divmod(_M0 * c0, 1 << 32)
        hi1, lo1 = divmod(_M1 * c2, 1 << 32)
        c0, c1, c2, c3 = (hi1 ^ c1 ^ k0) & _U32, lo1, (hi0 ^ c3 ^ k1) & _U32, lo0
        k0, k1 = (k0 + _W0) & _U32, (k1 + _W1) & _U32
    return c0, c1, c2, c3


def philox4x32_np(c0, c1, c2, c3, k0, k1):
    """Vectorised Philox over broadcastable uint32-valued arrays; returns 4 uint64 arrays."""
    c0, c1, c2, c3 = (np.asarray(x, dtype=np.uint64) & np.uint64(_U32) for x in (c0, c1, c2, c3))
    k0 = np.asarray(k0, dtype=np.uint64) & np.uint64(_U32)
    k1 = np.asarray(k1, dtype=np.uint64) & np.uint64(_U32)
    mask, shift = np.uint64(_U32), np.uint64(32)
    m0, m1, w0, w1 = np.uint64(_M0), np.uint64(_M1), np.uint64(_W0), np.uint64(_W1)
    for _ in range(10):
        p0 = c0 * m0
        p1 = c2 * m1
        c0, c1, c2, c3 = ((p1 >> shift) ^ c1 ^ k0) & mask, p1 & mask, ((p0 >> shift) ^ c3 ^ k1) & mask, p0 & mask
        k0 = (k0 + w0) & mask
        k1 = (k1 + w1) & mask
    return c0, c1, c2, c3


def random_word(seed, stream_id, position, substream=0, token=0):
    """The 32-bit word that addresses one token (rng.py:44-55)."""
    seed = _uint(seed, _U64, "seed")
    stream_id = _uint(stream_id, _U32, "stream_id")
    position = _uint(position, _U32, "position")
    substream = _uint(substream, _U32, "substream")
    token = _uint(token, (1 << 34) - 1, "token")
    words = philox4x32((stream_id, position, substream, token // 4), (seed & _U32, seed >> 32))
    return words[token % 4]


def words_for_tokens(seed, stream_id, position, substream, tokens):
    """Vectorised ``random_word`` for an integer array of token IDs (same words)."""
    seed = _uint(seed, _U64, "seed")
    stream_id = _uint(stream_id, _U32, "stream_id")
    position = _uint(position, _U32, "position")
    substream = _uint(substream, _U32, "substream")
    tokens = np.asarray(tokens, dtype=np.int64)
    if tokens.size and (tokens.min() < 0 or tokens.max() >= (1 << 34)):
        raise ValueError("token outside [0, 2**34)")
    blocks = (tokens // 4).astype(np.uint64)
    lanes = tokens % 4
    out = philox4x32_np(stream_id, position, substream, blocks, seed & _U32, seed >> 32)
    stacked = np.stack(out, axis=-1)
    return np.take_along_axis(stacked, lanes[..., None], axis=-1)[..., 0]


def uniform(seed, stream_id, position, substream=0, token=0):
    """(word + 0.5) / 2**32: exact in FP64 and strictly inside (0, 1) (rng.py:58-60)."""
    return (random_word(seed, stream_id, position, substream, token) + 0.5) / (1 << 32)


def gumbel(seed, stream_id, position, substream=0, token=0):
    """-log(-log(u)) with math.log, the oracle's noise (rng.py:63-64)."""
    return -math.log(-math.log(uniform(seed, stream_id, position, substream, token)))


def gumbel_from_word(word):
    """The same noise from an already generated word (identical float arithmetic)."""
    return -math.log(-math.log((int(word) + 0.5) / (1 << 32)))
