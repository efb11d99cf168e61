"""FP64 NumPy restatement of exactsample's semantic oracle.

Follows python/exactsample/reference.py (cited per function). It is a CPU
checker: tests compare the HIP path's tokens, accepted lengths and statuses
with it bit for bit. It never imports torch or the product package.

Differences from the reference are in speed only, never in the values:

* the packed mask is unpacked with NumPy bit arithmetic instead of a Python
  comprehension (same bits);
* the top-p "shortest prefix whose math.fsum reaches the target" loop, which
  calls math.fsum on every prefix (quadratic), keeps an exact integer running
  sum and compares it with the rounding midpoint below the target. math.fsum
  returns the correctly rounded exact sum, so both decide every prefix the
  same way (tests/test_oracle_distribution.py checks this prefix by prefix);
* with ``vectorized_rng=True`` (the default) the Philox words of the tokens
  that take part in a draw are produced by the NumPy Philox; the noise is then
  formed with the same ``math.log`` calls as the reference. With
  ``vectorized_rng=False`` every word comes from the scalar per-token Philox,
  exactly the reference's algorithm; the CPU baseline times that mode.
"""
import math
import operator

import numpy as np

from .rng import gumbel, gumbel_from_word, uniform, words_for_tokens
from .types import PathUsed, RequestParams, RngKey, Status, VerifyOutput

_UNIT_SHIFT = 1074  # every finite double is an integer multiple of 2**-1074


def _scalar_integer(value):
    """operator.index, rejecting bools (reference.py:11-17)."""
    if isinstance(value, (bool, np.bool_)):
        raise ValueError("booleans are not integer parameters")
    try:
        return operator.index(value)
    except TypeError as exc:
        raise ValueError("expected integer parameter") from exc


def unpack_mask(mask, vocab):
    """Bit t % 32 of int32 word t // 32; None allows everything (reference.py:20-27)."""
    if mask is None:
        return np.ones(vocab, dtype=bool)
    words = np.asarray(mask)
    if words.shape != ((vocab + 31) // 32,) or words.dtype.kind not in "iu" or words.dtype.itemsize != 4:
        raise ValueError("mask must contain ceil(vocab/32) int32 or uint32 words")
    words = words.astype(np.uint32, copy=False)
    tokens = np.arange(vocab)
    return ((words[tokens // 32] >> (tokens % 32).astype(np.uint32)) & np.uint32(1)).astype(bool)


def _units(weight):
    """The exact value of a non-negative double as an integer count of 2**-1074."""
    numerator, denominator = float(weight).as_integer_ratio()
    return numerator << (_UNIT_SHIFT - denominator.bit_length() + 1)


def _reaches(target):
    """A predicate on exact sums S (in 2**-1074 units): is round-to-nearest(S) >= target?

    round(S) >= t exactly when S lies above the midpoint between t and its
    predecessor, or on it when t has an even significand (ties to even).
    """
    target = float(target)
    if not target > 0:
        return lambda s: s >= 0 and float(s) / 2.0 ** _UNIT_SHIFT >= target
    below = float(np.nextafter(target, 0.0))
    twice_mid = _units(below) + _units(target)
    even = (np.float64(target).view(np.uint64) & np.uint64(1)) == 0
    return (lambda s: 2 * s >= twice_mid) if even else (lambda s: 2 * s > twice_mid)


def shortest_prefix(selected_weights, target):
    """Length of the shortest prefix whose math.fsum is >= target.

    Equivalent to the reference's loop (reference.py:76-83), which appends one
    weight at a time and stops at the first ``math.fsum(prefix) >= target``;
    when no prefix reaches the target the loop runs to the end. math.fsum is
    the correctly rounded exact sum, so the exact integer running sum decides
    each prefix the same way.
    """
    reaches = _reaches(target)
    total = 0
    count = 0
    for count, weight in enumerate(selected_weights, 1):
        total += _units(weight)
        if reaches(total):
            return count
    return count


def distribution(logits, *, temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, mask=None):
    """(FP64 probabilities, Status) for one target row (reference.py:30-86).

    Order: mask, temperature, min-p, stable top-k, shortest top-p prefix,
    normalisation. NaN/+inf anywhere, masked or not, is INVALID_INPUT; -inf
    carries zero mass.
    """
    values = np.asarray(logits)
    if values.ndim != 1 or values.size == 0 or values.dtype.kind not in "fiu":
        raise ValueError("logits must be a nonempty real vector")
    values = values.astype(np.float64, copy=True)
    probs = np.zeros(values.size, dtype=np.float64)
    allowed = unpack_mask(mask, values.size)
    try:
        k = _scalar_integer(top_k)
        temperature, top_p, min_p = float(temperature), float(top_p), float(min_p)
        valid = (math.isfinite(temperature) and temperature >= 0 and 0 <= k <= values.size
                 and math.isfinite(top_p) and 0 < top_p <= 1
                 and math.isfinite(min_p) and 0 <= min_p <= 1)
    except (ValueError, TypeError, OverflowError):
        valid = False
    if not valid or np.isnan(values).any() or np.isposinf(values).any():
        return probs, Status.INVALID_INPUT
    active = allowed & np.isfinite(values)
    if not active.any():
        return probs, Status.NO_VALID_TOKEN
    if temperature == 0:
        probs[int(np.argmax(np.where(active, values, -np.inf)))] = 1.0
        return probs, Status.OK
    maximum = np.max(values[active])
    with np.errstate(over="ignore", under="ignore"):
        shifted = (values - maximum) / temperature   # subtract first, then divide
        weights = np.where(active, np.exp(shifted), 0.0)
    active &= weights >= min_p
    active &= weights > 0.0
    ordered = np.flatnonzero(active)
    ordered = ordered[np.argsort(-values[ordered], kind="stable")]  # ties: ascending ID
    if k:
        ordered = ordered[:k]
    selected = weights[ordered]
    denominator = math.fsum(selected.tolist())
    if top_p < 1:
        count = shortest_prefix(selected, top_p * denominator)
        ordered = ordered[:count]
        denominator = math.fsum(weights[ordered].tolist())
    probs[ordered] = weights[ordered] / denominator
    return probs, Status.OK


def proposal_distribution(logits):
    """Actual q, normalised without any target processing (reference.py:89-91)."""
    return distribution(logits)


def sample_distribution(probs, *, seed, stream_id, position, substream=0, vectorized_rng=True):
    """argmax over p > 0 of log(p) + Gumbel, lowest ID on ties (reference.py:94-104)."""
    probs = np.asarray(probs, dtype=np.float64)
    if (probs.ndim != 1 or probs.size == 0 or not np.isfinite(probs).all() or (probs < 0).any()
            or not (probs > 0).any()):
        raise ValueError("probabilities must be nonnegative, finite, and have positive mass")
    support = np.flatnonzero(probs > 0)
    best_token, best_value = -1, -math.inf
    if vectorized_rng:
        words = words_for_tokens(seed, stream_id, position, substream, support)
        log = math.log
        for token, word, p in zip(support.tolist(), words.tolist(), probs[support].tolist()):
            score = log(p) + gumbel_from_word(word)
            if score > best_value:
                best_token, best_value = token, score
        return best_token
    for token in support:
        score = math.log(float(probs[token])) + gumbel(seed, stream_id, position, substream, int(token))
        if score > best_value:
            best_token, best_value = int(token), score
    return best_token


def _per_request(value, count, name):
    """Scalar broadcast or one value per request, keeping uint64 seeds exact (reference.py:107-115)."""
    arr = np.asarray(value, dtype=object)
    if arr.ndim == 0:
        return [arr.item()] * count
    if arr.shape != (count,):
        raise ValueError(f"{name} must be scalar or shape [{count}]")
    return list(arr)


def _bounded_int(value, bits):
    result = _scalar_integer(value)
    if not 0 <= result < (1 << bits):
        raise ValueError(f"integer outside uint{bits}")
    return result


def verify_reference(target_logits, cu_rows, draft_ids, *, params=None, rng: RngKey,
                     draft_logits=None, mask=None, mode="ratio", vectorized_rng=True):
    """Verify a ragged batch under the exactsample v1 contract (reference.py:125-255).

    A request with D drafts owns D+1 consecutive target rows (the last is the
    bonus row); ``draft_ids`` is [requests, max_draft]. Structural errors raise
    ValueError/TypeError; request-local errors give a status with all tokens -1
    and accepted_len 0.
    """
    if mode not in ("ratio", "coupled"):
        raise ValueError("mode must be 'ratio' or 'coupled'")
    params = RequestParams() if params is None else params
    if not isinstance(params, RequestParams) or not isinstance(rng, RngKey):
        raise TypeError("params/RNG must be RequestParams/RngKey")
    logits, offsets, drafts = map(np.asarray, (target_logits, cu_rows, draft_ids))
    if logits.ndim != 2 or logits.shape[1] == 0 or logits.dtype.kind not in "fiu":
        raise ValueError("target_logits must be a real [rows, vocab] array")
    rows, vocab = logits.shape
    if offsets.ndim != 1 or offsets.size == 0 or offsets.dtype.kind not in "iu":
        raise ValueError("cu_rows must be an integer [requests+1] vector")
    bounds = [int(x) for x in offsets]
    if bounds[0] != 0 or bounds[-1] != rows or any(b < a for a, b in zip(bounds[:-1], bounds[1:])):
        raise ValueError("cu_rows must be monotone, start at zero, and end at rows")
    requests = offsets.size - 1
    if drafts.ndim != 2 or drafts.shape[0] != requests or drafts.dtype.kind not in "iu":
        raise ValueError("draft_ids must be an integer [requests, max_draft] array")
    max_draft = drafts.shape[1]
    if any(b - a > max_draft + 1 for a, b in zip(bounds[:-1], bounds[1:])):
        raise ValueError("ragged segment exceeds draft_ids capacity")
    if mask is not None:
        mask = np.asarray(mask)
        if mask.shape != (rows, (vocab + 31) // 32) or mask.dtype.kind not in "iu" or mask.dtype.itemsize != 4:
            raise ValueError("mask must be packed int32 [rows, ceil(vocab/32)]")
    if draft_logits is not None:
        draft_logits = np.asarray(draft_logits)
        if draft_logits.shape != logits.shape or draft_logits.dtype.kind not in "fiu":
            raise ValueError("draft_logits must have target_logits shape and real dtype")
    positions = np.asarray(rng.positions)
    if positions.shape != (rows,):
        raise ValueError("rng.positions must have shape [rows]")
    fields = {name: _per_request(getattr(params, name), requests, name)
              for name in ("temperature", "top_k", "top_p", "min_p", "draft_kind")}
    seeds = _per_request(rng.seed, requests, "seed")
    streams = _per_request(rng.stream_id, requests, "stream_id")
    output = VerifyOutput(
        np.full((requests, max_draft + 1), -1, dtype=np.int64),
        np.zeros(requests, dtype=np.int32),
        np.full(requests, int(Status.OK), dtype=np.int32),
        np.full(requests, int(PathUsed.REFERENCE), dtype=np.int32),
    )

    def draw(p, address, substream):
        return sample_distribution(p, **address, substream=substream, vectorized_rng=vectorized_rng)

    for request in range(requests):
        start, end = bounds[request], bounds[request + 1]
        count = end - start - 1
        kind = fields["draft_kind"][request]
        # Metadata first (reference.py:181-196).
        if count < 0 or kind not in ("one_hot", "full") or (kind == "full" and mode == "coupled"):
            output.status[request] = Status.INVALID_INPUT
            continue
        if count and kind == "full" and draft_logits is None:
            output.status[request] = Status.INVALID_INPUT
            continue
        try:
            seed = _bounded_int(seeds[request], 64)
            stream = _bounded_int(streams[request], 32)
            row_positions = [_bounded_int(pos, 32) for pos in positions[start:end]]
        except (ValueError, TypeError, OverflowError):
            output.status[request] = Status.INVALID_INPUT
            continue
        if any(not 0 <= int(drafts[request, index]) < vocab for index in range(count)):
            output.status[request] = Status.INVALID_INPUT
            continue
        # Every target row, then every full-q proposal row, in order (reference.py:197-219).
        row_probs, proposal_probs = [], []
        local_status = Status.OK
        for row in range(start, end):
            probabilities, local_status = distribution(
                logits[row], mask=None if mask is None else mask[row],
                **{name: fields[name][request] for name in ("temperature", "top_k", "top_p", "min_p")})
            if local_status != Status.OK:
                break
            row_probs.append(probabilities)
        if local_status == Status.OK:
            for index in range(count):
                token = int(drafts[request, index])
                if kind == "full":
                    proposal, local_status = proposal_distribution(draft_logits[start + index])
                    if local_status != Status.OK:
                        break
                    if proposal[token] == 0:
                        local_status = Status.DRAFT_ZERO_PROB
                        break
                    proposal_probs.append(proposal)
        if local_status != Status.OK:
            output.status[request] = local_status
            continue
        # The sequential walk (reference.py:220-252).
        accepted = 0
        for index in range(count):
            p = row_probs[index]
            token = int(drafts[request, index])
            address = dict(seed=seed, stream_id=stream, position=row_positions[index])
            if mode == "coupled":
                sampled = draw(p, address, 0)
                accept = sampled == token
            else:
                q_token = 1.0 if kind == "one_hot" else float(proposal_probs[index][token])
                accept = uniform(seed, stream, row_positions[index], 1, 0) < min(1.0, float(p[token]) / q_token)
                if not accept:
                    if kind == "one_hot":
                        residual = p.copy()
                        residual[token] = 0.0
                    else:
                        residual = np.maximum(p - proposal_probs[index], 0.0)
                    if not (residual > 0).any():   # an empty residual is invalid, never token 0
                        output.status[request] = Status.INVALID_INPUT
                        output.tokens[request] = -1
                        break
                    sampled = draw(residual, address, 2)
            if not accept:
                output.tokens[request, index] = sampled
                break
            output.tokens[request, index] = token
            accepted += 1
        else:
            output.tokens[request, count] = draw(
                row_probs[count], dict(seed=seed, stream_id=stream, position=row_positions[count]), 0)
        if output.status[request] == Status.OK:
            output.accepted_len[request] = accepted
    return output
