"""CPU oracle for exactsample's sampling/verification path.

TEST INFRASTRUCTURE ONLY. Nothing in the product path (the ``exactsample`` package)
imports, links or runs anything from this package. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` use
it, and only as the checker or the timed CPU baseline.

The package restates, in FP64 NumPy, the reference oracle of
simon-jd/exactsample:

* ``rng``       Philox4x32-10 with the v1 counter layout
                (python/exactsample/rng.py:22-65, docs/rng.md:1-28)
* ``reference`` ``distribution``, ``sample_distribution`` and
                ``verify_reference`` (python/exactsample/reference.py:30-255)
* ``types``     the data model (python/exactsample/types.py:7-44)

How each function is pinned (none is checked by retyping its formula):

* ``philox4x32``: the three published Random123 known-answer vectors and the
  zero-key vector of docs/rng.md:26-27 (tests/test_oracle_rng.py).
* ``uniform``/``gumbel``: lane addressing KAT, closed forms, the open-interval
  property, and exhaustive range checks of the noise.
* ``distribution``: the reference's hand-calculated examples, the exhaustive
  V<=8 mask/top-k/top-p enumeration with its closed-form support, contract
  edge cases, and the exact-fsum top-p search checked against ``math.fsum``
  prefix by prefix.
* ``sample_distribution``/``verify_reference``: the reference's reject
  examples, the coupled == ordinary identity for every draft triple, slot
  permutation invariance, the exact laws of the verification chain, and the
  reference's own golden outputs on captured Qwen3-8B logits
  (results/logits/qwen3-8b-8x8.npz, results/a10/rtx4090/outputs-8x8-rtx4090.npz).
"""
from .reference import distribution, proposal_distribution, sample_distribution, verify_reference
from .rng import gumbel, philox4x32, random_word, uniform, words_for_tokens
from .types import PathUsed, RequestParams, RngKey, Status, VerifyOutput

__all__ = ["PathUsed", "RequestParams", "RngKey", "Status", "VerifyOutput",
           "distribution", "proposal_distribution", "sample_distribution",
           "verify_reference", "philox4x32", "random_word", "uniform", "gumbel",
           "words_for_tokens"]
