"""Calls depend on nothing a workspace held before them, and every vocabulary
the op accepts runs.

- Poisoning: a batch that uses every piece of per-call workspace state
  (multi-row requests and their arrival counters, min-p streaming rows and
  their published row maxima, top-k and top-p lists, binned top-p rows and
  their boundary area (arrival counter, gathered count and IDs, or for a
  flat row the bitmap of marked runs), full-row rows, the recompute counter)
  is called, every workspace byte is overwritten (0xFF, then random bytes),
  and the next calls must return the same outputs. This
  is the determinism check the reference runs under its sanitizer
  (tests/sanitizer/run.py:33-42, initcheck), made directly.
- Vocabularies past 64 register tiles per row (f16 and f64 rows, strided
  rows and list-free calls use 1,024-group tiles; f32/bf16 list calls
  4,096-group tiles) take slices of several tiles; the reference accepts any
  vocabulary up to INT32_MAX (csrc/bindings.cpp:63-64).
"""
import numpy as np
import pytest

from oracle import RequestParams, RngKey
from tests.gpu_helpers import run_and_compare

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _device(hip_device):
    from exactsample.cuda import load_library
    load_library()


def _mixed_batch(vocab=20000, seed=31, flat=False):
    g = np.random.default_rng(seed)
    drafts = [0, 3, 0, 2, 0, 0, 1, 0]
    offsets = np.concatenate([[0], np.cumsum(np.array(drafts) + 1)])
    rows = g.normal(0.0, 2.0, size=(offsets[-1], vocab))
    rows[:, g.integers(vocab, size=12)] += 9.0
    if flat:  # request 4 (top-p 0.8): thousands of tokens per quarter-unit bin, a dense boundary range
        rows[offsets[4]] = g.normal(0.0, 0.3, size=vocab)
    ids = np.full((len(drafts), 3), -1)
    for r, d in enumerate(drafts):
        ids[r, :d] = np.argsort(-rows[offsets[r]])[g.integers(0, 5, size=d)]
    params = RequestParams(temperature=[1.0, 0.8, 1.0, 0.6, 0.7, 0.0, 1.0, 1.2],
                           top_k=[0, 20, 0, 0, 0, 0, 0, 300],
                           top_p=[1.0, 0.95, 1.0, 0.9, 0.8, 1.0, 1.0, 1.0],
                           min_p=[0.0, 0.0, 0.05, 0.0, 0.0, 0.0, 0.02, 0.0])
    rng = RngKey([int(x) for x in g.integers(0, 2**40, size=len(drafts))], list(range(len(drafts))),
                 g.integers(0, 4096, size=offsets[-1]))
    return rows, offsets, ids, params, rng


@pytest.mark.parametrize("flat", [False, True])
@pytest.mark.parametrize("list_max", [256, 0])
def test_poisoned_workspace_gives_the_same_outputs(list_max, flat):
    import torch
    from exactsample.cuda import verify
    rows, offsets, ids, params, rng = _mixed_batch(flat=flat)
    out, _, args = run_and_compare(rows, offsets, ids, params=params, rng=rng, dtype=torch.float32,
                                   list_max=list_max)
    requests = len(offsets) - 1
    first = [getattr(out, f)[:requests].clone() for f in ("tokens", "accepted_len", "status", "path_used")]
    gen = torch.Generator(device="cpu").manual_seed(5)
    poisons = [lambda w: w.fill_(0xFF),
               lambda w: w.copy_(torch.randint(0, 256, w.shape, generator=gen, dtype=torch.uint8).to(w.device))]
    for poison in poisons:
        args["plan"].synchronize()
        poison(args["plan"].workspace)
        for f in ("tokens", "accepted_len", "status", "path_used"):
            getattr(args["out"], f).fill_(-7)
        verify(**args)
        args["plan"].synchronize()
        again = [getattr(args["out"], f)[:requests] for f in ("tokens", "accepted_len", "status", "path_used")]
        for a, b in zip(first, again):
            assert torch.equal(a, b)


@pytest.mark.parametrize("dtype, vocab, list_max, strided", [
    ("float16", 262148, 256, False),   # 65 slices of one 1,024-group tile: 2 tiles per slice
    ("float32", 300000, 0, False),     # list-free call: 1,024-group tiles, 74 of them
    ("float64", 270000, 256, True),    # strided rows: element loads
    ("bfloat16", 1048580, 256, False), # 65 slices of 4,096 groups: 2 tiles per slice
])
def test_vocabulary_past_sixty_four_tiles(dtype, vocab, list_max, strided):
    import torch
    g = np.random.default_rng(vocab)
    offsets = np.array([0, 1, 2, 4, 5, 6])
    rows = g.normal(0.0, 3.0, size=(offsets[-1], vocab))
    rows[:, g.integers(vocab, size=8)] += 7.0
    rows[:, -3:] += 12.0  # the largest logits in the last slice
    ids = np.full((5, 1), -1)
    ids[2, 0] = int(np.argmax(rows[2]))
    params = RequestParams(temperature=[1.0, 0.7, 0.9, 1.0, 0.0], top_k=[0, 40, 0, 0, 0],
                           top_p=[1.0, 1.0, 0.9, 1.0, 1.0], min_p=[0.0, 0.0, 0.0, 0.1, 0.0])
    rng = RngKey([3, 4, 5, 6, 7], [0, 1, 2, 3, 4], np.arange(offsets[-1]) + 11)
    run_and_compare(rows, offsets, ids, params=params, rng=rng, dtype=getattr(torch, dtype), list_max=list_max,
                    strided=strided)
    run_and_compare(rows, offsets, ids, params=params, rng=rng, dtype=getattr(torch, dtype), list_max=list_max,
                    strided=strided, dispatch="reference")
