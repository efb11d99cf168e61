"""Writes tests/golden/conformance_cases.json: the fused-path conformance cases
as data, read by tests/test_gpu_conformance.py.

    python tests/golden/make_conformance_cases.py

The case families are those the reference's fused-path tests exercise
(tests/test_fused.py:59-232): random ragged batches in both kept-set
representations, the top_k_top_p hint, scores and acceptance thresholds too
close for FP32 (which the FP64 recomputation must settle), the min-p
threshold at one part in 10^9, ties at large k, top-p over a full vocabulary
row and over flat rows, the top-p target on an exact prefix sum, masks over
a real vocabulary, and batch invariance. Every parameter of every case is
written out explicitly; logits are described by a generator spec
(``rows``) that the test expands with NumPy from the spec's own seed.
"""
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "conformance_cases.json")


def random_batch(index):
    """A ragged batch of six requests with mixed filters, kinds, ties and -inf."""
    g = np.random.default_rng(90210 + 17 * index)
    vocab = [37, 300, 2500][index % 3]
    drafts = g.integers(0, 4, size=6).tolist()
    mode = "coupled" if index % 4 == 3 else "ratio"
    kinds = ["one_hot" if mode == "coupled" or g.random() < 0.6 else "full" for _ in drafts]
    pick = lambda options: [options[int(i)] for i in g.integers(0, len(options), size=len(drafts))]  # noqa: E731
    params = dict(temperature=pick([0.0, 0.4, 1.0, 1.7]), top_k=pick([0, 1, 3, vocab // 3, vocab]),
                  top_p=pick([1.0, 0.9, 0.6]), min_p=pick([0.0, 0.0, 0.02, 0.3]), draft_kind=kinds)
    rows = int(np.sum(drafts) + len(drafts))
    return dict(
        name=f"random_batch_{index}", family="random_batch", drafts=drafts, mode=mode, params=params,
        rows=dict(kind="normal", seed=int(g.integers(2**31)), shape=[rows, vocab], scale=[1.0, 4.0][index % 2],
                  half_steps=index % 2 == 1, neg_inf=0.05),
        mask=dict(seed=int(g.integers(2**31)), allow=0.8) if index % 3 == 0 else None,
        q=dict(kind="normal", seed=int(g.integers(2**31)), shape=[rows, vocab], scale=2.0) if "full" in kinds else None,
        ids=g.integers(0, vocab, size=(len(drafts), 3)).tolist(),
        rng=dict(seed=[int(s) for s in g.integers(0, 2**62, size=len(drafts)) * 2 + 1],
                 stream=g.integers(0, 2**32, size=len(drafts)).tolist(),
                 positions=g.integers(0, 2**32, size=rows).tolist()))


def cases():
    out = [random_batch(i) for i in range(16)]
    out.append(dict(
        name="hint_batch", family="hint",
        offsets=[0, 1, 3, 4, 6, 7, 8], ids=[[11], [2300], [7], [42], [1999], [5]],
        rows=dict(kind="normal", seed=7007, shape=[8, 2500], scale=4.0, dead_rows=[7]),
        q=dict(kind="normal", seed=7008, shape=[8, 2500], scale=2.0),
        params=dict(temperature=[1.0, 0.0, 0.7, 0.6, 1.0, 0.8], top_k=[0, 0, 20, 0, 3, 0],
                    top_p=[1.0, 1.0, 0.95, 0.9, 1.0, 1.0], min_p=[0.0, 0.0, 0.0, 0.05, 0.0, 0.0],
                    draft_kind=["one_hot", "full", "one_hot", "one_hot", "one_hot", "one_hot"])))
    out.append(dict(name="near_tie_scores", family="near_tie", seed=99, stream=5, position=1000,
                    eps=[1e-10, -1e-10]))
    out.append(dict(name="near_threshold_acceptance", family="threshold", seed=4321, stream=2, position=50,
                    rel=[1e-12, -1e-12]))
    out.append(dict(name="min_p_edge", family="min_p_edge", logits=[0.0, -1.25, -3.0], rel=[-1e-9, 1e-9],
                    seeds=list(range(20))))
    out.append(dict(name="top_k_ties", family="top_k_ties", flat_vocab=5000, flat_k=[1, 100, 2047, 2049, 4999],
                    steps=dict(kind="normal", seed=5005, shape=[3, 3000], scale=1.0, eighths=True),
                    steps_k=[257, 1000, 2999], steps_min_p=0.001, steps_ids=[[-1], [7]]))
    out.append(dict(name="top_p_rows", family="top_p_rows",
                    full=dict(kind="normal", seed=1717, shape=[2, 151936], scale=3.0), full_settings=[[0, 0.9], [1000, 0.8]],
                    flat=dict(kind="normal", seed=1718, shape=[2, 20000], scale=0.5), flat_top_p=[0.9, 0.3]))
    out.append(dict(name="top_p_exact_prefix", family="top_p_prefix", vocab=4096, ones=50, counts=[3, 40], seed=2323))
    out.append(dict(name="masked_vocabulary", family="masked_vocab",
                    rows=dict(kind="normal", seed=1111, shape=[3, 151936], scale=3.0),
                    mask=dict(seed=1112, allow=0.9), top_k=[300, 5000], ids=[[17, 4]]))
    out.append(dict(name="batch_invariance", family="invariance", vocab=1000, drafts=[0, 3, 1, 2, 0],
                    rows_seed=3003, params=dict(temperature=[0.7, 1.0, 0.0, 0.5, 1.2], top_k=[0, 20, 0, 400, 5],
                                                top_p=[0.95, 0.9, 1.0, 1.0, 0.8], min_p=[0.0, 0.0, 0.0, 0.05, 0.0]),
                    seeds=[11, 22, 33, 44, 55], streams=[1, 2, 3, 4, 5],
                    orders=[[0, 1, 2, 3, 4], [4, 2, 0, 3, 1]], repeat=9))
    return out


if __name__ == "__main__":
    with open(OUT, "w") as f:
        json.dump(dict(about="fused-path conformance cases; written by make_conformance_cases.py",
                       cases=cases()), f, indent=1)
    print(OUT)
