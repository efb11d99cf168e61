"""Fused-path conformance on the GPU, from the case spec in
tests/golden/conformance_cases.json (written by make_conformance_cases.py).

Each case family checks one property of the device path against the FP64
oracle: random ragged batches in both kept-set representations (FP64 lists,
list_max 256, and the full-row path, list_max 0) and two logit dtypes; that
the top_k_top_p hint never changes a result; that scores, acceptance
thresholds and min-p thresholds too close for FP32 are settled in FP64 (and
counted in plan.fallbacks()); exact top-k cuts through ties; top-p over full
and flat rows and on an exact prefix sum; masked real-vocabulary rows; and
that a request's outputs do not depend on its batch, slot or the slice count.
"""
import dataclasses
import json
import os

import numpy as np
import pytest

from oracle import RequestParams, RngKey
from oracle.rng import gumbel, uniform
from tests.gpu_helpers import packed_mask, prepared, run_and_compare

pytestmark = pytest.mark.gpu

SPEC = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "conformance_cases.json")
with open(SPEC) as _f:
    CASES = {c["name"]: c for c in json.load(_f)["cases"]}


@pytest.fixture(autouse=True)
def _device(hip_device):
    from exactsample.cuda import load_library
    load_library()


def _torch_dtype(name):
    import torch
    return getattr(torch, name)


def logits_from(spec):
    """Expands a logits generator spec: N(0, scale^2) from its seed, optionally
    on a grid of halves or eighths, with a fraction of -inf and dead rows."""
    g = np.random.default_rng(spec["seed"])
    x = g.normal(0.0, spec["scale"], size=tuple(spec["shape"]))
    if spec.get("half_steps"):
        x = np.round(x * 2) / 2
    if spec.get("eighths"):
        x = np.round(x * 8) / 8
    if spec.get("neg_inf"):
        x[g.random(x.shape) < spec["neg_inf"]] = -np.inf
    for r in spec.get("dead_rows", []):
        x[r] = -np.inf
    return x


def mask_from(spec, shape):
    return packed_mask(np.random.default_rng(spec["seed"]).random(shape) < spec["allow"])


def _no_drafts(n):
    return np.empty((n, 0), np.int64)


# ---------------------------------------------------------------------------
RANDOM = sorted(n for n, c in CASES.items() if c["family"] == "random_batch")


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("list_max", [256, 0])
@pytest.mark.parametrize("name", RANDOM)
def test_random_batch(name, list_max, dtype):
    c = CASES[name]
    rows = logits_from(c["rows"])
    offsets = np.concatenate([[0], np.cumsum(np.array(c["drafts"]) + 1)])
    mask = mask_from(c["mask"], rows.shape) if c["mask"] else None
    q = logits_from(c["q"]) if c["q"] else None
    rng = RngKey(np.array(c["rng"]["seed"], dtype=np.uint64), c["rng"]["stream"], c["rng"]["positions"])
    run_and_compare(rows, offsets, np.array(c["ids"]), params=RequestParams(**c["params"]), rng=rng, mask=mask,
                    draft_logits=q, mode=c["mode"], list_max=list_max, dtype=_torch_dtype(dtype))


@pytest.mark.parametrize("hint", [True, False])
@pytest.mark.parametrize("mode", ["ratio", "coupled"])
def test_top_k_top_p_hint_changes_no_result(mode, hint):
    c = CASES["hint_batch"]
    params = RequestParams(**c["params"])
    extra = dict(draft_logits=logits_from(c["q"]))
    if mode == "coupled":  # a full proposal is invalid in coupled mode: make every draft one-hot
        params, extra = dataclasses.replace(params, draft_kind=["one_hot"] * len(c["ids"])), {}
    run_and_compare(logits_from(c["rows"]), np.array(c["offsets"]), np.array(c["ids"]), params=params, mode=mode,
                    top_k_top_p=hint, dtype=_torch_dtype("bfloat16"), **extra)


def test_scores_closer_than_fp32_are_settled_in_fp64():
    """Two tokens whose scores x + G differ by 1e-10: the token the FP64
    scores pick wins, and the FP32 certificate must have failed."""
    import torch
    c = CASES["near_tie_scores"]
    g0 = gumbel(c["seed"], c["stream"], c["position"], 0, 0)
    g1 = gumbel(c["seed"], c["stream"], c["position"], 0, 1)
    rng = RngKey(c["seed"], c["stream"], [c["position"]])
    for eps in c["eps"]:
        out, fallbacks, _ = run_and_compare(np.array([[0.0, g0 - g1 + eps]]), [0, 1], _no_drafts(1), list_max=0,
                                            dtype=torch.float64, rng=rng)
        assert out.tokens[0, 0].item() == int(eps > 0)
        assert fallbacks > 0
    _, fallbacks, _ = run_and_compare(np.array([[0.0, g0 - g1]], np.float32), [0, 1], _no_drafts(1), list_max=0,
                                      dtype=torch.float32, rng=rng)
    assert fallbacks > 0


def test_acceptance_closer_than_fp32_is_settled_in_fp64():
    """p(draft) within 1e-12 of the acceptance uniform, on either side."""
    import torch
    c = CASES["near_threshold_acceptance"]
    u = uniform(c["seed"], c["stream"], c["position"], 1, 0)
    rng = RngKey(c["seed"], c["stream"], [c["position"], c["position"] + 1])
    for rel in c["rel"]:
        p = u * (1 + rel)  # the target probability of draft token 0
        rows = np.array([[0.0, np.log(1 / p - 1)], [0.0, 0.0]])
        out, fallbacks, _ = run_and_compare(rows, [0, 2], [[0]], list_max=0, dtype=torch.float64, rng=rng)
        assert out.accepted_len[0].item() == int(rel > 0)
        assert fallbacks > 0


@pytest.mark.parametrize("list_max", [256, 0])
def test_min_p_threshold_at_one_part_in_a_billion(list_max):
    import torch
    c = CASES["min_p_edge"]
    rows = np.array([c["logits"]])
    for rel in c["rel"]:
        params = RequestParams(min_p=float(np.exp(c["logits"][1])) * (1 + rel))
        for seed in c["seeds"]:
            run_and_compare(rows, [0, 1], _no_drafts(1), list_max=list_max, dtype=torch.float64, params=params,
                            rng=RngKey(seed, 0, [seed]))


def test_top_k_cuts_through_ties():
    import torch
    c = CASES["top_k_ties"]
    flat = np.zeros((1, c["flat_vocab"]))
    for k in c["flat_k"]:
        for list_max in (256, 0):
            run_and_compare(flat, [0, 1], _no_drafts(1), list_max=list_max, params=RequestParams(top_k=k),
                            dtype=torch.float32)
    steps = logits_from(c["steps"])
    for k in c["steps_k"]:
        run_and_compare(steps, [0, 1, 3], c["steps_ids"], params=RequestParams(top_k=k, min_p=c["steps_min_p"]),
                        dtype=torch.bfloat16)


def test_top_p_over_full_and_flat_rows():
    import torch
    c = CASES["top_p_rows"]
    full = logits_from(c["full"])
    for k, p in c["full_settings"]:
        run_and_compare(full, [0, 2], [[5]], params=RequestParams(top_k=k, top_p=p, temperature=0.7),
                        dtype=torch.bfloat16)
    flat = logits_from(c["flat"])  # nuclei of thousands of tokens
    run_and_compare(flat, [0, 1, 2], _no_drafts(2), list_max=0, params=RequestParams(top_p=c["flat_top_p"]),
                    dtype=torch.float32)


@pytest.mark.parametrize("list_max", [256, 0])
def test_top_p_target_on_an_exact_prefix_sum(list_max):
    """`ones` tokens of weight exactly 1 over a tail 60 logits down: every
    prefix sum of the head is an integer, so top_p = count / ones puts the
    target exactly on one."""
    import torch
    c = CASES["top_p_exact_prefix"]
    g = np.random.default_rng(c["seed"])
    rows = g.normal(size=(1, c["vocab"])) - 60
    rows[0, g.choice(c["vocab"], c["ones"], replace=False)] = 0
    for count in c["counts"]:
        _, fallbacks, _ = run_and_compare(rows, [0, 1], _no_drafts(1), list_max=list_max,
                                          params=RequestParams(top_p=count / c["ones"]), dtype=torch.float32)
        if list_max == 0:
            assert fallbacks > 0


def test_masked_real_vocabulary():
    import torch
    c = CASES["masked_vocabulary"]
    rows = logits_from(c["rows"])
    mask = mask_from(c["mask"], rows.shape)
    for k in c["top_k"]:
        run_and_compare(rows, [0, 3], c["ids"], params=RequestParams(top_k=k, temperature=0.7), mask=mask,
                        dtype=torch.bfloat16)
    run_and_compare(rows[:1], [0, 1], _no_drafts(1), params=RequestParams(temperature=1.3), dtype=torch.bfloat16)


def test_outputs_do_not_depend_on_batch_slot_or_slice_count():
    import torch
    from exactsample.cuda import verify
    c = CASES["batch_invariance"]
    g = np.random.default_rng(c["rows_seed"])
    drafts, vocab = c["drafts"], c["vocab"]
    blocks = [g.normal(scale=3.0, size=(d + 1, vocab)) for d in drafts]
    chosen = [g.integers(0, vocab, size=d) for d in drafts]
    positions = [np.arange(d + 1) + 40 * i for i, d in enumerate(drafts)]

    def outputs(order):
        ids = np.full((len(order), 3), -1)
        for slot, i in enumerate(order):
            ids[slot, :drafts[i]] = chosen[i]
        offsets = np.concatenate([[0], np.cumsum([drafts[i] + 1 for i in order])])
        params = RequestParams(**{k: [v[i] for i in order] for k, v in c["params"].items()})
        rng = RngKey([c["seeds"][i] for i in order], [c["streams"][i] for i in order],
                     np.concatenate([positions[i] for i in order]))
        args = prepared(np.concatenate([blocks[i] for i in order]), offsets, ids, dtype=torch.bfloat16,
                        params=params, rng=rng)
        out = verify(**args)
        args["plan"].synchronize()
        return [(i, (out.tokens[s].tolist(), out.accepted_len[s].item(), out.status[s].item()))
                for s, i in enumerate(order)]

    reference = dict(outputs(c["orders"][0]))
    for order in c["orders"][1:]:
        assert dict(outputs(order)) == reference
    for i in range(len(drafts)):  # alone in its batch
        assert dict(outputs([i]))[i] == reference[i]
    # Many rows run fewer slices per row than few rows: the split must not matter.
    for i, result in outputs(list(range(len(drafts))) * c["repeat"]):
        assert result == reference[i]
