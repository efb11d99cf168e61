"""GPU parity at the benchmark's configurations (V = 151,936).

Every configuration is checked token for token against the FP64 oracle: the
128-request and 64 x 5 cells (every row must finish as a top-k list without
an FP64 fallback), temperature-only rows, the flatness configuration's top-p
and min-p rows in batches of 128 and 1, and the full ragged verification
configuration (256 requests, against its committed oracle outputs, and
under two other slot orders).
"""
import os
import sys

import numpy as np
import pytest

import bench
from oracle import RequestParams, RngKey
from tests.gpu_helpers import expected_for, row_diagnostics

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _device(hip_device):
    from exactsample.cuda import load_library
    load_library()


def _run(work, list_max=None):
    from exactsample.cuda import verify

    args = bench.device_args(work)
    if list_max is not None:
        args["plan"].list_max = list_max
    out = verify(**args, mode=work["mode"])
    keys = work["keys"]
    params = RequestParams(**work["params"])
    rng = RngKey([int(s) for s in keys["seed"]], [int(s) for s in keys["stream"]], keys["positions"])
    mask = None if work.get("allowed") is None else bench.packed_mask(work["allowed"])
    expected = expected_for(args, work["offsets"], work["ids"], params=params, rng=rng, mode=work["mode"], mask=mask)
    requests = len(work["offsets"]) - 1
    for field in ("tokens", "accepted_len", "status"):
        np.testing.assert_array_equal(getattr(out, field).cpu().numpy()[:requests], getattr(expected, field),
                                      err_msg=field)
    return args


def _routes(args):
    return [route for route, _ in row_diagnostics(args["plan"], args["target_logits"].shape[0])]


@pytest.mark.parametrize("cell", ["128x1", "64x5"])
def test_benchmark_cells_match_the_oracle(cell):
    args = _run(bench.CELLS[cell]())
    routes = row_diagnostics(args["plan"], args["target_logits"].shape[0])
    assert args["plan"].fallbacks() == 0
    assert all(route == 3 for route, _ in routes), sorted(set(routes))  # every row finished as a top-k list


def test_slice_maxima_in_the_last_group():
    """Each slice's largest logits sit in its last group of four.

    The tile loads copies of that group for positions past the slice's end;
    the candidate threshold must still count distinct tokens (a row here
    would otherwise store fewer than k candidates).
    """
    work = bench.config2(seed=12)
    rows = work["rows"]
    groups, slices = rows.shape[1] // 4, 10
    gps = -(-groups // slices)
    for s in range(slices):
        last = min((s + 1) * gps, groups) - 1
        rows[:, 4 * last:4 * last + 4] = rows.max(axis=1, keepdims=True) + np.arange(1, 5, dtype=np.float32)
    args = _run(work)
    assert args["plan"].fallbacks() == 0


def test_greedy_and_plain_temperature_rows():
    from exactsample.cuda import CudaRequestParams, verify
    import torch
    work = bench.config2(seed=5)
    temps = np.where(np.arange(128) % 2 == 0, 0.0, 1.0)
    args = bench.device_args(work)
    work["params"] = dict(temperature=temps.tolist(), top_k=[0] * 128, top_p=[1.0] * 128, min_p=[0.0] * 128)
    args["params"] = CudaRequestParams(torch.as_tensor(temps, device="cuda"),
                                       torch.zeros(128, dtype=torch.int64, device="cuda"),
                                       torch.ones(128, dtype=torch.float64, device="cuda"),
                                       torch.zeros(128, dtype=torch.float64, device="cuda"),
                                       torch.zeros(128, dtype=torch.int64, device="cuda"))
    out = verify(**args, mode="ratio")
    keys = work["keys"]
    rng = RngKey([int(s) for s in keys["seed"]], [int(s) for s in keys["stream"]], keys["positions"])
    expected = expected_for(args, work["offsets"], work["ids"], params=RequestParams(**work["params"]), rng=rng)
    np.testing.assert_array_equal(out.tokens.cpu().numpy()[:128], expected.tokens)


def test_top_k_union_beyond_the_merge_wave():
    """A top-k 64 row whose candidate union (792 tokens) is more than the merge
    wave takes (512): nine slices each hold 88 tokens at 1.5, 22 in every wave
    (one per other thread), so each slice's threshold is 1.5 and it stores
    all 88. The whole block finishes the row as a list instead; it needs the
    row's greedy token, which the merge wave finds (slices of top-k rows do
    not track it)."""
    import torch
    from tests.gpu_helpers import run_and_compare

    vocab, tile = 151936, 16 * 256  # groups per slice of the 16-group tile
    rows = np.zeros((2, vocab), np.float32)
    threads = (64 * np.arange(4)[:, None] + 2 * np.arange(22)[None, :]).ravel()  # 22 per wave
    for s in range(1, 10):
        rows[:, 4 * (s * tile + threads)] = 1.5
    rows[:, 7777] = 2.0  # the maximum, alone
    out, fallbacks, args = run_and_compare(rows, [0, 1, 2], np.empty((2, 0), np.int64), dtype=torch.float32,
                                           params=RequestParams(top_k=64, temperature=0.8))
    routes = row_diagnostics(args["plan"], 2)
    assert all(route == 3 for route, _ in routes), routes


# ---- Stream rows: temperature only and min-p, drawn slice by slice. ----
# Route 5 is the streaming draw; 100 + 8 / 9 the full-row path after a
# certificate the streaming draw could not give (scores or the acceptance
# too close for FP32).

@pytest.mark.parametrize("list_max", [256, 0])
def test_temperature_only_rows(list_max):
    """Eight rows at T = 1, no other filter (the CPU-timed configuration)."""
    args = _run(bench.config1(), list_max=list_max)
    assert all(r == 5 for r in _routes(args)), _routes(args)


def test_min_p_rows_with_thresholds_within_an_ulp():
    """128 rows, T = 0.7, min-p 0.05; every tenth row holds a token whose
    weight is within 1e-9 of the threshold (FP64 settles it)."""
    args = _run(bench.config3(filt="min_p"))
    assert all(r in (5, 108) for r in _routes(args)), sorted(set(_routes(args)))


def test_top_p_rows_with_boundaries_on_a_prefix_sum():
    """128 rows, T = 0.7, top-p 0.9; every tenth row puts the target exactly
    on a prefix sum (ten tokens of weight 1)."""
    _run(bench.config3(filt="top_p"))


@pytest.mark.parametrize("mode", ["ratio", "coupled"])
def test_temperature_only_drafts(mode):
    """Drafted requests at T = 1: ratio rows need the slices' kept mass and
    the residual draw (draft excluded); coupled rows the sample."""
    rng = np.random.default_rng(31)
    requests, drafts = 12, 3
    work = bench.config1(seed=31, requests=requests * (drafts + 1))
    work["offsets"] = np.arange(requests + 1, dtype=np.int64) * (drafts + 1)
    rows = work["rows"]
    ids = np.zeros((requests, drafts), np.int64)
    for r in range(requests):
        for d in range(drafts):
            row = rows[r * (drafts + 1) + d]
            ids[r, d] = int(np.argmax(row)) if rng.random() < 0.6 else int(rng.integers(0, rows.shape[1]))
    work["ids"] = ids
    work["keys"]["seed"] = work["keys"]["seed"][:requests]
    work["keys"]["stream"] = work["keys"]["stream"][:requests]
    work["mode"] = mode
    args = _run(work)
    assert all(r in (5, 108, 109) for r in _routes(args)), sorted(set(_routes(args)))


def test_stream_scores_too_close_for_fp32_across_slices():
    """Two tokens in different slices whose scores differ by 1e-10: the
    streaming draw cannot certify either, and FP64 decides."""
    from tests.gpu_helpers import run_and_compare
    from oracle.rng import gumbel
    import torch

    seed, stream, position = 77, 4, 321
    a_id, b_id = 1000, 100000  # in different slices
    ga, gb = gumbel(seed, stream, position, 0, a_id), gumbel(seed, stream, position, 0, b_id)
    for eps in (1e-10, -1e-10):
        row = np.full((1, 151936), -1000.0)
        row[0, a_id] = 0.0
        row[0, b_id] = ga - gb + eps
        out, fallbacks, args = run_and_compare(row, [0, 1], np.empty((1, 0), np.int64), dtype=torch.float64,
                                               rng=RngKey(seed, stream, [position]))
        assert out.tokens[0, 0].item() == (b_id if eps > 0 else a_id)
        assert _routes(args) == [108]


def test_min_p_picks_that_the_row_maximum_excludes():
    """Flat rows (sigma 0.3, T = 0.5, min-p 0.4: about 200 kept tokens
    spread over the slices). Each slice draws against its own maximum, below
    the row's, so its pick may fall under the row's threshold: the merge then
    scans that slice again against the row maximum."""
    rng = np.random.default_rng(8)
    rows = rng.normal(0.0, 0.3, size=(16, 151936)).astype(np.float32)
    work = dict(rows=rows, offsets=np.arange(17, dtype=np.int64), ids=np.full((16, 1), -1, np.int64),
                keys=dict(seed=np.arange(16, dtype=np.int64) + 3, stream=np.arange(16, dtype=np.int64),
                          positions=np.arange(16, dtype=np.int64) * 7),
                params=dict(temperature=0.5, top_k=0, top_p=1.0, min_p=0.4), mode="ratio")
    args = _run(work)
    assert all(r in (5, 108) for r in _routes(args)), sorted(set(_routes(args)))


@pytest.mark.parametrize("variant", ["full_ratio", "one_hot_coupled", "full_coupled"])
def test_ragged_masked_mixed_filters(variant):
    """24 requests of the ragged configuration: draft lengths 0..7, a mask
    allowing 10% of each row, mixed filters, permuted slots."""
    _run(bench.config5(requests=24, variant=variant))


# ---- The full ragged configuration: 256 requests, about 1,150 rows. ----
# Expected outputs: tests/golden/config5_outputs.npz, written by the FP64
# oracle with tests/golden/make_config5_golden.py, with the sha256 of every
# input. The three variants share their inputs; only the draft kind, the mode
# and the proposal logits differ.

CONFIG5_GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "config5_outputs.npz")


@pytest.fixture(scope="module")
def config5_full():
    return bench.config5(requests=256, variant="full_ratio")


def _variant(work, variant):
    out = dict(work)
    n = len(work["offsets"]) - 1
    out["params"] = dict(work["params"], draft_kind=["one_hot" if variant == "one_hot_coupled" else "full"] * n)
    out["mode"] = "ratio" if variant == "full_ratio" else "coupled"
    out["draft_logits"] = None if variant == "one_hot_coupled" else work["draft_logits"]
    return out


def _permuted(work, order):
    """The same requests in slots `order` (slot s holds request order[s])."""
    offsets = work["offsets"]
    spans = [np.arange(offsets[r], offsets[r + 1]) for r in order]
    rows = np.concatenate(spans)
    sizes = [len(s) for s in spans]
    out = dict(work)
    out["rows"] = work["rows"][rows]
    out["allowed"] = work["allowed"][rows]
    if work["draft_logits"] is not None:
        out["draft_logits"] = work["draft_logits"][rows]
    out["offsets"] = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    out["ids"] = work["ids"][order]
    out["keys"] = dict(seed=work["keys"]["seed"][order], stream=work["keys"]["stream"][order],
                       positions=work["keys"]["positions"][rows])
    out["params"] = {k: (list(np.asarray(v, dtype=object)[order]) if isinstance(v, list) else v)
                     for k, v in work["params"].items()}
    return out


def _device_outputs(work):
    from exactsample.cuda import verify
    args = bench.device_args(work)
    out = verify(**args, mode=work["mode"])
    args["plan"].synchronize()
    n = len(work["offsets"]) - 1
    return {f: getattr(out, f).cpu().numpy()[:n] for f in ("tokens", "accepted_len", "status", "path_used")}


@pytest.mark.parametrize("variant", ["full_ratio", "one_hot_coupled", "full_coupled"])
def test_full_ragged_configuration(config5_full, variant):
    import hashlib
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
    from make_config5_golden import input_digests
    golden = np.load(CONFIG5_GOLDEN)
    work = _variant(config5_full, variant)
    for name, value in input_digests(work).items():
        assert str(golden[f"{variant}/sha256/{name}"]) == value, f"input {name} differs from the golden batch's"
    got = _device_outputs(work)
    for field in ("tokens", "accepted_len", "status"):
        np.testing.assert_array_equal(got[field], golden[f"{variant}/{field}"], err_msg=field)
    assert (got["path_used"] == 1).all()
    if variant != "full_ratio":
        return
    # Batch invariance: the same requests in two other slot orders give
    # byte-identical per-request outputs.
    n = len(work["offsets"]) - 1
    for seed in (1, 2):
        order = np.random.default_rng(seed).permutation(n)
        moved = _device_outputs(_permuted(work, order))
        for field in ("tokens", "accepted_len", "status", "path_used"):
            assert hashlib.sha256(moved[field].tobytes()).digest() == hashlib.sha256(
                got[field][order].tobytes()).digest(), field


# ---- Top-p and min-p at batch 1: single rows of the flatness configuration. ----
@pytest.mark.parametrize("filt", ["top_p", "min_p"])
@pytest.mark.parametrize("row", [0, 1, 7, 10, 33, 90])
def test_flatness_rows_one_at_a_time(filt, row):
    """Rows 0, 10 and 90 are the constructed ones (a threshold within an ulp)."""
    _run(bench.config3_single(filt=filt, row=row))


# ---- Top-p with large nuclei: the reference benchmark's T = 0.7, top-p 0.9 setting. ----
@pytest.mark.parametrize("list_max", [256, 0])
@pytest.mark.parametrize("cell", ["128x1_T0.7_p0.9", "64x5_T0.7_p0.9"])
def test_top_p_cells_match_the_oracle(cell, list_max):
    """Nuclei of 1 to about 9,000 tokens (median 225): small ones finish as
    lists, large ones on the full-row path's binned boundary; list_max 0
    sends every row to the full-row path."""
    args = _run(bench.CELLS[cell](), list_max=list_max)
    routes = _routes(args)
    assert all(r in (3, 4) or r >= 100 for r in routes), sorted(set(routes))
