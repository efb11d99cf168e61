"""GPU parity with the oracle on the contract's cases.

Restates the reference's device tests (tests/test_cuda.py:90-225): every dtype
with strided inputs and several top-k, boundaries and packed masks, statuses
and request atomicity, full-q proposals, target-error priority, coupled ==
ordinary, the in-flight workspace guard, capacity and alias errors,
non-contiguous outputs, malformed offsets and a real-vocabulary row.
Every call goes through torch.ops.exactsample.verify_out and the C ABI.
"""
import math

import numpy as np
import pytest

from oracle import RequestParams, RngKey, Status, verify_reference
from tests.gpu_helpers import prepared, run_and_compare

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _device(hip_device):
    from exactsample.cuda import load_library
    load_library()  # a missing library on a GPU box is a failure, not a skip


DTYPES = ["float16", "bfloat16", "float32", "float64"]


@pytest.mark.parametrize("dispatch", ["reference", "fused"])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("k", [0, 1, 20, 35])
def test_dtypes_strides_and_top_k(dtype, k, dispatch):
    """Forced paths as the reference's test_cuda.py:44-55 runs them; the
    "reference" dispatch reports path_used 0 (every row on the exact full-row
    path), "fused" 1."""
    import torch
    rows = np.random.default_rng(42).normal(size=(6, 35))
    run_and_compare(rows, [0, 1, 3, 6], [[-1, -1], [2, -1], [3, 4]], params=RequestParams(top_k=k),
                    dtype=getattr(torch, dtype), strided=True, dispatch=dispatch)


@pytest.mark.parametrize("dispatch", ["reference", "fused"])
@pytest.mark.parametrize("list_max", [256, 0])
def test_boundaries_and_packed_masks(list_max, dispatch):
    for p in [.5, np.nextafter(.5, 1), 1.]:
        run_and_compare(np.zeros((4, 4)), [0, 4], [[0, 1, 2]], params=RequestParams(top_k=4, top_p=p),
                        list_max=list_max, dispatch=dispatch)
    mask = np.array([[-2147483648, 1]] * 3, np.int32)
    run_and_compare(np.zeros((3, 35)), [0, 3], [[31, 32]], mask=mask, params=RequestParams(top_k=20),
                    strided=True, list_max=list_max, dispatch=dispatch)


def test_reference_dispatch_on_benchmark_rows():
    """dispatch="reference" on 16 rows of the 128-request configuration
    (V = 151,936): the full-row path for every row, path_used 0."""
    import torch
    import bench
    work = bench.config2(seed=9, requests=16)
    keys = work["keys"]
    run_and_compare(work["rows"], work["offsets"], work["ids"], params=RequestParams(**work["params"]),
                    rng=RngKey([int(x) for x in keys["seed"]], [int(x) for x in keys["stream"]], keys["positions"]),
                    dtype=torch.float32, dispatch="reference")


def test_statuses_and_atomicity():
    for bad in [math.nan, math.inf, -math.inf]:
        run_and_compare([[0., -math.inf], [bad, bad]], [0, 2], [[1]])
    run_and_compare(np.zeros((2, 2)), [0, 2], [[0]], mask=np.zeros((2, 1), np.int32))
    run_and_compare(np.zeros((1, 2)), [0, 0, 1], np.empty((2, 0), np.int64))


def test_full_q_actual_distribution():
    run_and_compare(np.log([[3., 1.], [1., 1.]]), [0, 2], [[1]], params=RequestParams(draft_kind="full", top_k=1),
                    draft_logits=np.log([[1., 3.], [1., 1.]]))
    run_and_compare([[0., 0.], [0., 0.]], [0, 2], [[1]], params=RequestParams(draft_kind="full"),
                    draft_logits=[[0., -math.inf], [0., 0.]])


def test_future_target_error_takes_priority_over_q_zero():
    run_and_compare([[0., 0.], [math.nan, 0.]], [0, 2], [[1]], params=RequestParams(draft_kind="full"),
                    draft_logits=[[0., -math.inf], [0., 0.]])


def test_coupled_matches_ordinary_and_reordered_batch():
    rows = np.array([[0., 1., 2.], [1., 0., 2.], [2., 1., 0.]])
    rng = RngKey(777, 7, [20, 21, 22])
    expected = verify_reference(rows, [0, 1, 2, 3], np.empty((3, 0), np.int64),
                                rng=RngKey([777] * 3, [7] * 3, [20, 21, 22]))
    drafts = expected.tokens[:2, 0].reshape(1, 2)
    out, _, _ = run_and_compare(rows, [0, 3], drafts, rng=rng, mode="coupled")
    assert out.tokens.cpu().tolist() == [expected.tokens[:, 0].tolist()]
    run_and_compare(rows[[2, 0, 1]], [0, 1, 2, 3], np.empty((3, 0), np.int64),
                    rng=RngKey([777] * 3, [7] * 3, [22, 20, 21]))


def test_workspace_conflict_and_separate_plans():
    import torch
    from exactsample.cuda import verify
    if not hasattr(torch.cuda, "_sleep"):
        pytest.skip("torch.cuda._sleep unavailable for the in-flight fixture")
    args = prepared(np.zeros((1, 4)), [0, 1], np.empty((1, 0), np.int64))
    other = prepared(np.zeros((1, 4)), [0, 1], np.empty((1, 0), np.int64))
    first, second = torch.cuda.Stream(), torch.cuda.Stream()
    first.wait_stream(torch.cuda.current_stream())
    second.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(first):
        torch.cuda._sleep(100000000)
        verify(**args)
    with torch.cuda.stream(second):
        with pytest.raises(RuntimeError, match="in flight"):
            verify(**args)
        verify(**other)
    args["plan"].synchronize()
    other["plan"].synchronize()
    assert args["out"].tokens.cpu().tolist() == other["out"].tokens.cpu().tolist()


def test_capacity_failure_and_large_k():
    import torch
    from exactsample.cuda import verify
    out, _, _ = run_and_compare(np.zeros((1, 100)), [0, 1], np.empty((1, 0), np.int64),
                                params=RequestParams(top_k=65))
    assert out.path_used.cpu().tolist() == [1]
    args = prepared(np.zeros((1, 100)), [0, 1], np.empty((1, 0), np.int64))
    args["target_logits"] = torch.zeros((2, 100), device="cuda")
    with pytest.raises(ValueError, match="capacity"):
        verify(**args)


def test_rng_boundaries():
    out, _, _ = run_and_compare(np.zeros((3, 80)), [0, 1, 2, 3], np.empty((3, 0), np.int64),
                                params=RequestParams(top_k=[0, 20, 65]),
                                rng=RngKey([0, 2**63, 2**64 - 1], [0, 2**32 - 1, 9], [0, 2**32 - 1, 100]))
    assert out.path_used.cpu().tolist() == [1, 1, 1]


def test_output_alias_is_rejected():
    from exactsample.cuda import verify
    args = prepared(np.zeros((1, 4)), [0, 1], np.empty((1, 0), np.int64))
    args["out"].tokens = args["rng"].seed.reshape(1, 1)
    with pytest.raises(RuntimeError, match="alias"):
        verify(**args)


def test_noncontiguous_outputs():
    import torch
    from exactsample.cuda import verify
    args = prepared(np.zeros((3, 4)), [0, 1, 3], [[-1], [2]], strided=True)
    out = args["out"]
    backing = torch.full((2, 4), -777, dtype=torch.int64, device="cuda")
    out.tokens = backing[:, ::2]
    for field in ["accepted_len", "status", "path_used"]:
        setattr(out, field, torch.empty(4, dtype=torch.int32, device="cuda")[::2])
    result = verify(**args)
    args["plan"].synchronize()
    assert torch.all(backing[:, 1::2] == -777).item()
    assert result.status.cpu().tolist() == [0, 0]


@pytest.mark.parametrize("offsets", [[1, 1, 2], [0, 2, 1], [0, -1, 2], [0, 1, 3]])
def test_malformed_offsets_make_every_request_invalid(offsets):
    from exactsample.cuda import verify
    args = prepared(np.zeros((2, 4)), offsets, np.empty((2, 0), np.int64))
    out = verify(**args)
    args["plan"].synchronize()
    assert out.status.cpu().tolist() == [int(Status.INVALID_INPUT)] * 2
    assert out.tokens.cpu().tolist() == [[-1], [-1]]


@pytest.mark.parametrize("k", [0, 20])
def test_real_vocabulary_shape(k):
    import torch
    rows = np.random.default_rng(989).normal(size=(2, 151936))
    run_and_compare(rows, [0, 2], [[123]], params=RequestParams(top_k=k), dtype=torch.bfloat16)


def test_requests_without_rows_are_invalid():
    # No rows at all: only the request checks run (reference: verify.cu:6-56,
    # a segment of 1..max_draft+1 rows). The recompute count is cleared too.
    import torch
    from exactsample.cuda import CudaRequestParams, CudaRngKey, plan, verify
    work = plan(4, 4, 1, 8)
    work.workspace.fill_(0xff)  # stale header words from an earlier call
    out = work.allocate_output()
    one64 = torch.zeros(1, dtype=torch.int64, device="cuda")
    onef = torch.ones(1, dtype=torch.float64, device="cuda")
    verify(torch.zeros((0, 8), device="cuda"), torch.zeros(2, dtype=torch.int64, device="cuda"),
           torch.zeros((1, 1), dtype=torch.int64, device="cuda"),
           params=CudaRequestParams(onef, one64, onef, torch.zeros(1, dtype=torch.float64, device="cuda"), one64 * 0),
           rng=CudaRngKey(one64, one64, torch.zeros(0, dtype=torch.int64, device="cuda")), plan=work, out=out)
    assert work.fallbacks() == 0
    assert out.num_requests == 1
    assert out.status[:1].cpu().tolist() == [int(Status.INVALID_INPUT)]
    assert out.tokens[:1].cpu().tolist() == [[-1, -1]]
    assert out.accepted_len[:1].cpu().tolist() == [0]


def test_empty_batch_is_valid():
    import torch
    from exactsample.cuda import CudaRequestParams, CudaRngKey, plan, verify
    work = plan(4, 4, 1, 8)
    out = work.allocate_output()
    z64 = torch.zeros(0, dtype=torch.int64, device="cuda")
    zf = torch.zeros(0, dtype=torch.float64, device="cuda")
    verify(torch.zeros((0, 8), device="cuda"), torch.zeros(1, dtype=torch.int64, device="cuda"),
           torch.zeros((0, 1), dtype=torch.int64, device="cuda"),
           params=CudaRequestParams(zf, z64, zf, zf, z64), rng=CudaRngKey(z64, z64, z64), plan=work, out=out)
    work.synchronize()
    assert out.num_requests == 0
