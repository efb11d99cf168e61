"""GPU parity with the reference's own golden outputs on captured Qwen3-8B logits.

The reference committed its CUDA path's outputs for six workloads on a 64-row
bf16 capture (results/a10/rtx4090/outputs-8x8-rtx4090.npz), equal to its FP64
oracle for all 192 requests. The same workloads are rebuilt here
(tests/golden/capture.py) and run through torch.ops.exactsample.verify_out.
"""
import numpy as np
import pytest

from tests.golden import capture as cap

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _device(hip_device):
    from exactsample.cuda import load_library
    load_library()


@pytest.mark.parametrize("name,requests,drafts", cap.CELLS)
@pytest.mark.parametrize("list_max", [256, 0])
def test_captured_logits_match_reference_outputs(name, requests, drafts, list_max):
    import torch
    from exactsample.cuda import CudaRequestParams, CudaRngKey, plan, verify

    capture = cap.load_capture()
    rows, offsets, ids, seeds, streams, positions = cap.workload(capture, requests, drafts)
    logits = torch.as_tensor(capture["logits_bf16"][rows]).view(torch.bfloat16).to("cuda")
    p = cap.PARAMS[name]

    def full(value, dtype):
        return torch.full((requests,), value, device="cuda", dtype=dtype)

    params = CudaRequestParams(full(p["temperature"], torch.float64), full(p["top_k"], torch.int64),
                               full(p["top_p"], torch.float64), full(0.0, torch.float64), full(0, torch.int64))
    rng = CudaRngKey(torch.as_tensor(seeds, device="cuda"), torch.as_tensor(streams, device="cuda"),
                     torch.as_tensor(positions, device="cuda"))
    work = plan(logits.shape[0], requests, ids.shape[1], logits.shape[1])
    work.list_max = list_max
    out = verify(logits, torch.as_tensor(offsets, device="cuda"), torch.as_tensor(ids, device="cuda"),
                 params=params, rng=rng, plan=work, out=work.allocate_output())
    work.synchronize()
    expected = cap.expected_outputs(name, requests, drafts)
    for field in ("tokens", "accepted_len", "status"):
        np.testing.assert_array_equal(getattr(out, field)[:requests].cpu().numpy(), expected[field], err_msg=field)
    assert np.all(out.path_used[:requests].cpu().numpy() == 1)
    if list_max == 256:
        from tests.gpu_helpers import row_diagnostics
        diag = row_diagnostics(work, logits.shape[0])
        assert work.fallbacks() == 0, diag  # as the reference reports on this capture
