"""es_launch_static, the entry point that allocates nothing, against es_launch.

Two calls in a row through the C ABI, the second smaller than the first: a
ragged verification batch with masks and full proposals (the five-config
generator's 24-request subset, ratio mode), then 10 single-row requests at
T=0.6 / top-k 20 / top-p 0.95. Each call's tokens, accepted lengths, statuses
and paths from the library's static workspace must equal es_launch's with a
plan's workspace, byte for byte. The capacity check is made on the host.
"""
import ctypes

import numpy as np
import pytest

import bench
from exactsample import capi

pytestmark = pytest.mark.gpu


def _abi(args, mode):
    p, r, o = args["params"], args["rng"], args["out"]
    return capi.from_tensors(args["target_logits"], args["cu_rows"], args["draft_ids"], args.get("draft_logits"),
                             p.temperature, p.top_k, p.top_p, p.min_p, p.draft_kind, r.seed, r.stream_id,
                             r.positions, args.get("mask"), args["plan"].workspace, o.tokens, o.accepted_len,
                             o.status, o.path_used, mode=0 if mode == "ratio" else 1,
                             max_draft=args["plan"].max_draft)


def test_static_workspace_matches_es_launch(hip_device):
    import torch
    lib = capi.load()
    stream = torch.cuda.current_stream()
    for work in (bench.config5(requests=24, variant="full_ratio"), bench.config2(requests=10)):
        args = bench.device_args(work)
        abi = _abi(args, work["mode"])
        requests = len(work["offsets"]) - 1
        fields = ("tokens", "accepted_len", "status", "path_used")
        print(f"case: {requests} requests, {work['rows'].shape[0]} rows", flush=True)
        capi.launch(lib, abi, stream)
        torch.cuda.synchronize()
        want = [getattr(args["out"], f)[:requests].clone() for f in fields]
        for f in fields:
            getattr(args["out"], f).fill_(-7)
        capi.launch(lib, abi, stream, static_workspace=True)
        torch.cuda.synchronize()
        got = [getattr(args["out"], f)[:requests] for f in fields]
        for f, a, b in zip(fields, want, got):
            assert torch.equal(a, b), f
        assert bool((got[2] >= 0).all())


def test_static_capacity_is_checked_before_any_device_work(hip_device):
    lib = capi.load()
    a = capi.Arguments()
    a.rows, a.requests, a.vocab = 1362, 1362, 151936  # 8 + 1362 * 12320 bytes > 16 MiB
    assert lib.es_launch_static(ctypes.byref(a), None) == 8
    assert b"static workspace" in lib.es_error_string(8)
    assert lib.es_launch_static(None, None) == 1
