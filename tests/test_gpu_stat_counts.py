"""The reference's recorded statistical counts, reproduced draw for draw.

The reference ran its pre-registered statistical plan (tests/stat_plan.json)
on its CUDA fused path: ten cells of 2,000,000 draws each, request t keyed by
seed 65536 + t, stream 19, positions 101..., float64 logits, with list_max
256 (results/stat-cuda.json) and 0 (results/stat-cuda-predicate.json). A
bit-exact implementation reproduces every count exactly; a single differing
token anywhere in 20 million calls changes a count. The counts and keys are in
tests/golden/stat_counts.json (written by tests/golden/make_stat_fixture.py).
"""
import json
from pathlib import Path

import numpy as np
import pytest

FIXTURE = json.loads((Path(__file__).parent / "golden" / "stat_counts.json").read_text())
CELLS = {c["name"]: c for c in FIXTURE["cells"]}


def drafts_of(kind):
    return 3 if kind == "accepted" else 0 if kind == "sample" else 1


@pytest.mark.gpu
@pytest.mark.parametrize("list_max", [256, 0])
@pytest.mark.parametrize("name", list(CELLS))
def test_recorded_counts(name, list_max, hip_device):
    import torch
    from exactsample.cuda import CudaRequestParams, CudaRngKey, load_library, plan, verify

    load_library()
    cell = CELLS[name]
    kind, weights = cell["kind"], np.asarray(cell["weights"], dtype=np.float64)
    drafts, vocab = drafts_of(kind), len(weights)
    per = drafts + 1
    samples = FIXTURE["samples_per_cell"]
    batch = 65535 // per
    prm = {"temperature": 1.0, "top_k": 0, "top_p": 1.0, "min_p": 0.0, **cell["params"]}
    proposal = np.random.Generator(np.random.PCG64(FIXTURE["seed_start"] ^ 0x51A7))
    work = plan(batch * per, batch, drafts, vocab)
    work.list_max = list_max
    out = work.allocate_output()
    dev = torch.device("cuda")
    row_block = torch.as_tensor(np.tile(np.log(weights), (batch * per, 1)), device=dev)
    q_block = torch.as_tensor(np.tile(np.log([1.0, 3.0]), (batch * per, 1)), device=dev) if kind == "full" else None
    counts = np.zeros(len(cell["expected"]), dtype=np.int64)
    for begin in range(0, samples, batch):
        size = min(batch, samples - begin)
        ids = np.zeros((size, drafts), dtype=np.int64)
        if kind == "full":
            ids[:, 0] = (proposal.random(size) >= 0.25).astype(np.int64)

        def full(value, dtype):
            return torch.full((size,), value, dtype=dtype, device=dev)

        params = CudaRequestParams(full(prm["temperature"], torch.float64), full(prm["top_k"], torch.int64),
                                   full(prm["top_p"], torch.float64), full(prm["min_p"], torch.float64),
                                   full(1 if kind == "full" else 0, torch.int64))
        seeds = torch.arange(FIXTURE["seed_start"] + begin, FIXTURE["seed_start"] + begin + size, device=dev)
        positions = torch.arange(FIXTURE["position"], FIXTURE["position"] + per, device=dev).repeat(size)
        rng = CudaRngKey(seeds, full(FIXTURE["stream_id"], torch.int64), positions)
        offsets = torch.arange(size + 1, device=dev) * per
        verify(row_block[:size * per], offsets, torch.as_tensor(ids, device=dev), params=params, rng=rng,
               plan=work, out=out, draft_logits=None if q_block is None else q_block[:size * per],
               mode="coupled" if kind == "coupled" else "ratio")
        status = out.status[:size].cpu().numpy()
        assert np.all(status == 0), (name, begin, np.unique(status))
        observed = (out.accepted_len[:size] if kind == "accepted" else out.tokens[:size, 0]).cpu().numpy()
        assert observed.min() >= 0 and observed.max() < len(counts), (name, begin)
        counts += np.bincount(observed, minlength=len(counts))
    assert counts.tolist() == cell["counts"][str(list_max)]
