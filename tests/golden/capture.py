"""The reference's captured-logit workloads, rebuilt from its committed fixtures.

Fixtures (copied unchanged from the reference's results/):
  qwen3-8b-8x8.npz          64 bf16 rows of Qwen3-8B logits (V = 151,936) with
                            their sequence, step, absolute position and the
                            sampled token; sha256 08049ef7...1806
                            (results/logits/qwen3-8b-8x8.json)
  outputs-8x8-rtx4090.npz   the reference CUDA path's tokens, accepted lengths,
                            statuses and paths for six workloads on that
                            capture, equal to its FP64 oracle for all 192
                            requests (results/agreement-8x8.json)

Workload construction restates bench/sampler.py:44-72 (rows, drafts, keys)
with the cells of bench/agreement.py:27-28 and PARAMS of bench/sampler.py:37-41.
"""
import hashlib
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
CAPTURE = os.path.join(HERE, "qwen3-8b-8x8.npz")
OUTPUTS = os.path.join(HERE, "outputs-8x8-rtx4090.npz")
CAPTURE_SHA256 = "08049ef75adbbb67d400a4e5457a216d4927bf2aa3d3d6cfafc5f5c8b5fc1806"

PARAMS = {
    "qwen": dict(temperature=0.6, top_k=20, top_p=0.95),
    "temperature": dict(temperature=1.0, top_k=0, top_p=1.0),
    "top_p": dict(temperature=0.7, top_k=0, top_p=0.9),
}
CELLS = [("qwen", 64, 0), ("qwen", 16, 4), ("top_p", 64, 0), ("top_p", 16, 4),
         ("temperature", 24, 0), ("temperature", 8, 4)]


def load_capture():
    with open(CAPTURE, "rb") as f:
        digest = hashlib.sha256(f.read()).hexdigest()
    if digest != CAPTURE_SHA256:
        raise RuntimeError(f"capture fixture changed: {digest}")
    with np.load(CAPTURE) as data:
        return {k: data[k] for k in data.files}


def bf16_bits_to_float32(bits):
    """bf16 bit patterns (int16 view) to the float32 values they denote."""
    return (np.asarray(bits).astype(np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def workload(capture, requests, drafts):
    """(row indices, cu_rows, draft_ids, seeds, streams, positions) of one cell."""
    steps = int(capture["step"].max()) + 1
    sequences = int(capture["sequence"].max()) + 1
    rows = []
    ids = np.full((requests, max(drafts, 1)), -1, dtype=np.int64)
    for i in range(requests):
        sequence = i % sequences
        start = (i // sequences) * (drafts + 1) % (steps - drafts)
        first = sequence * steps + start
        rows += list(range(first, first + drafts + 1))
        ids[i, :drafts] = capture["sampled"][first:first + drafts]
    rows = np.array(rows)
    offsets = np.arange(requests + 1, dtype=np.int64) * (drafts + 1)
    seeds = np.arange(requests, dtype=np.int64) + 1000
    streams = np.arange(requests, dtype=np.int64)
    positions = capture["position"][rows].astype(np.int64)
    return rows, offsets, ids, seeds, streams, positions


def expected_outputs(name, requests, drafts):
    with np.load(OUTPUTS) as data:
        key = f"{name}-{requests}x{drafts}"
        return {field: data[f"{key}-{field}"] for field in ("tokens", "accepted_len", "status", "path_used")}
