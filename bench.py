"""Benchmark of exactsample_amd's verify on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--cells 128x1,64x5] [--no-cpu]

A "step" is one ``verify`` call over one batch of synthetic logits already
resident in HBM. The headline workload (value) is 128 requests x 1 row of
V = 151,936 fp32 logits at T=0.6, top-k 20, top-p 0.95; the second cell is 64
requests x (4 one-hot drafts + bonus) verified in ratio mode with the same
settings. Rows come from the peaked generator: base N(mu, sigma^2) with
mu ~ U(-5, 0), sigma ~ U(2, 4); one token + U(6, 14); 15 tokens + U(0, 8);
every even row rounded to the bf16 grid (values stay fp32).

Reported per cell: median and mean event time per call (warm: logits resident
as right after the LM head), median time after a 2 GiB read that evicts the
256 MB Infinity Cache (cold), and the HBM roofline of the call: algorithmic
bytes = one read of every logit row (+ outputs and parameters, < 0.1%).
``cpu_baseline`` times the FP64 oracle (oracle/, the reference algorithm with
its per-token scalar Philox) on a bounded sample of the headline rows, single
threaded.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

VOCAB = 151936
QWEN = dict(temperature=0.6, top_k=20, top_p=0.95, min_p=0.0)
HBM_PEAK = 8.0e12  # bytes/s, MI355X published


# ---------------------------------------------------------------------------
# Synthetic workloads (shared with tests/test_gpu_configs.py).
def peaked_rows(rng, rows, vocab=VOCAB, sigma=(2.0, 4.0)):
    """Per row: N(mu, sigma^2) with one token + U(6,14) and 15 tokens + U(0,8)."""
    mu = rng.uniform(-5.0, 0.0, size=(rows, 1))
    sd = rng.uniform(sigma[0], sigma[1], size=(rows, 1))
    out = (rng.standard_normal((rows, vocab)) * sd + mu).astype(np.float32)
    for r in range(rows):
        picks = rng.choice(vocab, 16, replace=False)
        out[r, picks[0]] += np.float32(rng.uniform(6, 14))
        out[r, picks[1:]] += rng.uniform(0, 8, size=15).astype(np.float32)
    return out


def round_to_bf16(x):
    """Round float32 values to the nearest bf16 (ties to even), kept as float32."""
    bits = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounded = (bits + np.uint32(0x7FFF) + ((bits >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)
    return rounded.view(np.float32)


def config2(seed=2, requests=128):
    """128 requests, one row each, T=0.6 k20 p0.95; even rows on the bf16 grid."""
    rng = np.random.default_rng(seed)
    rows = peaked_rows(rng, requests)
    rows[0::2] = round_to_bf16(rows[0::2])
    offsets = np.arange(requests + 1, dtype=np.int64)
    ids = np.full((requests, 1), -1, dtype=np.int64)
    keys = dict(seed=seed + np.arange(requests, dtype=np.int64), stream=np.arange(requests, dtype=np.int64),
                positions=rng.integers(0, 4096, size=requests).astype(np.int64))
    return dict(rows=rows, offsets=offsets, ids=ids, keys=keys, params=QWEN, mode="ratio")


def config4(seed=4, requests=64, drafts=4):
    """64 requests x (4 drafts + bonus); drafts from the row's top-8 w.p. 0.7, else uniform."""
    rng = np.random.default_rng(seed)
    n = requests * (drafts + 1)
    rows = peaked_rows(rng, n)
    rows[0::2] = round_to_bf16(rows[0::2])
    offsets = np.arange(requests + 1, dtype=np.int64) * (drafts + 1)
    ids = np.zeros((requests, drafts), dtype=np.int64)
    for r in range(requests):
        for d in range(drafts):
            row = rows[r * (drafts + 1) + d]
            if rng.random() < 0.7:
                top8 = np.argpartition(-row, 8)[:8]
                ids[r, d] = int(rng.choice(top8))
            else:
                ids[r, d] = int(rng.integers(0, VOCAB))
    keys = dict(seed=seed + np.arange(requests, dtype=np.int64), stream=np.arange(requests, dtype=np.int64),
                positions=rng.integers(0, 4096, size=n).astype(np.int64))
    return dict(rows=rows, offsets=offsets, ids=ids, keys=keys, params=QWEN, mode="ratio")


CELLS = {"128x1": config2, "64x5": config4}


def device_args(work, device="cuda"):
    import torch
    from exactsample_amd.cuda import CudaRequestParams, CudaRngKey, plan

    requests = len(work["offsets"]) - 1
    p = work["params"]

    def full(value, dtype):
        return torch.full((requests,), value, dtype=dtype, device=device)

    params = CudaRequestParams(full(p["temperature"], torch.float64), full(p["top_k"], torch.int64),
                               full(p["top_p"], torch.float64), full(p["min_p"], torch.float64),
                               full(0, torch.int64))
    rng = CudaRngKey(torch.as_tensor(work["keys"]["seed"], device=device),
                     torch.as_tensor(work["keys"]["stream"], device=device),
                     torch.as_tensor(work["keys"]["positions"], device=device))
    logits = torch.as_tensor(work["rows"], device=device)
    w = plan(logits.shape[0], requests, work["ids"].shape[1], logits.shape[1])
    return dict(target_logits=logits, cu_rows=torch.as_tensor(work["offsets"], device=device),
                draft_ids=torch.as_tensor(work["ids"], device=device), params=params, rng=rng, plan=w,
                out=w.allocate_output())


def algorithmic_bytes(work):
    """One read of every logit row plus parameters and outputs."""
    rows, vocab = work["rows"].shape
    requests = len(work["offsets"]) - 1
    k1 = work["ids"].shape[1] + 1
    params = requests * (5 * 8 + 2 * 8) + rows * 8 + (requests + 1) * 8 + work["ids"].size * 8
    outputs = requests * (k1 * 8 + 3 * 4)
    return rows * vocab * 4 + params + outputs


def time_cell(name, steps, warmup):
    import torch
    from exactsample_amd.cuda import verify

    work = CELLS[name]()
    args = device_args(work)
    stream = torch.cuda.current_stream()

    def call():
        return verify(**args, mode=work["mode"], top_k_top_p=True)

    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    # Per-call events on the stream the kernels run on.
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    stops = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        starts[i].record(stream)
        call()
        stops[i].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per_call = np.array([s.elapsed_time(e) * 1000.0 for s, e in zip(starts, stops)])
    # Cold: evict L2 and the Infinity Cache with a 2 GiB read first.
    flush = torch.ones(512 << 20, dtype=torch.float32, device="cuda")
    cold = []
    for _ in range(min(steps, 30)):
        flush.sum()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record(stream)
        call()
        e.record(stream)
        e.synchronize()
        cold.append(s.elapsed_time(e) * 1000.0)
    del flush
    fallbacks = args["plan"].fallbacks()
    nbytes = algorithmic_bytes(work)
    med = float(np.median(per_call))
    return dict(rows=int(work["rows"].shape[0]), requests=int(len(work["offsets"]) - 1),
                median_us=med, mean_us=float(per_call.mean()), p10_us=float(np.percentile(per_call, 10)),
                p90_us=float(np.percentile(per_call, 90)), cold_median_us=float(np.median(cold)),
                wall_ms=wall * 1000.0, bytes=int(nbytes), achieved_gbs=nbytes / (med * 1e-6) / 1e9,
                frac=nbytes / (med * 1e-6) / HBM_PEAK, fallbacks=int(fallbacks),
                accepted_mean=float(args["out"].accepted_len[:len(work["offsets"]) - 1].float().mean().item()))


def cpu_baseline(budget_s=12.0):
    """The FP64 oracle, single-threaded, on headline rows until the budget is spent."""
    from oracle import RequestParams, RngKey, verify_reference

    work = config2()
    rows = work["rows"].astype(np.float64)
    done, t0 = 0, time.perf_counter()
    while done < len(rows) and time.perf_counter() - t0 < budget_s:
        r = done
        verify_reference(rows[r:r + 1], [0, 1], np.empty((1, 0), np.int64), params=RequestParams(**QWEN),
                         rng=RngKey(int(work["keys"]["seed"][r]), int(work["keys"]["stream"][r]),
                                    [int(work["keys"]["positions"][r])]),
                         vectorized_rng=False)
        done += 1
    elapsed = time.perf_counter() - t0
    per_row = elapsed / done
    return dict(value=per_row * 128 * 1e6, unit="us/call (128 requests, extrapolated from the sample)",
                cores=1, kind="port",
                sample=f"{done} of the 128 headline rows ({elapsed:.1f} s) through oracle.verify_reference "
                       f"with per-token scalar Philox; the FP64 restatement of reference.py")


def main():
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--cells", default="128x1,64x5")
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    args = parser.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this path runs per device and is not sharded across GPUs "
              "(see DESIGN.md, 'More than one GPU').", file=sys.stderr)
        return 2
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 2
    from exactsample_amd.cuda import load_library
    load_library()
    cells = {}
    for name in args.cells.split(","):
        cells[name] = time_cell(name, args.steps, args.warmup)
        print(json.dumps({"cell": name, **cells[name]}), file=sys.stderr, flush=True)
    head = cells.get("128x1") or next(iter(cells.values()))
    cpu = None if args.no_cpu else cpu_baseline()
    line = {
        "metric": "median GPU µs/call, 128 req T0.6 k20 p0.95 + 64×4 verify; % of HBM peak",
        "value": round(head["median_us"], 3),
        "unit": "µs/call",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["median_us"] / 1000.0, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32 logits; fp32 screens, fp64 decisions",
        "data": "synthetic",
        "config": {"workload": "128 requests x 1 row, V=151936 fp32, T=0.6 top-k 20 top-p 0.95 (half the rows on "
                               "the bf16 grid); second cell 64 requests x (4 one-hot drafts + bonus), ratio mode",
                   "vocab": VOCAB, "cells": {k: {kk: (round(vv, 3) if isinstance(vv, float) else vv)
                                                 for kk, vv in v.items()} for k, v in cells.items()}},
        "roofline": {"bound": "hbm", "achieved": round(head["achieved_gbs"], 1), "peak": HBM_PEAK / 1e9,
                     "unit": "GB/s", "frac": round(head["frac"], 4), "traffic": None},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
