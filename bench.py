"""Benchmark of exactsample's verify (the gfx950 build) on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--cells 128x1,64x5,...] [--no-cpu]

A "step" is one ``verify`` call over one batch of synthetic logits already
resident in HBM. The headline workload (value) is 128 requests x 1 row of
V = 151,936 fp32 logits at T=0.6, top-k 20, top-p 0.95; the second cell is 64
requests x (4 one-hot drafts + bonus) verified in ratio mode with the same
settings. By default the same two batches are also timed as bfloat16 logits
(the dtype of the reference's own benchmark), both shapes at the reference
benchmark's other two settings (T = 1.0, and T = 0.7 top-p 0.9), and the other
configurations: 8 rows at T = 1; the flatness rows (sigma ~ U(0.5, 4)) at
T = 0.7 with top-p 0.9 or min-p 0.05, in batches of 128 and 1; and the ragged
256-request verification batch with masks and full proposals.
Rows come from the peaked generator: base N(mu, sigma^2) with
mu ~ U(-5, 0), sigma ~ U(2, 4); one token + U(6, 14); 15 tokens + U(0, 8);
every even row of the two headline shapes rounded to the bf16 grid (values
stay fp32).

Reported per cell, with every timed call queued behind a spin kernel so that
calls run back to back and events hold GPU time only: the median and mean time
per call through the C ABI (the value), the same through the torch op (which
also records the plan's completion event), the slice-stream kernel (es_main)
and the per-row finishing kernel (es_finish) timed apart by an event the
library records between them, and cold medians after a 2 GiB read that evicts
the 256 MB Infinity Cache. The roofline is the headline call's, cold:
algorithmic bytes (one read of every logit row, plus parameters and outputs,
< 0.1%) over the cold call's median time; warm call and es_main fractions are
reported beside it. ``traffic`` is es_main's HBM bytes per launch from the
committed FETCH_SIZE / WRITE_SIZE counter summary. A plain copy kernel of the
headline logits' size is timed first (the stream-copy rate measured on the
device, and the counters' calibration). ``cpu_baseline`` times the FP64 oracle
(oracle/, the reference algorithm with its per-token scalar Philox) on a
bounded sample of the headline rows, single threaded, and names the host CPU.
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


def _keys(rng, seed, requests, rows):
    return dict(seed=seed + np.arange(requests, dtype=np.int64), stream=np.arange(requests, dtype=np.int64),
                positions=rng.integers(0, 4096, size=rows).astype(np.int64))


def config1(seed=1, requests=8):
    """8 requests, one row each, temperature 1.0 and no other filter."""
    rng = np.random.default_rng(seed)
    rows = peaked_rows(rng, requests)
    return dict(rows=rows, offsets=np.arange(requests + 1, dtype=np.int64),
                ids=np.full((requests, 1), -1, dtype=np.int64), keys=_keys(rng, seed, requests, requests),
                params=dict(temperature=1.0, top_k=0, top_p=1.0, min_p=0.0), mode="ratio")


def config3(seed=3, requests=128, filt="top_p"):
    """Rows of flatness sigma ~ U(0.5, 4) at T=0.7 with top-p 0.9 (or min-p 0.05).

    Every tenth row is built so that FP32 cannot settle the threshold: for
    top-p, ten tokens at logit 0 and the rest at or below -100, so the target
    0.9 * 10 equals a prefix sum exactly; for min-p, one token whose weight is
    within a relative 1e-9 of 0.05 (above on even rows, below on odd ones).
    """
    rng = np.random.default_rng(seed)
    rows = peaked_rows(rng, requests, sigma=(0.5, 4.0))
    for r in range(0, requests, 10):
        if filt == "top_p":
            row = np.full(VOCAB, -100.0, np.float32) - rng.uniform(0, 20, VOCAB).astype(np.float32)
            row[rng.choice(VOCAB, 10, replace=False)] = 0.0
        else:
            row = rows[r] - rows[r].max()
            side = 1 + (1e-9 if (r // 10) % 2 == 0 else -1e-9)
            row[int(rng.integers(VOCAB))] = np.float32(0.7 * np.log(0.05 * side))
            row[int(rng.integers(VOCAB))] = 0.0
        rows[r] = row
    params = dict(temperature=0.7, top_k=0, top_p=0.9 if filt == "top_p" else 1.0,
                  min_p=0.05 if filt == "min_p" else 0.0)
    return dict(rows=rows, offsets=np.arange(requests + 1, dtype=np.int64),
                ids=np.full((requests, 1), -1, dtype=np.int64), keys=_keys(rng, seed, requests, requests),
                params=params, mode="ratio")


def config3_single(seed=3, filt="top_p", row=1):
    """Batch 1 of the flatness configuration: row `row` of its 128-row batch
    alone (rows 0, 10, 20, ... are the constructed ones), with that row's key."""
    work = config3(seed=seed, requests=128, filt=filt)
    keys = work["keys"]
    return dict(rows=work["rows"][row:row + 1].copy(), offsets=np.array([0, 1], dtype=np.int64),
                ids=np.full((1, 1), -1, dtype=np.int64), params=work["params"], mode="ratio",
                keys=dict(seed=keys["seed"][row:row + 1], stream=keys["stream"][row:row + 1],
                          positions=keys["positions"][row:row + 1]))


def config5(seed=5, requests=256, variant="full_ratio"):
    """Ragged verification: draft lengths ~ U{0..7}, a mask allowing a random
    10% of each row, filters by request {temperature only, top-k 4096, top-p
    0.99, min-p 0.02} at T=1, and requests in a permuted slot order.

    variant "full_ratio": full proposals q = log softmax(target + N(0, 1)) in
    fp32, drafts drawn from q, ratio mode; "one_hot_coupled": the same drafts
    as one-hot in coupled mode; "full_coupled": the literal combination, which
    the contract makes INVALID_INPUT for every request with drafts.
    """
    rng = np.random.default_rng(seed)
    drafts = rng.integers(0, 8, size=requests)
    order = rng.permutation(requests)
    drafts = drafts[order]
    offsets = np.concatenate([[0], np.cumsum(drafts + 1)]).astype(np.int64)
    n = int(offsets[-1])
    rows = peaked_rows(rng, n)
    noisy = rows + rng.standard_normal(rows.shape).astype(np.float32)
    q = (noisy - noisy.max(axis=1, keepdims=True)).astype(np.float32)
    q = (q - np.log(np.exp(q.astype(np.float64)).sum(axis=1, keepdims=True))).astype(np.float32)
    ids = np.full((requests, 7), -1, dtype=np.int64)
    for r in range(requests):
        for d in range(int(drafts[r])):
            g = -np.log(-np.log(rng.random(VOCAB)))
            ids[r, d] = int(np.argmax(q[offsets[r] + d] + g))
    allowed = rng.random((n, VOCAB)) < 0.1
    kinds = order % 4
    params = dict(temperature=[1.0] * requests,
                  top_k=[4096 if k == 1 else 0 for k in kinds],
                  top_p=[0.99 if k == 2 else 1.0 for k in kinds],
                  min_p=[0.02 if k == 3 else 0.0 for k in kinds],
                  draft_kind=["one_hot" if variant == "one_hot_coupled" else "full"] * requests)
    return dict(rows=rows, offsets=offsets, ids=ids, keys=_keys(rng, seed, requests, n), params=params,
                mode="ratio" if variant == "full_ratio" else "coupled", allowed=allowed,
                draft_logits=None if variant == "one_hot_coupled" else q)


def as_bf16(work):
    """The same rows handed over as bfloat16 (the reference's own benchmark dtype)."""
    work["rows"] = round_to_bf16(work["rows"])
    work["dtype"] = "bfloat16"
    return work


def with_params(work, **params):
    work["params"] = dict(QWEN, **params)
    return work


# The value is the first cell; the others are reported beside it. The bf16
# and other-settings cells follow the reference's own benchmark table
# (128 x 1 and 64 x 5 at the Qwen settings, T = 1.0, and T = 0.7 top-p 0.9).
CELLS = {
    "128x1": config2,
    "64x5": config4,
    "128x1_bf16": lambda: as_bf16(config2()),
    "64x5_bf16": lambda: as_bf16(config4()),
    "128x1_T1": lambda: with_params(config2(), temperature=1.0, top_k=0, top_p=1.0),
    "64x5_T1": lambda: with_params(config4(), temperature=1.0, top_k=0, top_p=1.0),
    "128x1_T0.7_p0.9": lambda: with_params(config2(), temperature=0.7, top_k=0, top_p=0.9),
    "64x5_T0.7_p0.9": lambda: with_params(config4(), temperature=0.7, top_k=0, top_p=0.9),
    # The other configurations: 8 rows at T = 1; the flatness rows (sigma ~
    # U(0.5, 4), T = 0.7) with top-p 0.9 or min-p 0.05 in batches of 128 and
    # 1 (row 1 of the 128-row batch: rows 0, 10, 20, ... are the constructed
    # ones); the full ragged verification batch with full proposals.
    "cfg1_8x1_T1": config1,
    "cfg3_128_p0.9": lambda: config3(filt="top_p"),
    "cfg3_128_minp0.05": lambda: config3(filt="min_p"),
    "cfg3_1_p0.9": lambda: config3_single(filt="top_p"),
    "cfg3_1_minp0.05": lambda: config3_single(filt="min_p"),
    "cfg5_256_full_ratio": lambda: config5(variant="full_ratio"),
}
DEFAULT_CELLS = ",".join(CELLS)


def packed_mask(allowed):
    """A boolean [rows, V] array as int32 words: bit t % 32 of word t // 32."""
    rows, vocab = allowed.shape
    padded = np.zeros((rows, -(-vocab // 32) * 32), dtype=bool)
    padded[:, :vocab] = allowed
    return np.packbits(padded.reshape(rows, -1, 32), axis=-1, bitorder="little").view("<u4").reshape(
        rows, -1).view(np.int32)


def device_args(work, device="cuda"):
    import torch
    from exactsample.cuda import CudaRequestParams, CudaRngKey, plan

    requests = len(work["offsets"]) - 1
    p = work["params"]

    def per_request(value, dtype):
        if np.ndim(value) == 0:
            return torch.full((requests,), value, dtype=dtype, device=device)
        return torch.as_tensor(np.asarray(value), dtype=dtype, device=device)

    kinds = p.get("draft_kind", "one_hot")
    kinds = [kinds] * requests if isinstance(kinds, str) else list(kinds)
    params = CudaRequestParams(per_request(p["temperature"], torch.float64), per_request(p["top_k"], torch.int64),
                               per_request(p["top_p"], torch.float64), per_request(p["min_p"], torch.float64),
                               per_request([0 if k == "one_hot" else 1 for k in kinds], torch.int64))
    rng = CudaRngKey(torch.as_tensor(work["keys"]["seed"], device=device),
                     torch.as_tensor(work["keys"]["stream"], device=device),
                     torch.as_tensor(work["keys"]["positions"], device=device))
    logits = torch.as_tensor(work["rows"], device=device).to(getattr(torch, work.get("dtype", "float32")))
    w = plan(logits.shape[0], requests, work["ids"].shape[1], logits.shape[1])
    args = dict(target_logits=logits, cu_rows=torch.as_tensor(work["offsets"], device=device),
                draft_ids=torch.as_tensor(work["ids"], device=device), params=params, rng=rng, plan=w,
                out=w.allocate_output())
    if work.get("allowed") is not None:
        args["mask"] = torch.as_tensor(packed_mask(work["allowed"]), device=device)
    if work.get("draft_logits") is not None:
        args["draft_logits"] = torch.as_tensor(work["draft_logits"], device=device)
    return args


def algorithmic_bytes(work):
    """One read of every logit row (and proposal row and mask word) plus
    parameters and outputs."""
    rows, vocab = work["rows"].shape
    elem = 2 if work.get("dtype") == "bfloat16" else 4
    requests = len(work["offsets"]) - 1
    k1 = work["ids"].shape[1] + 1
    params = requests * (5 * 8 + 2 * 8) + rows * 8 + (requests + 1) * 8 + work["ids"].size * 8
    outputs = requests * (k1 * 8 + 3 * 4)
    logits = rows * vocab * elem
    if work.get("draft_logits") is not None:
        logits += work["draft_logits"].size * elem
    if work.get("allowed") is not None:
        logits += rows * (-(-vocab // 32)) * 4
    return logits + params + outputs


class Events:
    """HIP timing events created with hipEventDisableSystemFence.

    An event that ends in a system-scope fence (torch.cuda.Event's) costs
    about 3.7 us of GPU time between back-to-back calls; without the fence the
    marker costs little and times the work it brackets more closely (the
    flag's documented use). Driven through the HIP runtime that torch loaded.
    """
    DISABLE_SYSTEM_FENCE = 0x20000000

    def __init__(self):
        import ctypes
        self._ct = ctypes
        self.hip = ctypes.CDLL("libamdhip64.so.7")
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.made = []

    def create(self, n):
        out = []
        for _ in range(n):
            e = self._ct.c_void_p()
            if self.hip.hipEventCreateWithFlags(self._ct.byref(e), self._ct.c_uint(self.DISABLE_SYSTEM_FENCE)):
                raise RuntimeError("hipEventCreateWithFlags failed")
            out.append(e.value)
        self.made += out
        return out

    def record(self, event, stream):
        if self.hip.hipEventRecord(event, stream.cuda_stream):
            raise RuntimeError("hipEventRecord failed")

    def us(self, a, b):
        ms = self._ct.c_float()
        self.hip.hipEventSynchronize(b)
        if self.hip.hipEventElapsedTime(self._ct.byref(ms), a, b):
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value * 1000.0

    def destroy(self):
        for e in self.made:
            self.hip.hipEventDestroy(e)
        self.made = []


_SPIN_RATE = []


def queue_ahead(us):
    """Enqueues a spin kernel of about `us` microseconds on the current stream.

    The calls enqueued behind it then run back to back, so the events around
    each call hold GPU time only, never the host's launch time. Callers ask
    for about 120 us per queued call."""
    import torch
    if not _SPIN_RATE:
        torch.cuda._sleep(1000)  # the first launch also loads the kernel: keep it out of the calibration
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        torch.cuda._sleep(4_000_000)
        b.record()
        b.synchronize()
        _SPIN_RATE.append(4_000_000 / (a.elapsed_time(b) * 1000.0))  # spin cycles per microsecond
    torch.cuda._sleep(int(_SPIN_RATE[0] * us))


def time_cell(name, steps, warmup):
    """Per-call GPU time of one cell, the two kernels timed apart, and cold calls.

    Every timed call is queued behind a spin kernel, so calls run back to back.
    - value: the C ABI (es_launch) with an event before and after each call;
    - op: the same through exactsample.cuda.verify (the torch op; it also
      records the plan's completion event each call, which costs GPU time);
    - split: es_launch with a third event recorded by the library between the
      slice-stream kernel (es_main) and the per-row finishing kernel
      (es_finish), via es_set_split_event: the dominant kernel's duration for
      the roofline;
    - cold: split calls, each after a 2 GiB read that evicts the 256 MB
      Infinity Cache.
    """
    import torch
    from exactsample import capi
    from exactsample.cuda import verify

    work = CELLS[name]()
    args = device_args(work)
    stream = torch.cuda.current_stream()
    lib = capi.load()
    p, r, o = args["params"], args["rng"], args["out"]
    abi = capi.from_tensors(args["target_logits"], args["cu_rows"], args["draft_ids"], args.get("draft_logits"),
                            p.temperature, p.top_k, p.top_p, p.min_p, p.draft_kind, r.seed, r.stream_id,
                            r.positions, args.get("mask"), args["plan"].workspace, o.tokens, o.accepted_len,
                            o.status, o.path_used, mode=0 if work["mode"] == "ratio" else 1,
                            max_draft=args["plan"].max_draft)
    requests = len(work["offsets"]) - 1
    ev = Events()

    def op():
        verify(**args, mode=work["mode"], top_k_top_p=True)

    def launch():
        capi.launch(lib, abi, stream)

    for _ in range(warmup):
        op()
    op_tokens = o.tokens[:requests].clone()
    for _ in range(warmup):
        launch()
    torch.cuda.synchronize()
    if not torch.equal(op_tokens, o.tokens[:requests]):
        raise RuntimeError("the C ABI and the torch op disagree")

    def per_call(fn, n, mid=False, before=None):
        a, b = ev.create(n), ev.create(n)
        m = ev.create(n) if mid else None
        if before is None:
            queue_ahead(n * 120.0)
        t0 = time.perf_counter()
        try:
            for i in range(n):
                if before is not None:
                    before()
                if mid:
                    lib.es_set_split_event(m[i])
                ev.record(a[i], stream)
                fn()
                ev.record(b[i], stream)
                if before is not None:
                    ev.us(a[i], b[i])  # one cold call at a time
        finally:
            lib.es_set_split_event(None)
        host = (time.perf_counter() - t0) / n * 1e6
        torch.cuda.synchronize()
        if not mid:
            return np.array([ev.us(x, y) for x, y in zip(a, b)]), host
        return (np.array([ev.us(x, y) for x, y in zip(a, m)]), np.array([ev.us(x, y) for x, y in zip(m, b)]),
                host)

    calls, host_abi = per_call(launch, steps)
    op_calls, host_op = per_call(op, steps)
    main, finish, _ = per_call(launch, steps, mid=True)
    flush = torch.ones(512 << 20, dtype=torch.float32, device="cuda")
    cold_main, cold_finish, _ = per_call(launch, min(steps, 30), mid=True, before=flush.sum)
    cold = cold_main + cold_finish
    del flush
    ev.destroy()
    fallbacks = args["plan"].fallbacks()
    nbytes = algorithmic_bytes(work)
    med = float(np.median(calls))
    main_avg = float(main.mean())
    cold_med = float(np.median(cold))
    return dict(rows=int(work["rows"].shape[0]), requests=requests,
                median_us=med, mean_us=float(calls.mean()), p10_us=float(np.percentile(calls, 10)),
                p90_us=float(np.percentile(calls, 90)),
                op_median_us=float(np.median(op_calls)), op_mean_us=float(op_calls.mean()),
                host_us_per_call_abi=host_abi, host_us_per_call_op=host_op,
                es_main_avg_us=main_avg, es_main_median_us=float(np.median(main)),
                es_finish_avg_us=float(finish.mean()), es_finish_median_us=float(np.median(finish)),
                cold_median_us=cold_med, cold_es_main_median_us=float(np.median(cold_main)),
                bytes=int(nbytes), call_gbs=nbytes / (med * 1e-6) / 1e9,
                cold_call_gbs=nbytes / (cold_med * 1e-6) / 1e9,
                es_main_gbs=nbytes / (main_avg * 1e-6) / 1e9,
                cold_es_main_gbs=nbytes / (float(np.median(cold_main)) * 1e-6) / 1e9,
                fallbacks=int(fallbacks),
                accepted_mean=float(o.accepted_len[:requests].float().mean().item()))


def copy_rate(nbytes, launches=10):
    """A plain copy kernel (torch.neg) over a buffer of `nbytes`: event GB/s of
    read + write, and the calibration launches for the FETCH_SIZE / WRITE_SIZE
    counters (each launch reads and writes exactly `nbytes`)."""
    import torch
    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.neg(src, out=dst)
    torch.cuda.synchronize()
    ev = Events()
    a, b = ev.create(launches), ev.create(launches)
    stream = torch.cuda.current_stream()
    queue_ahead(launches * 120.0)
    for i in range(launches):
        ev.record(a[i], stream)
        torch.neg(src, out=dst)
        ev.record(b[i], stream)
    torch.cuda.synchronize()
    us = float(np.median([ev.us(x, y) for x, y in zip(a, b)]))
    ev.destroy()
    return dict(bytes_each_way=int(nbytes), median_us=us, gbs=2 * nbytes / (us * 1e-6) / 1e9)


def measured_traffic(path=os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                                       "es_main_128x1_traffic.md")):
    """HBM bytes per es_main launch from the committed FETCH_SIZE / WRITE_SIZE
    summary (line "traffic_bytes_per_launch: N"), or None."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        return None
    return None


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), or None."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_baseline(budget_s=12.0):
    """The FP64 oracle, single-threaded, over the headline rows (cycling through
    them) until the budget is spent; scaled to one 128-request call."""
    from oracle import RequestParams, RngKey, verify_reference

    work = config2()
    rows = work["rows"].astype(np.float64)
    done, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        r = done % len(rows)
        verify_reference(rows[r:r + 1], [0, 1], np.empty((1, 0), np.int64), params=RequestParams(**QWEN),
                         rng=RngKey(int(work["keys"]["seed"][r]), int(work["keys"]["stream"][r]),
                                    [int(work["keys"]["positions"][r])]),
                         vectorized_rng=False)
        done += 1
    elapsed = time.perf_counter() - t0
    per_row = elapsed / done
    return dict(value=per_row * 128 * 1e6, unit="us/call (128 requests, from the sample's time per row)",
                cores=1, kind="port", cpu_model=cpu_model(), host_nproc=os.cpu_count(),
                host_affinity=len(os.sched_getaffinity(0)),
                sample=f"{done} rows of the 128-row headline batch, cycled ({elapsed:.1f} s), through "
                       f"oracle.verify_reference with per-token scalar Philox: the FP64 restatement of "
                       f"reference.py, single threaded")


def main():
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--cells", default=DEFAULT_CELLS, help=f"comma-separated cells of {', '.join(CELLS)}")
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
    from exactsample.cuda import load_library
    load_library()
    copy = copy_rate(VOCAB * 4 * 128)
    print(json.dumps({"copy": copy}), file=sys.stderr, flush=True)
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
                   "vocab": VOCAB, "copy_kernel": {k: round(v, 3) if isinstance(v, float) else v
                                                  for k, v in copy.items()},
                   "cells": {k: {kk: (round(vv, 3) if isinstance(vv, float) else vv)
                                 for kk, vv in v.items()} for k, v in cells.items()}},
        "roofline": {"bound": "hbm",
                     "kernel": "the whole call (es_main + es_finish), 128x1 cell, cold: each call after a 2 GiB "
                               "read that evicts the 256 MB Infinity Cache, timed with HIP events on the call's stream",
                     "achieved": round(head["cold_call_gbs"], 1), "peak": HBM_PEAK / 1e9,
                     "unit": "GB/s", "frac": round(head["cold_call_gbs"] * 1e9 / HBM_PEAK, 4),
                     "traffic": measured_traffic(),
                     "traffic_kernel": "es_main (FETCH_SIZE + WRITE_SIZE per launch)",
                     "call_warm_frac": round(head["call_gbs"] * 1e9 / HBM_PEAK, 4),
                     "es_main_warm_frac": round(head["es_main_gbs"] * 1e9 / HBM_PEAK, 4),
                     "es_main_cold_frac": round(head["cold_es_main_gbs"] * 1e9 / HBM_PEAK, 4)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
