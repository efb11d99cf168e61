"""Writes tests/golden/config5_outputs.npz: the FP64 oracle's outputs for the
full ragged verification configuration (256 requests, draft lengths U{0..7},
about 1,150 rows of V = 151,936, a mask allowing 10% of each row, mixed
filters, permuted slots), for its three variants, with the sha256 of every
input array so a change of generator is caught before outputs are compared.

    python tests/golden/make_config5_golden.py

The inputs come from bench.config5 (seed 5); the oracle is oracle.verify_reference.
"""
import hashlib
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
from oracle import RequestParams, RngKey, verify_reference  # noqa: E402

OUT = os.path.join(HERE, "config5_outputs.npz")
VARIANTS = ("full_ratio", "one_hot_coupled", "full_coupled")
REQUESTS = 256


def digest(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def input_digests(work):
    """sha256 of every input of a config-5 batch (params by value)."""
    keys = work["keys"]
    out = dict(rows=digest(work["rows"]), offsets=digest(work["offsets"]), ids=digest(work["ids"]),
               mask=digest(bench.packed_mask(work["allowed"])), seed=digest(keys["seed"]),
               stream=digest(keys["stream"]), positions=digest(keys["positions"]))
    if work["draft_logits"] is not None:
        out["draft_logits"] = digest(work["draft_logits"])
    return out


def oracle_outputs(work):
    keys = work["keys"]
    rng = RngKey([int(s) for s in keys["seed"]], [int(s) for s in keys["stream"]], keys["positions"])
    q = work["draft_logits"]
    return verify_reference(work["rows"].astype(np.float64), work["offsets"], work["ids"],
                            params=RequestParams(**work["params"]), rng=rng, mask=bench.packed_mask(work["allowed"]),
                            draft_logits=None if q is None else q.astype(np.float64), mode=work["mode"])


def main():
    arrays = {}
    for variant in VARIANTS:
        t0 = time.time()
        work = bench.config5(requests=REQUESTS, variant=variant)
        out = oracle_outputs(work)
        for name, value in input_digests(work).items():
            arrays[f"{variant}/sha256/{name}"] = np.array(value)
        arrays[f"{variant}/tokens"] = np.asarray(out.tokens)
        arrays[f"{variant}/accepted_len"] = np.asarray(out.accepted_len)
        arrays[f"{variant}/status"] = np.asarray(out.status)
        print(variant, f"{work['rows'].shape[0]} rows", f"{time.time() - t0:.1f} s",
              "statuses", np.bincount(np.asarray(out.status), minlength=4).tolist(), flush=True)
        del work, out
    np.savez_compressed(OUT, **arrays)
    print(OUT)


if __name__ == "__main__":
    main()
