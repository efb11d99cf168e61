"""GPU-side plumbing of the parity tests.

``prepared`` turns one batch (NumPy logits, offsets, draft IDs, parameters,
RNG key, optional mask and proposal logits) into the keyword arguments of
``exactsample.cuda.verify``: device tensors in the chosen logits dtype,
optionally with a stride of two elements in every last dimension, a plan
sized for the batch and its output buffers. ``run_and_compare`` makes the
call and checks tokens, accepted lengths and statuses against the oracle run
on exactly the values the device received (after rounding to the dtype).
"""
import struct

import numpy as np

from oracle import RequestParams, RngKey, verify_reference


def packed_mask(allowed):
    """Boolean [rows, V] -> int32 words [rows, ceil(V / 32)], token t at bit t % 32 of word t // 32."""
    allowed = np.asarray(allowed, dtype=bool)
    rows, vocab = allowed.shape
    width = -(-vocab // 32) * 32
    bits = np.pad(allowed, ((0, 0), (0, width - vocab)))
    return np.packbits(bits.reshape(rows, -1, 32), axis=-1, bitorder="little").view("<i4").reshape(rows, -1)


def _on_device(value, dtype, strided):
    """A device tensor holding `value`; with `strided`, its last dimension has element stride 2."""
    import torch
    host = torch.as_tensor(np.array(value), dtype=dtype)
    if not strided or host.ndim == 0 or host.shape[-1] == 0:
        return host.to("cuda")
    pairs = torch.zeros((*host.shape, 2), dtype=dtype, device="cuda")
    view = pairs[..., 0]
    view.copy_(host)
    return view


def _per_request(value, requests):
    """A scalar or per-request parameter as a list of `requests` Python values."""
    array = np.asarray(value, dtype=object)
    return [array.item()] * requests if array.ndim == 0 else [v for v in array]


def prepared(logits, cu_rows, draft_ids, *, params=None, rng=None, mask=None, draft_logits=None,
             dtype=None, strided=False, reference=False):
    """The verify() keyword arguments for one batch (see the module docstring)."""
    import torch
    from exactsample.cuda import CudaRequestParams, CudaRngKey, plan

    params = params or RequestParams()
    logits = np.asarray(logits)
    offsets = np.asarray(cu_rows)
    ids = np.asarray(draft_ids, dtype=np.int64)
    rows, vocab = logits.shape
    requests = offsets.size - 1
    rng = rng or RngKey(1234, 3, np.arange(rows))
    dtype = dtype or torch.float64

    def dev(value, kind):
        return _on_device(value, kind, strided)

    seeds = np.array([int(s) % 2**64 for s in _per_request(rng.seed, requests)], dtype=np.uint64).view(np.int64)
    kinds = [int(k != "one_hot") for k in _per_request(params.draft_kind, requests)]
    device_params = CudaRequestParams(
        temperature=dev(_per_request(params.temperature, requests), torch.float64),
        top_k=dev(_per_request(params.top_k, requests), torch.int64),
        top_p=dev(_per_request(params.top_p, requests), torch.float64),
        min_p=dev(_per_request(params.min_p, requests), torch.float64),
        draft_kind=dev(kinds, torch.int64))
    device_rng = CudaRngKey(seed=dev(seeds, torch.int64),
                            stream_id=dev(_per_request(rng.stream_id, requests), torch.int64),
                            positions=dev(np.asarray(rng.positions, dtype=np.int64), torch.int64))
    work = plan(rows, requests, ids.shape[1], vocab, reference=reference)
    kwargs = dict(target_logits=dev(logits, dtype), cu_rows=dev(offsets, torch.int64),
                  draft_ids=dev(ids, torch.int64), params=device_params, rng=device_rng, plan=work,
                  out=work.allocate_output())
    if mask is not None:
        kwargs["mask"] = dev(mask, torch.int32)
    if draft_logits is not None:
        kwargs["draft_logits"] = dev(draft_logits, dtype)
    return kwargs


def expected_for(args, offsets, ids, *, params=None, rng=None, mask=None, mode="ratio"):
    """The oracle on the values the device received."""
    host_rows = args["target_logits"].double().cpu().numpy()
    q = args.get("draft_logits")
    q = None if q is None else q.double().cpu().numpy()
    return verify_reference(host_rows, offsets, ids, params=params, rng=rng, mask=mask, draft_logits=q, mode=mode)


def run_and_compare(logits, offsets, ids, *, params=None, rng=None, mask=None, draft_logits=None, mode="ratio",
                    dispatch="fused", dtype=None, strided=False, list_max=256, top_k_top_p=True):
    """Runs one call, checks it against the oracle and returns (out, fallbacks, args)."""
    from exactsample.cuda import verify

    rng = rng or RngKey(1234, 3, np.arange(len(logits)))
    args = prepared(logits, offsets, ids, params=params, rng=rng, mask=mask, draft_logits=draft_logits,
                    dtype=dtype, strided=strided, reference=dispatch == "reference")
    args["plan"].list_max = list_max
    out = verify(**args, mode=mode, dispatch=dispatch, top_k_top_p=top_k_top_p)
    fallbacks = args["plan"].fallbacks()
    expected = expected_for(args, offsets, ids, params=params, rng=rng, mask=mask, mode=mode)
    requests = len(offsets) - 1
    for field in ("tokens", "accepted_len", "status"):
        np.testing.assert_array_equal(getattr(out, field).cpu().numpy()[:requests], getattr(expected, field),
                                      err_msg=field)
    path = 0 if dispatch == "reference" else 1
    assert np.all(out.path_used.cpu().numpy()[:requests] == path)
    return out, fallbacks, args


def row_diagnostics(plan, rows):
    """(route, fallbacks) of each row of the plan's last call, read from the workspace.

    route: 1 failed, 2 greedy, 3 top-k list, 4 top-p list, 5 streaming draw,
    100 + reason: the full-row path.
    """
    plan.synchronize()
    data = plan.workspace.cpu().numpy().tobytes()
    out = []
    for r in range(rows):
        base = 8 + r * 12320 + 32  # the row's state follows its 32-byte result
        _, _, _, _, _, _, _, fallbacks, route, _ = struct.unpack_from("<ddiiiiiiii", data, base)
        out.append((route, fallbacks))
    return out
