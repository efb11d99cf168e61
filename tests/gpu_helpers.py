"""Device-side setup for GPU parity tests (allocation stays outside ``verify``).

Mirrors the reference's tests/cuda_helpers.py:6-46: the same inputs become
device tensors of a chosen dtype (optionally with every last dimension
strided by two), a plan sized for them and its output buffers. ``compare``
then checks tokens, accepted lengths and statuses against the oracle run on
exactly the values the device saw (after rounding to the dtype).
"""
import numpy as np

from oracle import RequestParams, RngKey, verify_reference


def packed_mask(allowed):
    """Pack a boolean [rows, V] array into int32 words, bit t % 32 of word t // 32."""
    rows, vocab = allowed.shape
    bits = np.zeros((rows, (vocab + 31) // 32 * 32), np.uint64)
    bits[:, :vocab] = allowed
    words = (bits.reshape(rows, -1, 32) << np.arange(32, dtype=np.uint64)).sum(-1)
    return words.astype(np.uint32).view(np.int32)


def prepared(logits, cu_rows, draft_ids, *, params=None, rng=None, mask=None, draft_logits=None,
             dtype=None, strided=False, reference=False):
    import torch
    from exactsample_amd.cuda import CudaRequestParams, CudaRngKey, plan

    params = params or RequestParams()
    data = np.asarray(logits)
    offsets = np.asarray(cu_rows)
    ids = np.asarray(draft_ids, dtype=np.int64)
    rows, vocab = data.shape
    requests = len(offsets) - 1
    rng = rng or RngKey(1234, 3, np.arange(rows))
    dtype = dtype or torch.float64

    def tensor(value, kind):
        result = torch.as_tensor(np.array(value, copy=True), dtype=kind, device="cuda")
        if strided and result.ndim and result.shape[-1]:
            backing = torch.empty((*result.shape[:-1], result.shape[-1] * 2), dtype=kind, device="cuda")
            backing[..., ::2] = result
            result = backing[..., ::2]
        return result

    def per(value):
        array = np.asarray(value, dtype=object)
        return [array.item()] * requests if array.ndim == 0 else list(array)

    seeds = [int(s) if int(s) < 2**63 else int(s) - 2**64 for s in per(rng.seed)]
    gpu_params = CudaRequestParams(
        tensor(per(params.temperature), torch.float64), tensor(per(params.top_k), torch.int64),
        tensor(per(params.top_p), torch.float64), tensor(per(params.min_p), torch.float64),
        tensor([0 if k == "one_hot" else 1 for k in per(params.draft_kind)], torch.int64))
    gpu_rng = CudaRngKey(tensor(seeds, torch.int64), tensor(per(rng.stream_id), torch.int64),
                         tensor(rng.positions, torch.int64))
    work = plan(rows, requests, ids.shape[1], vocab, reference=reference)
    args = dict(target_logits=tensor(data, dtype), cu_rows=tensor(offsets, torch.int64),
                draft_ids=tensor(ids, torch.int64), params=gpu_params, rng=gpu_rng,
                plan=work, out=work.allocate_output())
    if mask is not None:
        args["mask"] = tensor(mask, torch.int32)
    if draft_logits is not None:
        args["draft_logits"] = tensor(draft_logits, dtype)
    return args


def expected_for(args, offsets, ids, *, params=None, rng=None, mask=None, mode="ratio"):
    """The oracle on the values the device received."""
    host_rows = args["target_logits"].double().cpu().numpy()
    q = args.get("draft_logits")
    q = None if q is None else q.double().cpu().numpy()
    return verify_reference(host_rows, offsets, ids, params=params, rng=rng, mask=mask, draft_logits=q, mode=mode)


def run_and_compare(logits, offsets, ids, *, params=None, rng=None, mask=None, draft_logits=None, mode="ratio",
                    dispatch="fused", dtype=None, strided=False, list_max=256, top_k_top_p=True):
    """Runs one call, checks it against the oracle and returns (out, fallbacks, args)."""
    from exactsample_amd.cuda import verify

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

    route: 1 failed, 2 greedy, 3 top-k list, 4 top-p list, 5 full-row path.
    """
    import struct
    plan.synchronize()
    data = plan.workspace.cpu().numpy().tobytes()
    out = []
    for r in range(rows):
        base = 8 + r * 12320 + 32  # the row's state follows its 32-byte result
        _, _, _, _, _, _, _, fallbacks, route, _ = struct.unpack_from("<ddiiiiiiii", data, base)
        out.append((route, fallbacks))
    return out
