"""Allocation-free device calls with explicit workspace ownership (PyTorch-ROCm).

The same API as the reference's python/exactsample/cuda.py:15-198: ``plan``
makes a ``CudaPlan`` (workspace, lock, completion event) once; ``verify``
enqueues one call of the gfx950 kernels on the current HIP stream through the
``torch.ops.exactsample.verify_out`` op, which validates the tensors and calls
the C ABI (include/exactsample_amd.h). Under PyTorch-ROCm the ``torch.cuda``
namespace drives HIP devices and streams, so names are kept.

Nothing here computes a result: without the built library every call raises.
"""
from __future__ import annotations

import ctypes
import os
import threading
from dataclasses import dataclass
from pathlib import Path
from typing import Any

_HERE = Path(__file__).resolve().parent
_OPS_NAME = "_exactsample_ops.so"
_LIB_NAME = "libexactsample_amd.so"
_clib = None


@dataclass(frozen=True)
class CudaRequestParams:
    temperature: Any  # device float64 [R]
    top_k: Any        # device int64 [R], 0 disables
    top_p: Any        # device float64 [R]
    min_p: Any        # device float64 [R]
    draft_kind: Any   # device int64 [R], 0 one-hot, 1 full


@dataclass(frozen=True)
class CudaRngKey:
    seed: Any       # device int64 [R]: the uint64 key bits in signed storage
    stream_id: Any  # device int64 [R], in [0, 2**32)
    positions: Any  # device int64 [rows], in [0, 2**32)


@dataclass
class CudaOutput:
    tokens: Any
    accepted_len: Any
    status: Any
    path_used: Any
    num_requests: int = 0


def c_library():
    """The C-ABI library (for sizes and offsets); raises if it was not built."""
    global _clib
    if _clib is None:
        path = _HERE / _LIB_NAME
        if not path.is_file():
            raise RuntimeError(f"exactsample library (libexactsample_amd.so) is missing: {path}. Build it with "
                               "`python -m exactsample.build`.")
        lib = ctypes.CDLL(str(path))
        lib.es_workspace_size.restype = ctypes.c_size_t
        lib.es_workspace_size.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int32]
        lib.es_fallback_counter_offset.restype = ctypes.c_size_t
        lib.es_fallback_counter_offset.argtypes = []
        _clib = lib
    return _clib


def load_library(path: str | os.PathLike[str] | None = None) -> None:
    """Registers the exactsample::verify_out op from the built shared object (no JIT build).

    EXACTSAMPLE_LIBRARY names another build; otherwise the one beside this file.
    """
    import torch

    if hasattr(torch.ops.exactsample, "verify_out"):
        return
    requested = path or os.environ.get("EXACTSAMPLE_LIBRARY")
    library = Path(requested) if requested else _HERE / _OPS_NAME
    if not library.is_file():
        raise RuntimeError(f"exactsample op library is missing: {library}. Build it with "
                           "`python -m exactsample.build`, or set EXACTSAMPLE_LIBRARY.")
    torch.ops.load_library(str(library.resolve()))


_PLAN_DIMENSIONS = ("max_rows", "max_requests", "max_draft", "vocab")


def _plan_dimension(name: str, value: Any) -> int:
    """A plan size: a plain int, at least 1 for the vocabulary and 0 otherwise, below 2**31."""
    smallest = 1 if name == "vocab" else 0
    is_integer = isinstance(value, int) and not isinstance(value, bool)
    if not is_integer or value < smallest:
        raise ValueError(f"{name} must be a nonnegative integer (vocab must be positive)")
    if value >= 2**31:
        raise ValueError(f"{name} exceeds kernel int32 indexing")
    return value


class CudaPlan:
    """A workspace for one call at a time. Calls on one stream queue safely;
    a call on another stream while one is in flight is refused.

    Inputs and outputs must stay unchanged until ``synchronize`` or stream
    order establishes completion. Graph capture is not supported.

    State: ``workspace`` (zeroed once: the kernels' arrival counters start at
    zero and every call leaves them at zero), a non-blocking lock that admits
    one host call at a time, the stream of the last call and an event recorded
    after it (which answers "is the last call still running?").
    """

    def __init__(self, max_rows: int, max_requests: int, max_draft: int, vocab: int,
                 *, device: Any = "cuda", caps: dict | None = None, reference: bool = False):
        import torch

        if caps:
            raise ValueError("caps is reserved; v1 supports the default capabilities only")
        sizes = dict(zip(_PLAN_DIMENSIONS, (max_rows, max_requests, max_draft, vocab)))
        for name, value in sizes.items():
            _plan_dimension(name, value)
        where = torch.device(device)
        if where.type != "cuda":
            raise ValueError("CudaPlan requires a CUDA device")
        index = torch.cuda.current_device() if where.index is None else where.index
        self.device = torch.device("cuda", index)
        self.max_rows, self.max_requests, self.max_draft, self.vocab = (sizes[k] for k in _PLAN_DIMENSIONS)
        # Kept sets of at most this many tokens are finished as an FP64 list;
        # 0 sends every filtered row to the full-row path (tests use both).
        self.list_max = 256
        self.reference = reference
        lib = c_library()
        self.workspace_bytes = int(lib.es_workspace_size(max_rows, vocab, int(bool(reference))))
        if self.workspace_bytes == 0:
            raise ValueError("workspace size overflow")
        self.workspace = torch.zeros(self.workspace_bytes, dtype=torch.uint8, device=self.device)
        self._fallback_offset = int(lib.es_fallback_counter_offset())
        self._lock = threading.Lock()
        self._done = torch.cuda.Event(enable_timing=False)
        self._last_stream = None
        self._held = ()
        # The event's first record creates it: do that here, not on the first call.
        self._done.record(torch.cuda.current_stream(self.device))
        self._done.synchronize()

    def allocate_output(self) -> CudaOutput:
        import torch

        def per_request(*shape, dtype):
            return torch.empty(shape, device=self.device, dtype=dtype)

        n = self.max_requests
        return CudaOutput(per_request(n, self.max_draft + 1, dtype=torch.int64), per_request(n, dtype=torch.int32),
                          per_request(n, dtype=torch.int32), per_request(n, dtype=torch.int32))

    def fallbacks(self) -> int:
        """FP64 recomputations the last call needed (synchronizes)."""
        import torch

        self.synchronize()
        word = self.workspace.narrow(0, self._fallback_offset, 4)
        return int(word.view(torch.int32).item())

    def synchronize(self) -> None:
        """Waits for this plan's last call; the workspace may then be used on any stream."""
        with self._lock:
            self._done.synchronize()
            self._release()

    # -- used by verify -------------------------------------------------
    def _claim(self, stream) -> None:
        """Refuses a call on another stream while the last call may still run."""
        if self._last_stream in (None, stream.cuda_stream):
            return
        if not self._done.query():
            raise RuntimeError("exactsample workspace is in flight on another stream; "
                               "synchronize or use a separate plan")

    def _enqueued(self, stream, tensors) -> None:
        """After a launch (or a failed one: work may be partly enqueued), keeps
        every tensor alive on `stream` and marks the plan busy there."""
        for t in tensors:
            if t is not None and t.device == self.device:
                t.record_stream(stream)
        self._held = tensors
        self._last_stream = stream.cuda_stream
        self._done.record(stream)

    def _release(self) -> None:
        self._held = ()
        self._last_stream = None


def plan(max_rows: int, max_requests: int, max_draft: int, vocab: int,
         caps: dict | None = None, *, device: Any = "cuda", reference: bool = False) -> CudaPlan:
    return CudaPlan(max_rows, max_requests, max_draft, vocab, device=device, caps=caps, reference=reference)


_MODES = {"ratio": 0, "coupled": 1}
_DISPATCH = {"auto": 0, "reference": 1, "fused": 2}


def _check_call(target_logits, cu_rows, params, rng, plan, mode, dispatch) -> int:
    """Host-side checks that need no device data; returns the request count."""
    if mode not in _MODES or dispatch not in _DISPATCH:
        raise ValueError("mode must be ratio/coupled; dispatch must be auto/reference/fused")
    if dispatch == "reference" and not plan.reference:
        raise ValueError("dispatch='reference' needs a plan made with reference=True")
    if not (isinstance(params, CudaRequestParams) and isinstance(rng, CudaRngKey)):
        raise TypeError("CUDA verify requires CudaRequestParams and CudaRngKey containing device tensors")
    if target_logits.ndim != 2 or cu_rows.ndim != 1 or cu_rows.numel() < 1:
        raise ValueError("target_logits must be 2D and cu_rows a nonempty 1D tensor")
    requests = cu_rows.numel() - 1
    rows, vocab = target_logits.shape
    if rows > plan.max_rows or requests > plan.max_requests or vocab != plan.vocab:
        raise ValueError("input exceeds plan capacity or has a different vocabulary")
    if target_logits.device != plan.device:
        raise ValueError("input and plan must be on the same CUDA device")
    return requests


def verify(target_logits, cu_rows, draft_ids, *, params: CudaRequestParams,
           rng: CudaRngKey, plan: CudaPlan, out: CudaOutput,
           draft_logits=None, mask=None, mode: str = "ratio", dispatch: str = "auto",
           top_k_top_p: bool = True) -> CudaOutput:
    """Verifies ragged proposals into existing buffers and returns ``out``.

    Every input is a device tensor already. ``draft_logits`` are log weights of
    the proposal distribution actually used (after its own filters); target
    filters never apply to q and bonus q rows are ignored. Only the first
    ``out.num_requests`` output rows belong to the call. Invalid values give a
    per-request status, asynchronously.

    ``top_k_top_p=False`` promises that no request has a top-k below the
    vocabulary or a top-p below 1; it only skips list work and never changes
    a result (a request that does filter takes the full-row path).
    """
    import torch

    requests = _check_call(target_logits, cu_rows, params, rng, plan, mode, dispatch)
    load_library()
    op_args = (target_logits, cu_rows, draft_ids, draft_logits, params.temperature, params.top_k,
               params.top_p, params.min_p, params.draft_kind, rng.seed, rng.stream_id, rng.positions,
               mask, plan.workspace, out.tokens, out.accepted_len, out.status, out.path_used)
    with torch.cuda.device(plan.device):
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("exactsample v1 does not support CUDA graph capture")
        stream = torch.cuda.current_stream(plan.device)
        if not plan._lock.acquire(blocking=False):
            raise RuntimeError("exactsample workspace is already in use by another host call")
        try:
            plan._claim(stream)
            present = [t for t in op_args if t is not None]
            if not all(isinstance(t, torch.Tensor) for t in present):
                raise TypeError("all CUDA arguments must be preallocated tensors")
            if any(t.requires_grad for t in present):
                raise ValueError("exactsample is an inference operator and does not support autograd")
            try:
                torch.ops.exactsample.verify_out(*op_args, _MODES[mode], _DISPATCH[dispatch], plan.max_draft,
                                                 plan.list_max if top_k_top_p else 0)
            finally:
                plan._enqueued(stream, op_args)
            out.num_requests = requests
        finally:
            plan._lock.release()
    return out
