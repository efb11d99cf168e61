"""ctypes binding of the C ABI (include/exactsample_amd.h), for callers without the torch op.

``Arguments`` mirrors ``es_arguments`` field for field; ``launch`` calls
``es_launch`` with raw device pointers and a HIP stream handle. It replaces
nothing in the reference (whose only binding is the torch op, csrc/bindings.cpp)
and performs none of the op's tensor checks: the caller owns the pointers and
strides. ``from_tensors`` fills the structure from PyTorch-ROCm tensors with the
same meaning as ``torch.ops.exactsample.verify_out``'s arguments.
"""
import ctypes
import os
from pathlib import Path

_HERE = Path(__file__).resolve().parent
DTYPES = {"float32": 0, "float64": 1, "float16": 2, "bfloat16": 3}


class Matrix(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("s0", ctypes.c_int64), ("s1", ctypes.c_int64),
                ("dtype", ctypes.c_int32), ("pad", ctypes.c_int32)]


class VecI64(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("stride", ctypes.c_int64)]


class VecF64(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("stride", ctypes.c_int64)]


class Arguments(ctypes.Structure):
    _fields_ = [
        ("target", Matrix), ("draft", Matrix),
        ("cu_rows", VecI64), ("top_k", VecI64), ("draft_kind", VecI64), ("seed", VecI64),
        ("stream", VecI64), ("position", VecI64),
        ("temperature", VecF64), ("top_p", VecF64), ("min_p", VecF64),
        ("draft_ids", ctypes.c_void_p), ("draft_s0", ctypes.c_int64), ("draft_s1", ctypes.c_int64),
        ("mask", ctypes.c_void_p), ("mask_s0", ctypes.c_int64), ("mask_s1", ctypes.c_int64),
        ("tokens", ctypes.c_void_p), ("token_s0", ctypes.c_int64), ("token_s1", ctypes.c_int64),
        ("accepted", ctypes.c_void_p), ("accepted_s", ctypes.c_int64),
        ("status", ctypes.c_void_p), ("status_s", ctypes.c_int64),
        ("path", ctypes.c_void_p), ("path_s", ctypes.c_int64),
        ("rows", ctypes.c_int64), ("requests", ctypes.c_int64), ("vocab", ctypes.c_int64),
        ("max_draft", ctypes.c_int64),
        ("mode", ctypes.c_int32), ("dispatch", ctypes.c_int32), ("list_max", ctypes.c_int32),
        ("pad", ctypes.c_int32),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_uint64),
    ]


EXPORTS = ["es_workspace_size", "es_launch", "es_launch_static", "es_error_string", "es_last_hip_error",
           "es_set_split_event", "es_check_gumbel", "es_check_weights", "es_fallback_counter_offset"]
STATIC_WORKSPACE_BYTES = 16 << 20  # ES_STATIC_WORKSPACE_BYTES


def load(path=None):
    """Opens libexactsample_amd.so (or `path`) and declares its signatures.

    A process must hold one HIP runtime. PyTorch-ROCm ships its own, which its
    libraries request by an unversioned name; loaded first, ours would bind the
    system runtime and torch would then load a second one. So torch, when
    installed, is imported first and the library binds the runtime torch loaded.
    """
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(str(path or os.environ.get("EXACTSAMPLE_CLIB") or _HERE / "libexactsample_amd.so"))
    lib.es_workspace_size.restype = ctypes.c_size_t
    lib.es_workspace_size.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int32]
    lib.es_launch.restype = ctypes.c_int32
    lib.es_launch.argtypes = [ctypes.POINTER(Arguments), ctypes.c_void_p]
    lib.es_launch_static.restype = ctypes.c_int32
    lib.es_launch_static.argtypes = [ctypes.POINTER(Arguments), ctypes.c_void_p]
    lib.es_error_string.restype = ctypes.c_char_p
    lib.es_error_string.argtypes = [ctypes.c_int32]
    lib.es_last_hip_error.restype = ctypes.c_char_p
    lib.es_last_hip_error.argtypes = []
    lib.es_check_gumbel.restype = ctypes.c_int32
    lib.es_check_gumbel.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_void_p]
    lib.es_check_weights.restype = ctypes.c_int32
    lib.es_check_weights.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_void_p]
    lib.es_set_split_event.restype = None
    lib.es_set_split_event.argtypes = [ctypes.c_void_p]
    lib.es_fallback_counter_offset.restype = ctypes.c_size_t
    lib.es_fallback_counter_offset.argtypes = []
    return lib


def from_tensors(target_logits, cu_rows, draft_ids, draft_logits, temperature, top_k, top_p, min_p, draft_kind,
                 seeds, stream_ids, positions, mask, workspace, tokens, accepted_len, status, path_used, *,
                 mode=0, dispatch=0, max_draft=None, list_max=256):
    """An Arguments structure over device tensors (the op's argument order)."""
    def matrix(t):
        if t is None:
            return Matrix(None, 0, 0, DTYPES[str(target_logits.dtype).replace("torch.", "")], 0)
        return Matrix(t.data_ptr(), t.stride(0), t.stride(1), DTYPES[str(t.dtype).replace("torch.", "")], 0)

    def vec(t, kind):
        return kind(t.data_ptr(), t.stride(0))

    a = Arguments()
    a.target, a.draft = matrix(target_logits), matrix(draft_logits)
    a.cu_rows, a.top_k, a.draft_kind = vec(cu_rows, VecI64), vec(top_k, VecI64), vec(draft_kind, VecI64)
    a.seed, a.stream, a.position = vec(seeds, VecI64), vec(stream_ids, VecI64), vec(positions, VecI64)
    a.temperature, a.top_p, a.min_p = vec(temperature, VecF64), vec(top_p, VecF64), vec(min_p, VecF64)
    a.draft_ids, a.draft_s0, a.draft_s1 = draft_ids.data_ptr(), draft_ids.stride(0), draft_ids.stride(1)
    if mask is not None:
        a.mask, a.mask_s0, a.mask_s1 = mask.data_ptr(), mask.stride(0), mask.stride(1)
    a.tokens, a.token_s0, a.token_s1 = tokens.data_ptr(), tokens.stride(0), tokens.stride(1)
    a.accepted, a.accepted_s = accepted_len.data_ptr(), accepted_len.stride(0)
    a.status, a.status_s = status.data_ptr(), status.stride(0)
    a.path, a.path_s = path_used.data_ptr(), path_used.stride(0)
    a.rows, a.vocab = target_logits.shape[0], target_logits.shape[1]
    a.requests = cu_rows.numel() - 1
    a.max_draft = draft_ids.shape[1] if max_draft is None else max_draft
    a.mode, a.dispatch, a.list_max = mode, dispatch, list_max
    a.workspace, a.workspace_bytes = workspace.data_ptr(), workspace.numel()
    return a


def launch(lib, args, stream=None, static_workspace=False):
    """es_launch (or, with `static_workspace`, es_launch_static) on `stream` (a HIP
    stream handle or a torch stream); raises on an error code."""
    handle = getattr(stream, "cuda_stream", stream)
    entry = lib.es_launch_static if static_workspace else lib.es_launch
    code = entry(ctypes.byref(args), ctypes.c_void_p(handle or 0))
    if code != 0:
        detail = lib.es_last_hip_error().decode()
        raise RuntimeError(f"es_launch failed: {lib.es_error_string(code).decode()}" + (f" ({detail})" if detail else ""))
