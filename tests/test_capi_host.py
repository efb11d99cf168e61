"""The C-ABI library without a GPU: it loads, exports what include/exactsample_amd.h
declares, sizes workspaces, and rejects malformed arguments on the host before
any HIP call (no kernel is launched by these tests)."""
import ctypes
import re
from pathlib import Path

import pytest

from exactsample import capi

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "exactsample_amd.h"


@pytest.fixture(scope="module")
def lib():
    path = ROOT / "exactsample" / "libexactsample_amd.so"
    if not path.is_file():
        pytest.skip("libexactsample_amd.so is not built (python -m exactsample.build)")
    return capi.load(path)


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(es_[a-z_0-9]+)\s*\(", text, re.M)))


def test_header_and_binding_agree():
    assert declared_functions() == sorted(capi.EXPORTS)


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_workspace_size_formula(lib):
    # 8 header bytes, then per row 32 (result) + max(12288, 20 V for the reference path).
    assert lib.es_workspace_size(128, 151936, 0) == 8 + 128 * (32 + 12288)
    assert lib.es_workspace_size(3, 151936, 1) == 8 + 3 * (32 + 20 * 151936)
    assert lib.es_workspace_size(0, 10, 0) == 8
    assert lib.es_fallback_counter_offset() == 4


def test_error_strings(lib):
    assert lib.es_error_string(0) == b"success"
    assert b"workspace" in lib.es_error_string(4)
    assert b"null" in lib.es_error_string(1)
    assert lib.es_last_hip_error() == b""


def arguments(rows=2, requests=1, vocab=1000, max_draft=1):
    """Structurally valid arguments with fake, never dereferenced addresses."""
    fake = 1 << 20
    a = capi.Arguments()
    a.target = capi.Matrix(fake, vocab, 1, 0, 0)
    a.draft = capi.Matrix(None, 0, 0, 0, 0)
    for field in ("cu_rows", "top_k", "draft_kind", "seed", "stream", "position"):
        setattr(a, field, capi.VecI64(fake, 1))
    for field in ("temperature", "top_p", "min_p"):
        setattr(a, field, capi.VecF64(fake, 1))
    a.draft_ids, a.draft_s0, a.draft_s1 = fake, max_draft, 1
    a.tokens, a.token_s0, a.token_s1 = fake, max_draft + 1, 1
    a.accepted, a.accepted_s = fake, 1
    a.status, a.status_s = fake, 1
    a.path, a.path_s = fake, 1
    a.rows, a.requests, a.vocab, a.max_draft = rows, requests, vocab, max_draft
    a.mode, a.dispatch, a.list_max = 0, 2, 256
    a.workspace, a.workspace_bytes = fake, capi.load().es_workspace_size(rows, vocab, 0)
    return a


@pytest.mark.parametrize("change, code", [
    (lambda a: setattr(a, "tokens", None), 1),
    (lambda a: setattr(a, "workspace", None), 1),
    (lambda a: setattr(a, "vocab", 0), 2),
    (lambda a: setattr(a, "rows", -1), 2),
    (lambda a: setattr(a, "mode", 2), 3),
    (lambda a: setattr(a, "list_max", 257), 3),
    (lambda a: setattr(a, "workspace_bytes", 64), 4),
    (lambda a: setattr(a, "workspace", (1 << 20) + 4), 5),
    (lambda a: setattr(a.target, "dtype", 9), 6),
    (lambda a: setattr(a, "draft", capi.Matrix(1 << 20, 1000, 1, 3, 0)), 6),
])
def test_host_checks_reject_before_launch(lib, change, code):
    a = arguments()
    change(a)
    assert lib.es_launch(ctypes.byref(a), None) == code


def test_null_arguments_and_empty_batch(lib):
    assert lib.es_launch(None, None) == 1
    a = arguments(rows=0, requests=0)
    a.target = capi.Matrix(None, 0, 0, 0, 0)
    assert lib.es_launch(ctypes.byref(a), None) == 0  # nothing to do, nothing launched


@pytest.mark.parametrize("dtype, vocab, list_max", [(2, 262148, 256), (0, 300000, 0), (3, 1048580, 256),
                                                    (1, 2**31 - 1, 256)])
def test_any_vocabulary_passes_the_host_checks(lib, dtype, vocab, list_max):
    """Vocabularies past 64 register tiles per row are accepted (slices of
    several tiles): without a device the call gets as far as the launch and
    reports ES_ERR_LAUNCH, never ES_ERR_BAD_DIMENSION. Run only where no HIP
    device is visible, since the addresses here are fake."""
    import torch
    if torch.cuda.device_count() > 0:
        pytest.skip("a HIP device is visible: the fake addresses must not reach a kernel")
    a = arguments(rows=3, requests=3, vocab=vocab, max_draft=0)
    a.target = capi.Matrix(1 << 20, vocab, 1, dtype, 0)
    a.list_max = list_max
    a.workspace_bytes = lib.es_workspace_size(3, vocab, 0)
    assert lib.es_launch(ctypes.byref(a), None) == 7
