"""Data model shared by the oracle and the tests.

Restates python/exactsample/types.py:7-44 (Status, PathUsed, RequestParams,
RngKey, VerifyOutput). The product package defines the same enums itself
(exactsample/types.py); tests check the two agree.
"""
from dataclasses import dataclass
from enum import IntEnum
from typing import Any


class Status(IntEnum):
    """Per-request status codes (docs/contract.md:21-28)."""
    OK = 0
    NO_VALID_TOKEN = 1
    INVALID_INPUT = 2
    DRAFT_ZERO_PROB = 3


class PathUsed(IntEnum):
    REFERENCE = 0
    FUSED = 1


@dataclass(frozen=True)
class RequestParams:
    """Scalars or one value per request; top_k=0 disables top-k."""
    temperature: Any = 1.0
    top_k: Any = 0
    top_p: Any = 1.0
    min_p: Any = 0.0
    draft_kind: Any = "one_hot"


@dataclass(frozen=True)
class RngKey:
    """seed: uint64, stream_id: uint32 (scalar or per request); positions: [rows]."""
    seed: Any
    stream_id: Any
    positions: Any


@dataclass
class VerifyOutput:
    tokens: Any
    accepted_len: Any
    status: Any
    path_used: Any
