"""exactsample: exact token sampling and speculative-draft verification on MI355X (gfx950).

A from-scratch gfx950 implementation of exactsample's device path behind the
same API: ``plan`` and ``verify`` (exactsample.cuda), the data model
(exactsample.types) and the ``torch.ops.exactsample.verify_out`` op, a thin
binding over the C ABI in include/exactsample_amd.h.

The FP64 CPU oracle of the reference (``verify_reference`` and friends) is not
part of this package; it lives in the repository's ``oracle/`` test
infrastructure.
"""
from .types import PathUsed, RequestParams, RngKey, Status, VerifyOutput

__version__ = "0.1.0"


def plan(*args, **kwargs):
    from .cuda import plan as implementation
    return implementation(*args, **kwargs)


def verify(*args, **kwargs):
    from .cuda import verify as implementation
    return implementation(*args, **kwargs)


__all__ = ["PathUsed", "RequestParams", "RngKey", "Status", "VerifyOutput", "plan", "verify"]
