"""The integer 4-bit storage formats (`std.dtypes`: `i4`, `u4`) as PyTorch holds
them -- bytes, the last axis halved, element 2k in the low four bits -- packed
and widened by the HIP kernels (`python/linnet/src/linnet/torch/packed.py:21-75`).
FP4 E2M1 (MXFP4) is outside this package's scope."""

from __future__ import annotations

import torch

from ..errors import LinnetError
from . import kernels

_FORMATS = ("i4", "u4")


def unpack4(packed: torch.Tensor, kind: str) -> torch.Tensor:
    """`packed`'s elements of format `kind`, widened: `u4` to uint8, `i4` to int8."""
    if kind not in _FORMATS:
        raise LinnetError(f"`{kind}` is not an integer 4-bit format ({', '.join(_FORMATS)})")
    return kernels.unpack4(packed, kind)


def pack4(x: torch.Tensor, kind: str) -> torch.Tensor:
    """`x` narrowed to format `kind` as bytes (its even last axis halved): integers
    wrap, floats round toward zero first."""
    if kind not in _FORMATS:
        raise LinnetError(f"`{kind}` is not an integer 4-bit format ({', '.join(_FORMATS)})")
    return kernels.pack4(x)


__all__ = ["pack4", "unpack4"]
