"""The error the package raises, named as the reference names its own
(`python/linnet/src/linnet/compiler.py:18-23`, `LinnetError`)."""

from __future__ import annotations


class LinnetError(Exception):
    """A shape, dtype, layout or device the quantized kernels cannot take, or a
    failure reported by the HIP library."""
