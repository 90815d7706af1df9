"""Group-wise 4-bit and 8-bit weight quantization with the reference's names,
layouts and rounding (`python/linnet/src/linnet/quant.py:1-136, 242-248`), computed
by the HIP kernels on the GPU.

Layouts (`std.quant::Int4GroupLinear`, `Int8GroupLinear`):

    int4: weight [Out, In/group, group/2] u8 (two codes a byte, low first),
          scale  [Out, In/group] (f32 here; stored in the model's dtype),
          zero   [Out, In/group] u8 in 0..15
    int8: weight [Out, In] i8 in -127..127, scale [Out, In/group]

Every function takes a numpy array or a torch tensor and returns the same kind
(numpy results are computed on `cuda:0` and copied back); the codes, scales and
zero points are bit for bit numpy's.
"""

from __future__ import annotations


import numpy as np
import torch

from .errors import LinnetError
from .torch import kernels

# Where the 8-bit linear layers switch kernels (`quant.py:73-80`): up to
# FEW_ROWS rows multiply the weight as it is, up to TILED_ROWS the weight-only
# tiled kernel beats the library GEMM over the weight dequantized for the call.
FEW_ROWS = 32
TILED_ROWS = 64


def _device_tensor(array: np.ndarray | torch.Tensor) -> tuple[torch.Tensor, bool]:
    if isinstance(array, torch.Tensor):
        return (array if array.is_cuda else array.to("cuda")), False
    if not torch.cuda.is_available():
        raise LinnetError("linnet_amd quantizes on the GPU; no GPU is available")
    return torch.from_numpy(np.ascontiguousarray(array)).to("cuda"), True


def _back(t: torch.Tensor, to_numpy: bool) -> np.ndarray | torch.Tensor:
    return t.cpu().numpy() if to_numpy else t


def quantize_int4_groups(weight, group: int = 128):
    """`(packed, scale, zero)` for an `[Out, In]` weight; `scale` is f32
    (`quant.py:83-99`)."""
    w, numpy = _device_tensor(weight)
    packed, scale, zero = kernels.quantize_int4(w, group)
    return _back(packed, numpy), _back(scale, numpy), _back(zero, numpy)


def pack_int4_groups(q, group: int):
    """`[Out, In]` codes in 0..15 as `[Out, In/group, group/2]` bytes, low nibble
    first (`quant.py:242-248`)."""
    codes, numpy = _device_tensor(q)
    out_features, in_features = codes.shape
    if group <= 0 or group % 2 or in_features % group:
        raise LinnetError(f"groups of {group} must be even and divide the {in_features} inputs")
    packed = kernels.pack4(codes.reshape(out_features, in_features // group, group))
    return _back(packed, numpy)


def dequantize_int4_groups(packed, scale, zero):
    """The f32 `[Out, In]` weight `(q - zero) * scale` (`quant.py:131-136`)."""
    p, numpy = _device_tensor(packed)
    s, _ = _device_tensor(scale)
    z, _ = _device_tensor(zero)
    weight = kernels.int4_weight(p, s.to(torch.float32), z)
    return _back(weight, numpy)


def quantize_int8_groups(weight, group: int = 128, dtype: str = "f32"):
    """`(q, scale)`: `scale = max|w| / 127` rounded to `dtype` first, then
    `q = clip(rint(w / scale), -127, 127)`; scale is f32 (`quant.py:102-121`)."""
    w, numpy = _device_tensor(weight)
    q, scale = kernels.quantize_int8(w, group, dtype)
    return _back(q, numpy), _back(scale, numpy)


def dequantize_int8_groups(q, scale):
    """The f32 `[Out, In]` weight `q * scale[group]` (`quant.py:124-128`)."""
    codes, numpy = _device_tensor(q)
    s, _ = _device_tensor(scale)
    out_features, in_features = codes.shape
    group = in_features // s.shape[1]
    weight = kernels.dequantize8(codes, s.to(torch.float32), False, group, 1, torch.float32)
    return _back(weight, numpy)


__all__ = [
    "FEW_ROWS",
    "TILED_ROWS",
    "dequantize_int4_groups",
    "dequantize_int8_groups",
    "pack_int4_groups",
    "quantize_int4_groups",
    "quantize_int8_groups",
]
