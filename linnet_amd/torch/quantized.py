"""`std.quant`'s 8-bit linear layers as the generated PyTorch runs them, with the
reference's names, operand tuples and dispatch
(`python/linnet/src/linnet/torch/quantized.py:1-218`), on the gfx950 HIP kernels.

Each layer is two calls: `*_operands` (prepare, once) and `*_linear` (per call).
On the GPU, in bf16 or f16:

- up to `TILED_ROWS` (64) rows: `kernels.w8a16` (one row: `gemv8`), the weight
  widened in registers, x unrounded;
- more rows: the weight dequantized for the call (`kernels.dequantize8`), then
  `F.linear` (hipBLASLt);
- past `FEW_ROWS` (32) rows and `rounded` (`numerics="fast"`): x rounded to 8 bits a
  row at a time (`fp8_rows` / `int8_rows`) and the two multiplied in 8 bits on
  MFMA (`fp8_mm`, replacing `torch._scaled_mm`; `int8_mm`).

Anywhere else on the GPU (f32 activations, shapes the kernels do not take) the
weight is dequantized by the HIP kernel and multiplied by `F.linear`. CPU
tensors raise: this package has no CPU path.
"""

from __future__ import annotations

import torch
import torch.nn.functional as functional

from ..errors import LinnetError
from ..quant import FEW_ROWS, TILED_ROWS
from . import kernels

_HALF = (torch.bfloat16, torch.float16)

Fp8Operands = tuple[torch.Tensor, torch.Tensor, torch.Tensor, int, int]
Fp8BlockOperands = tuple[torch.Tensor, torch.Tensor, torch.Tensor, int, int, int]
Int8Operands = tuple[torch.Tensor, torch.Tensor, int, int]
Int8GroupOperands = tuple[torch.Tensor, torch.Tensor, int, int]


def _gpu(weight: torch.Tensor) -> None:
    if not weight.is_cuda:
        raise LinnetError(f"linnet_amd runs on the GPU; the weight is on {weight.device}")


def _fp8_kernels(weight: torch.Tensor) -> int:
    """2: the weight-only kernels and the FP8 MFMA product run here; 0: neither
    (the reference's gate, `quantized.py:75-82`, with gfx950 for sm90)."""
    out_features, in_features = weight.shape
    return 0 if in_features % 128 else 2


def _int8_kernels(weight: torch.Tensor) -> int:
    """`quantized.py:85-87`: In % 128 == 0."""
    return int(weight.shape[1] % 128 == 0)


def _weight_only(flat: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor, fp8: bool, group: int = 0, row_block: int = 1) -> torch.Tensor:
    """`quantized.py:90-105`: one row -> gemv8, <= TILED_ROWS -> w8a16, more ->
    dequantize8 + F.linear."""
    rows = flat.shape[0]
    fused_group = group == 0 or group % 64 == 0
    if rows == 1 and fused_group:
        return kernels.gemv8(flat, weight, scale, fp8, group, row_block)
    if rows <= TILED_ROWS and fused_group:
        return kernels.w8a16(flat, weight, scale, fp8, group, row_block)
    dequantized = kernels.dequantize8(weight, scale, fp8, group, row_block, flat.dtype)
    return functional.linear(flat, dequantized)


def _finish(x: torch.Tensor, y: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
    y = y.reshape(*x.shape[:-1], y.shape[-1])
    return y if bias is None else y + bias


def fp8_operands(weight: torch.Tensor, scale: torch.Tensor, rounded: int) -> Fp8Operands:
    """`weight` [Out, In] FP8 E4M3 (or its bytes), `scale` [Out] (or [Out, 1]): the
    bytes, the same viewed as FP8 (the MFMA product reads them row-major; no
    transposed copy is needed), the scales as f32 [1, Out], `rounded`, the gate
    (`quantized.py:113-120`)."""
    _gpu(weight)
    weight = weight.contiguous().view(torch.uint8)
    fp8 = weight.view(torch.float8_e4m3fn)
    row = scale.float().reshape(1, -1).contiguous()
    return weight, fp8, row, rounded, _fp8_kernels(weight)


def fp8_linear(x: torch.Tensor, operands: Fp8Operands, bias: torch.Tensor | None) -> torch.Tensor:
    """`quantized.py:123-135`."""
    weight, fp8, scale, rounded, fast = operands
    flat = x.reshape(-1, x.shape[-1])
    if fast and flat.dtype in _HALF:
        if rounded and fast == 2 and flat.shape[0] > FEW_ROWS:
            q, rows = kernels.fp8_rows(flat)
            y = kernels.fp8_mm(q, fp8, rows, scale.reshape(-1), flat.dtype)
        else:
            y = _weight_only(flat, weight, scale.reshape(-1), True)
    else:
        decoded = kernels.dequantize8(weight, scale.reshape(-1), True, 0, 1, flat.dtype)
        y = functional.linear(flat, decoded)
    return _finish(x, y, bias)


def fp8_block_operands(weight: torch.Tensor, scale: torch.Tensor, rounded: int) -> Fp8BlockOperands:
    """`weight` [Out, In] FP8 E4M3, `scale` [Out/B, In/B]: bytes, FP8 view, f32
    scales, B, `rounded`, the gate (`quantized.py:138-151`): 2 where the FP8 x FP8
    block-scaled product takes the blocks (B = 128, as PyTorch's), 1 where only the
    weight-only kernels do."""
    _gpu(weight)
    weight = weight.contiguous().view(torch.uint8)
    block = weight.shape[0] // scale.shape[0]
    fast = _fp8_kernels(weight) if weight.shape[1] == block * scale.shape[1] else 0
    if block != 128 or weight.shape[0] % 128:
        fast = min(fast, 1)
    return weight, weight.view(torch.float8_e4m3fn), scale.float().contiguous(), block, rounded, fast


def fp8_block_linear(x: torch.Tensor, operands: Fp8BlockOperands, bias: torch.Tensor | None) -> torch.Tensor:
    """`quantized.py:154-173`: past FEW_ROWS rows with `rounded`, the rows rounded to
    FP8 per 128 inputs (`fp8_groups`) and the block-scaled FP8 product; else the
    weight-only kernels."""
    weight, fp8, scale, block, rounded, fast = operands
    flat = x.reshape(-1, x.shape[-1])
    if fast and flat.dtype in _HALF:
        rows = flat.shape[0]
        if rounded and fast == 2 and rows > FEW_ROWS:
            q, scales = kernels.fp8_groups(flat, block, rows)
            y = kernels.fp8_block_mm(q, fp8, scales, scale, flat.dtype)
        else:
            y = _weight_only(flat, weight, scale, True, block, block)
    else:
        decoded = kernels.dequantize8(weight, scale, True, block, block, flat.dtype)
        y = functional.linear(flat, decoded)
    return _finish(x, y, bias)


def int8_operands(weight: torch.Tensor, scale: torch.Tensor, rounded: int) -> Int8Operands:
    """`weight` [Out, In] i8, `scale` [Out]: the weight and f32 scales (`quantized.py:176-180`)."""
    _gpu(weight)
    weight = weight.contiguous()
    return weight, scale.float().reshape(-1).contiguous(), rounded, _int8_kernels(weight)


def int8_linear(x: torch.Tensor, operands: Int8Operands, bias: torch.Tensor | None) -> torch.Tensor:
    """`quantized.py:183-194`."""
    weight, scale, rounded, fast = operands
    flat = x.reshape(-1, x.shape[-1])
    if fast and flat.dtype in _HALF:
        if rounded and flat.shape[0] > FEW_ROWS:
            q, rows = kernels.int8_rows(flat)
            y = kernels.int8_mm(q, weight, rows, scale, flat.dtype)
        else:
            y = _weight_only(flat, weight, scale, False)
    else:
        y = functional.linear(flat, kernels.dequantize8(weight, scale, False, 0, 1, flat.dtype))
    return _finish(x, y, bias)


def int8_group_operands(weight: torch.Tensor, scale: torch.Tensor) -> Int8GroupOperands:
    """`weight` [Out, In] i8, `scale` [Out, In/group]: weight, f32 scales, group
    (`quantized.py:197-203`)."""
    _gpu(weight)
    weight = weight.contiguous()
    group = weight.shape[1] // scale.shape[1]
    fast = _int8_kernels(weight) if group % 16 == 0 else 0
    return weight, scale.float().contiguous(), group, fast


def int8_group_linear(x: torch.Tensor, operands: Int8GroupOperands, bias: torch.Tensor | None) -> torch.Tensor:
    """`quantized.py:206-218`."""
    weight, scale, group, fast = operands
    flat = x.reshape(-1, x.shape[-1])
    if fast and flat.dtype in _HALF:
        y = _weight_only(flat, weight, scale, False, group)
    else:
        y = functional.linear(flat, kernels.dequantize8(weight, scale, False, group, 1, flat.dtype))
    return _finish(x, y, bias)
