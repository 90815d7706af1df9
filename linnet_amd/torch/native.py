"""The quantized entries of the reference interpreter's `NATIVE` table
and its `take_inputs` gather (`python/linnet/src/linnet/torch/native.py:269-271,
417-480, 556-572`), keyed by the same
candidate names, running the HIP kernels. Each entry takes the call's arguments
as a tuple, as the interpreter passes them."""

from __future__ import annotations

from collections.abc import Callable, Sequence

import torch

from ..errors import LinnetError
from . import generated, kernels, quantized

Native = Callable[[Sequence[object]], torch.Tensor]


def _int4_groups_linear(args: Sequence[object]) -> torch.Tensor:
    """`std.quant::linear_int4_groups` (`native.py:417-423`)."""
    x, packed, scale, zero, bias = args
    assert isinstance(x, torch.Tensor) and isinstance(packed, torch.Tensor)
    assert isinstance(scale, torch.Tensor) and isinstance(zero, torch.Tensor)
    prepared = generated._int4_pack(packed, scale, zero)
    return generated._int4_linear(x, prepared, bias, packed, scale, zero)  # type: ignore[arg-type]


def _decode_fp8(args: Sequence[object]) -> torch.Tensor:
    """`std.quant::decode_fp8` (`native.py:426-429`): the bytes as `float8_e4m3fn`, widened."""
    (bits,) = args
    assert isinstance(bits, torch.Tensor)
    return bits.view(torch.float8_e4m3fn).float()


def _fp8_linear(rounded: int) -> Native:
    def run(args: Sequence[object]) -> torch.Tensor:
        x, weight, scale, bias = args
        return quantized.fp8_linear(x, quantized.fp8_operands(weight, scale, rounded), bias)  # type: ignore[arg-type]

    return run


def _fp8_block_linear(rounded: int) -> Native:
    def run(args: Sequence[object]) -> torch.Tensor:
        x, weight, scale, bias = args
        return quantized.fp8_block_linear(x, quantized.fp8_block_operands(weight, scale, rounded), bias)  # type: ignore[arg-type]

    return run


def _int8_linear(rounded: int) -> Native:
    def run(args: Sequence[object]) -> torch.Tensor:
        x, weight, scale, bias = args
        return quantized.int8_linear(x, quantized.int8_operands(weight, scale, rounded), bias)  # type: ignore[arg-type]

    return run


def _int8_group_linear(args: Sequence[object]) -> torch.Tensor:
    x, weight, scale, bias = args
    return quantized.int8_group_linear(x, quantized.int8_group_operands(weight, scale), bias)  # type: ignore[arg-type]


_GATHERED = (torch.bfloat16, torch.float16, torch.float32)


def _index_select(args: Sequence[object]) -> torch.Tensor:
    """`std.quant::take_inputs` (`native.py:269-271`): `x[..., order[k]]`.

    The interpreter's entry is generic (any dtype, and an index outside the axis
    raises). bf16 / f16 / f32 GPU tensors run the HIP gather kernel, whose
    out-of-range index would read 0, so the order is range-checked first (one
    host read of its extremes; skipped under graph capture, where the caller's
    order was checked when the layer was built). Other dtypes, and an order that
    is not a permutation-sized [n] vector, go to torch's own `index_select` on
    the GPU, which is what the reference calls. CPU tensors raise, as every
    entry of this package does."""
    x, order = args
    assert isinstance(x, torch.Tensor) and isinstance(order, torch.Tensor)
    if not x.is_cuda:
        raise LinnetError(f"linnet_amd runs on the GPU; take_inputs got x on {x.device}")
    if x.dtype not in _GATHERED or x.dim() == 0 or tuple(order.shape) != (x.shape[-1],):
        return x.index_select(-1, order.long())
    n = x.shape[-1]
    if order.numel() and not torch.cuda.is_current_stream_capturing():
        low, high = torch.aminmax(order)
        if int(low) < 0 or int(high) >= n:
            raise LinnetError(f"take_inputs: order holds indices outside [0, {n}): {int(low)}..{int(high)}")
    return kernels.take_inputs(x, order if order.dtype == torch.int32 else order.to(torch.int32))


NATIVE: dict[str, Native] = {
    "torch.ops.aten._weight_int4pack_mm": _int4_groups_linear,
    "linnet.decode_fp8": _decode_fp8,
    "linnet.fp8_linear": _fp8_linear(0),
    "torch._scaled_mm": _fp8_linear(1),
    "linnet.fp8_block_linear": _fp8_block_linear(0),
    "torch._scaled_mm(blocks)": _fp8_block_linear(1),
    "linnet.int8_linear": _int8_linear(0),
    "linnet.int8_linear(w8a8)": _int8_linear(1),
    "linnet.int8_group_linear": _int8_group_linear,
    "torch.index_select": _index_select,
}
