"""The quantized entries of the reference interpreter's `NATIVE` table
and its `take_inputs` gather (`python/linnet/src/linnet/torch/native.py:269-271,
417-480, 556-572`), keyed by the same
candidate names, running the HIP kernels. Each entry takes the call's arguments
as a tuple, as the interpreter passes them."""

from __future__ import annotations

from collections.abc import Callable, Sequence

import torch

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


def _index_select(args: Sequence[object]) -> torch.Tensor:
    """`std.quant::take_inputs` (`native.py:269-271`): `x[..., order[k]]`, on the HIP
    gather kernel."""
    x, order = args
    assert isinstance(x, torch.Tensor) and isinstance(order, torch.Tensor)
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
