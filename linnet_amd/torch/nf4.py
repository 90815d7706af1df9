"""`std.quant::Nf4Linear` on the HIP kernels (`stdlib/quant.linnet:177-215`).

The layer holds what `linnet_amd.quant.import_quantized` writes for a
bitsandbytes NF4 checkpoint: `weight` [Out, In/2] uint8 (QLoRA's 4-bit
NormalFloat codes, the first input of a pair in the low nibble), `absmax`
[Out, In/block] float32 and an optional `bias` in the activation dtype. Its
forward is `linear_nf4`: up to 16 rows of bf16 / f16 x (8 past In = 8192) read
the stored weight with the NF4 GEMV, once every 8 rows (4 past In = 8192); other calls widen the weight with the HIP
dequantize kernel (bit for bit the reference's `dequantize_nf4`) and multiply
in x's type, as the reference's body does.
"""

from __future__ import annotations

from pathlib import Path

import torch

from .. import weights
from ..errors import LinnetError
from . import kernels


def dequantize_nf4(q: torch.Tensor, absmax: torch.Tensor, block: int, dtype: torch.dtype) -> torch.Tensor:
    """`dequantize_nf4<Out, Blocks, Block, T>` (`stdlib/quant.linnet:180-187`)."""
    return kernels.nf4_dequantize(q, absmax, block, dtype)


def linear_nf4(x: torch.Tensor, q: torch.Tensor, absmax: torch.Tensor, bias: torch.Tensor | None = None,
               block: int = 64) -> torch.Tensor:
    """`linear_nf4<Block>(x, q, absmax, bias)` (`stdlib/quant.linnet:189-199`)."""
    return kernels.nf4_linear(x, q, absmax, block, bias)


class Nf4Linear(torch.nn.Module):
    """`Nf4Linear<In, Out, Block = 64, T = bf16>`: requires an even block that
    divides In (the block's `where` clause, quant.linnet:204-208)."""

    def __init__(self, in_features: int, out_features: int, block: int = 64, dtype: torch.dtype = torch.bfloat16,
                 bias: bool = False, device: torch.device | str | None = None) -> None:
        super().__init__()
        if block <= 0 or block % 2 or in_features % block:
            raise LinnetError(f"Nf4Linear: In={in_features} must split into even blocks of {block}")
        self.in_features, self.out_features, self.block, self.dtype = in_features, out_features, block, dtype
        self.weight = torch.nn.Parameter(
            torch.zeros(out_features, in_features // 2, dtype=torch.uint8, device=device), requires_grad=False)
        self.absmax = torch.nn.Parameter(
            torch.ones(out_features, in_features // block, dtype=torch.float32, device=device), requires_grad=False)
        self.bias = (torch.nn.Parameter(torch.zeros(out_features, dtype=dtype, device=device), requires_grad=False)
                     if bias else None)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.dtype != self.dtype:
            raise LinnetError(f"Nf4Linear: x is {x.dtype}, the layer {self.dtype}")
        return linear_nf4(x, self.weight, self.absmax, self.bias, self.block)

    def load(self, checkpoint: str | Path, prefix: str) -> Nf4Linear:
        """Reads `prefix + "weight"`, `"absmax"` and, when the layer has one,
        `"bias"` from a SafeTensors checkpoint (as `import_quantized` writes them)
        onto the layer's device."""
        index = weights.open_checkpoint(checkpoint)
        device = self.weight.device
        for name, param, dtype in (("weight", self.weight, torch.uint8), ("absmax", self.absmax, torch.float32),
                                   ("bias", self.bias, self.dtype)):
            if param is None:
                continue
            stored = index.get(prefix + name)
            if stored is None:
                raise LinnetError(f"Nf4Linear.load: {checkpoint} has no `{prefix + name}`")
            value = (weights.tensor_from(stored, dtype, device) if dtype == torch.uint8
                     else weights.float_tensor(stored, device).to(dtype))
            if tuple(value.shape) != tuple(param.shape):
                raise LinnetError(f"Nf4Linear.load: `{prefix + name}` is {tuple(value.shape)}, "
                                  f"the layer's {tuple(param.shape)}")
            param.data.copy_(value)
        return self


__all__ = ["Nf4Linear", "dequantize_nf4", "linear_nf4"]
