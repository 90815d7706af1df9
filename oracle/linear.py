"""The reference's CPU linear paths for `std.quant`'s layers, restated.

TEST INFRASTRUCTURE ONLY (see `oracle/__init__.py`): the checker for the HIP
kernels' outputs and the timed CPU baseline of `bench.py`.

The reference runs its CPU path through PyTorch on the CPU (dequantize, cast
to the activation dtype, `F.linear`), so these restatements do too. The fp64
products are the tolerance references: the weight dequantized exactly (f32
arithmetic that is exact for these formats), the product summed in f64.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as functional

from . import quant


def _codes(packed: torch.Tensor) -> torch.Tensor:
    out_features, groups, half = packed.shape
    return torch.stack([packed & 15, packed >> 4], dim=-1).reshape(out_features, groups, 2 * half)


def int4_groups_linear_interpreter(
    x: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor, bias: torch.Tensor | None
) -> torch.Tensor:
    """`native._int4_groups_linear` (`python/linnet/src/linnet/torch/native.py:417-423`):
    the interpreter's (CPU default) int4 linear -- per call, `(q - z) * s` in
    f32, cast to x's dtype, `F.linear`, then the bias."""
    out_features, groups, half = packed.shape
    q = _codes(packed)
    weight = (q.float() - zero.float()[..., None]) * scale.float()[..., None]
    y = functional.linear(x, weight.reshape(out_features, groups * 2 * half).to(x.dtype))
    return y if bias is None else y + bias


def int4_prepare_cpu(packed: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor) -> torch.Tensor:
    """The CPU branch of the generated `_int4_pack` (`src/backend/torch_source.cpp:1501-1504`):
    the weight dequantized once at prepare, in the scale's dtype."""
    out_features, groups, half = packed.shape
    q = _codes(packed)
    weight = (q.float() - zero.float()[..., None]) * scale.float()[..., None]
    return weight.reshape(out_features, groups * 2 * half).to(scale.dtype)


def int4_linear_generated_cpu(x: torch.Tensor, prepared: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
    """The CPU branch of the generated `_int4_linear` (`torch_source.cpp:1567-1570`):
    `F.linear` over the weight prepared once, then the bias."""
    flat = x.reshape(-1, x.shape[-1])
    y = functional.linear(flat, prepared).reshape(*x.shape[:-1], prepared.shape[0])
    return y if bias is None else y + bias


def int8_linear_cpu(x: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
    """`quantized.int8_linear`'s CPU branch (`torch/quantized.py:193`): per call,
    `(w.float() * s[:, None]).to(x.dtype)`, then `F.linear` and the bias."""
    flat = x.reshape(-1, x.shape[-1])
    s = scale.float().reshape(-1)
    y = functional.linear(flat, (weight.float() * s[:, None]).to(flat.dtype))
    y = y.reshape(*x.shape[:-1], y.shape[-1])
    return y if bias is None else y + bias


def int8_group_linear_cpu(x: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
    """`quantized.int8_group_linear`'s CPU branch (`torch/quantized.py:212-217`)."""
    flat = x.reshape(-1, x.shape[-1])
    out_features, in_features = weight.shape
    group = in_features // scale.shape[1]
    grouped = weight.float().reshape(out_features, in_features // group, group)
    decoded = (grouped * scale.float()[:, :, None]).reshape(out_features, in_features)
    y = functional.linear(flat, decoded.to(flat.dtype)).reshape(*x.shape[:-1], out_features)
    return y if bias is None else y + bias


def fp8_linear_cpu(x: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
    """`quantized.fp8_linear`'s CPU branch (`torch/quantized.py:133-134`): the FP8
    weight widened, times the per-row scale, cast to x's dtype, `F.linear`.
    The CPU path does not round the activations."""
    flat = x.reshape(-1, x.shape[-1])
    decoded = weight.contiguous().view(torch.uint8).view(torch.float8_e4m3fn).float() * scale.float().reshape(-1, 1)
    y = functional.linear(flat, decoded.to(flat.dtype)).reshape(*x.shape[:-1], weight.shape[0])
    return y if bias is None else y + bias


def fp8_block_linear_cpu(x: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
    """`quantized.fp8_block_linear`'s CPU branch (`torch/quantized.py:167-172`): the
    FP8 weight widened, each `B x B` block times its scale `scale[o / B, i / B]`
    in f32, cast to x's dtype, `F.linear`, then the bias. The CPU path does not
    round the activations."""
    flat = x.reshape(-1, x.shape[-1])
    out_features, in_features = weight.shape
    block = out_features // scale.shape[0]
    decoded = weight.contiguous().view(torch.uint8).view(torch.float8_e4m3fn).float()
    decoded = decoded.reshape(out_features // block, block, in_features // block, block) * scale.float()[:, None, :, None]
    y = functional.linear(flat, decoded.reshape(out_features, in_features).to(flat.dtype))
    y = y.reshape(*x.shape[:-1], out_features)
    return y if bias is None else y + bias


# ------------------------------------------------------------ fp64 references


def product_f64(x: np.ndarray, weight: np.ndarray) -> np.ndarray:
    """`x @ weight.T` summed in f64 (x, weight given as f32 values)."""
    return np.asarray(x, dtype=np.float64) @ np.asarray(weight, dtype=np.float64).T


def int4_reference_f64(x: np.ndarray, packed: np.ndarray, scale: np.ndarray, zero: np.ndarray) -> np.ndarray:
    """fp64 product with the exactly dequantized int4 weight (`quant.dequantize_int4_groups`)."""
    return product_f64(x, quant.dequantize_int4_groups(packed, scale, zero))


def rows8_product_f64(q: np.ndarray, xs: np.ndarray, wq: np.ndarray, ws: np.ndarray, fp8: bool) -> np.ndarray:
    """fp64 product of 8-bit rows with their scales and 8-bit weights with
    per-row scales: `(qx @ qw.T) * xs * ws`, the result `torch._scaled_mm` /
    `int8_mm` (`torch/kernels.py:805-843`) approximate."""
    if fp8:
        qx = quant.decode_fp8(q).astype(np.float64)
        qw = quant.decode_fp8(wq).astype(np.float64)
    else:
        qx = q.astype(np.float64)
        qw = wq.astype(np.float64)
    return (qx @ qw.T) * xs.reshape(-1, 1).astype(np.float64) * ws.reshape(1, -1).astype(np.float64)


def block_product_f64(q: np.ndarray, xs: np.ndarray, wq: np.ndarray, ws: np.ndarray, block: int = 128) -> np.ndarray:
    """fp64 block-scaled FP8 product: `sum_b (qx[:, b] @ qw[:, b].T) * xs[:, b] *
    ws[n / block, b]` over the `block`-input blocks b, FP8 codes decoded exactly --
    the result `torch._scaled_mm` with block-wise scales approximates
    (`torch/quantized.py:159-166`; dequantized operands, `:167-172`)."""
    qx = quant.decode_fp8(q).astype(np.float64)
    qw = quant.decode_fp8(wq).astype(np.float64)
    rows, depth = qx.shape
    width = qw.shape[0]
    x = (qx.reshape(rows, depth // block, block) * xs.astype(np.float64)[:, :, None]).reshape(rows, depth)
    w = (qw.reshape(width // block, block, depth // block, block) * ws.astype(np.float64)[:, None, :, None])
    return x @ w.reshape(width, depth).T


def mxfp4_experts_f64(x: np.ndarray, blocks: np.ndarray, scales: np.ndarray, experts: np.ndarray) -> np.ndarray:
    """fp64 `y[r, k, o] = sum_i x[r, k, i] * W[experts[r, k], o, i]` with `W` the
    dequantized MXFP4 experts (`stdlib/quant.linnet:343-356`, `mxfp4_experts`; the
    generated fallback, `torch_source.cpp:1595-1601`, computes it in f32)."""
    weight = quant.dequantize_mxfp4(blocks, scales).astype(np.float64)  # [E, Out, In]
    chosen = weight[np.asarray(experts)]  # [R, K, Out, In]
    return np.einsum("rki,rkoi->rko", np.asarray(x, dtype=np.float64), chosen)


def nf4_reference_f64(x: np.ndarray, codes: np.ndarray, absmax: np.ndarray, block: int,
                      bias: np.ndarray | None = None) -> np.ndarray:
    """`linear_nf4` (`stdlib/quant.linnet:189-199`) in f64 over the exact f32
    weight `quant.nf4_weight`: the tolerance reference of the NF4 GEMV."""
    y = product_f64(x, quant.nf4_weight(codes, absmax, block))
    return y if bias is None else y + np.asarray(bias, dtype=np.float64)
