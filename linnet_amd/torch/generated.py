"""The helpers generated PyTorch calls for `std.quant::linear_int4_groups`,
with the reference's names and contract (`src/backend/torch_source.cpp:1478-1571`):

    packed = _int4_pack(p_w, p_s, p_z)                   # in prepare(), once
    y = _int4_linear(x, packed, bias, p_w, p_s, p_z)     # in main(), per call

`_int4_pack` returns a 3-tuple when the HIP kernels take the layer (a GPU,
bf16 or f16 scales, a group of 32, 64 or a multiple of 128, In % 128 == 0):
the parameters themselves, read as they are stored, so nothing is repacked
and no bytes are held beyond the model's own. Otherwise it returns the
1-tuple of the weight dequantized once, by the HIP dequantize kernel, as the
reference's `_int4_pack` falls back (`torch_source.cpp:1501-1504`), and
`_int4_linear` multiplies it with `F.linear`.

`_int4_row_pack` / `_int4_row_linear` run `std.quant::Int4Linear` (per-row
signed int4) on the same kernels; `_int4_join` / `_int4_split` join sibling
int4 layers that read one input into one launch.

`_mxfp4_experts(x, blocks, scales, experts)` is the helper for
`std.quant::mxfp4_experts` (`torch_source.cpp:1579-1600`): the chosen experts'
MXFP4 weights multiplied by one HIP kernel; `_mxfp4_grouped` the one for the
shared and combine forms (`torch_source.cpp:1705-1735`) on the same kernel.

CPU tensors raise: this package has no CPU path.
"""

from __future__ import annotations

import torch
import torch.nn.functional as functional

from ..errors import LinnetError
from . import kernels

_FUSED_DTYPES = (torch.bfloat16, torch.float16)


def _fused_group(group: int) -> bool:
    return group in (32, 64) or (group > 0 and group % 128 == 0)


def _int4_pack(packed: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor) -> tuple[torch.Tensor, ...]:
    """Prepare-time: `(packed, scale, zero)` for the fused kernels, or
    `(dequantized weight,)`. `packed` is [Out, Groups, Group/2] u8."""
    if not packed.is_cuda:
        raise LinnetError("_int4_pack: linnet_amd runs on the GPU; the weight is on " + str(packed.device))
    out_features, groups, half = packed.shape
    group = 2 * half
    in_features = groups * group
    if scale.dtype in _FUSED_DTYPES and _fused_group(group) and in_features % 128 == 0:
        return (packed.contiguous(), scale.contiguous(), zero.contiguous())
    return (kernels.int4_weight(packed, scale, zero),)


def _int4_weight(raw: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor) -> torch.Tensor:
    """The weight dequantized, in `scale`'s dtype: one HIP kernel
    (`torch_source.cpp:1536-1550`)."""
    return kernels.int4_weight(raw, scale, zero)


def _int4_linear(
    x: torch.Tensor,
    packed: tuple[torch.Tensor, ...],
    bias: torch.Tensor | None,
    raw: torch.Tensor,
    scale: torch.Tensor,
    zero: torch.Tensor,
) -> torch.Tensor:
    """`x @ W.T (+ bias)` over `x`'s last axis (`torch_source.cpp:1553-1570`).
    With the fused 3-tuple, any number of rows runs one HIP kernel (few rows the
    skinny MFMA kernel, many the tiled dequant-GEMM) with the bias added in its
    epilogue; with the 1-tuple, `F.linear` over the dequantized weight."""
    flat = x.reshape(-1, x.shape[-1])
    if len(packed) == 3 and x.dtype == scale.dtype:
        p, s, z = packed
        y = kernels.int4_linear(flat, p, s, z, bias)
        return y.reshape(*x.shape[:-1], y.shape[-1])
    if not x.is_cuda:
        raise LinnetError("_int4_linear: linnet_amd runs on the GPU; x is on " + str(x.device))
    weight = packed[0] if len(packed) == 1 else kernels.int4_weight(raw, scale, zero)
    y = functional.linear(flat, weight.to(flat.dtype))
    y = y.reshape(*x.shape[:-1], y.shape[-1])
    return y if bias is None else y + bias


def _int4_row_pack(weight: torch.Tensor, scale: torch.Tensor) -> tuple[torch.Tensor, ...]:
    """Prepare-time for `std.quant::Int4Linear` (`stdlib/quant.linnet:101-111`;
    `weight` [Out, In/2] u8 of i4 values, `scale` [Out, 1] in the model dtype).
    The reference's generated module has no helper for this layer: it runs the
    body, `linear(x, cast<T>(f32(i4) * scale))`. Here the weight is rewritten once
    into the group layout `_int4_pack` returns -- each code the value plus 8, zero
    point 8, the row's scale for each group of 128 -- so the fused kernels read 4
    bits a weight; that copy holds In * Out / 2 bytes beside the parameter, as the
    reference's tinygemm repack does. Layers the kernels do not take (In % 128 != 0,
    f32 scales) get the 1-tuple of the weight dequantized once by the body's
    formula, on the GPU."""
    if not weight.is_cuda:
        raise LinnetError("_int4_row_pack: linnet_amd runs on the GPU; the weight is on " + str(weight.device))
    in_features = 2 * weight.shape[1]
    rows = scale.reshape(-1)
    if scale.dtype in _FUSED_DTYPES and in_features % 128 == 0:
        return kernels.int4_row_prepare(weight, rows, 128)
    if in_features % 32 == 0:
        return (kernels.int4_weight(*kernels.int4_row_prepare(weight, rows, in_features)),)
    values = kernels.unpack4(weight, "i4")
    return ((values.float() * rows.float()[:, None]).to(scale.dtype),)


def _int4_row_linear(x: torch.Tensor, packed: tuple[torch.Tensor, ...], bias: torch.Tensor | None) -> torch.Tensor:
    """`Int4Linear.forward`: `linear(x, dequantize_int4(weight, scale), bias)`
    (`stdlib/quant.linnet:108-110`) with the weight prepared by `_int4_row_pack`."""
    flat = x.reshape(-1, x.shape[-1])
    if len(packed) == 3 and x.dtype == packed[1].dtype:
        y = kernels.int4_linear(flat, *packed, bias)
        return y.reshape(*x.shape[:-1], y.shape[-1])
    if not x.is_cuda:
        raise LinnetError("_int4_row_linear: linnet_amd runs on the GPU; x is on " + str(x.device))
    weight = packed[0] if len(packed) == 1 else kernels.int4_weight(*packed)
    y = functional.linear(flat, weight.to(flat.dtype)).reshape(*x.shape[:-1], weight.shape[0])
    return y if bias is None else y + bias


def _int4_join(*packs: tuple[torch.Tensor, ...]) -> tuple[tuple[torch.Tensor, ...], tuple[int, ...]]:
    """Prepare-time join of sibling int4 layers that read one input (q, k and v;
    gate and up): their `_int4_pack` tuples stacked along the outputs, so that one
    kernel launch streams every sibling's weight, and each sibling's output count.
    The int4 form of the reference's joins of sibling `F.linear` and 8-bit layers
    (`src/backend/torch_source.cpp:77-158`, weights laid out one after another by
    `_adjacent`). Fused 3-tuples join as one 3-tuple (same group; the joined copy
    holds the siblings' bytes again, like `_adjacent` where the runtime did not
    place them together); dequantized 1-tuples as one dequantized weight."""
    if not packs:
        raise LinnetError("_int4_join: no layers")
    kinds = {len(p) for p in packs}
    if len(kinds) != 1:
        raise LinnetError("_int4_join: the siblings were prepared differently (fused and dequantized)")
    rows = tuple(int(p[0].shape[0]) for p in packs)
    if kinds == {3}:
        if len({tuple(p[0].shape[1:]) for p in packs}) != 1 or len({p[1].dtype for p in packs}) != 1:
            raise LinnetError("_int4_join: siblings share In, the group and the scale dtype")
        return tuple(torch.cat([p[i] for p in packs], dim=0) for i in range(3)), rows
    if len({p[0].shape[1] for p in packs}) != 1:
        raise LinnetError("_int4_join: siblings share In")
    return (torch.cat([p[0] for p in packs], dim=0),), rows


def _int4_split(y: torch.Tensor, rows: tuple[int, ...]) -> list[torch.Tensor]:
    """The siblings' outputs of a joined product (`y[..., a:b]` views, no copy)."""
    out, start = [], 0
    for n in rows:
        out.append(y[..., start : start + n])
        start += n
    return out


def _mxfp4_experts(x: torch.Tensor, blocks: torch.Tensor, scales: torch.Tensor, experts: torch.Tensor) -> torch.Tensor:
    """`std.quant::mxfp4_experts` as the generated module calls it
    (`torch_source.cpp:426-438, 1579-1600`): the chosen experts' MXFP4 bytes read as
    they are by one HIP kernel. The reference takes its kernel for up to 32 (row,
    slot) pairs and otherwise gathers the chosen experts as f32 weights; the HIP
    kernel runs at any count here (each pair still reads its own expert's bytes,
    never a widened copy). `x` is [R, K, In], or [R, 1, In] expanded by the caller
    for the shared form."""
    if not x.is_cuda:
        raise LinnetError("_mxfp4_experts: linnet_amd runs on the GPU; x is on " + str(x.device))
    return kernels.mxfp4_experts(x, blocks, scales, experts)


def _mxfp4_grouped(x: torch.Tensor, blocks: torch.Tensor, scales: torch.Tensor, experts: torch.Tensor,
                   weights: torch.Tensor | None = None) -> torch.Tensor:
    """`std.quant::mxfp4_linear_experts_shared` (no `weights`, `x` [R, In]: every
    chosen expert of a row reads the row) and `mxfp4_combine_experts` (`x` [R, K, In],
    the products weighed by `weights` [R, K] and summed per row in f32, as the
    reference's helper sums its grouped product, `torch_source.cpp:1705-1735`).
    The MXFP4 products run on the decode kernel, each (row, slot) pair reading its
    expert's bytes as stored: the semantics of the grouped path for any number of
    rows, without its expert-sorted MFMA schedule (each pair reads its expert again,
    from the caches past the first)."""
    if not x.is_cuda:
        raise LinnetError("_mxfp4_grouped: linnet_amd runs on the GPU; x is on " + str(x.device))
    rows, chosen = experts.shape
    if weights is None:
        if x.dim() != 2 or x.shape[0] != rows:
            raise LinnetError(f"_mxfp4_grouped: the shared form takes x [R, In] with R = {rows}")
        return kernels.mxfp4_experts(x[:, None, :].expand(rows, chosen, x.shape[1]), blocks, scales, experts)
    if x.dim() != 3 or tuple(x.shape[:2]) != (rows, chosen) or tuple(weights.shape) != (rows, chosen):
        raise LinnetError("_mxfp4_grouped: the combine form takes x [R, K, In] and weights [R, K]")
    y = kernels.mxfp4_experts(x, blocks, scales, experts)
    return (y.float() * weights.float()[..., None]).sum(1).to(x.dtype)
