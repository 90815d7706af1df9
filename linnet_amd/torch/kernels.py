"""PyTorch-facing wrappers of the HIP kernels, named as the reference's
`linnet.torch.kernels` names its Triton ones (`python/linnet/src/linnet/torch/kernels.py`).

Each wrapper checks shapes, dtypes and the device on the host, allocates the
output with PyTorch on the tensors' device, and calls the C ABI on PyTorch's
current stream: work is enqueued and never waited for, so every call may be
captured into a HIP graph. CPU tensors, or a missing library, raise
`LinnetError`: there is no CPU fallback.
"""

from __future__ import annotations

import ctypes
import dataclasses
import functools

import torch

from .. import _lib
from ..errors import LinnetError

_CODES = {torch.bfloat16: _lib.BF16, torch.float16: _lib.F16, torch.float32: _lib.F32}
_HALF = (torch.bfloat16, torch.float16)
KERNELS = {
    "auto": _lib.KERNEL_AUTO,
    "skinny": _lib.KERNEL_SKINNY,
    "tiled": _lib.KERNEL_TILED,
    "gemv": _lib.KERNEL_GEMV,
    "tiled128": _lib.KERNEL_TILED_128,
    "tiled256": _lib.KERNEL_TILED_256,
    "persistent": _lib.KERNEL_PERSISTENT,
    "split": _lib.KERNEL_SPLIT,
}
_KERNEL_NAMES = {code: name for name, code in KERNELS.items()}


def _ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _on_gpu(what: str, *tensors: torch.Tensor | None) -> torch.device:
    device: torch.device | None = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise LinnetError(f"{what}: the HIP kernels take GPU tensors, got one on {t.device}")
        if device is None:
            device = t.device
        elif t.device != device:
            raise LinnetError(f"{what}: tensors on {device} and {t.device}")
    assert device is not None
    return device


def _code(dtype: torch.dtype, what: str, allowed: tuple[torch.dtype, ...] = _HALF) -> int:
    if dtype not in allowed:
        raise LinnetError(f"{what}: dtype {dtype} is not one of {', '.join(map(str, allowed))}")
    return _CODES[dtype]


# ------------------------------------------------------------------ int4 groups


def int4_linear(
    x: torch.Tensor,
    packed: torch.Tensor,
    scale: torch.Tensor,
    zero: torch.Tensor,
    bias: torch.Tensor | None = None,
    kernel: str = "auto",
    out: torch.Tensor | None = None,
    order: torch.Tensor | None = None,
) -> torch.Tensor:
    """`F.linear(x, W) (+ bias)` for `x` [rows, In] (bf16 or f16) and the group-wise
    4-bit weight of `std.quant::linear_int4_groups` -- `packed` ([Out, Groups,
    Group/2] u8, the even value low), `scale` ([Out, Groups], x's dtype) and `zero`
    ([Out, Groups] u8) -- read once from HBM as they are stored. One row runs the
    one-token GEMV (one workgroup per CU) where its shape limits allow, few rows the
    skinny MFMA kernel, many the LDS-tiled dequant-GEMM (`kernel` may force one).
    In is a multiple of 128; the group is 32, 64 or a multiple of 128. `out`, if
    given, is a contiguous [rows, Out] tensor of x's dtype on x's device that
    receives the result (and is returned) instead of a new one.

    `order` ([In] int32, GPTQ's activation order) multiplies `take_inputs(x, order)`
    instead of x, as `Int4GroupLinear.forward` does (`stdlib/quant.linnet:163-174`):
    one row at group 128 gathers inside the one-token GEMV, other calls gather
    first with `take_inputs`'s kernel.

    Replaces `kernels.py:277-323` (`int4_linear`) and tinygemm's
    `aten._weight_int4pack_mm` (`src/backend/torch_source.cpp:1556-1558`)."""
    device = _on_gpu("int4_linear", x, packed, scale, zero, bias, order)
    if x.dim() != 2 or packed.dim() != 3:
        raise LinnetError(f"int4_linear: x is [rows, In] and packed [Out, Groups, Group/2], got {tuple(x.shape)} and {tuple(packed.shape)}")
    rows, depth = x.shape
    width, groups, half = packed.shape
    group = 2 * half
    if groups * group != depth:
        raise LinnetError(f"int4_linear: packed {tuple(packed.shape)} does not hold In={depth}")
    if packed.dtype != torch.uint8 or zero.dtype != torch.uint8:
        raise LinnetError("int4_linear: packed and zero are uint8")
    if tuple(scale.shape) != (width, groups) or tuple(zero.shape) != (width, groups):
        raise LinnetError(f"int4_linear: scale and zero are [{width}, {groups}]")
    code = _code(x.dtype, "int4_linear")
    if scale.dtype != x.dtype or (bias is not None and bias.dtype != x.dtype):
        raise LinnetError("int4_linear: scale and bias have x's dtype")
    if bias is not None and tuple(bias.shape) != (width,):
        raise LinnetError(f"int4_linear: bias is [{width}]")
    if kernel not in KERNELS:
        raise LinnetError(f"int4_linear: kernel is one of {', '.join(KERNELS)}")
    x = x.contiguous()
    packed, scale, zero = packed.contiguous(), scale.contiguous(), zero.contiguous()
    bias = None if bias is None else bias.contiguous()
    if out is None:
        y = torch.empty(rows, width, dtype=x.dtype, device=device)
    else:
        if tuple(out.shape) != (rows, width) or out.dtype != x.dtype or out.device != device or not out.is_contiguous():
            raise LinnetError(f"int4_linear: out is a contiguous [{rows}, {width}] {x.dtype} tensor on {device}")
        y = out
    if order is not None:
        if order.dtype != torch.int32 or tuple(order.shape) != (depth,):
            raise LinnetError(f"int4_linear: order is [{depth}] int32")
        order = order.contiguous()
        taken = torch.empty_like(x)
        with torch.cuda.device(device):
            _lib.call(
                "lnq_int4_linear_ordered", _ptr(x), _ptr(order), _ptr(packed), _ptr(scale), _ptr(zero), _ptr(bias),
                _ptr(y), _ptr(taken), rows, depth, width, group, code, KERNELS[kernel], _stream(device),
            )
        return y
    with torch.cuda.device(device):
        _, need = _workspace(rows, depth, width, group, code, KERNELS[kernel])
        if need:
            # The split GEMV's partial sums: memory of torch's caching allocator
            # (the graph pool under capture), freed when the call is enqueued.
            ws = torch.empty(need // 4, dtype=torch.float32, device=device)
            _lib.call(
                "lnq_int4_linear_ws", _ptr(x), _ptr(packed), _ptr(scale), _ptr(zero), _ptr(bias), _ptr(y),
                rows, depth, width, group, code, KERNELS[kernel], _ptr(ws), need, _stream(device),
            )
        else:
            _lib.call(
                "lnq_int4_linear", _ptr(x), _ptr(packed), _ptr(scale), _ptr(zero), _ptr(bias), _ptr(y),
                rows, depth, width, group, code, KERNELS[kernel], _stream(device),
            )
    return y


@dataclasses.dataclass
class XTiles:
    """Activations [rows, width] as x tiles (`lnq_x_tiles`): the matrix-core operand
    order of the few-row GEMVs, chunks of 32 rows, held flat in `data`."""

    data: torch.Tensor
    rows: int
    width: int

    @staticmethod
    def empty(rows: int, width: int, dtype: torch.dtype, device: torch.device) -> "XTiles":
        if width % 256:
            raise LinnetError(f"x tiles: the width {width} is not a multiple of 256")
        return XTiles(torch.empty(-(-rows // 32) * 32 * width, dtype=dtype, device=device), rows, width)

    @property
    def dtype(self) -> torch.dtype:
        return self.data.dtype

    @property
    def device(self) -> torch.device:
        return self.data.device

    def rows_major(self) -> torch.Tensor:
        """The [rows, width] tensor the tiles hold (a torch reordering, for tests)."""
        chunks = self.data.numel() // (32 * self.width)
        # chunk, s, b, H, t, j, c, then element e = e_lo + 4 e_hi at place 2 e_lo + e_hi
        t = self.data.view(chunks, self.width // 256, 2, 2, 4, 4, 16, 4, 2)
        t = t.permute(0, 2, 6, 1, 3, 4, 5, 8, 7).reshape(chunks * 32, self.width)
        return t[: self.rows]


def x_tiles(x: torch.Tensor) -> XTiles:
    """x [rows, width] (16-bit, width % 256 == 0) as x tiles."""
    device = _on_gpu("x_tiles", x)
    if x.dim() != 2 or x.element_size() != 2:
        raise LinnetError("x_tiles: x is a [rows, width] tensor of a 16-bit type")
    x = x.contiguous()
    xt = XTiles.empty(x.shape[0], x.shape[1], x.dtype, device)
    with torch.cuda.device(device):
        _lib.call("lnq_x_tiles", _ptr(x), _ptr(xt.data), x.shape[0], x.shape[1], _stream(device))
    return xt


def int4_linear_tiles(xt: XTiles, packed: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor,
                      bias: torch.Tensor | None = None, kernel: str = "auto",
                      out: torch.Tensor | None = None) -> torch.Tensor:
    """`int4_linear` of the activations held as x tiles (`lnq_int4_linear_tiles`):
    rows 1..64, the 32-row GEMV up to In = 4096, the split GEMV past it (a
    workspace of torch's) or when asked for. The bits of the same kernel on
    row-major x."""
    device = _on_gpu("int4_linear_tiles", xt.data, packed, scale, zero, bias)
    rows, depth = xt.rows, xt.width
    width, groups, half = packed.shape
    group = 2 * half
    if groups * group != depth:
        raise LinnetError(f"int4_linear_tiles: packed {tuple(packed.shape)} does not hold In={depth}")
    code = _code(xt.dtype, "int4_linear_tiles")
    if scale.dtype != xt.dtype or (bias is not None and bias.dtype != xt.dtype):
        raise LinnetError("int4_linear_tiles: scale and bias have x's dtype")
    if kernel not in ("auto", "gemv", "split"):
        raise LinnetError("int4_linear_tiles: kernel is auto, gemv or split")
    packed, scale, zero = packed.contiguous(), scale.contiguous(), zero.contiguous()
    bias = None if bias is None else bias.contiguous()
    if out is None:
        y = torch.empty(rows, width, dtype=xt.dtype, device=device)
    else:
        if tuple(out.shape) != (rows, width) or out.dtype != xt.dtype or out.device != device or not out.is_contiguous():
            raise LinnetError(f"int4_linear_tiles: out is a contiguous [{rows}, {width}] {xt.dtype} tensor on {device}")
        y = out
    with torch.cuda.device(device):
        need = 0
        if kernel == "split" or depth > 4096:
            _, need = _workspace(rows, depth, width, group, code, _lib.KERNEL_SPLIT)
        ws = torch.empty(max(need, 16) // 4, dtype=torch.float32, device=device) if need else None
        _lib.call(
            "lnq_int4_linear_tiles", _ptr(xt.data), _ptr(packed), _ptr(scale), _ptr(zero), _ptr(bias), _ptr(y),
            rows, depth, width, group, code, KERNELS[kernel], _ptr(ws), need, _stream(device),
        )
    return y


@dataclasses.dataclass
class SplitParts:
    """The K chunks' f32 partial sums [splits, rows, out] of a split product
    (`lnq_int4_linear_tiles_parts`), left for a consumer that adds them in chunk
    order and rounds once (`decode.rmsnorm` takes them as its residual delta)."""

    data: torch.Tensor

    def total(self, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
        """The product they make: the chunks added in order, rounded once (torch ops)."""
        v = self.data[0].clone()
        for part in self.data[1:]:
            v += part
        return v.to(dtype)


def int4_linear_tiles_parts(xt: XTiles, packed: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor) -> SplitParts:
    """The split GEMV of `int4_linear_tiles` (1..32 rows, In > 4096, no bias)
    without its reduction: the chunks' partial sums, whose ordered sum rounded
    once is `int4_linear_tiles`'s output bit for bit."""
    device = _on_gpu("int4_linear_tiles_parts", xt.data, packed, scale, zero)
    rows, depth = xt.rows, xt.width
    width, groups, half = packed.shape
    group = 2 * half
    if groups * group != depth:
        raise LinnetError(f"int4_linear_tiles_parts: packed {tuple(packed.shape)} does not hold In={depth}")
    code = _code(xt.dtype, "int4_linear_tiles_parts")
    if scale.dtype != xt.dtype:
        raise LinnetError("int4_linear_tiles_parts: scale has x's dtype")
    packed, scale, zero = packed.contiguous(), scale.contiguous(), zero.contiguous()
    with torch.cuda.device(device):
        _, need = _workspace(rows, depth, width, group, code, _lib.KERNEL_SPLIT)
        parts = torch.empty(max(need, 16) // 4, dtype=torch.float32, device=device)
        splits = ctypes.c_int32(0)
        _lib.call("lnq_int4_linear_tiles_parts", _ptr(xt.data), _ptr(packed), _ptr(scale), _ptr(zero), _ptr(parts),
                  need, rows, depth, width, group, code, ctypes.byref(splits), _stream(device))
    return SplitParts(parts[: splits.value * rows * width].view(splits.value, rows, width))


@functools.lru_cache(maxsize=4096)
def _workspace(rows: int, depth: int, width: int, group: int, code: int, kernel: int) -> tuple[int, int]:
    """(kernel code, workspace bytes) `lnq_int4_linear_ws` takes for the shape."""
    chosen, need = ctypes.c_int32(-1), ctypes.c_int64(0)
    _lib.call("lnq_int4_linear_workspace", rows, depth, width, group, code, kernel, ctypes.byref(chosen),
              ctypes.byref(need))
    return chosen.value, need.value


def _prologue_linear(what: str, prologue: int, x: torch.Tensor, operand: torch.Tensor, eps: float,
                     packed: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor, bias: torch.Tensor | None,
                     out: torch.Tensor | None) -> torch.Tensor:
    device = _on_gpu(what, x, operand, packed, scale, zero, bias)
    if x.dim() != 2 or packed.dim() != 3 or x.dtype != torch.bfloat16:
        raise LinnetError(f"{what}: x is [rows, In] bf16 and packed [Out, Groups, Group/2]")
    rows, depth = x.shape
    width, groups, half = packed.shape
    if groups * 2 * half != depth or packed.dtype != torch.uint8 or zero.dtype != torch.uint8:
        raise LinnetError(f"{what}: packed {tuple(packed.shape)} (uint8) does not hold In={depth}")
    if scale.dtype != torch.bfloat16 or tuple(scale.shape) != (width, groups) or tuple(zero.shape) != (width, groups):
        raise LinnetError(f"{what}: scale is [{width}, {groups}] bf16 and zero [{width}, {groups}] uint8")
    if bias is not None and (bias.dtype != torch.bfloat16 or tuple(bias.shape) != (width,)):
        raise LinnetError(f"{what}: bias is [{width}] bf16")
    x, operand = x.contiguous(), operand.contiguous()
    packed, scale, zero = packed.contiguous(), scale.contiguous(), zero.contiguous()
    bias = None if bias is None else bias.contiguous()
    if out is None:
        y = torch.empty(rows, width, dtype=x.dtype, device=device)
    elif tuple(out.shape) != (rows, width) or out.dtype != x.dtype or out.device != device or not out.is_contiguous():
        raise LinnetError(f"{what}: out is a contiguous [{rows}, {width}] bf16 tensor on {device}")
    else:
        y = out
    # The staging buffer, used where the prologue is not fused (more rows, another
    # group, an In no one-token kernel takes); one row's is a few KB.
    staged = torch.empty_like(x)
    norm = prologue == _lib.PROLOGUE_RMSNORM
    with torch.cuda.device(device):
        _lib.call("lnq_int4_linear_prologue", _ptr(x), None if norm else _ptr(operand), _ptr(operand) if norm else None,
                  float(eps), prologue, _ptr(packed), _ptr(scale), _ptr(zero), _ptr(bias), _ptr(y), _ptr(staged),
                  rows, depth, width, 2 * half, _lib.BF16, _lib.KERNEL_AUTO, _stream(device))
    return y


def int4_linear_rmsnorm(x: torch.Tensor, norm_weight: torch.Tensor, eps: float, packed: torch.Tensor,
                        scale: torch.Tensor, zero: torch.Tensor, bias: torch.Tensor | None = None,
                        out: torch.Tensor | None = None) -> torch.Tensor:
    """`int4_linear(rmsnorm(x, norm_weight, eps), ...)` (bf16; norm_weight f32 [In]):
    one row at group 128 in one kernel, the norm folded into the one-token GEMV as
    `r * (W (x * w))` (r = rsqrt(mean(x^2) + eps), the row's factor; x * w rounded
    to bf16 where `decode.rmsnorm` rounds x * r * w); more rows normalise first.
    With one row, `bias` = the residual stream's row gives residual + product (the
    residual add of the next layer, rounded as it rounds)."""
    if norm_weight.dtype != torch.float32 or tuple(norm_weight.shape) != (x.shape[-1],):
        raise LinnetError("int4_linear_rmsnorm: norm_weight is f32 [In]")
    return _prologue_linear("int4_linear_rmsnorm", _lib.PROLOGUE_RMSNORM, x, norm_weight, eps, packed, scale, zero,
                            bias, out)


def int4_linear_silu_mul(g: torch.Tensor, u: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor,
                         zero: torch.Tensor, bias: torch.Tensor | None = None,
                         out: torch.Tensor | None = None) -> torch.Tensor:
    """`int4_linear(silu(g) * u, ...)` (bf16, g and u [rows, In]): the MLP's down
    projection with SiLU(gate) * up folded into the one-token GEMV's staging of x
    (one row, group 128; the bits of `decode.silu_mul` then `int4_linear`); more
    rows compute the product first. `bias` as for `int4_linear_rmsnorm`."""
    if u.shape != g.shape or u.dtype != torch.bfloat16:
        raise LinnetError("int4_linear_silu_mul: u is bf16 of g's shape")
    return _prologue_linear("int4_linear_silu_mul", _lib.PROLOGUE_SILU_MUL, g, u, 0.0, packed, scale, zero, bias, out)


def take_inputs(x: torch.Tensor, order: torch.Tensor) -> torch.Tensor:
    """`std.quant::take_inputs` (`stdlib/quant.linnet:142-149`): `x[..., order[k]]`
    over x's last axis, in one HIP gather kernel; `order` is [N] int32 (the
    reference runs `x.index_select(-1, order.long())`,
    `src/backend/torch_source.cpp:397-398`). An index outside [0, N) reads 0."""
    device = _on_gpu("take_inputs", x, order)
    code = _code(x.dtype, "take_inputs", (torch.bfloat16, torch.float16, torch.float32))
    n = x.shape[-1] if x.dim() else 0
    if x.dim() == 0 or order.dtype != torch.int32 or tuple(order.shape) != (n,):
        raise LinnetError(f"take_inputs: order is [{n}] int32 over x's last axis")
    x, order = x.contiguous(), order.contiguous()
    taken = torch.empty_like(x)
    with torch.cuda.device(device):
        _lib.call("lnq_take_inputs", _ptr(x), _ptr(order), _ptr(taken), x.numel() // max(n, 1), n, code,
                  _stream(device))
    return taken


def int4_linear_plan(rows: int, in_features: int, out_features: int, group: int,
                     dtype: torch.dtype = torch.bfloat16, kernel: str = "auto") -> str:
    """The kernel `int4_linear` runs for this shape on the current device: "gemv"
    (33..64 rows: the few-token GEMV per 32-row chunk), "skinny", "split" (the
    32-row GEMV with K split over workgroups, a workspace of torch's), "tiled128",
    "tiled256" or "persistent". Raises as `int4_linear` would for a shape it refuses."""
    if kernel not in KERNELS:
        raise LinnetError(f"int4_linear_plan: kernel is one of {', '.join(KERNELS)}")
    chosen, _ = _workspace(rows, in_features, out_features, group, _code(dtype, "int4_linear_plan"), KERNELS[kernel])
    return _KERNEL_NAMES[chosen]


def int4_weight(raw: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor) -> torch.Tensor:
    """The weight dequantized, in `scale`'s dtype (bf16, f16 or f32), in one kernel:
    `(q - z) * s` in f32, rounded once -- bit for bit the reference's `_int4_weight`
    (`src/backend/torch_source.cpp:1536-1550`). Any even group."""
    device = _on_gpu("int4_weight", raw, scale, zero)
    width, groups, half = raw.shape
    code = _code(scale.dtype, "int4_weight", (torch.bfloat16, torch.float16, torch.float32))
    if raw.dtype != torch.uint8 or zero.dtype != torch.uint8:
        raise LinnetError("int4_weight: packed and zero are uint8")
    if tuple(scale.shape) != (width, groups) or tuple(zero.shape) != (width, groups):
        raise LinnetError(f"int4_weight: scale and zero are [{width}, {groups}]")
    raw, scale, zero = raw.contiguous(), scale.contiguous(), zero.contiguous()
    out = torch.empty(width, groups * 2 * half, dtype=scale.dtype, device=device)
    with torch.cuda.device(device):
        _lib.call("lnq_int4_dequantize", _ptr(raw), _ptr(scale), _ptr(zero), _ptr(out),
                  width, groups * 2 * half, 2 * half, code, _stream(device))
    return out


def quantize_int4(weight: torch.Tensor, group: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """`(packed [Out, In/group, group/2] u8, scale [Out, In/group] f32, zero u8)` of an
    f32 `[Out, In]` weight, rounded as `linnet.quant.quantize_int4_groups`
    (`python/linnet/src/linnet/quant.py:83-99`), bit for bit."""
    device = _on_gpu("quantize_int4", weight)
    if weight.dim() != 2:
        raise LinnetError(f"a linear weight is [Out, In]; this one is {list(weight.shape)}")
    width, depth = weight.shape
    if group <= 0 or group % 2 != 0 or depth % group != 0:
        raise LinnetError(f"groups of {group} must be even and divide the {depth} inputs")
    w = weight.to(torch.float32).contiguous()
    packed = torch.empty(width, depth // group, group // 2, dtype=torch.uint8, device=device)
    scale = torch.empty(width, depth // group, dtype=torch.float32, device=device)
    zero = torch.empty(width, depth // group, dtype=torch.uint8, device=device)
    with torch.cuda.device(device):
        _lib.call("lnq_int4_quantize", _ptr(w), _ptr(packed), _ptr(scale), _ptr(zero),
                  width, depth, group, _stream(device))
    return packed, scale, zero


def pack4(codes: torch.Tensor) -> torch.Tensor:
    """Integer codes (wrapped to 4 bits) two a byte along the last axis, low first
    (`torch/packed.py:61-75` for `i4`/`u4`)."""
    device = _on_gpu("pack4", codes)
    if codes.shape[-1] % 2:
        raise LinnetError(f"a 4-bit tensor's last axis is even, found shape {tuple(codes.shape)}")
    if codes.is_floating_point():
        codes = codes.trunc().to(torch.int64)
    as_bytes = (codes.to(torch.int64) & 15).to(torch.uint8).contiguous()
    out = torch.empty(*codes.shape[:-1], codes.shape[-1] // 2, dtype=torch.uint8, device=device)
    with torch.cuda.device(device):
        _lib.call("lnq_int4_pack", _ptr(as_bytes), _ptr(out), out.numel(), _stream(device))
    return out


def unpack4(packed: torch.Tensor, kind: str) -> torch.Tensor:
    """Packed bytes widened: `u4` codes as uint8, `i4` sign-extended to int8
    (`torch/packed.py:27-35`)."""
    device = _on_gpu("unpack4", packed)
    if kind not in ("u4", "i4"):
        raise LinnetError(f"`{kind}` is not an integer 4-bit format (i4, u4)")
    if packed.dtype != torch.uint8:
        raise LinnetError("unpack4: packed is uint8")
    packed = packed.contiguous()
    dtype = torch.int8 if kind == "i4" else torch.uint8
    out = torch.empty(*packed.shape[:-1], 2 * packed.shape[-1], dtype=dtype, device=device)
    with torch.cuda.device(device):
        _lib.call("lnq_int4_unpack", _ptr(packed), _ptr(out), packed.numel(), int(kind == "i4"), _stream(device))
    return out


def int4_row_prepare(weight: torch.Tensor, scale: torch.Tensor, group: int = 128
                     ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """`std.quant::Int4Linear`'s weight (`weight` [Out, In/2] u8 of signed 4-bit
    values, element 2k low; `scale` [Out] or [Out, 1], bf16 / f16 / f32) in the group
    layout `int4_linear` reads: `(packed [Out, In/group, group/2], scale [Out,
    In/group], zero [Out, In/group] = 8)`, each code the value plus 8, so the layer's
    weight `q * scale` is unchanged (`stdlib/quant.linnet:24-29, 101-111`)."""
    device = _on_gpu("int4_row_prepare", weight, scale)
    if weight.dtype != torch.uint8 or weight.dim() != 2:
        raise LinnetError("int4_row_prepare: the weight is [Out, In/2] uint8 bytes of i4 values")
    width, depth = weight.shape[0], 2 * weight.shape[1]
    code = _code(scale.dtype, "int4_row_prepare", (torch.bfloat16, torch.float16, torch.float32))
    if scale.numel() != width:
        raise LinnetError(f"int4_row_prepare: one scale a row ({width}), got {tuple(scale.shape)}")
    if depth % 32 or group <= 0 or group % 2 or depth % group:
        raise LinnetError(f"int4_row_prepare: In={depth} is a multiple of 32 split into even groups of {group}")
    weight, scale = weight.contiguous(), scale.contiguous()
    packed = torch.empty(width, depth // group, group // 2, dtype=torch.uint8, device=device)
    group_scale = torch.empty(width, depth // group, dtype=scale.dtype, device=device)
    zero = torch.empty(width, depth // group, dtype=torch.uint8, device=device)
    with torch.cuda.device(device):
        _lib.call("lnq_int4_row_prepare", _ptr(weight), _ptr(scale), _ptr(packed), _ptr(group_scale), _ptr(zero),
                  width, depth, group, code, _stream(device))
    return packed, group_scale, zero


def int4_repack(
    qweight: torch.Tensor,
    qzeros: torch.Tensor,
    packing: str,
    group: int,
    zero_offset: int = 0,
    order: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """A GPTQ (`qweight [In/8, Out]`) or AWQ (`qweight [In, Out/8]`) layer's int32 codes
    and `qzeros [In/group, Out/8]` as Int4GroupLinear's `(packed [Out, In/group,
    group/2] u8, zero [Out, In/group] u8)`; `order` (GPTQ in activation order, [In]
    int32) picks the checkpoint input each input of the result is. The repack of
    `import_quantized` (`python/linnet/src/linnet/quant.py:222-240, 300-340`)."""
    device = _on_gpu("int4_repack", qweight, qzeros, order)
    kinds = {"gptq": _lib.PACKING_GPTQ, "awq": _lib.PACKING_AWQ}
    if packing not in kinds:
        raise LinnetError(f"int4_repack: packing `{packing}` is neither gptq nor awq")
    if qweight.dtype != torch.int32 or qzeros.dtype != torch.int32 or qweight.dim() != 2 or qzeros.dim() != 2:
        raise LinnetError("int4_repack: qweight and qzeros are 2-D int32")
    if packing == "gptq":
        in_features, out_features = qweight.shape[0] * 8, qweight.shape[1]
    else:
        in_features, out_features = qweight.shape[0], qweight.shape[1] * 8
    if group <= 0 or in_features % group or group % 2:
        raise LinnetError(f"int4_repack: {in_features} inputs do not make even groups of {group}")
    groups = in_features // group
    if in_features % 8 or tuple(qzeros.shape) != (groups, out_features // 8):
        raise LinnetError(f"int4_repack: qzeros is [{groups}, {out_features // 8}], got {tuple(qzeros.shape)}")
    if order is not None:
        if packing != "gptq" or order.dtype != torch.int32 or tuple(order.shape) != (in_features,):
            raise LinnetError(f"int4_repack: an order is GPTQ's, [{in_features}] int32")
        order = order.contiguous()
        # The kernel reads whatever input an entry names (an entry out of range as
        # code 0): only a permutation gives the layer's weights, so anything else
        # is refused here, at load time (one host sync). A call being captured
        # into a graph cannot wait for the device: it is checked when the order is
        # first used eagerly, not while captured.
        if not torch.cuda.is_current_stream_capturing() and not torch.equal(
            torch.sort(order).values, torch.arange(in_features, dtype=torch.int32, device=device)
        ):
            raise LinnetError(f"int4_repack: order is not a permutation of 0..{in_features - 1}")
    if zero_offset not in (0, 1):
        raise LinnetError(f"int4_repack: zero_offset is 0 or 1, not {zero_offset}")
    qweight, qzeros = qweight.contiguous(), qzeros.contiguous()
    packed = torch.empty(out_features, groups, group // 2, dtype=torch.uint8, device=device)
    zero = torch.empty(out_features, groups, dtype=torch.uint8, device=device)
    with torch.cuda.device(device):
        _lib.call("lnq_int4_repack", _ptr(qweight), _ptr(qzeros), _ptr(order), kinds[packing], zero_offset,
                  in_features, out_features, groups, _ptr(packed), _ptr(zero), _stream(device))
    return packed, zero


# ------------------------------------------------------------------------ MXFP4


def mxfp4_experts(x: torch.Tensor, blocks: torch.Tensor, scales: torch.Tensor, experts: torch.Tensor) -> torch.Tensor:
    """`y[r, k, o] = sum_i x[r, k, i] * W[experts[r, k], o, i]`, with `W` the MXFP4
    weights `blocks` ([E, Out, G, 16] u8) and `scales` ([E, Out, G] u8, E8M0)
    read as they are and widened in registers (`torch/kernels.py:94-209`). `x` is
    [R, K, In] bf16 or f16 (an expanded view with a zero slot stride, for an input
    the chosen experts share, is read without a copy)."""
    device = _on_gpu("mxfp4_experts", x, blocks, scales, experts)
    if x.dim() != 3 or blocks.dim() != 4 or scales.dim() != 3 or experts.dim() != 2:
        raise LinnetError("mxfp4_experts: x [R, K, In], blocks [E, Out, G, 16], scales [E, Out, G], experts [R, K]")
    rows, chosen, width = x.shape
    count, out_features, groups, sixteen = blocks.shape
    if sixteen != 16 or blocks.dtype != torch.uint8 or scales.dtype != torch.uint8:
        raise LinnetError("mxfp4_experts: blocks are [E, Out, G, 16] and scales [E, Out, G], both uint8")
    if tuple(scales.shape) != (count, out_features, groups) or width != groups * 32:
        raise LinnetError(f"mxfp4_experts: x's In={width}, blocks {tuple(blocks.shape)}, scales {tuple(scales.shape)}")
    if tuple(experts.shape) != (rows, chosen) or experts.is_floating_point():
        raise LinnetError(f"mxfp4_experts: experts are integers [{rows}, {chosen}]")
    code = _code(x.dtype, "mxfp4_experts")
    if (x.stride(2) != 1 or x.data_ptr() % 16 or x.stride(0) % 8 or x.stride(1) % 8):
        x = x.contiguous()
    blocks, scales = blocks.contiguous(), scales.contiguous()
    ids = experts.to(torch.int64).contiguous()
    y = torch.empty(rows, chosen, out_features, dtype=x.dtype, device=device)
    with torch.cuda.device(device):
        _lib.call("lnq_mxfp4_experts", _ptr(x), x.stride(0), x.stride(1), _ptr(blocks), _ptr(scales), _ptr(ids),
                  _ptr(y), rows, chosen, count, out_features, width, code, _stream(device))
    return y


# ------------------------------------------------------------------------ 8-bit


def _scale_columns(weight: torch.Tensor, scale: torch.Tensor, group: int, row_block: int) -> None:
    width, depth = weight.shape
    if group == 0:
        if scale.numel() != width:
            raise LinnetError(f"one scale a row: {width} scales, got {tuple(scale.shape)}")
    else:
        if depth % group or width % row_block:
            raise LinnetError(f"scales of {row_block}x{group} blocks do not tile [{width}, {depth}]")
        if tuple(scale.shape) != (width // row_block, depth // group):
            raise LinnetError(f"scale is [{width // row_block}, {depth // group}], got {tuple(scale.shape)}")


def _bytes(weight: torch.Tensor) -> torch.Tensor:
    if weight.dtype == torch.float8_e4m3fn:
        return weight.contiguous().view(torch.uint8)
    if weight.dtype in (torch.int8, torch.uint8):
        return weight.contiguous().view(torch.uint8)
    raise LinnetError(f"8-bit weights are int8 or float8_e4m3fn (or their bytes), not {weight.dtype}")


def w8a16(x: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor, fp8: bool, group: int = 0, row_block: int = 1) -> torch.Tensor:
    """`F.linear(x, W)` for `x` [rows, In] (bf16/f16) and 8-bit weights [Out, In]
    (FP8 E4M3 bits or int8) times `scale` (f32; one a row when `group` is 0, else
    [Out/row_block, In/group]), widened in registers, x unrounded.
    Replaces `kernels.py:437-592` (`w8a16`) and, for one row, `gemv8` (`:375-434`)."""
    device = _on_gpu("w8a16", x, weight, scale)
    rows, depth = x.shape
    width = weight.shape[0]
    if weight.shape[1] != depth:
        raise LinnetError(f"w8a16: weight {tuple(weight.shape)} does not take In={depth}")
    _scale_columns(weight, scale, group, row_block)
    code = _code(x.dtype, "w8a16")
    if scale.dtype != torch.float32:
        raise LinnetError("w8a16: scales are f32 (the operands' form)")
    x, wb, scale = x.contiguous(), _bytes(weight), scale.contiguous()
    y = torch.empty(rows, width, dtype=x.dtype, device=device)
    with torch.cuda.device(device):
        _lib.call("lnq_w8a16", _ptr(x), _ptr(wb), _ptr(scale), _ptr(y), rows, width, depth,
                  int(fp8), group, row_block, code, _stream(device))
    return y


def gemv8(x: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor, fp8: bool, group: int = 0, row_block: int = 1) -> torch.Tensor:
    """One row `x` [1, In] times 8-bit weights (`kernels.py:375-434`): `w8a16` at one row."""
    if x.shape[0] != 1:
        raise LinnetError(f"gemv8 takes one row, got {x.shape[0]}")
    return w8a16(x, weight, scale, fp8, group, row_block)


def dequantize8(weight: torch.Tensor, scale: torch.Tensor, fp8: bool, group: int, row_block: int, dtype: torch.dtype) -> torch.Tensor:
    """The 8-bit weight widened, times its scale in f32, rounded to `dtype`
    (`kernels.py:595-666`)."""
    device = _on_gpu("dequantize8", weight, scale)
    width, depth = weight.shape
    _scale_columns(weight, scale, group, row_block)
    code = _code(dtype, "dequantize8", (torch.bfloat16, torch.float16, torch.float32))
    wb, scale = _bytes(weight), scale.to(torch.float32).contiguous()
    out = torch.empty(width, depth, dtype=dtype, device=device)
    with torch.cuda.device(device):
        _lib.call("lnq_dequantize8", _ptr(wb), _ptr(scale), _ptr(out), width, depth, int(fp8),
                  group, row_block, code, _stream(device))
    return out


def _rows8(x: torch.Tensor, fp8: bool) -> tuple[torch.Tensor, torch.Tensor]:
    device = _on_gpu("rows8", x)
    rows, depth = x.shape
    code = _code(x.dtype, "rows8", (torch.bfloat16, torch.float16, torch.float32))
    x = x.contiguous()
    q = torch.empty(rows, depth, dtype=torch.float8_e4m3fn if fp8 else torch.int8, device=device)
    scale = torch.empty(rows, 1, dtype=torch.float32, device=device)
    with torch.cuda.device(device):
        _lib.call("lnq_rows8", _ptr(x), _ptr(q), _ptr(scale), rows, depth, int(fp8), code, _stream(device))
    return q, scale


def fp8_rows(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Each row of `x` rounded to FP8 E4M3 with a scale of its own (`kernels.py:669-753`):
    the rows and the scales ([rows, 1], f32)."""
    return _rows8(x, True)


def int8_rows(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Each row of `x` rounded to int8 with a scale of its own (`kernels.py:669-753`)."""
    return _rows8(x, False)


def _mm8(q: torch.Tensor, weight: torch.Tensor, x_scale: torch.Tensor, scale: torch.Tensor, dtype: torch.dtype, fp8: bool,
         tile_n: int = 0) -> torch.Tensor:
    device = _on_gpu("mm8", q, weight, x_scale, scale)
    if tile_n not in (0, MM8_PERSISTENT, MM8_STREAM, 128, 256):
        raise LinnetError(f"mm8: tile_n is 0 (automatic), 1 (persistent), 2 (streaming), 128 or 256, not {tile_n}")
    rows, depth = q.shape
    width = weight.shape[0]
    if weight.shape[1] != depth:
        raise LinnetError(f"mm8: weight {tuple(weight.shape)} does not take In={depth}")
    if x_scale.numel() != rows or scale.numel() != width:
        raise LinnetError("mm8: one scale per row of x and per row of the weight")
    code = _code(dtype, "mm8")
    qb, wb = _bytes(q), _bytes(weight)
    xs = x_scale.to(torch.float32).contiguous()
    ws = scale.to(torch.float32).contiguous()
    y = torch.empty(rows, width, dtype=dtype, device=device)
    with torch.cuda.device(device):
        _lib.call("lnq_mm8_tiles", _ptr(qb), _ptr(wb), _ptr(xs), _ptr(ws), _ptr(y), rows, width, depth,
                  int(fp8), code, tile_n, _stream(device))
    return y


# `tile_n` naming the persistent 256 x 256 form of the 8-bit product, and its
# weight-streaming 256 x 128 form.
MM8_PERSISTENT = 1
MM8_STREAM = 2


def mm8_plan(rows: int, out_features: int, in_features: int, fp8: bool = True) -> int:
    """The kernel `fp8_mm` (fp8 True) or `int8_mm` takes for this shape on the
    current device: the tile width (128 or 256 output columns), MM8_PERSISTENT or
    MM8_STREAM."""
    tile = ctypes.c_int32(0)
    _lib.call("lnq_mm8_plan", rows, out_features, in_features, int(fp8), ctypes.byref(tile))
    return tile.value


def fp8_groups(x: torch.Tensor, group: int, padded: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Each `group` (128) inputs of each row of `x` [rows, In] rounded to FP8 E4M3 with
    a scale of their own, the rows padded with zeros (scale 1) to `padded`: `(q
    [padded, In] float8_e4m3fn, scales [padded, In/group] f32)`, the scales a
    column-major view (of a [In/group, padded] tensor) as the reference returns
    them (`torch/kernels.py:757-802`)."""
    device = _on_gpu("fp8_groups", x)
    if x.dim() != 2:
        raise LinnetError(f"fp8_groups: x is [rows, In], got {tuple(x.shape)}")
    rows, depth = x.shape
    code = _code(x.dtype, "fp8_groups", (torch.bfloat16, torch.float16, torch.float32))
    if group != 128 or depth % group:
        raise LinnetError(f"fp8_groups: groups of 128 dividing In={depth}, not {group}")
    if padded < rows:
        raise LinnetError(f"fp8_groups: padded {padded} < rows {rows}")
    x = x.contiguous()
    q = torch.empty(padded, depth, dtype=torch.float8_e4m3fn, device=device)
    scale = torch.empty(depth // group, padded, dtype=torch.float32, device=device)
    with torch.cuda.device(device):
        _lib.call("lnq_fp8_groups", _ptr(x), _ptr(q), _ptr(scale), rows, padded, depth, group, code, _stream(device))
    return q, scale.t()


def fp8_block_mm(q: torch.Tensor, weight: torch.Tensor, x_scale: torch.Tensor, scale: torch.Tensor,
                 dtype: torch.dtype) -> torch.Tensor:
    """The block-scaled FP8 product `torch._scaled_mm(q, weight.t(), scale_a=x_scale,
    scale_b=scale.t(), out_dtype=dtype)` computes for the reference
    (`torch/quantized.py:159-166`): `q` [rows, In] and `weight` [Out, In] FP8 E4M3,
    `x_scale` [rows, In/128] as `fp8_groups` returns it (a column-major view), `scale`
    [Out/128, In/128] f32; per 128-input block, the block's FP8 MFMA sums times
    both scales, added in f32, rounded once to `dtype`."""
    device = _on_gpu("fp8_block_mm", q, weight, x_scale, scale)
    rows, depth = q.shape
    width = weight.shape[0]
    if weight.shape[1] != depth or depth % 128 or width % 128:
        raise LinnetError(f"fp8_block_mm: weight {tuple(weight.shape)} against In={depth} (both % 128 == 0)")
    if tuple(scale.shape) != (width // 128, depth // 128):
        raise LinnetError(f"fp8_block_mm: scale is [{width // 128}, {depth // 128}], got {tuple(scale.shape)}")
    if tuple(x_scale.shape) != (rows, depth // 128):
        raise LinnetError(f"fp8_block_mm: x_scale is [{rows}, {depth // 128}], got {tuple(x_scale.shape)}")
    code = _code(dtype, "fp8_block_mm")
    # The kernel reads x_scale[b * stride + row]: a column-major [rows, In/128] view.
    xs = x_scale.to(torch.float32)
    if xs.stride(0) != 1 or (depth // 128 > 1 and xs.stride(1) < rows):
        xs = xs.t().contiguous().t()
    stride = xs.stride(1) if depth // 128 > 1 else max(rows, 1)
    qb, wb = _bytes(q.contiguous()), _bytes(weight.contiguous())
    ws = scale.to(torch.float32).contiguous()
    y = torch.empty(rows, width, dtype=dtype, device=device)
    with torch.cuda.device(device):
        _lib.call("lnq_mm8_block", _ptr(qb), _ptr(wb), _ptr(xs), stride, _ptr(ws), _ptr(y), rows, width, depth,
                  code, _stream(device))
    return y


def int8_mm(q: torch.Tensor, weight: torch.Tensor, x_scale: torch.Tensor, scale: torch.Tensor, dtype: torch.dtype,
            tile_n: int = 0) -> torch.Tensor:
    """`(q @ weight.T) * x_scale * scale` in `dtype` for int8 rows and int8 weights
    with one scale a row, summed exactly in int32 on MFMA (`kernels.py:805-915`).
    `tile_n` (128, 256, MM8_PERSISTENT or MM8_STREAM) names the kernel, 0 lets
    the library choose; every kernel gives the same bits."""
    return _mm8(q, weight, x_scale, scale, dtype, False, tile_n)


def fp8_mm(q: torch.Tensor, weight: torch.Tensor, x_scale: torch.Tensor, scale: torch.Tensor, dtype: torch.dtype,
           tile_n: int = 0) -> torch.Tensor:
    """`(q @ weight.T) * x_scale * scale` in `dtype` for FP8 E4M3 rows and weights on
    gfx950's FP8 MFMA, summed in f32: what `torch._scaled_mm(q, W.t(), scale_a,
    scale_b, out_dtype)` computes for the reference (`torch/quantized.py:129`).
    `tile_n` (128, 256, MM8_PERSISTENT or MM8_STREAM) names the kernel, 0 lets
    the library choose; every kernel gives the same bits."""
    return _mm8(q, weight, x_scale, scale, dtype, True, tile_n)


def quantize_int8(weight: torch.Tensor, group: int, dtype: str) -> tuple[torch.Tensor, torch.Tensor]:
    """`(q [Out, In] int8, scale [Out, In/group] f32)` as `linnet.quant.quantize_int8_groups`
    (`python/linnet/src/linnet/quant.py:102-121`), bit for bit."""
    device = _on_gpu("quantize_int8", weight)
    if weight.dim() != 2:
        raise LinnetError(f"a linear weight is [Out, In]; this one is {list(weight.shape)}")
    codes = {"bf16": _lib.BF16, "f16": _lib.F16, "f32": _lib.F32}
    if dtype not in codes:
        raise LinnetError(f"scales are stored as bf16, f16, or f32, not {dtype}")
    width, depth = weight.shape
    if group <= 0 or depth % group:
        raise LinnetError(f"groups of {group} must divide the {depth} inputs")
    w = weight.to(torch.float32).contiguous()
    q = torch.empty(width, depth, dtype=torch.int8, device=device)
    scale = torch.empty(width, depth // group, dtype=torch.float32, device=device)
    with torch.cuda.device(device):
        _lib.call("lnq_int8_quantize", _ptr(w), _ptr(q), _ptr(scale), width, depth, group, codes[dtype], _stream(device))
    return q, scale


# ------------------------------------------------------------------------- NF4


def _nf4_operands(what: str, codes: torch.Tensor, absmax: torch.Tensor, block: int) -> tuple[int, int]:
    """(Out, In) of an `Nf4Linear` weight: codes [Out, In/2] uint8, absmax
    [Out, In/block] float32 (`stdlib/quant.linnet:201-215`)."""
    if codes.dtype != torch.uint8 or codes.dim() != 2:
        raise LinnetError(f"{what}: the weight is [Out, In/2] uint8 bytes of NF4 codes")
    out_features, in_features = codes.shape[0], 2 * codes.shape[1]
    if block <= 0 or block % 2 or in_features % block:
        raise LinnetError(f"{what}: {in_features} inputs do not make even blocks of {block}")
    if absmax.dtype != torch.float32 or absmax.shape != (out_features, in_features // block):
        raise LinnetError(f"{what}: absmax is [{out_features}, {in_features // block}] float32, "
                          f"got {tuple(absmax.shape)} {absmax.dtype}")
    return out_features, in_features


def nf4_dequantize(codes: torch.Tensor, absmax: torch.Tensor, block: int, dtype: torch.dtype) -> torch.Tensor:
    """`dequantize_nf4` (`stdlib/quant.linnet:180-187`): the [Out, In] weight in
    `dtype`, `nf4(q) * absmax` in f32 rounded once, bit for bit."""
    device = _on_gpu("nf4_dequantize", codes, absmax)
    out_features, in_features = _nf4_operands("nf4_dequantize", codes, absmax, block)
    code = _code(dtype, "nf4_dequantize", (torch.bfloat16, torch.float16, torch.float32))
    codes, absmax = codes.contiguous(), absmax.contiguous()
    out = torch.empty(out_features, in_features, dtype=dtype, device=device)
    with torch.cuda.device(device):
        _lib.call("lnq_nf4_dequant", _ptr(codes), _ptr(absmax), _ptr(out), out_features, in_features, block, code,
                  _stream(device))
    return out


# Rows of x up to which `nf4_linear` reads the stored weight with the NF4 GEMV
# (8 rows a pass over the weight up to In = 8192, 4 past it); more rows widen
# the weight and multiply. bf16, graph-replayed, against 57 us for the widened
# weight and its product: 4096 -> 14336 at 1 / 8 / 16 rows 12.0 / 21.6 / 41.8
# us; 14336 -> 4096 at 1 / 8 / 12 rows 11.5 / 35.3 / 52.5 us.
NF4_GEMV_ROWS = 16
NF4_GEMV_ROWS_WIDE = 8  # In > 8192
NF4_GEMV_MAX_IN = 32768


def nf4_gemv_fits(rows: int, in_features: int, block: int, dtype: torch.dtype) -> bool:
    """Whether `nf4_linear` takes the GEMV for this call."""
    limit = NF4_GEMV_ROWS if in_features <= 8192 else NF4_GEMV_ROWS_WIDE
    return (dtype in _HALF and rows <= limit and block % 16 == 0 and in_features % block == 0
            and 0 < in_features <= NF4_GEMV_MAX_IN)


def nf4_gemv(x: torch.Tensor, codes: torch.Tensor, absmax: torch.Tensor, block: int,
             bias: torch.Tensor | None = None) -> torch.Tensor:
    """x [..., In] (bf16 / f16) times the NF4 weight's transpose (+ bias), the
    weight read as stored (`lnq_nf4_linear`)."""
    device = _on_gpu("nf4_gemv", x, codes, absmax, bias)
    out_features, in_features = _nf4_operands("nf4_gemv", codes, absmax, block)
    code = _code(x.dtype, "nf4_gemv")
    if x.shape[-1] != in_features:
        raise LinnetError(f"nf4_gemv: x has {x.shape[-1]} inputs, the weight {in_features}")
    if bias is not None and (bias.dtype != x.dtype or bias.numel() != out_features):
        raise LinnetError(f"nf4_gemv: bias is [{out_features}] {x.dtype}")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, in_features)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16 or (x2.shape[0] > 1 and x2.stride(0) < in_features):
        x2 = x2.contiguous()
        if in_features % 8:
            raise LinnetError("nf4_gemv: In must be a multiple of 8")
    codes, absmax = codes.contiguous(), absmax.contiguous()
    bias = None if bias is None else bias.contiguous()
    y = torch.empty(x2.shape[0], out_features, dtype=x.dtype, device=device)
    with torch.cuda.device(device):
        _lib.call("lnq_nf4_linear", _ptr(x2), max(x2.stride(0), in_features), x2.shape[0], _ptr(codes), _ptr(absmax),
                  _ptr(bias), _ptr(y), out_features, out_features, in_features, block, code, _stream(device))
    return y.reshape(*lead, out_features)


def nf4_linear(x: torch.Tensor, codes: torch.Tensor, absmax: torch.Tensor, block: int,
               bias: torch.Tensor | None = None) -> torch.Tensor:
    """`linear_nf4` (`stdlib/quant.linnet:189-199`): up to `NF4_GEMV_ROWS` rows of
    bf16 / f16 x (`NF4_GEMV_ROWS_WIDE` past In = 8192) on the NF4 GEMV; otherwise the weight widened by the HIP
    dequantize kernel, then multiplied in x's type (the reference's own body)."""
    _on_gpu("nf4_linear", x, codes, absmax, bias)
    out_features, in_features = _nf4_operands("nf4_linear", codes, absmax, block)
    rows = x.numel() // max(in_features, 1) if x.dim() else 0
    if nf4_gemv_fits(rows, in_features, block, x.dtype):
        return nf4_gemv(x, codes, absmax, block, bias)
    weight = nf4_dequantize(codes, absmax, block, x.dtype)
    return torch.nn.functional.linear(x, weight, bias)


def nf4_repack(packed: torch.Tensor, absmax: torch.Tensor, out_features: int, in_features: int, block: int,
               nested_absmax: torch.Tensor | None = None, nested_map: torch.Tensor | None = None,
               nested_block: int = 0, offset: float = 0.0) -> tuple[torch.Tensor, torch.Tensor]:
    """A bitsandbytes NF4 layer as `Nf4Linear` holds it (`quant.py:414-466`):
    (codes [Out, In/2] uint8 with the first input in the low nibble, absmax
    [Out, In/block] float32). `packed` is bitsandbytes' byte array (first code of
    a pair in the high nibble); `absmax` its f32 scales, or, with double
    quantization, their uint8 codes decoded through `nested_map` [256] and
    `nested_absmax` (one a `nested_block` scales) plus `offset`, in f32."""
    device = _on_gpu("nf4_repack", packed, absmax, nested_absmax, nested_map)
    if block <= 0 or block % 2 or in_features % block:
        raise LinnetError(f"nf4_repack: block {block} is not an even divisor of in_features {in_features}")
    if packed.dtype != torch.uint8 or packed.numel() * 2 != out_features * in_features:
        raise LinnetError(f"nf4_repack: packed holds {packed.numel()} {packed.dtype} elements; "
                          f"{out_features} x {in_features} codes take {out_features * in_features // 2} uint8")
    scales = out_features * in_features // block
    nested = nested_map is not None or nested_absmax is not None
    if nested:
        if nested_map is None or nested_absmax is None or nested_block <= 0:
            raise LinnetError("nf4_repack: double quantization takes nested_absmax, nested_map and nested_block")
        if nested_map.dtype != torch.float32 or nested_map.numel() != 256:
            raise LinnetError("nf4_repack: nested_map is 256 float32 values")
        if nested_absmax.dtype != torch.float32 or nested_absmax.numel() < -(-scales // nested_block):
            raise LinnetError(f"nf4_repack: {nested_absmax.numel()} nested scales for {scales} blocks of {nested_block}")
        if absmax.dtype != torch.uint8 or absmax.numel() != scales:
            raise LinnetError(f"nf4_repack: absmax holds {absmax.numel()} {absmax.dtype} elements; "
                              f"{scales} blocks take as many uint8 codes")
    elif absmax.dtype != torch.float32 or absmax.numel() != scales:
        raise LinnetError(f"nf4_repack: absmax holds {absmax.numel()} {absmax.dtype} elements; "
                          f"{scales} blocks take as many float32 scales")
    packed, absmax = packed.contiguous(), absmax.contiguous()
    nested_absmax = None if nested_absmax is None else nested_absmax.contiguous()
    nested_map = None if nested_map is None else nested_map.contiguous()
    codes = torch.empty(out_features, in_features // 2, dtype=torch.uint8, device=device)
    scale = torch.empty(out_features, in_features // block, dtype=torch.float32, device=device)
    with torch.cuda.device(device):
        _lib.call("lnq_nf4_repack", _ptr(packed), _ptr(absmax), _ptr(nested_absmax), _ptr(nested_map),
                  nested_block, ctypes.c_float(offset), _ptr(codes), _ptr(scale), out_features, in_features, block,
                  _stream(device))
    return codes, scale
