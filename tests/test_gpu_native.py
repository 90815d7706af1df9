"""Every entry of the interpreter table (`linnet_amd.torch.native.NATIVE`), executed
on the GPU with its arguments as one tuple, the way the reference's interpreter
passes a quantized layer's call (`python/linnet/src/linnet/torch/native.py:417-480,
556-566`: `(x, packed, scale, zero, bias)` for the int4 layer, `(x, weight, scale,
bias)` for the 8-bit ones), against the oracle's restatement of the reference's
CPU path for the same layer on the same inputs.

Bounds: `1e-2 * max|want|` where x is used as given (bf16 rounding of the
dequantized weight and of the output), `0.06 * max` where the entry rounds x to
8 bits (`torch._scaled_mm`, `linnet.int8_linear(w8a8)` past 32 rows), the
reference's own bounds (`tests/test_quant_groups.py:194-195`,
`tests/test_quant_8bit.py:341`). Row counts cover each dispatch branch: one row
(GEMV), 5 and 40 (few-row kernels; 40 is past `FEW_ROWS`, so the rounded
entries take the 8-bit product), 300 (tiled / dequantize + product)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from linnet_amd.errors import LinnetError
from linnet_amd.torch import native
from oracle import linear, quant

pytestmark = pytest.mark.gpu
DEV = "cuda"
ROWS = [1, 5, 40, 300]


def _check(got: torch.Tensor, want: torch.Tensor, bound: float) -> None:
    assert got.shape == want.shape and got.dtype == want.dtype
    g = got.float().cpu().numpy()
    w = want.float().numpy()
    err = float(np.abs(g - w).max())
    top = float(np.abs(w).max())
    print(f"max abs err {err:.3e}, rel to max {err / top:.3e} (bound {bound})")
    assert err <= bound * top


def _x(rows: int, width: int, seed: int) -> torch.Tensor:
    return torch.randn(rows, width, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16)


def _bias(out: int, seed: int) -> torch.Tensor:
    return (torch.randn(out, generator=torch.Generator().manual_seed(seed)) * 0.5).to(torch.bfloat16)


def test_every_entry_is_covered() -> None:
    assert set(native.NATIVE) == {
        "torch.ops.aten._weight_int4pack_mm", "linnet.decode_fp8", "linnet.fp8_linear", "torch._scaled_mm",
        "linnet.fp8_block_linear", "torch._scaled_mm(blocks)", "linnet.int8_linear", "linnet.int8_linear(w8a8)",
        "linnet.int8_group_linear", "torch.index_select",
    }


@pytest.mark.parametrize("rows", ROWS)
@pytest.mark.parametrize(("group", "with_bias"), [(128, True), (128, False), (64, True), (16, True)])
def test_int4_groups_linear_entry(rows: int, group: int, with_bias: bool) -> None:
    """`torch.ops.aten._weight_int4pack_mm` (`native.py:417-423`); group 16 is the
    fallback (the weight dequantized once, then the product)."""
    out, width = 384, 512
    w = np.random.default_rng(rows + group).standard_normal((out, width)).astype(np.float32) * 0.02
    packed, scale, zero = quant.quantize_int4_groups(w, group)
    p = torch.from_numpy(packed)
    s = torch.from_numpy(quant.to_bf16_bits(scale).view(np.int16)).view(torch.bfloat16)
    z = torch.from_numpy(zero)
    x = _x(rows, width, rows)
    bias = _bias(out, 3) if with_bias else None
    got = native.NATIVE["torch.ops.aten._weight_int4pack_mm"](
        (x.to(DEV), p.to(DEV), s.to(DEV), z.to(DEV), None if bias is None else bias.to(DEV)))
    want = linear.int4_groups_linear_interpreter(x, p, s, z, bias)
    _check(got, want, 1e-2)


def test_decode_fp8_entry() -> None:
    """Every byte: the non-NaN ones bit for bit the oracle's E4M3 decoding, the two
    NaN bytes NaN (torch's `float8_e4m3fn`, as the reference's entry)."""
    bits = torch.arange(256, dtype=torch.uint8)
    got = native.NATIVE["linnet.decode_fp8"]((bits.to(DEV),)).cpu().numpy()
    want = quant.decode_fp8(bits.numpy())
    finite = (bits.numpy() & 0x7F) != 0x7F
    np.testing.assert_array_equal(got[finite], want[finite])
    assert np.isnan(got[~finite]).all()


def _fp8_layer(out: int, width: int, seed: int) -> tuple[torch.Tensor, torch.Tensor]:
    full = torch.randn(out, width, generator=torch.Generator().manual_seed(seed)) * 0.02
    scale = full.abs().amax(1, keepdim=True) / 448.0
    return (full / scale).to(torch.float8_e4m3fn), scale.to(torch.bfloat16)


@pytest.mark.parametrize("rows", ROWS)
@pytest.mark.parametrize("key", ["linnet.fp8_linear", "torch._scaled_mm"])
def test_fp8_linear_entries(key: str, rows: int) -> None:
    out, width = 256, 1024
    weight, scale = _fp8_layer(out, width, rows)
    x, bias = _x(rows, width, rows + 1), _bias(out, 4)
    got = native.NATIVE[key]((x.to(DEV), weight.to(DEV), scale.to(DEV), bias.to(DEV)))
    want = linear.fp8_linear_cpu(x, weight, scale, bias)
    rounded = key == "torch._scaled_mm" and rows > 32
    _check(got, want, 0.06 if rounded else 1e-2)


@pytest.mark.parametrize("rows", ROWS)
@pytest.mark.parametrize("key", ["linnet.fp8_block_linear", "torch._scaled_mm(blocks)"])
def test_fp8_block_linear_entries(key: str, rows: int) -> None:
    out, width, block = 256, 512, 128
    g = torch.Generator().manual_seed(rows + 7)
    full = torch.randn(out, width, generator=g) * 0.02
    scale = full.reshape(out // block, block, width // block, block).abs().amax((1, 3)) / 448.0
    weight = (full / scale.repeat_interleave(block, 0).repeat_interleave(block, 1)).to(torch.float8_e4m3fn)
    x, bias = _x(rows, width, rows + 2), _bias(out, 5)
    got = native.NATIVE[key]((x.to(DEV), weight.to(DEV), scale.to(DEV), bias.to(DEV)))
    want = linear.fp8_block_linear_cpu(x, weight, scale, bias)
    rounded = key == "torch._scaled_mm(blocks)" and rows > 32
    _check(got, want, 0.06 if rounded else 1e-2)


@pytest.mark.parametrize("rows", ROWS)
@pytest.mark.parametrize("key", ["linnet.int8_linear", "linnet.int8_linear(w8a8)"])
def test_int8_linear_entries(key: str, rows: int) -> None:
    out, width = 320, 768
    w = np.random.default_rng(rows).standard_normal((out, width)).astype(np.float32) * 0.02
    q, scale = quant.quantize_int8_groups(w, width, "bf16")
    qt = torch.from_numpy(q)
    st = torch.from_numpy(scale).to(torch.bfloat16)  # [Out, 1], Int8Linear's scale
    x, bias = _x(rows, width, rows + 3), _bias(out, 6)
    got = native.NATIVE[key]((x.to(DEV), qt.to(DEV), st.to(DEV), bias.to(DEV)))
    want = linear.int8_linear_cpu(x, qt, st, bias)
    rounded = key == "linnet.int8_linear(w8a8)" and rows > 32
    _check(got, want, 0.06 if rounded else 1e-2)


@pytest.mark.parametrize("rows", ROWS)
@pytest.mark.parametrize("group", [128, 64, 24])
def test_int8_group_linear_entry(rows: int, group: int) -> None:
    """Groups of 128 and 64 run the fused kernels; 24 is not a multiple of 16, the
    reference's gate (`quantized.py:197-203`), so the weight is dequantized first."""
    out, width = 192, 768
    w = np.random.default_rng(rows + group).standard_normal((out, width)).astype(np.float32) * 0.02
    q, scale = quant.quantize_int8_groups(w, group, "bf16")
    qt = torch.from_numpy(q)
    st = torch.from_numpy(scale).to(torch.bfloat16)
    x, bias = _x(rows, width, rows + 4), _bias(out, 7)
    got = native.NATIVE["linnet.int8_group_linear"]((x.to(DEV), qt.to(DEV), st.to(DEV), bias.to(DEV)))
    want = linear.int8_group_linear_cpu(x, qt, st, bias)
    _check(got, want, 1e-2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32, torch.float64, torch.int32])
def test_index_select_entry(dtype: torch.dtype) -> None:
    """bf16 / f16 / f32 on the HIP gather, other dtypes on torch's `index_select`:
    bit for bit `x.index_select(-1, order)` either way, with int32 and int64
    orders."""
    g = torch.Generator().manual_seed(8)
    x = (torch.randn(3, 5, 200, generator=g) * 100).to(dtype)
    order = torch.randperm(200, generator=g)
    want = x.index_select(-1, order)
    for o in (order, order.to(torch.int32)):
        got = native.NATIVE["torch.index_select"]((x.to(DEV), o.to(DEV))).cpu()
        assert got.dtype == dtype and torch.equal(got, want)
    # An order that selects a subset, not a permutation-sized vector.
    sub = order[:17]
    assert torch.equal(native.NATIVE["torch.index_select"]((x.to(DEV), sub.to(DEV))).cpu(), x.index_select(-1, sub))


def test_index_select_entry_refuses_an_index_off_the_axis() -> None:
    """The reference's `index_select` raises on an index outside the axis; so does the
    entry (the HIP gather alone would read 0 there)."""
    x = torch.randn(2, 64, device=DEV).to(torch.bfloat16)
    order = torch.arange(64, device=DEV, dtype=torch.int32)
    order[5] = 64
    with pytest.raises(LinnetError, match="outside"):
        native.NATIVE["torch.index_select"]((x, order))
    order[5] = -1
    with pytest.raises(LinnetError, match="outside"):
        native.NATIVE["torch.index_select"]((x, order))
