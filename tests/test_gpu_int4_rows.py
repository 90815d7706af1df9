"""`std.quant::Int4Linear` (signed int4, one scale a row) on the GPU, against the oracle.

- the weight rewritten into the group layout dequantizes, bit for bit, to the
  oracle's `cast<T>(f32(i4) * scale)` (`stdlib/quant.linnet:22-29, 101-111`);
- the layer (`_int4_row_pack` + `_int4_row_linear`) is within `1e-2 * max|y|` of the
  f64 product with that weight, plus bias, at 1..300 rows -- GEMV, skinny MFMA and
  tiled GEMM kernels -- and through the dequantized fallback (In % 128 != 0, f32);
  max abs / rel errors are printed.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from linnet_amd.torch import generated, kernels
from oracle import quant

pytestmark = pytest.mark.gpu
DEV = "cuda"
_NAMES = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


def _raw(t: torch.Tensor) -> np.ndarray:
    t = t.contiguous().cpu()
    return t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.numpy()


def _layer(out: int, width: int, seed: int, dtype: torch.dtype):
    """Signed values -8..7 packed two a byte (element 2k low), per-row scales in the
    model dtype, `[Out, 1]` as the layer stores them."""
    g = torch.Generator().manual_seed(seed)
    weight = torch.randint(0, 256, (out, width // 2), generator=g, dtype=torch.uint8)
    scale = ((torch.rand(out, 1, generator=g) - 0.5) * 0.04).to(dtype)
    return weight, scale


def _oracle_weight(weight: torch.Tensor, scale: torch.Tensor) -> np.ndarray:
    name = _NAMES[scale.dtype]
    return quant.decode_storage(quant.dequantize_int4_rows(weight.cpu().numpy(), _raw(scale), name), name)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize(("out", "width", "group"), [(80, 256, 128), (64, 4096, 128), (7, 96, 32), (3, 64, 64)])
def test_prepared_weight_dequantizes_bit_for_bit(dtype: torch.dtype, out: int, width: int, group: int) -> None:
    weight, scale = _layer(out, width, out + width, dtype)
    packed, group_scale, zero = kernels.int4_row_prepare(weight.to(DEV), scale.to(DEV).reshape(-1), group)
    assert tuple(packed.shape) == (out, width // group, group // 2)
    assert bool((zero == 8).all())
    assert bool((group_scale == scale.to(DEV)).all())
    got = kernels.int4_weight(packed, group_scale, zero)
    np.testing.assert_array_equal(_raw(got), quant.encode_storage(_oracle_weight(weight, scale), _NAMES[dtype]))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows", [1, 4, 16, 100, 300])
@pytest.mark.parametrize(("out", "width"), [(1024, 4096), (80, 256)])
def test_layer_matches_the_oracle(dtype: torch.dtype, rows: int, out: int, width: int) -> None:
    weight, scale = _layer(out, width, rows, dtype)
    g = torch.Generator().manual_seed(rows + 1)
    x = torch.randn(rows, width, generator=g).to(dtype)
    bias = (torch.randn(out, generator=g) * 0.1).to(dtype)
    packed = generated._int4_row_pack(weight.to(DEV), scale.to(DEV))
    assert len(packed) == 3
    for b in (None, bias):
        y = generated._int4_row_linear(x.to(DEV), packed, None if b is None else b.to(DEV))
        torch.cuda.synchronize()
        ref = x.double().numpy() @ _oracle_weight(weight, scale).astype(np.float64).T
        if b is not None:
            ref = ref + b.double().numpy()[None, :]
        err = np.abs(y.double().cpu().numpy() - ref)
        print(f"rows {rows} out {out} in {width} {dtype} bias {b is not None}: max abs err {err.max():.3e}, "
              f"rel to max|y| {err.max() / np.abs(ref).max():.3e}")
        assert y.shape == (rows, out) and y.dtype == dtype
        assert err.max() <= 1e-2 * np.abs(ref).max()


@pytest.mark.parametrize(("dtype", "width"), [(torch.bfloat16, 96), (torch.float16, 50), (torch.float32, 256)])
def test_layer_fallback_matches_the_oracle(dtype: torch.dtype, width: int) -> None:
    """Shapes the fused kernels do not take: the dequantized weight, then `F.linear`."""
    weight, scale = _layer(24, width, width, dtype)
    packed = generated._int4_row_pack(weight.to(DEV), scale.to(DEV))
    assert len(packed) == 1
    np.testing.assert_array_equal(_raw(packed[0]), quant.encode_storage(_oracle_weight(weight, scale), _NAMES[dtype]))
    x = torch.randn(2, 3, width, generator=torch.Generator().manual_seed(2)).to(dtype)
    y = generated._int4_row_linear(x.to(DEV), packed, None)
    torch.cuda.synchronize()
    ref = x.double().numpy() @ _oracle_weight(weight, scale).astype(np.float64).T
    err = np.abs(y.double().cpu().numpy() - ref)
    print(f"fallback in {width} {dtype}: max abs err {err.max():.3e}, rel {err.max() / np.abs(ref).max():.3e}")
    assert y.shape == (2, 3, 24)
    assert err.max() <= 1e-2 * np.abs(ref).max()
