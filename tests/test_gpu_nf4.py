"""NF4 layers (`std.quant::Nf4Linear`, `stdlib/quant.linnet:177-215`) on the GPU.

- `lnq_nf4_dequant` is bit-exact against the oracle's `dequantize_nf4` (the f32
  product of the code's value and its block's absmax, rounded once) for bf16,
  f16 and f32, with rows whose bytes do and do not split in 8.
- The NF4 GEMV (`lnq_nf4_linear`, 1-16 rows of bf16 / f16 x, 8 a pass up to In = 8192) is checked against
  the oracle's f64 product over the exact f32 weight, within 1e-2 of the
  largest output plus the 16-bit rounding of each one (the reference's
  tolerance for its quantized products, `python/linnet/tests/test_quant_groups.py:165-195`):
  the kernel rounds each code's value to x's type, as the reference's body
  rounds the scaled weight to T. Shapes cover In below one unit a lane, a
  ragged last unit slot, In = 32768 (8 slots), blocks of 16 to 256, a bias,
  and Llama-3.1-8B's 4096 -> 14336 and 14336 -> 4096.
- More rows (past 16, or 8 past In = 8192), f32 and blocks the GEMV does not take go through the dequantize
  kernel and the product in x's type (the reference's body); f32 is held to
  1e-5 as the reference's NF4 test holds its f32 layer
  (`python/linnet/tests/test_nf4.py:103-115`).
- `import_quantized` on a bitsandbytes NF4 checkpoint built as the reference's
  test builds one (`test_nf4.py:49-80`: plain and double-quantized absmax, a
  bias), then `Nf4Linear` loaded from the output, against `x @ W.T + b`; the
  repack kernel is bit-exact against the oracle's `bnb_nf4_layer`.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from linnet_amd import quant as lquant
from linnet_amd.torch import kernels
from linnet_amd.torch.nf4 import Nf4Linear
from oracle import linear, quant

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
_NAMES = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


def _layer(out_features: int, in_features: int, block: int, seed: int) -> tuple[np.ndarray, np.ndarray]:
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 256, (out_features, in_features // 2)).astype(np.uint8)
    absmax = rng.uniform(0.02, 0.2, (out_features, in_features // block)).astype(np.float32)
    return codes, absmax


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize(("out_features", "in_features", "block"), [
    (8, 128, 64), (37, 72, 8), (3, 2, 2), (256, 4096, 64), (5, 48, 16)])
def test_dequant_is_bit_exact(dtype: torch.dtype, out_features: int, in_features: int, block: int) -> None:
    print(f"nf4 dequant {out_features}x{in_features} block {block} {dtype}", flush=True)
    codes, absmax = _layer(out_features, in_features, block, out_features + in_features)
    got = kernels.nf4_dequantize(torch.from_numpy(codes).to(DEV), torch.from_numpy(absmax).to(DEV), block, dtype)
    want = quant.dequantize_nf4(codes, absmax, block, _NAMES[dtype])
    raw = got.cpu()
    raw = raw.view(torch.int16).numpy().view(np.uint16) if dtype == torch.bfloat16 else raw.numpy()
    np.testing.assert_array_equal(raw, want)


def _check(got: torch.Tensor, want: np.ndarray) -> None:
    g = got.float().cpu().numpy()
    top = float(np.abs(want).max())
    err = np.abs(g - want)
    print(f"max abs err {err.max():.3e}, rel to max {err.max() / top:.3e}", flush=True)
    assert np.all(err <= 1e-2 * top + 8e-3 * np.abs(want))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows", [1, 2, 3, 4, 5, 8, 16])
@pytest.mark.parametrize(("out_features", "in_features", "block", "bias"), [
    (8, 128, 64, False), (40, 48, 16, True), (72, 4096, 64, True), (64, 4112, 16, False),
    (1000, 14336, 128, False), (130, 32768, 256, True), (14336, 4096, 64, False), (4096, 14336, 64, True)])
def test_gemv_against_f64(dtype: torch.dtype, rows: int, out_features: int, in_features: int, block: int,
                          bias: bool) -> None:
    print(f"nf4 gemv rows {rows} {out_features}x{in_features} block {block} bias {bias} {dtype}", flush=True)
    limit = kernels.NF4_GEMV_ROWS if in_features <= 8192 else kernels.NF4_GEMV_ROWS_WIDE
    assert kernels.nf4_gemv_fits(rows, in_features, block, dtype) == (rows <= limit)
    codes, absmax = _layer(out_features, in_features, block, rows * 7 + out_features)
    gen = torch.Generator().manual_seed(rows + in_features)
    x = torch.randn(rows, in_features, generator=gen).to(dtype)
    b = torch.randn(out_features, generator=gen).to(dtype) if bias else None
    # The GEMV itself at every row count (several passes past 8 rows), whatever nf4_linear picks.
    got = kernels.nf4_gemv(x.to(DEV), torch.from_numpy(codes).to(DEV), torch.from_numpy(absmax).to(DEV), block,
                           None if b is None else b.to(DEV))
    want = linear.nf4_reference_f64(x.float().numpy(), codes, absmax, block, None if b is None else b.float().numpy())
    _check(got, want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize(("rows", "out_features", "in_features", "block"), [
    (1, 64, 16, 16), (4, 40, 48, 16), (16, 72, 4096, 64), (3, 1000, 14336, 128)])
def test_gemv_uses_the_rounded_nf4_values(dtype: torch.dtype, rows: int, out_features: int, in_features: int,
                                          block: int) -> None:
    """The GEMV's arithmetic, pinned tightly: each code's value rounded to x's
    type, products summed in f32, each block's sum scaled by its absmax, the
    output rounded once. Against the f64 sum over the rounded values: half a unit
    in the last place of the output's type plus 16 f32 units of the row's
    absolute sum, so one wrong entry of the lookup table (or a bf16 / f16 bit
    pattern off by one) fails, where the 1e-2 tolerance above would not."""
    print(f"nf4 gemv table rows {rows} {out_features}x{in_features} block {block} {dtype}", flush=True)
    codes, absmax = _layer(out_features, in_features, block, rows + in_features + 3)
    x = torch.randn(rows, in_features, generator=torch.Generator().manual_seed(rows)).to(dtype)
    got = kernels.nf4_gemv(x.to(DEV), torch.from_numpy(codes).to(DEV), torch.from_numpy(absmax).to(DEV), block)
    values = torch.from_numpy(quant.NF4_VALUES.copy()).to(dtype).double().numpy()
    q = np.stack([codes & 15, codes >> 4], axis=-1).reshape(out_features, in_features)  # low nibble first
    w = values[q] * np.repeat(absmax.astype(np.float64), block, axis=1)
    terms = x.double().numpy()[:, None, :] * w[None, :, :]
    ref, mag = terms.sum(axis=-1), np.abs(terms).sum(axis=-1)
    half_ulp = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    err = np.abs(got.double().cpu().numpy() - ref)
    bound = half_ulp * np.abs(ref) + 2.0 ** -20 * mag + 2.0 ** -24
    print(f"max err / bound {float((err / bound).max()):.3f}", flush=True)
    assert np.all(err <= bound)


def test_gemv_takes_strided_rows_and_leading_axes() -> None:
    codes, absmax = _layer(96, 512, 64, 11)
    x = torch.randn(2, 3, 1024, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    view = x[..., 256:768]
    got = kernels.nf4_linear(view.to(DEV), torch.from_numpy(codes).to(DEV), torch.from_numpy(absmax).to(DEV), 64)
    assert got.shape == (2, 3, 96)
    want = linear.nf4_reference_f64(view.reshape(6, 512).float().numpy(), codes, absmax, 64).reshape(2, 3, 96)
    _check(got, want)


@pytest.mark.parametrize(("dtype", "rows", "block"), [
    (torch.bfloat16, 17, 64), (torch.float16, 33, 64), (torch.bfloat16, 3, 8), (torch.float32, 1, 64),
    (torch.float32, 40, 64)])
def test_wider_calls_widen_then_multiply(dtype: torch.dtype, rows: int, block: int) -> None:
    print(f"nf4 linear rows {rows} block {block} {dtype}", flush=True)
    assert not kernels.nf4_gemv_fits(rows, 1024, block, dtype)
    codes, absmax = _layer(200, 1024, block, rows)
    x = torch.randn(rows, 1024, generator=torch.Generator().manual_seed(rows)).to(dtype)
    b = torch.randn(200, generator=torch.Generator().manual_seed(1)).to(dtype)
    got = kernels.nf4_linear(x.to(DEV), torch.from_numpy(codes).to(DEV), torch.from_numpy(absmax).to(DEV), block,
                             b.to(DEV))
    want = linear.nf4_reference_f64(x.float().numpy(), codes, absmax, block, b.float().numpy())
    if dtype == torch.float32:
        np.testing.assert_allclose(got.cpu().numpy(), want, rtol=1e-5, atol=1e-5)
    else:
        _check(got, want)


def test_gemv_agrees_with_the_widened_product() -> None:
    """The two product paths on one bf16 layer: within the bf16 rounding of the
    weight and of the result."""
    codes, absmax = _layer(4096, 4096, 64, 3)
    c, a = torch.from_numpy(codes).to(DEV), torch.from_numpy(absmax).to(DEV)
    x = torch.randn(4, 4096, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).to(DEV)
    fast = kernels.nf4_gemv(x, c, a, 64)
    wide = torch.nn.functional.linear(x, kernels.nf4_dequantize(c, a, 64, torch.bfloat16))
    top = float(wide.float().abs().max())
    assert float((fast.float() - wide.float()).abs().max()) <= 1e-2 * top


@pytest.mark.parametrize("nested", [True, False])
def test_repack_is_bit_exact(nested: bool) -> None:
    rng = np.random.default_rng(9)
    out_features, in_features, block, nested_block = 48, 320, 64, 7
    packed = rng.integers(0, 256, out_features * in_features // 2).astype(np.uint8)
    blocks = out_features * in_features // block
    if nested:
        scale_codes = rng.integers(0, 256, blocks).astype(np.uint8)
        outer = rng.uniform(0.5, 1.5, -(-blocks // nested_block)).astype(np.float32)
        table = np.sort(rng.uniform(-1, 1, 256)).astype(np.float32)
        want = quant.bnb_nf4_layer(packed, scale_codes, out_features, in_features, block, outer, table, nested_block,
                                   0.37)
        got = kernels.nf4_repack(torch.from_numpy(packed).to(DEV), torch.from_numpy(scale_codes).to(DEV),
                                 out_features, in_features, block, torch.from_numpy(outer).to(DEV),
                                 torch.from_numpy(table).to(DEV), nested_block, 0.37)
    else:
        plain = rng.uniform(0.1, 2, blocks).astype(np.float32)
        want = quant.bnb_nf4_layer(packed, plain, out_features, in_features, block)
        got = kernels.nf4_repack(torch.from_numpy(packed).to(DEV), torch.from_numpy(plain).to(DEV), out_features,
                                 in_features, block)
    np.testing.assert_array_equal(got[0].cpu().numpy(), want[0])
    np.testing.assert_array_equal(got[1].cpu().numpy().view(np.uint32), want[1].view(np.uint32))


IN, OUT, BLOCK, NESTED_BLOCK = 128, 8, 64, 256
CONFIG = {"quant_method": "bitsandbytes", "load_in_4bit": True, "bnb_4bit_quant_type": "nf4"}


def _bnb_checkpoint(path: Path, nested: bool) -> tuple[np.ndarray, np.ndarray]:
    """A bitsandbytes NF4 layer at `model.proj` laid out as bitsandbytes saves one
    (weight flattened, first code of a pair in the high nibble, state as JSON
    bytes); returns the f32 weight and bias it stands for."""
    from safetensors.torch import save_file

    rng = np.random.default_rng(7)
    codes = rng.integers(0, 16, OUT * IN).astype(np.uint8)
    blocks = OUT * IN // BLOCK
    tensors = {
        "model.proj.weight": torch.from_numpy((codes[1::2] | (codes[0::2] << 4)).reshape(-1, 1)),
        "model.proj.weight.quant_map": torch.from_numpy(lquant.NF4.copy()),
    }
    state: dict[str, object] = {"quant_type": "nf4", "blocksize": BLOCK, "dtype": "bfloat16", "shape": [OUT, IN]}
    if nested:
        scale_codes = rng.integers(0, 256, blocks).astype(np.uint8)
        outer = rng.uniform(0.5, 1.5, -(-blocks // NESTED_BLOCK)).astype(np.float32)
        table = np.sort(rng.uniform(-1.0, 1.0, 256)).astype(np.float32)
        absmax = (table[scale_codes] * outer[np.arange(blocks) // NESTED_BLOCK] + np.float32(0.75)).astype(np.float32)
        tensors["model.proj.weight.absmax"] = torch.from_numpy(scale_codes)
        tensors["model.proj.weight.nested_absmax"] = torch.from_numpy(outer)
        tensors["model.proj.weight.nested_quant_map"] = torch.from_numpy(table)
        state |= {"nested_blocksize": NESTED_BLOCK, "nested_offset": 0.75}
    else:
        absmax = rng.uniform(0.1, 2.0, blocks).astype(np.float32)
        tensors["model.proj.weight.absmax"] = torch.from_numpy(absmax)
    encoded = np.frombuffer(json.dumps(state).encode("utf-8"), dtype=np.uint8).copy()
    tensors["model.proj.weight.quant_state.bitsandbytes__nf4"] = torch.from_numpy(encoded)
    bias = rng.standard_normal(OUT).astype(np.float32)
    tensors["model.proj.bias"] = torch.from_numpy(bias)
    save_file(tensors, str(path))
    weight = (quant.NF4_VALUES[codes].reshape(-1, BLOCK) * absmax[:, None]).reshape(OUT, IN)
    return weight.astype(np.float32), bias


@pytest.mark.parametrize("nested", [True, False])
def test_import_bitsandbytes_then_multiply(tmp_path: Path, nested: bool) -> None:
    weight, bias = _bnb_checkpoint(tmp_path / "bnb.safetensors", nested)
    done = lquant.import_quantized(tmp_path / "bnb.safetensors", tmp_path / "nf4.safetensors",
                                   bindings={"proj.weight": "model.proj.weight", "proj.bias": "model.proj.bias"},
                                   config=CONFIG)
    assert done == ["proj.weight"]
    x = np.random.default_rng(1).standard_normal((3, IN)).astype(np.float32)
    layer = Nf4Linear(IN, OUT, BLOCK, torch.float32, bias=True, device=DEV).load(tmp_path / "nf4.safetensors", "proj.")
    got = layer(torch.from_numpy(x).to(DEV)).cpu().numpy()
    np.testing.assert_allclose(got, x @ weight.T + bias, rtol=1e-5, atol=1e-5)
    half = Nf4Linear(IN, OUT, BLOCK, torch.bfloat16, bias=True, device=DEV).load(tmp_path / "nf4.safetensors", "proj.")
    xb = torch.from_numpy(x).to(torch.bfloat16)
    want = xb.float().numpy().astype(np.float64) @ weight.T.astype(np.float64) + torch.from_numpy(bias).to(
        torch.bfloat16).float().numpy()
    _check(half(xb.to(DEV)), want)


def test_import_rejects_other_bitsandbytes_types(tmp_path: Path) -> None:
    _bnb_checkpoint(tmp_path / "bnb.safetensors", False)
    with pytest.raises(lquant.LinnetError, match="only NF4 codes"):
        lquant.import_quantized(tmp_path / "bnb.safetensors", tmp_path / "o.safetensors",
                                config=CONFIG | {"bnb_4bit_quant_type": "fp4"})
    with pytest.raises(lquant.LinnetError, match="load_in_4bit"):
        lquant.import_quantized(tmp_path / "bnb.safetensors", tmp_path / "o.safetensors",
                                config={"quant_method": "bitsandbytes"})
