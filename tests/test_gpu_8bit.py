"""Parity of the 8-bit HIP path with the oracle, on the GPU, through the C ABI.

- int8 quantize, per-token FP8 / int8 rounding (rows8), dequantize8: bit for bit;
- weight-only products (gemv8 / w8a16) and 8-bit x 8-bit products (int8_mm, fp8_mm):
  within the reference's bounds, `0.01 * max|want|` for the weight-only kernels and
  the product of the rounded operands (`python/linnet/tests/test_quant_8bit.py:315-341`);
- the `quantized.*_operands / *_linear` dispatch against the reference CPU path,
  `0.06 * max` where the input is rounded to 8 bits (`test_quant_8bit.py:341`,
  `test_quant_fp8.py:196-220`).
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from linnet_amd.torch import kernels, quantized
from oracle import linear, quant

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLDEN = Path(__file__).parent / "golden"


def _err(got: np.ndarray, want: np.ndarray) -> tuple[float, float]:
    err = float(np.abs(got - want).max()) if got.size else 0.0
    top = float(np.abs(want).max()) if want.size else 0.0
    print(f"max abs err {err:.3e}, rel to max {err / max(top, 1e-30):.3e}")
    return err, top


@pytest.mark.parametrize(("out", "width", "group", "dtype"), [(256, 512, 128, "bf16"), (16, 4096, 4096, "f32"), (7, 96, 32, "f16"), (3, 10, 5, "bf16")])
def test_int8_quantize_matches_numpy(out: int, width: int, group: int, dtype: str) -> None:
    w = np.random.default_rng(out).standard_normal((out, width)).astype(np.float32)
    w[0, :group] = 0.0
    q, s = kernels.quantize_int8(torch.from_numpy(w).to(DEV), group, dtype)
    wq, ws = quant.quantize_int8_groups(w, group, dtype)
    np.testing.assert_array_equal(q.cpu().numpy(), wq)
    np.testing.assert_array_equal(s.cpu().numpy(), ws)


@pytest.mark.parametrize("fp8", [True, False])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
# Widths by the vector kernel's register paths (16-byte vectors a thread keeps:
# 2 / 4 / 8 / read again), for 2-byte inputs: 4096 and 2056 (2; 2056 leaves a
# thread's last vector past the row), 8192 (4), 16384 (8), 20000 (read again);
# f32 rows halve the vector, so 300 takes 2 and 16384 reads again; 300 and 1
# in 2-byte types take the scalar kernel.
@pytest.mark.parametrize(("rows", "width"), [(9, 300), (5, 4096), (3, 2056), (4, 8192), (1, 16384), (2, 20000), (3, 1)])
def test_rows8_matches_the_oracle(fp8: bool, dtype: torch.dtype, rows: int, width: int) -> None:
    g = torch.Generator().manual_seed(rows * 7 + width)
    x = torch.randn(rows, width, generator=g)
    x[0, : min(3, width)] *= 40
    if rows > 2:
        x[2] = 0.0
    x = x.to(dtype)
    q, s = (kernels.fp8_rows if fp8 else kernels.int8_rows)(x.to(DEV))
    wq, ws = quant.rows8(x.float().numpy(), fp8)
    np.testing.assert_array_equal(s.cpu().numpy(), ws)
    np.testing.assert_array_equal(q.cpu().view(torch.uint8 if fp8 else torch.int8).numpy(), wq.view(np.uint8) if fp8 else wq)


def test_rows8_golden_fixture() -> None:
    data = np.load(GOLDEN / "rows8.npz")
    x = torch.from_numpy(data["x_bits"].view(np.int16)).view(torch.bfloat16).to(DEV)
    q, s = kernels.fp8_rows(x)
    np.testing.assert_array_equal(q.view(torch.uint8).cpu().numpy(), data["fp8_q"])
    np.testing.assert_array_equal(s.cpu().numpy(), data["fp8_scale"])
    q, s = kernels.int8_rows(x)
    np.testing.assert_array_equal(q.cpu().numpy(), data["int8_q"])
    np.testing.assert_array_equal(s.cpu().numpy(), data["int8_scale"])


@pytest.mark.parametrize("fp8", [True, False])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize(("group", "row_block"), [(0, 1), (128, 1), (128, 128), (16, 1)])
def test_dequantize8_is_bit_exact(fp8: bool, dtype: torch.dtype, group: int, row_block: int) -> None:
    out, width = 256, 512
    g = torch.Generator().manual_seed(group + row_block)
    full = torch.randn(out, width, generator=g)
    w = (full * 20).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8) if fp8 else (full * 40).round().clamp(-127, 127).to(torch.int8)
    cols = 1 if group == 0 else width // group
    scale = torch.rand(out // row_block if group else out, cols, generator=g) * 0.01 + 1e-4
    if group == 0:
        scale = scale.reshape(-1)
    got = kernels.dequantize8(w.to(DEV), scale.to(DEV), fp8, group, row_block, dtype).cpu()
    widened = w.view(torch.float8_e4m3fn).float() if fp8 else w.float()
    if group == 0:
        full_scale = scale[:, None]
    else:
        full_scale = scale.repeat_interleave(row_block, 0).repeat_interleave(group, 1)
    want = (widened * full_scale).to(dtype)
    assert torch.equal(got.view(torch.int16 if dtype != torch.float32 else torch.int32), want.view(torch.int16 if dtype != torch.float32 else torch.int32))


def _eight_bit(out: int, width: int, fp8: bool, seed: int, group: int = 0, row_block: int = 1):
    g = torch.Generator().manual_seed(seed)
    full = torch.randn(out, width, generator=g) * 0.02
    if group == 0:
        scale = full.abs().amax(1) / (448.0 if fp8 else 127.0)
        wide = scale[:, None]
    else:
        blocked = full.reshape(out // row_block, row_block, width // group, group)
        scale = blocked.abs().amax((1, 3)) / (448.0 if fp8 else 127.0)
        wide = scale.repeat_interleave(row_block, 0).repeat_interleave(group, 1)
    q = (full / wide).to(torch.float8_e4m3fn).view(torch.uint8) if fp8 else (full / wide).round().clamp(-127, 127).to(torch.int8)
    deq = ((q.view(torch.float8_e4m3fn).float() if fp8 else q.float()) * wide).numpy()
    return q, scale.float(), deq


@pytest.mark.parametrize("fp8", [True, False])
@pytest.mark.parametrize(("rows", "out", "group", "row_block", "dtype"), [
    (1, 256, 0, 1, torch.bfloat16), (3, 72, 0, 1, torch.float16), (17, 256, 128, 1, torch.bfloat16),
    (64, 256, 128, 128, torch.bfloat16), (1, 4096, 0, 1, torch.bfloat16), (33, 40, 64, 1, torch.float16),
])
def test_weight_only_kernels(fp8: bool, rows: int, out: int, group: int, row_block: int, dtype: torch.dtype) -> None:
    width = 512
    if group and out % row_block:
        pytest.skip("blocks tile the weight")
    q, scale, deq = _eight_bit(out, width, fp8, seed=rows, group=group, row_block=row_block)
    x = torch.randn(rows, width, generator=torch.Generator().manual_seed(rows)).to(dtype)
    y = kernels.w8a16(x.to(DEV), q.to(DEV), scale.to(DEV), fp8, group, row_block).float().cpu().numpy()
    want = linear.product_f64(x.float().numpy(), deq)
    err, top = _err(y, want)
    assert err <= 0.01 * top


@pytest.mark.parametrize("fp8", [True, False])
@pytest.mark.parametrize(("out", "width", "group", "row_block", "dtype"), [
    (300, 1024, 0, 1, torch.bfloat16), (77, 2048, 128, 1, torch.float16), (256, 4096, 128, 128, torch.bfloat16),
    (40, 384, 0, 1, torch.bfloat16), (1000, 8192, 256, 1, torch.bfloat16), (128, 16384, 0, 1, torch.float16),
    (24, 512, 64, 1, torch.bfloat16), (300, 4096, 0, 1, torch.float16), (40, 4096, 256, 1, torch.bfloat16),
])
def test_one_row_kernels(fp8: bool, out: int, width: int, group: int, row_block: int, dtype: torch.dtype) -> None:
    """One row of x: the wide-read one-row kernels (K % 512 == 0, groups of 128k;
    K = 4096 on the per-wave x slices kernel, with ragged outputs) and the
    skinny kernel's one-row form (the rest), against the f64 product."""
    if group and out % row_block:
        pytest.skip("blocks tile the weight")
    q, scale, deq = _eight_bit(out, width, fp8, seed=out + width, group=group, row_block=row_block)
    x = torch.randn(1, width, generator=torch.Generator().manual_seed(width)).to(dtype)
    y = kernels.gemv8(x.to(DEV), q.to(DEV), scale.to(DEV), fp8, group, row_block).float().cpu().numpy()
    want = linear.product_f64(x.float().numpy(), deq)
    err, top = _err(y, want)
    assert err <= 0.01 * top


@pytest.mark.parametrize("fp8", [True, False])
@pytest.mark.parametrize(("rows", "out", "width"), [(33, 256, 512), (256, 200, 1024), (130, 128, 128), (1, 64, 256)])
def test_8bit_products(fp8: bool, rows: int, out: int, width: int) -> None:
    q, scale, deq = _eight_bit(out, width, fp8, seed=out)
    x = torch.randn(rows, width, generator=torch.Generator().manual_seed(rows)).to(torch.bfloat16)
    qx, xs = (kernels.fp8_rows if fp8 else kernels.int8_rows)(x.to(DEV))
    mm = kernels.fp8_mm if fp8 else kernels.int8_mm
    y = mm(qx, q.to(DEV), xs, scale.to(DEV), torch.bfloat16).float().cpu().numpy()
    want = linear.rows8_product_f64(qx.view(torch.uint8).cpu().numpy() if fp8 else qx.cpu().numpy(), xs.cpu().numpy(), q.numpy().view(np.uint8) if fp8 else q.numpy(), scale.numpy(), fp8)
    err, top = _err(y, want)
    assert err <= 0.01 * top
    exact = linear.product_f64(x.float().numpy(), deq)
    err, top = _err(y, exact)
    assert err <= 0.06 * top


@pytest.mark.parametrize("rows", [1, 3, 17, 64, 100])
@pytest.mark.parametrize("rounded", [0, 1])
@pytest.mark.parametrize("kind", ["fp8", "int8", "int8_group", "fp8_block"])
def test_quantized_dispatch_against_the_reference_cpu_path(kind: str, rounded: int, rows: int) -> None:
    """`test_quant_8bit.py:315-341`: within bf16's rounding of the product with the
    dequantized weight; rounded inputs within 8 bits'."""
    out, width = 256, 512
    fp8 = kind.startswith("fp8")
    group = 128 if kind in ("int8_group", "fp8_block") else 0
    row_block = 128 if kind == "fp8_block" else 1
    q, scale, deq = _eight_bit(out, width, fp8, seed=rows + rounded, group=group, row_block=row_block)
    x = torch.randn(rows, width, generator=torch.Generator().manual_seed(rows)).to(torch.bfloat16)
    bias = torch.randn(out, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    xd, qd, sd, bd = x.to(DEV), q.to(DEV), scale.to(DEV), bias.to(DEV)
    if kind == "fp8":
        got = quantized.fp8_linear(xd, quantized.fp8_operands(qd, sd.to(torch.bfloat16), rounded), bd)
        want = linear.fp8_linear_cpu(x, q.view(torch.float8_e4m3fn), scale.to(torch.bfloat16), bias)
    elif kind == "int8":
        got = quantized.int8_linear(xd, quantized.int8_operands(qd, sd.to(torch.bfloat16), rounded), bd)
        want = linear.int8_linear_cpu(x, q, scale.to(torch.bfloat16), bias)
    elif kind == "int8_group":
        got = quantized.int8_group_linear(xd, quantized.int8_group_operands(qd, sd.to(torch.bfloat16)), bd)
        want = linear.int8_group_linear_cpu(x, q, scale.to(torch.bfloat16), bias)
    else:
        got = quantized.fp8_block_linear(xd, quantized.fp8_block_operands(qd, sd.to(torch.bfloat16), rounded), bd)
        decoded = q.view(torch.float8_e4m3fn).float() * scale.to(torch.bfloat16).float().repeat_interleave(128, 0).repeat_interleave(128, 1)
        want = torch.nn.functional.linear(x, decoded.to(torch.bfloat16)) + bias
    err, top = _err(got.float().cpu().numpy(), want.float().numpy())
    is_rounded = rounded and rows > 32 and kind in ("fp8", "int8", "fp8_block")
    assert err <= (0.06 if is_rounded else 0.01) * top


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize(("rows", "padded", "width"), [(5, 8, 384), (1, 1, 128), (33, 36, 8192), (300, 300, 1152)])
def test_fp8_groups_matches_the_oracle(dtype: torch.dtype, rows: int, padded: int, width: int) -> None:
    """Codes and scales bit for bit, padded rows zero with scale 1, the scales a
    column-major view as `torch._scaled_mm` reads them."""
    g = torch.Generator().manual_seed(rows + width)
    x = (torch.randn(rows, width, generator=g) * torch.logspace(-3, 3, rows)[:, None]).to(dtype)
    x[0, :128] = 0
    q, s = kernels.fp8_groups(x.to(DEV), 128, padded)
    assert q.shape == (padded, width) and s.shape == (padded, width // 128) and s.stride(0) == 1
    want_q, want_s = quant.fp8_groups(x.float().numpy(), 128, padded)
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), want_q)
    assert np.array_equal(s.cpu().numpy(), want_s)


@pytest.mark.parametrize(("rows", "out", "width"), [(1, 128, 128), (37, 256, 384), (300, 384, 1024), (600, 512, 2048), (64, 1024, 8192)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fp8_block_product(rows: int, out: int, width: int, dtype: torch.dtype) -> None:
    """The block-scaled FP8 product of rows rounded per 128 inputs and FP8 weights
    with a scale per 128 x 128 block, against the fp64 block product of the same
    codes and scales (f32 sums and one rounding to 16 bits apart)."""
    g = torch.Generator().manual_seed(rows * 7 + out)
    x = torch.randn(rows, width, generator=g).to(dtype)
    w = torch.randn(out, width, generator=g) * 0.05
    ws = (torch.rand(out // 128, width // 128, generator=g) + 0.5) * 1e-3
    wq = (w / ws.repeat_interleave(128, 0).repeat_interleave(128, 1)).clamp(-448, 448).to(torch.float8_e4m3fn)
    q, xs = kernels.fp8_groups(x.to(DEV), 128, rows)
    y = kernels.fp8_block_mm(q, wq.to(DEV), xs, ws.to(DEV), dtype).float().cpu().numpy()
    want = linear.block_product_f64(q.view(torch.uint8).cpu().numpy(), xs.cpu().numpy(),
                                    wq.view(torch.uint8).numpy(), ws.numpy())
    err, top = _err(y, want)
    assert err <= 8e-3 * top
    assert np.all(np.abs(y - want) <= 8e-3 * np.abs(want) + 1e-3 * top)


def test_fp8_block_product_takes_row_major_scales() -> None:
    """x scales given row-major [rows, In/128] (not `fp8_groups`' view) give the same product."""
    g = torch.Generator().manual_seed(3)
    x = torch.randn(40, 512, generator=g).to(torch.bfloat16)
    wq = (torch.randn(256, 512, generator=g) * 40).clamp(-448, 448).to(torch.float8_e4m3fn)
    ws = torch.rand(2, 4, generator=g) + 0.5
    q, xs = kernels.fp8_groups(x.to(DEV), 128, 40)
    a = kernels.fp8_block_mm(q, wq.to(DEV), xs, ws.to(DEV), torch.bfloat16)
    b = kernels.fp8_block_mm(q, wq.to(DEV), xs.contiguous(), ws.to(DEV), torch.bfloat16)
    assert torch.equal(a, b)


@pytest.mark.parametrize("rows", [1, 256])
def test_fp8_baseline_shape(rows: int) -> None:
    """BASELINE config 4's shape (K=8192, N=28672), per-tensor scale broadcast into
    `Fp8Linear`'s per-row scale, the input rounded a token at a time past 32 rows:
    against dequantize + hipBLASLt within FP8's rounding bound."""
    k, n = 8192, 28672
    g = torch.Generator(device=DEV).manual_seed(0)
    w = torch.randn(n, k, generator=g, device=DEV) * 0.02
    s = (w.abs().max() / 448.0).float()
    q = (w / s).to(torch.float8_e4m3fn)
    scale = s.expand(n).contiguous().to(torch.bfloat16)
    x = torch.randn(rows, k, generator=g, device=DEV).to(torch.bfloat16)
    got = quantized.fp8_linear(x, quantized.fp8_operands(q, scale, 1), None).float()
    deq = kernels.dequantize8(q.view(torch.uint8), scale.float(), True, 0, 1, torch.bfloat16)
    want = (x.float() @ deq.float().T)
    err = (got - want).abs().max().item()
    top = want.abs().max().item()
    print(f"rows {rows}: max abs err {err:.3e} rel {err / top:.3e}")
    assert err <= (0.06 if rows > 32 else 0.01) * top


def test_config1_int8_per_row_gemv() -> None:
    """BASELINE config 1 exactly: W [4096, 4096] ~ N(0, 0.02) (f32, seed 0) quantized
    per row to int8 with f32 scales (`quantize_int8_groups(W, 4096, "f32")`), one bf16
    row of x ~ N(0, 1), through `Int8Linear`'s call (`int8_operands` / `int8_linear`,
    one row -> `gemv8`, the one-scale-a-row form of the one-row kernel), against the
    f64 product with the exactly dequantized weight within `1e-2 * max|want|`, and
    against the reference's CPU path (`quantized.py:193`) within the same bound."""
    g = torch.Generator().manual_seed(0)
    w = (torch.randn(4096, 4096, generator=g) * 0.02).numpy()
    q, scale = quant.quantize_int8_groups(w, 4096, "f32")
    assert scale.shape == (4096, 1)
    x = torch.randn(1, 4096, generator=g).to(torch.bfloat16)
    qt, st = torch.from_numpy(q), torch.from_numpy(scale)
    got = quantized.int8_linear(x.to(DEV), quantized.int8_operands(qt.to(DEV), st.to(DEV), 0), None)
    y = got.float().cpu().numpy()
    want = linear.product_f64(x.float().numpy(), quant.dequantize_int8_groups(q, scale))
    err, top = _err(y, want)
    assert err <= 0.01 * top
    cpu = linear.int8_linear_cpu(x, qt, st, None).float().numpy()
    err, top = _err(y, cpu)
    assert err <= 0.01 * top
