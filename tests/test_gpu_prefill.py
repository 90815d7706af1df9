"""Parity of the prefill products at BASELINE's full shapes, on the GPU, with the
kernel instance that ran pinned by the library's own plan query.

- Config 3 (int4 g128, M = 2048, and config 5's prompt, M = 1024, bf16 x N(0, 1)
  with 0.1% of the input channels scaled x20): a sampled block of 64 rows against the f64 product with the
  exactly dequantized weight (the oracle) within `1e-2 * max|y|`
  (`python/linnet/tests/test_quant_groups.py:194-195`), and the whole output
  against hipBLASLt over the HIP-dequantized weight (the reference's own prefill
  strategy, `src/backend/torch_source.cpp:1561-1566`);
- config 4 (FP8 e4m3 weight with a per-tensor scale, per-token FP8 rows, M =
  4096, K = 8192, N = 28672) and an int8 W8A8 shape, both on the 256-column
  `mm8_kernel`: 64 sampled rows against the f64 product of the rounded operands
  (the oracle) and against the unrounded product within `0.06 * max`
  (`test_quant_fp8.py:196-220`, `test_quant_8bit.py:341`);
- each tile width forced on ragged shapes, bf16 and f16, with a bias.
Max abs / rel errors are printed.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from linnet_amd.torch import kernels, quantized
from oracle import linear, quant

pytestmark = pytest.mark.gpu
DEV = "cuda"
SAMPLE = 64


def _outlier_x(rows: int, k: int, seed: int) -> torch.Tensor:
    """x ~ N(0, 1) bf16 with ceil(0.001 k) input channels (a seeded choice) x20."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, k, generator=g)
    channels = torch.randperm(k, generator=g)[: math.ceil(0.001 * k)]
    x[:, channels] *= 20.0
    return x.to(torch.bfloat16)


def _layer(n: int, k: int, seed: int):
    g = torch.Generator(device=DEV).manual_seed(seed)
    w = torch.randn(n, k, generator=g, device=DEV) * 0.02
    packed, scale, zero = kernels.quantize_int4(w, 128)
    return packed, scale.to(torch.bfloat16), zero


def _report(what: str, got: np.ndarray, want: np.ndarray) -> tuple[float, float]:
    err = float(np.abs(got - want).max())
    top = float(np.abs(want).max())
    print(f"{what}: max abs err {err:.4e}, rel to max|y| {err / top:.4e} (max|y| {top:.4e})", flush=True)
    return err, top


def _sample_rows(rows: int, seed: int) -> np.ndarray:
    return np.sort(np.random.default_rng(seed).choice(rows, size=min(SAMPLE, rows), replace=False))


# At 1024 rows the 128-column kernel runs 128-row tiles (256-row tiles would
# leave more than half the compute units idle); at 2048 rows, 256-row tiles.
# 224 tiles of 256 x 256 (1024 rows, N = 14336) fill 7/8 of the CUs: the
# 256-column kernel; at 2048 rows, 448 tiles, the persistent 256 x 256 form.
@pytest.mark.parametrize(("rows", "k", "n", "want_kernel"), [
    (2048, 4096, 14336, "persistent"), (2048, 4096, 4096, "tiled128"), (2048, 14336, 4096, "tiled128"),
    (1024, 14336, 4096, "tiled128"), (1024, 4096, 14336, "tiled256"),
])
def test_config3_prefill_matches_the_oracle(rows: int, k: int, n: int, want_kernel: str) -> None:
    print(f"config 3 rows={rows} k={k} n={n}", flush=True)
    assert kernels.int4_linear_plan(rows, k, n, 128) == want_kernel
    packed, scale, zero = _layer(n, k, seed=k + n)
    x = _outlier_x(rows, k, seed=k)
    xd = x.to(DEV)
    y = kernels.int4_linear(xd, packed, scale, zero)
    # The oracle on a sampled block of rows: f64 product with the exact weight.
    pick = _sample_rows(rows, seed=n)
    ref = linear.int4_reference_f64(x[pick].float().numpy(), packed.cpu().numpy(), scale.float().cpu().numpy(),
                                    zero.cpu().numpy())
    err, top = _report(f"int4 {want_kernel} vs f64 oracle ({len(pick)} rows)", y[pick].float().cpu().numpy(), ref)
    assert err <= 1e-2 * top
    # All rows: the reference's prefill strategy (dequantize, then the BLAS GEMM).
    w = kernels.int4_weight(packed, scale, zero)
    full = (xd.float() @ w.float().T)
    err, top = _report(f"int4 {want_kernel} vs dequantize + GEMM (all rows)", y.float().cpu().numpy(), full.cpu().numpy())
    assert err <= 1e-2 * top
    # Another prefill kernel agrees within bf16 rounding.
    other = "tiled256" if want_kernel == "tiled128" else "tiled128"
    y2 = kernels.int4_linear(xd, packed, scale, zero, kernel=other).float()
    assert (y2 - y.float()).abs().max().item() <= 1e-2 * top


@pytest.mark.parametrize("tile", ["tiled128", "tiled256"])
@pytest.mark.parametrize(("rows", "k", "n", "group", "dtype"), [
    (300, 1024, 200, 128, torch.bfloat16),  # ragged rows and columns, one partial tile of each
    (517, 2048, 1000, 64, torch.float16),
    (256, 512, 768, 32, torch.bfloat16),
    (96, 4096, 520, 256, torch.float16),
])
def test_each_tile_width_on_ragged_shapes(tile: str, rows: int, k: int, n: int, group: int, dtype: torch.dtype) -> None:
    print(f"{tile} rows={rows} k={k} n={n} group={group} {dtype}", flush=True)
    assert kernels.int4_linear_plan(rows, k, n, group, dtype, kernel=tile) == tile
    g = torch.Generator().manual_seed(rows + n)
    packed = torch.randint(0, 256, (n, k // group, group // 2), generator=g, dtype=torch.uint8)
    scale = (torch.rand(n, k // group, generator=g) * 0.02 + 0.001).to(dtype)
    zero = torch.randint(0, 16, (n, k // group), generator=g, dtype=torch.uint8)
    x = _outlier_x(rows, k, seed=rows).to(dtype)
    bias = torch.randn(n, generator=g).to(dtype)
    args = (packed.to(DEV), scale.to(DEV), zero.to(DEV))
    y = kernels.int4_linear(x.to(DEV), *args, kernel=tile)
    ref = linear.int4_reference_f64(x.float().numpy(), packed.numpy(), scale.float().numpy(), zero.numpy())
    err, top = _report(f"{tile} vs f64 oracle", y.float().cpu().numpy(), ref)
    assert err <= 1e-2 * top
    # the bias: the rounded product plus the bias, rounded again
    assert torch.equal(kernels.int4_linear(x.to(DEV), *args, bias.to(DEV), kernel=tile), y + bias.to(DEV))


def _fp8_weight(n: int, k: int, seed: int):
    g = torch.Generator(device=DEV).manual_seed(seed)
    w = torch.randn(n, k, generator=g, device=DEV) * 0.02
    s = (w.abs().max() / 448.0).float()
    return (w / s).to(torch.float8_e4m3fn), s


def test_config4_fp8_at_4096_rows_runs_the_persistent_form() -> None:
    rows, k, n = 4096, 8192, 28672
    print(f"config 4 rows={rows} k={k} n={n}", flush=True)
    assert kernels.mm8_plan(rows, n, k) == kernels.MM8_PERSISTENT
    q, s = _fp8_weight(n, k, seed=0)
    scale = s.expand(n).contiguous().to(torch.bfloat16)
    x = torch.randn(rows, k, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    xd = x.to(DEV)
    got = quantized.fp8_linear(xd, quantized.fp8_operands(q, scale, 1), None)
    qx, xs = kernels.fp8_rows(xd)
    assert torch.equal(got, kernels.fp8_mm(qx, q, xs, scale.float(), torch.bfloat16, tile_n=256))
    pick = _sample_rows(rows, seed=1)
    qx_s = qx[pick].cpu().view(torch.uint8).numpy()
    ref = linear.rows8_product_f64(qx_s, xs[pick].cpu().numpy(), q.cpu().view(torch.uint8).numpy(),
                                   scale.float().cpu().numpy(), True)
    err, top = _report("fp8 mm8p vs f64 product of the rounded operands", got[pick].float().cpu().numpy(), ref)
    assert err <= 1e-2 * top
    unrounded = linear.product_f64(x[pick].float().numpy(),
                                   (q.float() * scale.float()[:, None]).cpu().numpy())
    err, top = _report("fp8 mm8p vs f64 product of unrounded x", got[pick].float().cpu().numpy(), unrounded)
    assert err <= 0.06 * top
    narrow = kernels.fp8_mm(qx, q, xs, scale.float(), torch.bfloat16, tile_n=128)
    assert (narrow.float() - got.float()).abs().max().item() <= 1e-2 * top


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_int8_w8a8_at_256_wide_tiles(dtype: torch.dtype) -> None:
    """int8 rows x int8 weights (sums exact in int32) at 2048 x 8192 x 4096: 256 tiles of 256 columns."""
    rows, k, n = 2048, 4096, 8192
    print(f"int8 W8A8 rows={rows} k={k} n={n} {dtype}", flush=True)
    assert kernels.mm8_plan(rows, n, k, fp8=False) == 256
    g = torch.Generator(device=DEV).manual_seed(2)
    w = torch.randn(n, k, generator=g, device=DEV) * 0.02
    wq, ws = kernels.quantize_int8(w, k, "f32")
    x = _outlier_x(rows, k, seed=5).to(dtype)
    qx, xs = kernels.int8_rows(x.to(DEV))
    got = kernels.int8_mm(qx, wq, xs, ws.reshape(-1), dtype)
    assert torch.equal(got, kernels.int8_mm(qx, wq, xs, ws.reshape(-1), dtype, tile_n=256))
    pick = _sample_rows(rows, seed=3)
    ref = linear.rows8_product_f64(qx[pick].cpu().numpy(), xs[pick].cpu().numpy(), wq.cpu().numpy(),
                                   ws.cpu().numpy(), False)
    y = got[pick].float().cpu().numpy()
    err, top = _report("int8 mm8<256> vs f64 product of the rounded operands", y, ref)
    # exact int32 sums, two f32 scalings and one rounding to 16 bits per element
    ulp = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    assert np.all(np.abs(y - ref) <= ulp * np.abs(ref) + 1e-6 * top)
    narrow = kernels.int8_mm(qx, wq, xs, ws.reshape(-1), dtype, tile_n=128)
    assert torch.equal(narrow, got)


@pytest.mark.parametrize("fp8", [True, False])
@pytest.mark.parametrize("tile_n", [128, 256])
def test_mm8_tile_widths_on_ragged_shapes(fp8: bool, tile_n: int) -> None:
    rows, k, n = 333, 1024, 700
    print(f"mm8 fp8={fp8} tile_n={tile_n} rows={rows} k={k} n={n}", flush=True)
    g = torch.Generator().manual_seed(rows + tile_n)
    x = _outlier_x(rows, k, seed=9)
    if fp8:
        wq = (torch.randn(n, k, generator=g) * 40).clamp(-448, 448).to(torch.float8_e4m3fn)
        ws = torch.rand(n, generator=g) * 0.01 + 0.001
        qx, xs = kernels.fp8_rows(x.to(DEV))
        got = kernels.fp8_mm(qx, wq.to(DEV), xs, ws.to(DEV), torch.bfloat16, tile_n=tile_n)
        wbytes = wq.view(torch.uint8).numpy()
        qxb = qx.cpu().view(torch.uint8).numpy()
    else:
        wq = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
        ws = torch.rand(n, generator=g) * 0.01 + 0.001
        qx, xs = kernels.int8_rows(x.to(DEV))
        got = kernels.int8_mm(qx, wq.to(DEV), xs, ws.to(DEV), torch.bfloat16, tile_n=tile_n)
        wbytes = wq.numpy()
        qxb = qx.cpu().numpy()
    ref = linear.rows8_product_f64(qxb, xs.cpu().numpy(), wbytes, ws.numpy(), fp8)
    err, top = _report(f"mm8<{tile_n}> fp8={fp8}", got.float().cpu().numpy(), ref)
    assert err <= 1e-2 * top


def test_fp8_rounded_quantize_matches_the_oracle_at_config4_width() -> None:
    """The per-token FP8 rows of config 4's input (8192 wide, outlier channels): bit for bit."""
    x = _outlier_x(64, 8192, seed=11)
    q, s = kernels.fp8_rows(x.to(DEV))
    wq, ws = quant.rows8(x.float().numpy(), True)
    np.testing.assert_array_equal(s.cpu().numpy(), ws)
    np.testing.assert_array_equal(q.cpu().view(torch.uint8).numpy(), wq.view(np.uint8))


@pytest.mark.parametrize("fp8", [True, False])
@pytest.mark.parametrize(("rows", "k", "n"), [(333, 1024, 768), (1100, 512, 14336), (4096, 8192, 28672), (7, 256, 256)])
def test_mm8_persistent_form(fp8: bool, rows: int, k: int, n: int) -> None:
    """The persistent 256 x 256 form (one workgroup a CU walking its tiles; 1100
    rows x 14336 columns: 280 tiles, some workgroups two) against the f64 product
    of the rounded operands, and bit for bit against the 256-column tile kernel,
    which sums the same MFMAs in the same k order."""
    print(f"mm8 persistent fp8={fp8} rows={rows} k={k} n={n}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(rows + k)
    x = torch.randn(rows, k, generator=g, device=DEV).to(torch.bfloat16)
    if fp8:
        wq = (torch.randn(n, k, generator=g, device=DEV) * 40).clamp(-448, 448).to(torch.float8_e4m3fn)
        ws = torch.rand(n, generator=g, device=DEV) * 0.01 + 0.001
        qx, xs = kernels.fp8_rows(x)
        run = lambda t: kernels.fp8_mm(qx, wq, xs, ws, torch.bfloat16, tile_n=t)  # noqa: E731
    else:
        wq = torch.randint(-127, 128, (n, k), generator=g, device=DEV, dtype=torch.int8)
        ws = torch.rand(n, generator=g, device=DEV) * 0.01 + 0.001
        qx, xs = kernels.int8_rows(x)
        run = lambda t: kernels.int8_mm(qx, wq, xs, ws, torch.bfloat16, tile_n=t)  # noqa: E731
    got = run(kernels.MM8_PERSISTENT)
    assert torch.equal(got, run(256))
    pick = _sample_rows(rows, seed=2) if rows > 64 else np.arange(rows)
    wbytes = wq.cpu().view(torch.uint8).numpy() if fp8 else wq.cpu().numpy()
    qxb = qx[pick].cpu().view(torch.uint8).numpy() if fp8 else qx[pick].cpu().numpy()
    ref = linear.rows8_product_f64(qxb, xs[pick].cpu().numpy(), wbytes, ws.cpu().numpy(), fp8)
    err, top = _report(f"mm8 persistent fp8={fp8}", got[pick].float().cpu().numpy(), ref)
    assert err <= 1e-2 * top


def test_mm8_persistent_form_refuses_other_shapes() -> None:
    from linnet_amd.errors import LinnetError

    qx = torch.zeros(8, 256, dtype=torch.int8, device=DEV)
    xs = torch.ones(8, 1, device=DEV)
    for n, k in ((200, 256), (256, 384)):
        w = torch.zeros(n, k, dtype=torch.int8, device=DEV)
        with pytest.raises(LinnetError, match="persistent form"):
            kernels.int8_mm(qx[:, :k] if k <= 256 else torch.zeros(8, k, dtype=torch.int8, device=DEV), w, xs,
                            torch.ones(n, device=DEV), torch.bfloat16, tile_n=kernels.MM8_PERSISTENT)


@pytest.mark.parametrize("fp8", [True, False])
@pytest.mark.parametrize(("rows", "k", "n", "dtype"), [
    (256, 8192, 28672, torch.bfloat16),  # config 4 at 256 rows: 224 tiles, 64 steps (5 cycles of 12, 4 more)
    (333, 1024, 700, torch.bfloat16),    # ragged rows and columns, 8 steps: no full cycle
    (7, 128, 256, torch.float16),        # one step: later stages loaded from past K (zeros)
    (40, 1536, 4096, torch.bfloat16),    # 12 steps: one full cycle, nothing after it
])
def test_mm8_streaming_form(fp8: bool, rows: int, k: int, n: int, dtype: torch.dtype) -> None:
    """The weight-streaming form (x and weights in stages of their own, loaded by
    waves of their own) bit for bit against the 128-column tile kernel, which
    sums the same MFMAs in the same k order, and against the f64 product of the
    rounded operands."""
    print(f"mm8 streaming fp8={fp8} rows={rows} k={k} n={n} {dtype}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(rows + n)
    x = torch.randn(rows, k, generator=g, device=DEV).to(dtype)
    if fp8:
        wq = (torch.randn(n, k, generator=g, device=DEV) * 40).clamp(-448, 448).to(torch.float8_e4m3fn)
        ws = torch.rand(n, generator=g, device=DEV) * 0.01 + 0.001
        qx, xs = kernels.fp8_rows(x)
        run = lambda t: kernels.fp8_mm(qx, wq, xs, ws, dtype, tile_n=t)  # noqa: E731
    else:
        wq = torch.randint(-127, 128, (n, k), generator=g, device=DEV, dtype=torch.int8)
        ws = torch.rand(n, generator=g, device=DEV) * 0.01 + 0.001
        qx, xs = kernels.int8_rows(x)
        run = lambda t: kernels.int8_mm(qx, wq, xs, ws, dtype, tile_n=t)  # noqa: E731
    got = run(kernels.MM8_STREAM)
    assert torch.equal(got, run(128))
    if kernels.mm8_plan(rows, n, k, fp8) == kernels.MM8_STREAM:
        assert torch.equal(got, run(0))
    pick = _sample_rows(rows, seed=4) if rows > 64 else np.arange(rows)
    wbytes = wq.cpu().view(torch.uint8).numpy() if fp8 else wq.cpu().numpy()
    qxb = qx[pick].cpu().view(torch.uint8).numpy() if fp8 else qx[pick].cpu().numpy()
    ref = linear.rows8_product_f64(qxb, xs[pick].cpu().numpy(), wbytes, ws.cpu().numpy(), fp8)
    err, top = _report(f"mm8 streaming fp8={fp8}", got[pick].float().cpu().numpy(), ref)
    assert err <= 1e-2 * top


@pytest.mark.parametrize(("rows", "k", "n", "group", "dtype"), [
    (333, 1024, 768, 128, torch.bfloat16),   # a partial row tile
    (1100, 512, 14336, 128, torch.bfloat16),  # 280 tiles: some workgroups two
    (2048, 4096, 14336, 128, torch.bfloat16),  # config 3
    (96, 2048, 512, 256, torch.float16),
    (7, 256, 256, 64, torch.bfloat16),        # one tile of one group of steps
])
def test_int4_persistent_form(rows: int, k: int, n: int, group: int, dtype: torch.dtype) -> None:
    """The persistent 256 x 256 dequant-GEMM against the f64 product of the
    dequantized weight (sampled rows), and against the 256-column tiled kernel."""
    print(f"int4 persistent rows={rows} k={k} n={n} group={group} {dtype}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(rows + k)
    w = torch.randn(n, k, generator=g, device=DEV) * 0.02
    packed, scale, zero = kernels.quantize_int4(w, group)
    scale = scale.to(dtype)
    x = torch.randn(rows, k, generator=g, device=DEV).to(dtype)
    bias = torch.randn(n, generator=g, device=DEV).to(dtype)
    got = kernels.int4_linear(x, packed, scale, zero, kernel="persistent")
    pick = _sample_rows(rows, seed=5) if rows > 64 else np.arange(rows)
    wdq = kernels.int4_weight(packed, scale, zero).float().cpu().numpy().astype(np.float64)
    ref = x[pick].float().cpu().numpy().astype(np.float64) @ wdq.T
    err, top = _report("int4 persistent", got[pick].float().cpu().numpy(), ref)
    assert err <= 1e-2 * top
    tiled = kernels.int4_linear(x, packed, scale, zero, kernel="tiled256").float()
    assert (got.float() - tiled).abs().max().item() <= 1e-2 * top
    with_bias = kernels.int4_linear(x, packed, scale, zero, bias, kernel="persistent")
    assert torch.equal(with_bias, (got.float() + bias.float()).to(dtype))


def test_int4_persistent_form_refuses_other_shapes() -> None:
    from linnet_amd.errors import LinnetError

    for n, k, group in ((200, 256, 128), (256, 384, 128), (256, 256, 32)):
        packed = torch.zeros(n, k // group, group // 2, dtype=torch.uint8, device=DEV)
        scale = torch.ones(n, k // group, dtype=torch.bfloat16, device=DEV)
        zero = torch.zeros(n, k // group, dtype=torch.uint8, device=DEV)
        x = torch.zeros(300, k, dtype=torch.bfloat16, device=DEV)
        with pytest.raises(LinnetError, match="persistent kernel"):
            kernels.int4_linear(x, packed, scale, zero, kernel="persistent")
