"""Parity of the int4 HIP path with the oracle, on the GPU, through the C ABI.

- quantize / pack / unpack / dequantize: bit for bit;
- linear (skinny MFMA kernel and tiled dequant-GEMM): within `1e-2 * max|y|` of the
  f64 product with the exactly dequantized weight -- the reference's bound for its
  int4 kernel (`python/linnet/tests/test_quant_groups.py:194-195`) -- and against
  the reference CPU path's bf16 output; max abs / rel errors are printed;
- full BASELINE sizes through size-independent properties (linearity in x,
  agreement between the two kernels, and dequantize-then-GEMM).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from linnet_amd.torch import generated, kernels
from oracle import linear, quant

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _layer(out: int, width: int, group: int, seed: int, dtype: torch.dtype = torch.bfloat16):
    """Random packed bytes, scales of the model dtype, zero points 0..15 (as
    `tests/test_quant_groups.py:178-185` draws them)."""
    g = torch.Generator().manual_seed(seed)
    packed = torch.randint(0, 256, (out, width // group, group // 2), generator=g, dtype=torch.uint8)
    scale = (torch.rand(out, width // group, generator=g) * 0.02 + 0.001).to(dtype)
    zero = torch.randint(0, 16, (out, width // group), generator=g, dtype=torch.uint8)
    return packed, scale, zero


def _check_linear(x: torch.Tensor, packed, scale, zero, y: torch.Tensor, bias=None, bound: float = 1e-2) -> None:
    ref = linear.int4_reference_f64(x.float().cpu().numpy(), packed.cpu().numpy(), scale.float().cpu().numpy(), zero.cpu().numpy())
    if bias is not None:
        ref = ref + bias.float().cpu().numpy()[None, :]
    got = y.float().cpu().numpy()
    err = np.abs(got - ref)
    scale_ = np.abs(ref).max()
    print(f"max abs err {err.max():.3e}, rel to max|y| {err.max() / max(scale_, 1e-30):.3e}")
    assert got.shape == ref.shape
    assert err.max() <= bound * scale_


# --------------------------------------------------------------- codes, bytes


@pytest.mark.parametrize(("out", "width", "group"), [(64, 256, 128), (72, 512, 32), (33, 4096, 4096), (8, 96, 48), (5, 6, 2)])
def test_quantize_matches_numpy_bit_for_bit(out: int, width: int, group: int) -> None:
    rng = np.random.default_rng(out)
    w = (rng.standard_normal((out, width)) * 0.02).astype(np.float32)
    w[0, :group] = 0.125  # a constant group
    want = quant.quantize_int4_groups(w, group)
    got = kernels.quantize_int4(torch.from_numpy(w).to(DEV), group)
    for a, b in zip(got, want):
        np.testing.assert_array_equal(a.cpu().numpy(), b)


def test_quantize_matches_the_golden_fixture() -> None:
    from pathlib import Path

    data = np.load(Path(__file__).parent / "golden" / "int4_quantize.npz")
    packed, scale, zero = kernels.quantize_int4(torch.from_numpy(data["weight"]).to(DEV), int(data["group"]))
    np.testing.assert_array_equal(packed.cpu().numpy(), data["packed"])
    np.testing.assert_array_equal(scale.cpu().numpy(), data["scale"])
    np.testing.assert_array_equal(zero.cpu().numpy(), data["zero"])


def test_pack_and_unpack() -> None:
    g = torch.Generator().manual_seed(1)
    codes = torch.randint(-40, 40, (7, 10, 64), generator=g, dtype=torch.int64)
    got = kernels.pack4(codes.to(DEV)).cpu().numpy()
    np.testing.assert_array_equal(got, quant.pack4(codes.numpy(), "u4"))
    floats = torch.tensor([7.9, -8.2, 2.7, -9.5, 15.0, 16.0], dtype=torch.float32)
    np.testing.assert_array_equal(kernels.pack4(floats.to(DEV)).cpu().numpy(), quant.pack4(floats.numpy(), "i4"))
    for kind in ("u4", "i4"):
        np.testing.assert_array_equal(kernels.unpack4(torch.from_numpy(got).to(DEV), kind).cpu().numpy(), quant.unpack4(got, kind))
    empty = kernels.pack4(torch.zeros(0, 4, dtype=torch.int64, device=DEV))
    assert empty.shape == (0, 2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize(("out", "width", "group"), [(72, 512, 128), (16, 256, 32), (9, 192, 64), (4, 12, 6), (3, 4096, 4096)])
def test_dequantize_is_bit_exact(dtype: torch.dtype, out: int, width: int, group: int) -> None:
    """Bit for bit the reference's `(q.to(T) - z.to(T)) * s` (`tests/test_quant_groups.py:151-162`)."""
    packed, scale, zero = _layer(out, width, group, seed=out + width, dtype=dtype)
    got = kernels.int4_weight(packed.to(DEV), scale.to(DEV), zero.to(DEV)).cpu()
    levels = torch.stack([packed & 15, packed >> 4], dim=-1).reshape(out, width // group, group)
    want = ((levels.to(dtype) - zero.to(dtype)[..., None]) * scale[..., None]).reshape(out, width)
    assert torch.equal(got.view(torch.int16 if dtype != torch.float32 else torch.int32),
                       want.view(torch.int16 if dtype != torch.float32 else torch.int32))


# ------------------------------------------------------------------- linear


@pytest.mark.parametrize(
    ("rows", "group", "out", "dtype"),
    [
        (1, 128, 72, torch.bfloat16),  # decode, ragged outputs
        (3, 128, 64, torch.bfloat16),
        (4, 32, 72, torch.float16),
        (8, 128, 72, torch.bfloat16),  # test_quant_groups.py:169
        (16, 64, 8448, torch.bfloat16),
        (24, 128, 8448, torch.bfloat16),  # test_quant_groups.py:172
        (37, 32, 72, torch.float16),  # test_quant_groups.py:170
        (64, 256, 40, torch.bfloat16),
        (128, 64, 72, torch.bfloat16),  # test_quant_groups.py:171
        (160, 128, 64, torch.bfloat16),
        (300, 32, 200, torch.float16),
    ],
)
def test_int4_linear_multiplies_the_dequantized_weight(rows: int, group: int, out: int, dtype: torch.dtype) -> None:
    width = 512
    packed, scale, zero = _layer(out, width, group, seed=rows, dtype=dtype)
    x = torch.randn(rows, width, generator=torch.Generator().manual_seed(rows)).to(dtype)
    y = kernels.int4_linear(x.to(DEV), packed.to(DEV), scale.to(DEV), zero.to(DEV))
    assert y.shape == (rows, out) and y.dtype == dtype
    _check_linear(x, packed, scale, zero, y)


@pytest.mark.parametrize("kernel", ["skinny", "tiled"])
@pytest.mark.parametrize("rows", [1, 17, 64, 257])
def test_both_kernels_at_any_rows(kernel: str, rows: int) -> None:
    packed, scale, zero = _layer(96, 1024, 128, seed=7)
    x = torch.randn(rows, 1024, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    y = kernels.int4_linear(x.to(DEV), packed.to(DEV), scale.to(DEV), zero.to(DEV), kernel=kernel)
    _check_linear(x, packed, scale, zero, y)


def test_bias_is_added_after_the_rounded_product() -> None:
    """`y + bias` of the reference (`torch_source.cpp:1569-1570`): the bf16 product
    plus the bias, rounded again -- bit for bit the unfused composition."""
    packed, scale, zero = _layer(80, 256, 128, seed=11)
    bias = torch.randn(80, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    for rows, kernel in ((2, "skinny"), (70, "tiled")):
        x = torch.randn(rows, 256, generator=torch.Generator().manual_seed(rows)).to(torch.bfloat16).to(DEV)
        args = (packed.to(DEV), scale.to(DEV), zero.to(DEV))
        fused = kernels.int4_linear(x, *args, bias.to(DEV), kernel=kernel)
        plain = kernels.int4_linear(x, *args, kernel=kernel) + bias.to(DEV)
        assert torch.equal(fused, plain)


def test_generated_helpers_match_the_reference_cpu_path() -> None:
    """`_int4_pack` / `_int4_linear` against the reference's CPU generated path (bf16
    F.linear over the dequantized weight), on the same seeded inputs."""
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((256, 512)) * 0.02).astype(np.float32)
    p_np, s_np, z_np = quant.quantize_int4_groups(w, 128)
    p = torch.from_numpy(p_np)
    s = torch.from_numpy(quant.to_bf16_bits(s_np).view(np.int16)).view(torch.bfloat16)
    z = torch.from_numpy(z_np)
    bias = torch.randn(256, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    prepared = generated._int4_pack(p.to(DEV), s.to(DEV), z.to(DEV))
    assert len(prepared) == 3
    cpu_prepared = linear.int4_prepare_cpu(p, s, z)
    for rows in (1, 5, 33, 300):
        x = torch.randn(2, rows, 512, generator=torch.Generator().manual_seed(rows)).to(torch.bfloat16)
        got = generated._int4_linear(x.to(DEV), prepared, bias.to(DEV), p.to(DEV), s.to(DEV), z.to(DEV)).cpu()
        want = linear.int4_linear_generated_cpu(x, cpu_prepared, bias)
        assert got.shape == want.shape == (2, rows, 256)
        err = (got.float() - want.float()).abs().max().item()
        bound = 1e-2 * want.float().abs().max().item()
        print(f"rows {rows}: max abs err vs reference CPU path {err:.3e} (bound {bound:.3e})")
        assert err <= bound


def test_unsupported_groups_fall_back_to_the_dequantized_weight() -> None:
    """A group of 16 (or f32 scales) takes the reference's fallback: the weight
    dequantized once (here by the HIP kernel), then F.linear."""
    packed, scale, zero = _layer(32, 256, 16, seed=3)
    prepared = generated._int4_pack(packed.to(DEV), scale.to(DEV), zero.to(DEV))
    assert len(prepared) == 1
    x = torch.randn(3, 256, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)
    y = generated._int4_linear(x.to(DEV), prepared, None, packed.to(DEV), scale.to(DEV), zero.to(DEV))
    _check_linear(x, packed, scale, zero, y)


# ------------------------------------------------------------- one-token GEMV


@pytest.mark.parametrize(
    ("out", "width", "group", "dtype"),
    [
        (56, 4096, 128, torch.bfloat16),  # one 56-row workgroup (the 14336-row split)
        (100, 4096, 128, torch.bfloat16),  # ragged last workgroup
        (5, 256, 128, torch.bfloat16),  # one wave, 5 of 8 rows
        (2049, 1024, 128, torch.float16),  # 16 rows a workgroup, one row over
        (1024, 512, 256, torch.bfloat16),  # group 256: both halves share a group
        (300, 2048, 512, torch.float16),
        (4000, 768, 128, torch.bfloat16),  # 3 waves, 16 rows a workgroup
        (9000, 4096, 128, torch.bfloat16),  # 40 rows a workgroup (U8 = 5)
        (16384, 256, 128, torch.bfloat16),  # 64 rows a workgroup (U8 = 8)
        (6144, 1280, 128, torch.float16),  # 24 rows a workgroup (U8 = 3)
        (12288, 512, 128, torch.bfloat16),  # U8 = 6
        (8192, 256, 256, torch.bfloat16),  # U8 = 4
        (14336, 4096, 128, torch.bfloat16),  # the decode shape: 256 workgroups of 56 rows
        (1000, 2048, 128, torch.bfloat16),  # 8 waves, ragged last workgroup
        (4096, 4096, 256, torch.float16),  # group 256, 16 rows a workgroup
        # K > 4096: S slices of 256 inputs a wave
        (4096, 14336, 128, torch.bfloat16),  # the down projection: S = 4, 14 waves, 16 rows
        (24, 14336, 128, torch.float16),  # S = 4, one ragged 8-row workgroup
        (8192, 8192, 128, torch.bfloat16),  # S = 2, 16 waves, 32 rows
        (1000, 8192, 256, torch.float16),  # S = 2, group 256, 8 rows
        (5000, 6144, 128, torch.bfloat16),  # S = 2, 12 waves, 24 rows (odd U8)
        (3000, 12288, 1024, torch.bfloat16),  # S = 3, group 1024, 16 rows
        (20000, 1024, 128, torch.bfloat16),  # past 16384 outputs: two whole rounds, 500 workgroups of 40 rows
        (28672, 1024, 128, torch.bfloat16),  # two whole rounds: 512 workgroups of 56 rows (odd U8)
        (40008, 512, 128, torch.float16),  # three rounds: 715 workgroups of 56 rows, ragged last
    ],
)
def test_one_token_gemv_multiplies_the_dequantized_weight(out: int, width: int, group: int, dtype: torch.dtype) -> None:
    packed, scale, zero = _layer(out, width, group, seed=out + width, dtype=dtype)
    x = torch.randn(1, width, generator=torch.Generator().manual_seed(width)).to(dtype)
    args = (packed.to(DEV), scale.to(DEV), zero.to(DEV))
    y = kernels.int4_linear(x.to(DEV), *args, kernel="gemv")
    assert y.shape == (1, out) and y.dtype == dtype
    _check_linear(x, packed, scale, zero, y)
    # the skinny kernel sums in another order: the two agree within bf16 rounding
    other = kernels.int4_linear(x.to(DEV), *args, kernel="skinny").float()
    assert (y.float() - other).abs().max().item() <= 1e-2 * other.abs().max().item()


@pytest.mark.parametrize(("rows", "out"), [(17, 8192), (32, 8192), (45, 8192), (64, 8192), (5, 20000), (32, 20000),
                                           (34, 20000), (19, 28672)])
def test_wide_outputs_run_the_gemv_per_32_rows(rows: int, out: int) -> None:
    """5..64 rows over N >= 8192: the automatic choice runs the few-token GEMV
    once per 32-row chunk (with a ragged last chunk and the bias in each); past
    16384 outputs with more workgroups than CUs."""
    packed, scale, zero = _layer(out, 1024, 128, seed=rows)
    x = torch.randn(rows, 1024, generator=torch.Generator().manual_seed(rows)).to(torch.bfloat16)
    bias = torch.randn(out, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(DEV)
    args = (packed.to(DEV), scale.to(DEV), zero.to(DEV))
    assert kernels.int4_linear_plan(rows, 1024, out, 128) == "gemv"
    y = kernels.int4_linear(x.to(DEV), *args)
    _check_linear(x, packed, scale, zero, y)
    for c in range(0, rows, 32):
        assert torch.equal(y[c:c + 32], kernels.int4_linear(x[c:c + 32].to(DEV), *args, kernel="gemv"))
    assert torch.equal(kernels.int4_linear(x.to(DEV), *args, bias), y + bias)


def test_out_receives_the_product() -> None:
    packed, scale, zero = _layer(96, 512, 128, seed=8)
    args = (packed.to(DEV), scale.to(DEV), zero.to(DEV))
    for rows in (1, 3, 80):
        x = torch.randn(rows, 512, generator=torch.Generator().manual_seed(rows)).to(torch.bfloat16).to(DEV)
        out = torch.full((rows, 96), float("nan"), dtype=torch.bfloat16, device=DEV)
        got = kernels.int4_linear(x, *args, out=out)
        assert got.data_ptr() == out.data_ptr()
        assert torch.equal(out, kernels.int4_linear(x, *args))


def test_one_token_gemv_bias_is_added_after_the_rounded_product() -> None:
    packed, scale, zero = _layer(120, 1024, 128, seed=21)
    bias = torch.randn(120, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).to(DEV)
    x = torch.randn(1, 1024, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16).to(DEV)
    args = (packed.to(DEV), scale.to(DEV), zero.to(DEV))
    fused = kernels.int4_linear(x, *args, bias, kernel="gemv")
    plain = kernels.int4_linear(x, *args, kernel="gemv") + bias
    assert torch.equal(fused, plain)


def test_one_token_gemv_is_chosen_for_one_row_and_refuses_other_shapes() -> None:
    from linnet_amd.errors import LinnetError

    packed, scale, zero = _layer(64, 512, 32, seed=2)
    x = torch.randn(1, 512, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).to(DEV)
    with pytest.raises(LinnetError, match="one-token kernel"):
        kernels.int4_linear(x, packed.to(DEV), scale.to(DEV), zero.to(DEV), kernel="gemv")
    # group 32 at one row: auto falls back to the skinny kernel
    _check_linear(x.cpu(), packed, scale, zero, kernels.int4_linear(x, packed.to(DEV), scale.to(DEV), zero.to(DEV)))
    packed, scale, zero = _layer(64, 512, 128, seed=2)
    x33 = torch.randn(33, 512, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).to(DEV)
    with pytest.raises(LinnetError, match="one-token kernel"):
        kernels.int4_linear(x33, packed.to(DEV), scale.to(DEV), zero.to(DEV), kernel="gemv")


@pytest.mark.parametrize(
    ("rows", "out", "width", "group", "dtype"),
    [
        (2, 14336, 4096, 128, torch.bfloat16),  # config 2 shape, U8 = 7 (a last 8-row tile)
        (4, 14336, 4096, 128, torch.bfloat16),
        (16, 14336, 4096, 128, torch.bfloat16),
        (3, 4096, 4096, 128, torch.float16),  # U8 = 2
        (5, 2049, 1024, 128, torch.bfloat16),  # U8 = 2, ragged last workgroup, 16-row form
        (8, 6144, 1280, 256, torch.bfloat16),  # group 256, U8 = 3, 5 waves
        (16, 16384, 256, 128, torch.float16),  # U8 = 8, one wave
        (12, 100, 4096, 128, torch.bfloat16),  # one short workgroup
        (17, 14336, 4096, 128, torch.bfloat16),  # 32-row form: config 2 shape, U8 = 7
        (32, 14336, 4096, 128, torch.bfloat16),
        (24, 4096, 4096, 128, torch.float16),  # U8 = 2
        (32, 2049, 1024, 128, torch.bfloat16),  # ragged last workgroup
        (20, 6144, 1280, 256, torch.bfloat16),  # group 256, U8 = 3, 5 waves
        (32, 16384, 256, 128, torch.float16),  # U8 = 8, one wave
        (31, 100, 4096, 128, torch.bfloat16),  # one short workgroup
        (29, 28672, 4096, 128, torch.bfloat16),  # past 16384 outputs: more workgroups than CUs
        (4, 20000, 1024, 128, torch.bfloat16),  # 64-row workgroups would leave a last round 22% full:
        (16, 20000, 1024, 128, torch.float16),  # whole rounds instead, 500 workgroups of 40 rows
        (9, 28672, 1024, 128, torch.bfloat16),  # last round 75% full: 448 workgroups of 64 rows
    ],
)
def test_few_token_gemv_multiplies_the_dequantized_weight(rows: int, out: int, width: int, group: int, dtype: torch.dtype) -> None:
    """2..32 rows through the one-workgroup-per-CU GEMV (x row m in MFMA A row m;
    past 16 rows two A blocks per weight tile), against the f64 product and
    against the skinny kernel on the same inputs."""
    packed, scale, zero = _layer(out, width, group, seed=out + rows, dtype=dtype)
    x = torch.randn(rows, width, generator=torch.Generator().manual_seed(rows)).to(dtype)
    args = (x.to(DEV), packed.to(DEV), scale.to(DEV), zero.to(DEV))
    y = kernels.int4_linear(*args, kernel="gemv")
    _check_linear(x, packed, scale, zero, y)
    skinny = kernels.int4_linear(*args, kernel="skinny").float()
    assert (y.float() - skinny).abs().max().item() <= 1e-2 * skinny.abs().max().item()
    bias = torch.randn(out, generator=torch.Generator().manual_seed(3)).to(dtype).to(DEV)
    assert torch.equal(kernels.int4_linear(*args, bias, kernel="gemv"), y + bias)


# ------------------------------------------------------------ full BASELINE sizes


def _baseline_layer(n: int, k: int, seed: int = 0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    w = torch.randn(n, k, generator=g, device=DEV) * 0.02
    packed, scale, zero = kernels.quantize_int4(w, 128)
    return packed, scale.to(torch.bfloat16), zero


@pytest.mark.parametrize(("rows", "k", "n"), [(1, 4096, 14336), (4, 4096, 14336), (16, 4096, 14336), (32, 4096, 14336), (2048, 4096, 4096), (2048, 14336, 4096)])
def test_baseline_sizes_agree_with_dequantize_then_gemm(rows: int, k: int, n: int) -> None:
    """At the BASELINE shapes: the fused kernel equals hipBLASLt over the HIP
    dequantized weight (the reference's own prefill strategy) within bf16 rounding,
    and is linear in x (y(x1 + x2) = y(x1) + y(x2) within rounding)."""
    packed, scale, zero = _baseline_layer(n, k)
    g = torch.Generator(device=DEV).manual_seed(1)
    x = torch.randn(rows, k, generator=g, device=DEV).to(torch.bfloat16)
    y = kernels.int4_linear(x, packed, scale, zero)
    w = kernels.int4_weight(packed, scale, zero)
    ref = (x.float() @ w.float().T)
    err = (y.float() - ref).abs().max().item()
    top = ref.abs().max().item()
    print(f"rows {rows} k {k} n {n}: max abs err {err:.3e}, rel {err / top:.3e}")
    assert err <= 1e-2 * top
    x2 = torch.randn(rows, k, generator=g, device=DEV).to(torch.bfloat16)
    lhs = kernels.int4_linear((x.float() + x2.float()).to(torch.bfloat16), packed, scale, zero).float()
    rhs = y.float() + kernels.int4_linear(x2, packed, scale, zero).float()
    assert (lhs - rhs).abs().max().item() <= 2e-2 * top
