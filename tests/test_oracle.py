"""Pins of the CPU oracle (`oracle/`) against facts fixed independently of its
own formulas: PyTorch's bf16 / float8_e4m3fn conversions, the reference's
closed-form layouts and known answers, its tests' invariants
(`python/linnet/tests/test_quant_groups.py`, `test_quant_8bit.py`,
`test_quant_fp8.py`, `torch/test_quant.py`, `test_resources.py`), and brute force
on tiny inputs. Each test names the mistake it would catch."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import linear, quant
from tests.formats import calibrated_layer, pack_gptq


# ------------------------------------------------------------------ bf16 / fp8


def test_bf16_rounding_matches_torch() -> None:
    """to_bf16_bits is RNE (a truncation or round-half-up would fail the ties)."""
    rng = np.random.default_rng(0)
    values = (rng.standard_normal(20000) * 10.0 ** rng.integers(-30, 30, 20000)).astype(np.float32)
    bits = values.view(np.uint32)
    ties = ((bits & np.uint32(0xFFFF0000)) | np.uint32(0x8000)).view(np.float32)  # exact ties
    for v in (values, ties.astype(np.float32), np.array([0.0, -0.0, 1.0, -3.5, 65504.0], np.float32)):
        want = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        np.testing.assert_array_equal(quant.to_bf16_bits(v), want)
        np.testing.assert_array_equal(quant.from_bf16_bits(want), torch.from_numpy(v).to(torch.bfloat16).float().numpy())


def test_fp8_decode_matches_torch() -> None:
    """Every non-NaN E4M3 byte decodes as torch's float8_e4m3fn
    (`tests/test_quant_fp8.py:46-53`); the NaN bytes read as +-480 in the body."""
    table = np.arange(256, dtype=np.uint8)
    valid = (table & 0x7F) != 0x7F
    want = torch.from_numpy(table).view(torch.float8_e4m3fn).float().numpy()
    got = quant.decode_fp8(table)
    np.testing.assert_array_equal(got[valid], want[valid])
    assert got[0x7F] == 480.0 and got[0xFF] == -480.0
    assert got[0x08] == 2.0**-6 and got[0x01] == 2.0**-9 and got[0x7E] == 448.0


def test_fp8_encode_matches_torch() -> None:
    """encode_fp8 rounds to nearest even with subnormals, as torch's cast does:
    every representable value, every midpoint (tie) and random values in range."""
    table = np.arange(256, dtype=np.uint8)
    valid = (table & 0x7F) != 0x7F
    exact = quant.decode_fp8(table[valid])
    positive = np.unique(np.abs(exact))
    mids = ((positive[:-1].astype(np.float64) + positive[1:]) / 2).astype(np.float32)
    rng = np.random.default_rng(1)
    rand = (rng.standard_normal(50000) * 10.0 ** rng.uniform(-3, 2.5, 50000)).astype(np.float32)
    values = np.concatenate([exact, mids, -mids, rand, np.float32([0.0, -0.0, 1e-30, -1e-30])])
    values = np.clip(values, -448, 448).astype(np.float32)
    want = torch.from_numpy(values).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(quant.encode_fp8(values), want)


# ---------------------------------------------------------------- 4-bit layout


def test_pack_layout_closed_form() -> None:
    """Element 2k sits in the low nibble (`spec/03-types.md:39`,
    `torch/test_quant.py:48-59`); a swapped order fails."""
    codes = np.arange(16, dtype=np.uint8)[None, :]
    packed = quant.pack_int4_groups(codes, 16)
    assert packed.shape == (1, 1, 8)
    np.testing.assert_array_equal(packed.reshape(-1), np.array([0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE], np.uint8))
    np.testing.assert_array_equal(quant.unpack_int4_codes(packed).reshape(1, 16), codes)
    # i4: sign-extended (torch/test_quant.py:48-85's widen check).
    rng = np.random.default_rng(0)
    q4 = rng.integers(-8, 8, size=(6, 16)).astype(np.int8)
    low = q4[:, 0::2].astype(np.int32) & 15
    high = q4[:, 1::2].astype(np.int32) & 15
    bytes_ = ((high << 4) | low).astype(np.uint8)
    np.testing.assert_array_equal(quant.unpack4(bytes_, "i4"), q4)
    np.testing.assert_array_equal(quant.pack4(q4, "i4"), bytes_)
    np.testing.assert_array_equal(quant.pack4(np.array([2.7, -9.5]), "i4"), np.array([(2 & 15) | ((-9 & 15) << 4)], np.uint8))


def test_int4_rows_closed_form() -> None:
    """`dequantize_int4` on every code -8..7 with exact scales: `q * s` exactly,
    element 2k from the low nibble (a swapped nibble order, a missing sign
    extension or a column-indexed scale fails)."""
    values = np.array([np.arange(-8, 8), np.arange(7, -9, -1)], dtype=np.int8)
    low = values[:, 0::2].astype(np.int32) & 15
    high = values[:, 1::2].astype(np.int32) & 15
    packed = ((high << 4) | low).astype(np.uint8)
    for dtype in ("bf16", "f16", "f32"):
        scale = quant.encode_storage(np.array([[0.5], [-2.0]], np.float32), dtype)
        weight = quant.decode_storage(quant.dequantize_int4_rows(packed, scale, dtype), dtype)
        np.testing.assert_array_equal(weight, values.astype(np.float32) * np.array([[0.5], [-2.0]], np.float32))


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_int4_rows_match_torch(dtype: str) -> None:
    """Random [Out, In] i4 layers (Out != In, so a transposed scale fails): the
    oracle equals torch's `(q.float() * s.float()).to(T)` on int8 values drawn
    apart from the packing (`tests/torch/test_quant.py:68-95`'s construction)."""
    rng = np.random.default_rng(5)
    q4 = rng.integers(-8, 8, size=(12, 40)).astype(np.int8)
    low = q4[:, 0::2].astype(np.int32) & 15
    high = q4[:, 1::2].astype(np.int32) & 15
    packed = ((high << 4) | low).astype(np.uint8)
    torch_dtype = torch.bfloat16 if dtype == "bf16" else torch.float16
    scale = torch.tensor(rng.uniform(-0.3, 0.3, size=(12, 1)).astype(np.float32)).to(torch_dtype)
    expected = (torch.tensor(q4).float() * scale.float()).to(torch_dtype)
    raw = scale.view(torch.int16).numpy().view(np.uint16) if dtype == "bf16" else scale.numpy()
    got = quant.dequantize_int4_rows(packed, raw, dtype)
    want = expected.view(torch.int16).numpy().view(np.uint16) if dtype == "bf16" else expected.numpy()
    np.testing.assert_array_equal(got, want)


def test_int4_storage_bytes() -> None:
    """Int4GroupLinear<256, 64, 128, bf16> holds 64*2*64 + 64*2*2 + 64*2 bytes
    (`tests/test_resources.py:184-202`)."""
    w = np.random.default_rng(0).standard_normal((64, 256)).astype(np.float32)
    packed, scale, zero = quant.quantize_int4_groups(w, 128)
    total = packed.nbytes + quant.encode_storage(scale, "bf16").nbytes + zero.nbytes
    assert total == 64 * 2 * 64 + 64 * 2 * 2 + 64 * 2


# ------------------------------------------------------------------ int4 codes


def test_int4_rounding_within_half_a_step() -> None:
    """`tests/test_quant_groups.py:48-56`: |dequant - w| <= step / 2."""
    rng = np.random.default_rng(0)
    weight = rng.standard_normal((64, 256)).astype(np.float32)
    packed, scale, zero = quant.quantize_int4_groups(weight, 128)
    assert packed.shape == (64, 2, 64) and packed.dtype == np.uint8
    assert scale.shape == zero.shape == (64, 2) and scale.dtype == np.float32
    error = np.abs(quant.dequantize_int4_groups(packed, scale, zero) - weight)
    assert np.all(error <= np.repeat(scale, 128, axis=1) / 2 + 1e-6)
    assert zero.max() <= 15


def test_int4_known_answers() -> None:
    """Ramps and constants with exact answers: a step of (max-min)/16, a zero of
    the wrong sign, or floor instead of rint fails."""
    ramp = (np.arange(16, dtype=np.float32) * 0.25)[None, :]
    packed, scale, zero = quant.quantize_int4_groups(ramp, 16)
    assert scale[0, 0] == np.float32(0.25) and zero[0, 0] == 0
    np.testing.assert_array_equal(quant.unpack_int4_codes(packed).reshape(-1), np.arange(16))
    shifted = ((np.arange(16, dtype=np.float32) - 5) * 0.5)[None, :]
    packed, scale, zero = quant.quantize_int4_groups(shifted, 16)
    assert scale[0, 0] == np.float32(0.5) and zero[0, 0] == 5
    np.testing.assert_array_equal(quant.unpack_int4_codes(packed).reshape(-1), np.arange(16))
    const = np.full((2, 16), [[0.3], [-2.2]], dtype=np.float32)
    packed, scale, zero = quant.quantize_int4_groups(const, 16)
    np.testing.assert_array_equal(scale, np.ones((2, 1), np.float32))
    np.testing.assert_array_equal(zero.reshape(-1), [0, 2])
    np.testing.assert_array_equal(quant.unpack_int4_codes(packed).reshape(2, 16), np.zeros((2, 16)))
    # Half-way codes round to even: w/scale + zero = 0.5 -> 0, 2.5 -> 2.
    halves = np.array([[0.0, 0.5, 2.5, 15.0] * 4], dtype=np.float32)
    packed, scale, zero = quant.quantize_int4_groups(halves, 16)
    assert scale[0, 0] == 1.0 and zero[0, 0] == 0
    np.testing.assert_array_equal(quant.unpack_int4_codes(packed).reshape(-1)[:4], [0, 0, 2, 15])


def test_int4_codes_are_the_nearest_levels() -> None:
    """Brute force on tiny groups: each code is the level (c - z) * s nearest w
    among all 16 (off-by-one zero points or truncation fail)."""
    rng = np.random.default_rng(5)
    weight = (rng.standard_normal((8, 32)) * 0.02).astype(np.float32)
    packed, scale, zero = quant.quantize_int4_groups(weight, 16)
    codes = quant.unpack_int4_codes(packed).reshape(8, 32)
    for o in range(8):
        for i in range(32):
            g = i // 16
            levels = (np.arange(16) - float(zero[o, g])) * float(scale[o, g])
            assert codes[o, i] == int(np.argmin(np.abs(levels - float(weight[o, i]))))


def test_dequantized_weight_matches_torch_bf16_arithmetic() -> None:
    """The reference's own bit-exact check (`tests/test_quant_groups.py:151-162`):
    `(q.to(bf16) - z.to(bf16)) * s` in torch equals the oracle's dequantized bits."""
    rng = np.random.default_rng(2)
    out, groups, group = 72, 4, 128
    packed = rng.integers(0, 256, (out, groups, group // 2), dtype=np.uint8)
    scale = (rng.random((out, groups)) * 0.02 + 0.001).astype(np.float32)
    scale_bits = quant.to_bf16_bits(scale)
    zero = rng.integers(0, 16, (out, groups), dtype=np.uint8)
    got = quant.dequantize_int4_weight(packed, scale_bits, zero, "bf16")
    p = torch.from_numpy(packed)
    levels = torch.stack([p & 15, p >> 4], dim=-1).reshape(out, groups, group)
    s = torch.from_numpy(scale_bits.view(np.int16)).view(torch.bfloat16)
    z = torch.from_numpy(zero)
    want = ((levels.to(torch.bfloat16) - z.to(torch.bfloat16)[..., None]) * s[..., None]).reshape(out, -1)
    np.testing.assert_array_equal(got, want.view(torch.int16).numpy().view(np.uint16))
    # f16 and f32 storage follow the same one-rounding rule.
    for dtype, tdtype in (("f16", torch.float16), ("f32", torch.float32)):
        raw = quant.encode_storage(scale, dtype)
        st = torch.from_numpy(np.asarray(raw))
        want = ((levels.to(tdtype) - z.to(tdtype)[..., None]) * st[..., None]).reshape(out, -1).numpy()
        np.testing.assert_array_equal(quant.dequantize_int4_weight(packed, raw, zero, dtype), want)


# ------------------------------------------------------------------ int8 codes


def test_int8_rounding_within_half_a_step() -> None:
    """`tests/test_quant_8bit.py:235-242`; the scale is a bf16 value."""
    weight = np.random.default_rng(0).standard_normal((256, 512)).astype(np.float32)
    q, scale = quant.quantize_int8_groups(weight, 128, "bf16")
    assert q.dtype == np.int8 and q.shape == (256, 512) and scale.shape == (256, 4)
    error = np.abs(quant.dequantize_int8_groups(q, scale) - weight)
    assert np.all(error <= np.repeat(scale, 128, axis=1) / 2 + 1e-6)
    np.testing.assert_array_equal(quant.round_to_storage(scale, "bf16"), scale)
    assert np.abs(q).max() <= 127


def test_int8_known_answers() -> None:
    """max|w| = 127 gives scale 1 and q = round-half-even(w); a zero group gives
    scale 1 (`quant.py:116`); rounding the scale after the codes fails the bf16 case."""
    w = np.array([[127.0, -3.5, 2.5, 0.4, -127.0, 1.5, 0.0, 100.2]], dtype=np.float32)
    q, scale = quant.quantize_int8_groups(w, 8, "f32")
    assert scale[0, 0] == 1.0
    np.testing.assert_array_equal(q[0], [127, -4, 2, 0, -127, 2, 0, 100])
    q, scale = quant.quantize_int8_groups(np.zeros((1, 8), np.float32), 8, "bf16")
    assert scale[0, 0] == 1.0 and not q.any()
    # 1.0 / 127 is not a bf16 value: the codes are computed against its rounding.
    w = np.full((1, 4), [1.0, 0.5, 0.25, -1.0], dtype=np.float32)
    q, scale = quant.quantize_int8_groups(w, 4, "bf16")
    s = np.float32(torch.tensor(1.0 / 127).to(torch.bfloat16).item())
    assert scale[0, 0] == s
    np.testing.assert_array_equal(q[0], np.clip(np.round(w[0] / s), -127, 127))


# --------------------------------------------------------- activation rounding


def test_rows8_fp8_matches_torch_cast() -> None:
    """FP8 rows: the per-row scale max|x|/448 and torch's float8_e4m3fn cast of
    x / scale (a scale over 127, or a missing clamp, fails)."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal((9, 300)).astype(np.float32)
    x[2] *= 50
    x[4] = 0.0
    x = quant.from_bf16_bits(quant.to_bf16_bits(x)).reshape(x.shape)
    q, scale = quant.rows8(x, True)
    t = torch.from_numpy(x)
    s = torch.clamp(t.abs().amax(dim=1, keepdim=True), min=1e-12) / 448.0
    np.testing.assert_array_equal(scale, s.numpy())
    want = (t / s).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(q, want)


def test_rows8_int8_rounds_half_away_in_f32() -> None:
    """int8 rows: half away from zero, the +-0.5 added in f32 as the reference's
    kernel does (`torch/kernels.py:690-691`): 2.5 -> 3, -2.5 -> -3, and the f32
    edge 0.49999997 + 0.5 = 1.0 -> 1."""
    x = np.array([[127.0, 2.5, -2.5, 0.49999997, -0.5, 1.4999999, 126.5, -126.49]], dtype=np.float32)
    q, scale = quant.rows8(x, False)
    assert scale[0, 0] == 1.0
    np.testing.assert_array_equal(q[0], [127, 3, -3, 1, -1, 1, 127, -126])
    # Away from the f32 edge it is exact round-half-away (brute force).
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((4, 64)) * 30).astype(np.float32)
    q, scale = quant.rows8(x, False)
    v = x.astype(np.float64) / scale.astype(np.float64)
    exact = np.sign(v) * np.floor(np.abs(v) + 0.5)
    np.testing.assert_array_equal(q.astype(np.float64), np.clip(exact, -127, 127))


# -------------------------------------------------------------- CPU linear paths


def test_cpu_int4_paths_agree_with_fp64() -> None:
    """The interpreter path and the generated CPU path give the same bf16 output,
    within bf16 rounding of the f64 product with the dequantized weight."""
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((64, 256)) * 0.02).astype(np.float32)
    packed, scale, zero = quant.quantize_int4_groups(w, 128)
    scale_bits = quant.to_bf16_bits(scale)
    p = torch.from_numpy(packed)
    s = torch.from_numpy(scale_bits.view(np.int16)).view(torch.bfloat16)
    z = torch.from_numpy(zero)
    x = torch.randn(3, 256, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)
    interp = linear.int4_groups_linear_interpreter(x, p, s, z, None)
    gen = linear.int4_linear_generated_cpu(x, linear.int4_prepare_cpu(p, s, z), None)
    torch.testing.assert_close(interp, gen, rtol=0, atol=0)
    ref = linear.int4_reference_f64(x.float().numpy(), packed, quant.from_bf16_bits(scale_bits), zero)
    assert np.abs(interp.float().numpy() - ref).max() <= 1e-2 * np.abs(ref).max()


def test_cpu_8bit_paths_agree_with_fp64() -> None:
    rng = np.random.default_rng(1)
    w = rng.standard_normal((32, 256)).astype(np.float32)
    q, scale = quant.quantize_int8_groups(w, 256, "f32")
    x = torch.randn(2, 256, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    got = linear.int8_linear_cpu(x, torch.from_numpy(q), torch.from_numpy(scale.reshape(-1)), None)
    ref = linear.product_f64(x.float().numpy(), quant.dequantize_int8_groups(q, scale))
    assert np.abs(got.float().numpy() - ref).max() <= 1e-2 * np.abs(ref).max()
    full = torch.from_numpy(w)
    fs = full.abs().amax(dim=1, keepdim=True) / 448.0
    w8 = (full / fs).to(torch.float8_e4m3fn)
    got = linear.fp8_linear_cpu(x, w8, fs, None)
    ref = linear.product_f64(x.float().numpy(), (w8.float() * fs).numpy())
    assert np.abs(got.float().numpy() - ref).max() <= 1e-2 * np.abs(ref).max()


def _decoded_by_loop(q: np.ndarray, scale: np.ndarray, group: int) -> np.ndarray:
    """Brute force over (output, input): `bf16(f32(q[o, i]) * f32(s[o, i // group]))`,
    the weight `Int8GroupLinear` decodes (`stdlib/quant.linnet:60-72`), element by
    element, no reshape."""
    out_features, in_features = q.shape
    w = np.zeros((out_features, in_features), np.float32)
    for o in range(out_features):
        for i in range(in_features):
            w[o, i] = np.float32(q[o, i]) * np.float32(scale[o, i // group])
    return quant.from_bf16_bits(quant.to_bf16_bits(w))


def test_int8_group_cpu_path_against_a_loop() -> None:
    """`quantized.int8_group_linear`'s CPU branch on a layer with Out != In and 3
    groups, each scale a different power of two: rows of the identity read the
    decoded weight back exactly (one nonzero product per output), so a scale
    taken along the wrong axis, a transposed weight or a group index off by one
    changes the bits; a random x then matches the f64 loop sum to bf16's
    rounding, and the bias is added after the product."""
    rng = np.random.default_rng(11)
    out_features, in_features, group = 5, 96, 32
    q = rng.integers(-127, 128, size=(out_features, in_features)).astype(np.int8)
    scale = np.exp2(rng.integers(-6, 3, size=(out_features, in_features // group))).astype(np.float32)
    assert len(np.unique(scale)) > 3
    qt, st = torch.from_numpy(q), torch.from_numpy(scale)
    eye = torch.eye(in_features, dtype=torch.bfloat16)
    got = linear.int8_group_linear_cpu(eye, qt, st, None).float().numpy()
    np.testing.assert_array_equal(got, _decoded_by_loop(q, scale, group).T)

    x = rng.standard_normal((3, in_features)).astype(np.float32)
    xb = torch.from_numpy(x).to(torch.bfloat16)
    bias = torch.from_numpy(rng.standard_normal(out_features).astype(np.float32) * 50).to(torch.bfloat16)
    got = linear.int8_group_linear_cpu(xb, qt, st, bias).float().numpy()
    xs = xb.float().numpy().astype(np.float64)
    want = np.zeros((3, out_features))
    for r in range(3):
        for o in range(out_features):
            want[r, o] = sum(xs[r, i] * float(q[o, i]) * float(scale[o, i // group]) for i in range(in_features))
    want += bias.float().numpy()
    assert np.abs(got - want).max() <= 1e-2 * np.abs(want).max()


def test_int8_cpu_path_against_a_loop_with_bias() -> None:
    """`quantized.int8_linear`'s CPU branch, one scale a row: the identity reads back
    `bf16(q * s[o])` bit for bit (a scale per input instead of per output fails),
    and with a bias of the product's size the output is the loop sum plus the bias
    (a dropped or doubled bias fails)."""
    rng = np.random.default_rng(12)
    out_features, in_features = 6, 64
    q = rng.integers(-127, 128, size=(out_features, in_features)).astype(np.int8)
    scale = np.exp2(rng.integers(-7, 0, size=out_features)).astype(np.float32)
    qt, st = torch.from_numpy(q), torch.from_numpy(scale)
    eye = torch.eye(in_features, dtype=torch.bfloat16)
    got = linear.int8_linear_cpu(eye, qt, st, None).float().numpy()
    np.testing.assert_array_equal(got, _decoded_by_loop(q, scale[:, None], in_features).T)

    x = rng.standard_normal((2, in_features)).astype(np.float32)
    xb = torch.from_numpy(x).to(torch.bfloat16)
    plain = linear.int8_linear_cpu(xb, qt, st, None).float().numpy()
    bias = torch.from_numpy(np.abs(plain).max() * rng.standard_normal(out_features).astype(np.float32)).to(torch.bfloat16)
    got = linear.int8_linear_cpu(xb, qt, st, bias).float().numpy()
    xs = xb.float().numpy().astype(np.float64)
    want = np.array([[sum(xs[r, i] * float(q[o, i]) * float(scale[o]) for i in range(in_features))
                      for o in range(out_features)] for r in range(2)]) + bias.float().numpy()
    assert np.abs(got - want).max() <= 1e-2 * np.abs(want).max()
    # 3-d input: the leading axes are kept.
    got3 = linear.int8_linear_cpu(xb.reshape(2, 1, in_features), qt, st, bias)
    assert got3.shape == (2, 1, out_features)
    np.testing.assert_array_equal(got3.reshape(2, out_features).float().numpy(), got)


def test_fp8_block_cpu_path_against_a_loop() -> None:
    """`quantized.fp8_block_linear`'s CPU branch with 4 x 4 blocks on a 8 x 12
    weight (2 x 3 blocks, each scale a different power of two): the identity
    reads back `bf16(decode(w[o, i]) * s[o / 4, i / 4])` bit for bit (a block
    index on the wrong axis or a transposed scale fails), and a random x with a
    bias matches the f64 loop sum within bf16's rounding."""
    rng = np.random.default_rng(13)
    out_features, in_features, block = 8, 12, 4
    codes = rng.integers(0, 256, size=(out_features, in_features)).astype(np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x38  # no NaN bytes (1.0 instead)
    scale = np.exp2(rng.permutation(np.arange(-3, 3))).astype(np.float32).reshape(2, 3)
    wt = torch.from_numpy(codes).view(torch.float8_e4m3fn)
    st = torch.from_numpy(scale)
    values = quant.decode_fp8(codes)
    loop = np.zeros((out_features, in_features), np.float32)
    for o in range(out_features):
        for i in range(in_features):
            loop[o, i] = np.float32(values[o, i]) * scale[o // block, i // block]
    loop = quant.from_bf16_bits(quant.to_bf16_bits(loop))
    eye = torch.eye(in_features, dtype=torch.bfloat16)
    got = linear.fp8_block_linear_cpu(eye, wt, st, None).float().numpy()
    np.testing.assert_array_equal(got, loop.T)

    xb = torch.from_numpy(rng.standard_normal((3, in_features)).astype(np.float32)).to(torch.bfloat16)
    bias = torch.from_numpy(rng.standard_normal(out_features).astype(np.float32) * 100).to(torch.bfloat16)
    got = linear.fp8_block_linear_cpu(xb, wt, st, bias).float().numpy()
    xs = xb.float().numpy().astype(np.float64)
    want = np.array([[sum(xs[r, i] * float(values[o, i]) * float(scale[o // block, i // block])
                          for i in range(in_features)) for o in range(out_features)] for r in range(3)])
    want += bias.float().numpy()
    assert np.abs(got - want).max() <= 1e-2 * np.abs(want).max()


@pytest.mark.parametrize("fp8", [True, False])
def test_rows8_product_reference(fp8: bool) -> None:
    """The 8-bit product reference equals the dequantized operands' product."""
    rng = np.random.default_rng(6)
    x = rng.standard_normal((3, 128)).astype(np.float32)
    q, xs = quant.rows8(x, fp8)
    wq = (quant.encode_fp8(np.clip(rng.standard_normal((5, 128)) * 50, -448, 448).astype(np.float32)) if fp8
          else rng.integers(-127, 128, (5, 128)).astype(np.int8))
    ws = rng.random(5).astype(np.float32)
    got = linear.rows8_product_f64(q, xs, wq, ws, fp8)
    deq_x = (quant.decode_fp8(q) if fp8 else q.astype(np.float32)) * xs
    deq_w = (quant.decode_fp8(wq) if fp8 else wq.astype(np.float32)) * ws[:, None]
    np.testing.assert_allclose(got, deq_x.astype(np.float64) @ deq_w.astype(np.float64).T, rtol=1e-6)


# ------------------------------------------------------- GPTQ / AWQ repack

CALIBRATED = [("gptq", False), ("gptq", True), ("awq", False)]


@pytest.mark.parametrize(("method", "act_order"), CALIBRATED)
def test_repack_inverts_the_format_packers(method: str, act_order: bool) -> None:
    """Catches a wrong nibble order, a missed AWQ column reversal, zero points
    taken along the wrong axis or without GPTQ's offset: the result's input i
    holds the checkpoint's input order[i] (order the identity unless in
    activation order), its zero points are the checkpoint's transposed."""
    layer = calibrated_layer(method, act_order)
    packed, zero, order = quant.repack_int4(layer["qweight"], layer["qzeros"], method, layer["group"],
                                            1 if method == "gptq" else 0,
                                            layer["g_idx"] if method == "gptq" else None)
    assert (order is not None) == act_order
    source = order if order is not None else np.arange(layer["q"].shape[0])
    codes = quant.unpack_int4_codes(packed).reshape(packed.shape[0], -1)
    assert np.array_equal(codes, layer["q"][source].T)
    assert np.array_equal(zero, layer["zero"].T)
    if act_order:
        assert sorted(order.tolist()) == list(range(len(order)))
        assert np.array_equal(layer["g_idx"][order], np.arange(len(order)) // layer["group"])


@pytest.mark.parametrize(("method", "act_order"), CALIBRATED)
def test_repack_computes_the_format_formula(method: str, act_order: bool) -> None:
    """The repacked layer, its inputs gathered by `order` (`take_inputs`,
    `stdlib/quant.linnet:143-149`), computes `x @ W` for the format's own
    `W[i, o] = (q[i, o] - zero[g(i), o]) * scale[g(i), o]`
    (`test_quant_groups.py:228-273`)."""
    layer = calibrated_layer(method, act_order, seed=4)
    packed, zero, order = quant.repack_int4(layer["qweight"], layer["qzeros"], method, layer["group"],
                                            1 if method == "gptq" else 0,
                                            layer["g_idx"] if method == "gptq" else None)
    w = quant.dequantize_int4_groups(packed, np.ascontiguousarray(layer["scale"].T).astype(np.float32), zero)
    x = np.random.default_rng(5).standard_normal((3, layer["q"].shape[0]))
    taken = x[:, order] if order is not None else x
    np.testing.assert_allclose(taken @ w.T.astype(np.float64), x @ layer["weight"].astype(np.float64),
                               rtol=1e-5, atol=1e-5)


def test_gptq_second_format_has_no_zero_offset() -> None:
    """GPTQ's v2 checkpoints store zero points as they are (`quant.py:297-298`)."""
    rng = np.random.default_rng(8)
    q = rng.integers(0, 16, (64, 16))
    zero = rng.integers(0, 16, (1, 16))
    qweight, qzeros = pack_gptq(q, zero, offset=0)
    _, got, _ = quant.repack_int4(qweight, qzeros, "gptq", 64, 0, None)
    assert np.array_equal(got, zero.T)


# ------------------------------------------------- FP8 groups / block product


def test_fp8_groups_is_rows8_per_group() -> None:
    """Catches a scale taken over the row instead of the group, groups laid out
    wrongly, or padded rows that are not zero codes with scale 1."""
    rng = np.random.default_rng(13)
    x = (rng.standard_normal((3, 384)) * np.array([1.0, 100.0, 1e-3])[:, None]).astype(np.float32)
    x[1, 128:256] = 0.0  # an all-zero group: scale 1e-12 / 448, codes 0
    q, s = quant.fp8_groups(x, 128, 5)
    assert q.shape == (5, 384) and s.shape == (5, 3)
    for r in range(3):
        for g in range(3):
            cq, cs = quant.rows8(x[r:r + 1, 128 * g:128 * (g + 1)], True)
            assert np.array_equal(q[r, 128 * g:128 * (g + 1)], cq[0]) and s[r, g] == cs[0, 0]
    assert not q[3:].any() and np.all(s[3:] == 1.0)
    assert s[1, 1] == np.float32(1e-12) / np.float32(448.0)


def test_block_product_reference_against_a_loop() -> None:
    """The block product against a brute-force loop over blocks (catches a
    weight scale indexed by the wrong block axis or an x scale per row instead of
    per block)."""
    rng = np.random.default_rng(14)
    x = rng.standard_normal((2, 256)).astype(np.float32)
    q, xs = quant.fp8_groups(x, 128, 2)
    wq = quant.encode_fp8(np.clip(rng.standard_normal((256, 256)) * 30, -448, 448).astype(np.float32))
    ws = rng.random((2, 2)).astype(np.float32) + 0.5
    got = linear.block_product_f64(q, xs, wq, ws)
    dq, dw = quant.decode_fp8(q).astype(np.float64), quant.decode_fp8(wq).astype(np.float64)
    want = np.zeros((2, 256))
    for m in range(2):
        for n in range(256):
            for b in range(2):
                k = slice(128 * b, 128 * (b + 1))
                want[m, n] += (dq[m, k] @ dw[n, k]) * xs[m, b] * ws[n // 128, b]
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12 * np.abs(want).max())


# ---------------------------------------------------------------------- MXFP4


def test_mxfp4_decoding_from_the_format_definition() -> None:
    """E2M1: sign bit 3, exponent bits 1-2 (bias 1), mantissa bit 0, exponent 0
    subnormal (value = mantissa / 2); E8M0: 2^(s - 127). Catches a swapped nibble
    order, a wrong table entry or an off-by-one scale bias."""
    def e2m1(code: int) -> float:
        sign = -1.0 if code & 8 else 1.0
        exponent, mantissa = (code >> 1) & 3, code & 1
        value = mantissa * 0.5 if exponent == 0 else 2.0 ** (exponent - 1) * (1 + mantissa / 2)
        return sign * value

    assert [float(v) for v in quant.FP4_VALUES] == [e2m1(c) for c in range(16)]
    block = np.arange(16, dtype=np.uint8) | (np.arange(16, dtype=np.uint8)[::-1] << 4)  # byte j: low j, high 15-j
    got = quant.dequantize_mxfp4(block.reshape(1, 16), np.array([130], np.uint8))
    want = np.array([[e2m1(j) * 8, e2m1(15 - j) * 8] for j in range(16)], np.float32).reshape(32)
    assert np.array_equal(got, want)
    assert quant.dequantize_mxfp4(np.full((1, 16), 0x22, np.uint8), np.array([0], np.uint8))[0] == np.float32(2.0**-127)


def test_mxfp4_product_reference_against_a_loop() -> None:
    rng = np.random.default_rng(15)
    blocks = rng.integers(0, 256, (3, 4, 2, 16)).astype(np.uint8)
    scales = rng.integers(120, 134, (3, 4, 2)).astype(np.uint8)
    x = rng.standard_normal((2, 2, 64))
    experts = np.array([[2, 0], [1, 2]])
    got = linear.mxfp4_experts_f64(x, blocks, scales, experts)
    w = quant.dequantize_mxfp4(blocks, scales)
    for r in range(2):
        for k in range(2):
            for o in range(4):
                assert np.isclose(got[r, k, o], sum(x[r, k, i] * float(w[experts[r, k], o, i]) for i in range(64)),
                                  rtol=1e-12, atol=1e-12)


# ------------------------------------------------------------------------ NF4


def test_nf4_table_is_qloras_normal_quantiles() -> None:
    """QLoRA's NF4 (Dettmers et al. 2023, bitsandbytes' `create_normal_map` with
    offset 0.9677083): 8 positive quantiles of N(0, 1) at float32 linspace(offset,
    0.5, 9)[:-1], 7 negative ones at linspace(offset, 0.5, 8)[:-1], and 0, sorted
    and divided by the largest. Catches a mistyped or reordered entry."""
    from scipy.stats import norm

    offset = 0.9677083
    positive = norm.ppf(torch.linspace(offset, 0.5, 9)[:-1].numpy())
    negative = -norm.ppf(torch.linspace(offset, 0.5, 8)[:-1].numpy())
    values = np.sort(np.concatenate([positive, [0.0], negative]))
    values = values / values.max()
    np.testing.assert_array_equal(values.astype(np.float32), quant.NF4_VALUES)


def test_nf4_weight_from_the_layout_definition() -> None:
    """Byte j of a row holds inputs 2j (low nibble) and 2j + 1 (high); absmax
    [o, b] scales inputs b*block .. b*block + block - 1 of row o. Every element
    gets its own code and power-of-two scale, so a swapped nibble order, a block
    index along the wrong axis or a transposed scale fails."""
    out_features, in_features, block = 3, 16, 4
    codes = np.array([[(5 * o + 3 * i) % 16 for i in range(in_features)] for o in range(out_features)], np.uint8)
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
    absmax = np.array([[2.0 ** (4 * o + b - 3) for b in range(in_features // block)] for o in range(out_features)],
                      np.float32)
    got = quant.nf4_weight(packed, absmax, block)
    for o in range(out_features):
        for i in range(in_features):
            assert got[o, i] == np.float32(float(quant.NF4_VALUES[(5 * o + 3 * i) % 16]) * 2.0 ** (4 * o + i // block - 3))
    rng = np.random.default_rng(21)
    packed = rng.integers(0, 256, (5, 32)).astype(np.uint8)
    absmax = rng.uniform(0.01, 3.0, (5, 2)).astype(np.float32)
    weight = quant.nf4_weight(packed, absmax, 32)
    for dtype, torch_dtype in (("bf16", torch.bfloat16), ("f16", torch.float16)):
        want = torch.from_numpy(weight).to(torch_dtype).float().numpy()
        np.testing.assert_array_equal(quant.decode_storage(quant.dequantize_nf4(packed, absmax, 32, dtype), dtype), want)


def test_bnb_nf4_layer() -> None:
    """bitsandbytes packs the first code of a pair in the high nibble (the
    reference's test writes `codes[1::2] | codes[0::2] << 4`); double quantization
    decodes `nested_map[code] * nested_absmax[i // nested_block] + offset`. With
    exact binary values the decoded scales are known sums; a missed swap, a wrong
    nested index or a dropped offset fails."""
    rng = np.random.default_rng(3)
    out_features, in_features, block, nested_block = 4, 64, 16, 5
    codes = rng.integers(0, 16, out_features * in_features).astype(np.uint8)
    packed = (codes[1::2] | (codes[0::2] << 4)).astype(np.uint8)
    plain = rng.uniform(0.1, 2.0, out_features * in_features // block).astype(np.float32)
    got_codes, got_scale = quant.bnb_nf4_layer(packed, plain, out_features, in_features, block)
    unpacked = np.stack([got_codes & 15, got_codes >> 4], axis=-1).reshape(-1)
    np.testing.assert_array_equal(unpacked, codes)
    np.testing.assert_array_equal(got_scale.reshape(-1), plain)
    blocks = out_features * in_features // block
    scale_codes = rng.integers(0, 256, blocks).astype(np.uint8)
    nested_map = (np.arange(256, dtype=np.float32) - 128) / 64
    nested_absmax = np.array([0.5, 2.0, 4.0, 0.25], np.float32)
    _, decoded = quant.bnb_nf4_layer(packed, scale_codes, out_features, in_features, block, nested_absmax,
                                     nested_map, nested_block, 0.75)
    want = [(int(c) - 128) / 64 * float(nested_absmax[i // nested_block]) + 0.75 for i, c in enumerate(scale_codes)]
    np.testing.assert_array_equal(decoded.reshape(-1), np.array(want, np.float32))


def test_nf4_reference_against_a_loop() -> None:
    rng = np.random.default_rng(4)
    packed = rng.integers(0, 256, (3, 16)).astype(np.uint8)
    absmax = rng.uniform(0.5, 1.5, (3, 2)).astype(np.float32)
    x = rng.standard_normal((2, 32))
    bias = rng.standard_normal(3)
    got = linear.nf4_reference_f64(x, packed, absmax, 16, bias)
    for r in range(2):
        for o in range(3):
            want = bias[o]
            for i in range(32):
                code = int(packed[o, i // 2] >> (4 * (i % 2))) & 15
                want += x[r, i] * float(quant.NF4_VALUES[code] * absmax[o, i // 16])  # the weight is f32
            assert np.isclose(got[r, o], want, rtol=1e-12, atol=1e-12)
