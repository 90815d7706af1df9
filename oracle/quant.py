"""numpy restatement of the reference's quantize / pack / dequantize arithmetic.

TEST INFRASTRUCTURE ONLY (see `oracle/__init__.py`): imported by `tests/`,
`__graft_entry__.smoke()` and `bench.py`'s CPU-baseline leg, never by the
product path.

bf16 values are carried as their `uint16` bit patterns (numpy has no bf16).
Every reference citation is relative to the reference checkout's root; the
Python package lives at `python/linnet/src/linnet/`.
"""

from __future__ import annotations

import numpy as np

# ---------------------------------------------------------------- bit formats


def to_bf16_bits(values: np.ndarray) -> np.ndarray:
    """f32 values as bf16 bit patterns, rounded to nearest, ties to even.

    Restates `weights.py:74-79` (`to_bf16_bits`).
    Pin: equals `torch.Tensor.to(torch.bfloat16)` on every finite input
    (tests/test_oracle.py::test_bf16_rounding_matches_torch)."""
    bits = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32)
    rounded = bits + np.uint32(0x7FFF) + ((bits >> np.uint32(16)) & np.uint32(1))
    return (rounded >> np.uint32(16)).astype(np.uint16)


def from_bf16_bits(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns as f32. Restates `weights.py:82-84`. Exact widening."""
    return (np.asarray(bits).view(np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def round_to_storage(values: np.ndarray, dtype: str) -> np.ndarray:
    """f32 values rounded to storage dtype `dtype` ("bf16", "f16", "f32") and
    widened back to f32: `decode_floats(stored, encode_floats(v, stored))` of
    `weights.py:87-105`, as `quantize_int8_groups` applies it (`quant.py:117-118`)."""
    values = np.ascontiguousarray(values, dtype=np.float32)
    if dtype == "bf16":
        return from_bf16_bits(to_bf16_bits(values)).reshape(values.shape)
    if dtype == "f16":
        return values.astype(np.float16).astype(np.float32)
    if dtype == "f32":
        return values.copy()
    raise ValueError(f"scales are stored as bf16, f16, or f32, not {dtype}")


def encode_storage(values: np.ndarray, dtype: str) -> np.ndarray:
    """f32 values as the raw storage array of `dtype`: uint16 bits for bf16,
    float16 for f16, float32 for f32 (`weights.py:98-105`)."""
    values = np.ascontiguousarray(values, dtype=np.float32)
    if dtype == "bf16":
        return to_bf16_bits(values)
    if dtype == "f16":
        return values.astype(np.float16)
    if dtype == "f32":
        return values.copy()
    raise ValueError(f"scales are stored as bf16, f16, or f32, not {dtype}")


def decode_storage(raw: np.ndarray, dtype: str) -> np.ndarray:
    """Inverse of `encode_storage`: the stored values widened to f32."""
    if dtype == "bf16":
        return from_bf16_bits(raw)
    return np.asarray(raw).astype(np.float32)


def decode_fp8(bits: np.ndarray) -> np.ndarray:
    """FP8 E4M3 bytes as f32, by the canonical body of `std.quant::decode_fp8`
    (`stdlib/quant.linnet:227-235`): a normal value is `(8 + m) * 2**(e - 10)`,
    a subnormal one `m * 2**-9`; the NaN bytes 0x7F/0xFF read as +-480.

    Pin: equals `torch.float8_e4m3fn` widening on the 254 non-NaN bytes
    (`tests/test_quant_fp8.py:46-53`, restated in tests/test_oracle.py)."""
    wide = np.asarray(bits, dtype=np.uint8).astype(np.int32)
    exponent = (wide >> 3) & 15
    mantissa = wide & 7
    magnitude = np.where(exponent == 0, mantissa, mantissa + 8)
    power = (np.left_shift(1, np.maximum(exponent, 1) - 1)).astype(np.float32) * np.float32(
        0.001953125
    )
    value = magnitude.astype(np.float32) * power
    return np.where((wide & 128) == 0, value, -value).astype(np.float32)


def encode_fp8(values: np.ndarray) -> np.ndarray:
    """f32 values (already clamped to +-448) as FP8 E4M3 (OCP `e4m3fn`) bytes,
    rounded to nearest, ties to even: the `.to(float8e4nv)` cast of
    `torch/kernels.py:688-689` (Triton) and `torch.Tensor.to(float8_e4m3fn)`.

    Pin: equals torch's own `float8_e4m3fn` cast on every f32 input in range,
    including every tie (tests/test_oracle.py::test_fp8_encode_matches_torch)."""
    x = np.ascontiguousarray(values, dtype=np.float32)
    bits = x.view(np.uint32)
    sign = ((bits >> np.uint32(24)) & np.uint32(0x80)).astype(np.uint8)
    mag = np.abs(x)
    # Normal range (|x| >= 2**-6): round the 23-bit mantissa to 3 bits.
    mbits = mag.view(np.uint32)
    rounded = mbits + np.uint32(0x7FFFF) + ((mbits >> np.uint32(20)) & np.uint32(1))
    exp = (rounded >> np.uint32(23)).astype(np.int64) - 127 + 7
    man = ((rounded >> np.uint32(20)) & np.uint32(7)).astype(np.int64)
    normal = ((exp << 3) | man).astype(np.int64)
    # Subnormal range: multiples of 2**-9, rounded half to even (exact scaling).
    sub = np.rint(mag.astype(np.float64) * 512.0).astype(np.int64)  # 0..8; 8 is 2**-6
    code = np.where(mag >= np.float32(2.0**-6), normal, sub)
    code = np.minimum(code, 0x7E)  # saturate at 448
    return (code.astype(np.uint8) | sign).astype(np.uint8)


# ------------------------------------------------------------- 4-bit packing


def pack_int4_groups(q: np.ndarray, group: int) -> np.ndarray:
    """`[Out, In]` codes in 0..15 as `[Out, In/group, group/2]` bytes, the even
    element in the low nibble. Restates `quant.py:242-248`.

    Pin: closed form of `spec/03-types.md:39` / `torch/test_quant.py:48-59`
    (tests/test_oracle.py::test_pack_layout_closed_form)."""
    out_features, in_features = q.shape
    grouped = q.reshape(out_features, in_features // group, group).astype(np.uint8)
    return (grouped[..., 0::2] | (grouped[..., 1::2] << 4)).astype(np.uint8)


# ------------------------------------------------ GPTQ / AWQ checkpoint words

AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)  # quant.py:222-227: bits 4k hold output AWQ_ORDER[k]


def nibbles(words: np.ndarray, axis: int) -> np.ndarray:
    """The eight 4-bit values of each int32, lowest bits first, laid along `axis`
    (which grows eightfold). Restates `quant.py:230-239` (`_nibbles`).

    Pin: round trip of the GPTQ / AWQ packers the reference's tests write from
    the formats' definitions (`test_quant_groups.py:198-221`;
    tests/test_oracle.py::test_repack_inverts_the_format_packers)."""
    bits = np.asarray(words).astype(np.int64) & 0xFFFFFFFF
    values = (bits[..., None] >> np.arange(0, 32, 4, dtype=np.int64)) & 15
    values = np.moveaxis(values, -1, axis + 1)
    shape = list(np.asarray(words).shape)
    shape[axis] *= 8
    return values.reshape(shape).astype(np.uint8)


def repack_int4(
    qweight: np.ndarray, qzeros: np.ndarray, method: str, group: int, zero_offset: int, g_idx: np.ndarray | None
) -> tuple[np.ndarray, np.ndarray, np.ndarray | None]:
    """A GPTQ or AWQ layer's words as `(packed [Out, In/group, group/2], zero [Out,
    In/group] u8, order [In] int32 or None)`. Restates `import_quantized`'s per-layer
    repack (`quant.py:307-341`): GPTQ codes along the inputs, zero points along the
    outputs plus `zero_offset`, activation order as the stable argsort of `g_idx`;
    AWQ codes and zero points along the outputs, columns reversed through
    `AWQ_ORDER`.

    Pin: as `nibbles` (the format packers' round trip, with and without
    activation order) and the dequantized weight against the formats' own formula
    `W[i, o] = (q[i, o] - zero[g(i), o]) * scale[g(i), o]`
    (tests/test_oracle.py::test_repack_computes_the_format_formula)."""
    order = None
    if method == "gptq":
        q = nibbles(qweight, 0)  # [In, Out]
        zero = nibbles(qzeros, 1).astype(np.int32) + zero_offset
        in_features = q.shape[0]
        size = in_features if group <= 0 else group
        group_of = np.arange(in_features) // size
        if g_idx is not None and not np.array_equal(g_idx, group_of):
            order = np.argsort(g_idx, kind="stable").astype(np.int32)
            assert np.array_equal(g_idx[order], group_of), "groups of unequal size"
            q = q[order]
    else:
        reverse = [AWQ_ORDER.index(k) for k in range(8)]
        columns = np.arange(qweight.shape[1] * 8).reshape(-1, 8)[:, reverse].reshape(-1)
        q = nibbles(qweight, 1)[:, columns]
        zero = nibbles(qzeros, 1)[:, columns].astype(np.int32)
        size = q.shape[0] if group <= 0 else group
    packed = pack_int4_groups(np.ascontiguousarray(q.T), size)
    return packed, np.ascontiguousarray(zero.T).astype(np.uint8), order


def unpack_int4_codes(packed: np.ndarray) -> np.ndarray:
    """Each byte's two codes, low first, along the last axis (the last axis
    doubles). Restates `torch/packed.py:21-24` and `quant.py:133-134`."""
    packed = np.asarray(packed, dtype=np.uint8)
    pairs = np.stack([packed & 15, packed >> 4], axis=-1)
    return pairs.reshape(*packed.shape[:-1], 2 * packed.shape[-1])


def unpack4(packed: np.ndarray, kind: str) -> np.ndarray:
    """`torch/packed.py:27-35` for the integer kinds: `u4` codes as uint8, `i4`
    sign-extended to int8."""
    codes = unpack_int4_codes(packed)
    if kind == "u4":
        return codes
    if kind == "i4":
        return ((codes.astype(np.int8) ^ 8) - 8).astype(np.int8)
    raise ValueError(f"`{kind}` is not an integer 4-bit format (i4, u4)")


def pack4(values: np.ndarray, kind: str) -> np.ndarray:
    """`torch/packed.py:61-75` for the integer kinds: integers wrap to 4 bits
    (floats round toward zero first), two a byte, low first."""
    if kind not in ("i4", "u4"):
        raise ValueError(f"`{kind}` is not an integer 4-bit format (i4, u4)")
    values = np.asarray(values)
    if values.shape[-1] % 2:
        raise ValueError(f"a 4-bit tensor's last axis is even, found shape {values.shape}")
    codes = (np.trunc(values).astype(np.int64) if values.dtype.kind == "f" else values.astype(np.int64)) & 15
    pairs = codes.astype(np.uint8).reshape(*codes.shape[:-1], -1, 2)
    return (pairs[..., 0] | (pairs[..., 1] << 4)).astype(np.uint8)


# ------------------------------------------------------------ int4 quantize


def quantize_int4_groups(weight: np.ndarray, group: int = 128) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """`(packed, scale, zero)` for an `[Out, In]` weight; scale is f32.

    Restates `quant.py:83-99` step for step, in f32: `scale = (max - min) / 15`
    (0 or NaN -> 1), `zero = clip(rint(-min / scale), 0, 15)`,
    `q = clip(rint(w / scale) + zero, 0, 15)`, rint ties to even.

    Pins: error <= step / 2 (`tests/test_quant_groups.py:48-56`); known answers
    for ramps and constant groups; brute-force nearest level on tiny groups
    (tests/test_oracle.py)."""
    if weight.ndim != 2:
        raise ValueError(f"a linear weight is [Out, In]; this one is {list(weight.shape)}")
    out_features, in_features = weight.shape
    if group <= 0 or group % 2 != 0 or in_features % group != 0:
        raise ValueError(f"groups of {group} must be even and divide the {in_features} inputs")
    grouped = weight.astype(np.float32).reshape(out_features, in_features // group, group)
    low = grouped.min(axis=-1)
    high = grouped.max(axis=-1)
    scale = (high - low) / np.float32(15.0)
    scale = np.where(scale > 0, scale, np.float32(1.0)).astype(np.float32)
    zero = np.clip(np.round(-low / scale), 0, 15).astype(np.uint8)
    q = np.clip(np.round(grouped / scale[..., None]) + zero[..., None].astype(np.float32), 0, 15)
    return pack_int4_groups(q.reshape(out_features, in_features), group), scale, zero


def dequantize_int4_groups(packed: np.ndarray, scale: np.ndarray, zero: np.ndarray) -> np.ndarray:
    """The f32 `[Out, In]` weight `(q - zero) * scale`. Restates `quant.py:131-136`
    and the body of `std.quant::dequantize_int4_groups` (`stdlib/quant.linnet:118-126`)
    before its final cast."""
    out_features, groups, half = packed.shape
    q = unpack_int4_codes(packed).reshape(out_features, groups, 2 * half)
    weight = (q.astype(np.float32) - zero[..., None].astype(np.float32)) * scale[..., None].astype(np.float32)
    return weight.reshape(out_features, groups * 2 * half)


def dequantize_int4_weight(packed: np.ndarray, scale_raw: np.ndarray, zero: np.ndarray, dtype: str) -> np.ndarray:
    """The dequantized weight in the scale's storage dtype, returned as the raw
    storage array (bf16 bits / float16 / float32): `(q - z) * s` computed in f32
    and rounded once. Restates `_int4_weight`/`_int4_unpack`
    (`src/backend/torch_source.cpp:1518-1550`) and the CPU branch of `_int4_pack`
    (`torch_source.cpp:1501-1504`).

    Pin: equals torch's `(q.to(bf16) - z.to(bf16)) * s` bit for bit, the
    reference's own exact check (`tests/test_quant_groups.py:151-162`)."""
    scale = decode_storage(scale_raw, dtype)
    weight = dequantize_int4_groups(packed, scale, zero)
    return encode_storage(weight, dtype)


def dequantize_int4_rows(packed: np.ndarray, scale_raw: np.ndarray, dtype: str) -> np.ndarray:
    """`std.quant::dequantize_int4` as `Int4Linear.forward` calls it
    (`stdlib/quant.linnet:22-29, 101-111`, through `dequantize_int8`, lines 13-20):
    `packed` [Out, In/2] holds signed 4-bit values two a byte, element 2k low
    (`tests/torch/test_quant.py:62-66`); `scale_raw` [Out] or [Out, 1] is the
    per-row scale in storage dtype `dtype`, widened to f32. Returns the raw storage
    array of `cast<T>(f32(q) * f32(scale))`, one rounding.

    Pins: the closed form on every code -8..7 at exact scales, and on random
    layers the f64 product of independently drawn int8 values and scales rounded
    once (tests/test_oracle.py::test_int4_rows_*)."""
    q = unpack4(packed, "i4").astype(np.float32)
    scale = decode_storage(np.asarray(scale_raw).reshape(-1), dtype).astype(np.float32)
    if scale.shape[0] != q.shape[0]:
        raise ValueError(f"one scale a row: {q.shape[0]} rows, {scale.shape[0]} scales")
    return encode_storage(q * scale[:, None], dtype)


# ------------------------------------------------------------ int8 quantize


def quantize_int8_groups(weight: np.ndarray, group: int = 128, dtype: str = "f32") -> tuple[np.ndarray, np.ndarray]:
    """`(q, scale)` for an `[Out, In]` weight: `scale = max|w| / 127` (0 -> 1)
    rounded to the storage dtype first, then `q = clip(rint(w / scale), -127, 127)`.
    Restates `quant.py:102-121`; scale returned as f32.

    Pins: error <= step / 2 (`tests/test_quant_8bit.py:235-242`); the scale is a
    value of the storage dtype; known answers (tests/test_oracle.py)."""
    if weight.ndim != 2:
        raise ValueError(f"a linear weight is [Out, In]; this one is {list(weight.shape)}")
    out_features, in_features = weight.shape
    if group <= 0 or in_features % group != 0:
        raise ValueError(f"groups of {group} must divide the {in_features} inputs")
    grouped = weight.astype(np.float32).reshape(out_features, in_features // group, group)
    scale = np.abs(grouped).max(axis=-1) / np.float32(127.0)
    scale = np.where(scale > 0, scale, np.float32(1.0)).astype(np.float32)
    scale = round_to_storage(scale, dtype).reshape(scale.shape)
    q = np.clip(np.round(grouped / scale[..., None]), -127, 127).astype(np.int8)
    return q.reshape(out_features, in_features), scale


def dequantize_int8_groups(q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """Restates `quant.py:124-128`: the f32 weight `q * scale[group]`."""
    out_features, in_features = q.shape
    groups = scale.shape[1]
    grouped = q.astype(np.float32).reshape(out_features, groups, in_features // groups)
    return (grouped * scale[..., None].astype(np.float32)).reshape(out_features, in_features)


# --------------------------------------------------- per-token activation rounding


def rows8(x: np.ndarray, fp8: bool) -> tuple[np.ndarray, np.ndarray]:
    """Each row of `x` (f32 values of the bf16/f16 input) rounded to 8 bits with
    a scale of its own: `scale = max(max|x|, 1e-12) / (448 or 127)` in f32,
    `x / scale` in f32, then FP8 E4M3 of `clamp(., +-448)` (round to nearest
    even) or int8 `clamp(trunc(v +- 0.5), +-127)` (half away from zero, the add
    done in f32). Returns (codes as uint8 bytes / int8, scale `[rows, 1]` f32).

    Restates `torch/kernels.py:677-707` (`_rows8_kernel`), with IEEE division.
    Pins: fp8 codes equal torch's `float8_e4m3fn` cast of the same quotients;
    int8 codes equal round-half-away-from-zero computed exactly in Python on a
    brute-force sample (tests/test_oracle.py)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    largest = np.float32(448.0 if fp8 else 127.0)
    top = np.abs(x).max(axis=-1, keepdims=True) if x.shape[-1] else np.zeros((x.shape[0], 1), np.float32)
    scale = (np.maximum(top, np.float32(1e-12)) / largest).astype(np.float32)
    v = (x / scale).astype(np.float32)
    if fp8:
        return encode_fp8(np.clip(v, np.float32(-448.0), np.float32(448.0))), scale
    half = np.where(v >= 0, v + np.float32(0.5), v - np.float32(0.5)).astype(np.float32)
    return np.clip(np.trunc(half), -127, 127).astype(np.int8), scale


def fp8_groups(x: np.ndarray, group: int, padded: int) -> tuple[np.ndarray, np.ndarray]:
    """Each `group` inputs of each row of `x` (f32 values of the input) rounded to
    FP8 E4M3 with a scale of their own, `rows8`'s arithmetic per group, the rows
    padded with zeros (scale 1) to `padded`. Returns (codes [padded, In] uint8, scales
    [padded, In/group] f32). Restates `torch/kernels.py:757-795` (`_fp8_groups_kernel`,
    `_fp8_groups`), with IEEE division.

    Pin: each group equals `rows8` (already pinned against torch's cast) applied
    to that group alone, and padded rows are zero codes with scale 1
    (tests/test_oracle.py::test_fp8_groups_is_rows8_per_group)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, depth = x.shape
    groups = depth // group
    full = np.zeros((padded, depth), np.float32)
    full[:rows] = x
    grouped = full.reshape(padded * groups, group)
    codes, scale = rows8(grouped, True)
    scale = scale.reshape(padded, groups)
    scale[rows:] = np.float32(1.0)
    return codes.reshape(padded, depth), scale


# ---------------------------------------------------------------------- MXFP4

# E2M1 values by code, as the generated module's fallback tabulates them
# (`src/backend/torch_source.cpp:1585-1586`, `_FP4`).
FP4_VALUES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0],
                      dtype=np.float32)


def dequantize_mxfp4(blocks: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """MXFP4 blocks [..., G, 16] bytes and E8M0 scales [..., G] as the f32 weights
    [..., G * 32]: byte j's low nibble is element 2j, its high one 2j + 1, each
    E2M1 code's value times 2^(scale - 127). Restates `stdlib/quant.linnet:334-341`
    (`dequantize_mxfp4`) and the generated fallback (`torch_source.cpp:1597-1600`).

    Pin: `FP4_VALUES` against E2M1's definition (sign, two exponent bits of bias
    1, one mantissa bit, exponent 0 subnormal), the scale against `np.ldexp`, and
    the element order against a hand-built block
    (tests/test_oracle.py::test_mxfp4_decoding_from_the_format_definition)."""
    b = np.asarray(blocks, dtype=np.uint8)
    values = np.stack([FP4_VALUES[b & 15], FP4_VALUES[b >> 4]], axis=-1)
    values = values.reshape(*b.shape[:-1], 32)
    factor = np.ldexp(np.float32(1.0), np.asarray(scales).astype(np.int32) - 127).astype(np.float32)
    return (values * factor[..., None]).reshape(*b.shape[:-2], b.shape[-2] * 32)


# ------------------------------------------------------------------------ NF4

# QLoRA's NormalFloat-4 values by code, as bitsandbytes' map holds them (the
# reference's `NF4`, `python/linnet/src/linnet/quant.py:373-394`, and
# `std.dtypes::nf4`, `stdlib/dtypes.linnet:32-52`).
NF4_VALUES = np.array(
    [-1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453, -0.28444138169288635,
     -0.18477343022823334, -0.09105003625154495, 0.0, 0.07958029955625534, 0.16093020141124725,
     0.2461123019456863, 0.33791524171829224, 0.44070982933044434, 0.5626170039176941,
     0.7229568362236023, 1.0],
    dtype=np.float32,
)


def nf4_weight(codes: np.ndarray, absmax: np.ndarray, block: int) -> np.ndarray:
    """`dequantize_nf4` in f32 (`stdlib/quant.linnet:180-187`): codes [Out, In/2]
    bytes, the first input of a pair in the low nibble; absmax [Out, In/block];
    `weight[o, i] = NF4_VALUES[q[o, i]] * absmax[o, i // block]`, one f32 product.

    Pin: `NF4_VALUES` against QLoRA's construction (normal quantiles, scipy), and
    the nibble and block order against a hand-built layer whose every element
    is told apart (tests/test_oracle.py::test_nf4_table_is_qloras_normal_quantiles,
    ::test_nf4_weight_from_the_layout_definition)."""
    q = np.asarray(codes, dtype=np.uint8)
    values = np.stack([NF4_VALUES[q & 15], NF4_VALUES[q >> 4]], axis=-1).reshape(q.shape[0], 2 * q.shape[1])
    scale = np.asarray(absmax, dtype=np.float32)
    return (values.reshape(q.shape[0], -1, block) * scale[:, :, None]).reshape(values.shape).astype(np.float32)


def dequantize_nf4(codes: np.ndarray, absmax: np.ndarray, block: int, dtype: str) -> np.ndarray:
    """`dequantize_nf4<..., T>`: the f32 weight rounded to `dtype`, as the raw
    storage array of `encode_storage` (`cast<T>` of quant.linnet:186)."""
    return encode_storage(nf4_weight(codes, absmax, block), dtype)


def bnb_nf4_layer(packed: np.ndarray, absmax: np.ndarray, out_features: int, in_features: int, block: int,
                  nested_absmax: np.ndarray | None = None, nested_map: np.ndarray | None = None,
                  nested_block: int = 0, offset: float = 0.0) -> tuple[np.ndarray, np.ndarray]:
    """A bitsandbytes 4-bit NF4 layer as `Nf4Linear` holds it: (codes [Out, In/2]
    with each byte's nibbles swapped, absmax [Out, In/block] f32). Restates
    `_bnb_nf4` (`quant.py:414-466`): bitsandbytes keeps the first code of a pair in
    the high nibble; with double quantization a block's absmax is
    `nested_map[code] * nested_absmax[i // nested_block] + float32(offset)` in f32.

    Pin: a layer packed the way the reference's test writes bitsandbytes'
    (`codes[1::2] | codes[0::2] << 4`, `python/linnet/tests/test_nf4.py:49-75`)
    comes back as its codes, and nested scales built from exact binary values
    decode to their known sums (tests/test_oracle.py::test_bnb_nf4_layer)."""
    raw = np.asarray(packed, dtype=np.uint8).reshape(-1)
    swapped = ((raw >> 4) | (raw << 4)).astype(np.uint8)
    if nested_map is not None:
        codes = np.asarray(absmax, dtype=np.uint8).reshape(-1)
        outer = np.asarray(nested_absmax, dtype=np.float32).reshape(-1)
        scale = np.asarray(nested_map, dtype=np.float32).reshape(-1)[codes] * outer[np.arange(codes.size) // nested_block]
        scale = (scale + np.float32(offset)).astype(np.float32)
    else:
        scale = np.asarray(absmax, dtype=np.float32).reshape(-1)
    return swapped.reshape(out_features, in_features // 2), scale.reshape(out_features, in_features // block)
