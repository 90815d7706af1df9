"""Group-wise 4-bit and 8-bit weight quantization with the reference's names,
layouts and rounding (`python/linnet/src/linnet/quant.py:1-136, 242-248`), computed
by the HIP kernels on the GPU.

Layouts (`std.quant::Int4GroupLinear`, `Int8GroupLinear`):

    int4: weight [Out, In/group, group/2] u8 (two codes a byte, low first),
          scale  [Out, In/group] (f32 here; stored in the model's dtype),
          zero   [Out, In/group] u8 in 0..15
    int8: weight [Out, In] i8 in -127..127, scale [Out, In/group]

Every function takes a numpy array or a torch tensor and returns the same kind
(numpy results are computed on `cuda:0` and copied back); the codes, scales and
zero points are bit for bit numpy's.

`quantize_checkpoint` applies them to the linear weights of a SafeTensors
checkpoint, and `import_quantized` repacks a 4-bit GPTQ or AWQ checkpoint into
the same layout (plus `.order`, the inputs' order, for GPTQ's activation order),
both on the GPU (`quant.py:139-369`).
"""

from __future__ import annotations

import fnmatch
import json
import re
from collections.abc import Iterable, Mapping
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

from . import weights
from .errors import LinnetError
from .torch import kernels

# Where the 8-bit linear layers switch kernels (`quant.py:73-80`): up to
# FEW_ROWS rows multiply the weight as it is, up to TILED_ROWS the weight-only
# tiled kernel beats the library GEMM over the weight dequantized for the call.
FEW_ROWS = 32
TILED_ROWS = 64


def _device_tensor(array: np.ndarray | torch.Tensor) -> tuple[torch.Tensor, bool]:
    if isinstance(array, torch.Tensor):
        return (array if array.is_cuda else array.to("cuda")), False
    if not torch.cuda.is_available():
        raise LinnetError("linnet_amd quantizes on the GPU; no GPU is available")
    return torch.from_numpy(np.ascontiguousarray(array)).to("cuda"), True


def _back(t: torch.Tensor, to_numpy: bool) -> np.ndarray | torch.Tensor:
    return t.cpu().numpy() if to_numpy else t


def quantize_int4_groups(weight, group: int = 128):
    """`(packed, scale, zero)` for an `[Out, In]` weight; `scale` is f32
    (`quant.py:83-99`)."""
    w, numpy = _device_tensor(weight)
    packed, scale, zero = kernels.quantize_int4(w, group)
    return _back(packed, numpy), _back(scale, numpy), _back(zero, numpy)


def pack_int4_groups(q, group: int):
    """`[Out, In]` codes in 0..15 as `[Out, In/group, group/2]` bytes, low nibble
    first (`quant.py:242-248`)."""
    codes, numpy = _device_tensor(q)
    out_features, in_features = codes.shape
    if group <= 0 or group % 2 or in_features % group:
        raise LinnetError(f"groups of {group} must be even and divide the {in_features} inputs")
    packed = kernels.pack4(codes.reshape(out_features, in_features // group, group))
    return _back(packed, numpy)


def dequantize_int4_groups(packed, scale, zero):
    """The f32 `[Out, In]` weight `(q - zero) * scale` (`quant.py:131-136`)."""
    p, numpy = _device_tensor(packed)
    s, _ = _device_tensor(scale)
    z, _ = _device_tensor(zero)
    weight = kernels.int4_weight(p, s.to(torch.float32), z)
    return _back(weight, numpy)


def quantize_int8_groups(weight, group: int = 128, dtype: str = "f32"):
    """`(q, scale)`: `scale = max|w| / 127` rounded to `dtype` first, then
    `q = clip(rint(w / scale), -127, 127)`; scale is f32 (`quant.py:102-121`)."""
    w, numpy = _device_tensor(weight)
    q, scale = kernels.quantize_int8(w, group, dtype)
    return _back(q, numpy), _back(scale, numpy)


def dequantize_int8_groups(q, scale):
    """The f32 `[Out, In]` weight `q * scale[group]` (`quant.py:124-128`)."""
    codes, numpy = _device_tensor(q)
    s, _ = _device_tensor(scale)
    out_features, in_features = codes.shape
    group = in_features // s.shape[1]
    weight = kernels.dequantize8(codes, s.to(torch.float32), False, group, 1, torch.float32)
    return _back(weight, numpy)


# ---------------------------------------------------------------- checkpoints
#
# Both tools write a checkpoint with every tensor of the input under its Linnet
# path, the chosen linear layers replaced by the tensors of their quantized
# block: `P.weight`, `P.scale` (in the model's scale dtype) and, for 4 bits,
# `P.zero` -- plus `P.order` for a GPTQ layer in activation order -- where `P.`
# names the layer's parameters (`siblings`).


def siblings(path: str) -> str:
    """The prefix shared by the parameters of the block owning `path`'s weight:
    `"attn.q."` for `"attn.q.weight"`, `""` for a root block's `"weight"`, and
    `path + "."` for a path that is not a weight (the reference names them the
    same way, `quant.py:198-204`)."""
    head, dot, last = path.rpartition(".")
    return head + dot if last == "weight" else path + "."


def _scale_name(dtype: str) -> str:
    try:
        return weights.STORAGE[dtype]
    except KeyError:
        raise LinnetError(f"scale dtype {dtype!r}: choose bf16, f16 or f32") from None


def _bound(bindings: str | Path | Mapping[str, str] | None) -> dict[str, list[str]]:
    """Each checkpoint tensor's Linnet paths (its own name when unbound)."""
    if bindings is None:
        return {}
    table = dict(bindings) if isinstance(bindings, Mapping) else weights.read_bindings(bindings)
    return weights.paths_by_tensor({str(k): str(v) for k, v in table.items()})


def _block_tensors(prefix: str, dtype: str, weight: torch.Tensor, weight_dtype: str, scale: torch.Tensor,
                   zero: torch.Tensor | None = None, order: np.ndarray | None = None):
    """The checkpoint entries of one quantized block, in the order its parameters
    are declared (weight, scale, zero, order)."""
    yield prefix + "weight", weight_dtype, tuple(weight.shape), weights.tensor_bytes(weight)
    stored = _scale_name(dtype)
    yield prefix + "scale", stored, tuple(scale.shape), weights.encode_floats(scale, stored)
    if zero is not None:
        yield prefix + "zero", "U8", tuple(zero.shape), weights.tensor_bytes(zero)
    if order is not None:
        yield prefix + "order", "I32", (order.size,), order.astype("<i4").tobytes()


def _on_gpu(device: torch.device | str | None) -> torch.device:
    if not torch.cuda.is_available():
        raise LinnetError("the checkpoint tools of linnet_amd run their kernels on a GPU, and none is visible")
    return torch.device("cuda" if device is None else device)


def quantize_checkpoint(
    weights_path: str | Path,
    output: str | Path,
    *,
    patterns: Iterable[str],
    group: int = 128,
    dtype: str = "bf16",
    bindings: str | Path | Mapping[str, str] | None = None,
    bits: int = 4,
    device: torch.device | str | None = None,
) -> list[str]:
    """Quantizes a SafeTensors checkpoint on the GPU: every `.weight` whose Linnet
    path matches one of the glob `patterns` becomes an `Int4GroupLinear` (`bits`
    4: `.weight`, `.scale`, `.zero`) or `Int8GroupLinear` (`bits` 8: `.weight`,
    `.scale`) block with scales stored in `dtype`; every other tensor is copied.
    The codes and scales are those of `quantize_int4_groups` /
    `quantize_int8_groups`, bit for bit. Returns the quantized paths in file
    order. Replaces the reference's `quantize_checkpoint` (`quant.py:139-181`)."""
    if bits not in (4, 8):
        raise LinnetError(f"bits={bits}: the quantized blocks hold 4-bit or 8-bit weights")
    _scale_name(dtype)
    target = _on_gpu(device)
    globs = tuple(patterns)

    def chosen(path: str) -> bool:
        return path.endswith(".weight") and any(fnmatch.fnmatchcase(path, g) for g in globs)

    paths = _bound(bindings)
    writer = weights.CheckpointWriter()
    done: list[str] = []
    for stored in weights.open_checkpoint(weights_path).values():
        for path in paths.get(stored.name) or [stored.name]:
            if not chosen(path):
                writer.add(path, stored.dtype, stored.shape, stored)
                continue
            values = weights.float_tensor(stored, target)
            if bits == 4:
                packed, scale, zero = kernels.quantize_int4(values, group)
                block = _block_tensors(siblings(path), dtype, packed, "U8", scale, zero)
            else:
                q, scale = kernels.quantize_int8(values, group, dtype)
                block = _block_tensors(siblings(path), dtype, q, "I8", scale)
            for entry in block:
                writer.add(*entry)
            done.append(path)
    if not done:
        raise LinnetError(f"no `.weight` path matched {', '.join(globs) or 'the (empty) patterns'}")
    writer.write(output, {"format": "pt"})
    return done


# ------------------------------------------------------- GPTQ / AWQ import
#
# What a calibrated checkpoint's `quantization_config` may say, with the names
# GPTQ and AWQ give each setting, first name first.
_SETTINGS = {"bits": ("bits", "w_bit"), "group": ("group_size", "q_group_size")}


def _config_number(config: Mapping[str, object], setting: str, default: int) -> int:
    names = _SETTINGS[setting]
    raw = next((config[n] for n in names if n in config), default)
    if isinstance(raw, bool) or not isinstance(raw, (int, float, str)):
        raise LinnetError(f"quantization_config: {names[0]} = {raw!r} is not an integer")
    try:
        return int(raw)
    except ValueError:
        raise LinnetError(f"quantization_config: {names[0]} = {raw!r} is not an integer") from None


@dataclass(frozen=True)
class _Calibrated:
    """How a 4-bit calibrated checkpoint stores its layers: `method` ("gptq" or
    "awq"), the group size, and the offset added to each stored zero point (GPTQ's
    original format, `checkpoint_format` "gptq", stores zero - 1)."""

    method: str
    group: int
    zero_offset: int

    @classmethod
    def read(cls, config: Mapping[str, object]) -> _Calibrated:
        method = str(config.get("quant_method", "")).lower()
        if method not in ("gptq", "awq"):
            raise LinnetError(f"quant_method {method!r}: linnet_amd imports GPTQ and AWQ checkpoints")
        if _config_number(config, "bits", 4) != 4:
            raise LinnetError(f"{method.upper()} checkpoint of {config.get('bits', config.get('w_bit'))} bits: "
                              "only 4-bit layers become Int4GroupLinear")
        version = str(config.get("version", "gemm")).lower()
        if method == "awq" and version != "gemm":
            raise LinnetError(f"AWQ version {version!r}: only the GEMM packing of the words is read")
        original_gptq = method == "gptq" and config.get("checkpoint_format", "gptq") == "gptq"
        return cls(method, _config_number(config, "group", 128), 1 if original_gptq else 0)


def _config_beside(weights_path: str | Path) -> Mapping[str, object]:
    where = Path(weights_path)
    config_file = (where if where.is_dir() else where.parent) / "config.json"
    if not config_file.is_file():
        raise LinnetError(f"{config_file} does not exist: pass the quantization_config as `config`")
    document = json.loads(config_file.read_text(encoding="utf-8"))
    found = document.get("quantization_config") if isinstance(document, dict) else None
    if not isinstance(found, Mapping):
        raise LinnetError(f"{config_file} holds no quantization_config object")
    return found


# The tensors a calibrated layer `L` stores: `L.qweight`, `L.qzeros`, `L.scales`
# and, for GPTQ, `L.g_idx` (each input's group).
_LAYER_PARTS = ("qweight", "qzeros", "scales", "g_idx")


def _calibrated_layers(index: Mapping[str, weights.StoredTensor]) -> dict[str, dict[str, weights.StoredTensor]]:
    """Layer name -> its stored parts, for every layer with a `qweight`, by name."""
    parts: dict[str, dict[str, weights.StoredTensor]] = {}
    for name, stored in index.items():
        layer, _, part = name.rpartition(".")
        if part in _LAYER_PARTS:
            parts.setdefault(layer, {})[part] = stored
    return {layer: found for layer, found in sorted(parts.items()) if "qweight" in found}


def input_order(g_idx: np.ndarray, group: int, in_features: int | None = None) -> np.ndarray | None:
    """The order that makes each group's inputs contiguous, for a GPTQ layer
    quantized in activation order: `order[k]` is the input at position k once the
    inputs are sorted by group, ties kept in input order; None when every input
    already sits in group `i // group`. Every group must hold exactly `group`
    inputs. (`take_inputs(x, order)` then feeds the product, `stdlib/quant.linnet:163-174`.)"""
    ids = np.asarray(g_idx).reshape(-1).astype(np.int64)
    if in_features is not None and ids.size != in_features:
        raise LinnetError(f"g_idx has {ids.size} entries for {in_features} inputs")
    groups = ids.size // group
    if np.array_equal(ids, np.arange(ids.size) // group):
        return None
    if ids.size % group or ids.min(initial=0) < 0 or ids.max(initial=0) >= groups:
        raise LinnetError(f"g_idx names groups outside 0..{groups - 1}")
    sizes = np.bincount(ids, minlength=groups)
    if np.any(sizes != group):
        raise LinnetError(f"g_idx puts {sizes.min()}..{sizes.max()} inputs in a group of {group}")
    return np.argsort(ids, kind="stable").astype(np.int32)


def import_quantized(
    weights_path: str | Path,
    output: str | Path,
    *,
    bindings: str | Path | Mapping[str, str] | None = None,
    dtype: str = "bf16",
    config: Mapping[str, object] | None = None,
    device: torch.device | str | None = None,
) -> list[str]:
    """Converts a 4-bit GPTQ or AWQ checkpoint on the GPU: each calibrated layer
    (`qweight`, `qzeros`, `scales`, and GPTQ's `g_idx`) becomes an
    `Int4GroupLinear` block under its Linnet path -- `.weight`, `.scale` (stored in
    `dtype`), `.zero`, and `.order` for activation order -- with the repack kernel
    (`lnq_int4_repack`); every other tensor is copied. `config` is the
    checkpoint's `quantization_config`, read from the `config.json` beside
    `weights_path` when not given. Returns the layers' `.weight` paths. Replaces the
    GPTQ / AWQ part of the reference's `import_quantized` (`quant.py:259-369`). A
    bitsandbytes 4-bit NF4 checkpoint (`quant_method` "bitsandbytes") becomes
    `Nf4Linear` blocks instead (`.weight` [Out, In/2] U8, `.absmax` [Out, In/block]
    F32), through `lnq_nf4_repack` (`quant.py:402-499`); `dtype` is then unused."""
    config = config if config is not None else _config_beside(weights_path)
    if str(config.get("quant_method", "")).lower() == "bitsandbytes":
        return _import_nf4(weights_path, output, config, _bound(bindings), _on_gpu(device))
    calibrated = _Calibrated.read(config)
    _scale_name(dtype)
    target = _on_gpu(device)
    index = weights.open_checkpoint(weights_path)
    layers = _calibrated_layers(index)
    paths = _bound(bindings)
    writer = weights.CheckpointWriter()
    done: list[str] = []
    for layer, parts in layers.items():
        blocks = _import_layer(layer, parts, calibrated, target)
        name = layer + ".weight"
        for path in paths.get(name) or [name]:
            for entry in _block_tensors(siblings(path), dtype, *blocks):
                writer.add(*entry)
            done.append(path)
    if not done:
        raise LinnetError(f"{weights_path}: no `.qweight` tensor, so no {calibrated.method.upper()} layer to import")
    consumed = {f"{layer}.{part}" for layer, parts in layers.items() for part in parts}
    for name, stored in index.items():
        if name not in consumed:
            for path in paths.get(name) or [name]:
                writer.add(path, stored.dtype, stored.shape, stored)
    writer.write(output, {"format": "pt"})
    return done


def _import_layer(layer: str, parts: Mapping[str, weights.StoredTensor], calibrated: _Calibrated,
                  target: torch.device) -> tuple:
    """One calibrated layer as `(packed, "U8", scale [Out, Groups] f32, zero, order)`."""
    absent = [p for p in ("qzeros", "scales") if p not in parts]
    if absent:
        raise LinnetError(f"{layer}: `qweight` without {' and '.join(absent)}")
    words = weights.tensor_from(parts["qweight"], torch.int32, target)
    zero_words = weights.tensor_from(parts["qzeros"], torch.int32, target)
    scales = weights.float_tensor(parts["scales"], target)
    if words.dim() != 2 or zero_words.dim() != 2 or scales.dim() != 2:
        raise LinnetError(f"{layer}: qweight, qzeros and scales must be matrices")
    gptq = calibrated.method == "gptq"
    # GPTQ packs 8 inputs a word down the rows, AWQ 8 outputs a word along them.
    in_features = words.shape[0] * 8 if gptq else words.shape[0]
    out_features = words.shape[1] if gptq else words.shape[1] * 8
    group = calibrated.group if calibrated.group > 0 else in_features
    groups = in_features // group
    if in_features % group or zero_words.shape != (groups, out_features // 8) or scales.shape != (groups, out_features):
        raise LinnetError(f"{layer}: {in_features} inputs x {out_features} outputs do not fit groups of {group} "
                          f"(qzeros {tuple(zero_words.shape)}, scales {tuple(scales.shape)})")
    order = None
    if gptq and "g_idx" in parts:
        order = input_order(weights.tensor_from(parts["g_idx"], torch.int32, "cpu").numpy(), group, in_features)
    packed, zero = kernels.int4_repack(words, zero_words, calibrated.method, group, calibrated.zero_offset,
                                       None if order is None else torch.from_numpy(order).to(target))
    return packed, "U8", scales.t().contiguous(), zero, order


__all__ = [
    "NF4",
    "FEW_ROWS",
    "TILED_ROWS",
    "dequantize_int4_groups",
    "dequantize_int8_groups",
    "import_quantized",
    "input_order",
    "pack_int4_groups",
    "quantize_checkpoint",
    "quantize_int4_groups",
    "quantize_int8_groups",
    "siblings",
]


# ------------------------------------------------------- bitsandbytes NF4 import
#
# bitsandbytes saves a 4-bit `Linear4bit` layer under its weight's name W:
#   W                                   uint8: the weight flattened row-major, two
#                                       codes a byte, the earlier one in the high
#                                       nibble
#   W.absmax                            one scale per `blocksize` codes: float32, or
#                                       under double quantization a uint8 code
#   W.quant_map                         the 16 values the codes stand for
#   W.nested_absmax, W.nested_quant_map double quantization only: a float32 scale
#                                       per `nested_blocksize` absmax codes, and the
#                                       256 values those codes stand for
#   W.quant_state.bitsandbytes__<type>  uint8: the UTF-8 bytes of a JSON object with
#                                       "shape" and "blocksize" (and, under double
#                                       quantization, "nested_blocksize" and
#                                       "nested_offset")
_BNB_STATE = re.compile(r"(?P<weight>.+)\.quant_state\.bitsandbytes__(?P<codes>\w+)")
# The code type a `quantization_config` without `bnb_4bit_quant_type` means
# (BitsAndBytesConfig's default).
_BNB_DEFAULT_CODES = "fp4"

# NF4's 16 values by code (QLoRA's normal quantiles, as bitsandbytes' map holds
# them; the reference's `NF4`, quant.py:373-394).
NF4 = np.array(
    [-1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453, -0.28444138169288635,
     -0.18477343022823334, -0.09105003625154495, 0.0, 0.07958029955625534, 0.16093020141124725,
     0.2461123019456863, 0.33791524171829224, 0.44070982933044434, 0.5626170039176941,
     0.7229568362236023, 1.0],
    dtype=np.float32,
)


def _four_bit_codes(config: Mapping[str, object]) -> str:
    """The code type of a bitsandbytes checkpoint's 4-bit layers, refusing a
    configuration that has none (8-bit LLM.int8 layers) or whose codes are not
    NF4 (bitsandbytes' FP4 has no kernel here)."""
    if True not in (config.get("load_in_4bit"), config.get("_load_in_4bit")):
        raise LinnetError("bitsandbytes quantization_config without load_in_4bit: its layers are not 4-bit")
    codes = str(config.get("bnb_4bit_quant_type", _BNB_DEFAULT_CODES)).lower()
    if codes != "nf4":
        raise LinnetError(f"bitsandbytes 4-bit layers of {codes!r} codes: only NF4 codes have a kernel here")
    return codes


def _state_int(state: Mapping[str, object], key: str, weight: str) -> int | None:
    value = state.get(key)
    if value is None:
        return None
    if isinstance(value, bool) or not isinstance(value, int) or value <= 0:
        raise LinnetError(f"{weight}: quantization state field {key} = {value!r}, expected a positive integer")
    return value


@dataclass(frozen=True)
class _Nf4State:
    """A bitsandbytes 4-bit layer's saved state: the [Out, In] weight shape, the
    codes a scale covers, and, under double quantization, the absmax codes a
    nested scale covers and the offset added back to every decoded scale."""

    out_features: int
    in_features: int
    block: int
    nested_block: int = 0
    nested_offset: float = 0.0

    @property
    def blocks(self) -> int:
        return self.out_features * self.in_features // self.block

    @classmethod
    def decode(cls, stored: weights.StoredTensor, weight: str) -> _Nf4State:
        try:
            state = json.loads(bytes(stored.view()))
        except ValueError as err:  # bad UTF-8 or bad JSON
            raise LinnetError(f"{weight}: `{stored.name}` does not decode as JSON ({err})") from None
        if not isinstance(state, dict):
            raise LinnetError(f"{weight}: `{stored.name}` decodes to a JSON {type(state).__name__}, not an object")
        shape = state.get("shape")
        if not (isinstance(shape, list) and len(shape) == 2
                and all(isinstance(d, int) and not isinstance(d, bool) and d > 0 for d in shape)):
            raise LinnetError(f"{weight}: quantization state shape {shape!r}, expected [out_features, in_features]")
        block = _state_int(state, "blocksize", weight)
        if block is None:
            raise LinnetError(f"{weight}: the quantization state gives no blocksize")
        out_features, in_features = shape
        if block % 2 or in_features % block:
            raise LinnetError(f"{weight}: rows of {in_features} inputs are not whole blocks of {block} codes, "
                              "which Nf4Linear's [Out, In / block] absmax needs")
        nested_block = _state_int(state, "nested_blocksize", weight)
        offset = state.get("nested_offset")
        if (nested_block is None) != (offset is None):
            raise LinnetError(f"{weight}: double quantization needs both nested_blocksize and nested_offset")
        if nested_block is None:
            return cls(out_features, in_features, block)
        if isinstance(offset, bool) or not isinstance(offset, (int, float)):
            raise LinnetError(f"{weight}: nested_offset = {offset!r}, expected a number")
        return cls(out_features, in_features, block, nested_block, float(offset))

    def tensors(self, weight: str) -> dict[str, str]:
        """The checkpoint names of the layer's tensors, by role."""
        names = {"codes": weight, "absmax": weight + ".absmax", "values": weight + ".quant_map"}
        if self.nested_block:
            names |= {"outer": weight + ".nested_absmax", "table": weight + ".nested_quant_map"}
        return names


def _holds_nf4(stored: weights.StoredTensor) -> bool:
    """Whether a stored quant_map is NF4's 16 values in code order, exactly as its
    own dtype holds them (a 16-bit map as those values rounded to it, an f32 or
    f64 map as their f32 values)."""
    if stored.dtype not in weights.FLOAT_DTYPES or int(np.prod(stored.shape)) != 16:
        return False
    held = weights.tensor_from(stored, weights.FLOAT_DTYPES[stored.dtype], "cpu").reshape(-1)
    width = held.dtype if held.element_size() < 4 else torch.float32
    return torch.equal(held.to(width), torch.from_numpy(NF4).to(width))


def _import_nf4(weights_path: str | Path, output: str | Path, config: Mapping[str, object],
                paths: Mapping[str, list[str]], target: torch.device) -> list[str]:
    """`import_quantized` for a bitsandbytes 4-bit NF4 checkpoint: each layer,
    in checkpoint order, becomes `Nf4Linear`'s `.weight` (codes [Out, In/2], the
    first input in the low nibble) and `.absmax` ([Out, In/block] f32, nested
    scales decoded), through the HIP repack (`kernels.nf4_repack`); every other
    tensor is copied."""
    _four_bit_codes(config)
    index = weights.open_checkpoint(weights_path)
    writer = weights.CheckpointWriter()
    layer_tensors: set[str] = set()
    done: list[str] = []
    for name, stored in index.items():
        found = _BNB_STATE.fullmatch(name)
        if found is None:
            continue
        weight = found["weight"]
        if found["codes"].lower() != "nf4":
            raise LinnetError(f"{weight}: a layer of {found['codes']!r} codes: only NF4 codes have a kernel here")
        state = _Nf4State.decode(stored, weight)
        if not state.nested_block and weight + ".nested_absmax" in index:
            raise LinnetError(f"{weight}: the checkpoint holds nested scales, but the state has no nested_blocksize")
        names = state.tensors(weight)
        codes, absmax = _repack_nf4(weight, state, {role: index.get(n) for role, n in names.items()}, target)
        layer_tensors |= {name, *names.values()}
        for path in paths.get(weight) or [weight]:
            prefix = siblings(path)
            writer.add(prefix + "weight", "U8", tuple(codes.shape), weights.tensor_bytes(codes))
            writer.add(prefix + "absmax", "F32", tuple(absmax.shape), weights.tensor_bytes(absmax))
            done.append(path)
    if not done:
        raise LinnetError(f"{weights_path}: no tensor is a bitsandbytes 4-bit state "
                          "(`<weight>.quant_state.bitsandbytes__nf4`)")
    for name, stored in index.items():
        if name not in layer_tensors:
            for path in paths.get(name) or [name]:
                writer.add(path, stored.dtype, stored.shape, stored)
    writer.write(output, {"format": "pt"})
    return done


def _repack_nf4(weight: str, state: _Nf4State, parts: Mapping[str, weights.StoredTensor | None],
                target: torch.device) -> tuple[torch.Tensor, torch.Tensor]:
    """One layer's tensors, checked against its state, repacked on `target`."""
    from .torch import kernels

    absent = [role for role, stored in parts.items() if stored is None]
    if absent:
        raise LinnetError(f"{weight}: the checkpoint lacks the layer's {', '.join(absent)} "
                          f"({', '.join(state.tensors(weight)[role] for role in absent)})")
    if not _holds_nf4(parts["values"]):
        raise LinnetError(f"{weight}: `{parts['values'].name}` is not NF4's 16 values in code order")
    codes = weights.tensor_from(parts["codes"], torch.uint8, target).reshape(-1)
    if not state.nested_block:
        absmax = weights.float_tensor(parts["absmax"], target).reshape(-1)
        return kernels.nf4_repack(codes, absmax, state.out_features, state.in_features, state.block)
    if parts["absmax"].dtype != "U8":
        raise LinnetError(f"{weight}: double quantization stores absmax as U8 codes, not {parts['absmax'].dtype}")
    absmax_codes = weights.tensor_from(parts["absmax"], torch.uint8, target).reshape(-1)
    outer = weights.float_tensor(parts["outer"], target).reshape(-1)
    table = weights.float_tensor(parts["table"], target).reshape(-1)
    return kernels.nf4_repack(codes, absmax_codes, state.out_features, state.in_features, state.block, outer, table,
                              state.nested_block, state.nested_offset)
