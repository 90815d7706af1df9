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
# A bitsandbytes 4-bit layer `L` stores `L.weight` (two codes a byte, the first
# in the high nibble, the weight flattened), `L.weight.absmax` (one scale a
# block, or its uint8 code under double quantization), `L.weight.quant_map` (the
# 16 values), for double quantization `L.weight.nested_absmax` and
# `L.weight.nested_quant_map`, and its state -- shape, block size, nested block
# size and offset -- as JSON bytes in `L.weight.quant_state.bitsandbytes__<type>`.
_NF4_STATE = ".quant_state.bitsandbytes__"
_NF4_SIDE = (".absmax", ".quant_map", ".nested_absmax", ".nested_quant_map")

# NF4's 16 values by code (QLoRA's normal quantiles, as bitsandbytes' map holds
# them; the reference's `NF4`, quant.py:373-394).
NF4 = np.array(
    [-1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453, -0.28444138169288635,
     -0.18477343022823334, -0.09105003625154495, 0.0, 0.07958029955625534, 0.16093020141124725,
     0.2461123019456863, 0.33791524171829224, 0.44070982933044434, 0.5626170039176941,
     0.7229568362236023, 1.0],
    dtype=np.float32,
)


@dataclass(frozen=True)
class _Nf4Layer:
    """What a bitsandbytes NF4 layer's state says: its [Out, In] shape, the
    block size, and for double quantization the nested block size and offset."""

    weight: str
    out_features: int
    in_features: int
    block: int
    nested_block: int = 0
    offset: float = 0.0

    @classmethod
    def parse(cls, weight: str, stored: weights.StoredTensor) -> _Nf4Layer:
        try:
            state = json.loads(bytes(stored.view()).decode("utf-8"))
        except (UnicodeDecodeError, json.JSONDecodeError):
            state = None
        if not isinstance(state, dict):
            raise LinnetError(f"`{stored.name}` holds no quantization state")
        shape, block = state.get("shape"), state.get("blocksize")
        dims = [d for d in shape if isinstance(d, int) and not isinstance(d, bool)] if isinstance(shape, list) else []
        if len(dims) != 2 or len(shape) != 2 or not isinstance(block, int) or isinstance(block, bool):
            raise LinnetError(f"{weight}: its quantization state has no 2-d shape and block size")
        out_features, in_features = dims
        if block <= 0 or block % 2 or in_features % block:
            raise LinnetError(f"{weight}: {in_features} inputs do not make blocks of {block}")
        nested_block, offset = state.get("nested_blocksize"), state.get("nested_offset")
        if nested_block is None and offset is None:
            return cls(weight, out_features, in_features, block)
        if (not isinstance(nested_block, int) or isinstance(nested_block, bool) or nested_block <= 0
                or not isinstance(offset, (int, float)) or isinstance(offset, bool)):
            raise LinnetError(f"{weight}: its nested quantization state is incomplete")
        return cls(weight, out_features, in_features, block, nested_block, float(offset))


def _import_nf4(weights_path: str | Path, output: str | Path, config: Mapping[str, object],
                paths: Mapping[str, list[str]], target: torch.device) -> list[str]:
    """`import_quantized` for a bitsandbytes 4-bit NF4 checkpoint: each layer's
    codes repacked low nibble first and its absmax decoded on the GPU
    (`kernels.nf4_repack`), every other tensor copied."""
    from .torch import kernels

    if not config.get("load_in_4bit", config.get("_load_in_4bit", False)):
        raise LinnetError("bitsandbytes checkpoint without `load_in_4bit`: only its 4-bit layers import")
    kind = str(config.get("bnb_4bit_quant_type", "fp4")).lower()
    if kind != "nf4":
        raise LinnetError(f"bitsandbytes 4-bit type {kind!r}: only NF4 imports")
    index = weights.open_checkpoint(weights_path)
    writer = weights.CheckpointWriter()
    consumed: set[str] = set()
    done: list[str] = []
    for name in sorted(n for n in index if _NF4_STATE in n):
        weight, _, layer_kind = name.partition(_NF4_STATE)
        if layer_kind != "nf4":
            raise LinnetError(f"{weight}: bitsandbytes 4-bit type {layer_kind!r}: only NF4 imports")
        layer = _Nf4Layer.parse(weight, index[name])
        codes, absmax = _nf4_layer(layer, index, target, kernels)
        consumed |= {name, weight, *(weight + side for side in _NF4_SIDE)}
        for path in paths.get(weight) or [weight]:
            prefix = siblings(path)
            writer.add(prefix + "weight", "U8", tuple(codes.shape), weights.tensor_bytes(codes))
            writer.add(prefix + "absmax", "F32", tuple(absmax.shape), weights.tensor_bytes(absmax))
            done.append(path)
    if not done:
        raise LinnetError(f"{weights_path}: no bitsandbytes 4-bit layer (`{_NF4_STATE}nf4`)")
    for name, stored in index.items():
        if name not in consumed:
            for path in paths.get(name) or [name]:
                writer.add(path, stored.dtype, stored.shape, stored)
    writer.write(output, {"format": "pt"})
    return done


def _nf4_layer(layer: _Nf4Layer, index: Mapping[str, weights.StoredTensor], target: torch.device,
               kernels) -> tuple[torch.Tensor, torch.Tensor]:
    """One NF4 layer as `Nf4Linear` holds it: (codes [Out, In/2], absmax [Out, In/block])."""
    w = layer.weight
    missing = [w + side for side in (".absmax", ".quant_map") if w + side not in index]
    if w not in index or missing:
        raise LinnetError(f"{w}: the layer lacks {', '.join(missing) or 'its weight'}")
    quant_map = weights.float_tensor(index[w + ".quant_map"], "cpu").numpy().reshape(-1)
    if quant_map.shape != (16,) or not np.allclose(quant_map, NF4, rtol=0, atol=1e-6):
        raise LinnetError(f"{w}: its quantization map is not NF4's")
    stored = index[w]
    if stored.nbytes * 2 != layer.out_features * layer.in_features:
        raise LinnetError(f"{w}: {stored.nbytes} bytes for a [{layer.out_features}, {layer.in_features}] weight")
    packed = weights.tensor_from(stored, torch.uint8, target).reshape(-1)
    scales = layer.out_features * layer.in_features // layer.block
    nested = w + ".nested_absmax" in index
    if nested != bool(layer.nested_block):
        raise LinnetError(f"{w}: its nested quantization state is incomplete")
    if nested:
        if w + ".nested_quant_map" not in index:
            raise LinnetError(f"{w}: `.nested_absmax` without `.nested_quant_map`")
        scale_codes = weights.tensor_from(index[w + ".absmax"], torch.uint8, target).reshape(-1)
        outer = weights.float_tensor(index[w + ".nested_absmax"], target).reshape(-1)
        table = weights.float_tensor(index[w + ".nested_quant_map"], target).reshape(-1)
        if scale_codes.numel() != scales:
            raise LinnetError(f"{w}: {scale_codes.numel()} scales for blocks of {layer.block}")
        return kernels.nf4_repack(packed, scale_codes, layer.out_features, layer.in_features, layer.block,
                                  outer, table, layer.nested_block, layer.offset)
    absmax = weights.float_tensor(index[w + ".absmax"], target).reshape(-1)
    if absmax.numel() != scales:
        raise LinnetError(f"{w}: {absmax.numel()} scales for blocks of {layer.block}")
    return kernels.nf4_repack(packed, absmax, layer.out_features, layer.in_features, layer.block)
