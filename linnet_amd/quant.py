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

Entry = tuple[str, str, tuple[int, ...], "bytes | weights.TensorLocation"]


def _paths_of(bindings: str | Path | Mapping[str, str] | None) -> dict[str, list[str]]:
    """Checkpoint name -> the Linnet paths bound to it (`quant.py:184-195`)."""
    if bindings is None:
        mapping: dict[str, str] = {}
    elif isinstance(bindings, Mapping):
        mapping = {str(k): str(v) for k, v in bindings.items()}
    else:
        mapping = weights.read_bindings(bindings)
    return weights.paths_by_tensor(mapping)


def _prefix(path: str) -> str:
    """What names a weight's siblings: `proj.` for `proj.weight`, nothing for a
    root block's own `weight` (`quant.py:198-204`)."""
    if path == "weight":
        return ""
    return path.removesuffix("weight") if path.endswith(".weight") else path + "."


def _storage(dtype: str) -> str:
    if dtype not in weights.STORAGE:
        raise LinnetError(f"scales are stored as bf16, f16, or f32, not {dtype}")
    return weights.STORAGE[dtype]


def _scale_tensor(prefix: str, scale: torch.Tensor, dtype: str) -> Entry:
    stored = _storage(dtype)
    return (prefix + "scale", stored, tuple(scale.shape), weights.encode_floats(scale, stored))


def _int4_tensors(prefix: str, packed: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor, dtype: str) -> list[Entry]:
    """`.weight` (U8 `[Out, In/group, group/2]`), `.scale` in `dtype`, `.zero` (U8)
    (`quant.py:207-219`)."""
    _storage(dtype)
    return [
        (prefix + "weight", "U8", tuple(packed.shape), weights.tensor_bytes(packed)),
        _scale_tensor(prefix, scale, dtype),
        (prefix + "zero", "U8", tuple(zero.shape), weights.tensor_bytes(zero)),
    ]


def _gpu(device: torch.device | str | None) -> torch.device:
    if not torch.cuda.is_available():
        raise LinnetError("linnet_amd's checkpoint tools quantize and repack on the GPU; no GPU is available")
    return torch.device(device if device is not None else "cuda")


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
    """Writes `output` with every tensor of the checkpoint `weights_path` under its
    Linnet path, the `.weight` tensors whose path matches one of `patterns`
    quantized on the GPU: into `.weight`, `.scale` (in `dtype`) and `.zero` for
    `Int4GroupLinear` (`bits` 4), or `.weight` and `.scale` for `Int8GroupLinear`
    (`bits` 8); every other tensor copied as it is. Returns the quantized paths.
    The reference's `quantize_checkpoint` (`quant.py:139-181`), with its rounding
    bit for bit (the kernels of `quantize_int4_groups` / `quantize_int8_groups`)."""
    if bits not in (4, 8):
        raise LinnetError(f"weights are quantized to 4 or 8 bits, not {bits}")
    _storage(dtype)
    target = _gpu(device)
    paths_of = _paths_of(bindings)
    chosen = list(patterns)
    out: list[Entry] = []
    quantized: list[str] = []
    for tensor in weights.iter_safetensors(weights_path):
        for path in paths_of.get(tensor.name, [tensor.name]):
            if path.endswith(".weight") and any(fnmatch.fnmatchcase(path, p) for p in chosen):
                values = weights.float_tensor(tensor, target)
                prefix = _prefix(path)
                if bits == 8:
                    q, scale = kernels.quantize_int8(values, group, dtype)
                    out.append((prefix + "weight", "I8", tuple(q.shape), weights.tensor_bytes(q)))
                    out.append(_scale_tensor(prefix, scale, dtype))
                else:
                    packed, scale, zero = kernels.quantize_int4(values, group)
                    out += _int4_tensors(prefix, packed, scale, zero, dtype)
                quantized.append(path)
            else:
                out.append((path, tensor.dtype, tensor.shape, tensor.data))
    if not quantized:
        raise LinnetError("no weight matched " + ", ".join(chosen))
    weights.write_safetensors(output, out, metadata={"format": "pt"})
    return quantized


def _setting(config: Mapping[str, object], key: str, alias: str, default: int) -> int:
    """`config[key]` (or its AWQ name `alias`, or `default`) as an integer (`quant.py:251-256`)."""
    value = config.get(key, config.get(alias, default))
    if isinstance(value, bool) or not isinstance(value, (int, float, str)):
        raise LinnetError(f"the quantization_config's `{key}` is {value!r}, not a number")
    try:
        return int(value)
    except ValueError:
        raise LinnetError(f"the quantization_config's `{key}` is {value!r}, not a number") from None


def import_quantized(
    weights_path: str | Path,
    output: str | Path,
    *,
    bindings: str | Path | Mapping[str, str] | None = None,
    dtype: str = "bf16",
    config: Mapping[str, object] | None = None,
    device: torch.device | str | None = None,
) -> list[str]:
    """Writes `output` with a 4-bit GPTQ or AWQ checkpoint's quantized linear layers
    repacked on the GPU for `Int4GroupLinear` (`.weight`, `.scale` in `dtype`,
    `.zero`, and `.order` for a GPTQ layer in activation order) and every other
    tensor as it is, all under Linnet paths. `config` is the checkpoint's
    `quantization_config` (by default read from the `config.json` beside
    `weights_path`). Returns the quantized paths, as `.weight`. The reference's
    `import_quantized` (`quant.py:255-354`) for GPTQ and AWQ; its bitsandbytes NF4
    import (`Nf4Linear`) is not part of this build and raises."""
    if config is None:
        location = Path(weights_path)
        directory = location if location.is_dir() else location.parent
        try:
            document = json.loads((directory / "config.json").read_text(encoding="utf-8"))
        except FileNotFoundError:
            raise LinnetError(f"no config.json beside {weights_path}; pass `config`") from None
        config = document.get("quantization_config") if isinstance(document, dict) else None
        if not isinstance(config, Mapping):
            raise LinnetError(f"{directory / 'config.json'} has no quantization_config")
    method = str(config.get("quant_method", "")).lower()
    if method == "bitsandbytes":
        raise LinnetError("bitsandbytes NF4 checkpoints (Nf4Linear) are not imported by linnet_amd")
    if method not in ("gptq", "awq"):
        raise LinnetError(f"a {method or 'unnamed'} checkpoint is not GPTQ, AWQ or bitsandbytes")
    if _setting(config, "bits", "w_bit", 4) != 4:
        raise LinnetError("only 4-bit GPTQ and AWQ checkpoints repack into Int4GroupLinear")
    if method == "awq" and str(config.get("version", "gemm")).lower() != "gemm":
        raise LinnetError(f"AWQ's {config.get('version')} packing is not read; GEMM's is")
    group = _setting(config, "group_size", "q_group_size", 128)
    _storage(dtype)
    # GPTQ's first checkpoint format stores each zero point less one.
    zero_offset = 1 if method == "gptq" and config.get("checkpoint_format", "gptq") == "gptq" else 0
    target = _gpu(device)
    index = weights.safetensors_index(weights_path)
    paths_of = _paths_of(bindings)
    out: list[Entry] = []
    quantized: list[str] = []
    parts = (".qweight", ".qzeros", ".scales", ".g_idx")
    layers = sorted(name.removesuffix(".qweight") for name in index if name.endswith(".qweight"))
    taken = {layer + part for layer in layers for part in parts}

    def load(name: str, dtype_: torch.dtype) -> torch.Tensor:
        location = index[name]
        raw = weights.RawTensor(name, location.dtype, location.shape, location.read())
        return weights.tensor_from(raw, dtype_, target)

    for layer in layers:
        for part in (".qzeros", ".scales"):
            if layer + part not in index:
                raise LinnetError(f"{layer}: no `{part[1:]}` beside `qweight`")
        qweight = load(layer + ".qweight", torch.int32)
        qzeros = load(layer + ".qzeros", torch.int32)
        stored = index[layer + ".scales"]
        scales = weights.float_tensor(weights.RawTensor(layer + ".scales", stored.dtype, stored.shape, stored.read()), target)
        if qweight.dim() != 2 or qzeros.dim() != 2 or scales.dim() != 2:
            raise LinnetError(f"{layer}: qweight, qzeros and scales are 2-D")
        if method == "gptq":
            in_features, out_features = qweight.shape[0] * 8, qweight.shape[1]
        else:
            in_features, out_features = qweight.shape[0], qweight.shape[1] * 8
        size = in_features if group <= 0 else group
        groups = in_features // size if in_features % size == 0 else -1
        if groups < 0 or tuple(qzeros.shape) != (groups, out_features // 8) or tuple(scales.shape) != (groups, out_features):
            raise LinnetError(f"{layer}: {in_features} inputs do not make groups of {size}")
        order: np.ndarray | None = None
        if method == "gptq" and layer + ".g_idx" in index:
            ids = load(layer + ".g_idx", torch.int32).cpu().numpy().reshape(-1)
            group_of = np.arange(in_features) // size
            if not np.array_equal(ids, group_of):
                # Activation order: the groups hold inputs in another order. Taken
                # in that order, each group is contiguous (`quant.py:314-325`).
                order = np.argsort(ids, kind="stable").astype(np.int32)
                if not np.array_equal(ids[order], group_of):
                    raise LinnetError(f"{layer}: its groups are not all the same size")
        order_t = torch.from_numpy(order).to(target) if order is not None else None
        packed, zero = kernels.int4_repack(qweight, qzeros, method, size, zero_offset, order_t)
        scale = scales.t().contiguous()
        weight_name = layer + ".weight"
        for path in paths_of.get(weight_name, [weight_name]):
            prefix = _prefix(path)
            out += _int4_tensors(prefix, packed, scale, zero, dtype)
            if order is not None:
                out.append((prefix + "order", "I32", (in_features,), order.tobytes()))
            quantized.append(path)
    if not quantized:
        raise LinnetError(f"no {method.upper()} layer (`.qweight`) in {weights_path}")
    # Every other tensor as it is, under its paths (`quant.py:357-369`).
    for name, location in index.items():
        if name in taken:
            continue
        for path in paths_of.get(name, [name]):
            out.append((path, location.dtype, location.shape, location))
    weights.write_safetensors(output, out, metadata={"format": "pt"})
    return quantized


__all__ = [
    "FEW_ROWS",
    "TILED_ROWS",
    "dequantize_int4_groups",
    "dequantize_int8_groups",
    "import_quantized",
    "pack_int4_groups",
    "quantize_checkpoint",
    "quantize_int4_groups",
    "quantize_int8_groups",
]
