"""SafeTensors checkpoints read and written tensor by tensor, and the bindings
that map Linnet parameter paths onto checkpoint tensor names, for the checkpoint
tools of `linnet_amd.quant` (the reference's `python/linnet/src/linnet/weights.py`).

A SafeTensors file is an 8-byte little-endian header length, a JSON header (each
tensor's dtype name, shape and `data_offsets` into the data section, plus an
optional `__metadata__` object of strings), padded with spaces to a multiple of 8
bytes, then the tensors' bytes. Host code: bytes, JSON and PyTorch tensors, no
kernels.
"""

from __future__ import annotations

import json
import struct
from collections.abc import Iterable, Iterator, Mapping
from dataclasses import dataclass
from pathlib import Path

import torch

from .errors import LinnetError

# SafeTensors floating-point dtype names and the torch dtypes that read them
# (`decode_floats`, `weights.py:87-95`).
FLOAT_DTYPES = {"F64": torch.float64, "F32": torch.float32, "F16": torch.float16, "BF16": torch.bfloat16}
# Linnet's scale storage dtypes by their SafeTensors names (`dtypes.py` `DTYPES[...].safetensors`).
STORAGE = {"bf16": "BF16", "f16": "F16", "f32": "F32"}


@dataclass(frozen=True)
class RawTensor:
    """One tensor of a SafeTensors file as bytes (`weights.py:232-239`)."""

    name: str
    dtype: str  # the file's dtype name: BF16, F32, I32, U8, ...
    shape: tuple[int, ...]
    data: bytes


@dataclass(frozen=True)
class TensorLocation:
    """Where a tensor's bytes lie in a file (`weights.py:242-258`), for copying a
    tensor into a new file without holding it."""

    file: Path
    dtype: str
    shape: tuple[int, ...]
    start: int  # absolute byte offsets in the file
    end: int

    @property
    def nbytes(self) -> int:
        return self.end - self.start

    def read(self) -> bytes:
        with self.file.open("rb") as handle:
            handle.seek(self.start)
            data = handle.read(self.nbytes)
        if len(data) != self.nbytes:
            raise LinnetError(f"{self.file} ends inside a tensor")
        return data


def safetensors_files(weights: str | Path) -> list[Path]:
    """One `.safetensors` file, or every one in a directory (`weights.py:38-44`)."""
    path = Path(weights)
    files = sorted(path.glob("*.safetensors")) if path.is_dir() else [path]
    if not files or not all(file.exists() for file in files):
        raise LinnetError(f"no .safetensors files under {weights}")
    return files


def _header(file: Path) -> tuple[dict[str, object], int]:
    """A file's JSON header and the offset where its data section starts."""
    with file.open("rb") as handle:
        head = handle.read(8)
        if len(head) != 8:
            raise LinnetError(f"{file} is not a SafeTensors file (no header length)")
        (size,) = struct.unpack("<Q", head)
        text = handle.read(size)
    if len(text) != size:
        raise LinnetError(f"{file} ends inside its header")
    header = json.loads(text.decode("utf-8"))
    if not isinstance(header, dict):
        raise LinnetError(f"{file}: the header is not a JSON object")
    return header, 8 + size


def safetensors_index(weights: str | Path) -> dict[str, TensorLocation]:
    """Every tensor of a checkpoint by name, from the headers alone (`weights.py:287-304`)."""
    index: dict[str, TensorLocation] = {}
    for file in safetensors_files(weights):
        header, base = _header(file)
        for name, entry in header.items():
            if name == "__metadata__":
                continue
            if not isinstance(entry, dict) or not {"dtype", "shape", "data_offsets"} <= entry.keys():
                raise LinnetError(f"{file}: `{name}` has no dtype, shape and data_offsets")
            start, end = (int(o) for o in entry["data_offsets"])
            if not 0 <= start <= end:
                raise LinnetError(f"{file}: `{name}` has data_offsets {entry['data_offsets']}")
            index[str(name)] = TensorLocation(
                file=file,
                dtype=str(entry["dtype"]),
                shape=tuple(int(d) for d in entry["shape"]),
                start=base + start,
                end=base + end,
            )
    return index


def iter_safetensors(weights: str | Path) -> Iterator[RawTensor]:
    """A checkpoint's tensors one at a time, in header order (`weights.py:307-314`)."""
    for name, location in safetensors_index(weights).items():
        yield RawTensor(name, location.dtype, location.shape, location.read())


Data = bytes | TensorLocation


def write_safetensors(
    path: str | Path,
    tensors: Iterable[tuple[str, str, tuple[int, ...], Data]],
    metadata: Mapping[str, str] | None = None,
) -> Path:
    """Writes `(name, dtype, shape, data)` tensors in the order given, `data` the
    bytes or a `TensorLocation` copied in 64 MiB pieces (`weights.py:325-373`)."""
    entries = list(tensors)
    header: dict[str, object] = {}
    if metadata:
        header["__metadata__"] = {str(k): str(v) for k, v in metadata.items()}
    offset = 0
    for name, dtype, shape, data in entries:
        size = data.nbytes if isinstance(data, TensorLocation) else len(data)
        if name in header:
            raise LinnetError(f"`{name}` is written twice")
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [offset, offset + size]}
        offset += size
    encoded = json.dumps(header, separators=(",", ":")).encode("utf-8")
    encoded += b" " * (-len(encoded) % 8)
    target = Path(path)
    target.parent.mkdir(parents=True, exist_ok=True)
    with target.open("wb") as out:
        out.write(struct.pack("<Q", len(encoded)))
        out.write(encoded)
        for _, _, _, data in entries:
            if isinstance(data, TensorLocation):
                with data.file.open("rb") as source:
                    source.seek(data.start)
                    remaining = data.nbytes
                    while remaining:
                        chunk = source.read(min(remaining, 64 << 20))
                        if not chunk:
                            raise LinnetError(f"{data.file} ends inside a tensor")
                        out.write(chunk)
                        remaining -= len(chunk)
            else:
                out.write(data)
    return target


def read_bindings(bindings: str | Path) -> dict[str, str]:
    """A JSON object of Linnet parameter path -> checkpoint tensor name (`weights.py:108-113`)."""
    loaded = json.loads(Path(bindings).read_text(encoding="utf-8"))
    if not isinstance(loaded, dict):
        raise LinnetError("bindings must be a JSON object mapping parameter paths to tensor names")
    return {str(path): str(name) for path, name in loaded.items()}


def paths_by_tensor(mapping: Mapping[str, str]) -> dict[str, list[str]]:
    """The Linnet paths bound to each checkpoint tensor, in binding order (a tied
    embedding and output head share one; `weights.py:124-130`)."""
    paths: dict[str, list[str]] = {}
    for path, name in mapping.items():
        paths.setdefault(name, []).append(path)
    return paths


def tensor_from(raw: RawTensor, dtype: torch.dtype, device: torch.device | str) -> torch.Tensor:
    """A raw tensor's bytes as a torch tensor of `dtype`, shaped, on `device`."""
    itemsize = torch.empty((), dtype=dtype).element_size()
    count = 1
    for d in raw.shape:
        count *= d
    if len(raw.data) != count * itemsize:
        raise LinnetError(f"`{raw.name}`: {len(raw.data)} bytes for shape {list(raw.shape)} of {dtype}")
    if count == 0:
        return torch.empty(raw.shape, dtype=dtype, device=device)
    host = torch.frombuffer(bytearray(raw.data), dtype=dtype).reshape(raw.shape)
    return host.to(device)


def float_tensor(raw: RawTensor, device: torch.device | str) -> torch.Tensor:
    """A floating-point tensor (F64, F32, F16, BF16) as f32 on `device`: the values of
    `decode_floats` (`weights.py:87-95`; F64 rounded to nearest f32, the others exact)."""
    found = FLOAT_DTYPES.get(raw.dtype)
    if found is None:
        raise LinnetError(f"`{raw.name}` is {raw.dtype}, not a floating-point dtype")
    return tensor_from(raw, found, device).to(torch.float32)


def tensor_bytes(t: torch.Tensor) -> bytes:
    """A tensor's bytes, row-major (any device)."""
    flat = t.detach().contiguous().reshape(-1)
    if flat.numel() == 0:
        return b""
    return flat.cpu().view(torch.uint8).numpy().tobytes()


def encode_floats(values: torch.Tensor, dtype: str) -> bytes:
    """f32 values as the bytes of SafeTensors dtype `dtype` (BF16, F16, F32), each
    rounded to nearest, ties to even (`weights.py:98-105`)."""
    found = FLOAT_DTYPES.get(dtype)
    if found is None or found is torch.float64:
        raise LinnetError(f"{dtype} is not a scale storage dtype")
    return tensor_bytes(values.to(torch.float32).to(found))


__all__ = [
    "FLOAT_DTYPES",
    "STORAGE",
    "RawTensor",
    "TensorLocation",
    "encode_floats",
    "float_tensor",
    "iter_safetensors",
    "paths_by_tensor",
    "read_bindings",
    "safetensors_files",
    "safetensors_index",
    "tensor_bytes",
    "tensor_from",
    "write_safetensors",
]
