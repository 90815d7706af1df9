"""SafeTensors checkpoints for the checkpoint tools of `linnet_amd.quant`: files
memory-mapped and read tensor by tensor, new files streamed out, and the
bindings that put Linnet parameter paths on checkpoint tensor names (the
reference's tools read and write the same files, `python/linnet/src/linnet/weights.py`).

The format, from the SafeTensors specification: a little-endian u64 N, N bytes
of a JSON object mapping each tensor's name to `{"dtype", "shape",
"data_offsets": [begin, end]}` (offsets into the data section that follows)
plus an optional `"__metadata__"` object of strings, then the data section.
`CheckpointWriter` writes the header as compact JSON (no spaces), in the order
tensors were added, padded with spaces to a multiple of 8 bytes -- the bytes the
reference's writer and the `safetensors` package produce for the same tensors.
Host code: bytes, JSON and PyTorch tensors, no kernels.
"""

from __future__ import annotations

import itertools
import json
import mmap
import struct
from collections import defaultdict
from collections.abc import Iterable, Mapping
from dataclasses import dataclass, field
from pathlib import Path

import torch

from .errors import LinnetError

# SafeTensors dtype names of the floating-point types the tools read, and the
# torch dtypes that hold them.
FLOAT_DTYPES = {"F64": torch.float64, "F32": torch.float32, "F16": torch.float16, "BF16": torch.bfloat16}
# A Linnet scale dtype's SafeTensors name.
STORAGE = {"bf16": "BF16", "f16": "F16", "f32": "F32"}

_LENGTH = struct.Struct("<Q")


class _Mapping:
    """One checkpoint file, mapped read-only for as long as a tensor of it is alive."""

    def __init__(self, file: Path) -> None:
        self.file = file
        with file.open("rb") as handle:
            size = handle.seek(0, 2)
            self.bytes = mmap.mmap(handle.fileno(), 0, access=mmap.ACCESS_READ) if size else b""

    def __len__(self) -> int:
        return len(self.bytes)


@dataclass(frozen=True)
class StoredTensor:
    """A tensor of a checkpoint file: its name, SafeTensors dtype and shape, and
    where its bytes lie (absolute offsets `begin`..`end` in the mapped file)."""

    name: str
    dtype: str
    shape: tuple[int, ...]
    begin: int
    end: int
    mapping: _Mapping = field(repr=False, compare=False)

    @property
    def nbytes(self) -> int:
        return self.end - self.begin

    def view(self) -> memoryview:
        """The bytes, without a copy (read-only)."""
        return memoryview(self.mapping.bytes)[self.begin : self.end]

    def read(self) -> bytes:
        return bytes(self.view())


def checkpoint_files(weights: str | Path) -> list[Path]:
    """A `.safetensors` file, or a directory's `.safetensors` files in name order."""
    location = Path(weights)
    found = sorted(location.glob("*.safetensors")) if location.is_dir() else [location]
    missing = [str(f) for f in found if not f.is_file()]
    if not found or missing:
        raise LinnetError(f"{weights}: no SafeTensors file to read" + (f" ({', '.join(missing)})" if missing else ""))
    return found


def _tensors_of(file: Path) -> Iterable[StoredTensor]:
    mapped = _Mapping(file)
    if len(mapped) < _LENGTH.size:
        raise LinnetError(f"{file}: shorter than a SafeTensors header length")
    (length,) = _LENGTH.unpack_from(mapped.bytes, 0)
    data = _LENGTH.size + length
    if data > len(mapped):
        raise LinnetError(f"{file}: the header runs past the end of the file")
    header = json.loads(bytes(mapped.bytes[_LENGTH.size : data]).decode("utf-8"))
    if not isinstance(header, dict):
        raise LinnetError(f"{file}: the header is not a JSON object")
    for name, spec in header.items():
        if name == "__metadata__":
            continue
        try:
            begin, end = (int(o) for o in spec["data_offsets"])
            dtype, shape = str(spec["dtype"]), tuple(int(d) for d in spec["shape"])
        except (KeyError, TypeError, ValueError):
            raise LinnetError(f"{file}: tensor `{name}` lacks a dtype, shape or pair of data_offsets") from None
        if begin < 0 or end < begin or data + end > len(mapped):
            raise LinnetError(f"{file}: tensor `{name}` lies outside the data section ({begin}..{end})")
        yield StoredTensor(str(name), dtype, shape, data + begin, data + end, mapped)


def open_checkpoint(weights: str | Path) -> dict[str, StoredTensor]:
    """Every tensor of a checkpoint (a file or a directory of files) by name, in
    the order the headers list them. Only headers are read; a tensor's bytes are
    paged in when used."""
    found: dict[str, StoredTensor] = {}
    for file in checkpoint_files(weights):
        for stored in _tensors_of(file):
            if stored.name in found:
                raise LinnetError(f"`{stored.name}` is in both {found[stored.name].mapping.file} and {file}")
            found[stored.name] = stored
    return found


Data = bytes | bytearray | memoryview | StoredTensor


class CheckpointWriter:
    """Collects tensors, then writes them as one SafeTensors file in the order added."""

    def __init__(self) -> None:
        self._entries: list[tuple[str, str, tuple[int, ...], Data]] = []
        self._names: set[str] = set()

    def add(self, name: str, dtype: str, shape: Iterable[int], data: Data) -> None:
        if name in self._names:
            raise LinnetError(f"`{name}` would be written twice")
        self._names.add(name)
        self._entries.append((name, dtype, tuple(int(d) for d in shape), data))

    def __len__(self) -> int:
        return len(self._entries)

    def write(self, path: str | Path, metadata: Mapping[str, str] | None = None) -> Path:
        sizes = [d.nbytes if isinstance(d, (StoredTensor, memoryview)) else len(d) for _, _, _, d in self._entries]
        ends = list(itertools.accumulate(sizes))
        header: dict[str, object] = {"__metadata__": {str(k): str(v) for k, v in metadata.items()}} if metadata else {}
        for (name, dtype, shape, _), end, size in zip(self._entries, ends, sizes):
            header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [end - size, end]}
        text = json.dumps(header, separators=(",", ":")).encode("utf-8")
        text = text.ljust((len(text) + 7) // 8 * 8, b" ")
        target = Path(path)
        target.parent.mkdir(parents=True, exist_ok=True)
        with target.open("wb") as out:
            out.write(_LENGTH.pack(len(text)))
            out.write(text)
            for *_, data in self._entries:
                # A stored tensor is written straight from its file's mapping.
                out.write(data.view() if isinstance(data, StoredTensor) else data)
        return target


def write_checkpoint(
    path: str | Path,
    tensors: Iterable[tuple[str, str, Iterable[int], Data]],
    metadata: Mapping[str, str] | None = None,
) -> Path:
    """Writes `(name, dtype, shape, data)` tensors, in order, as one SafeTensors file."""
    writer = CheckpointWriter()
    for name, dtype, shape, data in tensors:
        writer.add(name, dtype, shape, data)
    return writer.write(path, metadata)


def read_bindings(bindings: str | Path) -> dict[str, str]:
    """A JSON file of `{Linnet parameter path: checkpoint tensor name}`."""
    loaded = json.loads(Path(bindings).read_text(encoding="utf-8"))
    if not isinstance(loaded, dict):
        raise LinnetError(f"{bindings}: bindings are a JSON object of parameter paths to tensor names")
    return {str(k): str(v) for k, v in loaded.items()}


def paths_by_tensor(mapping: Mapping[str, str]) -> dict[str, list[str]]:
    """Inverts bindings: each checkpoint tensor's paths, in binding order (a tied
    embedding and output head name the same tensor)."""
    inverse: defaultdict[str, list[str]] = defaultdict(list)
    for path, name in mapping.items():
        inverse[name].append(path)
    return dict(inverse)


def tensor_from(stored: StoredTensor, dtype: torch.dtype, device: torch.device | str) -> torch.Tensor:
    """A stored tensor's bytes read as `dtype`, in its shape, on `device`."""
    count = 1
    for d in stored.shape:
        count *= d
    width = torch.empty((), dtype=dtype).element_size()
    if stored.nbytes != count * width:
        raise LinnetError(f"`{stored.name}`: {stored.nbytes} bytes cannot hold {list(stored.shape)} of {dtype}")
    if not count:
        return torch.empty(stored.shape, dtype=dtype, device=device)
    host = torch.frombuffer(bytearray(stored.view()), dtype=dtype)
    return host.reshape(stored.shape).to(device)


def float_tensor(stored: StoredTensor, device: torch.device | str) -> torch.Tensor:
    """A floating-point tensor (F64, F32, F16 or BF16) widened or rounded to f32
    on `device` (round to nearest from F64; the others exactly)."""
    if stored.dtype not in FLOAT_DTYPES:
        raise LinnetError(f"`{stored.name}` holds {stored.dtype}, not floating-point values")
    return tensor_from(stored, FLOAT_DTYPES[stored.dtype], device).to(torch.float32)


def tensor_bytes(t: torch.Tensor) -> bytes:
    """A tensor's elements as bytes in row-major order, from any device."""
    flat = t.detach().reshape(-1).contiguous()
    return flat.cpu().view(torch.uint8).numpy().tobytes() if flat.numel() else b""


def encode_floats(values: torch.Tensor, dtype: str) -> bytes:
    """Values as SafeTensors dtype `dtype` (BF16, F16 or F32), each rounded to
    nearest with ties to even."""
    if dtype not in ("BF16", "F16", "F32"):
        raise LinnetError(f"{dtype} is not a dtype scales are stored in")
    return tensor_bytes(values.to(torch.float32).to(FLOAT_DTYPES[dtype]))


__all__ = [
    "FLOAT_DTYPES",
    "STORAGE",
    "CheckpointWriter",
    "StoredTensor",
    "checkpoint_files",
    "encode_floats",
    "float_tensor",
    "open_checkpoint",
    "paths_by_tensor",
    "read_bindings",
    "tensor_bytes",
    "tensor_from",
    "write_checkpoint",
]
