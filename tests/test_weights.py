"""SafeTensors I/O and bindings of `linnet_amd.weights` (host code, CPU): files it
writes read back through the independent `safetensors` package, files that
package writes read back through it, and the helpers of the checkpoint tools
(`python/linnet/src/linnet/weights.py:74-373`, `quant.py:184-204`)."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch
from safetensors import safe_open
from safetensors.torch import save_file

from linnet_amd import quant, weights
from linnet_amd.errors import LinnetError
from oracle import quant as oracle_quant


def _tensors() -> dict[str, torch.Tensor]:
    g = torch.Generator().manual_seed(0)
    return {
        "a.weight": torch.randn(3, 5, generator=g).to(torch.bfloat16),
        "b.scale": torch.randn(4, generator=g).to(torch.float16),
        "c.qweight": torch.randint(-2**31, 2**31 - 1, (2, 8), generator=g, dtype=torch.int32),
        "d.zero": torch.randint(0, 16, (7,), generator=g, dtype=torch.uint8),
        "e.empty": torch.zeros(0, 4),
    }


_NAMES = {torch.bfloat16: "BF16", torch.float16: "F16", torch.int32: "I32", torch.uint8: "U8", torch.float32: "F32"}


def test_written_files_read_back_through_safetensors(tmp_path: Path) -> None:
    tensors = _tensors()
    entries = [(n, _NAMES[t.dtype], tuple(t.shape), weights.tensor_bytes(t)) for n, t in tensors.items()]
    path = weights.write_checkpoint(tmp_path / "out.safetensors", entries, metadata={"format": "pt"})
    raw = path.read_bytes()
    size = int.from_bytes(raw[:8], "little")
    assert size % 8 == 0
    assert json.loads(raw[8:8 + size])["__metadata__"] == {"format": "pt"}
    with safe_open(str(path), framework="pt") as f:
        assert set(f.keys()) == set(tensors)
        for name, t in tensors.items():
            assert torch.equal(f.get_tensor(name), t)


def test_files_of_safetensors_read_back(tmp_path: Path) -> None:
    tensors = _tensors()
    save_file(tensors, str(tmp_path / "in.safetensors"))
    seen = weights.open_checkpoint(tmp_path / "in.safetensors")
    assert set(seen) == set(tensors)
    for name, t in tensors.items():
        raw = seen[name]
        assert raw.dtype == _NAMES[t.dtype] and raw.shape == tuple(t.shape)
        assert raw.read() == weights.tensor_bytes(t)
        assert torch.equal(weights.tensor_from(raw, t.dtype, "cpu"), t)
    assert torch.equal(weights.float_tensor(seen["a.weight"], "cpu"), tensors["a.weight"].float())


def test_copy_by_location_and_directories(tmp_path: Path) -> None:
    save_file({"x": torch.arange(10, dtype=torch.float32)}, str(tmp_path / "a.safetensors"))
    save_file({"y": torch.arange(6, dtype=torch.int32)}, str(tmp_path / "b.safetensors"))
    index = weights.open_checkpoint(tmp_path)
    assert list(index) == ["x", "y"]
    out = weights.write_checkpoint(
        tmp_path / "sub" / "c.safetensors",
        [(n, loc.dtype, loc.shape, loc) for n, loc in index.items()],
    )
    with safe_open(str(out), framework="pt") as f:
        assert torch.equal(f.get_tensor("x"), torch.arange(10, dtype=torch.float32))
        assert torch.equal(f.get_tensor("y"), torch.arange(6, dtype=torch.int32))
    with pytest.raises(LinnetError):
        weights.checkpoint_files(tmp_path / "missing.safetensors")
    with pytest.raises(LinnetError):
        weights.write_checkpoint(tmp_path / "d.safetensors", [("x", "U8", (1,), b"\0"), ("x", "U8", (1,), b"\0")])


def test_bf16_and_f16_encoding_rounds_to_nearest_even() -> None:
    v = np.random.default_rng(2).standard_normal(4096).astype(np.float32) * 1e3
    got = np.frombuffer(weights.encode_floats(torch.from_numpy(v), "BF16"), dtype=np.uint16)
    assert np.array_equal(got, oracle_quant.to_bf16_bits(v))
    got16 = np.frombuffer(weights.encode_floats(torch.from_numpy(v), "F16"), dtype=np.float16)
    assert np.array_equal(got16, v.astype(np.float16))
    with pytest.raises(LinnetError):
        weights.encode_floats(torch.from_numpy(v), "I8")


def test_bindings_and_prefixes(tmp_path: Path) -> None:
    path = tmp_path / "bindings.json"
    path.write_text(json.dumps({"embed.weight": "model.embed", "head.weight": "model.embed", "p.weight": "q"}))
    mapping = weights.read_bindings(path)
    assert weights.paths_by_tensor(mapping) == {"model.embed": ["embed.weight", "head.weight"], "q": ["p.weight"]}
    assert quant.siblings("weight") == "" and quant.siblings("a.b.weight") == "a.b." and quant.siblings("a") == "a."
    path.write_text("[1, 2]")
    with pytest.raises(LinnetError):
        weights.read_bindings(path)


def test_checkpoint_settings_and_errors(tmp_path: Path) -> None:
    """Host-side checks of the checkpoint tools that run before any GPU work."""
    assert quant._config_number({"w_bit": "4"}, "bits", 8) == 4
    assert quant._config_number({}, "group", 128) == 128
    assert quant._config_number({"q_group_size": 64.0}, "group", 128) == 64
    with pytest.raises(LinnetError):
        quant._config_number({"bits": [4]}, "bits", 4)
    with pytest.raises(LinnetError):
        quant._config_number({"bits": True}, "bits", 4)
    assert quant._Calibrated.read({"quant_method": "GPTQ"}) == quant._Calibrated("gptq", 128, 1)
    assert quant._Calibrated.read({"quant_method": "gptq", "checkpoint_format": "gptq_v2", "group_size": 32}) == \
        quant._Calibrated("gptq", 32, 0)
    assert quant._Calibrated.read({"quant_method": "awq", "w_bit": 4, "q_group_size": 64}) == quant._Calibrated("awq", 64, 0)
    with pytest.raises(LinnetError):
        quant.quantize_checkpoint(tmp_path / "x.safetensors", tmp_path / "y.safetensors", patterns=["*"], bits=3)
    with pytest.raises(LinnetError):
        quant.quantize_checkpoint(tmp_path / "x.safetensors", tmp_path / "y.safetensors", patterns=["*"], dtype="f64")
    save_file({"a": torch.zeros(8)}, str(tmp_path / "x.safetensors"))
    for config in ({"quant_method": "bitsandbytes"}, {"quant_method": "hqq"}, {"quant_method": "gptq", "bits": 8},
                   {"quant_method": "awq", "version": "gemv"}):
        with pytest.raises(LinnetError):
            quant.import_quantized(tmp_path / "x.safetensors", tmp_path / "y.safetensors", config=config)
    with pytest.raises(LinnetError, match="config.json"):
        quant.import_quantized(tmp_path / "x.safetensors", tmp_path / "y.safetensors")


def test_written_bytes_equal_the_safetensors_package(tmp_path: Path) -> None:
    """Given the tensors in the order the `safetensors` package lays them out, the
    file is byte for byte the package's own (compact JSON header, space padding)."""
    from safetensors.torch import save

    tensors = {k: v for k, v in _tensors().items() if v.numel()}
    expected = save(tensors, metadata={"format": "pt"})
    size = int.from_bytes(expected[:8], "little")
    order = [name for name in json.loads(expected[8:8 + size]) if name != "__metadata__"]
    entries = [(n, _NAMES[tensors[n].dtype], tuple(tensors[n].shape), weights.tensor_bytes(tensors[n])) for n in order]
    got = weights.write_checkpoint(tmp_path / "same.safetensors", entries, metadata={"format": "pt"}).read_bytes()
    assert got == expected


def test_input_order_sorts_inputs_by_group() -> None:
    """GPTQ's activation order: the stable sort of g_idx (each group's inputs in
    input order), checked against a brute-force listing; equal-size groups only."""
    rng = np.random.default_rng(6)
    g_idx = (np.arange(96) // 32)[rng.permutation(96)].astype(np.int32)
    order = quant.input_order(g_idx, 32, 96)
    brute = [i for g in range(3) for i in range(96) if g_idx[i] == g]
    assert order.dtype == np.int32 and order.tolist() == brute
    assert quant.input_order(np.arange(64, dtype=np.int32) // 32, 32) is None
    for bad in (np.r_[np.zeros(33), np.ones(31)], np.r_[np.zeros(32), np.full(32, 2)], np.full(64, -1)):
        with pytest.raises(LinnetError):
            quant.input_order(bad.astype(np.int32), 32)
    with pytest.raises(LinnetError):
        quant.input_order(g_idx, 32, 128)
