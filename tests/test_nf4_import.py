"""Host checks of the bitsandbytes NF4 importer (`linnet_amd.quant`): the
configuration gate, the saved state's decoding and the quant-map test. The
repack itself runs on the GPU (`test_gpu_nf4.py`)."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from linnet_amd import quant as lquant
from linnet_amd import weights
from linnet_amd.errors import LinnetError


def _stored(tmp_path: Path, tensors: dict[str, torch.Tensor]) -> dict[str, weights.StoredTensor]:
    save_file(tensors, str(tmp_path / "t.safetensors"))
    return weights.open_checkpoint(tmp_path / "t.safetensors")


def _state_bytes(state: object) -> torch.Tensor:
    return torch.from_numpy(np.frombuffer(json.dumps(state).encode("utf-8"), dtype=np.uint8).copy())


def test_config_gate() -> None:
    assert lquant._four_bit_codes({"load_in_4bit": True, "bnb_4bit_quant_type": "NF4"}) == "nf4"
    assert lquant._four_bit_codes({"_load_in_4bit": True, "bnb_4bit_quant_type": "nf4"}) == "nf4"
    with pytest.raises(LinnetError, match="load_in_4bit"):
        lquant._four_bit_codes({"load_in_8bit": True})
    with pytest.raises(LinnetError, match="'fp4' codes"):
        lquant._four_bit_codes({"load_in_4bit": True})  # bitsandbytes' default code type


def test_state_decoding(tmp_path: Path) -> None:
    index = _stored(tmp_path, {
        "plain": _state_bytes({"shape": [8, 128], "blocksize": 64, "quant_type": "nf4"}),
        "nested": _state_bytes({"shape": [8, 128], "blocksize": 64, "nested_blocksize": 256, "nested_offset": 0.5}),
        "list": _state_bytes([1, 2]),
        "noblock": _state_bytes({"shape": [8, 128]}),
        "ragged": _state_bytes({"shape": [8, 100], "blocksize": 64}),
        "half_nested": _state_bytes({"shape": [8, 128], "blocksize": 64, "nested_blocksize": 256}),
        "flag_shape": _state_bytes({"shape": [True, 128], "blocksize": 64}),
        "not_json": torch.tensor([0xFF, 0x00, 0x7B], dtype=torch.uint8),
    })
    plain = lquant._Nf4State.decode(index["plain"], "w")
    assert (plain.out_features, plain.in_features, plain.block, plain.nested_block, plain.blocks) == (8, 128, 64, 0, 16)
    assert set(plain.tensors("w")) == {"codes", "absmax", "values"}
    nested = lquant._Nf4State.decode(index["nested"], "w")
    assert (nested.nested_block, nested.nested_offset) == (256, 0.5)
    assert nested.tensors("w")["table"] == "w.nested_quant_map"
    for name, message in (("list", "not an object"), ("noblock", "no blocksize"), ("ragged", "whole blocks"),
                          ("half_nested", "both nested_blocksize"), ("flag_shape", "out_features, in_features"),
                          ("not_json", "does not decode")):
        with pytest.raises(LinnetError, match=message):
            lquant._Nf4State.decode(index[name], "w")


def test_quant_map_check(tmp_path: Path) -> None:
    nf4 = torch.from_numpy(lquant.NF4.copy())
    shuffled = nf4.flip(0)
    nudged = nf4.clone()
    nudged[3] = torch.nextafter(nudged[3], torch.tensor(0.0))
    index = _stored(tmp_path, {"f32": nf4, "bf16": nf4.to(torch.bfloat16), "f16": nf4.to(torch.float16),
                               "f64": nf4.to(torch.float64), "shuffled": shuffled, "nudged": nudged,
                               "short": nf4[:15].clone(), "codes": torch.arange(16, dtype=torch.uint8)})
    for name in ("f32", "bf16", "f16", "f64"):
        assert lquant._holds_nf4(index[name]), name
    for name in ("shuffled", "nudged", "short", "codes"):
        assert not lquant._holds_nf4(index[name]), name
