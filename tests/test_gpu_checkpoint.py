"""The checkpoint tools on the GPU (`linnet_amd.quant`): `import_quantized` for GPTQ
(first and second formats, activation order) and AWQ, and `quantize_checkpoint`
(4 and 8 bits), byte for byte against the CPU oracle's restatement of the
reference (`python/linnet/src/linnet/quant.py:139-369`); the imported layers
multiplying through the int4 kernels as the formats define the weight
(`test_quant_groups.py:228-273`); and the repack kernel alone at a full
Llama-sized shape against the oracle."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch
from safetensors import safe_open
from safetensors.torch import save_file

from linnet_amd import quant
from linnet_amd.errors import LinnetError
from linnet_amd.torch import kernels
from oracle import quant as oq
from tests.formats import calibrated_layer, pack_awq, pack_gptq

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _read(path: Path) -> dict[str, torch.Tensor]:
    with safe_open(str(path), framework="pt") as f:
        return {name: f.get_tensor(name) for name in f.keys()}


CASES = [
    # method, act_order, checkpoint_format, in, out, group
    ("gptq", False, "gptq", 512, 192, 128),
    ("gptq", True, "gptq", 512, 192, 128),
    ("gptq", False, "gptq_v2", 256, 64, 64),
    ("gptq", True, "gptq", 1024, 40, 32),
    ("awq", False, None, 512, 192, 128),
    ("awq", False, None, 384, 72, 64),
]


@pytest.mark.parametrize(("method", "act_order", "fmt", "in_features", "out_features", "group"), CASES)
def test_import_quantized_matches_the_oracle(
    tmp_path: Path, method: str, act_order: bool, fmt: str | None, in_features: int, out_features: int, group: int
) -> None:
    print(f"import_quantized {method} act_order={act_order} format={fmt} {in_features}x{out_features} g{group}", flush=True)
    layer = calibrated_layer(method, act_order, seed=in_features + out_features, in_features=in_features,
                             out_features=out_features, group=group)
    offset = 1 if method == "gptq" and fmt == "gptq" else 0
    if method == "gptq" and offset == 0:
        layer["qweight"], layer["qzeros"] = pack_gptq(layer["q"], layer["zero"], offset=0)
    tensors = {
        "model.proj.qweight": torch.from_numpy(layer["qweight"]),
        "model.proj.qzeros": torch.from_numpy(layer["qzeros"]),
        "model.proj.scales": torch.from_numpy(layer["scale"]),
        "model.norm.weight": torch.arange(8, dtype=torch.bfloat16),
    }
    if method == "gptq":
        tensors["model.proj.g_idx"] = torch.from_numpy(layer["g_idx"])
    save_file(tensors, str(tmp_path / "checkpoint.safetensors"))
    config: dict[str, object] = {"quant_method": method, "bits": 4, "group_size": group}
    if fmt is not None:
        config["checkpoint_format"] = fmt
    quantized = quant.import_quantized(
        tmp_path / "checkpoint.safetensors", tmp_path / "int4.safetensors",
        bindings={"proj.weight": "model.proj.weight", "norm.weight": "model.norm.weight"},
        dtype="f32", config=config,
    )
    assert quantized == ["proj.weight"]
    got = _read(tmp_path / "int4.safetensors")
    packed, zero, order = oq.repack_int4(layer["qweight"], layer["qzeros"], method, group, offset,
                                         layer["g_idx"] if method == "gptq" else None)
    assert set(got) == {"proj.weight", "proj.scale", "proj.zero", "norm.weight"} | ({"proj.order"} if act_order else set())
    assert np.array_equal(got["proj.weight"].numpy(), packed)
    assert np.array_equal(got["proj.zero"].numpy(), zero)
    assert np.array_equal(got["proj.scale"].numpy(), layer["scale"].T.astype(np.float32))
    assert torch.equal(got["norm.weight"], tensors["model.norm.weight"])
    if act_order:
        assert np.array_equal(got["proj.order"].numpy(), order)
    # The imported layer through the HIP kernels: x gathered by order (`take_inputs`),
    # then int4_linear, against x @ W of the format's own definition.
    x = torch.randn(3, in_features, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    taken = x[:, torch.from_numpy(order).long()] if act_order else x
    w = got["proj.weight"].to(DEV)
    y = kernels.int4_linear(taken.to(DEV), w, got["proj.scale"].to(torch.bfloat16).to(DEV), got["proj.zero"].to(DEV))
    want = x.double().numpy() @ layer["weight"].astype(np.float64)
    err = np.abs(y.float().cpu().numpy() - want).max()
    assert err <= 1e-2 * np.abs(want).max(), err


def test_import_quantized_reads_config_json_and_tied_paths(tmp_path: Path) -> None:
    layer = calibrated_layer("awq", False, seed=9, in_features=128, out_features=64, group=128)
    save_file({"m.qweight": torch.from_numpy(layer["qweight"]), "m.qzeros": torch.from_numpy(layer["qzeros"]),
               "m.scales": torch.from_numpy(layer["scale"])}, str(tmp_path / "model.safetensors"))
    (tmp_path / "config.json").write_text('{"quantization_config": {"quant_method": "awq", "w_bit": 4, '
                                          '"q_group_size": 128, "version": "GEMM"}}')
    quantized = quant.import_quantized(tmp_path / "model.safetensors", tmp_path / "out" / "q.safetensors",
                                       bindings={"a.weight": "m.weight", "b.weight": "m.weight"})
    assert quantized == ["a.weight", "b.weight"]
    got = _read(tmp_path / "out" / "q.safetensors")
    assert torch.equal(got["a.weight"], got["b.weight"]) and got["a.scale"].dtype == torch.bfloat16
    packed, zero, _ = oq.repack_int4(layer["qweight"], layer["qzeros"], "awq", 128, 0, None)
    assert np.array_equal(got["b.weight"].numpy(), packed) and np.array_equal(got["a.zero"].numpy(), zero)
    assert np.array_equal(got["a.scale"].view(torch.uint16).numpy(), oq.to_bf16_bits(layer["scale"].T.astype(np.float32)))


def test_import_quantized_rejects_unequal_groups(tmp_path: Path) -> None:
    layer = calibrated_layer("gptq", False, seed=2, in_features=256, out_features=64, group=64)
    g_idx = layer["g_idx"].copy()
    g_idx[0] = 1  # group 1 now holds 65 inputs
    save_file({"p.qweight": torch.from_numpy(layer["qweight"]), "p.qzeros": torch.from_numpy(layer["qzeros"]),
               "p.scales": torch.from_numpy(layer["scale"]), "p.g_idx": torch.from_numpy(g_idx)},
              str(tmp_path / "c.safetensors"))
    with pytest.raises(LinnetError, match="inputs in a group of"):
        quant.import_quantized(tmp_path / "c.safetensors", tmp_path / "o.safetensors",
                               config={"quant_method": "gptq", "bits": 4, "group_size": 64})


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
def test_quantize_checkpoint_matches_the_oracle(tmp_path: Path, bits: int, dtype: str) -> None:
    print(f"quantize_checkpoint bits={bits} dtype={dtype}", flush=True)
    g = torch.Generator().manual_seed(bits)
    tensors = {
        "model.layers.0.mlp.up_proj.weight": (torch.randn(96, 256, generator=g) * 0.02).to(torch.bfloat16),
        "model.layers.0.mlp.down_proj.weight": torch.randn(64, 384, generator=g) * 0.02,
        "model.layers.0.input_layernorm.weight": torch.ones(256, dtype=torch.float16),
        "model.embed_tokens.weight": torch.randn(10, 256, generator=g).to(torch.float16),
    }
    save_file(tensors, str(tmp_path / "model.safetensors"))
    quantized = quant.quantize_checkpoint(tmp_path / "model.safetensors", tmp_path / "q.safetensors",
                                          patterns=["*_proj.weight"], group=128, dtype=dtype, bits=bits)
    assert sorted(quantized) == ["model.layers.0.mlp.down_proj.weight", "model.layers.0.mlp.up_proj.weight"]
    got = _read(tmp_path / "q.safetensors")
    for name in quantized:
        prefix = name.removesuffix("weight")
        w = tensors[name].float().numpy()
        if bits == 4:
            packed, scale, zero = oq.quantize_int4_groups(w, 128)
            assert np.array_equal(got[prefix + "weight"].numpy(), packed)
            assert np.array_equal(got[prefix + "zero"].numpy(), zero)
        else:
            q, scale = oq.quantize_int8_groups(w, 128, dtype)
            assert np.array_equal(got[prefix + "weight"].numpy(), q)
            assert prefix + "zero" not in got
        stored = got[prefix + "scale"]
        assert np.array_equal(stored.float().numpy(), oq.round_to_storage(scale, dtype))
    for name in ("model.layers.0.input_layernorm.weight", "model.embed_tokens.weight"):
        assert torch.equal(got[name], tensors[name])
    with pytest.raises(LinnetError, match="path matched"):
        quant.quantize_checkpoint(tmp_path / "model.safetensors", tmp_path / "n.safetensors", patterns=["nothing*"])


@pytest.mark.parametrize(("method", "act_order"), [("gptq", False), ("gptq", True), ("awq", False)])
def test_repack_kernel_at_a_full_layer(method: str, act_order: bool) -> None:
    """The repack kernel alone at Llama-3.1-8B's up projection (In 4096, Out 14336)."""
    print(f"int4_repack {method} act_order={act_order} 4096x14336", flush=True)
    rng = np.random.default_rng(11)
    in_features, out_features, group = 4096, 14336, 128
    words = rng.integers(-2**31, 2**31 - 1, (in_features // 8, out_features) if method == "gptq"
                         else (in_features, out_features // 8), dtype=np.int64).astype(np.int32)
    qzeros = rng.integers(-2**31, 2**31 - 1, (in_features // group, out_features // 8), dtype=np.int64).astype(np.int32)
    g_idx = np.arange(in_features, dtype=np.int32) // group
    if act_order:
        g_idx = g_idx[rng.permutation(in_features)]
    packed, zero, order = oq.repack_int4(words, qzeros, method, group, 1 if method == "gptq" else 0,
                                         g_idx if method == "gptq" else None)
    order_t = torch.from_numpy(order).to(DEV) if order is not None else None
    got_p, got_z = kernels.int4_repack(torch.from_numpy(words).to(DEV), torch.from_numpy(qzeros).to(DEV), method,
                                       group, 1 if method == "gptq" else 0, order_t)
    assert np.array_equal(got_p.cpu().numpy(), packed)
    assert np.array_equal(got_z.cpu().numpy(), zero)


def test_repack_any_tile_edges() -> None:
    """Shapes that leave partial tiles on both axes (Out % 64, In % 256 nonzero)."""
    rng = np.random.default_rng(12)
    for in_features, out_features, group in ((264, 72, 8), (8, 8, 8), (520, 136, 40)):
        for method in ("gptq", "awq"):
            shape = (in_features // 8, out_features) if method == "gptq" else (in_features, out_features // 8)
            words = rng.integers(-2**31, 2**31 - 1, shape, dtype=np.int64).astype(np.int32)
            qzeros = rng.integers(-2**31, 2**31 - 1, (in_features // group, out_features // 8), dtype=np.int64).astype(np.int32)
            packed, zero, _ = oq.repack_int4(words, qzeros, method, group, 0, None)
            got_p, got_z = kernels.int4_repack(torch.from_numpy(words).to(DEV), torch.from_numpy(qzeros).to(DEV),
                                               method, group, 0)
            assert np.array_equal(got_p.cpu().numpy(), packed), (method, in_features, out_features)
            assert np.array_equal(got_z.cpu().numpy(), zero), (method, in_features, out_features)


def test_repack_refuses_an_order_that_is_not_a_permutation() -> None:
    from linnet_amd.errors import LinnetError

    g = torch.Generator().manual_seed(4)
    words = torch.randint(-2**31, 2**31 - 1, (32, 64), generator=g, dtype=torch.int32).to(DEV)
    qzeros = torch.randint(-2**31, 2**31 - 1, (2, 8), generator=g, dtype=torch.int32).to(DEV)
    good = torch.randperm(256, generator=g).to(torch.int32)
    kernels.int4_repack(words, qzeros, "gptq", 128, 1, good.to(DEV))
    repeated = good.clone()
    repeated[5] = repeated[6]
    out_of_range = good.clone()
    out_of_range[0] = 256
    for bad in (repeated, out_of_range):
        with pytest.raises(LinnetError, match="permutation"):
            kernels.int4_repack(words, qzeros, "gptq", 128, 1, bad.to(DEV))
