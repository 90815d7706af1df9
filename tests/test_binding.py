"""The generated-module binding (`linnet_amd.torch.binding`) on a stand-in `linnet`
package: the reference package needs Python >= 3.11 and is not importable here,
so `tests/linnet_standin.py` writes the few modules the binding touches
(`linnet.generated.import_generated`, `linnet.torch.compiled` holding that name,
`linnet.torch.quantized`, `linnet.torch.native.NATIVE`) and a generated-module
text shaped as `src/backend/torch_source.cpp:975-997, 1478-1571` emits it: its
own `_int4_pack` / `_int4_linear`, the 8-bit helpers imported by name, and
`prepare()` / `main()` that call them.

On the CPU the routed helpers are recognised by identity and by refusing CPU
tensors (this package has no CPU path); on the GPU the routed module's output is
compared with the module's own helpers (`test_gpu_binding.py`)."""

from __future__ import annotations

import pytest
import torch

from linnet_amd.errors import LinnetError
from linnet_amd.torch import binding, generated, native, quantized

from tests import linnet_standin


@pytest.fixture()
def standin(tmp_path):
    with linnet_standin.package(tmp_path) as linnet:
        yield linnet
    binding.uninstall()


def test_without_install_the_module_runs_its_own_helpers(standin) -> None:
    module = standin.compile_int4()
    assert module._int4_linear is not generated._int4_linear
    x, params = linnet_standin.int4_inputs("cpu")
    y = module.main(x, *module.prepare(*params), *params)
    assert y.shape == (3, 64)


def test_install_routes_every_later_generated_module(standin) -> None:
    binding.install()
    module = standin.compile_int4()
    assert module._int4_pack is generated._int4_pack
    assert module._int4_linear is generated._int4_linear
    assert module._int4_weight is generated._int4_weight
    assert module._fp8_linear is quantized.fp8_linear and module._fp8_operands is quantized.fp8_operands
    # the module's other globals are untouched
    assert module.torch is torch
    x, params = linnet_standin.int4_inputs("cpu")
    with pytest.raises(LinnetError, match="GPU"):
        module.prepare(*params)


def test_bind_generated_names_what_it_rebinds(standin) -> None:
    module = standin.compile_int4()
    bound = binding.bind_generated(module)
    assert bound == ["_int4_pack", "_int4_weight", "_int4_linear", "_fp8_operands", "_fp8_linear"]


def test_install_updates_the_interpreter_table_and_uninstall_restores_it(standin) -> None:
    table = standin.native_table()
    original = dict(table)
    binding.install()
    for key, entry in native.NATIVE.items():
        assert table[key] is entry
    binding.install()  # idempotent
    binding.uninstall()
    assert table == original
    assert standin.compiled_import() is standin.generated_import()


def test_modules_imported_before_install_keep_their_helpers(standin) -> None:
    before = standin.compile_int4()
    binding.install()
    after = standin.compile_int4()
    assert before._int4_linear is not generated._int4_linear
    assert after._int4_linear is generated._int4_linear
