"""Routes Linnet's generated PyTorch modules and its interpreter to the HIP kernels.

The reference's generated module carries its quantized-linear helpers as module
globals that `prepare()` and `main()` look up when they run:

- `_int4_pack`, `_int4_weight`, `_int4_linear`, defined in the module's own
  text (`src/backend/torch_source.cpp:978-980, 1478-1571`);
- `_mxfp4_experts` and `_mxfp4_grouped`, defined the same way
  (`torch_source.cpp:1579-1600, 1705-1735`);
- `_{kind}_operands` / `_{kind}_linear`, imported from `linnet.torch.quantized`
  (`torch_source.cpp:987-997`), and `_pack4` / `_unpack4` from
  `linnet.torch.packed` (`torch_source.cpp:984-986`).

`bind_generated(module)` rebinds each of those globals the module has to this
package's function of the same contract, so every later call of the module's
`prepare()` / `main()` runs the HIP kernels; nothing else in the module changes.
`install()` makes that happen for every module Linnet imports from then on: it
wraps `linnet.generated.import_generated` (`python/linnet/src/linnet/generated.py:36-49`,
also bound by name in `linnet.torch.compiled`, `torch/compiled.py:54, 1035-1038`)
and puts the HIP entries into the interpreter's `NATIVE` table
(`torch/native.py:556-566`). `uninstall()` restores what `install()` replaced.
"""

from __future__ import annotations

import importlib
import sys
from collections.abc import Callable
from types import ModuleType
from typing import Any

from . import generated, native, packed, quantized

# The 8-bit layer kinds whose helpers a generated module imports.
_EIGHT_BIT_KINDS = ("fp8", "fp8_block", "int8", "int8_group")


def helpers() -> dict[str, Callable[..., Any]]:
    """The generated-module globals this package provides, by name."""
    table: dict[str, Callable[..., Any]] = {
        "_int4_pack": generated._int4_pack,
        "_int4_weight": generated._int4_weight,
        "_int4_linear": generated._int4_linear,
        "_mxfp4_experts": generated._mxfp4_experts,
        "_mxfp4_grouped": generated._mxfp4_grouped,
        "_pack4": packed.pack4,
        "_unpack4": packed.unpack4,
    }
    for kind in _EIGHT_BIT_KINDS:
        table[f"_{kind}_operands"] = getattr(quantized, f"{kind}_operands")
        table[f"_{kind}_linear"] = getattr(quantized, f"{kind}_linear")
    return table


def bind_generated(module: ModuleType) -> list[str]:
    """Rebinds the quantized helpers `module` has (and only those) to the HIP
    ones; returns the names rebound, in order."""
    bound = []
    for name, function in helpers().items():
        if hasattr(module, name):
            setattr(module, name, function)
            bound.append(name)
    return bound


# What install() replaced: (module, attribute) -> original value, and the
# NATIVE entries it overwrote.
_saved: dict[tuple[str, str], Any] = {}
_saved_native: dict[str, Any] = {}


def _wrap(import_generated: Callable[..., ModuleType]) -> Callable[..., ModuleType]:
    def import_and_bind(*args: Any, **kwargs: Any) -> ModuleType:
        module = import_generated(*args, **kwargs)
        bind_generated(module)
        return module

    import_and_bind.__wrapped__ = import_generated  # type: ignore[attr-defined]
    import_and_bind.__doc__ = import_generated.__doc__
    return import_and_bind


def install(linnet_package: str = "linnet") -> None:
    """Routes every generated module Linnet imports from now on, and its
    interpreter's quantized entries, to the HIP kernels. Idempotent."""
    if _saved:
        return
    generated_module = importlib.import_module(f"{linnet_package}.generated")
    original = generated_module.import_generated
    wrapped = _wrap(original)
    # Modules that bound the name at their own import hold it too: imported
    # first, so that they take the original, then rebound with it.
    holders = [generated_module]
    for name in (f"{linnet_package}.torch.compiled",):
        module = sys.modules.get(name) or _try_import(name)
        if module is not None and getattr(module, "import_generated", None) is original:
            holders.append(module)
    for module in holders:
        _saved[(module.__name__, "import_generated")] = original
        module.import_generated = wrapped
    interpreter = _try_import(f"{linnet_package}.torch.native")
    if interpreter is not None and hasattr(interpreter, "NATIVE"):
        for key, entry in native.NATIVE.items():
            if key in interpreter.NATIVE:
                _saved_native[key] = interpreter.NATIVE[key]
            interpreter.NATIVE[key] = entry
        _saved[(interpreter.__name__, "NATIVE")] = None


def uninstall() -> None:
    """Undoes install(): modules imported meanwhile keep the HIP helpers."""
    for (name, attribute), value in list(_saved.items()):
        module = sys.modules.get(name)
        if module is None:
            continue
        if attribute == "NATIVE":
            for key in native.NATIVE:
                if key in _saved_native:
                    module.NATIVE[key] = _saved_native[key]
                else:
                    module.NATIVE.pop(key, None)
        else:
            setattr(module, attribute, value)
    _saved.clear()
    _saved_native.clear()


def _try_import(name: str) -> ModuleType | None:
    try:
        return importlib.import_module(name)
    except ImportError:
        return None


__all__ = ["bind_generated", "helpers", "install", "uninstall"]
