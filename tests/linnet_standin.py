"""A stand-in for the few modules of the reference `linnet` package that
`linnet_amd.torch.binding` touches, written into a temporary directory (the
reference package needs Python >= 3.11 and a built compiler, neither here):

- `linnet.generated.import_generated(directory, name, source)`: writes the
  source to a file and imports it as a new module
  (`python/linnet/src/linnet/generated.py:36-49`);
- `linnet.torch.compiled`: binds that function by name at import
  (`torch/compiled.py:54`) and imports generated source through it
  (`:1035-1038`);
- `linnet.torch.quantized` / `linnet.torch.packed`: the names the generated
  module imports (`torch_source.cpp:984-997`), here plain torch;
- `linnet.torch.native.NATIVE`: the interpreter's table (`torch/native.py:556-566`).

The generated text is shaped as the reference emitter writes it: a prelude
defining `_int4_pack` / `_int4_weight` / `_int4_linear` in its own text
(`torch_source.cpp:1478-1571`, here their CPU branches), the 8-bit helpers
imported by name, then `prepare()` / `main()` calling them by global name.
Test infrastructure only."""

from __future__ import annotations

import contextlib
import sys
import textwrap
from pathlib import Path
from types import ModuleType

import torch

FILES = {
    "linnet/__init__.py": "",
    "linnet/generated.py": '''
        import importlib.util, itertools, re, sys
        from pathlib import Path
        _imports = itertools.count()

        def import_generated(directory, name, source):
            path = Path(directory) / f"{name}.py"
            path.write_text(source)
            module_name = "linnet_generated_" + re.sub(r"\\W", "_", f"{name}_{next(_imports)}")
            spec = importlib.util.spec_from_file_location(module_name, path)
            module = importlib.util.module_from_spec(spec)
            sys.modules[module_name] = module
            spec.loader.exec_module(module)
            module.__linnet_path__ = path
            return module
        ''',
    "linnet/torch/__init__.py": "",
    "linnet/torch/compiled.py": '''
        from ..generated import import_generated

        def import_source(directory, source, name):
            return import_generated(directory, name, source)
        ''',
    "linnet/torch/quantized.py": '''
        import torch.nn.functional as F

        def fp8_operands(weight, scale, rounded):
            return ((weight.float() * scale.float().reshape(-1, 1)),)

        def fp8_linear(x, operands, bias):
            y = F.linear(x, operands[0].to(x.dtype))
            return y if bias is None else y + bias
        ''',
    "linnet/torch/packed.py": '''
        def pack4(x, kind):
            raise NotImplementedError

        def unpack4(packed, kind):
            raise NotImplementedError
        ''',
    "linnet/torch/native.py": '''
        def _int4_groups_linear(args):
            raise NotImplementedError

        def _index_select(args):
            raise NotImplementedError

        NATIVE = {"torch.ops.aten._weight_int4pack_mm": _int4_groups_linear, "torch.index_select": _index_select}
        ''',
}

# The generated module: the reference prelude's CPU branches of the int4 helpers,
# the 8-bit imports, and a step calling them by global name.
GENERATED = '''
import torch
import torch.nn.functional as F

def _int4_pack(packed, scale, zero):
    out_features, groups, half = packed.shape
    q = torch.stack([packed & 15, packed >> 4], dim=-1).reshape(out_features, groups, 2 * half)
    weight = (q.float() - zero.float()[..., None]) * scale.float()[..., None]
    return (weight.reshape(out_features, groups * 2 * half).to(scale.dtype),)


def _int4_weight(raw, scale, zero):
    return _int4_pack(raw, scale, zero)[0]


def _int4_linear(x, packed, bias, raw, scale, zero):
    flat = x.reshape(-1, x.shape[-1])
    y = F.linear(flat, packed[0])
    y = y.reshape(*x.shape[:-1], y.shape[-1])
    return y if bias is None else y + bias


from linnet.torch.quantized import fp8_linear as _fp8_linear
from linnet.torch.quantized import fp8_operands as _fp8_operands

PARAMETERS = ["proj.weight", "proj.scale", "proj.zero"]


def prepare(p_weight, p_scale, p_zero):
    return (_int4_pack(p_weight, p_scale, p_zero),)


def main(x, packed, p_weight, p_scale, p_zero):
    return _int4_linear(x, packed, None, p_weight, p_scale, p_zero)
'''


class Standin:
    def __init__(self, root: Path) -> None:
        self.root = root
        self.work = root / "work"
        self.work.mkdir()
        self.count = 0

    def compile_int4(self) -> ModuleType:
        """The generated module imported the way `linnet.torch.compiled` does it."""
        import linnet.torch.compiled as compiled

        self.count += 1
        return compiled.import_source(self.work, GENERATED, f"main_{self.count}")

    def native_table(self) -> dict:
        import linnet.torch.native as native

        return native.NATIVE

    def compiled_import(self):
        import linnet.torch.compiled as compiled

        return compiled.import_generated

    def generated_import(self):
        import linnet.generated as generated

        return generated.import_generated


@contextlib.contextmanager
def package(tmp_path: Path):
    """The stand-in importable as `linnet` for the duration of the block."""
    root = tmp_path / "site"
    for name, text in FILES.items():
        path = root / name
        path.parent.mkdir(parents=True, exist_ok=True)
        path.write_text(textwrap.dedent(text))
    if "linnet" in sys.modules:
        raise RuntimeError("a `linnet` package is already imported")
    sys.path.insert(0, str(root))
    try:
        yield Standin(tmp_path)
    finally:
        sys.path.remove(str(root))
        for name in [n for n in sys.modules if n == "linnet" or n.startswith(("linnet.", "linnet_generated_"))]:
            del sys.modules[name]


def int4_inputs(device: str, rows: int = 3, out_features: int = 64, in_features: int = 256):
    """x [rows, in] bf16 and an int4 g128 layer (packed, scale bf16, zero)."""
    g = torch.Generator().manual_seed(rows)
    x = torch.randn(rows, in_features, generator=g).to(torch.bfloat16)
    packed = torch.randint(0, 256, (out_features, in_features // 128, 64), generator=g, dtype=torch.uint8)
    scale = (torch.rand(out_features, in_features // 128, generator=g) * 0.02 + 0.001).to(torch.bfloat16)
    zero = torch.randint(0, 16, (out_features, in_features // 128), generator=g, dtype=torch.uint8)
    return x.to(device), (packed.to(device), scale.to(device), zero.to(device))
