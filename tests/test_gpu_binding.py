"""The generated-module binding on the GPU: a module imported after
`binding.install()` (the stand-in `linnet` of `tests/linnet_standin.py`) runs the
HIP helpers, and its step's output matches the same module text running its own
helpers (the reference prelude's dequantize-then-`F.linear` branch) within the
reference's int4 bound, `1e-2 * max|y|` (`python/linnet/tests/test_quant_groups.py:194-195`)."""

from __future__ import annotations

import pytest
import torch

from linnet_amd.torch import binding, generated
from tests import linnet_standin

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows", [1, 3, 100])
def test_routed_module_matches_its_own_helpers(tmp_path, rows: int) -> None:
    with linnet_standin.package(tmp_path) as standin:
        try:
            own = standin.compile_int4()
            binding.install()
            routed = standin.compile_int4()
            assert routed._int4_linear is generated._int4_linear
            x, params = linnet_standin.int4_inputs("cuda", rows=rows, out_features=200, in_features=512)
            want = own.main(x, *own.prepare(*params), *params).float()
            got = routed.main(x, *routed.prepare(*params), *params).float()
        finally:
            binding.uninstall()
    err = (got - want).abs().max().item()
    top = want.abs().max().item()
    print(f"rows {rows}: routed vs own helpers max abs err {err:.3e}, rel {err / top:.3e}")
    assert got.shape == want.shape and err <= 1e-2 * top
