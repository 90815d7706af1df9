"""`std.quant::take_inputs` and the int4 product in GPTQ's activation order, on the GPU.

- `kernels.take_inputs` (the HIP gather) equals `x[..., order]` bit for bit, with
  repeated indices, at any number of rows; an index outside [0, N) reads 0;
- an activation-order GPTQ layer, repacked by the HIP kernel with its order and
  multiplied by `int4_linear(..., order=)` -- one row through the gather fused into
  the one-token GEMV (In 4096, and In 14336 on the slices kernel), more rows gather
  first -- is within `1e-2 * max|y|` of `x @ W` in f64, W built from the GPTQ words
  by the format's definition (`(q - zero[g_idx[i]]) * scale[g_idx[i]]`,
  `stdlib/quant.linnet:163-174`); max abs / rel errors are printed;
- the fused one-row product equals, bit for bit, the unfused GEMV on the taken x.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from linnet_amd.torch import kernels
from tests.formats import calibrated_layer

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize(("rows", "n"), [(1, 4096), (3, 14336), (7, 100), (2, 1)])
def test_take_inputs_matches_index_select(dtype: torch.dtype, rows: int, n: int) -> None:
    g = torch.Generator().manual_seed(rows * n)
    x = torch.randn(rows, n, generator=g).to(dtype)
    for order in (torch.randperm(n, generator=g), torch.randint(0, n, (n,), generator=g)):
        got = kernels.take_inputs(x.to(DEV), order.to(torch.int32).to(DEV)).cpu()
        assert torch.equal(got, x.index_select(-1, order))


def test_take_inputs_keeps_leading_axes_and_reads_zero_outside() -> None:
    x = torch.randn(2, 3, 8, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    order = torch.tensor([7, 0, -1, 8, 3, 3, 1 << 30, 2], dtype=torch.int32)
    got = kernels.take_inputs(x.to(DEV), order.to(DEV)).cpu()
    assert got.shape == x.shape
    inside = (order >= 0) & (order < 8)
    assert torch.equal(got[..., inside], x[..., order[inside].long()])
    assert bool((got[..., ~inside] == 0).all())


def _ordered_layer(in_features: int, out_features: int, dtype: torch.dtype, seed: int):
    """An activation-order GPTQ layer (group 128, first format) as the package
    imports it: the HIP repack of its words with the order that sorts g_idx (each
    group's inputs contiguous), scales [Out, Groups] in `dtype`; and the [In, Out]
    weight of the format's definition."""
    layer = calibrated_layer("gptq", True, seed=seed, in_features=in_features, out_features=out_features, group=128)
    order = np.argsort(layer["g_idx"], kind="stable").astype(np.int32)
    order_t = torch.from_numpy(order).to(DEV)
    packed, zero = kernels.int4_repack(torch.from_numpy(layer["qweight"]).to(DEV),
                                       torch.from_numpy(layer["qzeros"]).to(DEV), "gptq", 128, 1, order_t)
    scale = torch.from_numpy(np.ascontiguousarray(layer["scale"].T)).to(dtype).to(DEV)
    # The format's weight with the scale as the kernel reads it (f16 exactly; bf16 rounded).
    weight = (layer["q"] - layer["zero"][layer["g_idx"]]).astype(np.float64)
    weight *= scale.double().cpu().numpy().T[layer["g_idx"]]
    return packed, scale, zero, order_t, weight


@pytest.mark.parametrize(("in_features", "out_features"), [(4096, 4096), (14336, 4096), (1024, 512)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_activation_order_layer_matches_the_format(in_features: int, out_features: int, dtype: torch.dtype) -> None:
    print(f"activation order {in_features}x{out_features} {dtype}", flush=True)
    packed, scale, zero, order, weight = _ordered_layer(in_features, out_features, dtype, in_features + out_features)
    for rows in (1, 4, 16, 100):
        x = torch.randn(rows, in_features, generator=torch.Generator().manual_seed(rows)).to(dtype)
        y = kernels.int4_linear(x.to(DEV), packed, scale, zero, order=order)
        want = x.double().numpy() @ weight
        err = np.abs(y.double().cpu().numpy() - want)
        top = np.abs(want).max()
        print(f"  rows {rows} ({kernels.int4_linear_plan(rows, in_features, out_features, 128, dtype)}): "
              f"max abs err {err.max():.3e}, rel to max|y| {err.max() / top:.3e}")
        assert err.max() <= 1e-2 * top
        if rows == 1:
            unfused = kernels.int4_linear(kernels.take_inputs(x.to(DEV), order), packed, scale, zero)
            assert torch.equal(y, unfused)


def test_order_and_kernel_choices_agree() -> None:
    """Every kernel a caller may force takes an order (gathering first where the
    gather is not fused) and agrees with the automatic choice."""
    packed, scale, zero, order, weight = _ordered_layer(1024, 512, torch.float16, 9)
    x = torch.randn(1, 1024, generator=torch.Generator().manual_seed(2)).to(torch.float16).to(DEV)
    auto = kernels.int4_linear(x, packed, scale, zero, order=order)
    for kernel in ("gemv", "skinny", "tiled128"):
        forced = kernels.int4_linear(x, packed, scale, zero, order=order, kernel=kernel)
        err = (forced.float() - auto.float()).abs().max().item()
        assert err <= 1e-2 * auto.float().abs().max().item(), (kernel, err)
