"""The MXFP4 experts kernel (`lnq_mxfp4_experts`) on the GPU against the oracle's
fp64 product of the dequantized experts (`stdlib/quant.linnet:334-356`): the
codes widened exactly, each block's sum scaled, the blocks added in f32, the
sum rounded once to bf16 / f16 -- so within the 16-bit rounding of the result.
Includes gpt-oss-20B's decode shapes (32 experts, top 4, 2880 -> 5760 and
2880 -> 2880), the shared-input form as an expanded view, repeated experts,
and out-of-range expert indices (zero rows)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from linnet_amd.torch import generated, kernels
from oracle import linear

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _case(rows: int, chosen: int, count: int, out: int, width: int, seed: int, dtype: torch.dtype):
    rng = np.random.default_rng(seed)
    blocks = rng.integers(0, 256, (count, out, width // 32, 16)).astype(np.uint8)
    scales = rng.integers(118, 136, (count, out, width // 32)).astype(np.uint8)
    experts = rng.integers(0, count, (rows, chosen)).astype(np.int64)
    x = torch.randn(rows, chosen, width, generator=torch.Generator().manual_seed(seed)).to(dtype)
    return x, blocks, scales, experts


def _check(got: torch.Tensor, want: np.ndarray) -> None:
    g = got.float().cpu().numpy()
    top = float(np.abs(want).max())
    err = float(np.abs(g - want).max())
    print(f"max abs err {err:.3e}, rel to max {err / top:.3e}")
    assert np.all(np.abs(g - want) <= 8e-3 * np.abs(want) + 1e-3 * top)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize(("rows", "chosen", "count", "out", "width"), [
    (1, 4, 32, 5760, 2880), (1, 4, 32, 2880, 2880), (3, 2, 5, 100, 256),
    (2, 3, 4, 40, 8192), (1, 1, 2, 16, 32), (5, 4, 8, 70, 96), (8, 4, 16, 64, 2048),
])
def test_mxfp4_experts_match_the_oracle(rows: int, chosen: int, count: int, out: int, width: int, dtype: torch.dtype) -> None:
    print(f"mxfp4_experts rows={rows} chosen={chosen} E={count} out={out} in={width} {dtype}", flush=True)
    x, blocks, scales, experts = _case(rows, chosen, count, out, width, seed=out + width, dtype=dtype)
    got = kernels.mxfp4_experts(x.to(DEV), torch.from_numpy(blocks).to(DEV), torch.from_numpy(scales).to(DEV),
                                torch.from_numpy(experts).to(DEV))
    assert got.shape == (rows, chosen, out) and got.dtype == dtype
    _check(got, linear.mxfp4_experts_f64(x.float().numpy(), blocks, scales, experts))


def test_shared_input_view_and_generated_helper() -> None:
    """The shared form ([R, 1, In] expanded over the chosen slots, a zero stride)
    equals the same input materialized per slot; the generated helper is the kernel."""
    x, blocks, scales, experts = _case(3, 4, 6, 96, 512, seed=1, dtype=torch.bfloat16)
    b, s, e = torch.from_numpy(blocks).to(DEV), torch.from_numpy(scales).to(DEV), torch.from_numpy(experts).to(DEV)
    one = x[:, :1].to(DEV)
    shared = generated._mxfp4_experts(one.expand(-1, 4, -1), b, s, e)
    dense = kernels.mxfp4_experts(one.expand(-1, 4, -1).contiguous(), b, s, e)
    assert torch.equal(shared, dense)
    _check(shared, linear.mxfp4_experts_f64(one.expand(-1, 4, -1).float().cpu().numpy(), blocks, scales, experts))


def test_out_of_range_experts_give_zero_rows() -> None:
    x, blocks, scales, experts = _case(2, 2, 3, 32, 64, seed=2, dtype=torch.bfloat16)
    experts[0, 1] = -1
    experts[1, 0] = 3
    got = kernels.mxfp4_experts(x.to(DEV), torch.from_numpy(blocks).to(DEV), torch.from_numpy(scales).to(DEV),
                                torch.from_numpy(experts).to(DEV)).float().cpu()
    assert not got[0, 1].any() and not got[1, 0].any()
    ok = experts.copy()
    ok[0, 1] = ok[1, 0] = 0
    want = linear.mxfp4_experts_f64(x.float().numpy(), blocks, scales, ok)
    _check(got[0, :1], want[0, :1])
    _check(got[1, 1:], want[1, 1:])


@pytest.mark.parametrize("rows", [1, 37, 256])
def test_grouped_forms(rows: int) -> None:
    """`mxfp4_linear_experts_shared` and `mxfp4_combine_experts` through the generated
    `_mxfp4_grouped` helper, against the fp64 dense forms of `stdlib/quant.linnet:358-406`."""
    print(f"mxfp4_grouped rows={rows}", flush=True)
    rng = np.random.default_rng(rows)
    count, out, width, chosen = 8, 96, 256, 4
    blocks = rng.integers(0, 256, (count, out, width // 32, 16)).astype(np.uint8)
    scales = rng.integers(118, 136, (count, out, width // 32)).astype(np.uint8)
    experts = rng.integers(0, count, (rows, chosen)).astype(np.int64)
    b, s, e = torch.from_numpy(blocks).to(DEV), torch.from_numpy(scales).to(DEV), torch.from_numpy(experts).to(DEV)
    x = torch.randn(rows, width, generator=torch.Generator().manual_seed(rows)).to(torch.bfloat16)
    shared = generated._mxfp4_grouped(x.to(DEV), b, s, e)
    want = linear.mxfp4_experts_f64(x.float().numpy()[:, None, :].repeat(chosen, 1), blocks, scales, experts)
    _check(shared, want)
    xk = torch.randn(rows, chosen, width, generator=torch.Generator().manual_seed(rows + 1)).to(torch.bfloat16)
    wk = torch.softmax(torch.randn(rows, chosen, generator=torch.Generator().manual_seed(2)), -1).to(torch.bfloat16)
    combined = generated._mxfp4_grouped(xk.to(DEV), b, s, e, wk.to(DEV))
    per_pair = linear.mxfp4_experts_f64(xk.float().numpy(), blocks, scales, experts)
    terms = per_pair * wk.float().numpy()[..., None]
    want_c = terms.sum(1)
    # Each pair's product is rounded to bf16 before the weighted sum (as the
    # reference's helper does), so the bound follows the terms, not their sum.
    got_c = combined.float().cpu().numpy()
    scale_c = np.abs(terms).sum(1)
    assert np.all(np.abs(got_c - want_c) <= 8e-3 * scale_c + 1e-3 * np.abs(want_c).max())

