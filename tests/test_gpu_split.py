"""The 32-row GEMV with K split over workgroups (`LNQ_KERNEL_SPLIT`,
`lnq_int4_linear_ws`), on the GPU: within `1e-2 * max|y|` of the f64 product
with the exactly dequantized weight (the reference's bound for its int4 kernel,
`python/linnet/tests/test_quant_groups.py:194-195`), the chunks added in a fixed
order (two calls give the same bits), the workspace contract of the C ABI, and
agreement with the unsplit kernels at the decode batch's full sizes."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from linnet_amd import _lib
from linnet_amd.errors import LinnetError
from linnet_amd.torch import kernels
from oracle import linear

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _layer(out: int, width: int, group: int, seed: int, dtype: torch.dtype = torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    packed = torch.randint(0, 256, (out, width // group, group // 2), generator=g, dtype=torch.uint8)
    scale = (torch.rand(out, width // group, generator=g) * 0.02 + 0.001).to(dtype)
    zero = torch.randint(0, 16, (out, width // group), generator=g, dtype=torch.uint8)
    return packed, scale, zero


def _check(x, packed, scale, zero, y, bias=None, what: str = "") -> None:
    ref = linear.int4_reference_f64(x.float().cpu().numpy(), packed.numpy(), scale.float().numpy(), zero.numpy())
    if bias is not None:
        ref = ref + bias.float().numpy()[None, :]
    got = y.float().cpu().numpy()
    err = np.abs(got - ref)
    top = np.abs(ref).max()
    print(f"{what}: max abs err {err.max():.3e}, rel to max|y| {err.max() / top:.3e}", flush=True)
    assert err.max() <= 1e-2 * top


@pytest.mark.parametrize(
    ("rows", "width", "out", "group", "dtype", "with_bias", "kernel"),
    [
        (16, 14336, 4096, 128, torch.bfloat16, False, "auto"),  # the decode batch's down projection, 16 rows
        (32, 14336, 4096, 128, torch.bfloat16, True, "auto"),  # and 32, the bias after the rounded sum
        (48, 8192, 1024, 128, torch.float16, False, "auto"),  # two chunks (32 + 16), 2 K chunks of 16 slices
        (64, 6144, 2048, 256, torch.bfloat16, True, "auto"),  # group 256, two full chunks, 12-slice chunks
        (33, 14336, 512, 128, torch.bfloat16, False, "auto"),  # a one-row second chunk
        (2, 14336, 4100, 128, torch.bfloat16, False, "split"),  # forced at 2 rows, out not a multiple of 64
        (24, 4096, 2048, 128, torch.bfloat16, True, "split"),  # in = 4096: 128-row blocks, 2 K chunks
        (32, 4096, 2112, 512, torch.float16, False, "split"),  # a partial last 128-row block, group 512
    ],
)
def test_split_gemv_multiplies_the_dequantized_weight(rows, width, out, group, dtype, with_bias, kernel) -> None:
    what = f"split rows={rows} in={width} out={out} group={group} {dtype} bias={with_bias} kernel={kernel}"
    print(what, flush=True)
    assert kernels.int4_linear_plan(rows, width, out, group, dtype, kernel=kernel) == "split"
    packed, scale, zero = _layer(out, width, group, seed=rows + width + out, dtype=dtype)
    g = torch.Generator().manual_seed(rows)
    x = torch.randn(rows, width, generator=g).to(dtype)
    bias = (torch.randn(out, generator=g) * 0.5).to(dtype) if with_bias else None
    args = (packed.to(DEV), scale.to(DEV), zero.to(DEV))
    y = kernels.int4_linear(x.to(DEV), *args, None if bias is None else bias.to(DEV), kernel=kernel)
    _check(x, packed, scale, zero, y, bias, what)
    again = kernels.int4_linear(x.to(DEV), *args, None if bias is None else bias.to(DEV), kernel=kernel)
    assert torch.equal(y, again)  # the chunks are added in a fixed order


def test_split_gemv_agrees_with_the_unsplit_kernels_at_full_size() -> None:
    """The decode batch's down projection (32 x 14336 -> 4096) and the lm_head's
    32 rows (4096 -> 128256) against the skinny kernel and the unsplit 32-row GEMV
    on the same inputs (the two sum in different orders: within 1e-2 of max|y|)."""
    for rows, width, out, other in ((32, 14336, 4096, "skinny"), (32, 4096, 128256, "gemv")):
        print(f"full size rows={rows} in={width} out={out} against {other}", flush=True)
        g = torch.Generator(device=DEV).manual_seed(out)
        w = torch.randn(out, width, generator=g, device=DEV) * 0.02
        packed, scale, zero = kernels.quantize_int4(w, 128)
        del w
        scale = scale.to(torch.bfloat16)
        x = torch.randn(rows, width, generator=g, device=DEV).to(torch.bfloat16)
        assert kernels.int4_linear_plan(rows, width, out, 128) == "split"
        got = kernels.int4_linear(x, packed, scale, zero).float()
        want = kernels.int4_linear(x, packed, scale, zero, kernel=other).float()
        err = float((got - want).abs().max()) / float(want.abs().max())
        print(f"  rel diff {err:.3e}", flush=True)
        assert err <= 1e-2
        del packed, scale, zero
        torch.cuda.empty_cache()


def test_workspace_contract_of_the_c_abi() -> None:
    """lnq_int4_linear_ws: with too little workspace the automatic choice runs
    lnq_int4_linear's kernel (same result within the bound); LNQ_KERNEL_SPLIT with
    too little, or misaligned, workspace is refused; lnq_int4_linear refuses the
    split kernel outright."""
    rows, width, out = 32, 14336, 1024
    packed, scale, zero = _layer(out, width, 128, seed=5)
    x = torch.randn(rows, width, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    xd, pd, sd, zd = x.to(DEV), packed.to(DEV), scale.to(DEV), zero.to(DEV)
    chosen, need = ctypes.c_int32(-1), ctypes.c_int64(0)
    _lib.call("lnq_int4_linear_workspace", rows, width, out, 128, _lib.BF16, _lib.KERNEL_AUTO,
              ctypes.byref(chosen), ctypes.byref(need))
    assert chosen.value == _lib.KERNEL_SPLIT and need.value == 4 * rows * out * 4
    ws = torch.empty(need.value // 4 + 4, dtype=torch.float32, device=DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def run(kernel: int, workspace: int, nbytes: int) -> torch.Tensor:
        y = torch.empty(rows, out, dtype=torch.bfloat16, device=DEV)
        _lib.call("lnq_int4_linear_ws", ctypes.c_void_p(xd.data_ptr()), ctypes.c_void_p(pd.data_ptr()),
                  ctypes.c_void_p(sd.data_ptr()), ctypes.c_void_p(zd.data_ptr()), None, ctypes.c_void_p(y.data_ptr()),
                  rows, width, out, 128, _lib.BF16, kernel, ctypes.c_void_p(workspace), nbytes, stream)
        return y

    for kernel, workspace, nbytes in ((_lib.KERNEL_AUTO, ws.data_ptr(), need.value),
                                      (_lib.KERNEL_SPLIT, ws.data_ptr(), need.value),
                                      (_lib.KERNEL_AUTO, ws.data_ptr(), need.value - 16),
                                      (_lib.KERNEL_AUTO, 0, 0)):
        print(f"lnq_int4_linear_ws kernel={kernel} workspace bytes={nbytes}", flush=True)
        _check(x, packed, scale, zero, run(kernel, workspace, nbytes), what=f"ws kernel={kernel} bytes={nbytes}")
    with pytest.raises(LinnetError, match="workspace bytes"):
        run(_lib.KERNEL_SPLIT, ws.data_ptr(), need.value - 16)
    with pytest.raises(LinnetError, match="workspace bytes"):
        run(_lib.KERNEL_SPLIT, ws.data_ptr() + 4, need.value)
    with pytest.raises(LinnetError, match="unknown kernel"):
        y = torch.empty(rows, out, dtype=torch.bfloat16, device=DEV)
        _lib.call("lnq_int4_linear", ctypes.c_void_p(xd.data_ptr()), ctypes.c_void_p(pd.data_ptr()),
                  ctypes.c_void_p(sd.data_ptr()), ctypes.c_void_p(zd.data_ptr()), None, ctypes.c_void_p(y.data_ptr()),
                  rows, width, out, 128, _lib.BF16, _lib.KERNEL_SPLIT, stream)
    torch.cuda.synchronize()


def test_split_gemv_in_a_graph_replays_like_eager() -> None:
    """Captured with its workspace (torch's graph pool) and replayed three times,
    the split call gives the eager bits each time."""
    rows, width, out = 32, 14336, 2048
    packed, scale, zero = (t.to(DEV) for t in _layer(out, width, 128, seed=9))
    x = torch.randn(rows, width, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16).to(DEV)
    eager = kernels.int4_linear(x, packed, scale, zero)
    y = torch.empty_like(eager)
    kernels.int4_linear(x, packed, scale, zero, out=y)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        kernels.int4_linear(x, packed, scale, zero, out=y)
    for i in range(3):
        y.zero_()
        graph.replay()
        torch.cuda.synchronize()
        print(f"replay {i}", flush=True)
        assert torch.equal(y, eager)
