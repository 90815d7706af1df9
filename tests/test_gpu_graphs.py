"""The prefill and 8-bit products replayed from HIP graphs, on the GPU.

Every kernel form of the prefill-shape products is captured together with its
host wrapper: the int4 dequant-GEMM as 128-column tiles, 256-column tiles and
the persistent 256 x 256 form; the per-row FP8 and int8 rounding; and the 8-bit
product as 128- and 256-column tiles, the persistent form and the
weight-streaming form. Each graph is replayed several times, with other eager
work and a synchronization between replays, and every replay must give the
eager call's bits. These kernels keep nothing between calls (no counters, no
cleared scratch), so a replay has no state to get wrong; the test holds them to
that. The decode-shape GEMVs, the split GEMV and the decode step are replayed
in their own tests.
"""

from __future__ import annotations

from typing import Callable

import pytest
import torch

from linnet_amd.torch import kernels

pytestmark = pytest.mark.gpu
DEV = "cuda"
REPLAYS = 3


def _as_tuple(out: torch.Tensor | tuple) -> tuple:
    return out if isinstance(out, tuple) else (out,)


def _replays_match(fn: Callable[[], torch.Tensor | tuple]) -> None:
    eager = _as_tuple(fn())
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = _as_tuple(fn())
    noise = torch.Generator(device=DEV).manual_seed(99)
    for i in range(REPLAYS):
        for t in captured:
            t.zero_()
        # Eager work of the program's own between replays: another kernel on the
        # same stream, then a synchronization.
        torch.randn(1 << 20, generator=noise, device=DEV).sum()
        graph.replay()
        torch.cuda.synchronize()
        for j, (got, want) in enumerate(zip(captured, eager)):
            assert torch.equal(got, want), f"replay {i}, output {j} differs from the eager call"
    del graph


@pytest.mark.parametrize(("kernel", "rows", "k", "n", "dtype"), [
    ("tiled128", 333, 1024, 768, torch.bfloat16),
    ("tiled256", 300, 2048, 1024, torch.float16),
    ("persistent", 1100, 512, 14336, torch.bfloat16),
])
def test_int4_prefill_forms_replay_like_eager(kernel: str, rows: int, k: int, n: int, dtype: torch.dtype) -> None:
    print(f"graph int4 {kernel} rows={rows} k={k} n={n} {dtype}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(rows + n)
    w = torch.randn(n, k, generator=g, device=DEV) * 0.02
    packed, scale, zero = kernels.quantize_int4(w, 128)
    scale = scale.to(dtype)
    x = torch.randn(rows, k, generator=g, device=DEV).to(dtype)
    bias = torch.randn(n, generator=g, device=DEV).to(dtype)
    _replays_match(lambda: kernels.int4_linear(x, packed, scale, zero, bias, kernel=kernel))


@pytest.mark.parametrize("fp8", [True, False])
@pytest.mark.parametrize(("tile_n", "rows", "k", "n"), [
    (128, 333, 1024, 700),
    (256, 333, 1024, 700),
    (kernels.MM8_PERSISTENT, 1100, 512, 14336),
    (kernels.MM8_STREAM, 256, 2048, 4096),
])
def test_8bit_products_replay_like_eager(fp8: bool, tile_n: int, rows: int, k: int, n: int) -> None:
    """The rounding of x and the product in one graph, as `Fp8Linear` /
    `Int8Linear` run them past the few-row threshold."""
    print(f"graph 8-bit fp8={fp8} tile_n={tile_n} rows={rows} k={k} n={n}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(rows + n + int(fp8))
    x = torch.randn(rows, k, generator=g, device=DEV).to(torch.bfloat16)
    ws = torch.rand(n, generator=g, device=DEV) * 0.01 + 0.001
    if fp8:
        wq = (torch.randn(n, k, generator=g, device=DEV) * 40).clamp(-448, 448).to(torch.float8_e4m3fn)

        def run():
            qx, xs = kernels.fp8_rows(x)
            return qx.view(torch.uint8), xs, kernels.fp8_mm(qx, wq, xs, ws, torch.bfloat16, tile_n=tile_n)
    else:
        wq = torch.randint(-127, 128, (n, k), generator=g, device=DEV, dtype=torch.int8)

        def run():
            qx, xs = kernels.int8_rows(x)
            return qx, xs, kernels.int8_mm(qx, wq, xs, ws, torch.bfloat16, tile_n=tile_n)

    _replays_match(run)
