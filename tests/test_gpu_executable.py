"""The executable-shaped C ABI on the GPU: `lnq_int4_linear_executable` driven the
way the reference runtime drives an `LnExecutable` (prepare once, execute per
call on the context's stream) gives `int4_linear`'s output bit for bit at one
row, a few rows and a prompt's rows (and with a bias), refuses tensors that do
not match the layer, and replays inside a HIP graph."""

from __future__ import annotations

import pytest
import torch

from linnet_amd import LinnetError, executable
from linnet_amd.torch import kernels

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _layer(out: int, width: int, group: int, seed: int):
    g = torch.Generator().manual_seed(seed)
    packed = torch.randint(0, 256, (out, width // group, group // 2), generator=g, dtype=torch.uint8)
    scale = (torch.rand(out, width // group, generator=g) * 0.02 + 0.001).to(torch.bfloat16)
    zero = torch.randint(0, 16, (out, width // group), generator=g, dtype=torch.uint8)
    return packed.to(DEV), scale.to(DEV), zero.to(DEV)


@pytest.mark.parametrize(("shape", "with_bias"), [((1, 4096), False), ((2, 3, 4096), True), ((300, 4096), False)])
def test_execute_equals_int4_linear(shape, with_bias: bool) -> None:
    print(f"executable x {shape} bias={with_bias}", flush=True)
    params = _layer(1000, 4096, 128, seed=len(shape))
    x = torch.randn(*shape, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(DEV)
    bias = torch.randn(1000, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).to(DEV)
    exe = executable.Int4LinearExecutable(4096, 1000, 128)
    exe.prepare(device_id=0)
    y = torch.empty(*shape[:-1], 1000, dtype=torch.bfloat16, device=DEV)
    exe.execute([x, *params] + ([bias] if with_bias else []), [y])
    want = kernels.int4_linear(x.reshape(-1, 4096), *params, bias if with_bias else None).reshape(y.shape)
    torch.cuda.synchronize()
    assert torch.equal(y, want)


def test_execute_refuses_tensors_of_another_layer() -> None:
    params = _layer(64, 512, 128, seed=1)
    exe = executable.Int4LinearExecutable(512, 64, 128)
    exe.prepare(device_id=0)
    x = torch.zeros(2, 512, dtype=torch.bfloat16, device=DEV)
    y = torch.empty(2, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(LinnetError, match="last axis"):
        exe.execute([torch.zeros(2, 256, dtype=torch.bfloat16, device=DEV), *params], [y])
    with pytest.raises(LinnetError, match="scale is"):
        exe.execute([x, params[0], params[1].float(), params[2]], [y])
    with pytest.raises(LinnetError, match="contiguous"):
        exe.execute([torch.zeros(512, 2, dtype=torch.bfloat16, device=DEV).t(), *params], [y])
    with pytest.raises(LinnetError, match="y is"):
        exe.execute([x, *params], [torch.empty(2, 65, dtype=torch.bfloat16, device=DEV)])
    with pytest.raises(LinnetError, match="device"):
        exe.execute([x.cpu(), *params], [y], device_type=None)


def test_execute_replays_in_a_graph() -> None:
    params = _layer(2048, 1024, 128, seed=5)
    exe = executable.Int4LinearExecutable(1024, 2048, 128)
    exe.prepare(device_id=0)
    x = torch.randn(4, 1024, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16).to(DEV)
    y = torch.empty(4, 2048, dtype=torch.bfloat16, device=DEV)
    eager = kernels.int4_linear(x, *params)
    exe.execute([x, *params], [y])
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        exe.execute([x, *params], [y])
    for _ in range(3):
        y.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager)
