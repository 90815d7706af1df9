"""The decode glue folded into the int4 GEMV (`lnq_int4_linear_prologue`), on the GPU.

- `int4_linear_silu_mul(g, u, ...)` == `int4_linear(decode.silu_mul(g, u), ...)` bit
  for bit at every shape;
- `int4_linear_rmsnorm(x, w, eps, ...)`: folded (one row, group 128, a one-token
  kernel's In) it computes r * (W (x * w)), so it is held to the product of the f64
  normed row with the exactly dequantized weight within 1e-2 * max|y| (the bound of
  every int4 product here) and to the two calls `int4_linear(decode.rmsnorm(...))`
  within the same bound (max errors printed); staged, it is the two calls bit for bit;
- with `bias` = the residual row, either equals `residual + the call without bias`
  rounded as torch's bf16 add rounds it.
One row at group 128 runs the one-token kernels (In 4096: the per-wave kernel; In
8192 and 14336: the slices kernel; Out from 100 to 28672); more rows, an In no
one-token kernel takes (11008), group 64 and more than 32768 outputs run the staged
path (the prologue's kernel, then `int4_linear`). The RMSNorm kernel itself is checked
against torch in `test_gpu_llama.py`.
"""

from __future__ import annotations

import pytest
import torch

from linnet_amd.torch import decode, kernels

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _layer(n: int, k: int, group: int, seed: int):
    g = torch.Generator(device=DEV).manual_seed(seed)
    w = torch.randn(n, k, generator=g, device=DEV) * 0.02
    packed, scale, zero = kernels.quantize_int4(w, group)
    return packed, scale.to(torch.bfloat16), zero


SHAPES = [(1, 4096, 6144, 128), (1, 4096, 28672, 128), (1, 4096, 100, 128), (1, 8192, 1024, 128),
          (1, 14336, 4096, 128), (3, 4096, 1024, 128), (1, 11008, 512, 128), (1, 4096, 512, 64), (17, 4096, 256, 128),
          (1, 4096, 40000, 128)]


@pytest.mark.parametrize(("rows", "k", "n", "group"), SHAPES)
def test_folded_rmsnorm_matches_the_two_calls(rows: int, k: int, n: int, group: int) -> None:
    print(f"rmsnorm prologue rows {rows} In {k} Out {n} group {group}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(k + n)
    w = _layer(n, k, group, rows)
    x = (torch.randn(rows, k, generator=g, device=DEV) * 3).to(torch.bfloat16)
    norm = 1 + 0.1 * torch.randn(k, generator=g, device=DEV)
    resid = torch.randn(n, generator=g, device=DEV).to(torch.bfloat16)
    folded = rows == 1 and group == 128 and k in (4096, 8192, 14336) and n <= 32768
    weight = kernels.int4_weight(*w).double()
    for eps in (1e-5, 1e-6):
        two = kernels.int4_linear(decode.rmsnorm(x.clone(), norm, eps), *w)
        got = kernels.int4_linear_rmsnorm(x, norm, eps, *w)
        if folded:
            xd = x.double()
            exact = (xd * torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + eps) * norm.double()) @ weight.T
            top = exact.abs().max().item()
            err = (got.double() - exact).abs().max().item()
            err_two = (got.double() - two.double()).abs().max().item()
            print(f"  eps {eps}: max abs err {err:.3e} ({err / top:.2e} of max|y|) vs f64; "
                  f"{err_two:.3e} vs the two calls", flush=True)
            assert err <= 1e-2 * top and err_two <= 1e-2 * top
        else:
            assert torch.equal(got, two)
        with_bias = kernels.int4_linear_rmsnorm(x, norm, eps, *w, bias=resid)
        assert torch.equal(with_bias, (got + resid).to(torch.bfloat16))


@pytest.mark.parametrize(("rows", "k", "n", "group"), SHAPES)
def test_folded_silu_mul_equals_the_two_calls(rows: int, k: int, n: int, group: int) -> None:
    print(f"silu_mul prologue rows {rows} In {k} Out {n} group {group}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(3 * k + n)
    w = _layer(n, k, group, rows + 7)
    # The two halves of a joined gate|up output, as the MLP reads them (column slices).
    gu = (torch.randn(rows, 2 * k, generator=g, device=DEV) * 4).to(torch.bfloat16)
    gate, up = gu[:, :k], gu[:, k:]
    resid = torch.randn(n, generator=g, device=DEV).to(torch.bfloat16)
    want = kernels.int4_linear(decode.silu_mul(gate, up), *w)
    assert torch.equal(kernels.int4_linear_silu_mul(gate, up, *w), want)
    assert torch.equal(kernels.int4_linear_silu_mul(gate, up, *w, bias=resid), (want + resid).to(torch.bfloat16))


def test_folded_calls_replay_in_a_graph() -> None:
    """Both folded calls captured in one graph, replayed three times with eager
    work between the replays: every replay equals the eager result."""
    w1, w2 = _layer(6144, 4096, 128, 1), _layer(4096, 14336, 128, 2)
    g = torch.Generator(device=DEV).manual_seed(5)
    x = torch.randn(1, 4096, generator=g, device=DEV).to(torch.bfloat16)
    norm = 1 + 0.1 * torch.randn(4096, generator=g, device=DEV)
    gu = torch.randn(1, 2 * 14336, generator=g, device=DEV).to(torch.bfloat16)
    eager = (kernels.int4_linear_rmsnorm(x, norm, 1e-5, *w1),
             kernels.int4_linear_silu_mul(gu[:, :14336], gu[:, 14336:], *w2, bias=x[0]))
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = (kernels.int4_linear_rmsnorm(x, norm, 1e-5, *w1),
               kernels.int4_linear_silu_mul(gu[:, :14336], gu[:, 14336:], *w2, bias=x[0]))
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(out, eager))
        kernels.int4_linear(x, *w1)
        torch.cuda.synchronize()
