"""The plugin adapter (`linnet_amd.backends.MI355XInt4`) against the
`linnet.backends` contract (`backends/contract.py:228-323`), with stand-in
types and graphs (`tests/backend_fakes.py`): which `linear_int4_groups` calls
it takes, what it compiles them to, and (GPU) that the executable computes the
product the reference's fallback computes, as `backends/conformance.py` checks
a backend: same inputs, outputs within a tolerance."""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from linnet_amd.backends import CALLEE, MI355XInt4
from tests.backend_fakes import TYPES, Graph


def _graph() -> tuple[Graph, list[bool]]:
    g = Graph()
    cases = [
        (dict(name="a", rows=4, out=256, inp=512, group=128), True),
        (dict(name="b", rows=1, out=64, inp=1024, group=64, dtype="f16", bias=True), True),
        (dict(name="c", rows=2, out=32, inp=512, group=16), False),  # group 16
        (dict(name="d", rows=2, out=32, inp=192, group=64), False),  # In % 128
        (dict(name="e", rows=2, out=32, inp=512, group=128, dtype="f32"), False),  # f32 x
        (dict(name="f", rows=2, out=32, inp=512, group=128, persistent=False), False),  # weight not a parameter
        (dict(name="h", rows=2, out=32, inp=512, group=128, extra_input=True), False),  # six arguments
    ]
    for kwargs, _ in cases:
        g.linear(**kwargs)
    return g, [ok for _, ok in cases]


def test_match_takes_the_calls_the_kernels_run() -> None:
    g, ok = _graph()
    backend = MI355XInt4(types=TYPES)
    assert backend.name == "linnet-amd" and backend.contract == 1
    taken = {r.call for r in backend.match(g, SimpleNamespace(kind="cuda", index=0))}
    assert taken == {i for i, good in enumerate(ok) if good}
    assert all(c.callee == CALLEE for c in g.calls)


def test_compile_describes_the_executable() -> None:
    g, _ = _graph()
    backend = MI355XInt4(types=TYPES)
    region = next(iter(backend.match(g, SimpleNamespace(kind="cuda", index=0))))
    made = backend.compile(region, SimpleNamespace(kind="cuda"), None)
    assert made.meta.holds == 0 and made.meta.capturable and made.meta.stream == "caller"
    assert [s.shape for s in made.meta.inputs] == [(4, 512)] and [s.shape for s in made.meta.outputs] == [(4, 256)]
    assert backend.estimate_cost(region, None) is None
    with pytest.raises(TYPES.PlanError):
        backend.compile(TYPES.Region(g, 0, 1, (), (), None), None, None)


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the answer without a GPU")
def test_probe_without_a_gpu() -> None:
    backend = MI355XInt4(types=TYPES)
    assert backend.probe(SimpleNamespace(kind="cpu", index=0)) is None
    assert backend.probe(SimpleNamespace(kind="cuda", index=0)) is None


@pytest.mark.gpu
def test_executable_conforms_to_the_fallback() -> None:
    """Region by region as `conform` runs them: the executable and the
    reference's fallback (dequantize, then `F.linear`) on the same inputs."""
    from linnet_amd.torch import kernels

    backend = MI355XInt4(types=TYPES)
    assert backend.probe(SimpleNamespace(kind="cuda", index=0)).dtypes == frozenset({"bf16", "f16"})
    g, _ = _graph()
    gen = torch.Generator(device="cuda").manual_seed(0)
    params = {}
    for call in g.calls:
        x, q, s, z, b = call.arguments[:5]
        out, groups, group = q.shape
        if group % 2 or s.dtype not in ("bf16", "f16"):
            continue
        dtype = torch.bfloat16 if s.dtype == "bf16" else torch.float16
        w = torch.randn(out, groups * group, generator=gen, device="cuda") * 0.02
        packed, scale, zero = kernels.quantize_int4(w, group)
        name = call.arguments[2]
        prefix = [p for p, v in g.parameters.items() if v == name.value][0].removesuffix("scale")
        params[prefix + "weight"], params[prefix + "scale"], params[prefix + "zero"] = packed, scale.to(dtype), zero
        if b.value is not None:
            params[prefix + "bias"] = torch.randn(out, generator=gen, device="cuda").to(dtype)
    context = SimpleNamespace(parameters=params, target=SimpleNamespace(kind="cuda", index=0))
    for region in backend.match(g, context.target):
        made = backend.compile(region, context.target, None)
        made.prepare(context)
        x, q, s, z, b = g.calls[region.call].arguments
        dtype = torch.bfloat16 if x.dtype == "bf16" else torch.float16
        xin = torch.randn(*x.shape, generator=gen, device="cuda").to(dtype)
        (got,) = made.execute([xin], [], context)
        prefix = [p for p, v in g.parameters.items() if v == s.value][0].removesuffix("scale")
        weight = kernels.int4_weight(params[prefix + "weight"], params[prefix + "scale"], params[prefix + "zero"])
        want = torch.nn.functional.linear(xin, weight)
        if b.value is not None:
            want = want + params[prefix + "bias"]
        err = (got.float() - want.float()).abs().max().item()
        assert got.shape == want.shape and err <= 1e-2 * want.float().abs().max().item(), err
    np.testing.assert_equal(len(list(backend.match(g, context.target))), 2)


def _ordered_graph() -> Graph:
    """Two layers in activation order (`take_inputs`, then the product); the second
    one's taken input is also read after it, so only its product is taken."""
    g = Graph()
    take = g.take("p", rows=1, inp=512)
    g.linear("p", rows=1, out=256, inp=512, group=128, x=take.results[0])
    take2 = g.take("r", rows=3, inp=256, dtype="f16")
    g.linear("r", rows=3, out=64, inp=256, group=128, dtype="f16", x=take2.results[0])
    g.read(take2.results[0])
    return g


def test_match_takes_an_ordered_layer_as_one_region() -> None:
    g = _ordered_graph()
    backend = MI355XInt4(types=TYPES)
    regions = list(backend.match(g, SimpleNamespace(kind="cuda", index=0)))
    assert [r.call for r in regions] == [1, 3]
    fused, plain = regions
    assert (fused.start, fused.stop) == (g.calls[0].start, g.calls[1].stop)
    assert fused.inputs == (g.calls[0].arguments[0].value,)
    assert (plain.start, plain.stop) == (g.calls[3].start, g.calls[3].stop)
    assert plain.inputs == (g.calls[2].results[0].value,)
    made = backend.compile(fused, SimpleNamespace(kind="cuda"), None)
    assert made._order == "p.order" and [s.shape for s in made.meta.inputs] == [(1, 512)]
    assert backend.compile(plain, SimpleNamespace(kind="cuda"), None)._order is None


@pytest.mark.gpu
def test_ordered_executable_conforms_to_the_fallback() -> None:
    """The fused region against the reference's body: `x.index_select(-1, order)`,
    then dequantize and `F.linear`."""
    from linnet_amd.torch import kernels

    backend = MI355XInt4(types=TYPES)
    g = _ordered_graph()
    gen = torch.Generator(device="cuda").manual_seed(3)
    params = {}
    for name, call in (("p.", g.calls[1]), ("r.", g.calls[3])):
        out, groups, group = call.arguments[1].shape
        dtype = torch.bfloat16 if call.arguments[2].dtype == "bf16" else torch.float16
        w = torch.randn(out, groups * group, generator=gen, device="cuda") * 0.02
        packed, scale, zero = kernels.quantize_int4(w, group)
        params[name + "weight"], params[name + "scale"], params[name + "zero"] = packed, scale.to(dtype), zero
        params[name + "order"] = torch.randperm(groups * group, generator=gen, device="cuda").to(torch.int32)
    context = SimpleNamespace(parameters=params, target=SimpleNamespace(kind="cuda", index=0))
    for region in backend.match(g, context.target):
        made = backend.compile(region, context.target, None)
        made.prepare(context)
        x = g.values[region.inputs[0]]
        dtype = torch.bfloat16 if x.dtype == "bf16" else torch.float16
        xin = torch.randn(*x.shape, generator=gen, device="cuda").to(dtype)
        (got,) = made.execute([xin], [], context)
        name = "p." if region.call == 1 else "r."
        weight = kernels.int4_weight(params[name + "weight"], params[name + "scale"], params[name + "zero"])
        taken = xin.index_select(-1, params[name + "order"].long()) if region.call == 1 else xin
        want = torch.nn.functional.linear(taken, weight)
        err = (got.float() - want.float()).abs().max().item()
        print(f"region {region.call}: max abs err {err:.3e}")
        assert got.shape == want.shape and err <= 1e-2 * want.float().abs().max().item(), err


def _nf4_graph() -> tuple[Graph, list[bool]]:
    g = Graph()
    cases = [
        (dict(name="n1", rows=1, out=96, inp=512, block=64), True),
        (dict(name="n2", rows=12, out=40, inp=256, block=32, dtype="f16", bias=True), True),
        (dict(name="n3", rows=2, out=32, inp=512, block=64, dtype="f32"), False),  # f32 x
        (dict(name="n4", rows=2, out=32, inp=512, block=64, persistent=False), False),  # codes not a parameter
        (dict(name="n5", rows=2, out=32, inp=510, block=85), False),  # odd block
        (dict(name="n6", rows=2, out=32, inp=512, block=64, absmax_dtype="bf16"), False),  # absmax not f32
    ]
    for kwargs, _ in cases:
        g.nf4(**kwargs)
    return g, [ok for _, ok in cases]


def test_match_takes_the_nf4_calls() -> None:
    from linnet_amd.backends import NF4_CALLEE

    g, ok = _nf4_graph()
    backend = MI355XInt4(types=TYPES)
    regions = list(backend.match(g, SimpleNamespace(kind="cuda", index=0)))
    assert {r.call for r in regions} == {i for i, good in enumerate(ok) if good}
    assert all(g.calls[r.call].callee == NF4_CALLEE for r in regions)
    made = backend.compile(regions[0], SimpleNamespace(kind="cuda"), None)
    assert made.meta.holds == 0 and [s.shape for s in made.meta.inputs] == [(1, 512)]
    assert [s.shape for s in made.meta.outputs] == [(1, 96)]


@pytest.mark.gpu
def test_nf4_executable_conforms_to_the_fallback() -> None:
    """The reference's body for `linear_nf4` (the widened weight, then the
    product) against the executable, region by region."""
    from linnet_amd.torch import kernels

    backend = MI355XInt4(types=TYPES)
    g, _ = _nf4_graph()
    gen = torch.Generator(device="cuda").manual_seed(3)
    params = {}
    for call in g.calls:
        x, q, a, b = call.arguments
        out, inp = q.shape
        params[[p for p, v in g.parameters.items() if v == a.value][0].removesuffix("absmax") + "weight"] = torch.randint(
            0, 256, (out, inp // 2), generator=gen, device="cuda", dtype=torch.uint8)
        params[[p for p, v in g.parameters.items() if v == a.value][0]] = torch.rand(
            *a.shape, generator=gen, device="cuda") * 0.1
        if b.value is not None:
            params[[p for p, v in g.parameters.items() if v == b.value][0]] = torch.randn(
                out, generator=gen, device="cuda").to(torch.float16 if x.dtype == "f16" else torch.bfloat16)
    context = SimpleNamespace(parameters=params, target=SimpleNamespace(kind="cuda", index=0))
    regions = list(backend.match(g, context.target))
    assert len(regions) == 2
    for region in regions:
        made = backend.compile(region, context.target, None)
        made.prepare(context)
        x, q, a, b = g.calls[region.call].arguments
        dtype = torch.bfloat16 if x.dtype == "bf16" else torch.float16
        xin = torch.randn(*x.shape, generator=gen, device="cuda").to(dtype)
        (got,) = made.execute([xin], [], context)
        prefix = [p for p, v in g.parameters.items() if v == a.value][0].removesuffix("absmax")
        block = q.shape[1] // a.shape[1]
        weight = kernels.nf4_dequantize(params[prefix + "weight"], params[prefix + "absmax"], block, torch.float32)
        want = xin.float() @ weight.T
        if b.value is not None:
            want = want + params[prefix + "bias"].float()
        err = (got.float() - want).abs().max().item()
        assert got.shape == want.shape and err <= 1e-2 * want.abs().max().item(), err
