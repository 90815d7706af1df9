"""This package's int4 product as a Linnet backend plugin: the contract of
`linnet.backends` (`python/linnet/src/linnet/backends/contract.py:228-323`,
`docs/backends.md`), shaped as the reference's own plugin example
(`examples/09-backends/marlin/linnet_marlin/__init__.py`).

A `std.quant::linear_int4_groups` call (an `Int4GroupLinear`) runs on
`lnq_int4_linear`: the HIP kernels read the model's int4 bytes, scales and zero
points as they are stored, so `prepare` converts nothing and the executable
holds no bytes of its own (Marlin keeps a repacked copy). A layer in GPTQ's
activation order (`take_inputs(x, order)` right before the product,
`stdlib/quant.linnet:163-174`) is taken as one region of both calls and runs on
`lnq_int4_linear_ordered`, the gather fused into the one-token GEMV. A
`std.quant::linear_nf4` call (an `Nf4Linear`, which the reference leaves to "a
backend with a 4-bit product", `stdlib/quant.linnet:189-199`) runs on the NF4
kernels the same way, its codes and absmax read as stored. `execute` enqueues on
the caller's stream and never waits, allocates its output with PyTorch, and may
be recorded into a HIP graph.

The contract's types (`Capabilities`, `ExecutableMeta`, `TensorSpec`, `Region`,
`PlanError`) are Linnet's: they are imported from `linnet.backends` and
`linnet.compiler` when the backend is made, unless `types` supplies objects
with the same fields (as the tests do where Linnet is not installed). A
package registers the backend in the `linnet.backends` entry-point group
(`backends/__init__.py:67-75`) as `linnet-amd = linnet_amd.backends:MI355XInt4`.
"""

from __future__ import annotations

import ctypes
from collections.abc import Iterable, Sequence
from types import SimpleNamespace
from typing import Any

import torch

from . import __version__, _lib
from .errors import LinnetError
from .torch import kernels

CALLEE = "std.quant::linear_int4_groups"
TAKE = "std.quant::take_inputs"
NF4_CALLEE = "std.quant::linear_nf4"
DTYPES = {"bf16": torch.bfloat16, "f16": torch.float16}


def _linnet_types() -> SimpleNamespace:
    try:
        from linnet.backends import Capabilities, ExecutableMeta, Region, TensorSpec  # type: ignore[import-not-found]
        from linnet.compiler import PlanError  # type: ignore[import-not-found]
    except ImportError as error:
        raise LinnetError("linnet is not installed: pass `types` with the contract's classes") from error
    return SimpleNamespace(Capabilities=Capabilities, ExecutableMeta=ExecutableMeta, Region=Region,
                           TensorSpec=TensorSpec, PlanError=PlanError)


def _fused_group(group: int) -> bool:
    """The groups the HIP kernels take (`lnq_int4_linear`)."""
    return group in (32, 64) or (group > 0 and group % 128 == 0)


class MI355XInt4:
    """Takes the group-wise int4 `linear` calls the gfx950 kernels run."""

    contract = 1  # the version of `linnet.backends` it is written for

    def __init__(self, types: Any = None) -> None:
        self._t = types if types is not None else _linnet_types()

    @property
    def name(self) -> str:
        return "linnet-amd"

    @property
    def version(self) -> str:
        return __version__

    def probe(self, target: Any) -> Any:
        """Capabilities on a gfx950 GPU (PyTorch on ROCm names it `cuda`), else None."""
        if target.kind != "cuda":
            return None
        try:
            lib = _lib.load()
        except LinnetError:
            return None
        is_gfx950, units = ctypes.c_int32(), ctypes.c_int32()
        if lib.lnq_device_probe(int(target.index), ctypes.byref(is_gfx950), ctypes.byref(units)) != _lib.LNQ_OK:
            return None
        if not is_gfx950.value:
            return None
        return self._t.Capabilities({"linnet_amd": self.version}, frozenset(DTYPES))

    def match(self, graph: Any, target: Any) -> Iterable[Any]:
        """Each `linear_int4_groups(x, q, scale, zero, bias)` call whose weight the
        kernels take: bf16 / f16 x with scales of its dtype, In % 128 == 0, a group
        of 32, 64 or a multiple of 128, the weight (and bias) persistent, x the
        region's one input."""
        persistent = set(graph.parameters.values())
        takes = _takes(graph, persistent)
        for call in graph.semantic_calls(CALLEE):
            if len(call.arguments) != 5:
                continue
            x, q, scale, zero, bias = call.arguments
            if len(q.shape) != 3:
                continue
            _, groups, group = q.shape
            if not (
                x.dtype in DTYPES
                and scale.dtype == x.dtype
                and (groups * group) % 128 == 0
                and _fused_group(group)
                and all(v.value in persistent for v in (q, scale, zero))
                and (bias.value is None or bias.value in persistent)
            ):
                continue
            take = takes.get(x.value)
            if take is not None and take.stop == call.start:
                # take_inputs, then the product: one region whose one input is the
                # untaken x, if nothing after it reads the taken x.
                region = self._t.Region.of(graph, take.start, call.stop, call.index)
                if tuple(region.inputs) == (take.arguments[0].value,) and len(region.outputs) == 1:
                    yield region
                    continue
            region = self._t.Region.of(graph, call.start, call.stop, call.index)
            if tuple(region.inputs) == (x.value,):
                yield region
        yield from self._match_nf4(graph, persistent)

    def _match_nf4(self, graph: Any, persistent: set[int]) -> Iterable[Any]:
        """Each `linear_nf4<Block>(x, q, absmax, bias)` call (`stdlib/quant.linnet:189-199`,
        an `Nf4Linear`): bf16 / f16 x, q [Out, In] nf4 and absmax [Out, In / Block]
        f32 parameters, an even Block; `nf4_linear` runs it (the NF4 GEMV up to 8
        rows, the widened weight and its product beyond)."""
        for call in graph.semantic_calls(NF4_CALLEE):
            if len(call.arguments) != 4:
                continue
            x, q, absmax, bias = call.arguments
            if len(q.shape) != 2 or len(absmax.shape) != 2 or absmax.shape[0] != q.shape[0] or not absmax.shape[1]:
                continue
            in_features, blocks = q.shape[1], absmax.shape[1]
            block = in_features // blocks
            if not (
                x.dtype in DTYPES
                and absmax.dtype == "f32"
                and block * blocks == in_features
                and block % 2 == 0
                and q.value in persistent
                and absmax.value in persistent
                and (bias.value is None or bias.value in persistent)
            ):
                continue
            region = self._t.Region.of(graph, call.start, call.stop, call.index)
            if tuple(region.inputs) == (x.value,):
                yield region

    def compile(self, region: Any, target: Any, options: Any) -> _Int4Linear | _Nf4Linear:
        graph = region.graph
        if region.call is None:
            raise self._t.PlanError("linnet-amd takes a `linear_int4_groups` call")
        call = graph.calls[region.call]
        path = {value: p for p, value in graph.parameters.items()}
        values = graph.values
        meta = self._t.ExecutableMeta(
            tuple(self._t.TensorSpec(values[v].shape, values[v].dtype) for v in region.inputs),
            tuple(self._t.TensorSpec(values[v].shape, values[v].dtype) for v in region.outputs),
            holds=0,
        )
        if call.callee == NF4_CALLEE:
            x, q, absmax, bias = call.arguments
            return _Nf4Linear(meta, (path[q.value], path[absmax.value]),
                              path[bias.value] if bias.value is not None else None, DTYPES[x.dtype],
                              q.shape[1] // absmax.shape[1])
        x, q, scale, zero, bias = call.arguments
        order = None
        if region.start != call.start:
            take = _takes(graph, set(path)).get(x.value)
            if take is None or region.start != take.start:
                raise self._t.PlanError("linnet-amd takes `take_inputs` only right before `linear_int4_groups`")
            order = path[take.arguments[1].value]
        return _Int4Linear(meta, (path[q.value], path[scale.value], path[zero.value]),
                           path[bias.value] if bias.value is not None else None, DTYPES[x.dtype], order)

    def estimate_cost(self, region: Any, target: Any) -> Any:
        return None  # the planner measures


def _takes(graph: Any, persistent: set[int]) -> dict[int, Any]:
    """The `take_inputs(x, order)` calls whose order is a parameter, by the value
    each makes."""
    found = {}
    for call in graph.semantic_calls(TAKE):
        if len(call.arguments) == 2 and len(call.results) == 1 and call.arguments[1].value in persistent:
            found[call.results[0].value] = call
    return found


class _Int4Linear:
    """One `linear_int4_groups` call (after its `take_inputs`, with `order`) on
    `lnq_int4_linear` / `lnq_int4_linear_ordered`."""

    def __init__(self, meta: Any, paths: tuple[str, str, str], bias: str | None, dtype: torch.dtype,
                 order: str | None = None) -> None:
        self._meta = meta
        self._paths = paths
        self._bias = bias
        self._dtype = dtype
        self._order = order

    @property
    def meta(self) -> Any:
        return self._meta

    def prepare(self, context: Any) -> None:
        """Nothing to convert: the kernels read the parameters as stored. Checks
        that they are where and what the kernels need."""
        q, scale, zero = (context.parameters[p] for p in self._paths)
        if not (q.is_cuda and scale.is_cuda and zero.is_cuda):
            raise LinnetError("linnet-amd: the int4 parameters are not on the GPU")
        if q.dtype != torch.uint8 or zero.dtype != torch.uint8 or scale.dtype != self._dtype:
            raise LinnetError("linnet-amd: int4 bytes and zero points are uint8, scales the input's dtype")
        if self._order is not None:
            order = context.parameters[self._order]
            if not order.is_cuda or order.dtype != torch.int32:
                raise LinnetError("linnet-amd: the input order is an int32 parameter on the GPU")

    def execute(self, inputs: Sequence[torch.Tensor], outputs: Sequence[torch.Tensor], context: Any) -> Sequence[torch.Tensor]:
        q, scale, zero = (context.parameters[p] for p in self._paths)
        bias = context.parameters[self._bias] if self._bias is not None else None
        order = context.parameters[self._order] if self._order is not None else None
        (x,) = inputs
        rows = x.reshape(-1, x.shape[-1])
        y = kernels.int4_linear(rows, q, scale, zero, bias, order=order)
        return [y.reshape(*x.shape[:-1], y.shape[-1])]


class _Nf4Linear:
    """One `linear_nf4` call on `kernels.nf4_linear`: the codes ([Out, In/2]
    bytes, as the model binds an nf4 parameter) and absmax read as stored."""

    def __init__(self, meta: Any, paths: tuple[str, str], bias: str | None, dtype: torch.dtype, block: int) -> None:
        self._meta = meta
        self._paths = paths
        self._bias = bias
        self._dtype = dtype
        self._block = block

    @property
    def meta(self) -> Any:
        return self._meta

    def prepare(self, context: Any) -> None:
        q, absmax = (context.parameters[p] for p in self._paths)
        if not (q.is_cuda and absmax.is_cuda):
            raise LinnetError("linnet-amd: the NF4 parameters are not on the GPU")
        if q.dtype != torch.uint8 or absmax.dtype != torch.float32:
            raise LinnetError("linnet-amd: NF4 codes are uint8 bytes and absmax float32")

    def execute(self, inputs: Sequence[torch.Tensor], outputs: Sequence[torch.Tensor], context: Any) -> Sequence[torch.Tensor]:
        q, absmax = (context.parameters[p] for p in self._paths)
        bias = context.parameters[self._bias] if self._bias is not None else None
        (x,) = inputs
        return [kernels.nf4_linear(x, q, absmax, self._block, bias)]


__all__ = ["CALLEE", "NF4_CALLEE", "TAKE", "MI355XInt4"]
