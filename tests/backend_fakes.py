"""Stand-ins for the `linnet.backends` types the plugin adapter uses, with the
fields of `python/linnet/src/linnet/backends/contract.py` and `graph.py` (Linnet
needs Python >= 3.11 and is not installed here). Not a test module."""

from __future__ import annotations

from dataclasses import dataclass, field
from types import SimpleNamespace


@dataclass(frozen=True)
class Capabilities:
    libraries: dict = field(default_factory=dict)
    dtypes: frozenset | None = None


@dataclass(frozen=True)
class TensorSpec:
    shape: tuple
    dtype: str
    layout: str = "contiguous"
    device: int = 0


@dataclass(frozen=True)
class ExecutableMeta:
    inputs: tuple
    outputs: tuple
    allocates: bool = True
    workspace: int = 0
    holds: int = 0
    capturable: bool = True
    stream: str = "caller"
    host: str = "python"
    effects: str = "pure"


class PlanError(Exception):
    pass


@dataclass(frozen=True)
class Value:
    id: int
    name: str
    shape: tuple
    dtype: str


@dataclass(frozen=True)
class Operand:
    value: int | None
    shape: tuple
    dtype: str


@dataclass(frozen=True)
class Call:
    index: int
    callee: str
    semantic: bool
    arguments: tuple
    results: tuple
    start: int
    stop: int


@dataclass(frozen=True)
class Region:
    graph: object
    start: int
    stop: int
    inputs: tuple
    outputs: tuple
    call: int | None = None

    @classmethod
    def of(cls, graph, start, stop, call=None):
        c = graph.calls[call]
        persistent = set(graph.parameters.values())
        inputs = tuple(a.value for a in c.arguments if a.value is not None and a.value not in persistent)
        return cls(graph, start, stop, inputs, tuple(r.value for r in c.results), call)


class Graph:
    """Calls of `linear_int4_groups` over values; `parameters` maps paths to values."""

    def __init__(self) -> None:
        self.calls: list[Call] = []
        self.values: dict[int, Value] = {}
        self.parameters: dict[str, int] = {}

    def value(self, shape, dtype, path=None) -> Operand:
        vid = len(self.values)
        self.values[vid] = Value(vid, f"v{vid}", tuple(shape), dtype)
        if path is not None:
            self.parameters[path] = vid
        return Operand(vid, tuple(shape), dtype)

    def linear(self, name, rows, out, inp, group, dtype="bf16", persistent=True, bias=False, extra_input=False):
        x = self.value((rows, inp), dtype)
        q = self.value((out, inp // group, group), "u4", f"{name}.weight" if persistent else None)
        s = self.value((out, inp // group), dtype, f"{name}.scale")
        z = self.value((out, inp // group), "u8", f"{name}.zero")
        b = self.value((out,), dtype, f"{name}.bias") if bias else Operand(None, (), dtype)
        args = (x, q, s, z, b) if not extra_input else (x, q, s, z, b, self.value((rows, inp), dtype))
        y = self.value((rows, out), dtype)
        n = len(self.calls)
        self.calls.append(Call(n, "std.quant::linear_int4_groups", True, args, (y,), 2 * n, 2 * n + 1))
        return self.calls[-1]

    def semantic_calls(self, callee=None):
        return (c for c in self.calls if c.semantic and (callee is None or c.callee == callee))


TYPES = SimpleNamespace(Capabilities=Capabilities, ExecutableMeta=ExecutableMeta, Region=Region,
                        TensorSpec=TensorSpec, PlanError=PlanError)
