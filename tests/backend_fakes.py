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
        """As `contract.py:151-220` computes them, over the calls inside the range:
        inputs are the values they read that none of them made (parameters
        aside), outputs the values they made that a call after the range reads or
        that the last call returns."""
        inside = [c for c in graph.calls if start <= c.start and c.stop <= stop]
        persistent = set(graph.parameters.values())
        made: set[int] = set()
        inputs: dict[int, None] = {}
        for c in inside:
            for a in c.arguments:
                if a.value is not None and a.value not in persistent and a.value not in made:
                    inputs[a.value] = None
            made.update(r.value for r in c.results)
        read_after = {a.value for c in graph.calls if c.start >= stop for a in c.arguments}
        last = {r.value for r in inside[-1].results}
        outputs = tuple(v for c in inside for v in (r.value for r in c.results) if v in read_after or v in last)
        return cls(graph, start, stop, tuple(inputs), outputs, call)


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

    def take(self, name, rows, inp, dtype="bf16"):
        """`std.quant::take_inputs(x, order)` with `order` the parameter `name.order`."""
        x = self.value((rows, inp), dtype)
        order = self.value((inp,), "i32", f"{name}.order")
        taken = self.value((rows, inp), dtype)
        n = len(self.calls)
        start = self.calls[-1].stop if self.calls else 0
        self.calls.append(Call(n, "std.quant::take_inputs", True, (x, order), (taken,), start, start + 1))
        return self.calls[-1]

    def linear(self, name, rows, out, inp, group, dtype="bf16", persistent=True, bias=False, extra_input=False,
               x=None):
        x = self.value((rows, inp), dtype) if x is None else x
        q = self.value((out, inp // group, group), "u4", f"{name}.weight" if persistent else None)
        s = self.value((out, inp // group), dtype, f"{name}.scale")
        z = self.value((out, inp // group), "u8", f"{name}.zero")
        b = self.value((out,), dtype, f"{name}.bias") if bias else Operand(None, (), dtype)
        args = (x, q, s, z, b) if not extra_input else (x, q, s, z, b, self.value((rows, inp), dtype))
        y = self.value((rows, out), dtype)
        n = len(self.calls)
        # Each call's range starts where the previous one stopped.
        start = self.calls[-1].stop if self.calls else 0
        self.calls.append(Call(n, "std.quant::linear_int4_groups", True, args, (y,), start, start + 1))
        return self.calls[-1]

    def nf4(self, name, rows, out, inp, block, dtype="bf16", bias=False, persistent=True, absmax_dtype="f32"):
        """`std.quant::linear_nf4<block>(x, q, absmax, bias)`."""
        x = self.value((rows, inp), dtype)
        q = self.value((out, inp), "nf4", f"{name}.weight" if persistent else None)
        a = self.value((out, inp // block), absmax_dtype, f"{name}.absmax")
        b = self.value((out,), dtype, f"{name}.bias") if bias else Operand(None, (), dtype)
        y = self.value((rows, out), dtype)
        n = len(self.calls)
        start = self.calls[-1].stop if self.calls else 0
        self.calls.append(Call(n, "std.quant::linear_nf4", True, (x, q, a, b), (y,), start, start + 1))
        return self.calls[-1]

    def read(self, operand):
        """A later call (another op) that reads `operand`."""
        n = len(self.calls)
        start = self.calls[-1].stop if self.calls else 0
        self.calls.append(Call(n, "std.core::other", True, (operand,), (), start, start + 1))
        return self.calls[-1]

    def semantic_calls(self, callee=None):
        return (c for c in self.calls if c.semantic and (callee is None or c.callee == callee))


TYPES = SimpleNamespace(Capabilities=Capabilities, ExecutableMeta=ExecutableMeta, Region=Region,
                        TensorSpec=TensorSpec, PlanError=PlanError)
