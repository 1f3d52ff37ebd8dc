"""KTIR intermediate representation: modules, functions, operations, types.

The shape of this model follows what the reference interpreter consumes
(``ir_types.py:524-600``): an ``Operation`` has result names, operand SSA
names, typed attributes and nested regions, and an ``IRFunction`` exposes
``arg_names``, ``grid`` and ``tensor_sizes`` (the first
``construct_memory_view`` per pointer argument, reference
``ir_types.py:565-573``).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Dict, Iterator, List, Optional, Tuple

# Element types understood by the backend.  ``index`` is 32-bit like the
# reference (``dtypes.py:24-39``); bf16 is an extension this backend adds.
ELEM_BYTES = {
    "f16": 2, "bf16": 2, "f32": 4, "f64": 8,
    "i1": 1, "i8": 1, "i16": 2, "i32": 4, "si32": 4, "ui32": 4, "index": 4, "i64": 8, "si64": 8,
}
FLOAT_TYPES = {"f16", "bf16", "f32", "f64"}
INT_TYPES = {"i1", "i8", "i16", "i32", "si32", "ui32", "index", "i64", "si64"}


def canonical_dtype(name: str) -> str:
    return {"fp16": "f16", "float16": "f16", "float32": "f32", "si32": "i32", "si64": "i64"}.get(name, name)


@dataclass(frozen=True)
class ShapedType:
    """``tensor<...>``, ``memref<...>`` or ``!ktdp.access_tile<...>``.

    ``shape`` entries are ints, or None for ``?`` dims.
    """
    kind: str              # "tensor" | "memref" | "access_tile" | "other"
    shape: Tuple[Optional[int], ...]
    elem: str

    def __str__(self):
        dims = "x".join("?" if d is None else str(d) for d in self.shape)
        pre = "!ktdp.access_tile" if self.kind == "access_tile" else self.kind
        return f"{pre}<{dims + 'x' if dims else ''}{self.elem}>"


@dataclass(frozen=True)
class ScalarType:
    name: str

    def __str__(self):
        return self.name


@dataclass
class Region:
    args: List[Tuple[str, Any]] = field(default_factory=list)   # block args (name, type)
    ops: List["Operation"] = field(default_factory=list)


@dataclass
class Operation:
    op_type: str
    results: List[str] = field(default_factory=list)
    operands: List[str] = field(default_factory=list)
    attributes: Dict[str, Any] = field(default_factory=dict)
    result_types: List[Any] = field(default_factory=list)
    operand_types: List[Any] = field(default_factory=list)
    regions: List[Region] = field(default_factory=list)
    text: str = ""

    @property
    def result(self) -> Optional[str]:
        return self.results[0] if self.results else None

    @property
    def result_type(self):
        return self.result_types[0] if self.result_types else None

    def __repr__(self):
        lhs = ", ".join(self.results)
        return f"{lhs + ' = ' if lhs else ''}{self.op_type}({', '.join(self.operands)})"


def iter_ops(ops: List[Operation]) -> Iterator[Operation]:
    for op in ops:
        yield op
        for r in op.regions:
            yield from iter_ops(r.ops)


@dataclass
class IRFunction:
    name: str
    arguments: List[Tuple[str, Any]]
    operations: List[Operation]
    grid: Tuple[int, int, int]
    tensor_sizes: Dict[str, Dict[str, Any]] = field(default_factory=dict)

    @property
    def arg_names(self) -> List[str]:
        return [n.lstrip("%") for n, _ in self.arguments]

    @property
    def num_cores(self) -> int:
        return self.grid[0] * self.grid[1] * self.grid[2]

    def __post_init__(self):
        for op in iter_ops(self.operations):
            if op.op_type == "ktdp.construct_memory_view" and op.operands:
                arg = op.operands[0].lstrip("%")
                if arg not in self.tensor_sizes:
                    self.tensor_sizes[arg] = {
                        "shape": tuple(op.attributes["shape"]),
                        "dtype": op.attributes["dtype"],
                    }

    def __repr__(self):
        t = ", ".join(f"{k}: {v['shape']}x{v['dtype']}" for k, v in self.tensor_sizes.items())
        return f"IRFunction({self.name}, grid={self.grid}, tensors=[{t}])"


@dataclass
class IRModule:
    functions: Dict[str, IRFunction] = field(default_factory=dict)
    aliases: Dict[str, str] = field(default_factory=dict)

    def get_function(self, name: str) -> IRFunction:
        if name not in self.functions:
            raise ValueError(f"Function '{name}' not found in module")
        return self.functions[name]

    def add_function(self, fn: IRFunction):
        self.functions[fn.name] = fn
