"""SSA graph IR recorded by the tracer.

A :class:`Graph` holds parameters (kernel inputs), nodes in program order and
results.  Every node produces one :class:`Value` with a static shape and
dtype.  Op names and attributes follow XLA-HLO vocabulary (the vocabulary of
the reference IR, nkipy/src/nkipy/core/backend/hlo.py:288-404), so the
reference's op semantics carry over; the graph is never serialised to HLO.

Reductions and dots carry an explicit accumulation dtype (``acc_dtype``):
floating sums accumulate in fp32 whatever the storage dtype.

Op vocabulary (attributes in brackets):
  constant [value: np.ndarray]
  elementwise unary: exponential log sqrt rsqrt negate abs sine cosine tan
      atan tanh ceil floor round_nearest_even sign not log_plus_one
      exponential_minus_one is_finite is_nan logistic
  elementwise binary: add subtract multiply divide power maximum minimum
      and or xor remainder floor_divide atan2
  compare [direction: EQ NE LT LE GT GE]      select (pred, on_true, on_false)
  convert (to the node dtype)                 copy
  broadcast_in_dim [broadcast_dimensions]     reshape
  transpose [permutation]                     slice [start, limit, strides]
  concatenate [dimension]                     pad [low, high, interior] (operand, value)
  reduce [dimensions, computation, acc_dtype] argmax / argmin [axis]
  cumsum [axis, acc_dtype]                    iota [dimension]
  dot [lhs_batch, rhs_batch, lhs_contract, rhs_contract, acc_dtype]
  take [axis] (operand, indices)              take_along_axis [axis]
  dynamic_update_slice [start] (operand, update)
  scatter_along_axis [axis] (operand, indices, updates)
  put_along_axis [axis] (operand, indices, values)
  scatter_strided [indices_per_dim] (operand, updates)
"""

from __future__ import annotations

import hashlib
import itertools
from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional, Sequence, Tuple

import numpy as np

from nkipy_amd.core import dtypes as dt

_ids = itertools.count()


class Value:
    """A tensor in the graph: a parameter or the result of one node."""

    __slots__ = ("id", "shape", "dtype", "node", "name", "parameter_id")

    def __init__(self, shape, dtype, node=None, name: str = "", parameter_id=None):
        self.id = next(_ids)
        self.shape = tuple(int(s) for s in shape)
        self.dtype = dt.canonical(dtype)
        self.node = node
        self.name = name
        self.parameter_id = parameter_id

    @property
    def is_parameter(self) -> bool:
        return self.parameter_id is not None

    @property
    def op(self) -> str:
        return "parameter" if self.node is None else self.node.op

    @property
    def size(self) -> int:
        n = 1
        for s in self.shape:
            n *= s
        return n

    @property
    def nbytes(self) -> int:
        return self.size * self.dtype.itemsize

    @property
    def ndim(self) -> int:
        return len(self.shape)

    def __repr__(self):
        nm = f" '{self.name}'" if self.name else ""
        return f"%{self.id}{nm}:{dt.name(self.dtype)}{list(self.shape)}"


class Node:
    __slots__ = ("op", "inputs", "out", "attrs", "loc")

    def __init__(self, op: str, inputs: Sequence[Value], attrs: Dict[str, Any], loc=None):
        self.op = op
        self.inputs = list(inputs)
        self.attrs = dict(attrs or {})
        self.loc = loc
        self.out: Optional[Value] = None

    def __repr__(self):
        a = {k: (f"<{v.dtype}{list(v.shape)}>" if isinstance(v, np.ndarray) else v)
             for k, v in self.attrs.items()}
        ins = ", ".join(f"%{v.id}" for v in self.inputs)
        return f"{self.out!r} = {self.op}({ins}) {a if a else ''}"


@dataclass
class AliasInfo:
    """A result that must live in a parameter's buffer (mutated input)."""

    output_index: int
    param_index: int
    param_name: str
    is_user_returned: bool


@dataclass
class Graph:
    name: str
    parameters: List[Value] = field(default_factory=list)
    nodes: List[Node] = field(default_factory=list)
    results: List[Value] = field(default_factory=list)
    aliases: List[AliasInfo] = field(default_factory=list)

    # -- construction ---------------------------------------------------
    def add_parameter(self, shape, dtype, name: str = "") -> Value:
        v = Value(shape, dtype, None, name=name, parameter_id=len(self.parameters))
        self.parameters.append(v)
        return v

    def add_node(self, op: str, inputs, shape, dtype, attrs=None, loc=None) -> Value:
        for v in inputs:
            if not isinstance(v, Value):
                raise TypeError(f"operand of {op} is not an IR value: {type(v)}")
        node = Node(op, inputs, attrs or {}, loc)
        node.out = Value(shape, dtype, node)
        self.nodes.append(node)
        return node.out

    def set_results(self, values: Sequence[Value]):
        self.results = list(values)

    # -- reference-compatible views (HLOModule.inputs/outputs) -------------
    @property
    def inputs(self) -> List[Value]:
        return self.parameters

    @property
    def outputs(self) -> List[Value]:
        return self.results

    @property
    def auto_aliased_indices(self) -> set:
        return {a.output_index for a in self.aliases if not a.is_user_returned}

    # -- analysis ---------------------------------------------------------
    def users(self) -> Dict[int, List[Node]]:
        u: Dict[int, List[Node]] = {}
        for n in self.nodes:
            for v in n.inputs:
                u.setdefault(v.id, []).append(n)
        return u

    def live_nodes(self) -> List[Node]:
        """Nodes reachable from the results, in program order."""
        live = set()
        stack = [v for v in self.results]
        while stack:
            v = stack.pop()
            if v.node is None or id(v.node) in live:
                continue
            live.add(id(v.node))
            stack.extend(v.node.inputs)
        return [n for n in self.nodes if id(n) in live]

    def content_hash(self) -> str:
        """Stable digest of the computation: ops, shapes, dtypes, attributes
        (constant payloads by content), parameter names and aliasing."""
        h = hashlib.sha256()
        ids: Dict[int, int] = {}

        def ref(v: Value) -> str:
            return str(ids[v.id])

        for p in self.parameters:
            ids[p.id] = len(ids)
            h.update(f"P{p.name}:{dt.name(p.dtype)}{p.shape};".encode())
        for n in self.live_nodes():
            ids[n.out.id] = len(ids)
            h.update(f"N{n.op}({','.join(ref(v) for v in n.inputs)})->"
                     f"{dt.name(n.out.dtype)}{n.out.shape}".encode())
            for k in sorted(n.attrs):
                v = n.attrs[k]
                if isinstance(v, np.ndarray):
                    h.update(f"{k}=<{v.dtype.str}{v.shape}>".encode())
                    h.update(np.ascontiguousarray(v).tobytes())
                elif isinstance(v, np.dtype):
                    h.update(f"{k}={dt.name(v)}".encode())
                else:
                    h.update(f"{k}={v!r}".encode())
        for r in self.results:
            h.update(f"R{ref(r)}:{r.name};".encode())
        for a in self.aliases:
            h.update(f"A{a.output_index}:{a.param_index}:{a.param_name}:{a.is_user_returned}".encode())
        return h.hexdigest()

    def pretty(self) -> str:
        lines = [f"graph {self.name}("
                 + ", ".join(repr(p) for p in self.parameters) + ")"]
        for n in self.nodes:
            lines.append("  " + repr(n))
        lines.append("  return " + ", ".join(repr(r) for r in self.results))
        return "\n".join(lines)

    def __str__(self):
        return self.pretty()
