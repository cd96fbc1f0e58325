"""Strided views of traced values.

Fused kernels read their operands in place: an operand that the NumPy code
reached through ``np.split``, ``reshape``, ``transpose``, ``np.repeat`` /
``broadcast_to`` and same-dtype copies is described by a base value (which
the lowering materialises contiguously) plus, for every dimension of the
operand, a list of ``(size, stride)`` factors in row-major order.  Most
dimensions have one factor; a dimension produced by ``np.repeat(k, r,
axis=2)`` on the head axis has two, ``[(n_kv, stride), (r, 0)]``, which is
how the attention kernel sees grouped-query heads without a copy.

Exact widening converts (bf16 / f16 -> f32) may sit anywhere in the chain;
``View.widened`` records them, so a kernel that reads the narrow base and
computes in fp32 sees the same values.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional, Tuple

import numpy as np

from nkipy_amd.core import dtypes as dt
from nkipy_amd.core.backend.ir import Node, Value

Factor = Tuple[int, int]  # (size, stride in elements)

_VIEW_OPS = ("transpose", "broadcast_in_dim", "reshape", "slice", "copy")


def _contiguous(shape) -> List[List[Factor]]:
    dims, s = [], 1
    for n in reversed(shape):
        dims.append([(int(n), s)])
        s *= int(n)
    return dims[::-1]


def _simplify(fs: List[Factor]) -> List[Factor]:
    """Drop size-1 factors, merge (a, s*b)(b, s) into (a*b, s)."""
    out: List[Factor] = []
    for n, s in fs:
        if n == 1:
            continue
        if out and out[-1][1] == n * s:
            out[-1] = (out[-1][0] * n, s)
        else:
            out.append((n, s))
    return out or [(1, 0)]


def _reshape(dims: List[List[Factor]], new_shape) -> Optional[List[List[Factor]]]:
    flat: List[Factor] = [f for d in dims for f in d if f[0] != 1]
    out: List[List[Factor]] = []
    i = 0
    for n in new_shape:
        n = int(n)
        if n == 1:
            out.append([(1, 0)])
            continue
        need, cur = n, []
        while need > 1:
            if i >= len(flat):
                return None
            f, s = flat[i]
            if f <= need:
                if need % f:
                    return None
                cur.append((f, s))
                need //= f
                i += 1
            else:
                if f % need:
                    return None
                # split (f, s) into (need, s * f/need) (outer) and (f/need, s)
                cur.append((need, s * (f // need)))
                flat[i] = (f // need, s)
                need = 1
        out.append(cur)
    if any(f[0] != 1 for f in flat[i:]):
        return None
    return out


@dataclass
class View:
    base: Value
    offset: int
    dims: List[List[Factor]]
    nodes: List[Node] = field(default_factory=list)  # layout nodes between the operand and base
    widened: bool = False

    @property
    def shape(self) -> Tuple[int, ...]:
        return tuple(int(np.prod([f[0] for f in d])) for d in self.dims)

    def simple(self, d: int) -> Optional[int]:
        """Stride of dim ``d`` if it is a single factor, else None."""
        fs = _simplify(self.dims[d])
        if len(fs) == 1:
            return fs[0][1] if fs[0][0] != 1 else 0
        return None

    def grouped(self, d: int) -> Optional[Tuple[int, int, int]]:
        """Dim ``d`` as (groups, group stride, repeat) with the index mapping
        i -> (i // repeat) * group stride; None if it is not of that form."""
        fs = _simplify(self.dims[d])
        if len(fs) == 1:
            n, s = fs[0]
            if s == 0:
                return 1, 0, n
            return n, s, 1
        if len(fs) == 2 and fs[1][1] == 0:
            return fs[0][0], fs[0][1], fs[1][0]
        return None

    def materialize_check(self, array: np.ndarray) -> np.ndarray:
        """Apply the view to a host copy of the base (tests, constants)."""
        flat = np.ascontiguousarray(array).reshape(-1)
        shape = [f[0] for d in self.dims for f in d]
        strides = [f[1] * flat.itemsize for d in self.dims for f in d]
        v = np.lib.stride_tricks.as_strided(flat[self.offset:], shape=shape, strides=strides)
        return np.array(v).reshape(self.shape)


def _step(node: Node, dims: List[List[Factor]], offset: int):
    """Factors of node.out from those of node.inputs[0]; None if inexpressible."""
    op = node.op
    src = node.inputs[0]
    out = node.out
    if op in ("copy", "convert"):
        return dims, offset
    if op == "transpose":
        return [dims[p] for p in node.attrs["permutation"]], offset
    if op == "broadcast_in_dim":
        bd = list(node.attrs["broadcast_dimensions"])
        res = []
        for d, n in enumerate(out.shape):
            if d in bd:
                j = bd.index(d)
                res.append(dims[j] if src.shape[j] == n else [(int(n), 0)])
            else:
                res.append([(int(n), 0)])
        return res, offset
    if op == "slice":
        res = []
        for d, (st, lim, sd) in enumerate(zip(node.attrs["start_indices"], node.attrs["limit_indices"],
                                              node.attrs["strides"])):
            n_out = out.shape[d]
            if st == 0 and sd == 1 and n_out == src.shape[d]:
                res.append(dims[d])
                continue
            fs = _simplify(dims[d])
            if len(fs) != 1:
                return None
            stride = fs[0][1]
            offset += int(st) * stride
            res.append([(int(n_out), stride * int(sd))])
        return res, offset
    if op == "reshape":
        r = _reshape(dims, out.shape)
        return (r, offset) if r is not None else None
    return None


def _is_view_node(n: Node, widen_ok: bool) -> bool:
    if n is None:
        return False
    if n.op in _VIEW_OPS:
        return n.op != "copy" or n.out.dtype == n.inputs[0].dtype
    if n.op == "convert" and widen_ok:
        return n.inputs[0].dtype in (dt.bfloat16, dt.float16) and n.out.dtype == dt.float32
    return False


def resolve(v: Value, widen_ok: bool = True) -> View:
    """Describe ``v`` as a strided view of the deepest value reachable
    through layout nodes (and exact widening converts)."""
    chain: List[Node] = []
    cur = v
    while not cur.is_parameter and _is_view_node(cur.node, widen_ok):
        chain.append(cur.node)
        cur = cur.node.inputs[0]
    # chain[0] produces v, chain[-1] reads cur.  Use chain[:stop]; the base
    # is the value chain[stop] produces (cur when the whole chain is used).
    # On an inexpressible step, restart with the base just above it.
    stop = len(chain)
    while True:
        base = cur if stop == len(chain) else chain[stop].out
        dims, off = _contiguous(base.shape), 0
        failed = None
        for k in range(stop - 1, -1, -1):
            r = _step(chain[k], dims, off)
            if r is None:
                failed = k
                break
            dims, off = r
        if failed is None:
            break
        stop = failed
    used = chain[:stop]
    widened = any(n.op == "convert" for n in used)
    return View(base, off, dims, used, widened)
