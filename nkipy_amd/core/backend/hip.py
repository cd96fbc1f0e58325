"""The ``"hip"`` trace context and graph-building helpers.

``HIPTraceContext`` satisfies the reference's trace-context protocol
(``backend_name``, ``set_source_location``, ``build_op``;
nkipy/src/nkipy/core/backend/hlo.py:1538-1585) while recording into this
package's own :class:`~nkipy_amd.core.backend.ir.Graph`.
"""

from __future__ import annotations

from typing import Optional, Sequence, Tuple

import numpy as np

from nkipy_amd.core import dtypes as dt
from nkipy_amd.core.backend import get_active_context
from nkipy_amd.core.backend.ir import Graph, Value
from nkipy_amd.core.backend.promotion import scalar_dtype


class HIPTraceContext:
    backend_name = "hip"

    def __init__(self, graph: Graph):
        self.graph = graph
        self._loc: Optional[Tuple[str, int]] = None

    # reference protocol ---------------------------------------------------
    def set_source_location(self, location):
        self._loc = location

    def build_op(self, op_name: str, operands: Sequence[Value], result_shape,
                 result_dtype, attributes=None, source_location=None) -> Value:
        loc = source_location if source_location is not None else self._loc
        return self.graph.add_node(op_name, operands, result_shape, result_dtype,
                                   attributes, loc)

    # conveniences ----------------------------------------------------------
    def add_parameter(self, shape, dtype, name="") -> Value:
        return self.graph.add_parameter(shape, dtype, name)

    def constant(self, value, dtype=None) -> Value:
        arr = np.asarray(value)
        if dtype is None:
            if arr.ndim == 0 and not isinstance(value, np.ndarray):
                dtype = scalar_dtype(value)
            else:
                dtype = arr.dtype
                if dtype == dt.float64:
                    dtype = dt.float32
                elif dtype == dt.int64:
                    dtype = dt.int32
                elif dtype == dt.uint64:
                    dtype = dt.uint32
        dtype = dt.canonical(dtype)
        payload = _cast_payload(arr, dtype)
        return self.build_op("constant", [], payload.shape, dtype, {"value": payload})


def _cast_payload(arr: np.ndarray, dtype: np.dtype) -> np.ndarray:
    """Store constant payloads in the target dtype's bit representation."""
    if arr.dtype == dtype:
        return np.array(arr, copy=True, order="C")
    if dtype == dt.bfloat16:
        src = dt.to_float32(arr) if arr.dtype.fields is not None else arr.astype(np.float32)
        return dt.to_bf16(src)
    if dtype == dt.float8_e4m3fn:
        return dt.to_e4m3fn(dt.to_float32(arr))
    if dtype in dt.FP8_TYPES:
        raise TypeError(f"constants of dtype {dt.name(dtype)} are not supported")
    if arr.dtype.fields is not None:
        arr = dt.to_float32(arr)
    return np.array(arr.astype(dtype), copy=False, order="C")


def get_hip_context() -> HIPTraceContext:
    ctx = get_active_context()
    if not isinstance(ctx, HIPTraceContext):
        raise RuntimeError("No HIP trace context is active.")
    return ctx


def broadcast_shapes(a: Tuple[int, ...], b: Tuple[int, ...]) -> Tuple[int, ...]:
    n = max(len(a), len(b))
    a2 = (1,) * (n - len(a)) + tuple(a)
    b2 = (1,) * (n - len(b)) + tuple(b)
    out = []
    for x, y in zip(a2, b2):
        if x == y or y == 1:
            out.append(x)
        elif x == 1:
            out.append(y)
        else:
            raise ValueError(f"operands could not be broadcast together with shapes {a} {b}")
    return tuple(out)


def broadcast_to(ctx: HIPTraceContext, v: Value, shape) -> Value:
    """NumPy-style broadcast of ``v`` to ``shape`` as one broadcast_in_dim
    (size-1 dimensions are dropped first by a reshape)."""
    shape = tuple(int(s) for s in shape)
    if v.shape == shape:
        return v
    nd = len(shape)
    if v.ndim > nd:
        raise ValueError(f"cannot broadcast {v.shape} to {shape}")
    offset = nd - v.ndim
    keep_dims = []
    keep_shape = []
    for i, s in enumerate(v.shape):
        tgt = shape[offset + i]
        if s == tgt:
            keep_dims.append(offset + i)
            keep_shape.append(s)
        elif s != 1:
            raise ValueError(f"cannot broadcast {v.shape} to {shape}")
    src = v
    if tuple(keep_shape) != v.shape:
        src = ctx.build_op("reshape", [v], tuple(keep_shape), v.dtype)
    return ctx.build_op("broadcast_in_dim", [src], shape, v.dtype,
                        {"broadcast_dimensions": tuple(keep_dims)})


def broadcast_operands(ctx: HIPTraceContext, *vals: Value):
    shape = ()
    for v in vals:
        shape = broadcast_shapes(shape, v.shape)
    return [broadcast_to(ctx, v, shape) for v in vals]


def convert(ctx: HIPTraceContext, v: Value, dtype) -> Value:
    dtype = dt.canonical(dtype)
    if v.dtype == dtype:
        return v
    return ctx.build_op("convert", [v], v.shape, dtype)


def reshape(ctx: HIPTraceContext, v: Value, shape) -> Value:
    shape = tuple(int(s) for s in shape)
    if v.shape == shape:
        return v
    return ctx.build_op("reshape", [v], shape, v.dtype)
