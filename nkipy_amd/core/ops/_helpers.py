"""Shared helpers of the ``"hip"`` op implementations."""

from __future__ import annotations

import numpy as np

from nkipy_amd.core import dtypes as dt
from nkipy_amd.core.backend.hip import get_hip_context
from nkipy_amd.core.backend.ir import Value
from nkipy_amd.core.tensor import NKIPyTensorRef


def ctx():
    return get_hip_context()


def val(x, dtype=None) -> Value:
    """IR value of a traced tensor, a scalar or a concrete array (constant)."""
    if isinstance(x, NKIPyTensorRef):
        return x.backend_tensor
    if isinstance(x, Value):
        return x
    c = ctx()
    if isinstance(x, np.ndarray) and dtype is None and x.dtype == dt.float64:
        return c.constant(x, dt.float32)
    return c.constant(x, dtype)


def wrap(v: Value) -> NKIPyTensorRef:
    return NKIPyTensorRef(v)


def is_traced(x) -> bool:
    return isinstance(x, NKIPyTensorRef)


def norm_axis(axis, ndim: int):
    """Tuple of non-negative axes (all axes for None)."""
    if axis is None:
        return tuple(range(ndim))
    if isinstance(axis, (list, tuple)):
        axes = tuple(int(a) + ndim if int(a) < 0 else int(a) for a in axis)
    else:
        a = int(axis)
        axes = (a + ndim if a < 0 else a,)
    for a in axes:
        if not 0 <= a < max(ndim, 1):
            raise np.exceptions.AxisError(f"axis {a} is out of bounds for array of dimension {ndim}")
    return axes


def acc_dtype(d) -> np.dtype:
    """Accumulator dtype for reductions and dots over storage dtype ``d``."""
    d = dt.canonical(d)
    if dt.is_float(d):
        return dt.float32
    if d == dt.bool_:
        return dt.int32
    if d in (dt.int64, dt.uint64):
        return d
    return dt.int32 if d.kind == "i" or d.itemsize < 4 else d


def shape_of(x):
    if isinstance(x, (NKIPyTensorRef, np.ndarray)):
        return tuple(x.shape)
    return ()
