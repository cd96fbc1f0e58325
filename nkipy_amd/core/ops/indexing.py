"""Indexing ops: where, static_slice, take, take_along_axis, put_along_axis,
dynamic_update_slice, scatter_along_axis, scatter_strided.

Semantics follow the reference (nkipy/src/nkipy/core/ops/indexing.py:17-112
for ``where``, 623-686 for ``static_slice``); index arrays are int32 on the
device.
"""

from __future__ import annotations

import numpy as np

from nkipy_amd.core import dtypes as dt
from nkipy_amd.core.backend.hip import broadcast_operands, broadcast_to, convert, reshape
from nkipy_amd.core.backend.promotion import find_common_type
from nkipy_amd.core.ops import elementwise as ew
from nkipy_amd.core.ops._helpers import ctx, norm_axis, val, wrap
from nkipy_amd.core.ops._registry import Op
from nkipy_amd.core.tensor import NKIPyTensorRef

where = Op("where")


@where.impl("hip")
def _where_hip(condition, x=None, y=None):
    if x is None or y is None:
        raise NotImplementedError("np.where(condition) without x and y is not supported")
    c = ctx()
    if isinstance(x, (int, float)) and isinstance(y, (int, float)) and not isinstance(x, bool):
        # two Python scalars: NumPy's default types, narrowed to 32 bits
        dtype = dt.float32 if isinstance(x, float) or isinstance(y, float) else dt.int32
    else:
        dtype = find_common_type(x, y)
    cond = ew._as_bool(c, condition) if isinstance(condition, NKIPyTensorRef) else \
        c.constant(np.asarray(condition, dtype=bool), dt.bool_)
    pv, xv, yv = broadcast_operands(c, cond, convert(c, val(x, dtype), dtype),
                                    convert(c, val(y, dtype), dtype))
    return wrap(c.build_op("select", [pv, xv, yv], xv.shape, dtype))


static_slice = Op("static_slice")


@static_slice.impl("hip")
def _static_slice_hip(x, start_indices, limit_indices, strides, squeeze_dims=()):
    c = ctx()
    v = val(x)
    start = tuple(int(s) for s in start_indices)
    limit = tuple(int(s) for s in limit_indices)
    strides = tuple(int(s) for s in strides)
    shape = tuple(max(0, -(-(b - a) // s)) for a, b, s in zip(start, limit, strides))
    if start == (0,) * v.ndim and limit == v.shape and strides == (1,) * v.ndim:
        r = v
    else:
        r = c.build_op("slice", [v], shape, v.dtype,
                       {"start_indices": start, "limit_indices": limit, "strides": strides})
    if squeeze_dims:
        r = reshape(c, r, tuple(s for i, s in enumerate(shape) if i not in set(squeeze_dims)))
    return wrap(r)


def _index_value(c, idx):
    if isinstance(idx, NKIPyTensorRef):
        v = idx.backend_tensor
        if not dt.is_int(v.dtype):
            raise TypeError("index tensors must have an integer dtype")
        return convert(c, v, dt.int32)
    arr = np.asarray(idx)
    if not np.issubdtype(arr.dtype, np.integer):
        raise TypeError("index arrays must have an integer dtype")
    return c.constant(arr.astype(np.int32), dt.int32)


take = Op("take")


@take.impl("hip")
def _take_hip(a, indices, axis=None, out=None, mode=None):
    c = ctx()
    v = val(a)
    if axis is None:
        v = reshape(c, v, (v.size,))
        axis = 0
    ax = norm_axis(axis, v.ndim)[0]
    if isinstance(indices, (int, np.integer)):
        idx = int(indices)
        start = [0] * v.ndim
        limit = list(v.shape)
        start[ax] = idx + v.shape[ax] if idx < 0 else idx
        limit[ax] = start[ax] + 1
        return _static_slice_hip(wrap(v), start, limit, [1] * v.ndim, [ax])
    iv = _index_value(c, indices)
    shape = v.shape[:ax] + iv.shape + v.shape[ax + 1:]
    return wrap(c.build_op("take", [v, iv], shape, v.dtype, {"axis": ax}))


take_along_axis = Op("take_along_axis")


@take_along_axis.impl("hip")
def _take_along_axis_hip(arr, indices, axis):
    c = ctx()
    v = val(arr)
    iv = _index_value(c, indices)
    if axis is None:  # NumPy: along the flattened array, 1-D indices
        if iv.ndim != 1:
            raise ValueError("with axis=None the indices must be 1-D")
        v = reshape(c, v, (v.size,))
        axis = 0
    ax = norm_axis(axis, v.ndim)[0]
    if iv.ndim != v.ndim:
        raise ValueError("indices and arr must have the same number of dimensions")
    # NumPy broadcasts the non-axis dimensions of indices against arr
    bshape = tuple(iv.shape[i] if i == ax else max(iv.shape[i], v.shape[i]) for i in range(v.ndim))
    iv = broadcast_to(c, iv, bshape)
    if any(v.shape[i] != bshape[i] for i in range(v.ndim) if i != ax):
        tgt = tuple(v.shape[i] if i == ax else bshape[i] for i in range(v.ndim))
        v = broadcast_to(c, v, tgt)
    return wrap(c.build_op("take_along_axis", [v, iv], bshape, v.dtype, {"axis": ax}))


put_along_axis = Op("put_along_axis")


@put_along_axis.impl("hip")
def _put_along_axis_hip(arr, indices, values, axis):
    c = ctx()
    v = val(arr)
    iv = _index_value(c, indices)
    shape = v.shape
    if axis is None:  # NumPy: into the flattened array, 1-D indices
        if iv.ndim != 1:
            raise ValueError("with axis=None the indices must be 1-D")
        v = reshape(c, v, (v.size,))
        axis = 0
    ax = norm_axis(axis, v.ndim)[0]
    vals = convert(c, broadcast_to(c, val(values, v.dtype), iv.shape), v.dtype)
    out = c.build_op("put_along_axis", [v, iv, vals], v.shape, v.dtype, {"axis": ax})
    return wrap(reshape(c, out, shape) if out.shape != shape else out)


dynamic_update_slice = Op("dynamic_update_slice")


@dynamic_update_slice.impl("hip")
def _dynamic_update_slice_hip(operand, update, start_indices, update_shape):
    c = ctx()
    v = val(operand)
    update_shape = tuple(int(s) for s in update_shape)
    u = val(update, v.dtype)
    u = convert(c, u, v.dtype)
    if u.shape != update_shape:
        # allow NumPy broadcasting of the value, including a squeezed int index
        try:
            u = broadcast_to(c, u, update_shape)
        except ValueError:
            squeezed = tuple(s for s in update_shape if s != 1)
            u = broadcast_to(c, reshape(c, u, tuple(s for s in u.shape if s != 1)), squeezed) \
                if u.size != 1 else broadcast_to(c, u, update_shape)
            u = reshape(c, u, update_shape)
    start = tuple(int(s) for s in start_indices)
    for d in range(v.ndim):
        if start[d] < 0 or start[d] + update_shape[d] > v.shape[d]:
            raise IndexError(f"slice assignment out of bounds on axis {d}")
    return wrap(c.build_op("dynamic_update_slice", [v, u], v.shape, v.dtype, {"start": start}))


scatter_along_axis = Op("scatter_along_axis")


@scatter_along_axis.impl("hip")
def _scatter_along_axis_hip(operand, indices, updates, axis):
    """operand[..., indices[i], ...] = updates[..., i, ...] along ``axis``."""
    c = ctx()
    v = val(operand)
    ax = norm_axis(axis, v.ndim)[0]
    iv = _index_value(c, indices)
    if iv.ndim == 0:
        iv = reshape(c, iv, (1,))
    iv = reshape(c, iv, (iv.size,))
    ushape = v.shape[:ax] + (iv.shape[0],) + v.shape[ax + 1:]
    u = convert(c, val(updates, v.dtype), v.dtype)
    if u.shape != ushape:
        if u.size == int(np.prod(ushape)):
            u = reshape(c, u, ushape)
        else:
            u = broadcast_to(c, u, ushape)
    return wrap(c.build_op("scatter_along_axis", [v, iv, u], v.shape, v.dtype, {"axis": ax}))


scatter_strided = Op("scatter_strided")


@scatter_strided.impl("hip")
def _scatter_strided_hip(operand, updates, indices_per_dim):
    c = ctx()
    v = val(operand)
    ushape = tuple(len(ix) for ix in indices_per_dim)
    u = convert(c, val(updates, v.dtype), v.dtype)
    if u.shape != ushape:
        u = broadcast_to(c, u, ushape) if u.size != int(np.prod(ushape)) else reshape(c, u, ushape)
    return wrap(c.build_op("scatter_strided", [v, u], v.shape, v.dtype,
                           {"indices_per_dim": tuple(tuple(int(i) for i in ix) for ix in indices_per_dim)}))
