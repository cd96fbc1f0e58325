"""Shape and layout ops: reshape, transpose, expand/squeeze, concatenate,
split, stack, repeat, tile, pad, flip, roll, diff, broadcast_to, copy,
copyto, astype.

Semantics follow NumPy and the reference's lowering
(nkipy/src/nkipy/core/ops/transform.py:14-79, 181-313, 402-498):
``split`` is a set of static slices, ``astype`` to the same dtype is a
``copy``, ``repeat``/``tile`` are broadcast + reshape.
"""

from __future__ import annotations

import numpy as np

from nkipy_amd.core import dtypes as dt
from nkipy_amd.core.backend.hip import broadcast_to as _bcast
from nkipy_amd.core.backend.hip import convert, reshape as _reshape
from nkipy_amd.core.ops._helpers import ctx, is_traced, norm_axis, val, wrap
from nkipy_amd.core.ops._registry import Op
from nkipy_amd.core.tensor import NKIPyTensorRef


def _resolve_shape(shape, size):
    if isinstance(shape, (int, np.integer)):
        shape = (int(shape),)
    shape = [int(s) for s in shape]
    if shape.count(-1) > 1:
        raise ValueError("can only specify one unknown dimension")
    if -1 in shape:
        known = 1
        for s in shape:
            if s != -1:
                known *= s
        if known == 0 or size % known:
            raise ValueError(f"cannot reshape array of size {size} into shape {tuple(shape)}")
        shape[shape.index(-1)] = size // known
    n = 1
    for s in shape:
        n *= s
    if n != size:
        raise ValueError(f"cannot reshape array of size {size} into shape {tuple(shape)}")
    return tuple(shape)


reshape = Op("reshape")


@reshape.impl("hip")
def _reshape_hip(x, newshape=None, order="C", shape=None):
    if order != "C":
        raise NotImplementedError("only C-order reshape is supported")
    if newshape is None:
        newshape = shape
    v = val(x)
    return wrap(_reshape(ctx(), v, _resolve_shape(newshape, v.size)))


transpose = Op("transpose")


@transpose.impl("hip")
def _transpose_hip(x, axes=None):
    v = val(x)
    if axes is None:
        perm = tuple(reversed(range(v.ndim)))
    else:
        perm = norm_axis(tuple(axes), v.ndim)
        if sorted(perm) != list(range(v.ndim)):
            raise ValueError("axes don't match array")
    if perm == tuple(range(v.ndim)):
        return wrap(v)
    shape = tuple(v.shape[p] for p in perm)
    return wrap(ctx().build_op("transpose", [v], shape, v.dtype, {"permutation": perm}))


swapaxes = Op("swapaxes")


@swapaxes.impl("hip")
def _swapaxes_hip(x, axis1, axis2):
    nd = val(x).ndim
    a, b = norm_axis(axis1, nd)[0], norm_axis(axis2, nd)[0]
    perm = list(range(nd))
    perm[a], perm[b] = perm[b], perm[a]
    return _transpose_hip(x, perm)


expand_dims = Op("expand_dims")


@expand_dims.impl("hip")
def _expand_dims_hip(x, axis):
    v = val(x)
    axes = axis if isinstance(axis, (list, tuple)) else (axis,)
    nd = v.ndim + len(axes)
    axes = sorted(a + nd if a < 0 else a for a in axes)
    shape = list(v.shape)
    for a in axes:
        shape.insert(a, 1)
    return wrap(_reshape(ctx(), v, tuple(shape)))


squeeze = Op("squeeze")


@squeeze.impl("hip")
def _squeeze_hip(x, axis=None):
    v = val(x)
    if axis is None:
        shape = tuple(s for s in v.shape if s != 1)
    else:
        axes = norm_axis(axis, v.ndim)
        for a in axes:
            if v.shape[a] != 1:
                raise ValueError("cannot select an axis to squeeze out which has size not equal to one")
        shape = tuple(s for i, s in enumerate(v.shape) if i not in axes)
    return wrap(_reshape(ctx(), v, shape))


broadcast_to = Op("broadcast_to")


@broadcast_to.impl("hip")
def _broadcast_to_hip(x, shape):
    if isinstance(shape, (int, np.integer)):
        shape = (int(shape),)
    return wrap(_bcast(ctx(), val(x), tuple(int(s) for s in shape)))


copy = Op("copy")


@copy.impl("hip")
def _copy_hip(x, order="K", subok=False):
    v = val(x)
    return wrap(ctx().build_op("copy", [v], v.shape, v.dtype))


astype = Op("astype")


@astype.impl("hip")
def _astype_hip(x, dtype, copy=True):
    v = val(x)
    d = dt.canonical(dtype)
    if d == dt.float64:
        d = dt.float32
    elif d == dt.int64:
        d = dt.int32
    if d == v.dtype:
        return wrap(ctx().build_op("copy", [v], v.shape, v.dtype))
    return wrap(convert(ctx(), v, d))


concatenate = Op("concatenate")


@concatenate.impl("hip")
def _concatenate_hip(arrays, axis=0, out=None, dtype=None):
    from nkipy_amd.core.backend.promotion import find_common_type

    arrays = list(arrays)
    if not arrays:
        raise ValueError("need at least one array to concatenate")
    common = arrays[0]
    for a in arrays[1:]:
        common = _Typed(find_common_type(common, a))
    target = dt.canonical(dtype) if dtype is not None else dt.canonical(common.dtype)
    c = ctx()
    vals = [convert(c, val(a, target), target) for a in arrays]
    if axis is None:
        vals = [_reshape(c, v, (v.size,)) for v in vals]
        axis = 0
    ax = norm_axis(axis, vals[0].ndim)[0]
    shape = list(vals[0].shape)
    for v in vals[1:]:
        if v.ndim != len(shape) or any(v.shape[i] != shape[i] for i in range(len(shape)) if i != ax):
            raise ValueError("all the input array dimensions except for the concatenation axis must match exactly")
    shape[ax] = sum(v.shape[ax] for v in vals)
    if len(vals) == 1:
        return wrap(vals[0])
    return wrap(c.build_op("concatenate", vals, tuple(shape), target, {"dimension": ax}))


class _Typed:
    def __init__(self, dtype):
        self.dtype = dtype


stack = Op("stack")


@stack.impl("hip")
def _stack_hip(arrays, axis=0, out=None, dtype=None):
    arrays = list(arrays)
    nd = val(arrays[0]).ndim + 1
    ax = axis + nd if axis < 0 else axis
    return _concatenate_hip([_expand_dims_hip(a, ax) for a in arrays], axis=ax, dtype=dtype)


split = Op("split")


@split.impl("hip")
def _split_hip(x, indices_or_sections, axis=0):
    from nkipy_amd.core.ops.indexing import static_slice

    v = val(x)
    ax = norm_axis(axis, v.ndim)[0]
    n = v.shape[ax]
    if isinstance(indices_or_sections, (int, np.integer)):
        k = int(indices_or_sections)
        if n % k:
            raise ValueError("array split does not result in an equal division")
        bounds = [i * (n // k) for i in range(k + 1)]
    else:
        bounds = [0] + [min(max(int(i), 0), n) for i in indices_or_sections] + [n]
    parts = []
    for a, b in zip(bounds[:-1], bounds[1:]):
        start = [0] * v.ndim
        limit = list(v.shape)
        start[ax], limit[ax] = a, max(a, b)
        parts.append(static_slice(x, start, limit, [1] * v.ndim, []))
    return parts


repeat = Op("repeat")


@repeat.impl("hip")
def _repeat_hip(x, repeats, axis=None):
    c = ctx()
    v = val(x)
    if axis is None:
        v = _reshape(c, v, (v.size,))
        axis = 0
    ax = norm_axis(axis, v.ndim)[0]
    if not isinstance(repeats, (int, np.integer)):
        raise NotImplementedError("repeat with per-element repeat counts is not supported")
    r = int(repeats)
    # (.., n, ..) -> (.., n, 1, ..) -> broadcast (.., n, r, ..) -> (.., n*r, ..)
    s1 = v.shape[:ax + 1] + (1,) + v.shape[ax + 1:]
    s2 = v.shape[:ax + 1] + (r,) + v.shape[ax + 1:]
    out = v.shape[:ax] + (v.shape[ax] * r,) + v.shape[ax + 1:]
    b = _bcast(c, _reshape(c, v, s1), s2)
    return wrap(_reshape(c, b, out))


tile = Op("tile")


@tile.impl("hip")
def _tile_hip(x, reps):
    c = ctx()
    v = val(x)
    reps = (reps,) if isinstance(reps, (int, np.integer)) else tuple(reps)
    nd = max(v.ndim, len(reps))
    shape = (1,) * (nd - v.ndim) + v.shape
    reps = (1,) * (nd - len(reps)) + reps
    # (s0, s1, ..) -> (1, s0, 1, s1, ..) -> broadcast (r0, s0, r1, s1, ..)
    s1, s2 = [], []
    for s, r in zip(shape, reps):
        s1 += [1, s]
        s2 += [r, s]
    b = _bcast(c, _reshape(c, v, tuple(s1)), tuple(s2))
    return wrap(_reshape(c, b, tuple(s * r for s, r in zip(shape, reps))))


pad = Op("pad")


def _edge_pad(c, v, low, high):
    """np.pad(mode="edge"): per axis, the first / last slice broadcast over
    the padding, concatenated around the operand."""
    for ax in range(v.ndim):
        lo, hi = low[ax], high[ax]
        if lo == 0 and hi == 0:
            continue
        n = v.shape[ax]

        def edge(i, count, v=v, ax=ax):
            start = [0] * v.ndim
            limit = list(v.shape)
            start[ax], limit[ax] = i, i + 1
            one = tuple(b - a for a, b in zip(start, limit))
            sl = c.build_op("slice", [v], one, v.dtype, {"start_indices": tuple(start),
                                                         "limit_indices": tuple(limit),
                                                         "strides": (1,) * v.ndim})
            tgt = list(v.shape)
            tgt[ax] = count
            return _bcast(c, sl, tuple(tgt))

        parts = ([edge(0, lo)] if lo else []) + [v] + ([edge(n - 1, hi)] if hi else [])
        shape = list(v.shape)
        shape[ax] = n + lo + hi
        v = c.build_op("concatenate", parts, tuple(shape), v.dtype, {"dimension": ax})
    return v


@pad.impl("hip")
def _pad_hip(x, pad_width, mode="constant", constant_values=0, **kw):
    if mode not in ("constant", "edge"):
        raise NotImplementedError(f"pad mode '{mode}' is not supported")
    c = ctx()
    v = val(x)
    pw = np.broadcast_to(np.asarray(pad_width, dtype=np.int64), (v.ndim, 2))
    low = tuple(int(a) for a in pw[:, 0])
    high = tuple(int(b) for b in pw[:, 1])
    if mode == "edge":
        if v.size == 0:
            raise ValueError("edge padding of an empty array")
        return wrap(_edge_pad(c, v, low, high))
    shape = tuple(s + a + b for s, a, b in zip(v.shape, low, high))
    pv = c.constant(constant_values, v.dtype)
    return wrap(c.build_op("pad", [v, pv], shape, v.dtype,
                           {"low": low, "high": high, "interior": (0,) * v.ndim}))


flip = Op("flip")


@flip.impl("hip")
def _flip_hip(x, axis=None):
    v = val(x)
    axes = norm_axis(axis, v.ndim)
    return wrap(ctx().build_op("reverse", [v], v.shape, v.dtype, {"dimensions": axes}))


roll = Op("roll")


@roll.impl("hip")
def _roll_hip(x, shift, axis=None):
    from nkipy_amd.core.ops.indexing import static_slice

    c = ctx()
    v = val(x)
    if axis is None:
        flat = wrap(_reshape(c, v, (v.size,)))
        return _reshape_hip(_roll_hip(flat, shift, 0), v.shape)
    shifts = shift if isinstance(shift, (list, tuple)) else [shift]
    axes = axis if isinstance(axis, (list, tuple)) else [axis]
    out = x
    for s, a in zip(shifts, axes):
        ov = val(out)
        a = norm_axis(a, ov.ndim)[0]
        n = ov.shape[a]
        s = int(s) % n if n else 0
        if s == 0:
            continue
        lo = [0] * ov.ndim
        hi = list(ov.shape)
        st = [1] * ov.ndim
        l1, h1 = list(lo), list(hi)
        l1[a] = n - s
        l2, h2 = list(lo), list(hi)
        h2[a] = n - s
        out = _concatenate_hip([static_slice(out, l1, h1, st, []),
                                static_slice(out, l2, h2, st, [])], axis=a)
    return out


diff = Op("diff")


@diff.impl("hip")
def _diff_hip(x, n=1, axis=-1):
    from nkipy_amd.core.ops import elementwise as ew
    from nkipy_amd.core.ops.indexing import static_slice

    out = x
    for _ in range(n):
        v = val(out)
        a = norm_axis(axis, v.ndim)[0]
        lo1, hi1 = [0] * v.ndim, list(v.shape)
        lo2, hi2 = [0] * v.ndim, list(v.shape)
        lo1[a] = 1
        hi2[a] = v.shape[a] - 1
        st = [1] * v.ndim
        out = ew.subtract(static_slice(out, lo1, hi1, st, []), static_slice(out, lo2, hi2, st, []))
    return out


copyto = Op("copyto")


@copyto.impl("hip")
def _copyto_hip(dst, src, casting="same_kind", where=None):
    if where is not None:
        raise NotImplementedError("copyto with where= is not supported")
    if not isinstance(dst, NKIPyTensorRef):
        raise TypeError("copyto destination must be a traced tensor")
    dst[...] = src
