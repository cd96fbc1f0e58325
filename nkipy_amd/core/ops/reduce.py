"""Reductions.

Semantics follow the reference (nkipy/src/nkipy/core/ops/reduce.py:14-157):
the result keeps the input dtype, ``keepdims`` is a reshape after the
reduction, ``mean`` is ``sum / count`` with the count as a weak float.  The
IR additionally records the accumulation dtype: floating reductions
accumulate in fp32 whatever the storage dtype.
"""

from __future__ import annotations

import builtins

import numpy as np

from nkipy_amd.core import dtypes as dt
from nkipy_amd.core.backend.hip import convert, reshape
from nkipy_amd.core.ops import elementwise as ew
from nkipy_amd.core.ops._helpers import acc_dtype, ctx, norm_axis, val, wrap
from nkipy_amd.core.ops._registry import Op


def _reduce(x, computation, axis=None, dtype=None, keepdims=False, initial=None, where=None):
    if where is not None:
        raise NotImplementedError("reductions with where= are not supported")
    c = ctx()
    v = val(x)
    if dtype is not None:
        v = convert(c, v, dtype)
    elif computation in ("add", "multiply") and (v.dtype == dt.bool_ or (dt.is_int(v.dtype) and v.dtype.itemsize < 4)):
        # NumPy sums / products of bool and small integers in the default
        # integer type (narrowed to 32 bits here)
        v = convert(c, v, dt.uint32 if v.dtype.kind == "u" else dt.int32)
    if computation in ("and", "or") and v.dtype != dt.bool_:
        v = ew._as_bool(c, v)
    dims = norm_axis(axis, v.ndim)
    out_shape = tuple(s for i, s in enumerate(v.shape) if i not in dims)
    r = c.build_op("reduce", [v], out_shape, v.dtype,
                   {"dimensions": dims, "computation": computation,
                    "acc_dtype": acc_dtype(v.dtype)})
    if keepdims:
        r = reshape(c, r, tuple(1 if i in dims else s for i, s in enumerate(v.shape)))
    out = wrap(r)
    if initial is not None:
        combine = {"add": ew.add, "maximum": ew.maximum, "minimum": ew.minimum,
                   "multiply": ew.multiply}[computation]
        out = combine(out, initial)
    return out


def _make(name, computation):
    op = Op(name)

    @op.impl("hip")
    def impl(x, axis=None, out=None, dtype=None, keepdims=False, initial=None, where=None):
        return _reduce(x, computation, axis, dtype, keepdims, initial, where)

    return op


sum = _make("sum", "add")
max = _make("max", "maximum")
min = _make("min", "minimum")
prod = _make("prod", "multiply")


def _count(shape, axis):
    n = 1
    for a in norm_axis(axis, len(shape)):
        n *= shape[a]
    return n


mean = Op("mean")


@mean.impl("hip")
def _mean_hip(x, axis=None, dtype=None, out=None, keepdims=False, where=None):
    v = val(x)
    if dtype is not None:
        x = wrap(convert(ctx(), v, dtype))
    elif not dt.is_float(v.dtype):
        x = wrap(convert(ctx(), v, dt.float32))
    s = _reduce(x, "add", axis, None, keepdims, None, where)
    return ew.divide(s, float(_count(v.shape, axis)))


var = Op("var")


@var.impl("hip")
def _var_hip(x, axis=None, dtype=None, out=None, ddof=0, keepdims=False, where=None):
    v = val(x)
    if dtype is not None:
        x = wrap(convert(ctx(), v, dtype))
    elif not dt.is_float(v.dtype):
        x = wrap(convert(ctx(), v, dt.float32))
    m = _mean_hip(x, axis=axis, keepdims=True)
    d = ew.subtract(x, m)
    s = _reduce(ew.multiply(d, d), "add", axis, None, keepdims)
    n = _count(v.shape, axis) - ddof
    return ew.divide(s, float(builtins.max(n, 0)))


std = Op("std")


@std.impl("hip")
def _std_hip(x, axis=None, dtype=None, out=None, ddof=0, keepdims=False, where=None):
    return ew.sqrt(_var_hip(x, axis=axis, dtype=dtype, ddof=ddof, keepdims=keepdims))


any = Op("any")


@any.impl("hip")
def _any_hip(x, axis=None, out=None, keepdims=False, where=None):
    return _reduce(x, "or", axis, None, keepdims)


all = Op("all")


@all.impl("hip")
def _all_hip(x, axis=None, out=None, keepdims=False, where=None):
    return _reduce(x, "and", axis, None, keepdims)


count_nonzero = Op("count_nonzero")


@count_nonzero.impl("hip")
def _count_nonzero_hip(x, axis=None, keepdims=False):
    c = ctx()
    b = convert(c, ew._as_bool(c, x), dt.int32)
    return _reduce(wrap(b), "add", axis, None, keepdims)


def _make_arg(name, kind):
    op = Op(name)

    @op.impl("hip")
    def impl(x, axis=None, out=None, keepdims=False):
        c = ctx()
        v = val(x)
        if axis is None:
            v = reshape(c, v, (v.size,))
            ax = 0
        else:
            ax = norm_axis(axis, v.ndim)[0]
        out_shape = tuple(s for i, s in enumerate(v.shape) if i != ax)
        r = c.build_op(kind, [v], out_shape, dt.int32, {"axis": ax})
        if keepdims:
            if axis is None:
                r = reshape(c, r, (1,) * val(x).ndim)
            else:
                r = reshape(c, r, tuple(1 if i == ax else s for i, s in enumerate(v.shape)))
        return wrap(r)

    return op


argmax = _make_arg("argmax", "argmax")
argmin = _make_arg("argmin", "argmin")

cumsum = Op("cumsum")


@cumsum.impl("hip")
def _cumsum_hip(x, axis=None, dtype=None, out=None):
    c = ctx()
    v = val(x)
    if dtype is not None:
        v = convert(c, v, dtype)
    if axis is None:
        v = reshape(c, v, (v.size,))
        ax = 0
    else:
        ax = norm_axis(axis, v.ndim)[0]
    return wrap(c.build_op("cumsum", [v], v.shape, v.dtype,
                           {"axis": ax, "acc_dtype": acc_dtype(v.dtype)}))
