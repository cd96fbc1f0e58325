"""Elementwise ops: binary arithmetic, comparisons, logical and unary ops.

Trace semantics follow the reference (nkipy/src/nkipy/core/ops/binary.py:
21-92 and unary.py:14-59): operands are promoted with the promotion rules,
broadcast NumPy-style, converted to the result dtype, then combined.
Transcendental unary ops on integer inputs compute in float32.
"""

from __future__ import annotations

import numpy as np

from nkipy_amd.core import dtypes as dt
from nkipy_amd.core.backend.hip import broadcast_operands, convert
from nkipy_amd.core.backend.promotion import find_common_type
from nkipy_amd.core.ops._helpers import ctx, val, wrap
from nkipy_amd.core.ops._registry import Op


def _binary_hip(opname):
    def impl(x, y, out=None, dtype=None, **kw):
        c = ctx()
        promoted = find_common_type(x, y)
        out_dtype = dt.canonical(dtype) if dtype is not None else promoted
        xv, yv = broadcast_operands(c, val(x, promoted), val(y, promoted))
        xv, yv = convert(c, xv, out_dtype), convert(c, yv, out_dtype)
        return wrap(c.build_op(opname, [xv, yv], xv.shape, out_dtype))

    return impl


def _make_binary(name, opname):
    op = Op(name)
    op.impl("hip")(_binary_hip(opname))
    return op


add = _make_binary("add", "add")
subtract = _make_binary("subtract", "subtract")
multiply = _make_binary("multiply", "multiply")
divide = _make_binary("divide", "divide")
power = _make_binary("power", "power")
maximum = _make_binary("maximum", "maximum")
minimum = _make_binary("minimum", "minimum")
bitwise_and = _make_binary("bitwise_and", "and")
bitwise_or = _make_binary("bitwise_or", "or")
bitwise_xor = _make_binary("bitwise_xor", "xor")
remainder = _make_binary("remainder", "remainder")
floor_divide = _make_binary("floor_divide", "floor_divide")
arctan2 = _make_binary("arctan2", "atan2")


def _compare_hip(direction):
    def impl(x, y, out=None, dtype=None, **kw):
        c = ctx()
        promoted = find_common_type(x, y)
        xv, yv = convert(c, val(x, promoted), promoted), convert(c, val(y, promoted), promoted)
        xv, yv = broadcast_operands(c, xv, yv)
        return wrap(c.build_op("compare", [xv, yv], xv.shape, dt.bool_,
                               {"comparison_direction": direction}))

    return impl


def _make_compare(name, direction):
    op = Op(name)
    op.impl("hip")(_compare_hip(direction))
    return op


equal = _make_compare("equal", "EQ")
not_equal = _make_compare("not_equal", "NE")
less = _make_compare("less", "LT")
less_equal = _make_compare("less_equal", "LE")
greater = _make_compare("greater", "GT")
greater_equal = _make_compare("greater_equal", "GE")


def _as_bool(c, x):
    v = val(x)
    if v.dtype == dt.bool_:
        return v
    zero = c.constant(0, v.dtype)
    zv, vv = broadcast_operands(c, zero, v)
    return c.build_op("compare", [vv, zv], vv.shape, dt.bool_, {"comparison_direction": "NE"})


def _logical_hip(opname):
    def impl(x, y, out=None, dtype=None, **kw):
        c = ctx()
        xv, yv = broadcast_operands(c, _as_bool(c, x), _as_bool(c, y))
        return wrap(c.build_op(opname, [xv, yv], xv.shape, dt.bool_))

    return impl


logical_and = Op("logical_and")
logical_and.impl("hip")(_logical_hip("and"))
logical_or = Op("logical_or")
logical_or.impl("hip")(_logical_hip("or"))
logical_xor = Op("logical_xor")
logical_xor.impl("hip")(_logical_hip("xor"))

logaddexp = Op("logaddexp")


@logaddexp.impl("hip")
def _logaddexp_hip(x, y, out=None, dtype=None, **kw):
    # log(e^x + e^y) = max(x, y) + log1p(exp(-|x - y|))
    m = maximum(x, y)
    d = abs_(subtract(x, y))
    return add(m, log1p(exp(negative(d))))


# ---------------------------------------------------------------------------
# unary
# ---------------------------------------------------------------------------
_FLOAT_ONLY = {
    "exponential", "log", "sqrt", "rsqrt", "sine", "cosine", "tan", "atan", "tanh",
    "log_plus_one", "exponential_minus_one", "log2", "logistic",
}


def _unary_hip(opname, out_bool=False):
    def impl(x, out=None, dtype=None, **kw):
        c = ctx()
        v = val(x)
        if opname in _FLOAT_ONLY and not dt.is_float(v.dtype):
            v = convert(c, v, dt.float32)
        rdt = dt.bool_ if out_bool else v.dtype
        r = c.build_op(opname, [v], v.shape, rdt)
        if dtype is not None:
            r = convert(c, r, dtype)
        return wrap(r)

    return impl


def _make_unary(name, opname, out_bool=False):
    op = Op(name)
    op.impl("hip")(_unary_hip(opname, out_bool))
    return op


abs_ = _make_unary("abs", "abs")
exp = _make_unary("exp", "exponential")
log = _make_unary("log", "log")
sqrt = _make_unary("sqrt", "sqrt")
negative = _make_unary("negative", "negate")
sin = _make_unary("sin", "sine")
cos = _make_unary("cos", "cosine")
tan = _make_unary("tan", "tan")
arctan = _make_unary("arctan", "atan")
tanh = _make_unary("tanh", "tanh")
ceil = _make_unary("ceil", "ceil")
floor = _make_unary("floor", "floor")
rint = _make_unary("rint", "round_nearest_even")
trunc = _make_unary("trunc", "trunc")
sign = _make_unary("sign", "sign")
log1p = _make_unary("log1p", "log_plus_one")
log2 = _make_unary("log2", "log2")
expm1 = _make_unary("expm1", "exponential_minus_one")
isnan = _make_unary("isnan", "is_nan", out_bool=True)
isfinite = _make_unary("isfinite", "is_finite", out_bool=True)
invert = _make_unary("invert", "not")
bitwise_not = invert

square = Op("square")


@square.impl("hip")
def _square_hip(x, out=None, dtype=None, **kw):
    return multiply(x, x, dtype=dtype)


reciprocal = Op("reciprocal")


@reciprocal.impl("hip")
def _reciprocal_hip(x, out=None, dtype=None, **kw):
    return divide(1.0 if dt.is_float(val(x).dtype) else 1, x, dtype=dtype)


logical_not = Op("logical_not")


@logical_not.impl("hip")
def _logical_not_hip(x, out=None, **kw):
    c = ctx()
    b = _as_bool(c, x)
    return wrap(c.build_op("not", [b], b.shape, dt.bool_))


round_ = Op("round")


@round_.impl("hip")
def _round_hip(x, decimals=0, out=None):
    if decimals == 0:
        return rint(x)
    scale = 10.0 ** decimals
    return divide(rint(multiply(x, scale)), scale)


clip = Op("clip")


@clip.impl("hip")
def _clip_hip(x, a_min=None, a_max=None, out=None, **kw):
    if a_min is None and "min" in kw:
        a_min = kw["min"]
    if a_max is None and "max" in kw:
        a_max = kw["max"]
    r = x
    if a_min is not None:
        r = maximum(r, a_min)
    if a_max is not None:
        r = minimum(r, a_max)
    return r
