"""Implicit dtype promotion of binary operands.

Restates the reference's promotion rules (nkipy/src/nkipy/core/backend/hlo.py:
1062-1237 table, 1285-1358 lookup, 1361-1395 scalar dtypes).  The rules are
kept identical on purpose: a kernel must trace to the same dtypes here as on
the reference so that both backends agree on every intermediate type.

Rules, as data rather than an enumerated table:
* Python ``int`` / ``float`` are *weak*: they adopt the other operand's type
  (weak float + integer -> float32; bool + weak int -> int32,
  bool + weak float -> float32).
* bool defers to everything.
* integers: same signedness -> wider; mixed -> the smallest signed type that
  holds both, float32 when one side is uint64.
* integer + float -> the float.
* float16 + bfloat16 -> float32; otherwise the wider float.
* fp8 (e4m3fn, e4m3, e5m2) defers to weak scalars, bool and integers, and
  yields to wider floats; two different fp8 variants do not mix.
* float64 is rejected.
"""

from __future__ import annotations

import numpy as np

from nkipy_amd.core import dtypes as dt


class _Weak:
    def __init__(self, name):
        self.name = name

    def __repr__(self):
        return self.name


WEAK_INT = _Weak("weak_int")
WEAK_FLOAT = _Weak("weak_float")

_SIGNED = [dt.int8, dt.int16, dt.int32, dt.int64]
_UNSIGNED = [dt.uint8, dt.uint16, dt.uint32, dt.uint64]


def type_key(val):
    """Promotion key of an operand: WEAK_INT/WEAK_FLOAT or an np.dtype."""
    if isinstance(val, bool):
        return dt.bool_
    if isinstance(val, int):
        return WEAK_INT
    if isinstance(val, float):
        return WEAK_FLOAT
    if isinstance(val, (np.bool_, np.integer, np.floating)):
        return np.dtype(type(val))
    d = getattr(val, "dtype", None)
    if d is not None:
        return dt.canonical(d)
    raise ValueError(f"Unsupported or unrecognized type: {type(val)}")


def _key_name(k) -> str:
    return k.name if isinstance(k, _Weak) else dt.name(k)


def _promote_pair(a, b):
    """Result for two distinct keys, or None when no implicit path exists."""
    # weak scalars
    if isinstance(a, _Weak) and isinstance(b, _Weak):
        return None
    if isinstance(b, _Weak):
        a, b = b, a
    if isinstance(a, _Weak):
        if b == dt.bool_:
            return dt.int32 if a is WEAK_INT else dt.float32
        if dt.is_int(b):
            return b if a is WEAK_INT else dt.float32
        return b  # floats, bf16, fp8 keep their type
    # bool
    if a == dt.bool_:
        return b
    if b == dt.bool_:
        return a
    a_fp8, b_fp8 = dt.is_fp8(a), dt.is_fp8(b)
    if a_fp8 and b_fp8:
        return None
    if a_fp8 or b_fp8:
        f8, other = (a, b) if a_fp8 else (b, a)
        if dt.is_int(other):
            return f8
        if other in (dt.float16, dt.float32, dt.bfloat16):
            return other
        return None
    a_int, b_int = dt.is_int(a), dt.is_int(b)
    if a_int and b_int:
        if (a in _SIGNED) == (b in _SIGNED):
            return a if a.itemsize >= b.itemsize else b
        s, u = (a, b) if a in _SIGNED else (b, a)
        if u == dt.uint64:
            return dt.float32
        need = 2 * u.itemsize
        return s if s.itemsize >= need else np.dtype(f"int{8 * need}")
    if a_int:
        return b
    if b_int:
        return a
    # two floats
    if {a, b} == {dt.float16, dt.bfloat16}:
        return dt.float32
    if dt.float32 in (a, b):
        return dt.float32
    return None


def lookup(t0, t1):
    if t0 == dt.float64 or t1 == dt.float64:
        raise TypeError(
            "Unsupported dtype: float64. Use .astype(dtype) to convert to a supported type."
        )
    if not isinstance(t0, _Weak) and t0 == t1:
        return t0
    return _promote_pair(t0, t1)


def find_common_type(x, y) -> np.dtype:
    t0, t1 = type_key(x), type_key(y)
    r = lookup(t0, t1)
    if r is None:
        raise TypeError(
            f"No implicit dtype promotion path for {_key_name(t0)} and "
            f"{_key_name(t1)}. Use .astype(dtype) explicitly."
        )
    return dt.canonical(r)


def scalar_dtype(scalar) -> np.dtype:
    """Strong dtype of a scalar constant (64-bit narrowed, float64 rejected)."""
    if isinstance(scalar, (bool, np.bool_)):
        return dt.bool_
    if isinstance(scalar, np.floating) and isinstance(scalar, np.float64):
        raise ValueError(
            "float64 is not supported on the device. Use .astype(np.float32) to convert explicitly."
        )
    if isinstance(scalar, np.int64):
        return dt.int32
    if isinstance(scalar, np.uint64):
        return dt.uint32
    if isinstance(scalar, (np.integer, np.floating)):
        return np.dtype(scalar.dtype)
    if isinstance(scalar, int):
        return dt.int32
    return dt.float32
