"""Creation ops: zeros / ones / full / empty (``*_like`` too), constant,
tril / triu / diag.

These have ``"cpu"`` implementations as well, so kernels that call them run
unchanged as plain NumPy (reference: nkipy/src/nkipy/core/ops/creation.py:
16-51, 288-387).  Under tracing a fill is a scalar constant broadcast to the
shape (no payload the size of the tensor is stored).
"""

from __future__ import annotations

import numpy as np

from nkipy_amd.core import dtypes as dt
from nkipy_amd.core.backend.hip import broadcast_to, convert
from nkipy_amd.core.ops._helpers import ctx, val, wrap
from nkipy_amd.core.ops._registry import Op


def _fill(shape, value, dtype):
    if isinstance(shape, (int, np.integer)):
        shape = (int(shape),)
    shape = tuple(int(s) for s in shape)
    d = dt.canonical(dtype) if dtype is not None else None
    if d is None:
        d = dt.float32 if isinstance(value, float) else (dt.bool_ if isinstance(value, bool) else dt.int32)
    if d == dt.float64:
        d = dt.float32
    c = ctx()
    return wrap(broadcast_to(c, c.constant(value, d), shape))


def _np_dtype(dtype):
    d = dt.canonical(dtype) if dtype is not None else None
    return d


zeros = Op("zeros")


@zeros.impl("hip")
def _zeros_hip(shape, dtype=np.float32, **kw):
    return _fill(shape, 0, dtype)


@zeros.impl("cpu")
def _zeros_cpu(shape, dtype=np.float32, **kw):
    return np.zeros(shape, dtype=_np_dtype(dtype))


full = Op("full")


@full.impl("hip")
def _full_hip(shape, fill_value, dtype=None, **kw):
    return _fill(shape, fill_value, dtype)


@full.impl("cpu")
def _full_cpu(shape, fill_value, dtype=None, **kw):
    return np.full(shape, fill_value, dtype=_np_dtype(dtype))


def _like(name, value):
    op = Op(name)

    @op.impl("hip")
    def impl(a, dtype=None, order="K", subok=True, shape=None, **kw):
        v = val(a)
        return _fill(shape if shape is not None else v.shape, value, dtype if dtype is not None else v.dtype)

    @op.impl("cpu")
    def impl_cpu(a, dtype=None, order="K", subok=True, shape=None, **kw):
        return getattr(np, name)(a, dtype=dtype, shape=shape)

    return op


zeros_like = _like("zeros_like", 0)
ones_like = _like("ones_like", 1)
empty_like = _like("empty_like", 0)

full_like = Op("full_like")


@full_like.impl("hip")
def _full_like_hip(a, fill_value, dtype=None, order="K", subok=True, shape=None, **kw):
    v = val(a)
    return _fill(shape if shape is not None else v.shape, fill_value, dtype if dtype is not None else v.dtype)


@full_like.impl("cpu")
def _full_like_cpu(a, fill_value, dtype=None, order="K", subok=True, shape=None, **kw):
    return np.full_like(a, fill_value, dtype=dtype, shape=shape)


constant = Op("constant")


@constant.impl("hip")
def _constant_hip(value, dtype=None):
    """Promote a concrete (trace-time) array to a graph constant."""
    return wrap(ctx().constant(np.asarray(value) if not np.isscalar(value) else value, dtype))


@constant.impl("cpu")
def _constant_cpu(value, dtype=None):
    return np.asarray(value, dtype=_np_dtype(dtype))


def _tri(name, lower):
    op = Op(name)

    @op.impl("hip")
    def impl(m, k=0):
        from nkipy_amd.core.ops.indexing import where

        v = val(m)
        n, cols = v.shape[-2], v.shape[-1]
        mask = np.tri(n, cols, k=k, dtype=bool) if lower else ~np.tri(n, cols, k=k - 1, dtype=bool)
        return where(mask, m, 0)

    @op.impl("cpu")
    def impl_cpu(m, k=0):
        return (np.tril if lower else np.triu)(m, k)

    return op


tril = _tri("tril", True)
triu = _tri("triu", False)

diag = Op("diag")


@diag.impl("hip")
def _diag_hip(v, k=0):
    from nkipy_amd.core.ops import elementwise as ew
    from nkipy_amd.core.ops.indexing import take

    x = val(v)
    c = ctx()
    if x.ndim == 1:
        n = x.shape[0] + abs(k)
        eye = np.eye(n, n, k=k, dtype=bool)
        # row i of the result holds v[i] (k >= 0) or v[i + k] (k < 0) on the diagonal
        if k >= 0:
            col = np.concatenate([np.arange(x.shape[0]), np.zeros(k, np.int64)])
            src = take(v, col.astype(np.int32), axis=0)
            from nkipy_amd.core.ops.indexing import where
            from nkipy_amd.core.ops.transform import _reshape_hip

            return where(eye, _reshape_hip(src, (n, 1)), 0)
        row = np.concatenate([np.zeros(-k, np.int64), np.arange(x.shape[0])])
        src = take(v, row.astype(np.int32), axis=0)
        from nkipy_amd.core.ops.indexing import where
        from nkipy_amd.core.ops.transform import _reshape_hip

        return where(eye, _reshape_hip(src, (1, n)), 0)
    if x.ndim == 2:
        rows, cols = x.shape
        i = np.arange(max(0, -k), min(rows, cols - k))
        flat_idx = (i * cols + i + k).astype(np.int32)
        from nkipy_amd.core.ops.transform import _reshape_hip

        return take(_reshape_hip(v, (rows * cols,)), flat_idx, axis=0)
    raise ValueError("Input must be 1- or 2-d.")


@diag.impl("cpu")
def _diag_cpu(v, k=0):
    return np.diag(v, k)
