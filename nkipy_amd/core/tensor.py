"""Tracer tensor: ``NKIPyTensorRef``.

During tracing every array argument of a kernel is replaced by an
``NKIPyTensorRef``.  NumPy calls on it arrive through ``__array_ufunc__`` /
``__array_function__`` (the NumPy dispatch protocols) and Python operators
through the mixins below; both end in the ``ops`` functions, which record IR.
Behaviour follows the reference tracer tensor
(nkipy/src/nkipy/core/tensor.py:318-851): same interception, same indexing
rules (static slices, one tensor index lowered to ``take``, the
``a[np.arange(N), idx]`` diagonal gather, ``None`` axes), same in-place
``__setitem__`` semantics that re-point the ref at a new value and mark it
mutated, and ``__array__`` refuses conversion to a concrete array.
"""

from __future__ import annotations

import inspect
import math
import os
from typing import Tuple, Union

import numpy as np

_PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def find_source_loc() -> Union[None, Tuple[str, int]]:
    """(filename, line) of the innermost caller outside this package."""
    frame = inspect.currentframe()
    try:
        f = frame.f_back
        while f is not None:
            fn = os.path.abspath(f.f_code.co_filename)
            if not fn.startswith(_PKG_ROOT) and "numpy" not in fn.split(os.sep)[-3:-1]:
                return (f.f_code.co_filename, f.f_lineno)
            f = f.f_back
        return None
    finally:
        del frame


def _set_source_location(location):
    from nkipy_amd.core.backend import set_source_location

    set_source_location(location)


def _ops():
    from nkipy_amd.core import ops

    return ops


class TensorArithmeticMixin:
    def __add__(self, o): return np.add(self, o)
    def __radd__(self, o): return np.add(o, self)
    def __sub__(self, o): return np.subtract(self, o)
    def __rsub__(self, o): return np.subtract(o, self)
    def __mul__(self, o): return np.multiply(self, o)
    def __rmul__(self, o): return np.multiply(o, self)
    def __truediv__(self, o): return np.divide(self, o)
    def __rtruediv__(self, o): return np.divide(o, self)
    def __floordiv__(self, o): return np.floor_divide(self, o)
    def __rfloordiv__(self, o): return np.floor_divide(o, self)
    def __mod__(self, o): return np.mod(self, o)
    def __rmod__(self, o): return np.mod(o, self)
    def __pow__(self, o): return np.power(self, o)
    def __rpow__(self, o): return np.power(o, self)
    def __matmul__(self, o): return np.matmul(self, o)
    def __rmatmul__(self, o): return np.matmul(o, self)
    def __abs__(self): return np.abs(self)
    def __neg__(self): return np.negative(self)
    def __pos__(self): return np.copy(self)
    # in-place forms rebind the name to a new traced value
    def __iadd__(self, o): return self.__add__(o)
    def __isub__(self, o): return self.__sub__(o)
    def __imul__(self, o): return self.__mul__(o)
    def __itruediv__(self, o): return self.__truediv__(o)
    def __ifloordiv__(self, o): return self.__floordiv__(o)
    def __imod__(self, o): return self.__mod__(o)
    def __ipow__(self, o): return self.__pow__(o)
    def __imatmul__(self, o): return self.__matmul__(o)
    def __lt__(self, o): return np.less(self, o)
    def __le__(self, o): return np.less_equal(self, o)
    def __gt__(self, o): return np.greater(self, o)
    def __ge__(self, o): return np.greater_equal(self, o)
    def __eq__(self, o): return np.equal(self, o)
    def __ne__(self, o): return np.not_equal(self, o)
    def __and__(self, o): return np.bitwise_and(self, o)
    def __rand__(self, o): return np.bitwise_and(o, self)
    def __or__(self, o): return np.bitwise_or(self, o)
    def __ror__(self, o): return np.bitwise_or(o, self)
    def __xor__(self, o): return np.bitwise_xor(self, o)
    def __rxor__(self, o): return np.bitwise_xor(o, self)
    def __invert__(self): return np.invert(self)

    __hash__ = object.__hash__


class TensorOperationMixin:
    def transpose(self, *axes):
        if not axes:
            return np.transpose(self)
        if len(axes) == 1 and isinstance(axes[0], (tuple, list)):
            return np.transpose(self, axes[0])
        return np.transpose(self, axes)

    def reshape(self, *shape):
        if not shape:
            raise TypeError("reshape() takes at least 1 argument (0 given)")
        if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
            return np.reshape(self, shape[0])
        return np.reshape(self, shape)

    def mean(self, axis=None, keepdims=False, **kw): return np.mean(self, axis=axis, keepdims=keepdims, **kw)
    def sum(self, axis=None, keepdims=False, **kw): return np.sum(self, axis=axis, keepdims=keepdims, **kw)
    def var(self, axis=None, keepdims=False, **kw): return np.var(self, axis=axis, keepdims=keepdims, **kw)
    def std(self, axis=None, keepdims=False, **kw): return np.std(self, axis=axis, keepdims=keepdims, **kw)
    def max(self, axis=None, keepdims=False, **kw): return np.max(self, axis=axis, keepdims=keepdims, **kw)
    def min(self, axis=None, keepdims=False, **kw): return np.min(self, axis=axis, keepdims=keepdims, **kw)
    def prod(self, axis=None, keepdims=False, **kw): return np.prod(self, axis=axis, keepdims=keepdims, **kw)
    def argmax(self, axis=None, **kw): return np.argmax(self, axis=axis, **kw)
    def argmin(self, axis=None, **kw): return np.argmin(self, axis=axis, **kw)
    def squeeze(self, axis=None): return np.squeeze(self, axis=axis)
    def copy(self): return np.copy(self)
    def clip(self, a_min=None, a_max=None): return np.clip(self, a_min, a_max)
    def ravel(self): return np.reshape(self, (-1,))
    def flatten(self): return np.reshape(self, (-1,))
    def swapaxes(self, a, b): return np.swapaxes(self, a, b)


def _expand_ellipsis(indices: tuple, ndim: int) -> tuple:
    n_ell = sum(1 for i in indices if i is Ellipsis)
    if n_ell == 0:
        return indices
    if n_ell > 1:
        raise IndexError("an index can only have a single ellipsis (...)")
    n_real = sum(1 for i in indices if i is not None and i is not Ellipsis)
    fill = ndim - n_real
    if fill < 0:
        raise IndexError(
            f"too many indices for tensor: tensor is {ndim}-dimensional, "
            f"but {n_real} non-ellipsis indices were given"
        )
    out = []
    for i in indices:
        out.extend([slice(None)] * fill if i is Ellipsis else [i])
    return tuple(out)


def _strip_newaxis(indices: tuple):
    """Drop ``None`` entries; return the rest and the output positions of
    the new axes."""
    kept, new_axes, pos = [], [], 0
    for i in indices:
        if i is None:
            new_axes.append(pos)
            pos += 1
            continue
        kept.append(i)
        if not isinstance(i, (int, np.integer)):
            pos += 1
    return tuple(kept), new_axes


def _norm_slice(s: slice, dim: int):
    start, stop, step = s.indices(dim)
    if step <= 0:
        raise NotImplementedError("negative slice steps are not supported during tracing")
    return start, max(stop, start), step


class NKIPyTensorRef(TensorArithmeticMixin, TensorOperationMixin):
    """Reference to a traced tensor (an IR value)."""

    __slots__ = ("backend_tensor", "_shape", "_dtype", "_name", "_original_parameter", "_is_mutated")
    _tensor_apis = {}

    def __init__(self, backend_tensor, name: str = None):
        self.backend_tensor = backend_tensor
        self._shape = tuple(backend_tensor.shape)
        self._dtype = backend_tensor.dtype
        self._name = name
        self._original_parameter = None
        self._is_mutated = False

    # -- array-like attributes -----------------------------------------
    @property
    def name(self): return self._name

    @property
    def shape(self) -> Tuple[int, ...]: return self._shape

    @property
    def dtype(self): return self._dtype

    @property
    def ndim(self) -> int: return len(self._shape)

    @property
    def size(self) -> int: return math.prod(self._shape)

    @property
    def T(self): return self.transpose()

    @property
    def itemsize(self) -> int: return self._dtype.itemsize

    @property
    def nbytes(self) -> int: return self.size * self._dtype.itemsize

    @property
    def strides(self) -> Tuple[int, ...]:
        out, s = [], self._dtype.itemsize
        for d in reversed(self._shape):
            out.append(s)
            s *= d
        return tuple(reversed(out))

    def __len__(self):
        if not self._shape:
            raise TypeError("len() of unsized object")
        return self._shape[0]

    def __array__(self, dtype=None, copy=None):
        raise TypeError(
            "NKIPyTensorRef cannot be converted to a numpy array: it is a node of a "
            "traced computation graph. np.array(tensor) / np.asarray(tensor) are not "
            "supported during tracing."
        )

    def __bool__(self):
        raise TypeError(
            "the truth value of a traced tensor is unknown at trace time; "
            "use np.where for data-dependent selection"
        )

    def __repr__(self):
        from nkipy_amd.core import dtypes as dt

        return f"NKIPyTensorRef(name={self._name}, shape={self._shape}, dtype={dt.name(self._dtype)})"

    def _rebind(self, result):
        self.backend_tensor = result.backend_tensor
        self._shape = result.shape
        self._dtype = result.dtype

    # -- NumPy protocols ----------------------------------------------------
    def astype(self, dtype):
        _set_source_location(find_source_loc())
        try:
            return _ops().astype(self, dtype)
        finally:
            _set_source_location(None)

    def __array_ufunc__(self, ufunc, method, *inputs, **kwargs):
        if method != "__call__":
            return NotImplemented
        _set_source_location(find_source_loc())
        try:
            return self.__array_function__(ufunc, (), inputs, kwargs)
        finally:
            _set_source_location(None)

    def __array_function__(self, func, types, args, kwargs):
        impl = self._tensor_apis.get(func)
        if impl is None:
            raise NotImplementedError(
                f"NumPy function '{getattr(func, '__name__', func)}' has not been "
                "implemented in NKIPy."
            )
        _set_source_location(find_source_loc())
        try:
            return impl(*args, **kwargs)
        finally:
            _set_source_location(None)

    # -- indexing -----------------------------------------------------------
    def __getitem__(self, indices):
        ops = _ops()
        _set_source_location(find_source_loc())
        try:
            if not isinstance(indices, tuple):
                indices = (indices,)
            indices = _expand_ellipsis(indices, self.ndim)
            indices, new_axes = _strip_newaxis(indices)
            if len(indices) > self.ndim:
                raise IndexError(f"too many indices for tensor of dimension {self.ndim}")
            indices = indices + (slice(None),) * (self.ndim - len(indices))
            for i in indices:
                if isinstance(i, (NKIPyTensorRef, np.ndarray)) and i.dtype == np.bool_:
                    raise NotImplementedError(
                        "Boolean indexing is not supported: a boolean mask gives a "
                        "data-dependent output shape."
                    )
            dyn = [(d, i) for d, i in enumerate(indices)
                   if isinstance(i, (NKIPyTensorRef, np.ndarray, list))]
            if not dyn:
                result = self._static_slice(indices)
            else:
                result = None
                if len(dyn) == 2:
                    result = self._diagonal_gather(dyn, ops)
                if result is None:
                    if len(dyn) > 1:
                        raise ValueError("Only one tensor index is currently supported")
                    d, idx = dyn[0]
                    static = tuple(slice(None) if k == d else i for k, i in enumerate(indices))
                    base = self
                    if any(not (isinstance(i, slice) and i == slice(None)) for i in static):
                        base = self._static_slice(static)
                        d -= sum(1 for i in static[:d] if isinstance(i, (int, np.integer)))
                    result = ops.take(base, idx, axis=d)
            if new_axes:
                result = ops.expand_dims(result, axis=new_axes)
            return result
        finally:
            _set_source_location(None)

    def _diagonal_gather(self, dyn, ops):
        (d1, i1), (d2, i2) = dyn

        def is_arange(i, n):
            return (isinstance(i, np.ndarray) and i.ndim == 1 and len(i) == n
                    and np.array_equal(i, np.arange(n)))

        if is_arange(i1, self.shape[d1]):
            ar_dim, g_dim, idx = d1, d2, i2
        elif is_arange(i2, self.shape[d2]):
            ar_dim, g_dim, idx = d2, d1, i1
        else:
            return None
        shp = [1] * self.ndim
        shp[ar_dim] = self.shape[ar_dim]
        if isinstance(idx, NKIPyTensorRef):
            idx = ops.reshape(idx, tuple(shp))
        else:
            idx = np.asarray(idx).reshape(shp)
        return ops.squeeze(ops.take_along_axis(self, idx, axis=g_dim), axis=g_dim)

    def _static_slice(self, indices):
        start, limit, strides, squeeze = [], [], [], []
        for d, i in enumerate(indices):
            n = self.shape[d]
            if isinstance(i, slice):
                a, b, s = _norm_slice(i, n)
                start.append(a)
                limit.append(b)
                strides.append(s)
            elif isinstance(i, (int, np.integer)):
                i = int(i)
                if i < 0:
                    i += n
                if not 0 <= i < n:
                    raise IndexError(f"index {i} is out of bounds for axis {d} with size {n}")
                start.append(i)
                limit.append(i + 1)
                strides.append(1)
                squeeze.append(d)
            else:
                raise ValueError(f"Unsupported index type in static slicing: {type(i)}")
        return _ops().static_slice(self, start, limit, strides, squeeze)

    def __setitem__(self, indices, value):
        ops = _ops()
        _set_source_location(find_source_loc())
        try:
            if not isinstance(indices, tuple):
                indices = (indices,)
            if any(i is None for i in indices):
                raise IndexError(
                    "cannot use a newaxis (None) in a setitem expression; use "
                    "np.expand_dims() on the value instead"
                )
            indices = _expand_ellipsis(indices, self.ndim)
            indices = indices + (slice(None),) * (self.ndim - len(indices))
            dyn = [(d, i) for d, i in enumerate(indices) if isinstance(i, NKIPyTensorRef)]
            self._is_mutated = True
            if dyn:
                if len(dyn) > 1:
                    raise ValueError("Only one tensor index is currently supported")
                d, idx = dyn[0]
                self._rebind(ops.scatter_along_axis(self, idx, value, axis=d))
                return
            strided = any(isinstance(i, slice) and i.step not in (None, 1) for i in indices)
            if strided:
                per_dim = []
                for d, i in enumerate(indices):
                    if isinstance(i, slice):
                        per_dim.append(list(range(*_norm_slice(i, self.shape[d]))))
                    else:
                        i = int(i)
                        per_dim.append([i + self.shape[d] if i < 0 else i])
                self._rebind(ops.scatter_strided(self, value, per_dim))
                return
            start, upd_shape = [], []
            for d, i in enumerate(indices):
                if isinstance(i, slice):
                    a, b, _ = _norm_slice(i, self.shape[d])
                    start.append(a)
                    upd_shape.append(b - a)
                else:
                    i = int(i)
                    start.append(i + self.shape[d] if i < 0 else i)
                    upd_shape.append(1)
            self._rebind(ops.dynamic_update_slice(self, value, start, tuple(upd_shape)))
        finally:
            _set_source_location(None)
