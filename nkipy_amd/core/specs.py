"""Kernel specifications: the inputs a NumPy kernel accepts.

Same interface as nkipy/core/specs.py:1-92 (``ShapeSpec``, ``TypeSpec``,
``InputSpec`` / ``ScalarInputSpec`` / ``TensorInputSpec``, ``KernelSpec``,
``CommonTypes``), so a module that lists ``kernel_specs`` for the reference
lists them for this package unchanged.  ``ShapeSpec.draw`` and
``KernelSpec.default_inputs`` / ``draw_inputs`` are additions used by the
conformance sweep: a shape drawn inside the constraints, and inputs built
from the defaults or drawn shapes and dtypes.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, List, Optional, Sequence, Tuple, Type, Union

import numpy as np

Dim = Union[int, Tuple[Optional[int], Optional[int]], None]


@dataclass
class ShapeSpec:
    """Allowed shapes, one entry per dimension: an ``int`` (exactly that
    size), a ``(min, max)`` pair (inclusive, ``None`` = unbounded) or
    ``None`` (any size).  ``default`` is the shape tests use by default."""

    dims: List[Dim]
    default: Tuple[int, ...]

    @staticmethod
    def _bounds(d: Dim) -> Tuple[int, Optional[int]]:
        if d is None:
            return 1, None
        if isinstance(d, int):
            return d, d
        lo, hi = d
        return (1 if lo is None else lo), hi

    def is_valid(self, shape: Sequence[int]) -> bool:
        if len(shape) != len(self.dims):
            return False
        for n, d in zip(shape, self.dims):
            lo, hi = self._bounds(d)
            if d is not None and (n < lo or (hi is not None and n > hi)):
                return False
        return True

    def draw(self, rng: np.random.Generator, limit: int = 64) -> Tuple[int, ...]:
        """A shape inside the constraints; open upper bounds stop at ``limit``
        (or at the lower bound when that is larger)."""
        out = []
        for d in self.dims:
            lo, hi = self._bounds(d)
            hi = max(lo, limit) if hi is None else hi
            out.append(int(rng.integers(lo, hi + 1)))
        return tuple(out)


@dataclass
class TypeSpec:
    """Allowed dtypes and the default one."""

    allowed: List[Type]
    default: Type

    def is_valid(self, dtype) -> bool:
        return any(np.dtype(dtype) == np.dtype(a) for a in self.allowed)


@dataclass(kw_only=True)
class InputSpec:
    dtype_spec: TypeSpec
    description: str = ""
    # used by default-input tests when set; a callable is called for the
    # value when a test needs it (large tables are then built only on use)
    default_value: Any = None


@dataclass(kw_only=True)
class ScalarInputSpec(InputSpec):
    description: str = "Scalar input"


@dataclass(kw_only=True)
class TensorInputSpec(InputSpec):
    shape_spec: ShapeSpec
    description: str = "Tensor input"


def _random_array(rng: np.random.Generator, shape, dtype) -> np.ndarray:
    dtype = np.dtype(dtype)
    if dtype == np.bool_:
        return rng.integers(0, 2, shape).astype(bool)
    if np.issubdtype(dtype, np.integer):
        info = np.iinfo(dtype)
        return rng.integers(max(info.min, -100), min(info.max, 100) + 1, shape).astype(dtype)
    return rng.standard_normal(shape, dtype=np.float32).astype(dtype)


@dataclass
class KernelSpec:
    """A kernel function and the inputs it takes."""

    function: Any
    inputs: List[InputSpec]
    is_pure_numpy: bool = True
    description: str = ""

    def default_inputs(self, rng: np.random.Generator) -> list:
        """Each input's ``default_value``, else random data of the default
        shape and dtype (the scalar default for a scalar input)."""
        out = []
        for spec in self.inputs:
            if spec.default_value is not None:
                v = spec.default_value
                out.append(v() if callable(v) else v)
            elif isinstance(spec, TensorInputSpec):
                out.append(_random_array(rng, spec.shape_spec.default, spec.dtype_spec.default))
            else:
                out.append(np.dtype(spec.dtype_spec.default).type(1))
        return out

    def input_stubs(self) -> list:
        """Stand-ins of the default inputs with their shapes and dtypes
        (zero-strided views of one zero: enough to trace the kernel, no data
        is built)."""
        out = []
        for spec in self.inputs:
            if isinstance(spec, TensorInputSpec):
                v = spec.default_value
                if v is not None and not callable(v):
                    out.append(v)
                else:
                    out.append(np.broadcast_to(np.zeros((), np.dtype(spec.dtype_spec.default)),
                                               tuple(spec.shape_spec.default)))
            else:
                v = spec.default_value
                out.append(v if v is not None else np.dtype(spec.dtype_spec.default).type(1))
        return out

    def draw_inputs(self, rng: np.random.Generator, limit: int = 64, same_shape: bool = True,
                    same_dtype: bool = True) -> list:
        """Random inputs of drawn shapes and dtypes.  With ``same_shape``
        tensor inputs whose specs have equal dims share one drawn shape (the
        elementwise kernels need that); with ``same_dtype`` all tensors take
        the first tensor's drawn dtype."""
        shapes = {}
        dtype = None
        out = []
        for spec in self.inputs:
            if not isinstance(spec, TensorInputSpec):
                out.append(np.dtype(spec.dtype_spec.default).type(1))
                continue
            key = repr(spec.shape_spec.dims)
            shape = shapes.get(key) if same_shape else None
            if shape is None:
                shape = spec.shape_spec.draw(rng, limit)
                shapes[key] = shape
            allowed = spec.dtype_spec.allowed
            dt = allowed[int(rng.integers(len(allowed)))]
            if same_dtype:
                dtype = dt if dtype is None else dtype
                dt = dtype if spec.dtype_spec.is_valid(dtype) else dt
            out.append(_random_array(rng, shape, dt))
        return out


class CommonTypes:
    FLOATS = TypeSpec(allowed=[np.float32, np.float16], default=np.float32)
    INTS = TypeSpec(allowed=[np.int8, np.int16, np.int32, np.int64], default=np.int32)
    BOOL = TypeSpec(allowed=[bool], default=bool)
