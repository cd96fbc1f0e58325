"""Elementwise sum of two 2-D tensors of any shape (tests/kernels/simple.py:
27-64 of the reference)."""

import numpy as np

from nkipy_amd.core.specs import CommonTypes, KernelSpec, ShapeSpec, TensorInputSpec


def add_tensors(a, b):
    return np.add(a, b)


def _operand(name):
    return TensorInputSpec(shape_spec=ShapeSpec(dims=[None, None], default=(32, 32)),
                           dtype_spec=CommonTypes.FLOATS, description=name)


kernel_specs = [KernelSpec(function=add_tensors, inputs=[_operand("lhs"), _operand("rhs")],
                           description="a + b, any 2-D shape")]
