"""Row softmax over the last axis (tests/kernels/softmax.py:7-27 of the
reference)."""

import numpy as np

from nkipy_amd.core.specs import CommonTypes, KernelSpec, ShapeSpec, TensorInputSpec


def row_softmax(x):
    shifted = x - np.max(x, axis=-1, keepdims=True)
    e = np.exp(shifted)
    return e / np.sum(e, axis=-1, keepdims=True)


kernel_specs = [KernelSpec(
    function=row_softmax,
    inputs=[TensorInputSpec(shape_spec=ShapeSpec(dims=[None, (2, 65536)], default=(32, 128)),
                            dtype_spec=CommonTypes.FLOATS, description="(rows, n)")],
    description="softmax over the last axis")]
