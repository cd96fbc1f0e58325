"""Sum of two row blocks of one tensor, rows 2..3 and rows 0..1
(tests/kernels/indexing.py:7-34 of the reference)."""

import numpy as np

from nkipy_amd.core.specs import CommonTypes, KernelSpec, ShapeSpec, TensorInputSpec


def row_blocks_sum(x):
    upper = x[0:2]
    lower = x[2:4, :]
    return np.add(lower, upper)


kernel_specs = [KernelSpec(
    function=row_blocks_sum,
    inputs=[TensorInputSpec(shape_spec=ShapeSpec(dims=[(4, None), None], default=(4, 4)),
                            dtype_spec=CommonTypes.FLOATS, description="at least 4 rows")],
    description="x[2:4] + x[0:2]")]
