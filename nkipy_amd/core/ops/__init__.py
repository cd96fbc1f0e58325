"""Backend-dispatched operations (the targets of the NumPy dispatch table)."""

from nkipy_amd.core.backend import get_backend, set_source_location
from nkipy_amd.core.ops._registry import Op
from nkipy_amd.core.ops.creation import (
    constant, diag, empty_like, full, full_like, ones_like, tril, triu, zeros, zeros_like,
)
from nkipy_amd.core.ops.elementwise import (
    abs_ as abs, add, arctan, arctan2, bitwise_and, bitwise_not, bitwise_or, bitwise_xor,
    ceil, clip, cos, divide, equal, exp, expm1, floor, floor_divide, greater, greater_equal,
    invert, isfinite, isnan, less, less_equal, log, log1p, log2, logaddexp, logical_and,
    logical_not, logical_or, logical_xor, maximum, minimum, multiply, negative, not_equal,
    power, reciprocal, remainder, rint, round_, sign, sin, sqrt, square, subtract, tan, tanh,
    trunc,
)
from nkipy_amd.core.ops.indexing import (
    dynamic_update_slice, put_along_axis, scatter_along_axis, scatter_strided, static_slice,
    take, take_along_axis, where,
)
from nkipy_amd.core.ops.linalg import dot, matmul, norm, outer, trace
from nkipy_amd.core.ops.nn import rms_norm, softmax, topk
from nkipy_amd.core.ops.reduce import (
    all, any, argmax, argmin, count_nonzero, cumsum, max, mean, min, prod, std, sum, var,
)
from nkipy_amd.core.ops.transform import (
    astype, broadcast_to, concatenate, copy, copyto, diff, expand_dims, flip, pad, repeat,
    reshape, roll, split, squeeze, stack, swapaxes, tile, transpose,
)

# Collectives and convolutions exist in the reference op set but are not part
# of this single-GPU backend; their Ops have no implementation and raise
# NotImplementedError naming the backend when called.
all_reduce = Op("all_reduce")
all_gather = Op("all_gather")
reduce_scatter = Op("reduce_scatter")
all_to_all = Op("all_to_all")
conv2d = Op("conv2d")
conv3d = Op("conv3d")
