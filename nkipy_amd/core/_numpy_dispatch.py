"""NumPy function -> op table for traced tensors.

The same mapping as the reference (nkipy/src/nkipy/core/_numpy_dispatch.py:
27-159): each NumPy function a kernel may call on an ``NKIPyTensorRef`` is
routed to an ``ops`` function.  ``np.put_along_axis`` mutates its argument,
so its entry re-points the traced tensor and marks it mutated for alias
detection.  Functions missing from the table raise NotImplementedError.
"""

import numpy as np

from nkipy_amd.core.tensor import NKIPyTensorRef


def _register(numpy_func, op):
    NKIPyTensorRef._tensor_apis[numpy_func] = op


def register_all_numpy_apis():
    from nkipy_amd.core import ops

    table = {
        # binary
        np.add: ops.add, np.subtract: ops.subtract, np.multiply: ops.multiply,
        np.divide: ops.divide, np.true_divide: ops.divide, np.power: ops.power,
        np.maximum: ops.maximum, np.minimum: ops.minimum,
        np.bitwise_and: ops.bitwise_and, np.bitwise_or: ops.bitwise_or,
        np.bitwise_xor: ops.bitwise_xor, np.logaddexp: ops.logaddexp,
        np.remainder: ops.remainder, np.mod: ops.remainder,
        np.floor_divide: ops.floor_divide,
        # comparison / logical
        np.equal: ops.equal, np.not_equal: ops.not_equal, np.greater: ops.greater,
        np.greater_equal: ops.greater_equal, np.less: ops.less,
        np.less_equal: ops.less_equal, np.logical_and: ops.logical_and,
        np.logical_or: ops.logical_or, np.logical_xor: ops.logical_xor,
        # unary
        np.abs: ops.abs, np.absolute: ops.abs, np.exp: ops.exp, np.log: ops.log,
        np.sqrt: ops.sqrt, np.square: ops.square, np.negative: ops.negative,
        np.reciprocal: ops.reciprocal, np.sin: ops.sin, np.cos: ops.cos, np.tan: ops.tan,
        np.arctan: ops.arctan, np.tanh: ops.tanh, np.ceil: ops.ceil, np.floor: ops.floor,
        np.rint: ops.rint, np.trunc: ops.trunc, np.sign: ops.sign, np.invert: ops.invert,
        np.bitwise_not: ops.bitwise_not, np.logical_not: ops.logical_not,
        np.clip: ops.clip, np.log1p: ops.log1p, np.log2: ops.log2, np.expm1: ops.expm1,
        np.round: ops.round_, np.around: ops.round_, np.isnan: ops.isnan,
        np.isfinite: ops.isfinite,
        # reductions
        np.sum: ops.sum, np.max: ops.max, np.amax: ops.max, np.min: ops.min,
        np.amin: ops.min, np.mean: ops.mean, np.any: ops.any, np.all: ops.all,
        np.var: ops.var, np.std: ops.std, np.argmax: ops.argmax, np.argmin: ops.argmin,
        np.cumsum: ops.cumsum, np.prod: ops.prod, np.count_nonzero: ops.count_nonzero,
        # linear algebra
        np.matmul: ops.matmul, np.dot: ops.dot, np.linalg.norm: ops.norm,
        np.outer: ops.outer, np.trace: ops.trace,
        # transforms
        np.reshape: ops.reshape, np.transpose: ops.transpose,
        np.expand_dims: ops.expand_dims, np.concatenate: ops.concatenate,
        np.split: ops.split, np.copy: ops.copy, np.repeat: ops.repeat,
        np.squeeze: ops.squeeze, np.pad: ops.pad, np.swapaxes: ops.swapaxes,
        np.stack: ops.stack, np.diff: ops.diff, np.flip: ops.flip, np.tile: ops.tile,
        np.roll: ops.roll, np.tril: ops.tril, np.triu: ops.triu, np.diag: ops.diag,
        # creation
        np.zeros_like: ops.zeros_like, np.ones_like: ops.ones_like,
        np.empty_like: ops.empty_like, np.full_like: ops.full_like,
        # indexing
        np.where: ops.where, np.take: ops.take, np.take_along_axis: ops.take_along_axis,
        # broadcast / copy
        np.broadcast_to: ops.broadcast_to, np.copyto: ops.copyto,
    }
    for f, op in table.items():
        _register(f, op)

    def _put_along_axis_inplace(arr, indices, values, axis):
        result = ops.put_along_axis(arr, indices, values, axis)
        if isinstance(arr, NKIPyTensorRef) and result is not None:
            arr._rebind(result)
            arr._is_mutated = True

    NKIPyTensorRef._tensor_apis[np.put_along_axis] = _put_along_axis_inplace
