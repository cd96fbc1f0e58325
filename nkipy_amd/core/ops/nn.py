"""Neural-network helper ops.

The reference declares ``softmax`` / ``rms_norm`` / ``topk`` ops
(nkipy/src/nkipy/core/ops/nn.py:12-14, 158-160) but gives softmax and
RMSNorm no implementation: kernels write them as NumPy compositions.  Here
both are the same compositions, so they trace to the graphs the pattern
matcher recognises.  ``topk(x, k, axis, is_ascend)`` returns (values,
uint32 indices) ordered best first (nn.py:19-152): on the device the
indices come from a row-selection kernel (last axis only, as in the
reference's device lowering) and the values are gathered at them.
"""

from __future__ import annotations

import numpy as np

from nkipy_amd.core.ops import elementwise as ew
from nkipy_amd.core.ops import reduce as rd
from nkipy_amd.core.ops._registry import Op

softmax = Op("softmax")


@softmax.impl("hip")
def _softmax_hip(x, axis=-1):
    e = ew.exp(ew.subtract(x, rd.max(x, axis=axis, keepdims=True)))
    return ew.divide(e, rd.sum(e, axis=axis, keepdims=True))


@softmax.impl("cpu")
def _softmax_cpu(x, axis=-1):
    e = np.exp(x - np.max(x, axis=axis, keepdims=True))
    return e / np.sum(e, axis=axis, keepdims=True)


rms_norm = Op("rms_norm")


@rms_norm.impl("hip")
def _rms_norm_hip(x, weight, eps=1e-6):
    ms = rd.mean(ew.multiply(x, x), axis=-1, keepdims=True)
    return ew.multiply(ew.divide(x, ew.sqrt(ew.add(ms, eps))), weight)


@rms_norm.impl("cpu")
def _rms_norm_cpu(x, weight, eps=1e-6):
    ms = np.mean(x * x, axis=-1, keepdims=True)
    return x / np.sqrt(ms + eps) * weight


topk = Op("topk")


@topk.impl("hip")
def _topk_hip(x, k, axis=0, is_ascend=False, out=None, dtype=None):
    from nkipy_amd.core import dtypes as dt
    from nkipy_amd.core.ops._helpers import ctx, val, wrap
    from nkipy_amd.core.ops.indexing import take_along_axis

    v = val(x)
    ax = axis + v.ndim if axis < 0 else axis
    if ax != v.ndim - 1:
        raise NotImplementedError("topk on this backend supports the last axis only")
    if not 0 < k <= v.shape[-1]:
        raise ValueError(f"k={k} must be in 1..{v.shape[-1]} (size of axis {ax})")
    shape = tuple(v.shape[:-1]) + (int(k),)
    idx = ctx().build_op("topk", [v], shape, dt.uint32, {"k": int(k), "largest": not is_ascend})
    return take_along_axis(wrap(v), wrap(idx), axis=ax), wrap(idx)


@topk.impl("cpu")
def _topk_cpu(x, k, axis=0, is_ascend=False, out=None, dtype=None):
    """Stable selection: best values first, ties by lower index."""
    x = np.asarray(x)
    ax = axis + x.ndim if axis < 0 else axis
    keys = x if is_ascend else -x
    order = np.argsort(keys, axis=ax, kind="stable")
    idx = np.take(order, np.arange(k), axis=ax)
    return np.take_along_axis(x, idx, axis=ax), idx.astype(np.uint32)
