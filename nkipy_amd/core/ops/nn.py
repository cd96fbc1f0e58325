"""Neural-network helper ops.

The reference declares ``softmax`` / ``rms_norm`` / ``topk`` ops
(nkipy/src/nkipy/core/ops/nn.py:12-14, 158-160) but gives softmax and
RMSNorm no implementation: kernels write them as NumPy compositions.  Here
both are the same compositions, so they trace to the graphs the pattern
matcher recognises; ``topk`` is not supported on this backend.
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
