"""RMSNorm kernels.

``rmsnorm_kernel`` follows examples/models/qwen3/kernels/rmsnorm.py:4-21
(fp32 compute, ``(z + eps)`` cast to the compute dtype, ``x / sqrt(z)``,
times weight, cast back).  ``residual_rmsnorm_kernel`` adds the residual in
the storage dtype first, as the decoder layer does
(examples/models/qwen3/kernels/transformer_layer.py:60).
"""

import numpy as np


def rmsnorm_kernel(x, weight, eps, compute_dtype=np.float32):
    original_dtype = x.dtype
    x = x.astype(compute_dtype)
    weight = weight.astype(compute_dtype)
    z = np.square(x)
    z = np.mean(z, axis=-1, keepdims=True)
    z = (z + eps).astype(x.dtype)
    z = x / np.sqrt(z)
    res = z * weight
    return res.astype(original_dtype)


def residual_rmsnorm_kernel(x, residual, weight, eps):
    h = x + residual
    return rmsnorm_kernel(h, weight, eps)
