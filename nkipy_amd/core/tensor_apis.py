"""Kernel-facing helper ops (reference: nkipy/src/nkipy/core/tensor_apis.py:5-24).

``softmax`` and ``rms_norm`` are traced as the NumPy compositions the row
kernels match (a last-axis softmax lowers to the fused softmax launch).
``conv2d`` / ``conv3d`` are exported for import compatibility; this
single-GPU backend has no implementation for them and calling one raises
``NotImplementedError`` naming the backend.
"""

from nkipy_amd.core.ops import (  # noqa: F401
    constant, conv2d, conv3d, full, full_like, ones_like, rms_norm, softmax, topk, zeros,
    zeros_like,
)

__all__ = [
    "constant",
    "topk",
    "rms_norm",
    "softmax",
    "conv2d",
    "conv3d",
    "zeros",
    "full",
]
