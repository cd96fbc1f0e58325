"""Row softmax kernels.

``softmax_kernel`` is the README kernel (README.md:125-128,
tests/kernels/softmax.py:7-10); ``softmax_upcast_kernel`` computes in fp32
and casts back (examples/models/qwen3_embedding/kernels/softmax.py:4-8).
"""

import numpy as np


def softmax_kernel(x):
    exp_x = np.exp(x - np.max(x, axis=-1, keepdims=True))
    sum_x = np.sum(exp_x, axis=-1, keepdims=True)
    return exp_x / sum_x


def softmax_upcast_kernel(x):
    original_dtype = x.dtype
    x = x.astype(np.float32)
    exp_x = np.exp(x - np.max(x, axis=-1, keepdims=True))
    return (exp_x / np.sum(exp_x, axis=-1, keepdims=True)).astype(original_dtype)
