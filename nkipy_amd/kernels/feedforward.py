"""SwiGLU feed-forward kernels.

``feedforward_kernel`` follows examples/models/qwen3/kernels/feedforward.py:
4-18 (fused gate_up weight, np.split, silu(x) = x * (1 / (1 + exp(-x)))).
``swiglu_mlp_kernel`` is the two-weight form of the benchmark workload:
y = (silu(x @ W_gate) * (x @ W_up)) @ W_down.  ``feedforward_bias_kernel``
adds the optional biases of examples/models/qwen3_embedding/kernels/ffn.py:
11-46.  ``linear_nt_kernel`` is x @ W.T with a torch-Linear (out, in) weight
(tests/kernels/mlp_dynamo.py:9-25).
"""

import numpy as np


def silu_kernel_(x):
    return x * (1 / (1 + np.exp(-x)))


def feedforward_kernel(x, gate_up_weight, down_weight):
    mm_gup = np.matmul(x, gate_up_weight)
    xg, x_v = np.split(mm_gup, 2, axis=-1)
    swish = silu_kernel_(xg)
    x0 = swish * x_v
    return x0 @ down_weight


def swiglu_mlp_kernel(x, w_gate, w_up, w_down):
    return (silu_kernel_(x @ w_gate) * (x @ w_up)) @ w_down


def feedforward_bias_kernel(x, gate_up_weight, down_weight, gate_up_bias=None, down_bias=None):
    mm_gup = np.matmul(x, gate_up_weight)
    if gate_up_bias is not None:
        mm_gup = mm_gup + gate_up_bias
    xg, x_up = np.split(mm_gup, 2, axis=-1)
    x0 = silu_kernel_(xg) * x_up
    out = x0 @ down_weight
    if down_bias is not None:
        out = out + down_bias
    return out


def linear_nt_kernel(x, weight):
    return np.matmul(x, np.transpose(weight))
