"""Gated MLP of one token with torch-layout (out, in) fp32 weights as a
graph exporter writes it (tests/kernels/mlp_dynamo.py:7-65 of the
reference): three matmuls against transposed weights, the logistic
sigmoid spelt out, SiLU(gate) * up."""

import numpy as np

from nkipy_amd.core.specs import CommonTypes, KernelSpec, ShapeSpec, TensorInputSpec

HIDDEN, FFN = 2048, 8192


def gated_mlp_token(w_gate, x, w_up, w_down):
    h = np.reshape(x, [1, HIDDEN])
    gate = np.reshape(np.matmul(h, np.transpose(w_gate, [1, 0])), [1, 1, FFN])
    up = np.reshape(np.matmul(h, np.transpose(w_up, [1, 0])), [1, 1, FFN])
    act = np.multiply(np.multiply(gate, 1 / (1 + np.exp(-gate))), up)
    out = np.matmul(np.reshape(act, [1, FFN]), np.transpose(w_down, [1, 0]))
    return np.reshape(out, [1, 1, HIDDEN])


_rng = np.random.default_rng(13)
W_GATE = (_rng.standard_normal((FFN, HIDDEN), dtype=np.float32) / np.sqrt(HIDDEN)).astype(np.float32)
X = _rng.standard_normal((HIDDEN,), dtype=np.float32)
W_UP = (_rng.standard_normal((FFN, HIDDEN), dtype=np.float32) / np.sqrt(HIDDEN)).astype(np.float32)
W_DOWN = (_rng.standard_normal((HIDDEN, FFN), dtype=np.float32) / np.sqrt(FFN)).astype(np.float32)


def _tensor(shape, value, what):
    return TensorInputSpec(shape_spec=ShapeSpec(dims=list(shape), default=shape), dtype_spec=CommonTypes.FLOATS,
                           default_value=value, description=what)


kernel_specs = [KernelSpec(
    function=gated_mlp_token,
    inputs=[_tensor((FFN, HIDDEN), W_GATE, "gate weight"), _tensor((HIDDEN,), X, "token"),
            _tensor((FFN, HIDDEN), W_UP, "up weight"), _tensor((HIDDEN, FFN), W_DOWN, "down weight")],
    description="SwiGLU MLP of one token")]
