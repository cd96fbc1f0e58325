"""Rotary-embedding tables from inverse frequencies and position ids as a
graph exporter writes them (tests/kernels/rope_dynamo.py:7-101 of the
reference): the outer product as a batched matmul of broadcast views, the
transpose, the duplicated half and cos / sin, each scaled by 1.0."""

import numpy as np

from nkipy_amd.core.specs import CommonTypes, KernelSpec, ShapeSpec, TensorInputSpec


def rope_cos_sin(inv_freq, position_ids):
    n = inv_freq.shape[0]
    freqs = np.broadcast_to(np.expand_dims(np.expand_dims(inv_freq, 0), 2), (1, n, 1))
    pos = np.expand_dims(position_ids, 1).astype(np.float32)      # (1, 1, T)
    angles = np.transpose(np.matmul(freqs, pos), (0, 2, 1))       # (1, T, n)
    full = np.concatenate([angles, angles], axis=-1)              # (1, T, 2n)
    return np.multiply(np.cos(full), 1.0), np.multiply(np.sin(full), 1.0)


_rng = np.random.default_rng(11)
INV_FREQ = _rng.uniform(0.0, 1.0, (32,)).astype(np.float32)
POSITIONS = _rng.integers(0, 16, (1, 7)).astype(np.int32)

kernel_specs = [KernelSpec(
    function=rope_cos_sin,
    inputs=[TensorInputSpec(shape_spec=ShapeSpec(dims=[32], default=(32,)), dtype_spec=CommonTypes.FLOATS,
                            default_value=INV_FREQ, description="inverse frequencies"),
            TensorInputSpec(shape_spec=ShapeSpec(dims=[1, 7], default=(1, 7)), dtype_spec=CommonTypes.INTS,
                            default_value=POSITIONS, description="position ids")],
    description="rotary cos / sin tables")]
