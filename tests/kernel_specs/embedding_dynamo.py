"""Vocabulary-sharded embedding lookup as a graph exporter writes it
(tests/kernels/embedding_dynamo.py:7-79 of the reference): this shard holds
rows [0, 16000) of a 32000-token vocabulary; ids outside the shard read row
0 and are zeroed.  Membership is computed with boolean bitwise ops, the row
offset by integer multiplies of booleans, and the zeroing by ``where`` with
a scalar -- the op mix of the exported graph (its second, empty id range
[32000, 32000) included)."""

import numpy as np

from nkipy_amd.core.specs import CommonTypes, KernelSpec, ShapeSpec, TensorInputSpec

VOCAB = 32000
SHARD_ROWS = 16000


def sharded_embedding(ids, table):
    lo, hi = 0, SHARD_ROWS
    in_shard = np.bitwise_and(np.greater_equal(ids, lo), np.less(ids, hi))
    in_empty = np.bitwise_and(np.greater_equal(ids, VOCAB), np.less(ids, VOCAB))
    offset = np.add(np.multiply(in_shard, lo, dtype=np.int32),
                    np.multiply(in_empty, SHARD_ROWS, dtype=np.int32))
    hit = np.bitwise_or(in_shard, in_empty)
    local = np.multiply(hit, np.subtract(ids, offset))
    rows = np.take(table, local, axis=0)
    miss = np.expand_dims(np.logical_not(hit), -1)
    return np.where(miss, np.float32(0.0), rows)


_rng = np.random.default_rng(7)
IDS = _rng.integers(0, VOCAB, (1, 128)).astype(np.int32)
TABLE = _rng.uniform(0.0, 1.0, (SHARD_ROWS, 2048)).astype(np.float32)

kernel_specs = [KernelSpec(
    function=sharded_embedding,
    inputs=[TensorInputSpec(shape_spec=ShapeSpec(dims=[None, None], default=(1, 128)),
                            dtype_spec=CommonTypes.INTS, default_value=IDS, description="token ids"),
            TensorInputSpec(shape_spec=ShapeSpec(dims=[None, None], default=(SHARD_ROWS, 2048)),
                            dtype_spec=CommonTypes.FLOATS, default_value=TABLE,
                            description="this shard's embedding rows")],
    description="embedding lookup of one vocabulary shard with masking")]
