"""Chunked causal linear attention, written as a vectorised NumPy kernel.

phi(x) = elu(x) + 1.  The sequence is cut into chunks of ``chunk`` steps:
per chunk, the key-value state before the chunk is the exclusive prefix sum
of the per-chunk phi(K)^T V products; the output combines the inter-chunk
term phi(Q) S with the causally masked intra-chunk term
(phi(Q) phi(K)^T * tril) V, normalised by phi(Q) z plus the masked row sums.
No reference kernel computes this (the reference's recurrent linear
attention is DeltaNet, examples/linear_attention/deltanet.py:74-128, whose
per-step Python loop unrolls into O(T) graph nodes); this formulation keeps
the traced graph a fixed size for any T.
"""

import numpy as np


def elu_plus_one(x):
    return np.where(x > 0, x + 1.0, np.exp(x))


def chunked_linear_attention_kernel(q, k, v, chunk=64):
    B, H, T, D = q.shape
    Dv = v.shape[-1]
    n = T // chunk
    qf = elu_plus_one(q.astype(np.float32)).reshape(B, H, n, chunk, D)
    kf = elu_plus_one(k.astype(np.float32)).reshape(B, H, n, chunk, D)
    vf = v.astype(np.float32).reshape(B, H, n, chunk, Dv)
    kv = np.matmul(np.swapaxes(kf, -1, -2), vf)          # per-chunk phi(K)^T V
    state = np.cumsum(kv, axis=2) - kv                   # state before each chunk
    ksum = np.sum(kf, axis=3)                            # per-chunk colsum phi(K)
    z = np.cumsum(ksum, axis=2) - ksum                   # normaliser before each chunk
    scores = np.matmul(qf, np.swapaxes(kf, -1, -2))      # intra-chunk phi(Q) phi(K)^T
    scores = scores * np.tril(np.ones((chunk, chunk), dtype=np.float32))
    num = np.matmul(qf, state) + np.matmul(scores, vf)
    den = np.sum(qf * np.expand_dims(z, 3), axis=-1, keepdims=True) + np.sum(scores, axis=-1, keepdims=True)
    return (num / den).reshape(B, H, T, Dv).astype(q.dtype)
