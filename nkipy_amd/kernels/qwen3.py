"""Qwen3 attention and greedy sampling as NumPy kernels, on one GPU.

``qwen3_attention_kernel`` follows examples/models/qwen3/kernels/
attention.py:25-156 with a tensor-parallel degree of 1 (the all-reduce of
the output projection is the identity): fused QKV projection split into
heads, per-head RMSNorm of q and k, RoPE from a cos / sin cache
(kernels/rope.py:4-48), the KV-cache write (``cache[:, :S] = k`` for
prefill, ``cache[:, start_pos] = k`` for one decode token, with start_pos a
runtime tensor), GQA by ``np.repeat``, scores over the whole cache
rounded to bf16, the causal mask row(s) of the current positions (-1e5 above
the diagonal), softmax, weighted values and the output projection.

``greedy_sampling`` follows kernels/sampling.py:113-148 on one device: the
final RMSNorm, logits of the last position and the index of the largest
logit by ``topk(k=1)``.
"""

import numpy as np

from nkipy_amd.core import tensor_apis
from nkipy_amd.kernels.rmsnorm import rmsnorm_kernel
from nkipy_amd.kernels.softmax import softmax_kernel

MASK_VALUE = -100000.0


def compute_cos_sin_cache(head_dim, max_seq_len, base=10000, dtype=np.float32):
    """cos / sin of position x frequency, frequencies base^(-2i/d) in float64
    (trace-time constants)."""
    inv = 1.0 / (base ** (np.arange(0, head_dim, 2)[: head_dim // 2] / head_dim))
    ang = np.outer(np.arange(max_seq_len, dtype=np.float32), inv)
    return np.cos(ang, dtype=np.float32).astype(dtype), np.sin(ang, dtype=np.float32).astype(dtype)


def apply_rotary_emb_kernel(xq, xk, freqs_cos, freqs_sin):
    """Split-half rotation of q and k (B, S, H, D) by tables (S, D/2)."""
    c = np.expand_dims(freqs_cos, axis=(0, 2))
    s = np.expand_dims(freqs_sin, axis=(0, 2))
    h = xq.shape[-1] // 2

    def rot(x):
        x0, x1 = x[:, :, :, :h], x[:, :, :, h:]
        return np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], axis=-1)

    return rot(xq), rot(xk)


def qwen3_attention_kernel(x, qkv_weight, q_norm_weight, k_norm_weight, norm_eps, n_heads, head_dim,
                           n_kv_heads, cache_k, cache_v, start_pos, o_weight, rope_base=1000000):
    """x (B, S, hidden) -> (B, S, hidden); updates cache_k / cache_v
    (B, max_seq, n_kv_heads, head_dim) in place.  ``start_pos=None`` is
    prefill of positions 0..S-1; otherwise S == 1 and the token sits at
    position start_pos (an int32 array of shape (1,))."""
    prefill = start_pos is None
    B, S, _ = x.shape
    q_end = n_heads * head_dim
    k_end = q_end + n_kv_heads * head_dim
    xq, xk, xv = np.split(np.matmul(x, qkv_weight), [q_end, k_end], axis=x.ndim - 1)
    xq = rmsnorm_kernel(xq.reshape(B, S, n_heads, head_dim), q_norm_weight, norm_eps)
    xk = rmsnorm_kernel(xk.reshape(B, S, n_kv_heads, head_dim), k_norm_weight, norm_eps)
    xv = xv.reshape(B, S, n_kv_heads, head_dim)

    # trace-time constants are built in fp32 and cast by traced ops (a host
    # astype to bf16 needs ml_dtypes, which this environment may lack)
    max_seq = cache_k.shape[1]
    cos, sin = compute_cos_sin_cache(head_dim, max_seq, base=rope_base)
    cos = tensor_apis.constant(cos).astype(x.dtype)
    sin = tensor_apis.constant(sin).astype(x.dtype)
    if prefill:
        cos, sin = cos[0:S], sin[0:S]
    else:
        cos, sin = cos[start_pos], sin[start_pos]
    xq, xk = apply_rotary_emb_kernel(xq, xk, cos, sin)

    if prefill:
        cache_k[:, :S] = xk
        cache_v[:, :S] = xv
    else:
        cache_k[:, start_pos] = xk
        cache_v[:, start_pos] = xv

    out = cached_attention(xq, cache_k, cache_v, start_pos).reshape(B, S, -1)
    return np.matmul(out, o_weight)


def cached_attention(xq, cache_k, cache_v, start_pos=None):
    """Attention of the queries xq (B, S, Hq, D) over the whole KV cache
    (B, MAXS, Hkv, D), as examples/models/qwen3/kernels/attention.py:107-143
    computes it: GQA by ``np.repeat``, scores (q @ k^T) / sqrt(D) cast to the
    activation dtype, plus the mask rows of the current positions (rows
    0..S-1 for prefill, row start_pos for one decode token) of a constant
    (MAXS, MAXS) triu mask, softmax, @ values -> (B, S, Hq, D)."""
    B, S, n_heads, head_dim = xq.shape
    max_seq, n_kv_heads = cache_k.shape[1], cache_k.shape[2]
    n_rep = n_heads // n_kv_heads
    keys = np.repeat(cache_k, n_rep, axis=2) if n_rep > 1 else cache_k
    values = np.repeat(cache_v, n_rep, axis=2) if n_rep > 1 else cache_v
    q = xq.transpose(0, 2, 1, 3)
    k = keys.transpose(0, 2, 1, 3)
    v = values.transpose(0, 2, 1, 3)
    scores = (q @ k.transpose(0, 1, 3, 2)) / np.float32(np.sqrt(head_dim))
    scores = scores.astype(xq.dtype)
    mask = tensor_apis.constant(np.triu(np.ones((max_seq, max_seq)) * MASK_VALUE, k=1).astype(np.float32))
    mask = mask.astype(scores.dtype)
    if start_pos is None:
        scores = scores + np.expand_dims(mask[:S, :max_seq], axis=[0, 1])
    else:
        scores = scores + np.expand_dims(mask[start_pos, :max_seq], axis=[0, 1])
    out = softmax_kernel(scores) @ v
    return out.transpose(0, 2, 1, 3)


def prefill_attention_kernel(xq, cache_k, cache_v):
    """The prefill half of :func:`cached_attention` as a kernel of its own."""
    return cached_attention(xq, cache_k, cache_v)


def greedy_sampling(h, norm_weight, lm_head_weight, norm_eps):
    """Index of the largest logit of the last position: (B, S, H) -> (B, 1)."""
    h = rmsnorm_kernel(h, norm_weight, norm_eps)
    logits = h[:, -1, :] @ lm_head_weight
    _, next_id = tensor_apis.topk(logits, k=1, axis=1)
    return next_id
