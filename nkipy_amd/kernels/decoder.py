"""Llama-style decoder layer with fp8 weights (prefill), as NumPy kernels.

The layer of tests/kernels/llama_decoder_dynamo.py:95-337 and examples/
models/qwen3/kernels/transformer_layer.py:17-66, written the way those
kernels write it:

    h    = rmsnorm(x) ;  q, k, v = split(h @ Wqkv^T)          (fused QKV)
    q, k = rope(q), rope(k)                                    (split-half)
    o    = softmax(q k^T / sqrt(d) + causal mask) v            (GQA via np.repeat)
    z    = x + o @ Wo^T
    y    = z + (silu(rmsnorm(z) @ Wg^T) * (rmsnorm(z) @ Wu^T)) @ Wd^T

Weights are torch-Linear (out, in) fp8 e4m3 codes with a per-output-channel
fp32 scale, dequantised in the kernel body as ``w8.astype(f32) * scale``
(the GEMM kernel reads the codes and applies the scale in its epilogue).
Activations are stored in the input's dtype (bf16); products, softmax and
the rotary embedding are computed in fp32.  The RMSNorm follows the cast
points of examples/models/qwen3/kernels/rmsnorm.py:4-21.
"""

import numpy as np

from nkipy_amd.kernels.feedforward import silu_kernel_
from nkipy_amd.kernels.rmsnorm import rmsnorm_kernel
from nkipy_amd.kernels.softmax import softmax_kernel

MASK_VALUE = -1.0e5


def rope_tables(head_dim, seq_len, theta):
    """cos / sin tables (seq_len, head_dim / 2) in fp32: angle = position *
    theta^(-2i / head_dim), as examples/models/qwen3/kernels/rope.py:4-20
    computes them (float64 frequencies, fp32 cos / sin)."""
    inv_freq = 1.0 / (theta ** (np.arange(0, head_dim, 2)[: head_dim // 2] / head_dim))
    angles = np.outer(np.arange(seq_len, dtype=np.float32), inv_freq)
    return np.cos(angles, dtype=np.float32), np.sin(angles, dtype=np.float32)


def rope_kernel(x, cos, sin):
    """Split-half rotary embedding of x (B, S, H, D) with tables (S, D/2),
    in fp32 (examples/models/qwen3/kernels/rope.py:23-48)."""
    c = cos[None, :, None, :]
    s = sin[None, :, None, :]
    half = x.shape[-1] // 2
    x0 = x[:, :, :, :half]
    x1 = x[:, :, :, half:]
    return np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], axis=-1)


def causal_gqa_attention_kernel(xq, xk, xv):
    """Causal softmax attention, q (B, S, Hq, D), k / v (B, S, Hkv, D) ->
    (B, S, Hq * D) in the input dtype.  KV heads are shared by groups of
    Hq / Hkv query heads (np.repeat, examples/models/qwen3/kernels/
    attention.py:15-22,109-110); scores, softmax and the weighted sum of
    values are fp32."""
    B, S, Hq, D = xq.shape
    n_rep = Hq // xk.shape[2]
    keys = np.repeat(xk, n_rep, axis=2)
    values = np.repeat(xv, n_rep, axis=2)
    q = xq.transpose(0, 2, 1, 3).astype(np.float32)
    kt = keys.transpose(0, 2, 3, 1).astype(np.float32)
    v = values.transpose(0, 2, 1, 3).astype(np.float32)
    scores = np.matmul(q, kt) / np.float32(np.sqrt(D))
    mask = np.triu(np.full((S, S), MASK_VALUE, dtype=np.float32), k=1)
    probs = softmax_kernel(scores + mask)
    out = np.matmul(probs, v)
    return out.transpose(0, 2, 1, 3).astype(xq.dtype).reshape(B, S, Hq * D)


def dequantize_fp8(w8, scale):
    """(out, in) fp8 codes times the per-output-channel fp32 scale."""
    return w8.astype(np.float32) * np.expand_dims(scale, 1)


def linear_fp8(x, w8, scale):
    """x @ dequant(W)^T, fp32 result."""
    return np.matmul(x, np.transpose(dequantize_fp8(w8, scale)))


def qkv_rope_fp8(h, wqkv, wqkv_scale, n_heads, n_kv_heads, rope_theta):
    """Fused QKV projection split into heads, RoPE on q and k:
    h (B, S, hidden) -> q (B, S, Hq, D), k / v (B, S, Hkv, D)."""
    B, S, _ = h.shape
    head_dim = wqkv.shape[0] // (n_heads + 2 * n_kv_heads)
    qkv = linear_fp8(h, wqkv, wqkv_scale).astype(h.dtype)
    q_end = n_heads * head_dim
    k_end = q_end + n_kv_heads * head_dim
    xq, xk, xv = np.split(qkv, [q_end, k_end], axis=-1)
    xq = xq.reshape(B, S, n_heads, head_dim)
    xk = xk.reshape(B, S, n_kv_heads, head_dim)
    xv = xv.reshape(B, S, n_kv_heads, head_dim)
    cos, sin = rope_tables(head_dim, S, rope_theta)
    xq = rope_kernel(xq, cos, sin).astype(h.dtype)
    xk = rope_kernel(xk, cos, sin).astype(h.dtype)
    return xq, xk, xv


def attention_block_fp8(x, norm_weight, wqkv, wqkv_scale, wo, wo_scale,
                        n_heads=32, n_kv_heads=8, rope_theta=5.0e5, eps=1e-5):
    """z = x + o_proj(attention(rope(qkv(rmsnorm(x))))), x (B, S, hidden)."""
    h = rmsnorm_kernel(x, norm_weight, eps)
    xq, xk, xv = qkv_rope_fp8(h, wqkv, wqkv_scale, n_heads, n_kv_heads, rope_theta)
    attn = causal_gqa_attention_kernel(xq, xk, xv)
    return x + linear_fp8(attn, wo, wo_scale).astype(x.dtype)


def mlp_block_fp8(z, norm_weight, w_gate, w_gate_scale, w_up, w_up_scale, w_down, w_down_scale,
                  eps=1e-5):
    """y = z + down(silu(gate(rmsnorm(z))) * up(rmsnorm(z)))."""
    h = rmsnorm_kernel(z, norm_weight, eps)
    act = (silu_kernel_(linear_fp8(h, w_gate, w_gate_scale)) * linear_fp8(h, w_up, w_up_scale)).astype(z.dtype)
    return z + linear_fp8(act, w_down, w_down_scale).astype(z.dtype)


def llama_decoder_layer_fp8(x, attn_norm_weight, wqkv, wqkv_scale, wo, wo_scale,
                            mlp_norm_weight, w_gate, w_gate_scale, w_up, w_up_scale,
                            w_down, w_down_scale, n_heads=32, n_kv_heads=8,
                            rope_theta=5.0e5, eps=1e-5):
    """One decoder layer, x (B, S, hidden) in the activation dtype."""
    z = attention_block_fp8(x, attn_norm_weight, wqkv, wqkv_scale, wo, wo_scale,
                            n_heads, n_kv_heads, rope_theta, eps)
    return mlp_block_fp8(z, mlp_norm_weight, w_gate, w_gate_scale, w_up, w_up_scale,
                         w_down, w_down_scale, eps)
