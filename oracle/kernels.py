"""NumPy restatements of the reference's CPU path for the hot-path kernels
(test infrastructure only; see oracle/__init__.py).

``*_kernel`` functions are the float32 NumPy formulas the reference runs on
the CPU; ``*_f64`` functions are float64 brute-force forms used to pin them.
bf16 inputs are float32 arrays holding bf16-rounded values.
"""

from __future__ import annotations

import numpy as np

from oracle.numerics import bf16_round

# ---------------------------------------------------------------------------
# softmax -- README.md:125-128, tests/kernels/softmax.py:7-10
# ---------------------------------------------------------------------------


def softmax_kernel(x):
    exp_x = np.exp(x - np.max(x, axis=-1, keepdims=True))
    sum_x = np.sum(exp_x, axis=-1, keepdims=True)
    return exp_x / sum_x


def softmax_steps_rounded(x, rnd=bf16_round):
    """softmax_kernel evaluated in a 16-bit type op by op (the reference's
    softmax on bf16 scores, examples/models/qwen3/kernels/softmax.py:4-6):
    x - max, exp, the sum (accumulated in fp32) and the divide each rounded
    by ``rnd``.  x holds values of that type as float32."""
    x = np.asarray(x, np.float32)
    e = rnd(np.exp(rnd(x - x.max(-1, keepdims=True))))
    tot = rnd(e.sum(-1, keepdims=True, dtype=np.float32))
    return rnd(e / tot)


def softmax_f64(x):
    x = np.asarray(x, dtype=np.float64)
    out = np.empty_like(x)
    flat = x.reshape(-1, x.shape[-1])
    o = out.reshape(-1, x.shape[-1])
    for i, row in enumerate(flat):
        e = np.exp(row - row.max())
        o[i] = e / e.sum()
    return out


# ---------------------------------------------------------------------------
# RMSNorm -- examples/models/qwen3/kernels/rmsnorm.py:4-21 (cast points kept:
# upcast to fp32, mean of squares, (z + eps) cast back to the fp32 dtype,
# x / sqrt(z), times weight, cast to the input dtype); residual as
# examples/models/qwen3/kernels/transformer_layer.py:60 (z = x + h1, in the
# storage dtype).
# ---------------------------------------------------------------------------


def rmsnorm_kernel(x, weight, eps, compute_dtype=np.float32, round_out=None):
    x = np.asarray(x).astype(compute_dtype)
    weight = np.asarray(weight).astype(compute_dtype)
    z = np.square(x)
    z = np.mean(z, axis=-1, keepdims=True)
    z = (z + np.float32(eps)).astype(x.dtype)
    z = x / np.sqrt(z)
    res = z * weight
    return round_out(res) if round_out is not None else res


def residual_rmsnorm_bf16(x, r, weight, eps):
    """bf16 storage: h = bf16(x + r); out = bf16(rmsnorm(h) * w)."""
    h = bf16_round(np.asarray(x, np.float32) + np.asarray(r, np.float32))
    return rmsnorm_kernel(h, weight, eps, round_out=bf16_round)


def rmsnorm_f64(h, weight, eps):
    h = np.asarray(h, dtype=np.float64)
    ms = np.array([np.dot(row, row) / row.size for row in h.reshape(-1, h.shape[-1])])
    ms = ms.reshape(h.shape[:-1] + (1,))
    return h / np.sqrt(ms + eps) * np.asarray(weight, np.float64)


# ---------------------------------------------------------------------------
# SwiGLU feed-forward -- examples/models/qwen3/kernels/feedforward.py:4-18
# (silu(x) = x * (1 / (1 + exp(-x))); gate_up fused then split), bias variant
# examples/models/qwen3_embedding/kernels/ffn.py:11-46.
# ---------------------------------------------------------------------------


def silu(x):
    return x * (1 / (1 + np.exp(-x)))


def swiglu_mlp(x, w_gate, w_up, w_down, round_h=None):
    """fp32 products and SwiGLU; ``round_h`` rounds the activation h (the
    intermediate a bf16 kernel stores) before the down projection."""
    x = np.asarray(x, np.float32)
    g = x @ np.asarray(w_gate, np.float32)
    u = x @ np.asarray(w_up, np.float32)
    h = silu(g) * u
    if round_h is not None:
        h = round_h(h)
    return h @ np.asarray(w_down, np.float32)


def feedforward_fused(x, gate_up, down, gate_up_bias=None, down_bias=None, round_h=None):
    mm = np.asarray(x, np.float32) @ np.asarray(gate_up, np.float32)
    if gate_up_bias is not None:
        mm = mm + gate_up_bias
    g, u = np.split(mm, 2, axis=-1)
    h = silu(g) * u
    if round_h is not None:
        h = round_h(h)
    out = h @ np.asarray(down, np.float32)
    if down_bias is not None:
        out = out + down_bias
    return out


def matmul_f64(a, b):
    """Textbook triple loop (tiny shapes only)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    M, K = a.shape
    K2, N = b.shape
    assert K == K2
    c = np.zeros((M, N))
    for i in range(M):
        for j in range(N):
            s = 0.0
            for k in range(K):
                s += a[i, k] * b[k, j]
            c[i, j] = s
    return c


# ---------------------------------------------------------------------------
# Chunked causal linear attention.  Nothing in the reference computes it;
# the nearest analogue is the recurrent DeltaNet kernel
# (examples/linear_attention/deltanet.py:74-128).  Feature map phi = elu + 1.
#   o_t = phi(q_t)^T S_t / (phi(q_t)^T z_t),
#   S_t = sum_{s<=t} phi(k_s) v_s^T,  z_t = sum_{s<=t} phi(k_s)
# ---------------------------------------------------------------------------


def elu_plus_one(x):
    x = np.asarray(x)
    return np.where(x > 0, x + 1, np.exp(np.minimum(x, 0)))


def linear_attention_chunked(q, k, v, chunk=64):
    """Chunk-by-chunk recurrence with an fp32 d x d state per head:
    inter-chunk phi(Q) S_prev plus the masked intra-chunk (phi(Q) phi(K)^T) V."""
    q = np.asarray(q, np.float32)
    k = np.asarray(k, np.float32)
    v = np.asarray(v, np.float32)
    B, H, T, D = q.shape
    assert T % chunk == 0
    qf, kf = elu_plus_one(q).astype(np.float32), elu_plus_one(k).astype(np.float32)
    out = np.empty((B, H, T, v.shape[-1]), np.float32)
    mask = np.tril(np.ones((chunk, chunk), np.float32))
    for b in range(B):
        for h in range(H):
            S = np.zeros((D, v.shape[-1]), np.float32)
            z = np.zeros(D, np.float32)
            for c0 in range(0, T, chunk):
                Q = qf[b, h, c0:c0 + chunk]
                K = kf[b, h, c0:c0 + chunk]
                V = v[b, h, c0:c0 + chunk]
                A = (Q @ K.T) * mask
                num = Q @ S + A @ V
                den = Q @ z + A.sum(axis=1)
                out[b, h, c0:c0 + chunk] = num / den[:, None]
                S = S + K.T @ V
                z = z + K.sum(axis=0)
    return out


def linear_attention_quadratic_f64(q, k, v):
    """O(T^2) masked form in float64 (tiny T)."""
    qf = elu_plus_one(np.asarray(q, np.float64))
    kf = elu_plus_one(np.asarray(k, np.float64))
    v = np.asarray(v, np.float64)
    T = q.shape[-2]
    mask = np.tril(np.ones((T, T)))
    A = np.einsum("bhtd,bhsd->bhts", qf, kf) * mask
    return np.einsum("bhts,bhsd->bhtd", A, v) / A.sum(-1, keepdims=True)


# ---------------------------------------------------------------------------
# Causal GQA attention -- examples/models/qwen3/kernels/attention.py:109-140
# (np.repeat of KV heads, q @ k^T / sqrt(d), causal mask, softmax, @ v).
# q (B, S, Hq, D), k / v (B, S, Hkv, D) -> (B, S, Hq, D).
# ---------------------------------------------------------------------------


def causal_gqa_attention(q, k, v, scale=None, causal=True):
    """``causal=False`` drops the mask (every query sees every key)."""
    q = np.asarray(q, np.float32)
    k = np.asarray(k, np.float32)
    v = np.asarray(v, np.float32)
    B, S, Hq, D = q.shape
    rep = Hq // k.shape[2]
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    kk = np.repeat(k, rep, axis=2).transpose(0, 2, 3, 1)   # (B, Hq, D, S)
    vv = np.repeat(v, rep, axis=2).transpose(0, 2, 1, 3)   # (B, Hq, S, D)
    s = (q.transpose(0, 2, 1, 3) @ kk) * np.float32(scale)
    if causal:
        s = s + np.triu(np.full((S, S), -np.inf, np.float32), 1)
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    p = p / p.sum(-1, keepdims=True)
    return (p @ vv).transpose(0, 2, 1, 3)


def causal_attention_f64_loop(q, k, v, causal=True):
    """Per-query float64 loop (tiny shapes): pins causal_gqa_attention."""
    q, k, v = (np.asarray(a, np.float64) for a in (q, k, v))
    B, S, Hq, D = q.shape
    rep = Hq // k.shape[2]
    out = np.zeros_like(q)
    for b in range(B):
        for h in range(Hq):
            for t in range(S):
                n = t + 1 if causal else S
                w = np.array([q[b, t, h] @ k[b, s, h // rep] for s in range(n)]) / np.sqrt(D)
                w = np.exp(w - w.max())
                out[b, t, h] = (w[:, None] * v[b, :n, h // rep]).sum(0) / w.sum()
    return out


# ---------------------------------------------------------------------------
# Rotary embedding -- examples/models/qwen3/kernels/rope.py:4-48 (tables:
# float64 frequencies 1 / theta^(2i/d), fp32 cos / sin of position * freq;
# split-half rotation in fp32).
# ---------------------------------------------------------------------------


def rope_tables(head_dim, seq_len, theta):
    freqs = 1.0 / (theta ** (np.arange(0, head_dim, 2)[: head_dim // 2] / head_dim))
    ang = np.outer(np.arange(seq_len, dtype=np.float32), freqs)
    return np.cos(ang, dtype=np.float32), np.sin(ang, dtype=np.float32)


def rope_split_half(x, cos, sin):
    """x (B, S, H, D) fp32 values; tables (S, D/2).  fp32 result."""
    x = np.asarray(x, np.float32)
    h = x.shape[-1] // 2
    c = cos[None, :, None, :]
    s = sin[None, :, None, :]
    x0, x1 = x[..., :h], x[..., h:]
    return np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], axis=-1)


def rope_complex_f64(x, theta):
    """Rotation as complex multiplication in float64 (pins rope_split_half):
    (x0 + i x1) * exp(i * pos * freq)."""
    x = np.asarray(x, np.float64)
    B, S, H, D = x.shape
    h = D // 2
    freqs = theta ** (-2.0 * np.arange(h) / D)
    ph = np.exp(1j * np.arange(S)[:, None] * freqs[None, :])[None, :, None, :]
    z = (x[..., :h] + 1j * x[..., h:]) * ph
    return np.concatenate([z.real, z.imag], axis=-1)


def rope_split_half_bf16_steps(x, cos, sin):
    """The rotation as examples/models/qwen3/kernels/rope.py:23-48 computes
    it on bf16 arrays (attention.py:84-97 casts the tables to the activation
    dtype): x (B, S, H, D) and the tables (S or 1, D/2) hold bf16 values, and
    every product, the difference and the sum are rounded to bf16 (each
    product of two bf16 values is exact in fp32)."""
    x = np.asarray(x, np.float32)
    h = x.shape[-1] // 2
    c = bf16_round(np.asarray(cos, np.float32))[None, :, None, :]
    s = bf16_round(np.asarray(sin, np.float32))[None, :, None, :]
    x0, x1 = x[..., :h], x[..., h:]
    return np.concatenate([bf16_round(bf16_round(x0 * c) - bf16_round(x1 * s)),
                           bf16_round(bf16_round(x0 * s) + bf16_round(x1 * c))], axis=-1)


def qwen3_head_prologue(qkv, q_norm_weight, k_norm_weight, eps, n_heads, n_kv_heads, head_dim, positions,
                        theta):
    """q and k of examples/models/qwen3/kernels/attention.py:72-97 from the
    bf16 QKV projection (B, S, (Hq + 2 Hkv) D): split into heads, per-head
    RMSNorm (fp32 arithmetic, bf16 result), the bf16-step rotation with the
    fp32 tables cast to bf16 and taken at ``positions`` (one per token of
    the sequence axis).  Returns (q, k) as bf16 values."""
    qkv = np.asarray(qkv, np.float32)
    B, S, _ = qkv.shape
    D = head_dim
    q = qkv[..., :n_heads * D].reshape(B, S, n_heads, D)
    k = qkv[..., n_heads * D:(n_heads + n_kv_heads) * D].reshape(B, S, n_kv_heads, D)
    q = rmsnorm_kernel(q, q_norm_weight, eps, round_out=bf16_round)
    k = rmsnorm_kernel(k, k_norm_weight, eps, round_out=bf16_round)
    cos, sin = rope_tables(D, int(np.max(positions)) + 1, theta)
    pos = np.asarray(positions)
    return (rope_split_half_bf16_steps(q, cos[pos], sin[pos]),
            rope_split_half_bf16_steps(k, cos[pos], sin[pos]))


# ---------------------------------------------------------------------------
# fp8 decoder layer -- tests/kernels/llama_decoder_dynamo.py:95-337 with the
# weights of a torch Linear (out, in) stored as e4m3fn codes and a per-output
# channel fp32 scale; the cast points of the NumPy kernel
# (bf16 storage after each projection, after RoPE, after attention, after
# each residual add; fp32 products, softmax and RoPE).
# ---------------------------------------------------------------------------


def linear_fp8(x, codes, scale):
    from oracle.numerics import dequantize_e4m3fn

    w = dequantize_e4m3fn(codes, scale, axis=1)
    return np.asarray(x, np.float32) @ w.T


def decoder_attention_fp8(x, w, pos0=0):
    """Returns (attention output before o_proj (B, S, Hq*D), z = x + o_proj).
    ``pos0``: position of the first token (the RoPE tables start there)."""
    B, S, hid = x.shape
    Hq, Hkv, eps, theta = w["n_heads"], w["n_kv_heads"], w["eps"], w["rope_theta"]
    D = hid // Hq
    h = rmsnorm_kernel(x, w["attn_norm"], eps, round_out=bf16_round)
    qkv = bf16_round(linear_fp8(h, w["wqkv"], w["wqkv_scale"]))
    q = qkv[..., :Hq * D].reshape(B, S, Hq, D)
    k = qkv[..., Hq * D:(Hq + Hkv) * D].reshape(B, S, Hkv, D)
    v = qkv[..., (Hq + Hkv) * D:].reshape(B, S, Hkv, D)
    cos, sin = rope_tables(D, pos0 + S, theta)
    cos, sin = cos[pos0:], sin[pos0:]
    q = bf16_round(rope_split_half(q, cos, sin))
    k = bf16_round(rope_split_half(k, cos, sin))
    a = bf16_round(causal_gqa_attention(q, k, v)).reshape(B, S, Hq * D)
    z = bf16_round(x + bf16_round(linear_fp8(a, w["wo"], w["wo_scale"])))
    return a, z


def decoder_mlp_fp8(z, w):
    """Returns (silu(gate) * up in bf16, y = z + down)."""
    h = rmsnorm_kernel(z, w["mlp_norm"], w["eps"], round_out=bf16_round)
    g = linear_fp8(h, w["w_gate"], w["w_gate_scale"])
    u = linear_fp8(h, w["w_up"], w["w_up_scale"])
    act = bf16_round(silu(g) * u)
    y = bf16_round(z + bf16_round(linear_fp8(act, w["w_down"], w["w_down_scale"])))
    return act, y


def decoder_layer_fp8(x, w):
    a, z = decoder_attention_fp8(x, w)
    act, y = decoder_mlp_fp8(z, w)
    return {"attn": a, "z": z, "act": act, "y": y}


def decoder_layer_fp8_rows(x_seq, w, rows):
    """The layer for selected positions of ONE sequence x_seq (S, hidden):
    projections of every position up to max(rows), attention and everything
    after it only for ``rows``.  Same cast points as decoder_layer_fp8."""
    S, hid = x_seq.shape
    Hq, Hkv, eps, theta = w["n_heads"], w["n_kv_heads"], w["eps"], w["rope_theta"]
    D = hid // Hq
    rows = np.asarray(rows)
    T = int(rows.max()) + 1
    x = np.asarray(x_seq[:T], np.float32)
    h = rmsnorm_kernel(x, w["attn_norm"], eps, round_out=bf16_round)
    qkv = bf16_round(linear_fp8(h, w["wqkv"], w["wqkv_scale"]))
    cos, sin = rope_tables(D, S, theta)
    q = bf16_round(rope_split_half(qkv[None, rows, :Hq * D].reshape(1, len(rows), Hq, D),
                                   cos[rows], sin[rows]))[0]
    k = bf16_round(rope_split_half(qkv[None, :, Hq * D:(Hq + Hkv) * D].reshape(1, T, Hkv, D),
                                   cos[:T], sin[:T]))[0]
    v = qkv[:, (Hq + Hkv) * D:].reshape(T, Hkv, D)
    rep = Hq // Hkv
    a = np.empty((len(rows), Hq, D), np.float32)
    for i, t in enumerate(rows):
        for hh in range(Hq):
            g = hh // rep
            s = (k[:t + 1, g] @ q[i, hh]) * np.float32(1.0 / np.sqrt(D))
            p = np.exp(s - s.max())
            a[i, hh] = (p / p.sum()) @ v[:t + 1, g]
    a = bf16_round(a).reshape(len(rows), Hq * D)
    z = bf16_round(x[rows] + bf16_round(linear_fp8(a, w["wo"], w["wo_scale"])))
    act, y = decoder_mlp_fp8(z, w)
    return {"attn": a, "z": z, "act": act, "y": y}


def decoder_oproj_residual(x, attn, w):
    """z = x + o_proj(attn), both rounded to bf16 (x, attn: (..., hidden))."""
    return bf16_round(np.asarray(x, np.float32) + bf16_round(linear_fp8(attn, w["wo"], w["wo_scale"])))


def decoder_down_residual(z, act, w):
    """y = z + down(act), both rounded to bf16."""
    return bf16_round(np.asarray(z, np.float32) + bf16_round(linear_fp8(act, w["w_down"], w["w_down_scale"])))


# ---------------------------------------------------------------------------
# top-k -- nkipy/src/nkipy/core/ops/nn.py:22-60 (CPU: argpartition of -x,
# then the k picks sorted best first; indices uint32).  Rows are assumed free
# of ties (the reference leaves their order to argpartition / argsort).
# ---------------------------------------------------------------------------


def topk(x, k, axis=-1, is_ascend=False):
    x = np.asarray(x)
    keys = x if is_ascend else -x
    part = np.argpartition(keys, k - 1, axis=axis)
    idx = np.take(part, np.arange(k), axis=axis)
    vals = np.take_along_axis(keys, idx, axis=axis)
    order = np.argsort(vals, axis=axis)
    idx = np.take_along_axis(idx, order, axis=axis)
    return np.take_along_axis(x, idx, axis=axis), idx.astype(np.uint32)


def greedy_sampling_bf16(h, norm_weight, lm_head, eps):
    """examples/models/qwen3/kernels/sampling.py:113-148 on one device: final
    RMSNorm (bf16 out), logits of the last position rounded to bf16 (fp32
    accumulation), index of the largest logit.  (B, S, H) -> (B, 1) uint32."""
    hn = rmsnorm_kernel(h, norm_weight, eps, round_out=bf16_round)
    logits = bf16_round(np.asarray(hn[:, -1, :], np.float32) @ np.asarray(lm_head, np.float32))
    return topk(logits, 1, axis=1)[1]


# ---------------------------------------------------------------------------
# Decode attention -- examples/models/qwen3/kernels/attention.py:101-140 at
# one decode position: the cache holds keys / values of positions 0..pos
# (the mask row of position pos removes the rest), q @ k^T divided by
# sqrt(d), softmax, weighted values.  The bf16 cast points of the traced
# NumPy code are optional: the product rounded to bf16 (a bf16 matmul), the
# scaled score rounded (``.astype(bf16)``), softmax evaluated in bf16 (each
# of s - m, exp, the fp32-accumulated sum and the quotient rounded).
# q (B, Hq, D), cache (B, Smax, Hkv, D) -> (B, Hq, D) fp32.
# ---------------------------------------------------------------------------


def decode_attention(q, cache_k, cache_v, pos, round_prod=False, round_score=False, softmax_bf16=False):
    q = np.asarray(q, np.float32)
    B, Hq, D = q.shape
    Hkv = cache_k.shape[2]
    rep = Hq // Hkv
    r = bf16_round
    n = int(pos) + 1
    out = np.zeros((B, Hq, D), np.float32)
    for b in range(B):
        for h in range(Hq):
            k = np.asarray(cache_k[b, :n, h // rep], np.float32)
            v = np.asarray(cache_v[b, :n, h // rep], np.float32)
            s = (k.astype(np.float64) @ q[b, h].astype(np.float64)).astype(np.float32)
            if round_prod:
                s = r(s)
            s = s / np.float32(np.sqrt(D))
            if round_score:
                s = r(s)
            d = s - s.max()
            e = np.exp(r(d) if softmax_bf16 else d)
            if softmax_bf16:
                e = r(e)
            tot = np.float32(e.sum(dtype=np.float32))
            p = e / (r(tot) if softmax_bf16 else tot)
            if softmax_bf16:
                p = r(p)
            out[b, h] = (p.astype(np.float64) @ v.astype(np.float64)).astype(np.float32)
    return out


def qwen3_decode_layer(x, qkv_weight, q_norm_weight, k_norm_weight, eps, n_heads, n_kv_heads, head_dim,
                       cache_k, cache_v, pos, o_weight, theta=1.0e6):
    """One decode token per sequence through examples/models/qwen3/kernels/
    attention.py:25-156 (tensor-parallel degree 1, start_pos = pos): the bf16
    QKV projection, the head prologue (:func:`qwen3_head_prologue`), the
    cache rows at pos overwritten with k and v, attention over the cache
    with the traced cast points (:func:`decode_attention`; the mask row adds
    -1e5 past pos, whose weights are exactly 0), the bf16 weighted values and
    the bf16 output projection.  Returns (out (B, 1, hidden), cache_k,
    cache_v) as bf16 values (the caches are copies)."""
    x = np.asarray(x, np.float32)
    B = x.shape[0]
    H, Hkv, D = n_heads, n_kv_heads, head_dim
    qkv = bf16_round((x.astype(np.float64) @ np.asarray(qkv_weight, np.float64)).astype(np.float32))
    q, k = qwen3_head_prologue(qkv, q_norm_weight, k_norm_weight, eps, H, Hkv, D, np.array([pos]), theta)
    v = qkv[..., (H + Hkv) * D:].reshape(B, 1, Hkv, D)
    ck = np.array(cache_k, np.float32, copy=True)
    cv = np.array(cache_v, np.float32, copy=True)
    ck[:, pos] = k[:, 0]
    cv[:, pos] = v[:, 0]
    att = bf16_round(decode_attention(q[:, 0], ck, cv, pos, True, True, True))
    out = att.reshape(B, 1, H * D).astype(np.float64) @ np.asarray(o_weight, np.float64)
    return bf16_round(out.astype(np.float32)), ck, cv


# ---------------------------------------------------------------------------
# Qwen3 prefill attention over a KV cache -- examples/models/qwen3/kernels/
# attention.py:107-140 with bf16 activations (start_pos None): keys / values
# are the whole cache (B, MAXS, Hkv, D) with np.repeat GQA; the product q k^T
# of bf16 operands is a bf16 array; ``/ np.float32(sqrt(D))`` promotes it to
# fp32, ``.astype(bf16)`` rounds the score; the mask rows [:S, :MAXS] of
# triu(ones * -1e5, k=1) cast to bf16 are added in bf16; the softmax
# (kernels/softmax.py:4-6) runs op by op in bf16 (max, subtract, exp, sum,
# divide, each result rounded); the bf16 weights @ values give bf16.
# Products accumulate in float64 and are rounded once (to fp32, then to the
# array's dtype); the bf16 sum accumulates in fp32 and is rounded once.
# ---------------------------------------------------------------------------


def qwen3_prefill_attention(q, cache_k, cache_v, rows=None, round_prod=True, round_score=True,
                            softmax_bf16=True, round_weights=True, causal=True):
    """q (B, S, Hq, D), caches (B, MAXS, Hkv, D), bf16 values in fp32 arrays
    -> (B, len(rows), Hq, D) fp32 holding the bf16 output values of the
    query positions ``rows`` (all S by default).  The flags drop single cast
    points (used to show that each one matters); ``round_weights=False``
    keeps each weight e / sum(e) unrounded (the one cast point a flash
    kernel, which divides after the weighted sum, does not take);
    ``causal=False`` drops the mask (every query sees every cache row)."""
    q = np.asarray(q, np.float32)
    B, S, Hq, D = q.shape
    MAXS, Hkv = cache_k.shape[1], cache_k.shape[2]
    rep = Hq // Hkv
    rows = np.arange(S) if rows is None else np.asarray(rows)
    r = bf16_round
    keep = r if softmax_bf16 else (lambda a: a)
    if causal:
        mask = r(np.triu(np.ones((MAXS, MAXS)) * -100000, k=1).astype(np.float32))[rows, :MAXS]
    else:
        mask = np.zeros((len(rows), MAXS), np.float32)
    out = np.zeros((B, len(rows), Hq, D), np.float32)
    for b in range(B):
        for h in range(Hq):
            k = np.asarray(cache_k[b, :, h // rep], np.float64)
            v = np.asarray(cache_v[b, :, h // rep], np.float64)
            s = (q[b, rows, h].astype(np.float64) @ k.T).astype(np.float32)
            if round_prod:
                s = r(s)
            s = s / np.float32(np.sqrt(D))
            if round_score:
                s = r(s)
            s = r(s + mask) if round_score else s + mask
            d = keep(s - s.max(-1, keepdims=True))
            e = keep(np.exp(d))
            tot = keep(e.sum(-1, keepdims=True, dtype=np.float32))
            p = keep(e / tot) if round_weights else e / tot
            out[b, :, h] = r((p.astype(np.float64) @ v).astype(np.float32))
    return out
