"""Grouped-query attention with a KV cache and rotary embedding, fp32, as a
graph exporter writes it (tests/kernels/attention_dynamo.py:7-209 of the
reference): 7 new tokens, hidden 2048, 32 query / 8 key-value heads of 64,
a 16-slot cache written at the tokens' positions, scores scaled by 1/8 plus
an additive mask, softmax, the weighted values and the output projection.
Projections multiply by transposed torch-layout (out, in) weights, RoPE is
the rotate-half form (negated second half first), and the 8 cache heads are
broadcast to 32 through an expand + copy + reshape.  Returns the output and
the attention probabilities."""

import numpy as np

from nkipy_amd.core.specs import CommonTypes, KernelSpec, ShapeSpec, TensorInputSpec

T, HID, D, HQ, HKV, SLOTS = 7, 2048, 64, 32, 8, 16
MASKED = -10000.0


def _project_heads(h, w):
    y = np.matmul(h, np.transpose(w, [1, 0]))
    return np.transpose(np.reshape(y, [1, T, -1, D]), [0, 2, 1, 3])   # (1, heads, T, D)


def _rotate(t, cos, sin):
    half = D // 2
    swapped = np.concatenate([np.negative(t[:, :, :, half:]), t[:, :, :, :half]], -1)
    return np.add(np.multiply(t, cos), np.multiply(swapped, sin))


def _heads_for_queries(cache):
    """(1, HKV, SLOTS, D) -> (HQ, SLOTS, D): kv head g serves query heads
    g * (HQ / HKV) ..."""
    grouped = np.broadcast_to(np.expand_dims(cache, 2), [1, HKV, HQ // HKV, SLOTS, D])
    return np.reshape(np.copy(grouped), [HQ, SLOTS, D])


def attention_block(x, wq, wk, wv, cos, sin, positions, cache_k, cache_v, mask, wo):
    """-> (output (1, T, HID), probabilities (1, HQ, T, SLOTS), updated caches)."""
    h = np.reshape(x, [T, HID])
    c, s = np.expand_dims(cos, 1), np.expand_dims(sin, 1)
    q = _rotate(_project_heads(h, wq), c, s)
    k = _rotate(_project_heads(h, wk), c, s)
    v = _project_heads(h, wv)
    new_k = np.copy(cache_k)
    new_k[:, :, positions] = k
    new_v = np.copy(cache_v)
    new_v[:, :, positions] = v
    keys_t = np.transpose(_heads_for_queries(new_k), [0, 2, 1])                # (HQ, D, SLOTS)
    scores = np.reshape(np.matmul(np.reshape(q, [HQ, T, D]), keys_t), [1, HQ, T, SLOTS])
    scores = np.add(np.multiply(scores, 0.125), mask)
    e = np.exp(np.subtract(scores, np.max(scores, axis=-1, keepdims=True)))
    probs = np.divide(e, np.sum(e, axis=-1, keepdims=True))
    o = np.matmul(np.reshape(probs, [HQ, T, SLOTS]), _heads_for_queries(new_v))  # (HQ, T, D)
    o = np.reshape(np.transpose(np.reshape(o, [1, HQ, T, D]), [0, 2, 1, 3]), [T, HQ * D])
    out = np.reshape(np.matmul(o, np.transpose(wo, [1, 0])), [1, T, HID])
    return out, probs, new_k, new_v


def gqa_attention(x, wq, wk, wv, cos, sin, positions, cache_k, cache_v, mask, wo):
    out, probs, _, _ = attention_block(x, wq, wk, wv, cos, sin, positions, cache_k, cache_v, mask, wo)
    return out, probs


def rope_tables(positions, dim=D, base=10000.0):
    """cos / sin (1, T, dim) of the rotate-half form for integer positions."""
    inv = 1.0 / (base ** (np.arange(0, dim, 2, dtype=np.float32) / dim))
    ang = np.outer(np.asarray(positions, np.float32), inv.astype(np.float32))
    full = np.concatenate([ang, ang], -1)[None]
    return np.cos(full).astype(np.float32), np.sin(full).astype(np.float32)


def causal_mask(positions):
    """Additive mask (1, 1, T, SLOTS): slot l is hidden from the token at
    position p when l > p."""
    p = np.asarray(positions)[:, None]
    return np.where(np.arange(SLOTS)[None, :] > p, np.float32(MASKED), np.float32(0.0))[None, None]


_rng = np.random.default_rng(17)
POSITIONS = np.sort(_rng.choice(SLOTS, T, replace=False)).astype(np.int32)
_COS, _SIN = rope_tables(POSITIONS)


def _w(rows, cols, seed):
    """N(0, 1/cols) weights (rows, cols), built on use."""
    return lambda: (np.random.default_rng(seed).standard_normal((rows, cols), dtype=np.float32)
                    / np.float32(np.sqrt(cols)))


def _t(shape, value, what, types=CommonTypes.FLOATS):
    return TensorInputSpec(shape_spec=ShapeSpec(dims=list(shape), default=tuple(shape)), dtype_spec=types,
                           default_value=value, description=what)


_CACHE = lambda seed: (lambda: np.random.default_rng(seed).normal(0, 0.02, (1, HKV, SLOTS, D)).astype(np.float32))

kernel_specs = [KernelSpec(
    function=gqa_attention,
    inputs=[_t((1, T, HID), lambda: np.random.default_rng(1).standard_normal((1, T, HID), dtype=np.float32),
               "hidden states"),
            _t((HQ * D, HID), _w(HQ * D, HID, 31), "q weight (out, in)"),
            _t((HKV * D, HID), _w(HKV * D, HID, 32), "k weight (out, in)"),
            _t((HKV * D, HID), _w(HKV * D, HID, 33), "v weight (out, in)"),
            _t((1, T, D), _COS, "cos table"), _t((1, T, D), _SIN, "sin table"),
            _t((T,), POSITIONS, "cache slots of the tokens", CommonTypes.INTS),
            _t((1, HKV, SLOTS, D), _CACHE(2), "key cache"), _t((1, HKV, SLOTS, D), _CACHE(3), "value cache"),
            _t((1, 1, T, SLOTS), causal_mask(POSITIONS), "additive mask"),
            _t((HID, HQ * D), _w(HID, HQ * D, 34), "o weight (out, in)")],
    description="GQA attention step with KV-cache write and rotate-half RoPE")]
