"""One Llama decoder step of a one-layer model, fp32, as a graph exporter
writes it (tests/kernels/llama_decoder_dynamo.py:6-337 of the reference):
token embedding, rotary tables from inverse frequencies, RMSNorm spelt out
(power, sum / n, + eps, sqrt, 1 / x), the attention block of
``attention_dynamo`` with its KV-cache writes, the residual, the gated MLP,
the second residual, the final RMSNorm, and logits of the last token
against the (tied) embedding table.  Returns both updated caches and the
logits."""

import numpy as np

from kernel_specs.attention_dynamo import (
    D, HID, HKV, HQ, SLOTS, T, _CACHE, _t, _w, attention_block, causal_mask,
)
from kernel_specs.rope_dynamo import rope_cos_sin
from nkipy_amd.core.specs import CommonTypes, KernelSpec

VOCAB, FFN = 128256, 8192


def _rmsnorm(x, weight):
    ms = np.divide(np.sum(np.power(x, 2), axis=(-1,), keepdims=True), x.shape[-1])
    inv = np.divide(1, np.sqrt(np.add(ms, 1e-05)))
    return np.multiply(weight, np.multiply(x, inv))


def _mlp(h, w_gate, w_up, w_down):
    rows = np.reshape(h, [T, HID])
    gate = np.reshape(np.matmul(rows, np.transpose(w_gate, [1, 0])), [1, T, FFN])
    up = np.reshape(np.matmul(rows, np.transpose(w_up, [1, 0])), [1, T, FFN])
    act = np.multiply(np.multiply(gate, np.divide(1, np.add(1, np.exp(np.negative(gate))))), up)
    return np.reshape(np.matmul(np.reshape(act, [T, FFN]), np.transpose(w_down, [1, 0])), [1, T, HID])


def llama_step(token_ids, table, positions, rope_positions, cache_k, mask, inv_freq, attn_norm, wq, wk, wv,
               cache_v, wo, mlp_norm, w_gate, w_up, w_down, final_norm):
    x = np.take(table, token_ids, axis=0)                          # (1, T, HID)
    cos, sin = rope_cos_sin(inv_freq, rope_positions)
    attn, _, new_k, new_v = attention_block(_rmsnorm(x, attn_norm), wq, wk, wv, cos, sin, positions,
                                            cache_k, cache_v, mask, wo)
    z = np.add(x, attn)
    y = np.add(z, _mlp(_rmsnorm(z, mlp_norm), w_gate, w_up, w_down))
    last = _rmsnorm(y, final_norm)[:, T - 1:, :]
    logits = np.matmul(np.reshape(last, [1, HID]), np.transpose(table, [1, 0]))
    return new_k, new_v, np.reshape(logits, [1, 1, VOCAB])


POSITIONS = np.arange(T, dtype=np.int32)
INV_FREQ = (1.0 / (10000.0 ** (np.arange(0, D, 2, dtype=np.float32) / D))).astype(np.float32)
_ones = lambda: np.ones(HID, np.float32)

kernel_specs = [KernelSpec(
    function=llama_step,
    inputs=[_t((1, T), np.random.default_rng(23).integers(0, 50000, (1, T)).astype(np.int32), "token ids",
               CommonTypes.INTS),
            _t((VOCAB, HID), lambda: np.random.default_rng(29).normal(0, 0.02, (VOCAB, HID)).astype(np.float32),
               "embedding table (tied lm head)"),
            _t((T,), POSITIONS, "cache slots", CommonTypes.INTS),
            _t((1, T), POSITIONS[None], "rotary positions", CommonTypes.INTS),
            _t((1, HKV, SLOTS, D), _CACHE(5), "key cache"),
            _t((1, 1, T, SLOTS), causal_mask(POSITIONS), "additive mask"),
            _t((D // 2,), INV_FREQ, "inverse frequencies"),
            _t((HID,), _ones, "attention norm weight"),
            _t((HQ * D, HID), _w(HQ * D, HID, 31), "q weight"),
            _t((HKV * D, HID), _w(HKV * D, HID, 32), "k weight"),
            _t((HKV * D, HID), _w(HKV * D, HID, 33), "v weight"),
            _t((1, HKV, SLOTS, D), _CACHE(6), "value cache"),
            _t((HID, HQ * D), _w(HID, HQ * D, 34), "o weight"),
            _t((HID,), _ones, "mlp norm weight"),
            _t((FFN, HID), _w(FFN, HID, 35), "gate weight"),
            _t((FFN, HID), _w(FFN, HID, 36), "up weight"),
            _t((HID, FFN), _w(HID, FFN, 37), "down weight"),
            _t((HID,), _ones, "final norm weight")],
    description="one-layer Llama step: embedding, attention with KV cache, MLP, logits")]
