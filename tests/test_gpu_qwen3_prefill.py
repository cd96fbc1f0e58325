"""Qwen3 prefill attention (examples/models/qwen3/kernels/attention.py:
107-140 with start_pos None) on the GPU: queries 0..S-1 against the whole
bf16 KV cache of MAXS rows, scores rounded to bf16 after the product and
after the divide by sqrt(d), mask rows [:S, :MAXS] of a constant triu mask,
bf16 softmax, @ values.

* The traced kernel lowers to one attention step (three launches over the
  keys: row max, row sum, weighted values; no score matrix in memory) and
  matches the oracle's op-by-op bf16 form on every query row at the bf16
  bar, bit for bit on at least 99.8% of the outputs; cache rows past S
  hold stale values, which the mask hides.
* The whole bf16 Qwen3 attention layer (projection, q / k RMSNorm, RoPE,
  cache write, attention, output projection) lowered with the fused
  attention equals the same graph lowered onto the generic dot / softmax
  kernels, which follow every traced cast point op by op.
"""

import os

import numpy as np
import pytest
from parity import assert_close, ulp_bf16

from nkipy_amd.core import dtypes as dt
from nkipy_amd.core.trace import NKIPyKernel
from nkipy_amd.dispatch.lower import lower
from nkipy_amd.runtime import DeviceKernel, DeviceTensor
from oracle import kernels as K
from oracle import numerics as N

pytestmark = pytest.mark.gpu


def _name():
    return os.environ.get("PYTEST_CURRENT_TEST", "?").split(" ")[0]


@pytest.mark.parametrize("B,S,MAXS,Hq,Hkv", [(1, 2048, 4096, 32, 8), (2, 256, 512, 8, 2),
                                             (1, 384, 384, 4, 4), (1, 128, 1024, 16, 1)])
def test_prefill_attention_matches_oracle(gpu, B, S, MAXS, Hq, Hkv):
    from nkipy_amd.kernels.qwen3 import prefill_attention_kernel

    D = 128
    rng = np.random.default_rng(S + MAXS + Hq)
    print(f"prefill attention B={B} S={S} MAXS={MAXS} Hq={Hq} Hkv={Hkv}", flush=True)
    q = N.bf16_round(rng.standard_normal((B, S, Hq, D)))
    ck = N.bf16_round(rng.standard_normal((B, MAXS, Hkv, D)))
    cv = N.bf16_round(rng.standard_normal((B, MAXS, Hkv, D)))
    args = [dt.to_bf16(a) for a in (q, ck, cv)]
    dk = DeviceKernel.compile_and_load(prefill_attention_kernel, *args, name=f"prefill_{B}_{S}_{MAXS}")
    assert dk.plan.kernel_kinds == ["attention"], dk.plan.kernel_kinds
    ins = {n: DeviceTensor.from_numpy(a, name=n) for n, a in zip(dk.input_tensors_info, args)}
    out = dt.to_float32(dk(ins)["output0"].numpy())
    assert out.shape == (B, S, Hq, D)
    for r0 in range(0, S, 256):  # every query row, 256 at a time
        rows = np.arange(r0, min(S, r0 + 256))
        ref = K.qwen3_prefill_attention(q, ck, cv, rows=rows)
        assert_close(out[:, rows], ref, _name(), axis=-1)
        d = np.abs(out[:, rows] - ref)
        ulp = ulp_bf16(ref)
        print(f"rows {r0}..: identical {np.mean(d == 0):.5f}, max {np.max(d / ulp):.2f} ulp, "
              f"over 1 ulp {np.mean(d > ulp):.2e}", flush=True)
        # every cast point is the traced code's: what differs is the order of
        # the fp32 sums (q.k, the weight sum, p.v), which moves a rounding
        # across a bf16 boundary now and then
        assert np.mean(d == 0) >= 0.998


def test_prefill_attention_ignores_cache_rows_past_s(gpu):
    """Rows S..MAXS-1 of the cache are masked for every query: values there
    (here large ones) change nothing, bit for bit."""
    from nkipy_amd.kernels.qwen3 import prefill_attention_kernel

    B, S, MAXS, Hq, Hkv, D = 1, 256, 768, 8, 2, 128
    rng = np.random.default_rng(5)
    q = N.bf16_round(rng.standard_normal((B, S, Hq, D)))
    ck = N.bf16_round(rng.standard_normal((B, MAXS, Hkv, D)))
    cv = N.bf16_round(rng.standard_normal((B, MAXS, Hkv, D)))
    outs = []
    for fill in (0.0, 300.0):
        k2, v2 = ck.copy(), cv.copy()
        k2[:, S:] = fill
        v2[:, S:] = -fill
        args = [dt.to_bf16(a) for a in (q, k2, v2)]
        dk = DeviceKernel.compile_and_load(prefill_attention_kernel, *args, name="prefill_stale")
        ins = {n: DeviceTensor.from_numpy(a, name=n) for n, a in zip(dk.input_tensors_info, args)}
        outs.append(dt.numpy_storage(dk(ins)["output0"].numpy()))
    np.testing.assert_array_equal(outs[0], outs[1])


def test_qwen3_prefill_layer_fused_equals_generic(gpu):
    from nkipy_amd.dispatch.patterns import default_patterns
    from nkipy_amd.dispatch.patterns_attention import AttentionPattern
    from nkipy_amd.kernels.qwen3 import qwen3_attention_kernel

    B, S, MAXS, HID, H, D, HKV = 2, 256, 512, 512, 8, 128, 2

    def prefill(x, qkv_weight, q_norm_weight, k_norm_weight, cache_k, cache_v, o_weight):
        return qwen3_attention_kernel(x, qkv_weight, q_norm_weight, k_norm_weight, 1e-6, H, D, HKV,
                                      cache_k, cache_v, None, o_weight)

    rng = np.random.default_rng(13)
    host = {"x": N.bf16_round(rng.standard_normal((B, S, HID))),
            "qkv_weight": N.bf16_round(rng.standard_normal((HID, (H + 2 * HKV) * D)) * 0.05),
            "q_norm_weight": N.bf16_round(rng.uniform(0.5, 1.5, D)),
            "k_norm_weight": N.bf16_round(rng.uniform(0.5, 1.5, D)),
            "cache_k": N.bf16_round(rng.standard_normal((B, MAXS, HKV, D))),
            "cache_v": N.bf16_round(rng.standard_normal((B, MAXS, HKV, D))),
            "o_weight": N.bf16_round(rng.standard_normal((H * D, HID)) * 0.05)}
    order = ("x", "qkv_weight", "q_norm_weight", "k_norm_weight", "cache_k", "cache_v", "o_weight")
    args = [dt.to_bf16(host[n]) for n in order]
    graph = NKIPyKernel.trace(prefill).specialize(*args)
    fused = DeviceKernel(graph, lower(graph), "prefill_fused")
    kinds = fused.plan.kernel_kinds
    assert "attention" in kinds and "dot" not in kinds and "softmax" not in kinds, kinds
    generic_pats = [p for p in default_patterns() if not isinstance(p, AttentionPattern)]
    generic = DeviceKernel(graph, lower(graph, generic_pats), "prefill_generic")
    assert "attention" not in generic.plan.kernel_kinds
    names = [p.name for p in graph.parameters]
    outs = []
    for dk in (fused, generic):
        ins = {n: DeviceTensor.from_numpy(a, name=n) for n, a in zip(names, args)}
        res = dk(ins)
        outs.append({k: dt.to_float32(v.numpy()) for k, v in res.items()})
    np.testing.assert_array_equal(outs[0]["cache_k"], outs[1]["cache_k"])
    np.testing.assert_array_equal(outs[0]["cache_v"], outs[1]["cache_v"])
    # rows past S of the cache are untouched
    np.testing.assert_array_equal(outs[0]["cache_k"][:, S:], host["cache_k"][:, S:])
    assert_close(outs[0]["output0"], outs[1]["output0"], _name(), axis=-1)
