"""Decode attention (one query token against a KV cache) on the GPU: the
fused kernel against the oracle's NumPy form of the Qwen3 decode step
(examples/models/qwen3/kernels/attention.py:101-140), and the traced bf16
Qwen3 attention layer lowered with the fused kernel against the same graph
lowered onto the generic kernels (which follow the traced cast points op by
op)."""

import os

import numpy as np
import pytest
from parity import assert_close

from nkipy_amd.core import dtypes as dt
from nkipy_amd.dispatch import launchers as LA
from nkipy_amd.runtime import DeviceKernel, DeviceTensor
from oracle import kernels as K
from oracle import numerics as N

pytestmark = pytest.mark.gpu


def _close(got, ref):
    name = os.environ.get("PYTEST_CURRENT_TEST", "?").split(" ")[0]
    assert_close(got, ref, name, axis=-1)


@pytest.mark.parametrize("B,Smax,Hq,Hkv,pos", [(1, 128, 4, 1, 0), (2, 256, 8, 2, 100), (2, 300, 4, 2, 299),
                                                (3, 1024, 16, 4, 1023), (1, 1024, 16, 1, 600),
                                                (1, 4096, 32, 8, 4095), (2, 5000, 8, 2, 4321),
                                                (1, 8192, 4, 4, 129), (2, 700, 16, 2, 650), (3, 384, 12, 4, 200)])
@pytest.mark.parametrize("casts", [True, False])
def test_decode_attention_kernel(gpu, B, Smax, Hq, Hkv, pos, casts):
    """Splits of 128 cache positions: one (pos 0), a partial last split
    (300, 5000 rows; pos 4321), splits past pos left out (pos 129 of 8192)."""
    D = 128
    rng = np.random.default_rng(B * Smax + Hq + pos)
    q = N.bf16_round(rng.standard_normal((B, Hq, D)))
    ck = N.bf16_round(rng.standard_normal((B, Smax, Hkv, D)))
    cv = N.bf16_round(rng.standard_normal((B, Smax, Hkv, D)))
    tq, tk, tv = (DeviceTensor.from_numpy(dt.to_bf16(a)) for a in (q, ck, cv))
    tp = DeviceTensor.from_numpy(np.array([pos], np.int32))
    to = DeviceTensor.empty((B, Hq, D), dt.bfloat16)
    flags = (LA.DEC_RND_PROD | LA.DEC_RND_SCORE | LA.DEC_SOFTMAX_BF16) if casts else 0
    st = {"q": (Hq * D, D), "k": (Smax * Hkv * D, Hkv * D, D), "v": (Smax * Hkv * D, Hkv * D, D),
          "o": (Hq * D, D)}
    ws = DeviceTensor.empty((LA.decode_attention_workspace_bytes(B, Smax, Hq),), dt.uint8)
    for launch in LA.decode_attention(tq.ptr, tk.ptr, tv.ptr, to.ptr, tp.ptr, B, Smax, Hq, Hkv, D,
                                      float(np.sqrt(D)), st, flags | LA.DEC_DIVIDE, ws_ptr=ws.ptr):
        launch.run(gpu)
    gpu.sync()
    got = dt.to_float32(to.numpy())
    ref = K.decode_attention(q, ck, cv, pos, casts, casts, casts)
    _close(got, ref)


def test_qwen3_decode_fused_equals_generic(gpu):
    from nkipy_amd.core.trace import NKIPyKernel
    from nkipy_amd.dispatch.lower import lower
    from nkipy_amd.dispatch.patterns import default_patterns
    from nkipy_amd.dispatch.patterns_attention import DecodeAttentionPattern
    from nkipy_amd.kernels.qwen3 import qwen3_attention_kernel

    B, MAXS, HID, H, D, HKV = 2, 512, 512, 8, 128, 2

    def decode(x, qkv_weight, q_norm_weight, k_norm_weight, cache_k, cache_v, start_pos, o_weight):
        return qwen3_attention_kernel(x, qkv_weight, q_norm_weight, k_norm_weight, 1e-6, H, D, HKV,
                                      cache_k, cache_v, start_pos, o_weight)

    rng = np.random.default_rng(11)
    host = {"x": N.bf16_round(rng.standard_normal((B, 1, HID))),
            "qkv_weight": N.bf16_round(rng.standard_normal((HID, (H + 2 * HKV) * D)) * 0.05),
            "q_norm_weight": N.bf16_round(rng.uniform(0.5, 1.5, D)),
            "k_norm_weight": N.bf16_round(rng.uniform(0.5, 1.5, D)),
            "cache_k": N.bf16_round(rng.standard_normal((B, MAXS, HKV, D))),
            "cache_v": N.bf16_round(rng.standard_normal((B, MAXS, HKV, D))),
            "o_weight": N.bf16_round(rng.standard_normal((H * D, HID)) * 0.05)}
    pos = np.array([300], np.int32)
    args = [dt.to_bf16(host[n]) for n in ("x", "qkv_weight", "q_norm_weight", "k_norm_weight", "cache_k",
                                          "cache_v")] + [pos, dt.to_bf16(host["o_weight"])]
    graph = NKIPyKernel.trace(decode).specialize(*args)
    fused = DeviceKernel(graph, lower(graph), "decode_fused")
    assert "decode_attention" in fused.plan.kernel_kinds
    generic_pats = [p for p in default_patterns() if not isinstance(p, DecodeAttentionPattern)]
    generic = DeviceKernel(graph, lower(graph, generic_pats), "decode_generic")
    assert "decode_attention" not in generic.plan.kernel_kinds
    names = [p.name for p in graph.parameters]
    outs = []
    for dk in (fused, generic):
        ins = {n: DeviceTensor.from_numpy(a, name=n) for n, a in zip(names, args)}
        res = dk(ins)
        outs.append({k: dt.to_float32(v.numpy()) for k, v in res.items()})
    np.testing.assert_array_equal(outs[0]["cache_k"], outs[1]["cache_k"])
    np.testing.assert_array_equal(outs[0]["cache_v"], outs[1]["cache_v"])
    _close(outs[0]["output0"], outs[1]["output0"])
    # the token's keys went to position 300
    assert np.abs(outs[0]["cache_k"][:, 300] - host["cache_k"][:, 300]).max() > 0
    np.testing.assert_array_equal(outs[0]["cache_k"][:, 301:], host["cache_k"][:, 301:])


@pytest.mark.parametrize("B,MAXS,HID,H,HKV,pos", [(2, 512, 512, 8, 2, 300), (8, 4096, 4096, 32, 8, 4000),
                                                  (32, 512, 1024, 8, 2, 77)])
def test_qwen3_decode_layer_matches_oracle(gpu, B, MAXS, HID, H, HKV, pos):
    """The traced bf16 Qwen3 attention layer for one decode token per
    sequence (projections on the split-K kernels, the fused head prologue,
    the cache writes, the split decode attention) against the oracle's
    composition of the same steps: the output at the bf16 bar, the new
    cache rows within a rounding step of the norm's sum order, every other
    cache row untouched."""
    from nkipy_amd.kernels.qwen3 import qwen3_attention_kernel

    D = 128
    print(f"qwen3 decode layer B={B} MAXS={MAXS} HID={HID} H={H}/{HKV} pos={pos}", flush=True)

    def decode(x, qkv_weight, q_norm_weight, k_norm_weight, cache_k, cache_v, start_pos, o_weight):
        return qwen3_attention_kernel(x, qkv_weight, q_norm_weight, k_norm_weight, 1e-6, H, D, HKV,
                                      cache_k, cache_v, start_pos, o_weight)

    rng = np.random.default_rng(B + pos)
    host = {"x": N.bf16_round(rng.standard_normal((B, 1, HID))),
            "qkv_weight": N.bf16_round(rng.standard_normal((HID, (H + 2 * HKV) * D)) * HID ** -0.5),
            "q_norm_weight": N.bf16_round(rng.uniform(0.5, 1.5, D)),
            "k_norm_weight": N.bf16_round(rng.uniform(0.5, 1.5, D)),
            "cache_k": N.bf16_round(rng.standard_normal((B, MAXS, HKV, D))),
            "cache_v": N.bf16_round(rng.standard_normal((B, MAXS, HKV, D))),
            "o_weight": N.bf16_round(rng.standard_normal((H * D, HID)) * (H * D) ** -0.5)}
    args = [dt.to_bf16(host[n]) for n in ("x", "qkv_weight", "q_norm_weight", "k_norm_weight", "cache_k",
                                          "cache_v")] + [np.array([pos], np.int32), dt.to_bf16(host["o_weight"])]
    dk = DeviceKernel.compile_and_load(decode, *args, name=f"qwen3_decode_b{B}")
    assert "decode_attention" in dk.plan.kernel_kinds and "head_rope" in dk.plan.kernel_kinds
    names = list(dk.input_tensors_info)
    ins = {n: DeviceTensor.from_numpy(a, name=n) for n, a in zip(names, args)}
    res = {k: dt.to_float32(v.numpy()) for k, v in dk(ins).items()}
    out, ck, cv = K.qwen3_decode_layer(host["x"], host["qkv_weight"], host["q_norm_weight"], host["k_norm_weight"],
                                       1e-6, H, HKV, D, host["cache_k"], host["cache_v"], pos, host["o_weight"])
    _close(res["output0"], out)
    for name, ref in (("cache_k", ck), ("cache_v", cv)):
        got = res[name]
        rest = np.ones(MAXS, bool)
        rest[pos] = False
        np.testing.assert_array_equal(got[:, rest], ref[:, rest])
        _close(got[:, pos], ref[:, pos])
