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


def _check_rows(out, q, ck, cv, causal=True, step=256):
    """Every query row against the op-by-op oracle at the bf16 bar, and
    bit for bit on at least 99.8% of the outputs."""
    S = q.shape[1]
    for r0 in range(0, S, step):
        rows = np.arange(r0, min(S, r0 + step))
        ref = K.qwen3_prefill_attention(q, ck, cv, rows=rows, causal=causal)
        assert_close(out[:, rows], ref, _name(), axis=-1)
        same = np.mean(out[:, rows] == ref)
        print(f"rows {r0}..: identical {same:.5f}", flush=True)
        assert same >= 0.998


def test_bf16_attention_unmasked_statistics_chunks(gpu):
    """The bf16 score / bf16 softmax form without a mask (every query sees
    every key, as an encoder's attention does): the statistics kernels run
    over all S keys of every query block, in five 512-key chunks at S =
    2560, and the result matches the op-by-op oracle."""
    from nkipy_amd.kernels.softmax import softmax_kernel

    def bf16_attention(xq, xk, xv):
        B, S, Hq, D = xq.shape
        rep = Hq // xk.shape[2]
        q = xq.transpose(0, 2, 1, 3)
        k = np.repeat(xk, rep, axis=2).transpose(0, 2, 1, 3)
        v = np.repeat(xv, rep, axis=2).transpose(0, 2, 1, 3)
        s = ((q @ k.transpose(0, 1, 3, 2)) / np.float32(np.sqrt(D))).astype(xq.dtype)
        return (softmax_kernel(s) @ v).transpose(0, 2, 1, 3)

    B, S, Hq, Hkv, D = 1, 2560, 4, 2, 128
    rng = np.random.default_rng(29)
    q, k, v = (N.bf16_round(rng.standard_normal((B, S, h, D))) for h in (Hq, Hkv, Hkv))
    args = [dt.to_bf16(a) for a in (q, k, v)]
    # (a fresh lowering: the test reads the plan's launch arguments)
    dk = DeviceKernel.compile_and_load(bf16_attention, *args, name="bf16_attention_unmasked",
                                       use_cached_if_exists=False)
    assert dk.plan.kernel_kinds == ["attention"], dk.plan.kernel_kinds
    (launches,) = [st.launches(lambda v: 1 << 40) for st in dk.plan.steps]
    assert [l.args.causal for l in launches] == [0, 0, 0] and launches[0].args.nch == 5
    ins = {n: DeviceTensor.from_numpy(a, name=n) for n, a in zip(dk.input_tensors_info, args)}
    out = dt.to_float32(dk(ins)["output0"].numpy())
    _check_rows(out, q, k, v, causal=False, step=512)


def test_prefill_attention_long_rows_many_chunks(gpu):
    """S = 5120 causal: 640-key chunks (S / 8 rounded up to 128 keys), eight
    for the last query blocks, against the op-by-op oracle."""
    from nkipy_amd.kernels.qwen3 import prefill_attention_kernel

    B, S, MAXS, Hq, Hkv, D = 1, 5120, 5120, 2, 1, 128
    rng = np.random.default_rng(31)
    q = N.bf16_round(rng.standard_normal((B, S, Hq, D)))
    ck, cv = (N.bf16_round(rng.standard_normal((B, MAXS, Hkv, D))) for _ in range(2))
    args = [dt.to_bf16(a) for a in (q, ck, cv)]
    dk = DeviceKernel.compile_and_load(prefill_attention_kernel, *args, name="prefill_long",
                                       use_cached_if_exists=False)
    (launches,) = [st.launches(lambda v: 1 << 40) for st in dk.plan.steps]
    assert (launches[0].args.ckb, launches[0].args.nch) == (20, 8)
    ins = {n: DeviceTensor.from_numpy(a, name=n) for n, a in zip(dk.input_tensors_info, args)}
    out = dt.to_float32(dk(ins)["output0"].numpy())
    _check_rows(out, q, ck, cv, step=1024)


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
