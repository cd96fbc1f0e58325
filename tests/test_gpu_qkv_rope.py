"""QKV projection with RoPE folded into the GEMM epilogue.

The traced form is the decoder's (tests/kernels/llama_decoder_dynamo.py:
150-178, examples/models/qwen3/kernels/attention.py:44-66): a fused QKV
projection cast to bf16, split into heads, and the split-half rotation of
q and k in fp32 with one bf16 rounding.  The fused launch must equal the
separate GEMM + two RoPE launches bit for bit (same accumulation, same cast
points), and the NumPy form within the bf16 bar.
"""

import numpy as np
import pytest
from parity import assert_close

from nkipy_amd.core import dtypes as dt
from nkipy_amd.core.trace import NKIPyKernel
from nkipy_amd.dispatch.lower import lower
from nkipy_amd.dispatch.patterns import default_patterns
from nkipy_amd.dispatch.patterns_attention import QkvRopeFusion
from nkipy_amd.dispatch.patterns_gemm import GemmPattern
from nkipy_amd.kernels.decoder import qkv_rope_fp8, rope_kernel, rope_tables
from nkipy_amd.runtime import DeviceKernel, DeviceTensor
from oracle import kernels as K
from oracle import numerics as N

D = 128
THETA = 5.0e5


def _quantize(rng, shape):
    """N(0, 0.02) weights -> e4m3fn codes (uint8) with per-output-channel
    scales amax / 448, converted by torch."""
    import torch

    w = torch.from_numpy(rng.standard_normal(shape, dtype=np.float32) * 0.02)
    scale = (w.abs().amax(dim=1) / 448.0).clamp_min(1e-12)
    codes = (w / scale[:, None]).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    return codes, scale.numpy().astype(np.float32)


def _run(graph, plan, inputs, name):
    dk = DeviceKernel(graph, plan, name)
    out = dk({k: DeviceTensor.from_numpy(v, name=k) for k, v in inputs.items()})
    return [dt.to_float32(out[f"output{i}"].numpy()) for i in range(len(out))]


def _both(fn, inputs):
    graph = NKIPyKernel.trace(fn).specialize(*inputs.values())
    fused = lower(graph)
    # the plain projection on one K loop per tile, as the fused kernel sums
    plain = lower(graph, [GemmPattern(split_k=False) if isinstance(p, GemmPattern) else p
                          for p in default_patterns() if not isinstance(p, QkvRopeFusion)])
    assert "gemm_rope" in fused.kernel_kinds and "rope" not in fused.kernel_kinds
    assert plain.kernel_kinds.count("rope") == 2
    return _run(graph, fused, inputs, "fused"), _run(graph, plain, inputs, "plain")


@pytest.mark.gpu
@pytest.mark.parametrize("B,S,Hq,Hkv,hid", [(2, 256, 4, 2, 512), (1, 384, 8, 1, 1024), (3, 96, 2, 2, 256)])
def test_qkv_rope_fp8(gpu, B, S, Hq, Hkv, hid):
    """fp8 NT weights with per-channel scales; M = B * S not a multiple of
    the 256-row tile in two of the cases, and rows of several sequences."""
    print(f"qkv_rope fp8 B={B} S={S} Hq={Hq} Hkv={Hkv} hid={hid}", flush=True)
    rng = np.random.default_rng(B * 1000 + S + Hq)
    x = N.bf16_round(rng.standard_normal((B, S, hid), dtype=np.float32))
    codes, scale = _quantize(rng, ((Hq + 2 * Hkv) * D, hid))

    def fn(h, w, s):
        return qkv_rope_fp8(h, w, s, Hq, Hkv, THETA)

    inputs = {"h": dt.to_bf16(x), "w": codes.view(dt.float8_e4m3fn), "s": scale}
    fused, plain = _both(fn, inputs)
    for f, p in zip(fused, plain):
        np.testing.assert_array_equal(f, p)
    qkv = N.bf16_round(K.linear_fp8(x, codes, scale))
    cos, sin = K.rope_tables(D, S, THETA)
    q_ref = N.bf16_round(K.rope_split_half(qkv[..., :Hq * D].reshape(B, S, Hq, D), cos, sin))
    k_ref = N.bf16_round(K.rope_split_half(qkv[..., Hq * D:(Hq + Hkv) * D].reshape(B, S, Hkv, D), cos, sin))
    v_ref = qkv[..., (Hq + Hkv) * D:].reshape(B, S, Hkv, D)
    assert_close(fused[0], q_ref, "rope(q) fp8", axis=-1)
    assert_close(fused[1], k_ref, "rope(k) fp8", axis=-1)
    assert_close(fused[2], v_ref, "v fp8", axis=-1)


@pytest.mark.gpu
def test_qkv_rope_bf16_nn(gpu):
    """bf16 (in, out) weights: the NN kernel's rotary variant."""
    B, S, Hq, Hkv, hid = 2, 128, 4, 1, 384
    print(f"qkv_rope bf16 nn B={B} S={S} Hq={Hq} Hkv={Hkv} hid={hid}", flush=True)
    rng = np.random.default_rng(11)
    x = N.bf16_round(rng.standard_normal((B, S, hid), dtype=np.float32))
    w = N.bf16_round(rng.standard_normal((hid, (Hq + 2 * Hkv) * D), dtype=np.float32) * 0.05)
    cos, sin = rope_tables(D, S, THETA)

    def fn(h, w):
        qkv = np.matmul(h, w).astype(h.dtype)
        q, k, v = np.split(qkv, [Hq * D, (Hq + Hkv) * D], axis=-1)
        q = rope_kernel(q.reshape(B, S, Hq, D), cos, sin).astype(h.dtype)
        k = rope_kernel(k.reshape(B, S, Hkv, D), cos, sin).astype(h.dtype)
        return q, k, v.reshape(B, S, Hkv, D)

    fused, plain = _both(fn, {"h": dt.to_bf16(x), "w": dt.to_bf16(w)})
    for f, p in zip(fused, plain):
        np.testing.assert_array_equal(f, p)
    qkv = N.bf16_round(np.matmul(x, w))
    ocos, osin = K.rope_tables(D, S, THETA)
    assert_close(fused[0], N.bf16_round(K.rope_split_half(qkv[..., :Hq * D].reshape(B, S, Hq, D), ocos, osin)),
                 "rope(q) bf16", axis=-1)
    assert_close(fused[1], N.bf16_round(K.rope_split_half(
        qkv[..., Hq * D:(Hq + Hkv) * D].reshape(B, S, Hkv, D), ocos, osin)), "rope(k) bf16", axis=-1)
