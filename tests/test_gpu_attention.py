"""GPU parity of the causal GQA flash-attention kernel against the oracle."""

import os

import numpy as np
import pytest
from parity import assert_close

from nkipy_amd.core import dtypes as dt
from nkipy_amd.dispatch import launchers as LA
from nkipy_amd.runtime import DeviceTensor
from oracle import kernels as K
from oracle import numerics as N

pytestmark = pytest.mark.gpu


def _close(got, ref, tol=2e-2, axis=-1):
    """bf16 bar of tests/parity.py (rtol 2e-2, atol min(1e-2, 2e-2 RMS))."""
    name = os.environ.get("PYTEST_CURRENT_TEST", "?").split(" ")[0]
    assert_close(got, ref, name, rtol=tol, axis=axis)


def _run(gpu, q, k, v, **variant):
    B, S, Hq, D = q.shape
    Hkv = k.shape[2]
    t = [DeviceTensor.from_numpy(dt.to_bf16(a)) for a in (q, k, v)]
    o = DeviceTensor.empty(q.shape, dt.bfloat16)
    st = {"q": (S * Hq * D, Hq * D, D), "k": (S * Hkv * D, Hkv * D, D),
          "v": (S * Hkv * D, Hkv * D, D), "o": (S * Hq * D, Hq * D, D)}
    LA.attention(t[0].ptr, t[1].ptr, t[2].ptr, o.ptr, B, S, Hq, Hkv, D, 1 / np.sqrt(D), st, **variant).run(gpu)
    gpu.sync()
    return dt.to_float32(o.numpy())


@pytest.mark.parametrize("shape", [(1, 128, 1, 1), (1, 256, 4, 1), (2, 384, 8, 2)])
def test_attention_small(gpu, shape):
    B, S, Hq, Hkv = shape
    rng = np.random.default_rng(S + Hq)
    q = N.bf16_round(rng.standard_normal((B, S, Hq, 128)))
    k = N.bf16_round(rng.standard_normal((B, S, Hkv, 128)))
    v = N.bf16_round(rng.standard_normal((B, S, Hkv, 128)))
    _close(_run(gpu, q, k, v), K.causal_gqa_attention(q, k, v))


@pytest.mark.parametrize("waves,key_block,ring", [(4, 64, False), (8, 64, False), (4, 32, False), (4, 32, True),
                                                   (8, 32, True)])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("shape", [(1, 128, 1, 1), (1, 256, 4, 1), (2, 512, 8, 2), (1, 768, 2, 2),
                                   (1, 1152, 2, 1)])
def test_attention_variants(gpu, waves, key_block, ring, causal, shape):
    """Every kernel variant (waves per workgroup, keys per block, the
    four-slot ring), masked and unmasked, including the diagonal blocks a
    workgroup's waves skip and sequences whose block counts leave every
    remainder of the ring kernel's four-way unrolled loop."""
    B, S, Hq, Hkv = shape
    if S % (32 * waves):
        pytest.skip(f"{waves} waves take query blocks of {32 * waves}")
    print(f"attention variant waves={waves} key_block={key_block} ring={ring} causal={causal} shape={shape}",
          flush=True)
    rng = np.random.default_rng(S + Hq + waves + key_block)
    q = N.bf16_round(rng.standard_normal((B, S, Hq, 128)))
    k = N.bf16_round(rng.standard_normal((B, S, Hkv, 128)))
    v = N.bf16_round(rng.standard_normal((B, S, Hkv, 128)))
    got = _run(gpu, q, k, v, causal=causal, waves=waves, key_block=key_block, ring=ring)
    _close(got, K.causal_gqa_attention(q, k, v, causal=causal))


@pytest.mark.parametrize("causal", [True, False])
def test_attention_ring_offset_raised(gpu, causal):
    """Scores that grow along the keys (q . k rises with the key index) make
    later blocks exceed the first block's offset by far more than 2^16, so the
    ring kernel's recompute path (offset raised, O and l rescaled) runs on
    many blocks; the result still matches the float64 softmax."""
    B, S, Hq, Hkv = 1, 512, 2, 1
    rng = np.random.default_rng(7)
    q = np.abs(rng.standard_normal((B, S, Hq, 128))) * 0.3 + 0.2
    ramp = np.linspace(0.0, 8.0, S)[None, :, None, None]
    k = (np.abs(rng.standard_normal((B, S, Hkv, 128))) * 0.3 + 0.2) * ramp
    q, k = N.bf16_round(q), N.bf16_round(k)
    v = N.bf16_round(rng.standard_normal((B, S, Hkv, 128)))
    print(f"ring offset raised causal={causal}", flush=True)
    got = _run(gpu, q, k, v, causal=causal, ring=True)
    _close(got, K.causal_gqa_attention(q, k, v, causal=causal))


def test_attention_config_all_sequences(gpu):
    """Decoder config: batch 8 x seq 2048, 32 query / 8 KV heads, head_dim
    128; every sequence against the oracle."""
    B, S, Hq, Hkv = 8, 2048, 32, 8
    rng = np.random.default_rng(42)
    q = N.bf16_round(rng.standard_normal((B, S, Hq, 128)) * 0.5)
    k = N.bf16_round(rng.standard_normal((B, S, Hkv, 128)) * 0.5)
    v = N.bf16_round(rng.standard_normal((B, S, Hkv, 128)))
    got = _run(gpu, q, k, v)
    for b in range(B):
        ref = K.causal_gqa_attention(q[b:b + 1], k[b:b + 1], v[b:b + 1])
        _close(got[b:b + 1], ref)


def test_noncausal_gqa_attention_traced(gpu):
    """Unmasked softmax(q k^T / sqrt(d)) v with GQA lowers to the fused
    kernel with the mask off, and matches the float64 loop."""
    from nkipy_amd.kernels.softmax import softmax_kernel
    from nkipy_amd.runtime import DeviceKernel, baremetal_jit

    def full_attention(xq, xk, xv):
        B, S, Hq, D = xq.shape
        rep = Hq // xk.shape[2]
        q = xq.transpose(0, 2, 1, 3).astype(np.float32)
        kt = np.repeat(xk, rep, axis=2).transpose(0, 2, 3, 1).astype(np.float32)
        v = np.repeat(xv, rep, axis=2).transpose(0, 2, 1, 3).astype(np.float32)
        p = softmax_kernel(np.matmul(q, kt) / np.float32(np.sqrt(D)))
        return np.matmul(p, v).transpose(0, 2, 1, 3).astype(xq.dtype)

    B, S, Hq, Hkv = 1, 256, 4, 2
    rng = np.random.default_rng(17)
    q = N.bf16_round(rng.standard_normal((B, S, Hq, 128)) * 0.5)
    k = N.bf16_round(rng.standard_normal((B, S, Hkv, 128)) * 0.5)
    v = N.bf16_round(rng.standard_normal((B, S, Hkv, 128)))
    args = [dt.to_bf16(a) for a in (q, k, v)]
    dk = DeviceKernel.compile_and_load(full_attention, *args)
    assert dk.plan.kernel_kinds == ["attention"]
    got = dt.to_float32(baremetal_jit(full_attention)(*args))
    ref = K.causal_gqa_attention(q, k, v, causal=False)
    _close(got, ref)
    rows = [0, 77, 255]
    _close(got[:, rows], K.causal_attention_f64_loop(q, k, v, causal=False)[:, rows])
