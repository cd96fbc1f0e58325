"""GPU parity of the fused per-head RMSNorm + bf16-step RoPE launch
(``nk_head_rope_bf16``): the Qwen3 attention prologue (examples/models/
qwen3/kernels/attention.py:72-97, rope.py:4-48) lowered with the fused
pattern against the same graph lowered onto the generic steps (row norm
kernel, elementwise programs, gathers), bit for bit, and against the
oracle's op-by-op form; decode (runtime position) and prefill (sliced
tables) forms, head dims 64 and 128, partial workgroups, positions at and
past the table ends."""

import os

import numpy as np
import pytest
from parity import assert_close

from nkipy_amd.core import dtypes as dt
from nkipy_amd.core import tensor_apis
from nkipy_amd.core.trace import NKIPyKernel
from nkipy_amd.dispatch.lower import lower
from nkipy_amd.dispatch.patterns import default_patterns
from nkipy_amd.dispatch.patterns_attention import HeadRopePattern
from nkipy_amd.kernels.qwen3 import apply_rotary_emb_kernel, compute_cos_sin_cache
from nkipy_amd.kernels.rmsnorm import rmsnorm_kernel
from nkipy_amd.runtime import DeviceKernel, DeviceTensor
from oracle import kernels as K
from oracle import numerics as N

pytestmark = pytest.mark.gpu

EPS = 1e-6
THETA = 1.0e6


def _prologue(H, Hkv, D, MAXS, decode):
    def split_norm(qkv, q_norm_weight, k_norm_weight):
        B, S, _ = qkv.shape
        xq, xk, _ = np.split(qkv, [H * D, (H + Hkv) * D], axis=2)
        xq = rmsnorm_kernel(xq.reshape(B, S, H, D), q_norm_weight, EPS)
        xk = rmsnorm_kernel(xk.reshape(B, S, Hkv, D), k_norm_weight, EPS)
        cos, sin = compute_cos_sin_cache(D, MAXS, base=THETA)
        return xq, xk, tensor_apis.constant(cos).astype(qkv.dtype), tensor_apis.constant(sin).astype(qkv.dtype)

    if decode:
        def prologue(qkv, q_norm_weight, k_norm_weight, start_pos):
            xq, xk, cos, sin = split_norm(qkv, q_norm_weight, k_norm_weight)
            return apply_rotary_emb_kernel(xq, xk, cos[start_pos], sin[start_pos])
    else:
        def prologue(qkv, q_norm_weight, k_norm_weight):
            xq, xk, cos, sin = split_norm(qkv, q_norm_weight, k_norm_weight)
            S = qkv.shape[1]
            return apply_rotary_emb_kernel(xq, xk, cos[0:S], sin[0:S])
    return prologue


def _run_both(fn, args):
    """Outputs of the fused lowering and of the lowering without the
    pattern, as float32 arrays; asserts which steps each took."""
    g = NKIPyKernel.trace(fn).specialize(*args)
    fused_plan = lower(g)
    generic_plan = lower(g, [p for p in default_patterns() if not isinstance(p, HeadRopePattern)])
    assert fused_plan.kernel_kinds.count("head_rope") == 1, fused_plan.kernel_kinds
    assert "head_rope" not in generic_plan.kernel_kinds
    names = [p.name for p in g.parameters]
    outs = []
    for i, plan in enumerate((fused_plan, generic_plan)):
        dk = DeviceKernel(g, plan, f"{fn.__name__}_{i}")
        res = dk({n: DeviceTensor.from_numpy(a, name=n) for n, a in zip(names, args)})
        outs.append([dt.to_float32(res[k].numpy()) for k in sorted(res)])
    return outs


def _check_oracle(got, ref, name):
    """The norm's fp32 sum of squares follows the row kernel's order, not
    NumPy's: a mean may round differently, which moves a whole row by up to
    a bf16 step.  Most outputs equal the oracle; all within one step."""
    assert np.mean(got == ref) >= 0.99, name
    assert_close(got, ref, name, axis=-1)


DECODE = [(1, 32, 8, 128, 4096, 4000), (3, 8, 2, 128, 512, 0), (2, 4, 4, 64, 256, 255), (8, 16, 4, 128, 1024, 517),
          (5, 12, 3, 64, 300, 131)]


@pytest.mark.parametrize("B,H,Hkv,D,MAXS,pos", DECODE)
def test_head_rope_decode(gpu, B, H, Hkv, D, MAXS, pos):
    print(f"head rope decode B={B} H={H}/{Hkv} D={D} MAXS={MAXS} pos={pos}", flush=True)
    rng = np.random.default_rng(B * 100 + pos)
    qkv = N.bf16_round(rng.standard_normal((B, 1, (H + 2 * Hkv) * D)) * 1.5)
    wq, wk = N.bf16_round(rng.uniform(0.5, 1.5, D)), N.bf16_round(rng.uniform(0.5, 1.5, D))
    args = [dt.to_bf16(qkv), dt.to_bf16(wq), dt.to_bf16(wk), np.array([pos], np.int32)]
    fused, generic = _run_both(_prologue(H, Hkv, D, MAXS, True), args)
    for a, b in zip(fused, generic):
        np.testing.assert_array_equal(a, b)
    q, k = K.qwen3_head_prologue(qkv, wq, wk, EPS, H, Hkv, D, np.array([pos]), THETA)
    _check_oracle(fused[0], q, "head rope decode q")
    _check_oracle(fused[1], k, "head rope decode k")


@pytest.mark.parametrize("pos", [-3, 1030])
def test_head_rope_position_outside_table(gpu, pos):
    """A position past either end of the table reads the row the gather
    step reads (negative from the end, then clamped): fused equals generic."""
    rng = np.random.default_rng(7)
    H, Hkv, D, MAXS = 8, 2, 128, 1024
    qkv = N.bf16_round(rng.standard_normal((2, 1, (H + 2 * Hkv) * D)))
    w = N.bf16_round(rng.uniform(0.5, 1.5, D))
    args = [dt.to_bf16(qkv), dt.to_bf16(w), dt.to_bf16(w), np.array([pos], np.int32)]
    fused, generic = _run_both(_prologue(H, Hkv, D, MAXS, True), args)
    for a, b in zip(fused, generic):
        np.testing.assert_array_equal(a, b)
    row = min(pos + MAXS if pos < 0 else pos, MAXS - 1)
    q, k = K.qwen3_head_prologue(qkv, w, w, EPS, H, Hkv, D, np.array([row]), THETA)
    _check_oracle(fused[0], q, "head rope clamped q")


PREFILL = [(2, 64, 8, 2, 128, 512), (1, 300, 4, 1, 128, 512), (3, 37, 6, 2, 64, 64), (1, 2048, 32, 8, 128, 4096)]


@pytest.mark.parametrize("B,S,H,Hkv,D,MAXS", PREFILL)
def test_head_rope_prefill(gpu, B, S, H, Hkv, D, MAXS):
    print(f"head rope prefill B={B} S={S} H={H}/{Hkv} D={D} MAXS={MAXS}", flush=True)
    rng = np.random.default_rng(S + D)
    qkv = N.bf16_round(rng.standard_normal((B, S, (H + 2 * Hkv) * D)))
    wq, wk = N.bf16_round(rng.uniform(0.5, 1.5, D)), N.bf16_round(rng.uniform(0.5, 1.5, D))
    args = [dt.to_bf16(qkv), dt.to_bf16(wq), dt.to_bf16(wk)]
    fused, generic = _run_both(_prologue(H, Hkv, D, MAXS, False), args)
    for a, b in zip(fused, generic):
        np.testing.assert_array_equal(a, b)
    q, k = K.qwen3_head_prologue(qkv, wq, wk, EPS, H, Hkv, D, np.arange(S), THETA)
    _check_oracle(fused[0], q, "head rope prefill q")
    _check_oracle(fused[1], k, "head rope prefill k")


def test_rope_only_bf16_tables(gpu):
    """No norm, bf16 tables given as arguments, one tensor of heads: the
    rotation alone equals the oracle's op-by-op form bit for bit."""
    B, S, H, D = 2, 48, 5, 128

    def rot(x, cos, sin):
        c = np.expand_dims(cos, axis=(0, 2))
        s = np.expand_dims(sin, axis=(0, 2))
        x0, x1 = x[:, :, :, :D // 2], x[:, :, :, D // 2:]
        return np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], axis=-1)

    rng = np.random.default_rng(3)
    x = N.bf16_round(rng.standard_normal((B, S, H, D)) * 3.0)
    cos, sin = K.rope_tables(D, S, THETA)
    cb, sb = N.bf16_round(cos), N.bf16_round(sin)
    args = [dt.to_bf16(x), dt.to_bf16(cb), dt.to_bf16(sb)]
    fused, generic = _run_both(rot, args)
    np.testing.assert_array_equal(fused[0], generic[0])
    np.testing.assert_array_equal(fused[0], K.rope_split_half_bf16_steps(x, cb, sb))


def _decode_prologue_with_cache(H, Hkv, D):
    def prologue(qkv, q_norm_weight, k_norm_weight, cache_k, cache_v, start_pos):
        B, S, _ = qkv.shape
        xq, xk, xv = np.split(qkv, [H * D, (H + Hkv) * D], axis=2)
        xq = rmsnorm_kernel(xq.reshape(B, S, H, D), q_norm_weight, EPS)
        xk = rmsnorm_kernel(xk.reshape(B, S, Hkv, D), k_norm_weight, EPS)
        cos, sin = compute_cos_sin_cache(D, cache_k.shape[1], base=THETA)
        cos = tensor_apis.constant(cos).astype(qkv.dtype)
        sin = tensor_apis.constant(sin).astype(qkv.dtype)
        xq, xk = apply_rotary_emb_kernel(xq, xk, cos[start_pos], sin[start_pos])
        cache_k[:, start_pos] = xk
        cache_v[:, start_pos] = xv.reshape(B, S, Hkv, D)
        return xq
    return prologue


@pytest.mark.parametrize("B,H,Hkv,D,MAXS,pos", [(2, 8, 2, 128, 512, 300), (8, 32, 8, 128, 4096, 4000),
                                                 (3, 4, 4, 64, 256, -2), (1, 8, 2, 128, 256, 259)])
def test_head_rope_writes_cache_rows(gpu, B, H, Hkv, D, MAXS, pos):
    """The decode prologue with its cache writes (cache[:, pos] = k, v) in
    the same launch: q and both caches bit-identical to the generic
    lowering (norm kernel, programs, gathers and scatters), a negative
    position counting from the end, a position past the cache dropping the
    writes as the scatter does (and reading the clamped table row)."""
    print(f"head rope cache writes B={B} H={H}/{Hkv} D={D} MAXS={MAXS} pos={pos}", flush=True)
    rng = np.random.default_rng(B * 7 + MAXS)
    qkv = N.bf16_round(rng.standard_normal((B, 1, (H + 2 * Hkv) * D)))
    wq, wk = N.bf16_round(rng.uniform(0.5, 1.5, D)), N.bf16_round(rng.uniform(0.5, 1.5, D))
    ck = N.bf16_round(rng.standard_normal((B, MAXS, Hkv, D)))
    cv = N.bf16_round(rng.standard_normal((B, MAXS, Hkv, D)))
    args = [dt.to_bf16(qkv), dt.to_bf16(wq), dt.to_bf16(wk), dt.to_bf16(ck), dt.to_bf16(cv),
            np.array([pos], np.int32)]
    fn = _decode_prologue_with_cache(H, Hkv, D)
    g = NKIPyKernel.trace(fn).specialize(*args)
    fused_plan = lower(g)
    generic_plan = lower(g, [p for p in default_patterns() if not isinstance(p, HeadRopePattern)])
    assert fused_plan.kernel_kinds == ["head_rope"], fused_plan.kernel_kinds
    assert "gather" in generic_plan.kernel_kinds
    names = [p.name for p in g.parameters]
    outs = []
    for i, plan in enumerate((fused_plan, generic_plan)):
        dk = DeviceKernel(g, plan, f"cache_prologue_{i}")
        res = dk({n: DeviceTensor.from_numpy(a, name=n) for n, a in zip(names, args)})
        outs.append({k: dt.to_float32(v.numpy()) for k, v in res.items()})
    for k in outs[0]:
        np.testing.assert_array_equal(outs[0][k], outs[1][k], err_msg=k)
    row = pos + MAXS if pos < 0 else pos
    if row < MAXS:
        q, k = K.qwen3_head_prologue(qkv, wq, wk, EPS, H, Hkv, D, np.array([row]), THETA)
        _check_oracle(outs[0]["output0"], q, "head rope cache q")
        _check_oracle(outs[0]["cache_k"][:, row], k[:, 0], "head rope cache k")
        np.testing.assert_array_equal(outs[0]["cache_v"][:, row],
                                      qkv[:, 0, (H + Hkv) * D:].reshape(B, Hkv, D))
        keep = np.arange(MAXS) != row
    else:
        keep = np.ones(MAXS, bool)  # the scatter drops a position past the cache
    np.testing.assert_array_equal(outs[0]["cache_k"][:, keep], ck[:, keep])
    np.testing.assert_array_equal(outs[0]["cache_v"][:, keep], cv[:, keep])


def _projected_prologue(H, Hkv, D):
    prologue = _decode_prologue_with_cache(H, Hkv, D)

    def fn(x, qkv_weight, q_norm_weight, k_norm_weight, cache_k, cache_v, start_pos):
        return prologue(np.matmul(x, qkv_weight), q_norm_weight, k_norm_weight, cache_k, cache_v, start_pos)
    return fn


@pytest.mark.parametrize("B,H,Hkv,D,hid,planes", [(8, 32, 8, 128, 4096, 16), (1, 8, 2, 128, 512, 2),
                                                   (16, 16, 4, 64, 2048, 8), (3, 32, 8, 128, 8192, 20),
                                                   (1, 4, 2, 64, 16384, None)])
def test_head_rope_adds_projection_planes(gpu, B, H, Hkv, D, hid, planes):
    """The decode projection of one token per sequence feeding the head
    prologue: the prologue adds the projection's fp32 partial-sum planes
    itself (two launches) and its q and cache rows equal those of the
    lowering that reduces the planes in their own launch first (three
    launches), bit for bit; a sequence whose token is all -0.0 checks the
    signed zero the reduction's + 0 turns into +0.  Past 32 planes the
    reduction keeps its launch."""
    from nkipy_amd.dispatch.patterns_attention import ProjectionPlanesFusion

    print(f"projection planes B={B} H={H}/{Hkv} D={D} hid={hid} planes={planes}", flush=True)
    MAXS, pos = 256, 100
    rng = np.random.default_rng(B * 13 + hid)
    x = N.bf16_round(rng.standard_normal((B, 1, hid)))
    x[0] = -0.0
    w = N.bf16_round(rng.standard_normal((hid, (H + 2 * Hkv) * D)) * hid ** -0.5)
    wq, wk = N.bf16_round(rng.uniform(0.5, 1.5, D)), N.bf16_round(rng.uniform(0.5, 1.5, D))
    ck = N.bf16_round(rng.standard_normal((B, MAXS, Hkv, D)))
    cv = N.bf16_round(rng.standard_normal((B, MAXS, Hkv, D)))
    args = [dt.to_bf16(a) for a in (x, w, wq, wk, ck, cv)] + [np.array([pos], np.int32)]
    g = NKIPyKernel.trace(_projected_prologue(H, Hkv, D)).specialize(*args)
    fused = lower(g)
    split = lower(g, [p for p in default_patterns() if not isinstance(p, ProjectionPlanesFusion)])
    syms = lambda p: [l.symbol for s in p.steps for l in s.launches(lambda v: 1 << 20)]
    assert fused.kernel_kinds == split.kernel_kinds == ["gemm", "head_rope"], fused.kernel_kinds
    sf, ss = syms(fused), syms(split)
    assert ss[1:] == ["nk_gemv_out_bf16", "nk_head_rope_bf16"], ss
    if planes is None:
        assert sf == ss, sf
    else:
        assert sf == [ss[0], "nk_head_rope_bf16"], sf
        assert fused.steps[1].launches(lambda v: 1 << 20)[0].args.nplanes == planes
    names = [p.name for p in g.parameters]
    outs = []
    for i, plan in enumerate((fused, split)):
        dk = DeviceKernel(g, plan, f"projected_prologue_{i}")
        res = dk({n: DeviceTensor.from_numpy(a, name=n) for n, a in zip(names, args)})
        outs.append({k: dt.numpy_storage(v.numpy()) for k, v in res.items()})
    for k in outs[0]:
        np.testing.assert_array_equal(outs[0][k], outs[1][k], err_msg=k)
    assert not np.signbit(dt.to_float32(outs[0]["cache_v"])[0, pos]).any()
