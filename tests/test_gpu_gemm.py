"""GPU parity of the MFMA GEMM kernels (launcher level) against NumPy fp32
matmul on the same bf16 / fp8 values, across layouts, edge tiles and fused
epilogues."""

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


def _bf16(rng, shape, scale=1.0):
    return N.bf16_round(rng.standard_normal(shape) * scale)


def _close(got, ref, tol=2e-2, axis=None, rounded=None):
    """bf16 bar of tests/parity.py (rtol 2e-2, atol min(1e-2, 2e-2 RMS))."""
    name = os.environ.get("PYTEST_CURRENT_TEST", "?").split(" ")[0]
    assert_close(got, ref, name, rtol=tol, axis=axis, rounded=rounded)


def _run(gpu, launch):
    launch.run(gpu)
    gpu.sync()


SHAPES = [(256, 256, 64), (512, 768, 320), (300, 520, 136), (64, 40, 16), (1000, 1000, 1000)]


# pp: the 8-wave kernel (default) and the 4-wave kernel
PP = [True, False]
# fp8 NT weights also have the 8-wave kernel with 64-deep K stages
PP8 = [True, False, "k64"]


def _kern(pp):
    return {"pingpong": pp is not False, "stage64": pp == "k64" if pp is not False else None}


@pytest.mark.parametrize("pp", PP)
@pytest.mark.parametrize("layout", ["nn", "nt"])
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("out", ["bf16", "f32"])
def test_gemm_bf16(gpu, layout, shape, out, pp):
    M, Nn, Kk = shape
    if layout == "nn" and Nn % 8:
        pytest.skip("NN needs N % 8 == 0")
    rng = np.random.default_rng(M + Nn + Kk)
    a = _bf16(rng, (M, Kk))
    b = _bf16(rng, (Kk, Nn) if layout == "nn" else (Nn, Kk), 0.05)
    bmat = b if layout == "nn" else b.T
    ref = a.astype(np.float64) @ bmat.astype(np.float64)
    ad = DeviceTensor.from_numpy(dt.to_bf16(a))
    bd = DeviceTensor.from_numpy(dt.to_bf16(b))
    cdt = dt.bfloat16 if out == "bf16" else dt.float32
    cd = DeviceTensor.empty((M, Nn), cdt)
    _run(gpu, LA.gemm(ad.ptr, bd.ptr, cd.ptr, M, Nn, Kk, layout=layout, b_dtype=dt.bfloat16, c_dtype=cdt,
                      pingpong=pp))
    got = dt.to_float32(cd.numpy())
    if out == "f32":
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4 * np.abs(ref).max())
    else:
        _close(got, ref)


@pytest.mark.parametrize("pp", PP)
@pytest.mark.parametrize("layout", ["nn", "nt"])
def test_gemm_swiglu(gpu, layout, pp):
    M, F, Kk = 512, 384, 256
    rng = np.random.default_rng(7)
    x = _bf16(rng, (M, Kk))
    wg = _bf16(rng, (Kk, F), 0.05)
    wu = _bf16(rng, (Kk, F), 0.05)
    ref = K.silu(x.astype(np.float64) @ wg) * (x.astype(np.float64) @ wu)
    if layout == "nn":
        # fused gate_up weight (K, 2F): up is a column offset of the same matrix
        gu = np.concatenate([wg, wu], axis=1)
        bd = DeviceTensor.from_numpy(dt.to_bf16(gu))
        b0, b1, ldb = bd.ptr, bd.ptr + F * 2, 2 * F
    else:
        gd = DeviceTensor.from_numpy(dt.to_bf16(np.ascontiguousarray(wg.T)))
        ud = DeviceTensor.from_numpy(dt.to_bf16(np.ascontiguousarray(wu.T)))
        b0, b1, ldb, bd = gd.ptr, ud.ptr, Kk, (gd, ud)
    xd = DeviceTensor.from_numpy(dt.to_bf16(x))
    hd = DeviceTensor.empty((M, F), dt.bfloat16)
    _run(gpu, LA.gemm(xd.ptr, b0, hd.ptr, M, F, Kk, layout=layout, b_dtype=dt.bfloat16,
                      c_dtype=dt.bfloat16, ldb=ldb, up_ptr=b1, pingpong=pp))
    _close(dt.to_float32(hd.numpy()), ref)


@pytest.mark.parametrize("pp", PP8)
def test_gemm_fp8_nt_scales_bias_residual(gpu, pp):
    M, Nn, Kk = 384, 512, 448
    rng = np.random.default_rng(11)
    x = _bf16(rng, (M, Kk))
    w = (rng.standard_normal((Nn, Kk)) * 0.02).astype(np.float32)
    codes, scale = N.quantize_per_channel_e4m3fn(w, axis=1)
    wdq = N.dequantize_e4m3fn(codes, scale, axis=1)
    bias = N.bf16_round(rng.standard_normal(Nn) * 0.1)
    res = N.bf16_round(rng.standard_normal((M, Nn)))
    ref = x.astype(np.float64) @ wdq.T.astype(np.float64) + bias + res
    xd = DeviceTensor.from_numpy(dt.to_bf16(x))
    wd = DeviceTensor.from_numpy(codes.view(dt.float8_e4m3fn))
    sd = DeviceTensor.from_numpy(scale.astype(np.float32))
    bd = DeviceTensor.from_numpy(dt.to_bf16(bias))
    rd = DeviceTensor.from_numpy(dt.to_bf16(res))
    cd = DeviceTensor.empty((M, Nn), dt.bfloat16)
    _run(gpu, LA.gemm(xd.ptr, wd.ptr, cd.ptr, M, Nn, Kk, layout="nt", b_dtype=dt.float8_e4m3fn,
                      c_dtype=dt.bfloat16, scale_ptr=sd.ptr, bias_ptr=bd.ptr, resid_ptr=rd.ptr,
                      **_kern(pp)))
    _close(dt.to_float32(cd.numpy()), ref)


@pytest.mark.parametrize("pp", PP8)
@pytest.mark.parametrize("Kk", [16, 64, 128, 192, 208, 576])
def test_gemm_fp8_nt_k_tiles(gpu, Kk, pp):
    """fp8 NT weights stream through an LDS ring (three stages in the 4-wave
    kernel, two in the 8-wave one); K of 1..9 tiles of 64 covers every ring
    phase at the loop exit (fp32 output, so the check is at
    fp32-accumulation level)."""
    M, Nn = 320, 272
    rng = np.random.default_rng(Kk)
    x = _bf16(rng, (M, Kk))
    w = (rng.standard_normal((Nn, Kk)) * 0.02).astype(np.float32)
    codes, scale = N.quantize_per_channel_e4m3fn(w, axis=1)
    ref = x.astype(np.float64) @ N.dequantize_e4m3fn(codes, scale, axis=1).T.astype(np.float64)
    xd = DeviceTensor.from_numpy(dt.to_bf16(x))
    wd = DeviceTensor.from_numpy(codes.view(dt.float8_e4m3fn))
    sd = DeviceTensor.from_numpy(scale.astype(np.float32))
    cd = DeviceTensor.empty((M, Nn), dt.float32)
    _run(gpu, LA.gemm(xd.ptr, wd.ptr, cd.ptr, M, Nn, Kk, layout="nt", b_dtype=dt.float8_e4m3fn,
                      c_dtype=dt.float32, scale_ptr=sd.ptr, **_kern(pp)))
    np.testing.assert_allclose(cd.numpy(), ref, rtol=1e-4, atol=1e-4 * np.abs(ref).max())


@pytest.mark.parametrize("pp", PP8)
def test_gemm_fp8_swiglu_nt(gpu, pp):
    M, F, Kk = 256, 256, 512
    rng = np.random.default_rng(12)
    x = _bf16(rng, (M, Kk))
    wg = (rng.standard_normal((F, Kk)) * 0.02).astype(np.float32)
    wu = (rng.standard_normal((F, Kk)) * 0.02).astype(np.float32)
    cg, sg = N.quantize_per_channel_e4m3fn(wg, axis=1)
    cu, su = N.quantize_per_channel_e4m3fn(wu, axis=1)
    g = x.astype(np.float64) @ N.dequantize_e4m3fn(cg, sg, axis=1).T
    u = x.astype(np.float64) @ N.dequantize_e4m3fn(cu, su, axis=1).T
    ref = K.silu(g) * u
    t = [DeviceTensor.from_numpy(v) for v in (dt.to_bf16(x), cg.view(dt.float8_e4m3fn), cu.view(dt.float8_e4m3fn),
                                              sg.astype(np.float32), su.astype(np.float32))]
    hd = DeviceTensor.empty((M, F), dt.bfloat16)
    _run(gpu, LA.gemm(t[0].ptr, t[1].ptr, hd.ptr, M, F, Kk, layout="nt", b_dtype=dt.float8_e4m3fn,
                      c_dtype=dt.bfloat16, scale_ptr=t[3].ptr, up_ptr=t[2].ptr, up_scale_ptr=t[4].ptr,
                      **_kern(pp)))
    _close(dt.to_float32(hd.numpy()), ref)


@pytest.mark.parametrize("shape", [(256, 256, 64), (300, 520, 208), (520, 272, 576), (64, 40, 16),
                                   (1000, 768, 1000 // 16 * 16)])
@pytest.mark.parametrize("variant", ["plain", "f32", "swiglu", "bias_resid"])
def test_gemm_fp8_stage64_bit_exact(gpu, shape, variant):
    """The 64-deep-stage kernel accumulates over k in the same order as the
    32-deep one: outputs equal bit for bit, edge tiles and K tails included."""
    M, Nn, Kk = shape
    print(f"gemm fp8 stage64 {variant} M={M} N={Nn} K={Kk}", flush=True)
    rng = np.random.default_rng(M + Nn + Kk)
    x = _bf16(rng, (M, Kk))
    w = (rng.standard_normal((Nn, Kk)) * 0.02).astype(np.float32)
    codes, scale = N.quantize_per_channel_e4m3fn(w, axis=1)
    xd = DeviceTensor.from_numpy(dt.to_bf16(x))
    wd = DeviceTensor.from_numpy(codes.view(dt.float8_e4m3fn))
    sd = DeviceTensor.from_numpy(scale.astype(np.float32))
    kw = {"scale_ptr": sd.ptr}
    keep = []
    out_dt = dt.float32 if variant == "f32" else dt.bfloat16
    n_out = Nn
    if variant == "swiglu":
        wu = (rng.standard_normal((Nn, Kk)) * 0.02).astype(np.float32)
        cu, su = N.quantize_per_channel_e4m3fn(wu, axis=1)
        keep = [DeviceTensor.from_numpy(cu.view(dt.float8_e4m3fn)), DeviceTensor.from_numpy(su.astype(np.float32))]
        kw.update(up_ptr=keep[0].ptr, up_scale_ptr=keep[1].ptr)
    if variant == "bias_resid":
        keep = [DeviceTensor.from_numpy(dt.to_bf16(N.bf16_round(rng.standard_normal(Nn) * 0.1))),
                DeviceTensor.from_numpy(dt.to_bf16(N.bf16_round(rng.standard_normal((M, Nn))))),]
        kw.update(bias_ptr=keep[0].ptr, resid_ptr=keep[1].ptr, round_before_resid=True)
    outs = []
    # 32-deep kernel; 64-deep with the direct epilogue; 64-deep with the
    # output staged through LDS (where the output allows it)
    runs = [(False, None), (True, False)] + ([(True, True)] if out_dt == dt.bfloat16 else [])
    for k64, staged in runs:
        cd = DeviceTensor.empty((M, n_out), out_dt)
        _run(gpu, LA.gemm(xd.ptr, wd.ptr, cd.ptr, M, Nn, Kk, layout="nt", b_dtype=dt.float8_e4m3fn,
                          c_dtype=out_dt, stage64=k64, staged=staged, **kw))
        outs.append(dt.to_float32(cd.numpy()) if out_dt == dt.bfloat16 else cd.numpy())
    for o in outs[1:]:
        np.testing.assert_array_equal(o, outs[0])



@pytest.mark.parametrize("shape", [(256, 256, 64), (300, 520, 136), (520, 272, 600), (64, 40, 16),
                                   (1000, 768, 1000), (256, 512, 4128)])
@pytest.mark.parametrize("variant", ["plain", "f32", "swiglu", "bias_resid"])
def test_gemm_bf16_nn_stage64_bit_exact(gpu, shape, variant):
    """bf16 K x N weights: the kernel with 64-deep A stages reads the same
    fragments in the same MFMA order as the 32-deep one, so outputs equal
    bit for bit (edge tiles, K tails of 8 / 24 / 32 past a 64-k block, and
    the output staged through LDS included); the 32-deep output also meets
    the bf16 bar against NumPy."""
    M, Nn, Kk = shape
    print(f"gemm bf16 nn stage64 {variant} M={M} N={Nn} K={Kk}", flush=True)
    rng = np.random.default_rng(M * 7 + Nn + Kk)
    x = _bf16(rng, (M, Kk))
    w = _bf16(rng, (Kk, Nn), 0.05)
    xd = DeviceTensor.from_numpy(dt.to_bf16(x))
    wd = DeviceTensor.from_numpy(dt.to_bf16(w))
    kw, keep = {}, []
    out_dt = dt.float32 if variant == "f32" else dt.bfloat16
    ref = x.astype(np.float64) @ w.astype(np.float64)
    if variant == "swiglu":
        # fused gate_up weight (K, 2N): up is a column offset, ldb = 2N
        wu = _bf16(rng, (Kk, Nn), 0.05)
        wd = DeviceTensor.from_numpy(dt.to_bf16(np.concatenate([w, wu], axis=1)))
        kw.update(up_ptr=wd.ptr + Nn * 2, ldb=2 * Nn)
        ref = K.silu(ref) * (x.astype(np.float64) @ wu.astype(np.float64))
    if variant == "bias_resid":
        bias = N.bf16_round(rng.standard_normal(Nn) * 0.1)
        res = N.bf16_round(rng.standard_normal((M, Nn)))
        keep = [DeviceTensor.from_numpy(dt.to_bf16(bias)), DeviceTensor.from_numpy(dt.to_bf16(res))]
        kw.update(bias_ptr=keep[0].ptr, resid_ptr=keep[1].ptr, round_before_resid=True)
        ref = N.bf16_round(ref + bias) + res
    outs = []
    runs = [(False, None), (True, False)] + ([(True, True)] if out_dt == dt.bfloat16 else [])
    for k64, staged in runs:
        cd = DeviceTensor.empty((M, Nn), out_dt)
        launch = LA.gemm(xd.ptr, wd.ptr, cd.ptr, M, Nn, Kk, layout="nn", b_dtype=dt.bfloat16,
                         c_dtype=out_dt, stage64=k64, staged=staged, **kw)
        assert launch.symbol.startswith("nk_gemm8k_" if k64 else "nk_gemm8_")
        _run(gpu, launch)
        outs.append(dt.to_float32(cd.numpy()) if out_dt == dt.bfloat16 else cd.numpy())
    for o in outs[1:]:
        np.testing.assert_array_equal(o, outs[0])
    if out_dt == dt.float32:
        np.testing.assert_allclose(outs[0], ref, rtol=1e-4, atol=1e-4 * np.abs(ref).max())
    else:
        _close(outs[0], ref)


def test_fp8_decode_all_codes(gpu):
    """The fp8 -> bf16 decode used by the GEMM staging, on every E4M3FN code
    (zeros, subnormals, normals, +-448, NaN) against the oracle's table."""
    from nkipy_amd.dispatch.generic import decode_e4m3

    codes = np.tile(np.arange(256, dtype=np.uint8), 4)
    src = DeviceTensor.from_numpy(codes.view(dt.float8_e4m3fn))
    dst = DeviceTensor.empty(codes.shape, dt.bfloat16)
    decode_e4m3(src.ptr, dst.ptr, codes.size).run(gpu)
    gpu.sync()
    got = dt.to_float32(dst.numpy())
    ref = N.E4M3FN_TABLE[codes]
    nan = np.isnan(ref)
    np.testing.assert_array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan], ref[~nan])
    # signed zero survives
    bits = dst.numpy().view(np.uint16)
    assert bits[0x80] == 0x8000 and bits[0x00] == 0x0000


@pytest.mark.parametrize("shape", [(300, 520, 136), (256, 256, 64), (130, 264, 200)])
def test_gemm_fp8_nn_scales(gpu, shape):
    """fp8 (in, out) weights: codes staged through registers and transposed."""
    M, Nn, Kk = shape
    rng = np.random.default_rng(M * 3 + Kk)
    x = _bf16(rng, (M, Kk))
    w = (rng.standard_normal((Nn, Kk)) * 0.02).astype(np.float32)
    codes, scale = N.quantize_per_channel_e4m3fn(w, axis=1)
    ref = x.astype(np.float64) @ N.dequantize_e4m3fn(codes, scale, axis=1).T.astype(np.float64)
    xd = DeviceTensor.from_numpy(dt.to_bf16(x))
    wd = DeviceTensor.from_numpy(np.ascontiguousarray(codes.T).view(dt.float8_e4m3fn))
    sd = DeviceTensor.from_numpy(scale.astype(np.float32))
    cd = DeviceTensor.empty((M, Nn), dt.bfloat16)
    _run(gpu, LA.gemm(xd.ptr, wd.ptr, cd.ptr, M, Nn, Kk, layout="nn", b_dtype=dt.float8_e4m3fn,
                      c_dtype=dt.bfloat16, scale_ptr=sd.ptr))
    _close(dt.to_float32(cd.numpy()), ref)


@pytest.mark.parametrize("pp", PP)
@pytest.mark.parametrize("group_m", [1, 3, 6])
def test_gemm_tile_walk_group(gpu, group_m, pp):
    """The tile-walk group size only reorders tiles: results are bit-identical
    to the default walk, including a ragged edge (tiles_m = 5, tiles_n = 3)."""
    M, Nn, Kk = 1100, 700, 320
    rng = np.random.default_rng(group_m)
    a = _bf16(rng, (M, Kk))
    b = _bf16(rng, (Nn, Kk), 0.05)
    ad = DeviceTensor.from_numpy(dt.to_bf16(a))
    bd = DeviceTensor.from_numpy(dt.to_bf16(b))
    outs = []
    for g in (0, group_m):
        cd = DeviceTensor.empty((M, Nn), dt.bfloat16)
        launch = LA.gemm(ad.ptr, bd.ptr, cd.ptr, M, Nn, Kk, layout="nt", b_dtype=dt.bfloat16,
                         c_dtype=dt.bfloat16, pingpong=pp)
        launch.args.group_m = g
        _run(gpu, launch)
        outs.append(cd.numpy())
    np.testing.assert_array_equal(outs[0], outs[1])
    _close(dt.to_float32(outs[1]), a.astype(np.float64) @ b.T.astype(np.float64))


def test_traced_residual_keeps_cast_points(gpu):
    """``z + (x @ W^T).astype(bf16)``: the product is rounded to bf16 before
    the residual add, as the NumPy code says (the fused epilogue must not add
    the fp32 product).  Cancellation between z and the product exposes a
    missing rounding as errors of a whole ulp of the product."""
    from nkipy_amd.runtime import DeviceKernel, baremetal_jit

    def proj_residual(z, x, w):
        return z + np.matmul(x, np.transpose(w)).astype(z.dtype)

    rng = np.random.default_rng(31)
    m, n, k = 256, 512, 1024
    x = N.bf16_round(rng.standard_normal((m, k)))
    w = N.bf16_round(rng.standard_normal((n, k)) * 0.3)
    prod = N.bf16_round(x @ w.T)
    z = N.bf16_round(-prod + rng.standard_normal((m, n)) * 0.05)  # y = z + prod is small
    args = [dt.to_bf16(a) for a in (z, x, w)]
    dk = DeviceKernel.compile_and_load(proj_residual, *args)
    assert dk.plan.kernel_kinds == ["gemm"]
    got = dt.to_float32(baremetal_jit(proj_residual)(*args))
    p = x.astype(np.float64) @ w.T.astype(np.float64)
    ref = N.bf16_round(z + N.bf16_round(p))
    _close(got, ref, rounded=p)
    # without the rounding of the product, most elements would be off
    unrounded = N.bf16_round(z + p)
    assert np.mean(unrounded != ref) > 0.2


@pytest.mark.parametrize("M,seq,nq,nk,nv,K", [(300, 100, 1024, 128, 128, 512), (256, 64, 128, 128, 256, 256),
                                             (520, 130, 384, 256, 128, 192)])
def test_gemm_rope_staged_bit_exact(gpu, M, seq, nq, nk, nv, K):
    """The rotary epilogue staged through LDS equals the direct one bit for
    bit, on tiles that mix q / k or k / v heads, on edge rows and columns."""
    print(f"gemm rope staged M={M} seq={seq} nq={nq} nk={nk} nv={nv} K={K}", flush=True)
    NC = nq + nk + nv
    rng = np.random.default_rng(M + NC + K)
    x = _bf16(rng, (M, K))
    w = (rng.standard_normal((NC, K)) * 0.02).astype(np.float32)
    codes, scale = N.quantize_per_channel_e4m3fn(w, axis=1)
    ang = np.arange(seq)[:, None] * (5.0e5 ** (-np.arange(64) / 64.0))[None, :]
    cos = DeviceTensor.from_numpy(np.cos(ang).astype(np.float32))
    sin = DeviceTensor.from_numpy(np.sin(ang).astype(np.float32))
    xd = DeviceTensor.from_numpy(dt.to_bf16(x))
    wd = DeviceTensor.from_numpy(codes.view(dt.float8_e4m3fn))
    sd = DeviceTensor.from_numpy(scale.astype(np.float32))
    outs = []
    for staged in (False, True):
        q = DeviceTensor.empty((M, nq), dt.bfloat16)
        k = DeviceTensor.empty((M, nk), dt.bfloat16)
        c = DeviceTensor.from_numpy(np.zeros((M, NC), dtype=dt.bfloat16))
        rope = LA.GemmRope(cos.ptr, sin.ptr, q.ptr, k.ptr, 64, seq, nq, nk)
        _run(gpu, LA.gemm(xd.ptr, wd.ptr, c.ptr, M, NC, K, layout="nt", b_dtype=dt.float8_e4m3fn,
                          c_dtype=dt.bfloat16, scale_ptr=sd.ptr, rope=rope, staged=staged))
        outs.append([dt.to_float32(t.numpy()) for t in (q, k)] + [dt.to_float32(c.numpy())[:, nq + nk:]])
    for a, b in zip(*outs):
        np.testing.assert_array_equal(b, a)
