"""GPU parity of the few-row projection kernels (the decode case: the VALU
form up to 8 rows, the MFMA form up to 32 rows of bf16 K x N weights, the
MFMA GEMM over K ranges) against NumPy float64 matmul on the same bf16 /
fp8 values, across layouts, row counts, N and K tails and the GEMM's
epilogues; against each other on the same operands; and the lowering of
decode-shaped projections onto them."""

import os

import numpy as np
import pytest
from parity import assert_close, launch_symbols

from nkipy_amd.core import dtypes as dt
from nkipy_amd.dispatch import launchers as LA
from nkipy_amd.runtime import DeviceTensor
from oracle import kernels as K
from oracle import numerics as N

pytestmark = pytest.mark.gpu


def _close(got, ref, **kw):
    name = os.environ.get("PYTEST_CURRENT_TEST", "?").split(" ")[0]
    assert_close(got, ref, name, **kw)


def _run(gpu, launches):
    for launch in launches:
        launch.run(gpu)
    gpu.sync()


def _weights(rng, layout, Nn, Kk, fp8):
    """bf16 or fp8 weights (NN: K x N, NT: N x K) -> (device array, per-column
    scales or None, float64 K x N matrix of their values)."""
    shape = (Kk, Nn) if layout == "nn" else (Nn, Kk)
    w = (rng.standard_normal(shape) * 0.05).astype(np.float32)
    if not fp8:
        wb = N.bf16_round(w)
        mat = wb if layout == "nn" else wb.T
        return dt.to_bf16(wb), None, mat.astype(np.float64)
    axis = 0 if layout == "nn" else 1  # the input-feature axis
    codes, scale = N.quantize_per_channel_e4m3fn(w, axis=axis)
    deq = N.dequantize_e4m3fn(codes, scale, axis=axis).astype(np.float64)
    return codes.view(dt.float8_e4m3fn), scale.reshape(-1).astype(np.float32), deq if layout == "nn" else deq.T


CASES = [  # (layout, fp8, M, N, K): row counts 1 / 3 / 8, N and K tails
    ("nn", False, 1, 6144, 4096), ("nn", False, 3, 264, 1000), ("nn", False, 8, 4096, 2048),
    ("nn", True, 1, 512, 1032), ("nn", True, 5, 1000, 4096),
    ("nt", False, 1, 4096, 4096), ("nt", False, 2, 100, 1000), ("nt", False, 8, 1000, 520),
    ("nt", True, 1, 4096, 14336), ("nt", True, 4, 4104, 1008), ("nt", True, 7, 300, 2048),
]


@pytest.mark.parametrize("layout,fp8,M,Nn,Kk", CASES)
@pytest.mark.parametrize("epi", ["plain", "f32", "bias_resid", "rounded"])
def test_gemv_matches_float64(gpu, layout, fp8, M, Nn, Kk, epi):
    rng = np.random.default_rng(M * 7 + Nn + Kk)
    print(f"gemv {layout} fp8={fp8} M={M} N={Nn} K={Kk} {epi}", flush=True)
    x = N.bf16_round(rng.standard_normal((M, Kk)))
    wdev, scale, wmat = _weights(rng, layout, Nn, Kk, fp8)
    prod = x.astype(np.float64) @ wmat
    bias = N.bf16_round(rng.standard_normal(Nn) * 0.1)
    res = N.bf16_round(rng.standard_normal((M, Nn)))
    out = dt.float32 if epi == "f32" else dt.bfloat16
    kw = {}
    ref = prod
    t = {"x": DeviceTensor.from_numpy(dt.to_bf16(x)), "w": DeviceTensor.from_numpy(wdev)}
    if scale is not None:
        t["s"] = DeviceTensor.from_numpy(scale)
        kw["scale_ptr"] = t["s"].ptr
    if epi in ("bias_resid", "rounded"):
        t["b"] = DeviceTensor.from_numpy(dt.to_bf16(bias))
        t["r"] = DeviceTensor.from_numpy(dt.to_bf16(res))
        kw.update(bias_ptr=t["b"].ptr, resid_ptr=t["r"].ptr)
        if epi == "rounded":  # ((x @ w).astype(bf16) + bias).astype(bf16) + r
            kw.update(round_before_bias=True, round_before_resid=True)
            ref = N.bf16_round(N.bf16_round(prod) + bias) + res
        else:
            ref = prod + bias + res
    c = DeviceTensor.empty((M, Nn), out)
    ws = DeviceTensor.empty((LA.gemv_workspace_bytes(M, Nn, Kk, layout, fp8),), dt.uint8)
    _run(gpu, LA.gemv(t["x"].ptr, t["w"].ptr, c.ptr, M, Nn, Kk, layout=layout,
                      b_dtype=dt.float8_e4m3fn if fp8 else dt.bfloat16, c_dtype=out, ws_ptr=ws.ptr, **kw))
    got = c.numpy() if out == dt.float32 else dt.to_float32(c.numpy())
    if out == dt.float32:  # fp32-accumulation level
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4 * np.abs(ref).max())
    else:
        _close(got, ref, axis=-1, rounded=N.bf16_round(prod) if epi == "rounded" else None)


@pytest.mark.parametrize("layout,fp8,M,Nn,Kk", [("nn", False, 1, 14336, 4096), ("nt", True, 8, 2056, 4096),
                                                ("nn", True, 3, 1024, 520), ("nt", False, 1, 700, 3000)])
def test_gemv_swiglu(gpu, layout, fp8, M, Nn, Kk):
    rng = np.random.default_rng(Nn + Kk)
    x = N.bf16_round(rng.standard_normal((M, Kk)))
    wg, sg, mg = _weights(rng, layout, Nn, Kk, fp8)
    wu, su, mu = _weights(rng, layout, Nn, Kk, fp8)
    ref = K.silu(x.astype(np.float64) @ mg) * (x.astype(np.float64) @ mu)
    t = [DeviceTensor.from_numpy(v) for v in (dt.to_bf16(x), wg, wu)]
    kw = {}
    if fp8:
        s = [DeviceTensor.from_numpy(v) for v in (sg, su)]
        kw = {"scale_ptr": s[0].ptr, "up_scale_ptr": s[1].ptr}
    h = DeviceTensor.empty((M, Nn), dt.bfloat16)
    ws = DeviceTensor.empty((LA.gemv_workspace_bytes(M, Nn, Kk, layout, fp8, swiglu=True),), dt.uint8)
    _run(gpu, LA.gemv(t[0].ptr, t[1].ptr, h.ptr, M, Nn, Kk, layout=layout,
                      b_dtype=dt.float8_e4m3fn if fp8 else dt.bfloat16, c_dtype=dt.bfloat16, ws_ptr=ws.ptr,
                      up_ptr=t[2].ptr, **kw))
    _close(dt.to_float32(h.numpy()), ref, axis=-1)


@pytest.mark.parametrize("layout,fp8", [("nn", False), ("nt", False), ("nt", True)])
def test_gemv_against_mfma_gemm(gpu, layout, fp8):
    """Same operands through the split-K kernels and the MFMA GEMM: fp32
    results within the difference of two summation orders."""
    M, Nn, Kk = 4, 2048, 4096
    rng = np.random.default_rng(5)
    x = N.bf16_round(rng.standard_normal((M, Kk)))
    wdev, scale, _ = _weights(rng, layout, Nn, Kk, fp8)
    t = [DeviceTensor.from_numpy(v) for v in (dt.to_bf16(x), wdev)]
    kw = {}
    if fp8:
        sd = DeviceTensor.from_numpy(scale)
        kw["scale_ptr"] = sd.ptr
    bt = dt.float8_e4m3fn if fp8 else dt.bfloat16
    c1, c2 = DeviceTensor.empty((M, Nn), dt.float32), DeviceTensor.empty((M, Nn), dt.float32)
    ws = DeviceTensor.empty((LA.gemv_workspace_bytes(M, Nn, Kk, layout, fp8),), dt.uint8)
    _run(gpu, LA.gemv(t[0].ptr, t[1].ptr, c1.ptr, M, Nn, Kk, layout=layout, b_dtype=bt, c_dtype=dt.float32,
                      ws_ptr=ws.ptr, **kw))
    _run(gpu, [LA.gemm(t[0].ptr, t[1].ptr, c2.ptr, M, Nn, Kk, layout=layout, b_dtype=bt, c_dtype=dt.float32,
                       **kw)])
    a, b = c1.numpy(), c2.numpy()
    np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-5 * np.abs(b).max())


@pytest.mark.parametrize("layout,symbol", [("nn", "nk_gemv_mfma_nn_bf16_t1"), ("nt", "nk_gemv_nt_bf16_m1")])
def test_decode_projection_lowers_to_gemv(gpu, layout, symbol):
    """A traced decode-shaped projection (x (1, 1, 4096) @ W, W (4096, 6144)
    or W^T with W (6144, 4096), bf16) lowers to the few-row kernels (bf16
    K x N weights: the MFMA form) and matches float64."""
    from nkipy_amd.runtime import DeviceKernel, baremetal_jit

    def proj_nn(x, w):
        return np.matmul(x, w)

    def proj_nt(x, w):
        return np.matmul(x, w.T)

    proj = proj_nn if layout == "nn" else proj_nt
    rng = np.random.default_rng(3)
    x = N.bf16_round(rng.standard_normal((1, 1, 4096)))
    w = N.bf16_round(rng.standard_normal((4096, 6144) if layout == "nn" else (6144, 4096)) * 0.02)
    args = [dt.to_bf16(a) for a in (x, w)]
    dk = DeviceKernel.compile_and_load(proj, *args)
    assert dk.plan.kernel_kinds == ["gemm"]
    assert launch_symbols(dk.plan) == [symbol, "nk_gemv_out_bf16"]
    got = dt.to_float32(baremetal_jit(proj)(*args))
    wm = w.astype(np.float64) if layout == "nn" else w.astype(np.float64).T
    _close(got, x.astype(np.float64) @ wm, axis=-1)


# ---------------------------------------------------------------------------
# The MFMA form of the few-row projection (bf16 K x N weights, M <= 32)
# ---------------------------------------------------------------------------
MFMA_CASES = [  # (M, N, K, ldb): 16-row tiles full / partial / two, N and K tails, strided weights
    (1, 6144, 4096, None), (5, 264, 1000, None), (8, 4096, 14336, None), (13, 1000, 328, 1008),
    (16, 2048, 4104, None), (17, 520, 2056, None), (32, 4096, 4096, 4104), (2, 24576, 520, None),
]


@pytest.mark.parametrize("M,Nn,Kk,ldb", MFMA_CASES)
@pytest.mark.parametrize("epi", ["plain", "f32", "bias_resid", "rounded"])
def test_gemv_mfma_matches_float64(gpu, M, Nn, Kk, ldb, epi):
    rng = np.random.default_rng(M * 11 + Nn + Kk)
    ks, kc = LA.gemv_mfma_split(M, Nn, Kk)
    print(f"gemv_mfma M={M} N={Nn} K={Kk} ldb={ldb} {epi} split={ks}x{kc}", flush=True)
    x = N.bf16_round(rng.standard_normal((M, Kk)))
    ld = Nn if ldb is None else ldb
    wfull = N.bf16_round(rng.standard_normal((Kk, ld)) * 0.05)
    wmat = wfull[:, :Nn].astype(np.float64)
    prod = x.astype(np.float64) @ wmat
    bias = N.bf16_round(rng.standard_normal(Nn) * 0.1)
    res = N.bf16_round(rng.standard_normal((M, Nn)))
    out = dt.float32 if epi == "f32" else dt.bfloat16
    kw = {}
    ref = prod
    t = {"x": DeviceTensor.from_numpy(dt.to_bf16(x)), "w": DeviceTensor.from_numpy(dt.to_bf16(wfull))}
    if epi in ("bias_resid", "rounded"):
        t["b"] = DeviceTensor.from_numpy(dt.to_bf16(bias))
        t["r"] = DeviceTensor.from_numpy(dt.to_bf16(res))
        kw.update(bias_ptr=t["b"].ptr, resid_ptr=t["r"].ptr)
        if epi == "rounded":
            kw.update(round_before_bias=True, round_before_resid=True)
            ref = N.bf16_round(N.bf16_round(prod) + bias) + res
        else:
            ref = prod + bias + res
    c = DeviceTensor.empty((M, Nn), out)
    ws = DeviceTensor.empty((LA.gemv_mfma_workspace_bytes(M, Nn, Kk),), dt.uint8)
    _run(gpu, LA.gemv_mfma(t["x"].ptr, t["w"].ptr, c.ptr, M, Nn, Kk, c_dtype=out, ws_ptr=ws.ptr, ldb=ld, **kw))
    got = c.numpy() if out == dt.float32 else dt.to_float32(c.numpy())
    if out == dt.float32:
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4 * np.abs(ref).max())
    else:
        _close(got, ref, axis=-1, rounded=N.bf16_round(prod) if epi == "rounded" else None)


@pytest.mark.parametrize("M,Nn,Kk,fused", [(1, 14336, 4096, False), (8, 1536, 2048, True), (17, 520, 1000, False),
                                            (32, 768, 4096, True)])
def test_gemv_mfma_swiglu(gpu, M, Nn, Kk, fused):
    """silu(x @ G) * (x @ U) on the MFMA few-row form: separate gate / up
    weights, or one (K, 2N) weight with the up half N columns in (ldb 2N)."""
    rng = np.random.default_rng(M + Nn + Kk)
    print(f"gemv_mfma swiglu M={M} N={Nn} K={Kk} fused={fused} split={LA.gemv_mfma_split(M, Nn, Kk, True)}",
          flush=True)
    x = N.bf16_round(rng.standard_normal((M, Kk)))
    g = N.bf16_round(rng.standard_normal((Kk, Nn)) * 0.05)
    u = N.bf16_round(rng.standard_normal((Kk, Nn)) * 0.05)
    ref = K.silu(x.astype(np.float64) @ g.astype(np.float64)) * (x.astype(np.float64) @ u.astype(np.float64))
    xd = DeviceTensor.from_numpy(dt.to_bf16(x))
    if fused:
        wd = DeviceTensor.from_numpy(dt.to_bf16(np.concatenate([g, u], axis=1)))
        gp, up, ldb = wd.ptr, wd.ptr + Nn * 2, 2 * Nn
        keep = [wd]
    else:
        gd, ud = DeviceTensor.from_numpy(dt.to_bf16(g)), DeviceTensor.from_numpy(dt.to_bf16(u))
        gp, up, ldb = gd.ptr, ud.ptr, Nn
        keep = [gd, ud]
    h = DeviceTensor.empty((M, Nn), dt.bfloat16)
    ws = DeviceTensor.empty((LA.gemv_mfma_workspace_bytes(M, Nn, Kk, swiglu=True),), dt.uint8)
    launches = LA.gemv_mfma(xd.ptr, gp, h.ptr, M, Nn, Kk, c_dtype=dt.bfloat16, ws_ptr=ws.ptr, ldb=ldb, up_ptr=up)
    assert launches[0].symbol.startswith("nk_gemv_mfma_nn_bf16_swiglu_")
    _run(gpu, launches)
    del keep
    _close(dt.to_float32(h.numpy()), ref, axis=-1)


NT_MFMA_CASES = [  # (fp8, M, N, K): NT weights (bf16 / fp8), row tiles full / partial / two, N and K tails
    (False, 2, 6144, 4096), (False, 13, 1000, 328), (False, 32, 520, 2056), (False, 8, 4096, 14336),
    (True, 4, 6144, 4096), (True, 16, 1000, 336), (True, 17, 264, 4096), (True, 8, 4096, 14336),
]


@pytest.mark.parametrize("fp8,M,Nn,Kk", NT_MFMA_CASES)
@pytest.mark.parametrize("epi", ["plain", "f32", "bias_resid"])
def test_gemv_mfma_nt_matches_float64(gpu, fp8, M, Nn, Kk, epi):
    rng = np.random.default_rng(M * 13 + Nn + Kk)
    print(f"gemv_mfma nt fp8={fp8} M={M} N={Nn} K={Kk} {epi} split={LA.gemv_mfma_split(M, Nn, Kk)}", flush=True)
    x = N.bf16_round(rng.standard_normal((M, Kk)))
    wdev, scale, wmat = _weights(rng, "nt", Nn, Kk, fp8)
    prod = x.astype(np.float64) @ wmat
    out = dt.float32 if epi == "f32" else dt.bfloat16
    t = {"x": DeviceTensor.from_numpy(dt.to_bf16(x)), "w": DeviceTensor.from_numpy(wdev)}
    kw, ref = {}, prod
    if scale is not None:
        t["s"] = DeviceTensor.from_numpy(scale)
        kw["scale_ptr"] = t["s"].ptr
    if epi == "bias_resid":
        bias = N.bf16_round(rng.standard_normal(Nn) * 0.1)
        res = N.bf16_round(rng.standard_normal((M, Nn)))
        t["b"] = DeviceTensor.from_numpy(dt.to_bf16(bias))
        t["r"] = DeviceTensor.from_numpy(dt.to_bf16(res))
        kw.update(bias_ptr=t["b"].ptr, resid_ptr=t["r"].ptr)
        ref = prod + bias + res
    c = DeviceTensor.empty((M, Nn), out)
    ws = DeviceTensor.empty((LA.gemv_mfma_workspace_bytes(M, Nn, Kk),), dt.uint8)
    launches = LA.gemv_mfma(t["x"].ptr, t["w"].ptr, c.ptr, M, Nn, Kk, c_dtype=out, ws_ptr=ws.ptr, layout="nt",
                            b_dtype=dt.float8_e4m3fn if fp8 else dt.bfloat16, **kw)
    assert launches[0].symbol.startswith(f"nk_gemv_mfma_nt_{'e4m3' if fp8 else 'bf16'}_t")
    _run(gpu, launches)
    got = c.numpy() if out == dt.float32 else dt.to_float32(c.numpy())
    if out == dt.float32:
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4 * np.abs(ref).max())
    else:
        _close(got, ref, axis=-1)


@pytest.mark.parametrize("fp8,M,Nn,Kk", [(False, 8, 1536, 2048), (True, 8, 1024, 4096), (True, 32, 520, 1024)])
def test_gemv_mfma_nt_swiglu(gpu, fp8, M, Nn, Kk):
    rng = np.random.default_rng(Nn + Kk + M)
    x = N.bf16_round(rng.standard_normal((M, Kk)))
    wg, sg, mg = _weights(rng, "nt", Nn, Kk, fp8)
    wu, su, mu = _weights(rng, "nt", Nn, Kk, fp8)
    ref = K.silu(x.astype(np.float64) @ mg) * (x.astype(np.float64) @ mu)
    t = [DeviceTensor.from_numpy(v) for v in (dt.to_bf16(x), wg, wu)]
    kw = {}
    if fp8:
        s = [DeviceTensor.from_numpy(v) for v in (sg, su)]
        kw = {"scale_ptr": s[0].ptr, "up_scale_ptr": s[1].ptr}
    h = DeviceTensor.empty((M, Nn), dt.bfloat16)
    ws = DeviceTensor.empty((LA.gemv_mfma_workspace_bytes(M, Nn, Kk, swiglu=True),), dt.uint8)
    launches = LA.gemv_mfma(t[0].ptr, t[1].ptr, h.ptr, M, Nn, Kk, c_dtype=dt.bfloat16, ws_ptr=ws.ptr, layout="nt",
                            b_dtype=dt.float8_e4m3fn if fp8 else dt.bfloat16, up_ptr=t[2].ptr, **kw)
    assert "_swiglu_t" in launches[0].symbol
    _run(gpu, launches)
    _close(dt.to_float32(h.numpy()), ref, axis=-1)


def test_fp8_decode_batch_projection_lowers_to_mfma_nt(gpu):
    """A traced 8-token fp8 projection (x @ dequant(W)^T with per-output
    scales, as the fp8 decoder layer's) takes the MFMA few-row NT form."""
    from nkipy_amd.kernels.decoder import linear_fp8
    from nkipy_amd.runtime import DeviceKernel, baremetal_jit

    def proj(x, w, s):
        return linear_fp8(x, w, s).astype(x.dtype)

    rng = np.random.default_rng(8)
    x = N.bf16_round(rng.standard_normal((8, 1, 4096)))
    wdev, scale, wmat = _weights(rng, "nt", 6144, 4096, True)
    args = [dt.to_bf16(x), wdev, scale]
    dk = DeviceKernel.compile_and_load(proj, *args)
    assert dk.plan.kernel_kinds == ["gemm"]
    assert launch_symbols(dk.plan) == ["nk_gemv_mfma_nt_e4m3_t1", "nk_gemv_out_bf16"]
    got = dt.to_float32(baremetal_jit(proj)(*args))
    _close(got, x.astype(np.float64) @ wmat, axis=-1)


def test_gemv_mfma_against_valu_form(gpu):
    """The same operands through the MFMA and the VALU few-row kernels: fp32
    results within the difference of two summation orders."""
    M, Nn, Kk = 8, 4096, 4096
    rng = np.random.default_rng(6)
    x = N.bf16_round(rng.standard_normal((M, Kk)))
    w = N.bf16_round(rng.standard_normal((Kk, Nn)) * 0.05)
    t = [DeviceTensor.from_numpy(dt.to_bf16(v)) for v in (x, w)]
    c1, c2 = DeviceTensor.empty((M, Nn), dt.float32), DeviceTensor.empty((M, Nn), dt.float32)
    w1 = DeviceTensor.empty((LA.gemv_mfma_workspace_bytes(M, Nn, Kk),), dt.uint8)
    w2 = DeviceTensor.empty((LA.gemv_workspace_bytes(M, Nn, Kk, "nn", False),), dt.uint8)
    _run(gpu, LA.gemv_mfma(t[0].ptr, t[1].ptr, c1.ptr, M, Nn, Kk, c_dtype=dt.float32, ws_ptr=w1.ptr))
    _run(gpu, LA.gemv(t[0].ptr, t[1].ptr, c2.ptr, M, Nn, Kk, layout="nn", b_dtype=dt.bfloat16,
                      c_dtype=dt.float32, ws_ptr=w2.ptr))
    a, b = c1.numpy(), c2.numpy()
    np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-5 * np.abs(b).max())


# ---------------------------------------------------------------------------
# The MFMA GEMM over K ranges (8 < M <= 256: a decode batch)
# ---------------------------------------------------------------------------
SPLITK = [  # (layout, fp8, M, N, K): K ranges of 64-multiples, the last with a tail
    ("nn", False, 32, 6144, 4096), ("nn", False, 200, 264, 520), ("nn", False, 9, 1024, 1000),
    ("nt", False, 16, 1000, 1000), ("nt", False, 64, 4096, 4096), ("nt", True, 64, 4104, 1008),
    ("nt", True, 33, 512, 14336), ("nt", True, 256, 4096, 4096),
]


@pytest.mark.parametrize("layout,fp8,M,Nn,Kk", SPLITK)
@pytest.mark.parametrize("epi", ["plain", "f32", "bias_resid", "rounded"])
def test_gemm_splitk_matches_float64(gpu, layout, fp8, M, Nn, Kk, epi):
    split = LA.gemm_splitk_split(M, Nn, Kk, fp8=fp8)
    print(f"gemm splitk {layout} fp8={fp8} M={M} N={Nn} K={Kk} {epi} split={split}", flush=True)
    rng = np.random.default_rng(M * 3 + Nn + Kk)
    x = N.bf16_round(rng.standard_normal((M, Kk)))
    wdev, scale, wmat = _weights(rng, layout, Nn, Kk, fp8)
    prod = x.astype(np.float64) @ wmat
    bias = N.bf16_round(rng.standard_normal(Nn) * 0.1)
    res = N.bf16_round(rng.standard_normal((M, Nn)))
    out = dt.float32 if epi == "f32" else dt.bfloat16
    kw, ref = {}, prod
    t = {"x": DeviceTensor.from_numpy(dt.to_bf16(x)), "w": DeviceTensor.from_numpy(wdev)}
    if scale is not None:
        t["s"] = DeviceTensor.from_numpy(scale)
        kw["scale_ptr"] = t["s"].ptr
    if epi in ("bias_resid", "rounded"):
        t["b"] = DeviceTensor.from_numpy(dt.to_bf16(bias))
        t["r"] = DeviceTensor.from_numpy(dt.to_bf16(res))
        kw.update(bias_ptr=t["b"].ptr, resid_ptr=t["r"].ptr)
        if epi == "rounded":
            kw.update(round_before_bias=True, round_before_resid=True)
            ref = N.bf16_round(N.bf16_round(prod) + bias) + res
        else:
            ref = prod + bias + res
    c = DeviceTensor.empty((M, Nn), out)
    ws = DeviceTensor.empty((LA.gemm_splitk_workspace_bytes(M, Nn, Kk, fp8=fp8),), dt.uint8)
    _run(gpu, LA.gemm_splitk(t["x"].ptr, t["w"].ptr, c.ptr, M, Nn, Kk, layout=layout,
                             b_dtype=dt.float8_e4m3fn if fp8 else dt.bfloat16, c_dtype=out, ws_ptr=ws.ptr, **kw))
    got = c.numpy() if out == dt.float32 else dt.to_float32(c.numpy())
    if out == dt.float32:
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4 * np.abs(ref).max())
    else:
        _close(got, ref, axis=-1, rounded=N.bf16_round(prod) if epi == "rounded" else None)


@pytest.mark.parametrize("layout,fp8,M,Nn,Kk", [("nn", False, 48, 2048, 4096), ("nt", True, 24, 1024, 2048),
                                                ("nt", False, 130, 300, 712)])
def test_gemm_splitk_swiglu(gpu, layout, fp8, M, Nn, Kk):
    rng = np.random.default_rng(Nn + Kk + M)
    x = N.bf16_round(rng.standard_normal((M, Kk)))
    wg, sg, mg = _weights(rng, layout, Nn, Kk, fp8)
    wu, su, mu = _weights(rng, layout, Nn, Kk, fp8)
    ref = K.silu(x.astype(np.float64) @ mg) * (x.astype(np.float64) @ mu)
    t = [DeviceTensor.from_numpy(v) for v in (dt.to_bf16(x), wg, wu)]
    kw = {}
    if fp8:
        s = [DeviceTensor.from_numpy(v) for v in (sg, su)]
        kw = {"scale_ptr": s[0].ptr, "up_scale_ptr": s[1].ptr}
    h = DeviceTensor.empty((M, Nn), dt.bfloat16)
    ws = DeviceTensor.empty((LA.gemm_splitk_workspace_bytes(M, Nn, Kk, swiglu=True, fp8=fp8),), dt.uint8)
    launches = LA.gemm_splitk(t[0].ptr, t[1].ptr, h.ptr, M, Nn, Kk, layout=layout,
                              b_dtype=dt.float8_e4m3fn if fp8 else dt.bfloat16, c_dtype=dt.bfloat16,
                              ws_ptr=ws.ptr, up_ptr=t[2].ptr, **kw)
    assert len(launches) == 3
    _run(gpu, launches)
    _close(dt.to_float32(h.numpy()), ref, axis=-1)


@pytest.mark.parametrize("layout,fp8", [("nn", False), ("nt", False), ("nt", True)])
def test_gemm_splitk_against_unsplit(gpu, layout, fp8):
    """Same operands through the K ranges and through one K loop: fp32
    results within the difference of the two summation orders."""
    M, Nn, Kk = 40, 3072, 4096
    rng = np.random.default_rng(9)
    x = N.bf16_round(rng.standard_normal((M, Kk)))
    wdev, scale, _ = _weights(rng, layout, Nn, Kk, fp8)
    t = [DeviceTensor.from_numpy(v) for v in (dt.to_bf16(x), wdev)]
    kw = {}
    if fp8:
        sd = DeviceTensor.from_numpy(scale)
        kw["scale_ptr"] = sd.ptr
    bt = dt.float8_e4m3fn if fp8 else dt.bfloat16
    c1, c2 = DeviceTensor.empty((M, Nn), dt.float32), DeviceTensor.empty((M, Nn), dt.float32)
    ws = DeviceTensor.empty((LA.gemm_splitk_workspace_bytes(M, Nn, Kk, fp8=fp8),), dt.uint8)
    assert LA.gemm_splitk_split(M, Nn, Kk, fp8=fp8)[0] > 1
    _run(gpu, LA.gemm_splitk(t[0].ptr, t[1].ptr, c1.ptr, M, Nn, Kk, layout=layout, b_dtype=bt,
                             c_dtype=dt.float32, ws_ptr=ws.ptr, **kw))
    _run(gpu, [LA.gemm(t[0].ptr, t[1].ptr, c2.ptr, M, Nn, Kk, layout=layout, b_dtype=bt, c_dtype=dt.float32,
                       **kw)])
    a, b = c1.numpy(), c2.numpy()
    np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-5 * np.abs(b).max())


@pytest.mark.parametrize("M,symbol", [(32, "nk_gemv_mfma_nn_bf16_t2"), (64, "nk_gemm8k_nn_bf16_f32_splitk")])
def test_decode_batch_projection_lowers_to_splitk(gpu, M, symbol):
    """A traced decode-batch projection (x (M, 1, 4096) @ W (4096, 6144),
    bf16): 32 tokens take the MFMA few-row form, 64 the MFMA GEMM over K
    ranges; both match float64."""
    from nkipy_amd.runtime import DeviceKernel, baremetal_jit

    def proj(x, w):
        return np.matmul(x, w)

    rng = np.random.default_rng(4)
    x = N.bf16_round(rng.standard_normal((M, 1, 4096)))
    w = N.bf16_round(rng.standard_normal((4096, 6144)) * 0.02)
    args = [dt.to_bf16(a) for a in (x, w)]
    dk = DeviceKernel.compile_and_load(proj, *args)
    assert launch_symbols(dk.plan) == [symbol, "nk_gemv_out_bf16"]
    got = dt.to_float32(baremetal_jit(proj)(*args))
    _close(got, x.astype(np.float64) @ w.astype(np.float64), axis=-1)
