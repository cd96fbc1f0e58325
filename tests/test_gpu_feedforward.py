"""GPU parity of the traced SwiGLU feed-forward kernels (fused MFMA GEMMs)
against the oracle's fp32 NumPy formula.

Tolerance for bf16 outputs: |got - ref| <= 2e-2 * (|ref| + rms(ref)), i.e.
rtol 2e-2 with an absolute floor of 2e-2 of the output's RMS (dot products
near zero have no meaningful relative error)."""

import os

import numpy as np
import pytest
from parity import assert_close, launch_symbols

from nkipy_amd.core import dtypes as dt
from nkipy_amd.kernels import feedforward_kernel, linear_nt_kernel, swiglu_mlp_kernel
from nkipy_amd.runtime import DeviceKernel, DeviceTensor, baremetal_jit
from oracle import kernels as K
from oracle import numerics as N

pytestmark = pytest.mark.gpu


def _close(got, ref, tol=2e-2, axis=None):
    """bf16 bar of tests/parity.py (rtol 2e-2, atol min(1e-2, 2e-2 RMS))."""
    name = os.environ.get("PYTEST_CURRENT_TEST", "?").split(" ")[0]
    assert_close(got, ref, name, rtol=tol, axis=axis)


def _inputs(M, H, F, seed=42):
    rng = np.random.default_rng(seed)
    x = N.bf16_round(rng.standard_normal((M, H)))
    wg = N.bf16_round(rng.standard_normal((H, F)) * 0.02)
    wu = N.bf16_round(rng.standard_normal((H, F)) * 0.02)
    wd = N.bf16_round(rng.standard_normal((F, H)) * 0.02)
    return x, wg, wu, wd


def test_swiglu_mlp_small(gpu):
    x, wg, wu, wd = _inputs(512, 1024, 2048)
    args = [dt.to_bf16(a) for a in (x, wg, wu, wd)]
    kinds = DeviceKernel.compile_and_load(swiglu_mlp_kernel, *args).plan.kernel_kinds
    assert kinds == ["gemm_swiglu", "gemm"]
    y = dt.to_float32(baremetal_jit(swiglu_mlp_kernel)(*args))
    _close(y, K.swiglu_mlp(x, wg, wu, wd, round_h=N.bf16_round))


def test_feedforward_fused_gate_up(gpu):
    x, wg, wu, wd = _inputs(256, 512, 1536, seed=3)
    x3 = x.reshape(2, 128, 512)
    gu = np.concatenate([wg, wu], axis=1)
    args = [dt.to_bf16(a) for a in (x3, gu, wd)]
    assert DeviceKernel.compile_and_load(feedforward_kernel, *args).plan.kernel_kinds == ["gemm_swiglu", "gemm"]
    y = dt.to_float32(baremetal_jit(feedforward_kernel)(*args))
    _close(y, K.feedforward_fused(x3, gu, wd, round_h=N.bf16_round))


@pytest.mark.parametrize("fused", [False, True])
def test_decode_batch_mlp_on_few_row_kernels(gpu, fused):
    """A decode batch (8 tokens) through the traced SwiGLU MLP, separate or
    fused gate / up weights: both GEMMs take the MFMA few-row kernels (the
    gate / up pair in its SwiGLU form) and match the oracle."""
    x, wg, wu, wd = _inputs(8, 2048, 1536, seed=9)
    if fused:
        x3 = x.reshape(8, 1, 2048)
        args = [dt.to_bf16(a) for a in (x3, np.concatenate([wg, wu], axis=1), wd)]
        fn, ref = feedforward_kernel, K.feedforward_fused(x3, np.concatenate([wg, wu], axis=1), wd,
                                                          round_h=N.bf16_round)
    else:
        args = [dt.to_bf16(a) for a in (x, wg, wu, wd)]
        fn, ref = swiglu_mlp_kernel, K.swiglu_mlp(x, wg, wu, wd, round_h=N.bf16_round)
    dk = DeviceKernel.compile_and_load(fn, *args)
    assert dk.plan.kernel_kinds == ["gemm_swiglu", "gemm"]
    assert launch_symbols(dk.plan) == ["nk_gemv_mfma_nn_bf16_swiglu_t1", "nk_gemv_out_bf16_swiglu",
                                       "nk_gemv_mfma_nn_bf16_t1", "nk_gemv_out_bf16"]
    y = dt.to_float32(baremetal_jit(fn)(*args))
    _close(y, ref, axis=-1)


def test_linear_nt(gpu):
    rng = np.random.default_rng(5)
    x = N.bf16_round(rng.standard_normal((7, 1, 2048)))
    w = N.bf16_round(rng.standard_normal((8192, 2048)) * 0.02)
    y = dt.to_float32(baremetal_jit(linear_nt_kernel)(dt.to_bf16(x), dt.to_bf16(w)))
    _close(y, x @ w.T)


def test_swiglu_mlp_config_all_rows(gpu):
    """Config: x (4096, 4096), W_gate / W_up (4096, 14336), W_down (14336, 4096).
    Every row is checked against the oracle."""
    M, H, F = 4096, 4096, 14336
    x, wg, wu, wd = _inputs(M, H, F)
    args = [dt.to_bf16(a) for a in (x, wg, wu, wd)]
    k = DeviceKernel.compile_and_load(swiglu_mlp_kernel, *args, name="swiglu_cfg")
    assert k.plan.kernel_kinds == ["gemm_swiglu", "gemm"]
    ins = {n: DeviceTensor.from_numpy(a, name=n) for n, a in zip(("x", "w_gate", "w_up", "w_down"), args)}
    out = k(ins)["output0"].numpy()
    _close(dt.to_float32(out), K.swiglu_mlp(x, wg, wu, wd, round_h=N.bf16_round))
