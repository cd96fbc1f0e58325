"""GPU parity of the fused row kernels (K1a softmax, K1b residual RMSNorm)
against the oracle, through the traced entry points."""

import json
import os

import numpy as np
import pytest
from parity import ulp_bf16

from nkipy_amd.core import dtypes as dt
from nkipy_amd.kernels import residual_rmsnorm_kernel, rmsnorm_kernel, softmax_kernel, softmax_upcast_kernel
from nkipy_amd.runtime import DeviceKernel, DeviceTensor, baremetal_jit
from oracle import kernels as K
from oracle import numerics as N

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _rel(y, ref):
    return float(np.max(np.abs(y.astype(np.float64) - ref) / np.maximum(np.abs(ref), 1e-30)))


def _kinds(fn, *args):
    return DeviceKernel.compile_and_load(fn, *args).plan.kernel_kinds


def test_softmax_config_parity(gpu):
    """Config: x fp32 (2048, 4096) ~ N(0,1)*4, rel-err <= 1e-5 vs NumPy."""
    rng = np.random.default_rng(42)
    x = (rng.standard_normal((2048, 4096)) * 4).astype(np.float32)
    assert _kinds(softmax_kernel, x) == ["softmax"]
    y = baremetal_jit(softmax_kernel)(x)
    ref = K.softmax_kernel(x)
    assert y.dtype == np.float32 and y.shape == x.shape
    assert _rel(y, ref) <= 1e-5
    assert _rel(y, K.softmax_f64(x)) <= 1e-5


def test_softmax_notebook_golden(gpu):
    data = json.load(open(os.path.join(GOLDEN, "softmax_notebooks.json")))
    for case in data["cases"]:
        x = np.array(case["input"], np.float32)
        y = baremetal_jit(softmax_kernel)(x)
        np.testing.assert_allclose(y, case["output"], rtol=0, atol=1e-6)


# (3, 3000), (2, 4088), (6, 1000): rows that end inside the last chunk of a
# register variant (loads past the end read zeros, stores are dropped)
@pytest.mark.parametrize("shape", [(1, 1), (3, 100), (7, 128), (5, 8192), (2, 20000), (2, 3, 64), (4, 2),
                                   (3, 3000), (2, 4088), (6, 1000)])
def test_softmax_ragged_shapes(gpu, shape):
    rng = np.random.default_rng(sum(shape))
    x = (rng.standard_normal(shape) * 4).astype(np.float32)
    y = baremetal_jit(softmax_kernel)(x)
    assert _rel(y, K.softmax_f64(x)) <= 1e-5


def test_softmax_extreme_values(gpu):
    x = np.array([[1e30, 0.0, -1e30, 5.0], [-50.0, -50.0, -50.0, -50.0]], np.float32)
    x = np.tile(x, (1, 2))
    y = baremetal_jit(softmax_kernel)(x)
    np.testing.assert_allclose(y, K.softmax_f64(x), rtol=1e-6, atol=1e-30)


def test_softmax_bf16_upcast(gpu):
    rng = np.random.default_rng(3)
    xf = N.bf16_round(rng.standard_normal((64, 1024)) * 3)
    y = baremetal_jit(softmax_upcast_kernel)(dt.to_bf16(xf))
    assert y.dtype == dt.bfloat16
    ref = N.bf16_round(K.softmax_kernel(xf))
    np.testing.assert_allclose(dt.to_float32(y), ref, rtol=2e-2, atol=1e-6)
    assert _kinds(softmax_upcast_kernel, dt.to_bf16(xf)) == ["softmax"]


@pytest.mark.parametrize("shape", [(64, 1024), (2048, 4096), (5, 8192), (3, 100), (33, 4088)])
def test_softmax_bf16_steps(gpu, shape):
    """softmax_kernel on bf16 x runs each step in bf16 (x - max, exp, sum,
    divide): the kernel rounds the same steps, so the output equals the
    op-by-op oracle except where an fp32 exp or sum lands on the other side
    of a bf16 rounding boundary (one step at most)."""
    rng = np.random.default_rng(shape[1])
    xf = N.bf16_round(rng.standard_normal(shape) * 4)
    kinds = DeviceKernel.compile_and_load(softmax_kernel, dt.to_bf16(xf)).plan.kernel_kinds
    assert kinds == ["softmax"]
    y = dt.to_float32(baremetal_jit(softmax_kernel)(dt.to_bf16(xf)))
    ref = K.softmax_steps_rounded(xf)
    d = np.abs(y - ref)
    same = float(np.mean(d == 0))
    print(f"softmax bf16 steps {shape}: identical {same:.6f}, max {np.max(d / ulp_bf16(ref)):.2f} ulp", flush=True)
    assert same >= 0.999
    assert np.all(d <= ulp_bf16(ref))


def _bf16_inputs(shape, seed=42):
    rng = np.random.default_rng(seed)
    x = N.bf16_round(rng.standard_normal(shape))
    r = N.bf16_round(rng.standard_normal(shape))
    w = N.bf16_round(rng.uniform(0.5, 1.5, shape[-1]))
    return x, r, w


def test_residual_rmsnorm_config_parity(gpu):
    """Config: x, r bf16 (8192, 4096); w bf16 ~ U(0.5, 1.5); eps 1e-6; rtol 2e-2."""
    x, r, w = _bf16_inputs((8192, 4096))
    args = (dt.to_bf16(x), dt.to_bf16(r), dt.to_bf16(w), 1e-6)
    assert _kinds(residual_rmsnorm_kernel, *args) == ["rmsnorm"]
    y = dt.to_float32(baremetal_jit(residual_rmsnorm_kernel)(*args))
    ref = K.residual_rmsnorm_bf16(x, r, w, 1e-6)
    np.testing.assert_allclose(y, ref, rtol=2e-2, atol=0)
    # same cast points: almost every element is bit-identical
    assert np.mean(y == ref) > 0.99


@pytest.mark.parametrize("shape", [(1, 8), (3, 40), (5, 4096), (2, 3, 96), (4, 9000), (2, 13), (3, 3000), (2, 1000)])
def test_rmsnorm_shapes_f32(gpu, shape):
    rng = np.random.default_rng(len(shape))
    x = rng.standard_normal(shape).astype(np.float32)
    w = rng.uniform(0.5, 1.5, shape[-1]).astype(np.float32)
    y = baremetal_jit(rmsnorm_kernel)(x, w, 1e-6)
    ref = K.rmsnorm_f64(x, w, 1e-6)
    assert _rel(y, ref) <= 1e-5
    assert _kinds(rmsnorm_kernel, x, w, 1e-6) == ["rmsnorm"]


def test_rmsnorm_llama_reciprocal_form(gpu):
    """tests/kernels/llama_decoder_dynamo.py:95-107: sum(pow(x,2))/N, 1/sqrt, w * (x * rsqrt)."""

    def llama_norm(x, w):
        pow_1 = np.power(x, 2)
        s = np.sum(pow_1, axis=(-1,), keepdims=True)
        mean = np.divide(s, pow_1.shape[-1])
        add = np.add(mean, 1e-05)
        rsqrt = np.divide(1, np.sqrt(add))
        return np.multiply(w, np.multiply(x, rsqrt))

    rng = np.random.default_rng(11)
    x = rng.standard_normal((1, 7, 2048)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 2048).astype(np.float32)
    assert _kinds(llama_norm, x, w) == ["rmsnorm"]
    y = baremetal_jit(llama_norm)(x, w)
    assert _rel(y, K.rmsnorm_f64(x, w, 1e-5)) <= 1e-5


@pytest.mark.parametrize("shape", [(5, 1000), (3, 3000), (2, 4088)])
def test_residual_rmsnorm_partial_chunks(gpu, shape):
    """Rows ending inside a register variant's last chunk (bf16, residual)."""
    x, r, w = _bf16_inputs(shape, seed=shape[1])
    args = (dt.to_bf16(x), dt.to_bf16(r), dt.to_bf16(w), 1e-6)
    y = dt.to_float32(baremetal_jit(residual_rmsnorm_kernel)(*args))
    np.testing.assert_allclose(y, K.residual_rmsnorm_bf16(x, r, w, 1e-6), rtol=2e-2, atol=0)


def test_residual_rmsnorm_with_residual_output(gpu):
    """The residual sum escapes (it is also returned): the kernel writes it too."""

    def kern(x, r, w):
        h = x + r
        return h, rmsnorm_kernel(h, w, 1e-6)

    x, r, w = _bf16_inputs((64, 512), seed=9)
    args = (dt.to_bf16(x), dt.to_bf16(r), dt.to_bf16(w))
    assert _kinds(kern, *args) == ["rmsnorm"]
    h, y = baremetal_jit(kern)(*args)
    np.testing.assert_array_equal(dt.to_float32(h), N.bf16_round(x + r))
    np.testing.assert_allclose(dt.to_float32(y), K.residual_rmsnorm_bf16(x, r, w, 1e-6), rtol=2e-2)


def test_device_kernel_reuse_and_benchmark(gpu):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((256, 1024)) * 4).astype(np.float32)
    k = DeviceKernel.compile_and_load(softmax_kernel, x, name="softmax_reuse")
    xin = DeviceTensor.from_numpy(x, name="x")
    out = k(inputs={"x": xin})
    np.testing.assert_allclose(out["output0"].numpy(), K.softmax_kernel(x), rtol=1e-5, atol=1e-9)
    res = k.benchmark(inputs={"x": xin}, outputs=out, warmup_iter=2, benchmark_iter=5)
    assert res.iterations == 5 and res.mean_ms > 0
    res_h = k.benchmark(inputs={"x": xin}, outputs=out, warmup_iter=1, benchmark_iter=3, mode="host")
    assert res_h.iterations == 3
