"""Top-k and greedy sampling on the GPU against the oracle's NumPy forms
(nkipy/src/nkipy/core/ops/nn.py:22-60; examples/models/qwen3/kernels/
sampling.py:113-148)."""

import numpy as np
import pytest

from nkipy_amd.core import dtypes as dt
from nkipy_amd.core import tensor_apis
from nkipy_amd.runtime import DeviceKernel, baremetal_jit
from oracle import kernels as K
from oracle import numerics as N

pytestmark = pytest.mark.gpu


def _topk_kernel(k, asc):
    def topk_kernel(x):
        return tensor_apis.topk(x, k, axis=-1, is_ascend=asc)

    return topk_kernel


@pytest.mark.parametrize("rows,n,k", [(1, 7, 1), (3, 1000, 1), (4, 1000, 4), (2, 5000, 64), (5, 64, 64)])
@pytest.mark.parametrize("asc", [False, True])
def test_topk_f32(gpu, rows, n, k, asc):
    rng = np.random.default_rng(rows * n + k)
    x = (rng.permuted(np.tile(np.arange(n), (rows, 1)), axis=1) - n / 2).astype(np.float32) * 0.25
    fn = _topk_kernel(k, asc)
    kinds = DeviceKernel.compile_and_load(fn, x).plan.kernel_kinds
    assert kinds[0] == "topk" and kinds[-1] == "gather"
    v, i = baremetal_jit(fn)(x)
    rv, ri = K.topk(x, k, axis=-1, is_ascend=asc)
    assert i.dtype == np.uint32 and v.dtype == np.float32
    np.testing.assert_array_equal(i, ri)
    np.testing.assert_array_equal(v, rv)


def test_topk_bf16_batched_rows(gpu):
    rng = np.random.default_rng(3)
    x = (rng.permuted(np.tile(np.arange(256), (2, 3, 1)), axis=2) - 128).astype(np.float32)  # exact in bf16
    v, i = baremetal_jit(_topk_kernel(5, False))(dt.to_bf16(x))
    rv, ri = K.topk(x, 5, axis=-1)
    np.testing.assert_array_equal(i, ri)
    np.testing.assert_array_equal(dt.to_float32(v), rv)


def test_greedy_sampling(gpu):
    from nkipy_amd.kernels.qwen3 import greedy_sampling

    B, S, H, V = 2, 3, 256, 4000
    rng = np.random.default_rng(5)
    h = N.bf16_round(rng.standard_normal((B, S, H)))
    w = N.bf16_round(rng.uniform(0.5, 1.5, H))
    lm = N.bf16_round(rng.standard_normal((H, V)) * 0.1)

    def sample(h, norm_weight, lm_head_weight):
        return greedy_sampling(h, norm_weight, lm_head_weight, 1e-6)

    got = baremetal_jit(sample)(*[dt.to_bf16(a) for a in (h, w, lm)])
    assert got.shape == (B, 1) and got.dtype == np.uint32
    ref = K.greedy_sampling_bf16(h, w, lm, 1e-6)
    # the pick is a largest bf16 logit (ties between equal bf16 logits would
    # be a legitimate difference; none occur at this seed)
    np.testing.assert_array_equal(got, ref)
