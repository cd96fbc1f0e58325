"""Conformance of the generic lowering: small NumPy kernels run on the GPU
and compared with the same function run directly by NumPy (the two-mode
idiom of the reference's tests, tests/unit/test_tensor_api.py:30-48)."""

import numpy as np
import pytest

from nkipy_amd.runtime import baremetal_jit

pytestmark = pytest.mark.gpu

R = np.random.default_rng(42)
A = R.standard_normal((6, 8)).astype(np.float32)
B = R.standard_normal((6, 8)).astype(np.float32)
V = R.standard_normal((8,)).astype(np.float32)
M = R.standard_normal((8, 5)).astype(np.float32)
T3 = R.standard_normal((2, 6, 8)).astype(np.float32)
I = R.integers(-20, 20, (6, 8)).astype(np.int32)
IDX = np.array([3, 0, 5, 1], np.int32)

CASES = {
    "add_broadcast": (lambda a, v: a + v, (A, V)),
    "sub_scalar": (lambda a: 3.0 - a, (A,)),
    "mul_div": (lambda a, b: a * b / (np.abs(b) + 1.0), (A, B)),
    "exp_log_sqrt": (lambda a: np.log(np.exp(a) + 1.0) + np.sqrt(np.abs(a)), (A,)),
    "tanh_sin_cos": (lambda a: np.tanh(a) + np.sin(a) * np.cos(a), (A,)),
    "max_min_clip": (lambda a, b: np.clip(np.maximum(a, b) - np.minimum(a, b), -0.5, 0.5), (A, B)),
    "where_compare": (lambda a, b: np.where(a > b, a, b * 2.0), (A, B)),
    "power_square": (lambda a: np.power(a, 2) + np.square(a), (A,)),
    "reciprocal_neg": (lambda a: np.reciprocal(np.abs(a) + 1.0) - a, (A,)),
    "floor_ceil_round": (lambda a: np.floor(a * 3) + np.ceil(a) + np.round(a * 2), (A,)),
    "sum_axis0": (lambda a: np.sum(a, axis=0), (A,)),
    "sum_all": (lambda a: np.sum(a), (A,)),
    "max_keepdims": (lambda a: np.max(a, axis=-1, keepdims=True), (A,)),
    "mean_var_std": (lambda a: np.mean(a, axis=1) + np.var(a, axis=1) + np.std(a, axis=1), (A,)),
    "min_prod": (lambda a: np.min(a, axis=1) * np.prod(a[:, :3], axis=1), (A,)),
    "argmax_argmin": (lambda a: (np.argmax(a, axis=1), np.argmin(a, axis=0)), (A,)),
    "matmul": (lambda a, m: a @ m, (A, M)),
    "matmul_batched": (lambda t, m: t @ m, (T3, M)),
    "matmul_transposed": (lambda a, b: a @ b.T, (A, B)),
    "transpose_3d": (lambda t: np.transpose(t, (2, 0, 1)) * 1.0, (T3,)),
    "reshape_chain": (lambda t: (t.reshape(12, 8) + 1.0).reshape(2, 48), (T3,)),
    "concat_split": (lambda a, b: np.split(np.concatenate([a, b], axis=1), 4, axis=1)[2] * 2.0, (A, B)),
    "stack": (lambda a, b: np.stack([a, b], axis=0) + 0.0, (A, B)),
    "slice_step": (lambda a: a[1:5:2, ::3] + 1.0, (A,)),
    "expand_squeeze": (lambda a: np.squeeze(np.expand_dims(a, 1), 1) * 2.0, (A,)),
    "broadcast_to": (lambda v: np.broadcast_to(v, (3, 8)) + 0.0, (V,)),
    "repeat_tile": (lambda a: np.repeat(a, 2, axis=0) + np.tile(a, (2, 1)), (A,)),
    "flip_roll": (lambda a: np.flip(a, axis=1) + np.roll(a, 2, axis=1), (A,)),
    "pad": (lambda a: np.pad(a, ((1, 2), (0, 3))), (A,)),
    "diff_cumsum": (lambda a: np.cumsum(np.diff(a, axis=1), axis=1), (A,)),
    "take": (lambda a, i: np.take(a, i, axis=0) * 1.0, (A, IDX)),
    "take_along_axis": (lambda a: np.take_along_axis(a, np.argsort(np.arange(48).reshape(6, 8) % 5, axis=1).astype(np.int32), axis=1) + 0.0, (A,)),
    "int_ops": (lambda i: (i // 3) + (i % 7) + np.abs(i), (I,)),
    "astype_roundtrip": (lambda a: (a * 10).astype(np.int32).astype(np.float32), (A,)),
    "tril_triu": (lambda a: np.tril(a) - np.triu(a, 1), (A,)),
    "logical": (lambda a, b: np.where(np.logical_and(a > 0, np.logical_not(b > 0)), 1.0, 0.0), (A, B)),
    "norm_outer": (lambda v: np.outer(v, v) / np.linalg.norm(v), (V,)),
    "any_count": (lambda a: np.sum(np.any(a > 1.0, axis=1)) + np.count_nonzero(a > 0), (A,)),
    "getitem_int_and_newaxis": (lambda t: t[1, :, None, 2] * 1.0, (T3,)),
    "passthrough_param": (lambda a: a, (A,)),
    "zeros_like_fill": (lambda a: np.zeros_like(a) + np.full_like(a, 2.0), (A,)),
}


def _cmp(got, exp):
    if isinstance(exp, tuple):
        assert isinstance(got, tuple) and len(got) == len(exp)
        for g, e in zip(got, exp):
            _cmp(g, e)
        return
    exp = np.asarray(exp)
    got = np.asarray(got)
    assert got.shape == exp.shape, (got.shape, exp.shape)
    if np.issubdtype(exp.dtype, np.floating):
        np.testing.assert_allclose(got, exp, rtol=2e-5, atol=2e-5)
    else:
        np.testing.assert_array_equal(got.astype(np.int64), exp.astype(np.int64))


@pytest.mark.parametrize("name", sorted(CASES))
def test_generic_case(gpu, name):
    fn, args = CASES[name]
    expected = fn(*args)
    got = baremetal_jit(fn)(*args)
    _cmp(got, expected)


def test_setitem_alias_writeback(gpu):
    """A mutated input is written back into the caller's array and the kernel
    returns only what it returns (reference: tests/unit/test_alias.py)."""

    def kern(cache, upd):
        cache[1:3, 2:6] = upd
        return cache * 2.0

    cache = np.arange(48, dtype=np.float32).reshape(6, 8)
    upd = -np.ones((2, 4), np.float32)
    exp_cache = cache.copy()
    exp_cache[1:3, 2:6] = upd
    out = baremetal_jit(kern)(cache, upd)
    np.testing.assert_array_equal(out, exp_cache * 2.0)
    np.testing.assert_array_equal(cache, exp_cache)


def test_setitem_mutation_only_kernel_returns_none(gpu):
    def kern(cache, upd):
        cache[:, 0] = upd

    cache = np.zeros((4, 3), np.float32)
    upd = np.arange(4, dtype=np.float32)
    assert baremetal_jit(kern)(cache, upd) is None
    np.testing.assert_array_equal(cache[:, 0], upd)


def test_dynamic_index_setitem(gpu):
    def kern(cache, pos, row):
        cache[pos] = row
        return cache + 0.0

    cache = np.zeros((5, 4), np.float32)
    pos = np.array([3], np.int32)
    row = np.ones((1, 4), np.float32) * 7
    out = baremetal_jit(kern)(cache, pos, row)
    exp = np.zeros((5, 4), np.float32)
    exp[3] = 7
    np.testing.assert_array_equal(out, exp)


def test_alias_deferred_reader_sees_old_contents(gpu):
    """A fused read of a mutated input that precedes the update must see the
    old contents, also when the fused chain is evaluated after the update."""

    def kern(cache, new):
        old = cache * 2.0
        cache[0:1] = new
        return old + 1.0

    cache = np.arange(32, dtype=np.float32).reshape(4, 8)
    new = -np.ones((1, 8), np.float32)
    exp_cache = cache.copy()
    exp_out = kern(exp_cache, new)
    out = baremetal_jit(kern)(cache, new)
    np.testing.assert_array_equal(out, exp_out)
    np.testing.assert_array_equal(cache, exp_cache)


def test_alias_overlapping_self_update(gpu):
    def kern(cache):
        cache[1:3] = cache[0:2]
        return cache + 0.0

    cache = np.arange(32, dtype=np.float32).reshape(4, 8)
    exp_cache = cache.copy()
    exp_out = kern(exp_cache)
    out = baremetal_jit(kern)(cache)
    np.testing.assert_array_equal(out, exp_out)
    np.testing.assert_array_equal(cache, exp_cache)
