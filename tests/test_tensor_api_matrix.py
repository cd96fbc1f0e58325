"""The tensor-API matrix: NumPy operations traced one kernel at a time.

Case tables in the categories of the reference's tests/unit/
test_tensor_api.py -- unary (:133-171), bitwise (:174-244), comparison
(:246-266), matmul contraction and 1-D promotion (:269-348), reductions
(:351-490), broadcast / copy / transpose / repeat (:493-646), take /
put_along_axis / take_along_axis (:649-864), rotary embedding by index
(:867-903), where (:905-1025), index assignment and extraction
(:1028-1130), topk (:1132-1190) and the math / shape helpers after it
(:1548-3550).  Each case is lowered on the CPU; on the GPU it runs through
``baremetal_jit`` and is compared with the same function run by NumPy
(``parity.assert_matches_numpy``: fp32 1e-4 relative plus 1e-4 of the
output RMS, fp16 1e-2, integers exactly).
"""

import numpy as np
import pytest
from parity import assert_matches_numpy

from nkipy_amd.core import tensor_apis
from nkipy_amd.core.trace import NKIPyKernel
from nkipy_amd.dispatch.lower import lower

R = np.random.default_rng(2024)


def u(*shape, dtype=np.float32):
    return R.random(shape).astype(dtype)


def n(*shape, dtype=np.float32):
    return R.standard_normal(shape).astype(dtype)


def ints(lo, hi, *shape, dtype=np.int32):
    return R.integers(lo, hi, shape).astype(dtype)


CASES = {}


def case(name, fn, *args):
    assert name not in CASES, name
    CASES[name] = (fn, args)


# unary, fp32 (256, 256): inputs in [0, 1) as the reference draws them
for f in (np.abs, np.arctan, np.ceil, np.cos, np.exp, np.floor, np.log, np.negative, np.reciprocal, np.rint,
          np.sqrt, np.sin, np.sign, np.tan, np.tanh, np.trunc, np.square, np.log1p, np.log2, np.expm1):
    case(f"unary_{f.__name__}", lambda a, f=f: f(a), u(256, 256) + 0.01)
case("unary_sign_mixed", np.sign, n(64, 64))
case("round", lambda a: np.round(a * 10), n(32, 32))
case("round_decimals", lambda a: np.round(a, 2), n(32, 32))
for dt_ in (np.int8, np.uint8):
    lo = -100 if dt_ == np.int8 else 0
    x8, y8 = ints(lo, 100, 64, 64, dtype=dt_), ints(lo, 100, 64, 64, dtype=dt_)
    case(f"bitwise_not_{dt_.__name__}", np.bitwise_not, x8)
    case(f"logical_not_{dt_.__name__}", np.logical_not, x8)
    for f in (np.bitwise_and, np.bitwise_xor, np.bitwise_or):
        case(f"{f.__name__}_{dt_.__name__}", lambda a, b, f=f: f(a, b), x8, y8)
case("bitwise_dunders", lambda a, b: ((a & b) | (a ^ b)) + (~a), ints(-50, 50, 16, 16), ints(-50, 50, 16, 16))

# binary, fp32 (256, 256)
for f in (np.add, np.divide, np.maximum, np.minimum, np.multiply, np.subtract, np.power, np.greater_equal,
          np.less, np.logaddexp):
    case(f"binary_{f.__name__}", lambda a, b, f=f: f(a, b), u(256, 256) + 0.01, u(256, 256) + 0.01)
case("remainder", np.remainder, n(32, 32) * 10, u(32, 32) * 3 + 0.5)
case("mod_operator", lambda a, b: a % b, n(32, 32) * 10, u(32, 32) * 3 + 0.5)
case("floor_divide", np.floor_divide, n(32, 32) * 10, u(32, 32) * 3 + 0.5)
case("floor_divide_operator", lambda a, b: a // b, n(32, 32) * 10, u(32, 32) * 3 + 0.5)
case("pred_scalar_promotion", lambda a: (a > 0.5) * 2.0 + (a < 0.25), u(32, 32))
for dt_ in (np.float32, np.float16):
    a_, b_ = u(128, 128, dtype=dt_), u(128, 128, dtype=dt_)
    b_[::3] = a_[::3]  # some equal pairs
    for f in (np.equal, np.not_equal, np.greater, np.less_equal, np.less, np.greater_equal):
        case(f"compare_{f.__name__}_{np.dtype(dt_).name}", lambda a, b, f=f: f(a, b), a_, b_)

# matmul contraction and 1-D promotion
for lhs, rhs in (((64, 128), (128, 64)), ((128, 256), (256, 512)), ((1, 2, 128, 512), (512, 256)),
                 ((128, 512), (1, 2, 512, 256)), ((1, 2, 128, 512), (1, 2, 512, 256)),
                 ((1, 1, 128, 512), (1, 1, 1, 512, 256)), ((64,), (2, 64, 32)), ((2, 32, 64), (64,)),
                 ((64,), (2, 3, 64, 32)), ((2, 3, 32, 64), (64,)), ((64,), (64,))):
    case(f"matmul_{'x'.join(map(str, lhs))}_{'x'.join(map(str, rhs))}", np.matmul, u(*lhs), u(*rhs))
case("dot_2d", np.dot, u(16, 32), u(32, 8))
case("dot_1d", np.dot, u(32), u(32))
case("outer", np.outer, u(16), u(24))
case("matmul_operator_transposed", lambda a, b: a @ b.T, n(24, 40), n(16, 40))

# reductions
for f in (np.mean, np.max, np.min, np.sum):
    case(f"reduce_{f.__name__}_last", lambda a, f=f: f(a, axis=(-1,)), u(128, 128))
    for shp in ((64, 64), (32, 32, 32), (16, 16, 16, 16)):
        case(f"reduce_{f.__name__}_all_{len(shp)}d", lambda a, f=f: f(a), u(*shp))
for shp in ((64, 64), (32, 32, 32)):
    for kd in (True, False):
        case(f"sum_all_keepdims{int(kd)}_{len(shp)}d", lambda a, kd=kd: np.sum(a, axis=None, keepdims=kd), u(*shp))
case("mean_axis1", lambda a: np.mean(a, axis=1), u(64, 64))
case("any_axis0", lambda a: np.any(a > 0.9, axis=0), u(32, 64))
case("sums_of_two_dtypes", lambda a, b: (np.sum(a, axis=1), np.sum(b, axis=1)), u(16, 32), ints(-9, 9, 16, 32))
case("prod", lambda a: np.prod(a, axis=1), u(8, 6) + 0.5)
case("prod_keepdims", lambda a: np.prod(a, axis=0, keepdims=True), u(6, 8) + 0.5)
case("var_axis", lambda a: np.var(a, axis=1), n(16, 32))
case("var_keepdims", lambda a: np.var(a, axis=0, keepdims=True), n(16, 32))
case("std_axis0", lambda a: np.std(a, axis=0), n(16, 32))
case("std_all", lambda a: np.std(a), n(16, 32))
case("argmax", lambda a: np.argmax(a, axis=1), n(16, 32))
case("argmax_axis0", lambda a: np.argmax(a, axis=0), n(16, 32))
case("argmax_all", lambda a: np.argmax(a), n(16, 32))
case("argmax_keepdims", lambda a: np.argmax(a, axis=1, keepdims=True), n(16, 32))
case("argmin", lambda a: np.argmin(a, axis=1), n(16, 32))
case("argmin_all", lambda a: np.argmin(a), n(16, 32))
case("count_nonzero", lambda a: np.count_nonzero(a > 0), n(16, 32))
case("linalg_norm", lambda a: np.linalg.norm(a), n(16, 32))
case("linalg_norm_axis_keepdims", lambda a: np.linalg.norm(a, axis=1, keepdims=True), n(16, 32))
case("cumsum", lambda a: np.cumsum(a, axis=1), n(8, 32))
case("cumsum_axis0", lambda a: np.cumsum(a, axis=0), n(8, 32))
case("cumsum_all", lambda a: np.cumsum(a), n(4, 8))
case("cumsum_middle", lambda a: np.cumsum(a, axis=1), n(3, 8, 5))
case("trace", np.trace, n(12, 12))
case("log_sum_exp", lambda a: np.log(np.sum(np.exp(a), axis=1)), n(16, 32))
case("row_standardize", lambda a: (a - a.mean(axis=1, keepdims=True)) / a.std(axis=1, keepdims=True), n(16, 32))
case("cosine_similarity", lambda a, b: np.sum(a * b, axis=1) / (np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1)),
     n(16, 32), n(16, 32))
case("tensor_methods", lambda a: (a.mean(axis=0), a.sum(axis=1), a.max(axis=1), a.min(axis=0), a.var(axis=1),
                                  a.std(axis=0), a.argmax(axis=1), a.argmin(axis=0)), n(8, 16))

# layout
for src, dst in (((2, 1), (2, 2)), ((1, 2), (2, 2)), ((1, 1, 2), (2, 2, 2)), ((1, 2, 1), (2, 2, 2)),
                 ((2, 1, 1), (2, 2, 2)), ((2, 2, 1), (2, 2, 2)), ((2, 1, 2), (2, 2, 2)), ((1, 2, 2), (2, 2, 2)),
                 ((2, 2), (2, 2, 2)), ((1, 2), (1, 1, 2, 2)), ((1, 2), (2, 2, 2, 2)), ((4, 8), (4, 8))):
    case(f"broadcast_{'x'.join(map(str, src))}_to_{'x'.join(map(str, dst))}",
         lambda a, dst=dst: np.broadcast_to(a, dst), u(*src))
case("copy", np.copy, u(8, 8))
case("copy_method", lambda a: a.copy(), u(8, 8))
for shp, axes in (((2, 3), (1, 0)), ((2, 3), (0, 1)), ((2, 3, 4), (0, 1, 2)), ((2, 3, 4), (0, 2, 1)),
                  ((2, 3, 4), (2, 0, 1)), ((2, 3, 4), (2, 1, 0))):
    case(f"transpose_{'x'.join(map(str, shp))}_{''.join(map(str, axes))}",
         lambda a, axes=axes: np.transpose(a, axes), u(*shp))
case("swapaxes", lambda a: np.swapaxes(a, 0, 2), u(2, 3, 4))
case("swapaxes_method", lambda a: a.swapaxes(1, 2), u(2, 3, 4))
case("ravel_method", lambda a: a.ravel(), u(3, 5))
for shp, rep, ax in (((2, 3), 2, 0), ((2, 3), 2, None), ((2, 3), 3, 1), ((2, 3, 4), 2, None),
                     ((2, 3, 4), 2, 0), ((2, 3, 4), 3, 1), ((2, 3, 4), 4, 2), ((4, 8), 2, -1)):
    case(f"repeat_{'x'.join(map(str, shp))}_{rep}_{ax}", lambda a, rep=rep, ax=ax: np.repeat(a, rep, axis=ax),
         u(*shp))
case("repeat_numpy_int", lambda a: np.repeat(a, np.int64(2), axis=0), u(3, 4))
case("concatenate", lambda a, b: np.concatenate([a, b], axis=0), u(3, 4), u(5, 4))
case("concatenate_single", lambda a: np.concatenate([a], axis=1), u(3, 4))
case("concatenate_negative_axis", lambda a, b: np.concatenate([a, b], axis=-1), u(3, 4), u(3, 2))
case("split_equal", lambda a: tuple(np.split(a, 2, axis=1)), u(4, 8))
case("split_indices", lambda a: tuple(np.split(a, [1, 5], axis=0)), u(8, 3))
case("split_negative_axis", lambda a: tuple(np.split(a, 4, axis=-1)), u(2, 8))
case("reshape_infer", lambda a: np.reshape(a, (-1, 6)), u(4, 3, 2))
case("squeeze", lambda a: np.squeeze(a, axis=1), u(4, 1, 3))
case("squeeze_all", lambda a: np.squeeze(a), u(1, 4, 1, 3))
case("squeeze_method", lambda a: a.squeeze(0), u(1, 4, 3))
case("stack", lambda a, b: np.stack([a, b]), u(3, 4), u(3, 4))
case("stack_axis", lambda a, b: np.stack([a, b], axis=-1), u(3, 4), u(3, 4))
case("expand_dims_list", lambda a: np.expand_dims(a, [0, 2]), u(3, 4))
case("expand_dims_negative", lambda a: np.expand_dims(a, -1), u(3, 4))
case("flip", lambda a: np.flip(a, axis=1), u(4, 6))
case("flip_axis0", lambda a: np.flip(a, axis=0), u(4, 6))
case("tile", lambda a: np.tile(a, 3), u(2, 3))
case("tile_multi", lambda a: np.tile(a, (2, 2)), u(2, 3))
case("roll", lambda a: np.roll(a, 2, axis=1), u(3, 7))
case("roll_axis0", lambda a: np.roll(a, -1, axis=0), u(5, 3))
case("diff", lambda a: np.diff(a, axis=1), u(4, 7))
case("diff_n2", lambda a: np.diff(a, n=2, axis=0), u(6, 3))
case("pad_constant", lambda a: np.pad(a, 2), u(4, 5))
case("pad_asymmetric", lambda a: np.pad(a, ((1, 0), (0, 3))), u(4, 5))
case("pad_edge", lambda a: np.pad(a, 1, mode="edge"), u(4, 5))
case("pad_edge_asymmetric", lambda a: np.pad(a, ((0, 2), (1, 0)), mode="edge"), u(4, 5))
case("tril", np.tril, u(6, 6))
case("triu", np.triu, u(6, 6))
case("tril_k", lambda a: np.tril(a, k=-1), u(6, 6))
case("diagonal_gather", lambda a: a[np.arange(6), np.arange(6)], u(6, 6))
case("clip", lambda a: np.clip(a, 0.2, 0.7), u(16, 16))
case("clip_no_min", lambda a: np.clip(a, None, 0.5), u(16, 16))
case("clip_no_max", lambda a: np.clip(a, 0.5, None), u(16, 16))
case("clip_method", lambda a: a.clip(0.1, 0.3), u(16, 16))
case("hard_sigmoid", lambda a: np.clip(a / 6 + 0.5, 0, 1), n(16, 16) * 4)
case("softplus", lambda a: np.log1p(np.exp(a)), n(16, 16))
case("isnan_isfinite", lambda a: (np.isnan(a), np.isfinite(a)), n(8, 8))
case("passthrough", lambda a: a, u(4, 4))
case("passthrough_with_compute", lambda a, b: (a, a + b), u(4, 4), u(4, 4))
case("zeros_full_standalone", lambda a: a + np.zeros((4, 4), np.float32) + np.full((4, 4), 2.5, np.float32), u(4, 4))
case("like_functions", lambda a: (np.zeros_like(a), np.ones_like(a), np.full_like(a, 3.0),
                                  np.zeros_like(a, dtype=np.int32), np.full_like(a, 7, dtype=np.int32)), u(4, 4))
case("weighted_average", lambda a, w: (a * w).sum(axis=1) / w.sum(), u(8, 16), u(16))

# take / put_along_axis / take_along_axis
for shp, idx, ax in (((2, 3), [0, 1], None), ((2, 3), [[0, 1]], None), ((2, 3), [[0, 1], [1, 0]], None),
                     ((2, 3), [0, 1], 0), ((2, 3), [[0, 1]], 1), ((2, 3), [[0, 1], [1, 0]], 0),
                     ((2, 3), [[0, 1], [1, 0]], 1), ((2, 3, 4), [0, 1], 0), ((2, 3, 4), [[0, 1]], 1),
                     ((2, 3, 4), [[0, 1], [1, 0]], 0), ((2, 3, 4), [[0, 1], [1, 0]], 1),
                     ((2, 3, 4), [[0, 1], [1, 0]], 2)):
    tag = f"{'x'.join(map(str, shp))}_idx{'x'.join(map(str, np.asarray(idx).shape))}_{ax}"
    case(f"take_tensor_idx_{tag}", lambda a, i, ax=ax: np.take(a, i, axis=ax), u(*shp),
         np.asarray(idx, np.uint32))
    case(f"take_const_idx_{tag}", lambda a, idx=idx, ax=ax: np.take(a, np.asarray(idx, np.uint32), axis=ax), u(*shp))
for k in (0, 1, -1):
    case(f"take_scalar_{k}", lambda a, k=k: np.take(a, k), u(2, 3))
for shp, idx, val, ax in (((2, 3), [[1, 0, 0]], [[4, 5, 6]], 0), ((2, 3), [[1], [0]], [[4], [5]], 1),
                          ((2, 3), [1, 0], [4, 5], None)):
    def put(a, i, v, ax=ax):
        b = np.copy(a)
        np.put_along_axis(b, i, v, axis=ax)
        return b
    tag = f"{np.asarray(idx).shape}_{ax}".replace(" ", "")
    case(f"put_along_axis_{tag}", put, u(*shp), np.asarray(idx, np.uint32), np.asarray(val, np.float32))

    def put_scalar(a, i, ax=ax, s=float(np.asarray(val).flat[0])):
        b = np.copy(a)
        np.put_along_axis(b, i, s, axis=ax)
        return b
    case(f"put_along_axis_scalar_{tag}", put_scalar, u(*shp), np.asarray(idx, np.uint32))
    case(f"take_along_axis_{tag}", lambda a, i, ax=ax: np.take_along_axis(a, i, axis=ax), u(*shp),
         np.asarray(idx, np.uint32))
case("take_along_axis_rows", lambda a, i: np.take_along_axis(a, i, axis=0), u(2048, 64),
     ints(0, 2048, 128, 1, dtype=np.uint32))
case("take_along_axis_flat", lambda a, i: np.take_along_axis(a, i, axis=None), u(10, 20, 30),
     ints(0, 6000, 50, dtype=np.uint32))


def _rotary_by_index(x, cos_idx, sin_idx, fc, fs):
    x0 = np.take(x, cos_idx, axis=x.ndim - 1)
    x1 = np.take(x, sin_idx, axis=x.ndim - 1)
    out = np.empty_like(x)
    out[:, :, :, cos_idx] = x0 * fc - x1 * fs
    out[:, :, :, sin_idx] = x0 * fs + x1 * fc
    return out


for B, L, HD, H in ((1, 1, 2, 1), (2, 3, 10, 4)):
    case(f"rotary_interleaved_{B}_{L}_{HD}_{H}", _rotary_by_index, u(B, L, H, HD),
         np.arange(0, HD, 2, dtype=np.int32), np.arange(1, HD, 2, dtype=np.int32),
         u(B, L, 1, HD // 2), u(B, L, 1, HD // 2))

# where
for shp in ((64, 64), (256, 256), (128, 512), (1, 2, 128, 256), (2, 3, 4)):
    case(f"where_{'x'.join(map(str, shp))}", np.where, ints(0, 2, *shp, dtype=np.uint8), u(*shp), u(*shp))
for shp in ((64, 64), (2, 3, 4), (10, 64, 512)):
    cond = ints(0, 2, shp[0], dtype=np.uint8).reshape((shp[0],) + (1,) * (len(shp) - 1))
    case(f"where_first_dim_{'x'.join(map(str, shp))}", np.where, cond, u(*shp), u(*shp))
for shp in ((2, 3), (2, 3, 4, 5)):
    fixed = R.integers(0, 2, shp[0]).astype(bool)
    case(f"where_const_cond_{'x'.join(map(str, shp))}",
         lambda a, b, c=fixed, k=len(shp): np.where(np.expand_dims(c, tuple(range(1, k))), a, b), u(*shp), u(*shp))
case("where_scalar_y", lambda c, a: np.where(c, a, 0.0), ints(0, 2, 4, 4, dtype=np.uint8), u(4, 4))
case("where_scalar_x", lambda c, a: np.where(c, 1.0, a), ints(0, 2, 4, 4, dtype=np.uint8), u(4, 4))


# index assignment / extraction along a middle axis
def _assign(a, b, t):
    a[:, t, :] = b
    return a


for shp, k in (((5, 10, 15), 3), ((10, 20, 30), 5), ((15, 25, 35), 7)):
    t = R.choice(shp[1], size=k, replace=False).astype(np.int32)
    case(f"index_assign_{shp[1]}_{k}", _assign, u(*shp), u(shp[0], k, shp[2]), t)
    case(f"index_extract_{shp[1]}_{k}", lambda a, t: a[:, t, :], u(*shp), ints(0, shp[1], k))

# topk (values and indices; ties are absent in continuous random data)
for shp, k, ax in (((5,), 1, 0), ((10,), 2, 0), ((15,), 3, 0), ((5, 10), 1, 1), ((10, 20), 2, 1), ((15, 25), 3, 1)):
    case(f"topk_{'x'.join(map(str, shp))}_{k}", lambda a, k=k, ax=ax: tensor_apis.topk(a, k=k, axis=ax), u(*shp))
for shp, k in (((10,), 3), ((5, 10), 2)):
    case(f"topk_ascending_{'x'.join(map(str, shp))}_{k}",
         lambda a, k=k: tensor_apis.topk(a, k=k, axis=-1, is_ascend=True), u(*shp))


@pytest.mark.parametrize("name", sorted(CASES))
def test_case_lowers(name):
    fn, args = CASES[name]
    plan = lower(NKIPyKernel.trace(fn).specialize(*args))
    assert plan is not None


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(CASES))
def test_case_on_gpu(gpu, name):
    from nkipy_amd.runtime import baremetal_jit

    fn, args = CASES[name]
    expected = fn(*[np.copy(a) for a in args])
    got = baremetal_jit(fn)(*[np.copy(a) for a in args])
    assert_matches_numpy(got, expected, name)
