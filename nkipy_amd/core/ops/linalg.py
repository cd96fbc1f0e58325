"""Linear algebra: matmul, dot, outer, trace, norm.

``matmul`` follows NumPy's rules (1-D promotion, broadcast batch
dimensions) and records one ``dot`` node with dot_general dimension numbers
and fp32 accumulation for floating inputs, like the reference
(nkipy/src/nkipy/core/ops/linalg.py:16-126).  A rank-2 right operand is
contracted without materialising a broadcast, so ``x[B, S, K] @ W[K, N]``
stays a single (B*S) x K x N GEMM.
"""

from __future__ import annotations

import numpy as np

from nkipy_amd.core import dtypes as dt
from nkipy_amd.core.backend.hip import broadcast_shapes, broadcast_to, convert, reshape
from nkipy_amd.core.backend.promotion import find_common_type
from nkipy_amd.core.ops import elementwise as ew
from nkipy_amd.core.ops import reduce as rd
from nkipy_amd.core.ops._helpers import acc_dtype, ctx, norm_axis, val, wrap
from nkipy_amd.core.ops._registry import Op


def _dot(c, a, b, lhs_batch, rhs_batch, lhs_contract, rhs_contract, out_dtype):
    lhs_free = [i for i in range(a.ndim) if i not in lhs_batch and i not in lhs_contract]
    rhs_free = [i for i in range(b.ndim) if i not in rhs_batch and i not in rhs_contract]
    for la, rb in zip(lhs_contract, rhs_contract):
        if a.shape[la] != b.shape[rb]:
            raise ValueError(
                f"matmul: contracting dimension mismatch {a.shape} vs {b.shape}"
            )
    shape = ([a.shape[i] for i in lhs_batch] + [a.shape[i] for i in lhs_free]
             + [b.shape[i] for i in rhs_free])
    return c.build_op("dot", [a, b], tuple(shape), out_dtype, {
        "lhs_batch": tuple(lhs_batch), "rhs_batch": tuple(rhs_batch),
        "lhs_contract": tuple(lhs_contract), "rhs_contract": tuple(rhs_contract),
        "acc_dtype": acc_dtype(out_dtype),
    })


matmul = Op("matmul")


@matmul.impl("hip")
def _matmul_hip(x, y, out=None, dtype=None, **kw):
    c = ctx()
    promoted = find_common_type(x, y)
    out_dtype = dt.canonical(dtype) if dtype is not None else promoted
    a, b = val(x, promoted), val(y, promoted)
    if a.ndim == 0 or b.ndim == 0:
        raise ValueError("matmul: Input operand does not have enough dimensions")
    a, b = convert(c, a, promoted), convert(c, b, promoted)
    squeeze_m = a.ndim == 1
    squeeze_n = b.ndim == 1
    if squeeze_m:
        a = reshape(c, a, (1, a.shape[0]))
    if squeeze_n:
        b = reshape(c, b, (b.shape[0], 1))
    if a.shape[-1] != b.shape[-2]:
        raise ValueError(
            f"matmul: Input operand 1 has a mismatch in its core dimension 0 "
            f"(size {b.shape[-2]} is different from {a.shape[-1]})"
        )
    if b.ndim == 2:
        r = _dot(c, a, b, [], [], [a.ndim - 1], [0], promoted)
    else:
        batch = broadcast_shapes(a.shape[:-2], b.shape[:-2])
        a = broadcast_to(c, a, batch + a.shape[-2:])
        b = broadcast_to(c, b, batch + b.shape[-2:])
        nb = len(batch)
        r = _dot(c, a, b, list(range(nb)), list(range(nb)), [nb + 1], [nb], promoted)
    shape = list(r.shape)
    if squeeze_n:
        shape.pop(-1)
    if squeeze_m:
        shape.pop(-2 if not squeeze_n else -1)
    r = reshape(c, r, tuple(shape))
    if out_dtype != promoted:
        r = convert(c, r, out_dtype)
    return wrap(r)


dot = Op("dot")


@dot.impl("hip")
def _dot_hip(x, y, out=None):
    a, b = val(x), val(y)
    if a.ndim == 0 or b.ndim == 0:
        return ew.multiply(x, y)
    if a.ndim <= 2 and b.ndim <= 2:
        return _matmul_hip(x, y)
    c = ctx()
    promoted = find_common_type(x, y)
    a, b = convert(c, a, promoted), convert(c, b, promoted)
    rc = b.ndim - 2 if b.ndim >= 2 else 0
    return wrap(_dot(c, a, b, [], [], [a.ndim - 1], [rc], promoted))


outer = Op("outer")


@outer.impl("hip")
def _outer_hip(a, b, out=None):
    c = ctx()
    av, bv = val(a), val(b)
    av = reshape(c, av, (av.size, 1))
    bv = reshape(c, bv, (1, bv.size))
    return ew.multiply(wrap(av), wrap(bv))


trace = Op("trace")


@trace.impl("hip")
def _trace_hip(a, offset=0, axis1=0, axis2=1, dtype=None, out=None):
    v = val(a)
    if v.ndim != 2 or axis1 != 0 or axis2 != 1:
        raise NotImplementedError("trace is supported for 2-D inputs over axes (0, 1)")
    n, m = v.shape
    mask = np.eye(n, m, k=offset, dtype=bool)
    from nkipy_amd.core.ops.indexing import where

    z = where(mask, a, 0)
    return rd.sum(z, dtype=dtype)


norm = Op("norm")


@norm.impl("hip")
def _norm_hip(x, ord=None, axis=None, keepdims=False):
    v = val(x)
    if ord in (None, 2, "fro") and (ord != 2 or axis is not None or v.ndim == 1):
        return ew.sqrt(rd.sum(ew.multiply(x, x), axis=axis, keepdims=keepdims))
    if ord == 1 and (v.ndim == 1 or axis is not None):
        return rd.sum(ew.abs_(x), axis=axis, keepdims=keepdims)
    if ord in (np.inf, float("inf")) and (v.ndim == 1 or axis is not None):
        return rd.max(ew.abs_(x), axis=axis, keepdims=keepdims)
    raise NotImplementedError(f"norm with ord={ord!r} on a {v.ndim}-D input is not supported")
