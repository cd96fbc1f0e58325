"""Dtype vocabulary of the backend.

NumPy has no bfloat16 or float8 types.  When ``ml_dtypes`` is importable the
reference's dtypes are used as-is (nkipy/src/nkipy/core/language.py:4-9 takes
them from neuronxcc, which re-exports ml_dtypes).  Otherwise each is a
one-field structured NumPy dtype of the right width, so arrays of it can be
created, viewed, copied to and from the device and compared by dtype, while
their values are converted explicitly with the helpers below.

fp8 is OCP E4M3FN (bias 7, max 448, NaN = S.1111.111), the format gfx950's
MFMA reads.  The reference's ``float8_e4m3`` (IEEE-like, max 240) is accepted
as a separate dtype for tracing but has no device kernels.
"""

from __future__ import annotations

import numpy as np

try:  # pragma: no cover - depends on the environment
    import ml_dtypes as _mld

    bfloat16 = np.dtype(_mld.bfloat16)
    float8_e4m3fn = np.dtype(_mld.float8_e4m3fn)
    float8_e4m3 = np.dtype(_mld.float8_e4m3)
    float8_e5m2 = np.dtype(_mld.float8_e5m2)
    HAVE_ML_DTYPES = True
except ImportError:
    bfloat16 = np.dtype([("bfloat16", "<u2")])
    float8_e4m3fn = np.dtype([("float8_e4m3fn", "u1")])
    float8_e4m3 = np.dtype([("float8_e4m3", "u1")])
    float8_e5m2 = np.dtype([("float8_e5m2", "u1")])
    HAVE_ML_DTYPES = False

float32 = np.dtype(np.float32)
float16 = np.dtype(np.float16)
float64 = np.dtype(np.float64)
int8 = np.dtype(np.int8)
int16 = np.dtype(np.int16)
int32 = np.dtype(np.int32)
int64 = np.dtype(np.int64)
uint8 = np.dtype(np.uint8)
uint16 = np.dtype(np.uint16)
uint32 = np.dtype(np.uint32)
uint64 = np.dtype(np.uint64)
bool_ = np.dtype(np.bool_)

_SPECIAL = {
    "bfloat16": bfloat16,
    "bf16": bfloat16,
    "float8_e4m3fn": float8_e4m3fn,
    "float8_e4m3": float8_e4m3,
    "float8_e5m2": float8_e5m2,
}
_SPECIAL_NAMES = {v: k for k, v in reversed(list(_SPECIAL.items()))}
_SPECIAL_NAMES[bfloat16] = "bfloat16"

FP8_TYPES = (float8_e4m3fn, float8_e4m3, float8_e5m2)
LOW_FLOATS = (bfloat16, float16) + FP8_TYPES


def canonical(d) -> np.dtype:
    """np.dtype for any dtype-like: numpy types, strings, torch dtypes."""
    if isinstance(d, np.dtype):
        return d
    if isinstance(d, str) and d in _SPECIAL:
        return _SPECIAL[d]
    tname = getattr(d, "__module__", None)
    if tname == "torch":
        return from_torch_dtype(d)
    return np.dtype(d)


def name(d) -> str:
    d = canonical(d)
    return _SPECIAL_NAMES.get(d, d.name)


def itemsize(d) -> int:
    return canonical(d).itemsize


def is_float(d) -> bool:
    d = canonical(d)
    return d.kind == "f" or d in LOW_FLOATS


def is_fp8(d) -> bool:
    return canonical(d) in FP8_TYPES


def is_int(d) -> bool:
    return canonical(d).kind in "iu"


def is_bool(d) -> bool:
    return canonical(d) == bool_


# ---------------------------------------------------------------------------
# bf16 <-> fp32 on the host (round to nearest even)
# ---------------------------------------------------------------------------
def f32_to_bf16_bits(a) -> np.ndarray:
    """uint16 bit patterns of float32 values rounded to bf16 (RNE, quiet NaN)."""
    a = np.asarray(a, dtype=np.float32)
    shape = a.shape
    u = np.ascontiguousarray(a).reshape(-1).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    if nan.any():
        r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r.reshape(shape)


def bf16_bits_to_f32(b) -> np.ndarray:
    b = np.asarray(b)
    shape = b.shape
    b = np.ascontiguousarray(b).reshape(-1).view(np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32).reshape(shape)


def round_to_bf16(a) -> np.ndarray:
    """float32 array holding the bf16-rounded values of ``a``."""
    return bf16_bits_to_f32(f32_to_bf16_bits(a))


def to_bf16(a) -> np.ndarray:
    """Array of dtype ``bfloat16`` (bit patterns) from float values."""
    if HAVE_ML_DTYPES:  # pragma: no cover
        return np.asarray(a, dtype=np.float32).astype(bfloat16)
    return f32_to_bf16_bits(a).view(bfloat16)


def bf16_to_f32(a) -> np.ndarray:
    if HAVE_ML_DTYPES:  # pragma: no cover
        return np.asarray(a).astype(np.float32)
    a = np.asarray(a)
    return bf16_bits_to_f32(np.ascontiguousarray(a).reshape(-1).view(np.uint16)).reshape(a.shape)


# ---------------------------------------------------------------------------
# fp8 E4M3FN on the host
# ---------------------------------------------------------------------------
def _e4m3fn_table() -> np.ndarray:
    t = np.empty(256, dtype=np.float32)
    for b in range(256):
        s = -1.0 if b & 0x80 else 1.0
        e = (b >> 3) & 0xF
        m = b & 0x7
        if (b & 0x7F) == 0x7F:
            t[b] = np.nan
        elif e == 0:
            t[b] = s * (m / 8.0) * 2.0**-6
        else:
            t[b] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return t


E4M3FN_VALUES = _e4m3fn_table()
E4M3FN_MAX = 448.0


def e4m3fn_bits_to_f32(b) -> np.ndarray:
    b = np.asarray(b)
    return E4M3FN_VALUES[np.ascontiguousarray(b).reshape(-1).view(np.uint8)].reshape(b.shape)


def f32_to_e4m3fn_bits(a, saturate: bool = True) -> np.ndarray:
    """Round float32 to E4M3FN (nearest, ties to even).  Out-of-range values
    saturate to +-448 (``saturate``) or become NaN."""
    a = np.asarray(a, dtype=np.float32)
    finite_vals = E4M3FN_VALUES[:127]  # 0x00..0x7e, ascending non-negative
    mag = np.abs(a)
    idx = np.searchsorted(finite_vals, mag, side="left")
    idx = np.clip(idx, 0, 126)
    lo = np.clip(idx - 1, 0, 126)
    hi = idx
    dlo = np.abs(mag - finite_vals[lo])
    dhi = np.abs(finite_vals[hi] - mag)
    # ties go to the even code (mantissa LSB 0)
    pick_hi = (dhi < dlo) | ((dhi == dlo) & (hi % 2 == 0))
    code = np.where(pick_hi, hi, lo).astype(np.uint8)
    over = mag > E4M3FN_MAX
    if saturate:
        code = np.where(over, np.uint8(0x7E), code)
    else:
        # beyond the rounding midpoint of the largest value -> NaN
        code = np.where(mag >= 464.0, np.uint8(0x7F), code)
    code = np.where(np.isnan(a), np.uint8(0x7F), code)
    sign = (np.signbit(a) & ~np.isnan(a)).astype(np.uint8) << 7
    return (code | sign).astype(np.uint8)


def to_e4m3fn(a, saturate: bool = True) -> np.ndarray:
    return f32_to_e4m3fn_bits(a, saturate).view(float8_e4m3fn)


# ---------------------------------------------------------------------------
# torch interop (torch is optional)
# ---------------------------------------------------------------------------
def _torch():
    import torch

    return torch


def torch_dtype(d):
    torch = _torch()
    d = canonical(d)
    table = {
        float32: torch.float32, float16: torch.float16, bfloat16: torch.bfloat16,
        float8_e4m3fn: torch.float8_e4m3fn, float8_e5m2: torch.float8_e5m2,
        int8: torch.int8, int16: torch.int16, int32: torch.int32, int64: torch.int64,
        uint8: torch.uint8, bool_: torch.bool, float64: torch.float64,
    }
    if d == uint32 and hasattr(torch, "uint32"):
        return torch.uint32
    if d not in table:
        raise TypeError(f"no torch dtype for {name(d)}")
    return table[d]


def from_torch_dtype(td) -> np.dtype:
    torch = _torch()
    table = {
        torch.float32: float32, torch.float16: float16, torch.bfloat16: bfloat16,
        torch.float8_e4m3fn: float8_e4m3fn, torch.float8_e5m2: float8_e5m2,
        torch.int8: int8, torch.int16: int16, torch.int32: int32, torch.int64: int64,
        torch.uint8: uint8, torch.bool: bool_, torch.float64: float64,
    }
    if hasattr(torch, "uint32"):
        table[torch.uint32] = uint32
    if td not in table:
        raise TypeError(f"unsupported torch dtype {td}")
    return table[td]


def numpy_storage(a: np.ndarray) -> np.ndarray:
    """View of ``a`` with a plain integer dtype of the same width when its
    dtype is a structured stand-in (bf16 / fp8); otherwise ``a``."""
    if a.dtype.fields is not None:
        return a.view({1: np.uint8, 2: np.uint16}[a.dtype.itemsize])
    return a


def to_float32(a) -> np.ndarray:
    """Float32 values of an array of any supported dtype."""
    a = np.asarray(a)
    d = a.dtype
    if d == bfloat16:
        return bf16_to_f32(a)
    if d == float8_e4m3fn and not HAVE_ML_DTYPES:
        return e4m3fn_bits_to_f32(a)
    return a.astype(np.float32)
