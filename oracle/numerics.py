"""bf16 and fp8 (E4M3FN) numerics for the oracle (test infrastructure only).

bf16 values are carried as float32 arrays holding RNE-rounded values (no
ml_dtypes here).  The rounding is the closed form: add 0x7FFF plus the kept
least-significant bit to the float32 bit pattern, truncate the low 16 bits.
E4M3FN decoding is the closed form (-1)^s * 2^(e-7) * (1 + m/8), subnormals
2^-6 * m/8, S.1111.111 = NaN.
"""

import numpy as np


def bf16_round(a):
    a = np.asarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(a), a, out).astype(np.float32)


def bf16_bits(a):
    return (bf16_round(a).view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def e4m3fn_decode(codes):
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    s = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    val = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    val = s * val
    return np.where((c & 0x7F) == 0x7F, np.nan, val).astype(np.float32)


E4M3FN_TABLE = e4m3fn_decode(np.arange(256))


def e4m3fn_round(a):
    """Round to the nearest E4M3FN value (ties to even), saturating at +-448.
    Quantum 2^(e-3) in the binade [2^e, 2^(e+1)), e >= -6 (subnormals share
    the quantum 2^-9); np.rint rounds half to even, which is the even mantissa."""
    a = np.asarray(a, dtype=np.float64)
    mag = np.abs(a)
    with np.errstate(divide="ignore"):
        e = np.floor(np.log2(np.where(mag > 0, mag, 1.0)))
    e = np.maximum(e, -6.0)
    q = np.exp2(e - 3.0)
    r = np.minimum(np.rint(mag / q) * q, 448.0)
    return (np.sign(a) * r).astype(np.float32)


def e4m3fn_encode(a):
    """E4M3FN code of the nearest value (see e4m3fn_round)."""
    a = np.asarray(a, dtype=np.float32)
    r = e4m3fn_round(a)
    pos = E4M3FN_TABLE[:0x7F]
    code = np.searchsorted(pos, np.abs(r)).astype(np.uint8)
    sign = np.signbit(r).astype(np.uint8) << 7
    return np.where(np.isnan(a), np.uint8(0x7F), code | sign).astype(np.uint8)


def quantize_per_channel_e4m3fn(w, axis=-1):
    """Per-output-channel symmetric quantisation: scale = amax / 448 over the
    reduction axis ``axis`` (the input-feature axis); returns (codes, scale)."""
    w = np.asarray(w, dtype=np.float32)
    amax = np.max(np.abs(w), axis=axis, keepdims=True)
    scale = np.where(amax > 0, amax / 448.0, 1.0).astype(np.float32)
    codes = e4m3fn_encode(w / scale)
    return codes, np.squeeze(scale, axis=axis)


def dequantize_e4m3fn(codes, scale, axis=-1):
    return (E4M3FN_TABLE[np.asarray(codes, np.uint8)] * np.expand_dims(scale, axis)).astype(np.float32)
