"""Host-side launchers of the hand-written gfx950 kernels.

Each launcher checks operand shapes / dtypes / alignment on the host, picks a
kernel variant and a launch shape, and packs the kernel's argument struct.
It returns a :class:`Launch` -- nothing here touches device memory -- so the
same code serves direct calls, compiled kernel plans and the benchmark.
Argument structs mirror the C structs in ``csrc/kernels/*.hip`` field by
field; the kernel manifest's ``kernarg_size`` is checked at launch.
"""

from __future__ import annotations

import ctypes
import functools
from dataclasses import dataclass, field
from typing import List, Tuple

import numpy as np

from nkipy_amd.core import dtypes as dt


class LaunchError(ValueError):
    """Operands do not fit what a kernel and its grid assume."""


@dataclass
class Launch:
    module: str
    symbol: str
    grid: Tuple[int, int, int]
    block: Tuple[int, int, int]
    args: ctypes.Structure
    shared: int = 0
    # algorithmic work of this launch, for roofline reporting
    bytes: int = 0
    flops: int = 0
    note: str = ""
    extra: dict = field(default_factory=dict)

    def function(self, rt):
        return rt.function(self.module, self.symbol)

    def run(self, rt):
        self.function(rt).launch(self.grid, self.block, self.args, self.shared)


# dtype tag used in kernel symbol names
_TAG = {
    dt.float32: "f32",
    dt.bfloat16: "bf16",
    dt.float16: "f16",
}


def dtype_tag(d) -> str:
    d = dt.canonical(d)
    try:
        return _TAG[d]
    except KeyError:
        raise LaunchError(f"dtype {dt.name(d)} has no kernel variant") from None


# ---------------------------------------------------------------------------
# Row softmax
# ---------------------------------------------------------------------------
class SoftmaxArgs(ctypes.Structure):
    _fields_ = [
        ("x", ctypes.c_void_p),
        ("y", ctypes.c_void_p),
        ("rows", ctypes.c_int64),
        ("n", ctypes.c_int32),
        ("flags", ctypes.c_int32),
    ]


SMX_ROUND_OPS = 1


# (block, chunks) register variants of softmax: a row of up to
# block*chunks*8 elements, first fit wins.  Rows of up to 4096 elements take
# one wave of 64 lanes x 8 chunks (MI355X, fp32 (2048, 4096): 14.4 us against
# 16.0-17.3 us for 128 x 4 and 14.9-15.8 us for 256 x 2).
_ROW_REG_VARIANTS = [(64, 1), (256, 1), (64, 8), (512, 4)]
# every (block, chunks) pair compiled for the row kernels
_ALL_REG_VARIANTS = {(64, 1), (128, 4), (256, 1), (256, 2), (512, 1), (256, 4), (512, 4)}
_SOFTMAX_REG_VARIANTS = _ALL_REG_VARIANTS | {(64, 8)}
_SOFTMAX_TYPES = {("f32", "f32"), ("bf16", "bf16"), ("bf16", "f32"), ("f32", "bf16"), ("f16", "f16")}


def _row_variant(n: int, elem_bytes: int, ptr_align_ok: bool):
    """Pick the register-resident variant for a row of n elements, or None."""
    if n % 8 != 0 or not ptr_align_ok:
        return None
    for block, chunks in _ROW_REG_VARIANTS:
        if n <= block * chunks * 8:
            # do not leave most of a large block idle
            return block, chunks
    return None


def softmax_rows(x_ptr: int, y_ptr: int, rows: int, n: int, in_dtype, out_dtype,
                 block_chunks=None, round_ops: bool = False) -> Launch:
    """y[r, :] = softmax(x[r, :]) over rows of n contiguous elements.
    ``round_ops``: the softmax runs in the 16-bit input type (x - max, exp,
    sum and divide each rounded to it, the sum accumulated in fp32)."""
    ti, to = dtype_tag(in_dtype), dtype_tag(out_dtype)
    if (ti, to) not in _SOFTMAX_TYPES:
        raise LaunchError(f"softmax has no {ti}->{to} variant")
    if rows <= 0 or n <= 0:
        raise LaunchError(f"softmax needs rows > 0 and n > 0, got rows={rows}, n={n}")
    if rows >= 2**31:
        raise LaunchError("softmax: too many rows for one launch")
    aligned = x_ptr % 16 == 0 and y_ptr % 16 == 0
    var = _row_variant(n, dt.itemsize(in_dtype), aligned)
    if block_chunks is not None and var is not None:
        if n > block_chunks[0] * block_chunks[1] * 8 or tuple(block_chunks) not in _SOFTMAX_REG_VARIANTS:
            raise LaunchError(f"softmax variant {block_chunks} does not fit n={n}")
        var = tuple(block_chunks)
    if round_ops and dt.itemsize(in_dtype) != 2:
        raise LaunchError("softmax steps round only to a 16-bit input type")
    args = SoftmaxArgs(x_ptr, y_ptr, rows, n, SMX_ROUND_OPS if round_ops else 0)
    nbytes = rows * n * (dt.itemsize(in_dtype) + dt.itemsize(out_dtype))
    if var is None:
        return Launch("rowwise", f"nk_softmax_loop_{ti}_{to}", (rows, 1, 1), (256, 1, 1),
                      args, bytes=nbytes, note="loop")
    block, chunks = var
    return Launch("rowwise", f"nk_softmax_reg_{ti}_{to}_b{block}_c{chunks}",
                  (rows, 1, 1), (block, 1, 1), args, bytes=nbytes)


# ---------------------------------------------------------------------------
# Residual + RMSNorm
# ---------------------------------------------------------------------------
class RmsNormArgs(ctypes.Structure):
    _fields_ = [
        ("x", ctypes.c_void_p),
        ("r", ctypes.c_void_p),
        ("w", ctypes.c_void_p),
        ("y", ctypes.c_void_p),
        ("h", ctypes.c_void_p),
        ("rows", ctypes.c_int64),
        ("n", ctypes.c_int32),
        ("eps", ctypes.c_float),
        ("flags", ctypes.c_int32),
        ("pad", ctypes.c_int32),
    ]


RMS_RES = 1
RMS_ROUND_H = 2
RMS_WRITE_H = 4
RMS_MUL_RECIP = 8
RMS_W = 16

# RMSNorm (block, chunks), first fit wins.  A chunk past the row's end still
# issues its (zero-returning) loads, so the tightest fit is taken: residual
# bf16 (8192, 4096) measured 33.8 us with 256 x 2 against 35.7 us with 256 x 4.
_RMS_REG_VARIANTS = [(64, 1), (256, 1), (256, 2), (256, 4), (512, 4)]


def rmsnorm_rows(x_ptr: int, y_ptr: int, rows: int, n: int, dtype, eps: float,
                 r_ptr: int = 0, w_ptr: int = 0, h_ptr: int = 0,
                 round_h: bool = True, mul_recip: bool = False,
                 block_chunks=None) -> Launch:
    """y = h / sqrt(mean(h*h) + eps) * w with h = x (+ r), rows of n elements.

    Every operand has the storage dtype ``dtype``; ``w`` has n elements.
    ``round_h`` rounds x + r to ``dtype`` before use (the add happened in the
    storage dtype); ``mul_recip`` multiplies by 1/sqrt instead of dividing.
    """
    tag = dtype_tag(dtype)
    if rows <= 0 or n <= 0:
        raise LaunchError(f"rmsnorm needs rows > 0 and n > 0, got rows={rows}, n={n}")
    if rows >= 2**31:
        raise LaunchError("rmsnorm: too many rows for one launch")
    flags = 0
    if r_ptr:
        flags |= RMS_RES
        if round_h:
            flags |= RMS_ROUND_H
        if h_ptr:
            flags |= RMS_WRITE_H
    elif h_ptr:
        raise LaunchError("rmsnorm: h output requested without a residual")
    if w_ptr:
        flags |= RMS_W
    if mul_recip:
        flags |= RMS_MUL_RECIP
    ptrs = [p for p in (x_ptr, y_ptr, r_ptr, w_ptr, h_ptr) if p]
    aligned = all(p % 16 == 0 for p in ptrs)
    isz = dt.itemsize(dtype)
    nbytes = rows * n * isz * (2 + (1 if r_ptr else 0) + (1 if h_ptr else 0)) + (n * isz if w_ptr else 0)
    args = RmsNormArgs(x_ptr, r_ptr or None, w_ptr or None, y_ptr, h_ptr or None,
                       rows, n, float(eps), flags, 0)
    var = None
    if n % 8 == 0 and aligned:
        if block_chunks is not None:
            var = tuple(block_chunks)
            if n > var[0] * var[1] * 8 or var not in _ALL_REG_VARIANTS:
                raise LaunchError(f"rmsnorm variant {var} too small for n={n}")
        else:
            for b, c in _RMS_REG_VARIANTS:
                if n <= b * c * 8:
                    var = (b, c)
                    break
    if var is None:
        return Launch("rowwise", f"nk_rmsnorm_loop_{tag}", (rows, 1, 1), (256, 1, 1), args,
                      bytes=nbytes, note="loop")
    b, c = var
    kind = "res" if r_ptr else "reg"
    return Launch("rowwise", f"nk_rmsnorm_{kind}_{tag}_b{b}_c{c}", (rows, 1, 1), (b, 1, 1), args,
                  bytes=nbytes)


def as_ptr(a) -> int:
    """Device address of a DeviceTensor-like object or an int."""
    if isinstance(a, (int, np.integer)):
        return int(a)
    return int(a.ptr)


# ---------------------------------------------------------------------------
# MFMA GEMM (csrc/kernels/gemm.hip)
# ---------------------------------------------------------------------------
class GemmArgs(ctypes.Structure):
    _fields_ = [
        ("A", ctypes.c_void_p), ("B0", ctypes.c_void_p), ("B1", ctypes.c_void_p),
        ("C", ctypes.c_void_p), ("bias", ctypes.c_void_p), ("scale0", ctypes.c_void_p),
        ("scale1", ctypes.c_void_p), ("resid", ctypes.c_void_p),
        ("M", ctypes.c_int64), ("N", ctypes.c_int64), ("K", ctypes.c_int64),
        ("lda", ctypes.c_int64), ("ldb", ctypes.c_int64), ("ldc", ctypes.c_int64),
        ("tiles_m", ctypes.c_int32), ("tiles_n", ctypes.c_int32),
        ("flags", ctypes.c_int32), ("group_m", ctypes.c_int32),
        ("rope_cos", ctypes.c_void_p), ("rope_sin", ctypes.c_void_p),
        ("rope_q", ctypes.c_void_p), ("rope_k", ctypes.c_void_p),
        ("rope_ts", ctypes.c_int64), ("rope_seq", ctypes.c_int32),
        ("rope_nq", ctypes.c_int32), ("rope_nk", ctypes.c_int32), ("rope_pad", ctypes.c_int32),
        ("ksplit", ctypes.c_int32), ("kc", ctypes.c_int32),
    ]


class GemmRope:
    """Rotary embedding folded into a QKV projection's epilogue: columns
    0 .. nq-1 (q heads) and nq .. nq+nk-1 (k heads) of the product, heads of
    128, are rotated by fp32 tables (position, 64) with row stride
    ``table_stride`` (row m at position m % seq) and written to q_ptr (M x nq)
    and k_ptr (M x nk), bf16; C receives only the columns after them."""

    HEAD_DIM = 128

    def __init__(self, cos_ptr, sin_ptr, q_ptr, k_ptr, table_stride, seq, nq, nk):
        self.cos_ptr, self.sin_ptr, self.q_ptr, self.k_ptr = cos_ptr, sin_ptr, q_ptr, k_ptr
        self.table_stride, self.seq, self.nq, self.nk = int(table_stride), int(seq), int(nq), int(nk)


GEMM_BIAS = 1
GEMM_SCALE = 2
GEMM_RESID = 4
GEMM_VEC = 8
GEMM_RND_BIAS = 16
GEMM_RND_RESID = 32
GEMM_ROWS16 = 64
GEMM_BM = 256
GEMM_BN = 256


def gemm(a_ptr: int, b_ptr: int, c_ptr: int, M: int, N: int, K: int, *, layout: str,
         b_dtype, c_dtype, lda: int = None, ldb: int = None, ldc: int = None,
         bias_ptr: int = 0, scale_ptr: int = 0, resid_ptr: int = 0,
         up_ptr: int = 0, up_scale_ptr: int = 0, pingpong: bool = None,
         round_before_bias: bool = False, round_before_resid: bool = False,
         rope: GemmRope = None, stage64: bool = None, staged: bool = None) -> Launch:
    """C[M, N] = A[M, K] @ B (+ epilogue) on bf16 MFMA, fp32 accumulation.

    ``layout`` "nn": B is K x N row-major (ldb >= N); "nt": B is N x K
    row-major (ldb >= K).  ``b_dtype`` bf16 or float8_e4m3fn (then
    ``scale_ptr`` gives fp32 per-column scales).  With ``up_ptr`` the kernel
    computes the SwiGLU product silu(A @ B) * (A @ B_up) instead (B_up has the
    layout and leading dimension of B).  ``bias_ptr`` (bf16, N) and
    ``resid_ptr`` (C dtype, M x N, leading dimension ldc) are added;
    ``round_before_bias`` / ``round_before_resid`` round the running value to
    bf16 before that add (the cast points of ``(x @ w).astype(bf16) + r``).
    ``pingpong`` selects the 8-wave kernel (two waves per SIMD alternating
    between MFMAs and fragment loads; the default where it exists, i.e. for
    every layout except fp8 NN weights) or the 4-wave kernel.  ``rope``
    (:class:`GemmRope`) selects the 8-wave kernel whose epilogue applies the
    rotary embedding to the q / k columns.  ``stage64`` (default: wherever
    it exists, i.e. on the 8-wave kernel for fp8 NT weights and for bf16 NN
    weights without a rotary epilogue) selects 64-deep A stages in LDS
    (whole 128-byte lines per global read).  ``staged``
    (default: wherever it applies, i.e. 64-deep stages and a bf16 output in
    aligned 16-byte row chunks) writes the output tile through LDS so that
    every global store covers whole lines.
    """
    if layout not in ("nn", "nt"):
        raise LaunchError(f"unknown GEMM layout {layout}")
    b_dtype, c_dtype = dt.canonical(b_dtype), dt.canonical(c_dtype)
    fp8 = b_dtype == dt.float8_e4m3fn
    if not fp8 and b_dtype != dt.bfloat16:
        raise LaunchError(f"GEMM weights must be bf16 or float8_e4m3fn, got {dt.name(b_dtype)}")
    if c_dtype not in (dt.bfloat16, dt.float32):
        raise LaunchError(f"GEMM output must be bf16 or float32, got {dt.name(c_dtype)}")
    if M <= 0 or N <= 0 or K <= 0:
        raise LaunchError(f"GEMM needs positive sizes, got M={M} N={N} K={K}")
    lda = K if lda is None else lda
    ldb = (N if layout == "nn" else K) if ldb is None else ldb
    ldc = N if ldc is None else ldc
    swiglu = bool(up_ptr)
    if K % 8 or lda % 8 or ldb % 8:
        raise LaunchError("GEMM needs K, lda and ldb to be multiples of 8 (16-byte rows)")
    if lda < K or ldc < N or (layout == "nn" and ldb < N) or (layout == "nt" and ldb < K):
        raise LaunchError("GEMM leading dimension smaller than the matrix")
    balign = 8 if (fp8 and layout == "nn") else 16
    for p, al in ((a_ptr, 16), (b_ptr, balign), (up_ptr, balign)):
        if p and p % al:
            raise LaunchError("GEMM operand pointer is not aligned for 128-bit access")
    if fp8 and layout == "nt" and (K % 16 or ldb % 16):
        raise LaunchError("NT GEMM with fp8 weights needs K and ldb to be multiples of 16 (16-byte rows)")
    # operands are addressed with 32-bit byte offsets from one base
    b_rows = N if layout == "nt" else K
    if M * lda * 2 >= 2**31 or b_rows * ldb * b_dtype.itemsize >= 2**31:
        raise LaunchError("GEMM operands must be smaller than 2 GiB each")
    if layout == "nn" and N % 8:
        raise LaunchError("NN GEMM needs N to be a multiple of 8")
    if fp8 and not scale_ptr:
        raise LaunchError("fp8 weights need per-column scales")
    if swiglu and (fp8 != bool(up_scale_ptr)):
        raise LaunchError("SwiGLU with fp8 weights needs scales for both weights")
    if swiglu and (bias_ptr or resid_ptr or c_dtype != dt.bfloat16):
        raise LaunchError("the SwiGLU epilogue writes bf16 without bias / residual")
    bn = GEMM_BN // 2 if swiglu else GEMM_BN
    tiles_m = -(-M // GEMM_BM)
    tiles_n = -(-N // bn)
    if tiles_m * tiles_n >= 2**31:
        raise LaunchError("GEMM grid too large")
    flags = (GEMM_BIAS if bias_ptr else 0) | (GEMM_SCALE if scale_ptr else 0) | (GEMM_RESID if resid_ptr else 0)
    if round_before_bias and bias_ptr:
        flags |= GEMM_RND_BIAS
    if round_before_resid and resid_ptr:
        flags |= GEMM_RND_RESID
    # 4-element vector access to C (and the residual) when rows keep 8 / 16-byte alignment
    vbytes = 4 * c_dtype.itemsize
    if ldc % 4 == 0 and c_ptr % vbytes == 0 and (not resid_ptr or resid_ptr % vbytes == 0):
        flags |= GEMM_VEC
    # bf16 rows in aligned 16-byte chunks, a residual (if any) added to the
    # bf16-rounded value: the output tile may be staged through LDS
    if c_dtype == dt.bfloat16 and N % 8 == 0 and ldc % 8 == 0 and c_ptr % 16 == 0 and (
            not resid_ptr or (round_before_resid and resid_ptr % 16 == 0)):
        flags |= GEMM_ROWS16
    args = GemmArgs(a_ptr, b_ptr, up_ptr or None, c_ptr, bias_ptr or None, scale_ptr or None,
                    up_scale_ptr or None, resid_ptr or None, M, N, K, lda, ldb, ldc,
                    tiles_m, tiles_n, flags, 0)
    if rope is not None:
        hd = GemmRope.HEAD_DIM
        if swiglu or bias_ptr or resid_ptr or c_dtype != dt.bfloat16 or pingpong is False:
            raise LaunchError("the rotary epilogue is a plain bf16 projection on the 8-wave kernel")
        if rope.nq % hd or rope.nk % hd or rope.nq + rope.nk <= 0 or rope.nq + rope.nk > N:
            raise LaunchError(f"rotated columns must be whole heads of {hd} within N, got "
                              f"{rope.nq} + {rope.nk} of {N}")
        if rope.seq <= 0 or M % rope.seq:
            raise LaunchError(f"rows ({M}) must be whole sequences of {rope.seq} positions")
        if rope.table_stride % 4 or rope.table_stride < hd // 2:
            raise LaunchError("rope tables need a row stride that is a multiple of 4 and covers 64")
        if any(p % 16 for p in (rope.cos_ptr, rope.sin_ptr)) or any(
                p % 8 for p in (rope.q_ptr, rope.k_ptr)) or not (rope.q_ptr and rope.k_ptr):
            raise LaunchError("rope tables must be 16-byte and outputs 8-byte aligned")
        args.rope_cos, args.rope_sin = rope.cos_ptr, rope.sin_ptr
        args.rope_q, args.rope_k = rope.q_ptr, rope.k_ptr
        args.rope_ts, args.rope_seq = rope.table_stride, rope.seq
        args.rope_nq, args.rope_nk = rope.nq, rope.nk
    btag = "e4m3" if fp8 else "bf16"
    ctag = "bf16" if c_dtype == dt.bfloat16 else "f32"
    has_pp = not (fp8 and layout == "nn")
    if pingpong is None:
        pingpong = has_pp
    if pingpong and not has_pp:
        raise LaunchError("the 8-wave GEMM has no fp8 NN variant")
    has_k64 = bool(pingpong and ((fp8 and layout == "nt") or (not fp8 and layout == "nn" and rope is None)))
    if stage64 is None:  # the default wherever it exists: whole-line global reads
        stage64 = has_k64
    if stage64 and not has_k64:
        raise LaunchError("64-deep K stages exist on the 8-wave kernel for fp8 NT weights and for bf16 NN "
                          "weights without a rotary epilogue")
    prefix = ("nk_gemm8k" if stage64 else "nk_gemm8") if pingpong else "nk_gemm"
    if swiglu:
        symbol = f"{prefix}_swiglu_{layout}_{btag}_bf16"
    else:
        symbol = f"{prefix}_{layout}_{btag}_{ctag}" + ("_rope" if rope is not None else "")
    can_stage = bool(stage64 and (flags & GEMM_ROWS16) and (
        rope is None or (rope.q_ptr % 16 == 0 and rope.k_ptr % 16 == 0)))
    if staged is None:
        staged = can_stage
    if staged and not can_stage:
        raise LaunchError("the staged epilogue needs 64-deep stages and a bf16 output in aligned 16-byte row "
                          "chunks (a residual added after the bf16 rounding; 16-byte aligned rotary outputs)")
    if staged:
        symbol += "_r16"  # the output tile staged through LDS
    n_mm = 2 if swiglu else 1
    nbytes = M * K * 2 + n_mm * N * K * b_dtype.itemsize + M * N * c_dtype.itemsize
    return Launch("gemm", symbol, (tiles_m * tiles_n, 1, 1), (512 if pingpong else 256, 1, 1), args,
                  bytes=nbytes, flops=2 * M * N * K * n_mm)


SPLITK_TARGET_WGS = 256  # one 8-wave GEMM workgroup per CU


def gemm_splitk_split(M: int, N: int, K: int, swiglu: bool = False, fp8: bool = False):
    """(ksplit, kc) for :func:`gemm_splitk`: K ranges of kc (a multiple of
    64) so that tiles x ranges is about one workgroup per CU.  Past 64 rows
    each range's fp32 partial plane (4 M N bytes, written once and read once)
    costs as much as its share of the K loop saves, so the planes are held
    to half the weight bytes (measured at 4096 x 4096: 256 rows in 16 ranges
    66 us against 80 us in one loop, 128 rows in 8 ranges 42 us); ksplit 1
    when the tiles alone fill the part."""
    tiles = -(-M // GEMM_BM) * -(-N // GEMM_BN)
    ks = max(1, min(SPLITK_TARGET_WGS // tiles, -(-K // 64)))
    if M > 64:
        ks = max(1, min(ks, (N * K * (1 if fp8 else 2)) // (2 * 4 * M * N)))
    kc = -(-(-(-K // ks)) // 64) * 64
    return -(-K // kc), kc


def gemm_splitk_useful(M: int, N: int, K: int, swiglu: bool = False, fp8: bool = False) -> bool:
    """Whether the K-range form beats one K loop per tile: up to 64 rows
    whenever it splits; up to 256 rows only when the tiles leave most CUs
    idle (at most 32 tiles) -- 512 or more rows, or 256 rows of a 14336-wide
    projection, measured slower split."""
    if M > GEMM_BM or (M > 64 and -(-N // GEMM_BN) > 32):
        return False
    return gemm_splitk_split(M, N, K, swiglu, fp8)[0] > 1


def gemm_splitk_workspace_bytes(M: int, N: int, K: int, swiglu: bool = False, fp8: bool = False) -> int:
    ks, _ = gemm_splitk_split(M, N, K, swiglu, fp8)
    return 4 * ks * M * N * (2 if swiglu else 1)


def gemm_splitk(a_ptr: int, b_ptr: int, c_ptr: int, M: int, N: int, K: int, *, layout: str, b_dtype, c_dtype,
                ws_ptr: int, lda: int = None, ldb: int = None, ldc: int = None, bias_ptr: int = 0,
                scale_ptr: int = 0, resid_ptr: int = 0, up_ptr: int = 0, up_scale_ptr: int = 0,
                round_before_bias: bool = False, round_before_resid: bool = False) -> List[Launch]:
    """The operation of :func:`gemm` (no rotary form) for few rows: the MFMA
    kernels over K ranges (grid y) into fp32 partial planes in the workspace
    at ``ws_ptr`` (``gemm_splitk_workspace_bytes``; the SwiGLU form runs the
    gate and the up weights into two sets of planes), then the reduction of
    :func:`gemv` adds the ranges in order and applies the epilogue.  bf16 NN,
    bf16 NT and fp8 NT weights."""
    if layout not in ("nn", "nt"):
        raise LaunchError(f"unknown GEMM layout {layout}")
    b_dtype, c_dtype = dt.canonical(b_dtype), dt.canonical(c_dtype)
    fp8 = b_dtype == dt.float8_e4m3fn
    if fp8 and layout == "nn":
        raise LaunchError("the split-K GEMM has no fp8 NN variant")
    if not fp8 and b_dtype != dt.bfloat16:
        raise LaunchError(f"GEMM weights must be bf16 or float8_e4m3fn, got {dt.name(b_dtype)}")
    if c_dtype not in (dt.bfloat16, dt.float32):
        raise LaunchError(f"GEMM output must be bf16 or float32, got {dt.name(c_dtype)}")
    if M <= 0 or N <= 0 or K <= 0:
        raise LaunchError(f"GEMM needs positive sizes, got M={M} N={N} K={K}")
    if not ws_ptr or ws_ptr % 16:
        raise LaunchError("the split-K GEMM needs a 16-byte aligned workspace")
    swiglu = bool(up_ptr)
    lda = K if lda is None else lda
    ldb = (N if layout == "nn" else K) if ldb is None else ldb
    ldc = N if ldc is None else ldc
    if swiglu and (fp8 != bool(up_scale_ptr)):
        raise LaunchError("SwiGLU with fp8 weights needs scales for both weights")
    if swiglu and (bias_ptr or resid_ptr or c_dtype != dt.bfloat16):
        raise LaunchError("the SwiGLU epilogue writes bf16 without bias / residual")
    if fp8 and not scale_ptr:
        raise LaunchError("fp8 weights need per-column scales")
    ks, kc = gemm_splitk_split(M, N, K, swiglu, fp8)
    plane = M * N
    launches = []
    for i, bp in enumerate([b_ptr] + ([up_ptr] if swiglu else [])):
        # the operand checks of gemm(); fp32 partial sums, no epilogue
        part = gemm(a_ptr, bp, ws_ptr + 4 * i * ks * plane, M, N, K, layout=layout, b_dtype=b_dtype,
                    c_dtype=dt.float32, lda=lda, ldb=ldb, ldc=N, pingpong=True,
                    scale_ptr=1 if fp8 else 0)
        args = part.args
        args.scale0 = None
        args.flags &= GEMM_VEC
        args.ksplit, args.kc = ks, kc
        launches.append(Launch("gemm", part.symbol + "_splitk", (part.grid[0], ks, 1), part.block, args,
                               bytes=M * K * 2 + N * K * b_dtype.itemsize + 4 * ks * plane,
                               flops=2 * M * N * K))
    flags = (GEMM_BIAS if bias_ptr else 0) | (GEMM_SCALE if scale_ptr else 0) | (GEMM_RESID if resid_ptr else 0)
    if round_before_bias and bias_ptr:
        flags |= GEMM_RND_BIAS
    if round_before_resid and resid_ptr:
        flags |= GEMM_RND_RESID
    out = GemvArgs(a_ptr, b_ptr, up_ptr or None, c_ptr, bias_ptr or None, scale_ptr or None,
                   up_scale_ptr or None, resid_ptr or None, ws_ptr, M, N, K, lda, ldb, ldc, ks, kc, flags, 0)
    ctag = "bf16" if c_dtype == dt.bfloat16 else "f32"
    sw = "_swiglu" if swiglu else ""
    launches.append(Launch("gemv", f"nk_gemv_out_{ctag}{sw}", (-(-plane // 64), 1, 1), (256, 1, 1), out,
                           bytes=4 * ks * plane * len(launches) + plane * c_dtype.itemsize))
    return launches


# ---------------------------------------------------------------------------
# Projections of a few rows (csrc/kernels/gemv.hip)
# ---------------------------------------------------------------------------
class GemvArgs(ctypes.Structure):
    _fields_ = [
        ("A", ctypes.c_void_p), ("B0", ctypes.c_void_p), ("B1", ctypes.c_void_p),
        ("C", ctypes.c_void_p), ("bias", ctypes.c_void_p), ("scale0", ctypes.c_void_p),
        ("scale1", ctypes.c_void_p), ("resid", ctypes.c_void_p), ("ws", ctypes.c_void_p),
        ("M", ctypes.c_int64), ("N", ctypes.c_int64), ("K", ctypes.c_int64),
        ("lda", ctypes.c_int64), ("ldb", ctypes.c_int64), ("ldc", ctypes.c_int64),
        ("ksplit", ctypes.c_int32), ("kc", ctypes.c_int32), ("flags", ctypes.c_int32), ("pad", ctypes.c_int32),
    ]


GEMV_MAX_M = 8  # rows the split-K projection kernels take


def gemv_preferred(M: int, layout: str, fp8: bool) -> bool:
    """Whether :func:`gemv` beats the MFMA GEMM over K ranges for M rows
    (measured on 4096 x 4096 / 6144 projections: one row for bf16 weights,
    up to four for fp8 NT, any row count the split-K GEMM lacks)."""
    if M == 1 or (fp8 and layout == "nn"):
        return M <= GEMV_MAX_M
    return fp8 and M <= 4
GEMV_MAX_KC = 1024
GEMV_NT_ROWS = 16  # weight rows (output columns) per NT workgroup
_GEMV_TARGET_WGS = 1024


def gemv_split(M: int, N: int, K: int, layout: str, fp8: bool):
    """(ksplit, kc): K ranges of kc (at most 1024, a multiple of 8, or of 16
    for NT fp8 weights) so that the partial-sum grid has about 1024
    workgroups."""
    blocks = -(-N // 256) if layout == "nn" else -(-N // GEMV_NT_ROWS)
    step = 16 if (fp8 and layout == "nt") else 8
    ks = max(1, min(-(-_GEMV_TARGET_WGS // blocks), -(-K // step)))
    kc = -(-(-(-K // ks)) // step) * step
    if kc > GEMV_MAX_KC:
        kc = GEMV_MAX_KC
    return -(-K // kc), kc


def gemv_workspace_bytes(M: int, N: int, K: int, layout: str, fp8: bool, swiglu: bool = False) -> int:
    """fp32 partial sums of every K range (twice for the SwiGLU form)."""
    ks, _ = gemv_split(M, N, K, layout, fp8)
    return 4 * ks * M * N * (2 if swiglu else 1)


def gemv(a_ptr: int, b_ptr: int, c_ptr: int, M: int, N: int, K: int, *, layout: str, b_dtype, c_dtype,
         ws_ptr: int, lda: int = None, ldb: int = None, ldc: int = None, bias_ptr: int = 0,
         scale_ptr: int = 0, resid_ptr: int = 0, up_ptr: int = 0, up_scale_ptr: int = 0,
         round_before_bias: bool = False, round_before_resid: bool = False) -> List[Launch]:
    """The operation of :func:`gemm` (same operands and epilogues, no rotary
    form) for M <= 8 rows: partial sums over K ranges into the workspace at
    ``ws_ptr`` (``gemv_workspace_bytes``), then the splits added in order and
    the epilogue.  Two launches."""
    if layout not in ("nn", "nt"):
        raise LaunchError(f"unknown GEMM layout {layout}")
    b_dtype, c_dtype = dt.canonical(b_dtype), dt.canonical(c_dtype)
    fp8 = b_dtype == dt.float8_e4m3fn
    if not fp8 and b_dtype != dt.bfloat16:
        raise LaunchError(f"GEMM weights must be bf16 or float8_e4m3fn, got {dt.name(b_dtype)}")
    if c_dtype not in (dt.bfloat16, dt.float32):
        raise LaunchError(f"GEMM output must be bf16 or float32, got {dt.name(c_dtype)}")
    if not (0 < M <= GEMV_MAX_M) or N <= 0 or K <= 0:
        raise LaunchError(f"the split-K projection takes 1..{GEMV_MAX_M} rows, got M={M} N={N} K={K}")
    lda = K if lda is None else lda
    ldb = (N if layout == "nn" else K) if ldb is None else ldb
    ldc = N if ldc is None else ldc
    swiglu = bool(up_ptr)
    if K % 8 or lda % 8 or ldb % 8:
        raise LaunchError("GEMM needs K, lda and ldb to be multiples of 8 (16-byte rows)")
    if lda < K or ldc < N or (layout == "nn" and ldb < N) or (layout == "nt" and ldb < K):
        raise LaunchError("GEMM leading dimension smaller than the matrix")
    if layout == "nn" and N % 8:
        raise LaunchError("NN GEMM needs N to be a multiple of 8")
    if fp8 and layout == "nt" and (K % 16 or ldb % 16):
        raise LaunchError("NT GEMM with fp8 weights needs K and ldb to be multiples of 16 (16-byte rows)")
    balign = 8 if (fp8 and layout == "nn") else 16
    for p, al in ((a_ptr, 16), (b_ptr, balign), (up_ptr, balign), (ws_ptr, 16)):
        if p and p % al:
            raise LaunchError("GEMM operand pointer is not aligned for 128-bit access")
    if not ws_ptr:
        raise LaunchError("the split-K projection needs a workspace")
    if fp8 and not scale_ptr:
        raise LaunchError("fp8 weights need per-column scales")
    if swiglu and (fp8 != bool(up_scale_ptr)):
        raise LaunchError("SwiGLU with fp8 weights needs scales for both weights")
    if swiglu and (bias_ptr or resid_ptr or c_dtype != dt.bfloat16):
        raise LaunchError("the SwiGLU epilogue writes bf16 without bias / residual")
    ks, kc = gemv_split(M, N, K, layout, fp8)
    blocks = -(-N // 256) if layout == "nn" else -(-N // GEMV_NT_ROWS)
    if blocks * ks >= 2**31 or M * N >= 2**31:
        raise LaunchError("GEMM grid too large")
    flags = (GEMM_BIAS if bias_ptr else 0) | (GEMM_SCALE if scale_ptr else 0) | (GEMM_RESID if resid_ptr else 0)
    if round_before_bias and bias_ptr:
        flags |= GEMM_RND_BIAS
    if round_before_resid and resid_ptr:
        flags |= GEMM_RND_RESID
    args = GemvArgs(a_ptr, b_ptr, up_ptr or None, c_ptr, bias_ptr or None, scale_ptr or None,
                    up_scale_ptr or None, resid_ptr or None, ws_ptr, M, N, K, lda, ldb, ldc, ks, kc, flags, 0)
    mt = 1 if M == 1 else (4 if M <= 4 else 8)
    btag = "e4m3" if fp8 else "bf16"
    sw = "_swiglu" if swiglu else ""
    n_mm = 2 if swiglu else 1
    ctag = "bf16" if c_dtype == dt.bfloat16 else "f32"
    return [Launch("gemv", f"nk_gemv_{layout}_{btag}{sw}_m{mt}", (blocks * ks, 1, 1), (256, 1, 1), args,
                   bytes=M * K * 2 + n_mm * N * K * b_dtype.itemsize + 4 * ks * M * N * n_mm,
                   flops=2 * M * N * K * n_mm),
            Launch("gemv", f"nk_gemv_out_{ctag}{sw}", (-(-M * N // 64), 1, 1), (256, 1, 1), args,
                   bytes=4 * ks * M * N * n_mm + M * N * c_dtype.itemsize)]


GEMV_MFMA_MAX_M = 32
GEMV_MFMA_MAX_KC = 512  # A's rows of the range in LDS: 16 x 512 or 32 x 256
_GEMV_MFMA_TARGET_WGS = 512


def gemv_mfma_split(M: int, N: int, K: int, swiglu: bool = False):
    """(ksplit, kc) of :func:`gemv_mfma`: K ranges of 256 while the grid of
    column blocks (256 columns, 128 for the SwiGLU pair) x ksplit
    workgroups stays within one round of 512 (two per CU), else the
    shortest range (a multiple of 32, at most 512 for 16 rows, 256 for 32)
    that keeps it there.  Measured with cold weights: a second round of
    workgroups costs more than longer ranges do."""
    tiles = -(-N // (128 if swiglu else 256))
    kmax = GEMV_MFMA_MAX_KC if M <= 16 else GEMV_MFMA_MAX_KC // 2
    kc = 256
    ks = -(-K // kc)
    if tiles * ks > _GEMV_MFMA_TARGET_WGS:
        ks = max(1, _GEMV_MFMA_TARGET_WGS // tiles)
        kc = min(kmax, -(-(-(-K // ks)) // 32) * 32)
        ks = -(-K // kc)
    return ks, kc


def gemv_mfma_preferred(M: int, N: int, K: int, swiglu: bool = False, layout: str = "nn",
                        fp8: bool = False) -> bool:
    """Whether :func:`gemv_mfma` is the form for M rows (measured with cold
    weights at 4096 / 6144 / 24576 x 4096 and 4096 x 14336 against the VALU
    form and the MFMA GEMM over K ranges): bf16 NN weights up to 16 rows (at
    one row it ties the VALU form), NT weights (bf16 or fp8) from 2 to 16
    rows (one NT row streams faster on the VALU form), and 32 rows while
    ranges of 256 keep the grid within one round of workgroups.  No fp8 NN
    form."""
    if M <= 0 or (fp8 and layout == "nn") or (layout == "nt" and M == 1):
        return False
    if M <= 16:
        return True
    tiles = -(-N // (128 if swiglu else 256))
    return M <= GEMV_MFMA_MAX_M and tiles * -(-K // 256) <= _GEMV_MFMA_TARGET_WGS


def gemv_mfma_workspace_bytes(M: int, N: int, K: int, swiglu: bool = False) -> int:
    ks, _ = gemv_mfma_split(M, N, K, swiglu)
    return 4 * ks * M * N * (2 if swiglu else 1)


def gemv_mfma(a_ptr: int, b_ptr: int, c_ptr: int, M: int, N: int, K: int, *, c_dtype, ws_ptr: int,
              layout: str = "nn", b_dtype=dt.bfloat16, lda: int = None, ldb: int = None, ldc: int = None,
              bias_ptr: int = 0, scale_ptr: int = 0, resid_ptr: int = 0, up_ptr: int = 0, up_scale_ptr: int = 0,
              round_before_bias: bool = False, round_before_resid: bool = False) -> List[Launch]:
    """The operation of :func:`gemv` with the products on MFMA (16-row
    tiles, up to 32 rows): bf16 NN weights (K x N) through an LDS ring, or
    NT weights (N x K, bf16 or fp8 e4m3 with per-column scales) loaded
    straight into registers.  Partial sums over K ranges into the workspace
    at ``ws_ptr`` (``gemv_mfma_workspace_bytes``), then the reduction of
    :func:`gemv` (ranges added in order, then the epilogue; silu(x @ W) *
    (x @ U) with the up weights at ``up_ptr``, same layout and ``ldb``).
    Two launches."""
    if layout not in ("nn", "nt"):
        raise LaunchError(f"unknown GEMM layout {layout}")
    b_dtype, c_dtype = dt.canonical(b_dtype), dt.canonical(c_dtype)
    fp8 = b_dtype == dt.float8_e4m3fn
    if b_dtype != dt.bfloat16 and not (fp8 and layout == "nt"):
        raise LaunchError(f"the MFMA projection takes bf16 weights, or fp8 NT weights; got {dt.name(b_dtype)} "
                          f"{layout.upper()}")
    if c_dtype not in (dt.bfloat16, dt.float32):
        raise LaunchError(f"GEMM output must be bf16 or float32, got {dt.name(c_dtype)}")
    if not (0 < M <= GEMV_MFMA_MAX_M) or N <= 0 or K <= 0:
        raise LaunchError(f"the MFMA projection takes 1..{GEMV_MFMA_MAX_M} rows, got M={M} N={N} K={K}")
    lda = K if lda is None else lda
    ldb = (N if layout == "nn" else K) if ldb is None else ldb
    ldc = N if ldc is None else ldc
    swiglu = bool(up_ptr)
    if K % 8 or lda % 8 or ldb % 8 or (layout == "nn" and N % 8):
        raise LaunchError("the MFMA projection needs K, lda, ldb (and N for NN weights) to be multiples of 8")
    if fp8 and (K % 16 or ldb % 16):
        raise LaunchError("fp8 NT weights need K and ldb to be multiples of 16 (16-byte rows)")
    if lda < K or ldc < N or ldb < (N if layout == "nn" else K):
        raise LaunchError("GEMM leading dimension smaller than the matrix")
    for p, al in ((a_ptr, 16), (b_ptr, 16), (ws_ptr, 16)) + (((up_ptr, 16),) if swiglu else ()):
        if not p or p % al:
            raise LaunchError("GEMM operand, weight and workspace pointers must be aligned for 128-bit access")
    if fp8 and not scale_ptr:
        raise LaunchError("fp8 weights need per-column scales")
    if swiglu and (fp8 != bool(up_scale_ptr)):
        raise LaunchError("SwiGLU with fp8 weights needs scales for both weights")
    if swiglu and (bias_ptr or resid_ptr or c_dtype != dt.bfloat16):
        raise LaunchError("the SwiGLU epilogue writes bf16 without bias / residual")
    ks, kc = gemv_mfma_split(M, N, K, swiglu)
    if kc % 32 or kc > GEMV_MFMA_MAX_KC // (1 if M <= 16 else 2):
        raise LaunchError(f"K range of {kc} does not fit the MFMA projection")
    wbytes = kc * ldb * 2 if layout == "nn" else N * ldb * b_dtype.itemsize
    if wbytes >= 2**31 or M * lda * 2 >= 2**31 or M * N >= 2**31:
        raise LaunchError("the MFMA projection addresses its weights with 32-bit offsets")
    flags = (GEMM_BIAS if bias_ptr else 0) | (GEMM_SCALE if scale_ptr else 0) | (GEMM_RESID if resid_ptr else 0)
    if round_before_bias and bias_ptr:
        flags |= GEMM_RND_BIAS
    if round_before_resid and resid_ptr:
        flags |= GEMM_RND_RESID
    args = GemvArgs(a_ptr, b_ptr, up_ptr or None, c_ptr, bias_ptr or None, scale_ptr or None,
                    up_scale_ptr or None, resid_ptr or None, ws_ptr, M, N, K, lda, ldb, ldc, ks, kc, flags, 0)
    tiles = 1 if M <= 16 else 2
    n_mm = 2 if swiglu else 1
    sw = "_swiglu" if swiglu else ""
    btag = "e4m3" if fp8 else "bf16"
    ctag = "bf16" if c_dtype == dt.bfloat16 else "f32"
    blocks = -(-N // (128 if swiglu else 256))
    return [Launch("gemv", f"nk_gemv_mfma_{layout}_{btag}{sw}_t{tiles}", (blocks * ks, 1, 1), (256, 1, 1), args,
                   bytes=M * K * 2 + n_mm * N * K * b_dtype.itemsize + 4 * ks * M * N * n_mm,
                   flops=2 * M * N * K * n_mm),
            Launch("gemv", f"nk_gemv_out_{ctag}{sw}", (-(-M * N // 64), 1, 1), (256, 1, 1), args,
                   bytes=4 * ks * M * N * n_mm + M * N * c_dtype.itemsize)]


class HeadRopeTarget(ctypes.Structure):
    _fields_ = [("x", ctypes.c_void_p), ("out", ctypes.c_void_p), ("w", ctypes.c_void_p)] + \
        [(f"{t}_{s}", ctypes.c_int64) for t in "xo" for s in ("sb", "ss", "sh")] + \
        [("x_half", ctypes.c_int64), ("rows", ctypes.c_int64), ("blocks", ctypes.c_int64),
         ("o_sp", ctypes.c_int64), ("o_rows", ctypes.c_int64),
         ("eps", ctypes.c_float), ("H", ctypes.c_int32), ("flags", ctypes.c_int32), ("pad", ctypes.c_int32)]


class HeadRopeArgs(ctypes.Structure):
    _fields_ = [("t", HeadRopeTarget * 3), ("cos_t", ctypes.c_void_p), ("sin_t", ctypes.c_void_p),
                ("pos", ctypes.c_void_p), ("t_row", ctypes.c_int64), ("t_ss", ctypes.c_int64),
                ("t_rows", ctypes.c_int64), ("S", ctypes.c_int32), ("D", ctypes.c_int32),
                ("tflags", ctypes.c_int32), ("pad", ctypes.c_int32),
                ("plane", ctypes.c_int64), ("nplanes", ctypes.c_int32), ("pad2", ctypes.c_int32)]


HR_NORM, HR_MUL_RECIP, HR_W, HR_COPY, HR_PLANES = 1, 2, 4, 8, 16
HR_MAX_PLANES = 32  # partial-sum planes the head prologue adds itself
HR_TABLE_F32 = 1


@dataclass
class HeadRopeSpec:
    """One tensor of heads for :func:`head_rope`: bf16 rows of D elements at
    ``x_ptr`` through element strides (b, s, h), the second half of a row
    ``x_half`` elements after the first; rotated rows to ``out_ptr`` through
    ``out_strides``.  ``norm``: RMSNorm each row first (``eps``, optional
    bf16 weight at ``w_ptr``, ``mul_recip`` for the 1/sqrt form).  ``copy``:
    the rows unchanged instead (no norm, no rotation).  ``out_pos_stride``:
    the rows go to position pos (the runtime position, negative from the
    end, dropped outside ``out_positions``) of the output's position axis of
    that element stride (a cache write)."""
    x_ptr: int
    out_ptr: int
    H: int
    x_strides: tuple
    out_strides: tuple
    x_half: int
    norm: bool = False
    eps: float = 0.0
    w_ptr: int = 0
    mul_recip: bool = False
    copy: bool = False
    out_pos_stride: int = 0
    out_positions: int = 0


def head_rope(targets, cos_ptr: int, sin_ptr: int, B: int, S: int, D: int, *, table_f32: bool,
              pos_ptr: int = 0, table_row: int = 0, table_stride: int = 0, table_rows: int = 1,
              planes: Tuple[int, int] = None) -> Launch:
    """Per-head RMSNorm (optional) and split-half rotary embedding in bf16
    steps of one or two tensors of heads (q and k) sharing cos / sin tables:
    y = bf16(norm(x)); out = [bf16(bf16(y0 c) - bf16(y1 s)), bf16(bf16(y0 s)
    + bf16(y1 c))].  Tables are read at element ``row * table_row + s *
    table_stride + f`` (fp32 rounded to bf16 when ``table_f32``, else bf16),
    with row the int32 at ``pos_ptr`` (negative from the end, clamped into
    ``table_rows``) or 0.  ``planes = (plane, count)``: every target's x
    addresses fp32 partial sums of a few-row projection (``count`` planes of
    ``plane`` elements, the workspace of :func:`gemv_mfma` with ldc = N and
    no epilogue terms), which the kernel adds as ``nk_gemv_out_bf16`` does,
    so the projection's reduction launch is not needed."""
    targets = list(targets)
    if planes is not None and not (0 < int(planes[1]) <= HR_MAX_PLANES and int(planes[0]) > 0
                                   and int(planes[0]) % 8 == 0):
        raise LaunchError(f"head_rope adds 1..{HR_MAX_PLANES} partial-sum planes of a multiple of 8 elements, "
                          f"got {planes}")
    if not 1 <= len(targets) <= 3:
        raise LaunchError("head_rope takes one to three tensors of heads")
    if D % 16 or not 16 <= D <= 128:
        raise LaunchError(f"head_rope needs a head dim that is a multiple of 16 up to 128, got {D}")
    half = D // 2
    tw = 4 if table_f32 else 8  # table elements per 16 bytes
    if any(int(v) % tw for v in (table_row, table_stride)) or any(p % 16 for p in (cos_ptr, sin_ptr)):
        raise LaunchError("head_rope tables must keep 16-byte alignment")
    if pos_ptr and (pos_ptr % 4 or table_rows < 1):
        raise LaunchError("head_rope runtime position needs an aligned int32 and a table of rows")
    args = HeadRopeArgs()
    rows_all = 0
    for i, t in enumerate(targets):
        if any(int(v) % 8 for v in tuple(t.x_strides) + tuple(t.out_strides) + (t.x_half,)):
            raise LaunchError("head_rope strides must keep 16-byte alignment")
        if any(p % 16 for p in (t.x_ptr, t.out_ptr, t.w_ptr)):
            raise LaunchError("head_rope operands must be 16-byte aligned")
        rows = B * S * t.H
        rows_all += rows
        if rows <= 0:
            raise LaunchError("head_rope needs at least one row")
        if t.copy and t.norm:
            raise LaunchError("head_rope: a copied tensor is not normalised")
        if t.out_pos_stride and (not pos_ptr or t.out_positions < 1 or int(t.out_pos_stride) % 8):
            raise LaunchError("head_rope: a write at the runtime position needs the position, the output's "
                              "positions and an aligned stride")
        flags = (HR_NORM if t.norm else 0) | (HR_MUL_RECIP if t.norm and t.mul_recip else 0) | \
            (HR_W if t.norm and t.w_ptr else 0) | (HR_COPY if t.copy else 0) | (HR_PLANES if planes else 0)
        args.t[i] = HeadRopeTarget(t.x_ptr, t.out_ptr, t.w_ptr or None, *[int(v) for v in t.x_strides],
                                   *[int(v) for v in t.out_strides], int(t.x_half), rows, -(-rows // 16),
                                   int(t.out_pos_stride), int(t.out_positions), float(t.eps), int(t.H), flags, 0)
    if rows_all >= 2**31:
        raise LaunchError("head_rope: too many rows for one launch")
    args.cos_t, args.sin_t, args.pos = cos_ptr, sin_ptr, pos_ptr or None
    args.t_row, args.t_ss, args.t_rows = int(table_row), int(table_stride), int(table_rows)
    args.S, args.D, args.tflags = S, D, HR_TABLE_F32 if table_f32 else 0
    if planes is not None:
        args.plane, args.nplanes = int(planes[0]), int(planes[1])
    blocks = sum(int(args.t[i].blocks) for i in range(len(targets)))
    tb = 4 if table_f32 else 2
    xb = 4 * int(planes[1]) if planes is not None else 2
    return Launch("rope", "nk_head_rope_bf16", (blocks, 1, 1), (256, 1, 1), args,
                  bytes=rows_all * D * (xb + 2) + 2 * S * half * tb,
                  flops=rows_all * D * (6 + (4 if any(t.norm for t in targets) else 0)))


# ---------------------------------------------------------------------------
# Chunked causal linear attention (csrc/kernels/linattn.hip)
# ---------------------------------------------------------------------------
class LinAttnArgs(ctypes.Structure):
    _fields_ = [("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
                ("o", ctypes.c_void_p), ("part", ctypes.c_void_p), ("BH", ctypes.c_int64),
                ("T", ctypes.c_int64), ("nseg", ctypes.c_int32), ("rchunks", ctypes.c_int32),
                ("vmax", ctypes.c_void_p)]


class LinAttnStateArgs(ctypes.Structure):
    _fields_ = [("k", ctypes.c_void_p), ("v", ctypes.c_void_p), ("part", ctypes.c_void_p),
                ("BH", ctypes.c_int64), ("T", ctypes.c_int64), ("nranges", ctypes.c_int32),
                ("rchunks", ctypes.c_int32), ("vmax", ctypes.c_void_p)]


LINATTN_CHUNK = 64
LINATTN_D = 128
# the scan is serial over a sequence's chunks; with fewer than this many
# workgroups the sequence is cut into segments whose prefix states come from
# a separate partial-sum kernel
LINATTN_TARGET_WGS = 256


def linear_attention_split(BH: int, T: int, ranges_per_segment: int = None):
    """(segments per sequence, chunks per partial-sum range, ranges) for the
    linear-attention scan of BH sequences of length T; ``ranges_per_segment``
    (1, 2 or 4) overrides the partial-sum range policy."""
    nchunks = T // LINATTN_CHUNK
    nseg = 1
    while (BH * nseg < LINATTN_TARGET_WGS and nchunks % (2 * nseg) == 0
           and nchunks // (2 * nseg) >= 8):
        nseg *= 2
    cs = nchunks // nseg
    # One partial sum per earlier segment when that already occupies 3/4 of
    # the CUs: the partial-sum kernel runs one workgroup per CU with a deep
    # prefetch, so fewer, longer ranges beat a second round of workgroups
    # (and halve the partial-state traffic); else halves or quarters.
    wgs = BH * (nseg - 1)
    if ranges_per_segment is not None:
        if ranges_per_segment not in (1, 2, 4) or cs % ranges_per_segment:
            raise LaunchError(f"{ranges_per_segment} ranges per segment of {cs} chunks")
        rchunks = cs // ranges_per_segment
    elif cs % 4 or 4 * wgs >= 3 * LINATTN_TARGET_WGS:
        rchunks = cs
    elif 2 * wgs >= LINATTN_TARGET_WGS:
        rchunks = cs // 2
    else:
        rchunks = cs // 4
    nranges = (nseg - 1) * (cs // rchunks)
    return nseg, rchunks, nranges


def linear_attention_workspace_bytes(BH: int, T: int, ranges_per_segment: int = None) -> int:
    """Device workspace (fp32 partial prefix states) the launch needs; 0 if
    the sequences run unsegmented."""
    _, _, nranges = linear_attention_split(BH, T, ranges_per_segment)
    return BH * nranges * (LINATTN_D + 1) * LINATTN_D * 4


# The fp16 operand window of the kernel (csrc/kernels/linattn.hip): a
# sequence whose largest |v| is below 2^-13 has its V and S / 256 operands
# in the fp16 subnormal range (relative precision lost); 65536 and above
# overflow fp16.  bf16 bit patterns of those bounds:
LINATTN_VMAX_LOW_BITS = 0x3900   # 2^-13
LINATTN_VMAX_HIGH_BITS = 0x4780  # 65536 (the first bf16 value fp16 cannot hold)


def linear_attention(q_ptr: int, k_ptr: int, v_ptr: int, o_ptr: int, BH: int, T: int,
                     D: int = 128, Dv: int = 128, chunk: int = 64, part_ptr: int = 0,
                     ranges_per_segment: int = None, vmax_ptr: int = 0) -> List[Launch]:
    """o = causal linear attention with phi = elu + 1 over (BH, T, D) bf16
    sequences, chunk 64, head dims 128 (the compiled variant).

    Returns the launches in order: when the sequences are cut into segments,
    a partial-sum kernel writes the prefix states into ``part_ptr`` (a
    workspace of :func:`linear_attention_workspace_bytes` bytes) before the
    scan reads them.  With ``vmax_ptr`` (BH uint32 words) the scan writes
    each sequence's max |v| as bf16 bits there, for
    :func:`check_linear_attention_vmax` after the launches complete."""
    if (D, Dv, chunk) != (LINATTN_D, LINATTN_D, LINATTN_CHUNK):
        raise LaunchError(f"linear attention kernel is built for d = d_v = 128, chunk 64; "
                          f"got d={D}, d_v={Dv}, chunk={chunk}")
    if BH <= 0 or T <= 0 or T % chunk:
        raise LaunchError(f"linear attention needs T a positive multiple of {chunk}, got T={T}")
    if any(p % 16 for p in (q_ptr, k_ptr, v_ptr, o_ptr)):
        raise LaunchError("linear attention operands must be 16-byte aligned")
    nseg, rchunks, nranges = linear_attention_split(BH, T, ranges_per_segment)
    if BH * nseg >= 2**31 or BH * max(nranges, 1) >= 2**31:
        raise LaunchError("linear attention grid too large")
    if nranges and not part_ptr:
        raise LaunchError(f"linear attention of {BH} x {T} runs in {nseg} segments and needs a "
                          f"workspace of {linear_attention_workspace_bytes(BH, T, ranges_per_segment)} bytes")
    if part_ptr % 16:
        raise LaunchError("linear attention workspace must be 16-byte aligned")
    if vmax_ptr % 4:
        raise LaunchError("linear attention max |v| words must be 4-byte aligned")
    n = T // chunk
    flops_chunk = 2 * chunk * chunk * D + 2 * chunk * D * Dv + 2 * chunk * chunk * Dv + 2 * D * Dv * chunk
    launches = []
    if nranges:
        launches.append(Launch("linattn", "nk_linattn_state_c64_d128", (BH * nranges, 1, 1),
                               (512, 1, 1),
                               LinAttnStateArgs(k_ptr, v_ptr, part_ptr, BH, T, nranges, rchunks, vmax_ptr or None),
                               bytes=2 * BH * nranges * rchunks * chunk * D * 2,
                               flops=BH * nranges * rchunks * 2 * chunk * D * Dv))
    launches.append(Launch("linattn", "nk_linattn_c64_d128", (BH * nseg, 1, 1), (512, 1, 1),
                           LinAttnArgs(q_ptr, k_ptr, v_ptr, o_ptr, part_ptr or None, BH, T, nseg, rchunks,
                                       vmax_ptr or None),
                           bytes=4 * BH * T * D * 2, flops=BH * n * flops_chunk))
    return launches


class LinearAttentionRangeError(ValueError):
    """Values of v outside the fp16 operand window of the linear-attention
    kernel: the result is not within the kernel's accuracy."""


def check_linear_attention_vmax(words: np.ndarray, what: str = "linear attention"):
    """Raise LinearAttentionRangeError naming the sequences whose max |v|
    (bf16 bits, as the scan reports them) lies outside the kernel's fp16
    operand window.  All-zero sequences are exact (o = 0) and pass."""
    bits = np.asarray(words, np.uint32)
    low = np.nonzero((bits > 0) & (bits < LINATTN_VMAX_LOW_BITS))[0]
    high = np.nonzero(bits >= LINATTN_VMAX_HIGH_BITS)[0]
    if not len(low) and not len(high):
        return
    val = lambda b: float(np.array([int(b) << 16], np.uint32).view(np.float32)[0])
    parts = []
    if len(low):
        parts.append(f"{len(low)} sequence(s) (first: {int(low[0])}, max |v| {val(bits[low[0]]):.3g}) have max |v| "
                     f"below 2^-13, where v and the running state go subnormal in the kernel's fp16 operands")
    if len(high):
        parts.append(f"{len(high)} sequence(s) (first: {int(high[0])}, max |v| {val(bits[high[0]]):.3g}) have |v| "
                     f"of 65536 or more (or non-finite), beyond fp16")
    raise LinearAttentionRangeError(
        f"{what}: " + "; ".join(parts) + ". The output is linear in v: scale v by a power of two "
        "into the window and the output back.")


# ---------------------------------------------------------------------------
# Causal GQA attention (csrc/kernels/attention.hip)
# ---------------------------------------------------------------------------
class AttnArgs(ctypes.Structure):
    _fields_ = [("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
                ("o", ctypes.c_void_p)] + \
        [(f"{t}_{s}", ctypes.c_int64) for t in "qkvo" for s in ("sb", "ss", "sh")] + \
        [("B", ctypes.c_int32), ("S", ctypes.c_int32), ("Hq", ctypes.c_int32),
         ("Hkv", ctypes.c_int32), ("scale", ctypes.c_float), ("causal", ctypes.c_int32),
         ("div", ctypes.c_float), ("rdiv", ctypes.c_float), ("flags", ctypes.c_int32),
         ("rowstat", ctypes.c_void_p), ("ckb", ctypes.c_int32), ("nch", ctypes.c_int32)]


# score cast points of the traced code before its softmax, and its softmax in
# bf16 (the values of the decode kernel's DEC_* flags)
ATT_RND_PROD, ATT_RND_SCORE, ATT_SOFTMAX_BF16, ATT_DIVIDE = 1, 2, 4, 8


@functools.lru_cache(maxsize=64)
def divide_rounds_as_multiply(div: float) -> bool:
    """Whether bf16(RN(s / div)) == bf16(RN(s * RN(1 / div))) for every
    finite bf16 s, checked over all of them: then a score divided by ``div``
    and rounded to bf16 needs no correctly rounded quotient, the product by
    the reciprocal rounds to the same bf16 value."""
    s = (np.arange(1 << 16, dtype=np.uint32) << 16).view(np.float32)
    s = s[np.isfinite(s)]
    d = np.float32(div)
    with np.errstate(over="ignore", under="ignore"):
        return bool(np.array_equal(dt.round_to_bf16(s / d), dt.round_to_bf16(s * (np.float32(1) / d))))


def attention_stat_chunks(S: int, causal: bool = True):
    """Key chunks of the bf16 softmax's row statistics: (32-key blocks per
    chunk, most chunks of a query block, chunks summed over the S / 128
    query blocks).  Chunks of 512 keys, or of S / 8 rounded up to 128 keys
    when S passes 4096, so a row has at most 8."""
    ckb = 4 * max(4, -(-S // 1024))
    per_qb = [-(-((qb + 1) * 4 if causal else S // 32) // ckb) for qb in range(S // 128)]
    return ckb, max(per_qb), sum(per_qb)


def attention_rowstat_bytes(B: int, S: int, Hq: int, causal: bool = True) -> int:
    """Workspace of the bf16 softmax (ATT_SOFTMAX_BF16): per query and key
    chunk, the max score and the sum of the weights, as fp32."""
    return 2 * 4 * attention_stat_chunks(S, causal)[1] * B * Hq * S


def attention(q_ptr: int, k_ptr: int, v_ptr: int, o_ptr: int, B: int, S: int, Hq: int, Hkv: int,
              D: int, scale: float, strides: dict, causal: bool = True, waves: int = None,
              key_block: int = None, ring: bool = None, score_flags: int = 0,
              divisor: float = None, rowstat_ptr: int = 0):
    """Flash-style attention over bf16 q (B, S, Hq, D), k / v (B, S, Hkv, D) and
    o (B, S, Hq, D), each addressed by element strides {"q": (sb, ss, sh), ...}
    with the head dim contiguous.  KV head of query head h is h // (Hq // Hkv).
    ``waves`` (4 or 8) waves of 32 queries share a workgroup's K / V tiles;
    ``key_block`` (64 or 32) keys per step.  Variants: (4, 64), (8, 64) and
    (4, 32), the last with three workgroups per CU; ``ring`` selects the
    software-pipelined (4, 32) kernel over a four-slot K / V ring.

    ``score_flags`` (ATT_*) give each score the traced code's cast points
    before the softmax: ATT_RND_PROD rounds q.k to bf16, ATT_DIVIDE divides
    by ``divisor`` (fp32, correctly rounded quotient) instead of multiplying
    by ``scale``, ATT_RND_SCORE rounds the scaled score to bf16.  Any flag
    selects the ring kernel's score-transform variant (4 waves).

    ATT_SOFTMAX_BF16 (with ATT_RND_SCORE) runs the softmax with the bf16
    cast points of the traced code (examples/models/qwen3/kernels/
    softmax.py:4-6 on bf16 scores): d = bf16(s - max), e = bf16(exp d),
    l = bf16(sum e), p = bf16(e / l), o = bf16(sum p v).  It takes three
    launches over the keys (the row max and the row sum, each over key
    chunks, then the weighted values) sharing a workspace of
    ``attention_rowstat_bytes`` at ``rowstat_ptr``; the result is then a
    list of three launches instead of one launch."""
    if D != 128:
        raise LaunchError(f"attention kernel is built for head_dim 128, got {D}")
    if S % 128 or S <= 0:
        raise LaunchError(f"attention needs the sequence length to be a multiple of 128, got {S}")
    if Hq % Hkv:
        raise LaunchError("query heads must be a multiple of KV heads")
    for name in "qkvo":
        st = strides[name]
        if any(s % 8 for s in st):
            raise LaunchError("attention strides must keep 16-byte alignment")
    for p in (q_ptr, k_ptr, v_ptr, o_ptr):
        if p % 16:
            raise LaunchError("attention operands must be 16-byte aligned")
    if not scale > 0:
        raise LaunchError("attention kernel needs a positive score scale")
    if S * max(strides["k"][1], strides["v"][1], 128) * 2 >= 2**31:
        raise LaunchError("attention K / V rows of one sequence must span less than 2 GiB")
    if score_flags & ~(ATT_RND_PROD | ATT_RND_SCORE | ATT_SOFTMAX_BF16 | ATT_DIVIDE):
        raise LaunchError(f"unknown attention score flags {score_flags:#x}")
    smx_bf16 = bool(score_flags & ATT_SOFTMAX_BF16)
    if smx_bf16:
        if not score_flags & ATT_RND_SCORE:
            raise LaunchError("the bf16 softmax runs on scores rounded to bf16 (ATT_RND_SCORE)")
        if not rowstat_ptr or rowstat_ptr % 4:
            raise LaunchError("the bf16 softmax needs a 4-byte aligned row statistics workspace")
    vals = [q_ptr, k_ptr, v_ptr, o_ptr]
    for name in "qkvo":
        vals += list(strides[name])
    div = np.float32(1.0)
    if score_flags & ATT_DIVIDE:
        div = np.float32(divisor if divisor is not None else 1.0 / scale)
        if not (np.isfinite(div) and div > 0):
            raise LaunchError("attention score divisor must be finite and positive")
        # a quotient rounded to bf16 right away: the product by RN(1 / div)
        # when it gives the same bf16 score for every bf16 product
        if score_flags & ATT_RND_SCORE and divide_rounds_as_multiply(float(div)):
            score_flags &= ~ATT_DIVIDE
            scale = float(np.float32(1) / div)
    ckb, nch, items_per_head = attention_stat_chunks(S, causal) if smx_bf16 else (0, 0, 0)
    args = AttnArgs(*vals, B, S, Hq, Hkv, float(scale), 1 if causal else 0, float(div),
                    float(np.float32(1.0) / np.float32(div)), int(score_flags), int(rowstat_ptr), ckb, nch)
    if score_flags:
        if (waves or 4, key_block or 32, True if ring is None else ring) != (4, 32, True):
            raise LaunchError("attention score cast points exist on the 4-wave ring kernel only")
        waves, key_block, ring = 4, 32, True
    # default: 4 waves, 32-key blocks (three workgroups per CU); measured at
    # (8, 2048, 32 / 8 heads) 319.5 us mean of eight runs against 328 us for
    # (4, 64) and 326 us for (8, 64)
    waves = 4 if waves is None else waves
    key_block = 32 if key_block is None else key_block
    # default: the ring kernel (4 waves, 32-key blocks, software pipelined
    # over a four-slot K / V ring); explicit (waves, key_block) pick the others
    ring = (waves, key_block) == (4, 32) if ring is None else ring
    if ring and (waves, key_block) not in ((4, 32), (8, 32)):
        raise LaunchError("the ring attention kernels run 4 or 8 waves over 32-key blocks")
    suffix = {4: "_sp", 8: "_sp8"}[waves] if ring else {(4, 64): "", (8, 64): "_w8", (4, 32): "_k32"}.get(
        (waves, key_block))
    if suffix is None:
        raise LaunchError(f"no attention variant with {waves} waves and {key_block}-key blocks")
    if S % (32 * waves):
        raise LaunchError(f"attention with {waves} waves needs S to be a multiple of {32 * waves}")
    nblocks = B * Hq * (S // (32 * waves))
    if nblocks >= 2**31:
        raise LaunchError("attention grid too large")
    flops = 4 * B * Hq * S * S * D // (2 if causal else 1)
    sym = "nk_attention_causal_d128" + suffix + ("_xf" if score_flags else "")
    if smx_bf16:
        qk_bytes = (B * S * Hq * D + B * S * Hkv * D) * 2
        stat = 4 * nch * B * Hq * S
        nstat = B * Hq * items_per_head
        if nstat >= 2**31:
            raise LaunchError("attention statistics grid too large")
        return [Launch("attention", "nk_attention_rowmax_d128", (nstat, 1, 1), (256, 1, 1), args,
                       bytes=qk_bytes + stat, flops=flops // 2),
                Launch("attention", "nk_attention_rowsum_d128", (nstat, 1, 1), (256, 1, 1), args,
                       bytes=qk_bytes + 2 * stat, flops=flops // 2),
                Launch("attention", sym + "_bf16", (nblocks, 1, 1), (64 * waves, 1, 1), args,
                       bytes=(2 * B * S * Hq * D + 2 * B * S * Hkv * D) * 2 + 2 * stat, flops=flops)]
    return Launch("attention", sym, (nblocks, 1, 1), (64 * waves, 1, 1), args,
                  bytes=(2 * B * S * Hq * D + 2 * B * S * Hkv * D) * 2, flops=flops)


class DecodeAttnArgs(ctypes.Structure):
    _fields_ = [("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
                ("o", ctypes.c_void_p), ("pos", ctypes.c_void_p)] + \
        [(f"{t}_{s}", ctypes.c_int64) for t, ss in (("q", "bh"), ("k", "bsh"), ("v", "bsh"), ("o", "bh"))
         for s in {"bh": ("sb", "sh"), "bsh": ("sb", "ss", "sh")}[ss]] + \
        [("B", ctypes.c_int32), ("Smax", ctypes.c_int32), ("Hq", ctypes.c_int32), ("Hkv", ctypes.c_int32),
         ("scale", ctypes.c_float), ("flags", ctypes.c_int32), ("ws", ctypes.c_void_p),
         ("nsplit", ctypes.c_int32)]


DEC_RND_PROD, DEC_RND_SCORE, DEC_SOFTMAX_BF16, DEC_DIVIDE = 1, 2, 4, 8
DEC_MAX_REP = 16
DEC_SPLIT = 128  # keys per split


def decode_attention_workspace_bytes(B: int, Smax: int, Hq: int) -> int:
    """Workspace of the decode step (fp32): the scores of every cache
    position, each split's max, each split's partial output and the row's
    max and weight sum, for every query head."""
    nsplit = -(-Smax // DEC_SPLIT)
    return 4 * B * Hq * (Smax + nsplit + nsplit * 128 + 2)


def decode_attention(q_ptr: int, k_ptr: int, v_ptr: int, o_ptr: int, pos_ptr: int, B: int, Smax: int,
                     Hq: int, Hkv: int, D: int, scale: float, strides: dict, flags: int = 0,
                     ws_ptr: int = 0) -> List[Launch]:
    """One query token per sequence against a bf16 KV cache: q (B, Hq, D),
    k / v cache (B, Smax, Hkv, D) and o (B, Hq, D) through element strides
    {"q": (sb, sh), "k": (sb, ss, sh), "v": (sb, ss, sh), "o": (sb, sh)}
    with d contiguous; keys 0..pos attend, pos an int32 in device memory.
    ``flags``: DEC_RND_PROD / DEC_RND_SCORE round the product / the scaled
    score to bf16, DEC_SOFTMAX_BF16 rounds every softmax result to bf16,
    DEC_DIVIDE divides by ``scale`` instead of multiplying.

    Four launches over splits of DEC_SPLIT cache positions (scores and
    split maxima, each row's max and weight sum, per-split weighted values,
    their sum in split order) sharing a workspace of
    ``decode_attention_workspace_bytes`` at ``ws_ptr``."""
    if D != 128:
        raise LaunchError(f"decode attention kernel is built for head_dim 128, got {D}")
    if Hkv <= 0 or Hq % Hkv:
        raise LaunchError("query heads must be a multiple of KV heads")
    rep = Hq // Hkv
    if rep > DEC_MAX_REP:
        raise LaunchError(f"decode attention serves at most {DEC_MAX_REP} query heads per KV head")
    if Smax <= 0 or Smax >= 2**31 - DEC_SPLIT:
        raise LaunchError(f"decode attention cache length out of range: {Smax}")
    if not ws_ptr or ws_ptr % 16:
        raise LaunchError("decode attention needs a 16-byte aligned workspace")
    if any(int(x) % 8 for x in tuple(strides["k"]) + tuple(strides["v"])) or k_ptr % 16 or v_ptr % 16:
        raise LaunchError("decode attention K / V rows must be 16-byte aligned")
    if q_ptr % 2 or o_ptr % 2 or pos_ptr % 4 or not pos_ptr:
        raise LaunchError("decode attention operands are misaligned")
    if not scale > 0:
        raise LaunchError("decode attention needs a positive score scale")
    nsplit = -(-Smax // DEC_SPLIT)
    if B * Hkv * nsplit >= 2**31 or B * Hq >= 2**31:
        raise LaunchError("decode attention grid too large")
    rounded = DEC_RND_PROD | DEC_RND_SCORE
    if flags & DEC_DIVIDE and flags & rounded == rounded and divide_rounds_as_multiply(scale):
        # a bf16 product divided and rounded to bf16 equals its product by
        # RN(1 / scale) rounded to bf16, for every bf16 product (checked)
        scale = float(np.float32(1) / np.float32(scale))
        flags &= ~DEC_DIVIDE
    args = DecodeAttnArgs(q_ptr, k_ptr, v_ptr, o_ptr, pos_ptr, *strides["q"], *strides["k"], *strides["v"],
                          *strides["o"], B, Smax, Hq, Hkv, float(scale), int(flags), int(ws_ptr), nsplit)
    kv = B * Smax * Hkv * D * 2  # one cache's bytes (an upper bound: keys past pos are not read)
    sc = 4 * B * Hq * Smax
    rt = next(r for r in (1, 2, 4, 8, 16) if r >= rep)  # kernels for up to rt queries per KV head
    return [Launch("attention", f"nk_decode_scores_d128_r{rt}", (B * Hkv * nsplit, 1, 1), (256, 1, 1), args,
                   bytes=kv + B * Hq * D * 2 + sc, flops=2 * B * Hq * Smax * D),
            Launch("attention", "nk_decode_rowstat_d128", (B * Hq, 1, 1), (256, 1, 1), args, bytes=sc),
            Launch("attention", f"nk_decode_values_d128_r{rt}", (B * Hkv * nsplit, 1, 1), (256, 1, 1), args,
                   bytes=kv + sc + 4 * B * Hq * nsplit * D, flops=2 * B * Hq * Smax * D),
            Launch("attention", "nk_decode_combine_d128", (B * Hq, 1, 1), (128, 1, 1), args,
                   bytes=4 * B * Hq * nsplit * D + B * Hq * D * 2)]


# ---------------------------------------------------------------------------
# Rotary position embedding (csrc/kernels/rope.hip)
# ---------------------------------------------------------------------------
class RopeArgs(ctypes.Structure):
    _fields_ = [("x", ctypes.c_void_p), ("cos_t", ctypes.c_void_p), ("sin_t", ctypes.c_void_p),
                ("out", ctypes.c_void_p)] + \
        [(f"{t}_{s}", ctypes.c_int64) for t in "xo" for s in ("sb", "ss", "sh")] + \
        [("x_half", ctypes.c_int64), ("t_ss", ctypes.c_int64), ("groups", ctypes.c_int64),
         ("S", ctypes.c_int32), ("H", ctypes.c_int32), ("half", ctypes.c_int32),
         ("nthreads", ctypes.c_int32)]


def rope(x_ptr: int, cos_ptr: int, sin_ptr: int, out_ptr: int, B: int, S: int, H: int, D: int,
         x_strides, out_strides, x_half: int, table_stride: int) -> Launch:
    """Split-half rotary embedding of bf16 x (B, S, H, D) read through element
    strides (sb, ss, sh) with d contiguous, the second half ``x_half``
    elements after the first; fp32 cos / sin tables indexed [s * table_stride
    + d]; bf16 out through ``out_strides``."""
    if D % 16 or D <= 0:
        raise LaunchError(f"rope needs the head dim to be a multiple of 16, got {D}")
    half = D // 2
    if any(int(s) % 8 for s in tuple(x_strides) + tuple(out_strides) + (x_half,)):
        raise LaunchError("rope strides must keep 16-byte alignment")
    if table_stride % 4 or table_stride < half:
        raise LaunchError("rope tables need a row stride that is a multiple of 4 and covers D/2")
    if any(p % 16 for p in (x_ptr, cos_ptr, sin_ptr, out_ptr)):
        raise LaunchError("rope operands must be 16-byte aligned")
    groups = B * S * H * (half // 8)
    blocks = max(1, min((groups + 255) // 256, 65536))
    args = RopeArgs(x_ptr, cos_ptr, sin_ptr, out_ptr, *[int(s) for s in x_strides],
                    *[int(s) for s in out_strides], int(x_half), int(table_stride), groups,
                    S, H, half, blocks * 256)
    return Launch("rope", "nk_rope_bf16", (blocks, 1, 1), (256, 1, 1), args,
                  bytes=2 * B * S * H * D * 2 + 2 * S * half * 4, flops=6 * B * S * H * half)
