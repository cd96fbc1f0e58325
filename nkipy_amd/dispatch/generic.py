"""Generic lowering of graph nodes that no fused kernel pattern covers.

Elementwise and layout nodes are fused into *programs* for the
``nk_ew_program`` kernel.  A program is evaluated over the index space of
the value it produces; layout ops between a producer and its consumer are
affine index maps (broadcast, transpose, slice, reverse, size-1 reshapes),
so they compose into the load strides of the program's inputs instead of
being materialised.  Reductions and dots likewise read their operands
through composed strides.  Everything else (gather/scatter, cumsum,
concatenate, pad, dynamic-update-slice) has a small dedicated step.
"""

from __future__ import annotations

import ctypes
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

from nkipy_amd.core import dtypes as dt
from nkipy_amd.core.backend.ir import Value
from nkipy_amd.dispatch.launchers import Launch, LaunchError
from nkipy_amd.dispatch.plan import Step

# ---------------------------------------------------------------------------
# dtype codes and op codes shared with csrc/kernels/generic.hip
# ---------------------------------------------------------------------------
DT_CODE = {
    dt.float32: 0, dt.float16: 1, dt.bfloat16: 2, dt.float8_e4m3fn: 3, dt.int8: 4,
    dt.int16: 5, dt.int32: 6, dt.int64: 7, dt.uint8: 8, dt.uint16: 9, dt.uint32: 10,
    dt.uint64: 11, dt.bool_: 12, dt.float64: 13,
}

OP_LOAD, OP_CONST, OP_IOTA = 0, 1, 2
UNARY_CODES = {
    "negate": 10, "abs": 11, "exponential": 12, "log": 13, "sqrt": 14, "rsqrt": 15,
    "sine": 16, "cosine": 17, "tan": 18, "atan": 19, "tanh": 20, "ceil": 21, "floor": 22,
    "round_nearest_even": 23, "trunc": 24, "sign": 25, "not": 26, "log_plus_one": 27,
    "exponential_minus_one": 28, "is_finite": 29, "is_nan": 30, "logistic": 31, "log2": 32,
    "convert": 33, "copy": 33,
}
BINARY_CODES = {
    "add": 40, "subtract": 41, "multiply": 42, "divide": 43, "power": 44, "maximum": 45,
    "minimum": 46, "and": 47, "or": 48, "xor": 49, "remainder": 50, "floor_divide": 51,
    "atan2": 52,
}
COMPARE_CODES = {"EQ": 60, "NE": 61, "LT": 62, "LE": 63, "GT": 64, "GE": 65}
OP_SELECT = 70

EW_OPS = set(UNARY_CODES) | set(BINARY_CODES) | {"compare", "select", "iota"}
LAYOUT_OPS = {"broadcast_in_dim", "transpose", "slice", "reverse"}

EW_MAX_RANK = 6
EW_MAX_IN = 8
EW_MAX_INSTR = 40
EW_REGS = 16
RED_MAX_RANK = 6


def dtype_code(d) -> int:
    d = dt.canonical(d)
    if d not in DT_CODE:
        raise LaunchError(f"dtype {dt.name(d)} is not supported by the generic kernels")
    return DT_CODE[d]


def contiguous_strides(shape) -> np.ndarray:
    s = np.ones(len(shape), dtype=np.int64)
    for i in range(len(shape) - 2, -1, -1):
        s[i] = s[i + 1] * shape[i + 1]
    return s


# ---------------------------------------------------------------------------
# ctypes mirrors of the kernel argument structs
# ---------------------------------------------------------------------------
class EwInput(ctypes.Structure):
    _fields_ = [("ptr", ctypes.c_void_p), ("strides", ctypes.c_int64 * EW_MAX_RANK),
                ("dtype", ctypes.c_int32), ("pad", ctypes.c_int32)]


class EwInstr(ctypes.Structure):
    _fields_ = [("op", ctypes.c_int16), ("dst", ctypes.c_int8), ("a", ctypes.c_int8),
                ("b", ctypes.c_int8), ("c", ctypes.c_int8), ("dtype", ctypes.c_int8),
                ("flags", ctypes.c_int8), ("imm", ctypes.c_double)]


class EwArgs(ctypes.Structure):
    _fields_ = [
        ("out", ctypes.c_void_p), ("out_offset", ctypes.c_int64),
        ("out_strides", ctypes.c_int64 * EW_MAX_RANK), ("shape", ctypes.c_int64 * EW_MAX_RANK),
        ("total", ctypes.c_int64), ("rank", ctypes.c_int32), ("n_in", ctypes.c_int32),
        ("n_instr", ctypes.c_int32), ("out_dtype", ctypes.c_int32),
        ("result_reg", ctypes.c_int32), ("pad", ctypes.c_int32), ("nthreads", ctypes.c_int64),
        ("inp", EwInput * EW_MAX_IN), ("prog", EwInstr * EW_MAX_INSTR),
    ]


class ReduceArgs(ctypes.Structure):
    _fields_ = [
        ("inp", ctypes.c_void_p), ("out", ctypes.c_void_p),
        ("out_shape", ctypes.c_int64 * RED_MAX_RANK), ("out_strides", ctypes.c_int64 * RED_MAX_RANK),
        ("red_shape", ctypes.c_int64 * RED_MAX_RANK), ("red_strides", ctypes.c_int64 * RED_MAX_RANK),
        ("n_out", ctypes.c_int64), ("n_red", ctypes.c_int64),
        ("out_rank", ctypes.c_int32), ("red_rank", ctypes.c_int32), ("op", ctypes.c_int32),
        ("in_dtype", ctypes.c_int32), ("out_dtype", ctypes.c_int32), ("acc_f32", ctypes.c_int32),
    ]


class DotArgs(ctypes.Structure):
    _fields_ = [
        ("A", ctypes.c_void_p), ("B", ctypes.c_void_p), ("C", ctypes.c_void_p),
        ("batch", ctypes.c_int64), ("M", ctypes.c_int64), ("N", ctypes.c_int64), ("K", ctypes.c_int64),
        ("sab", ctypes.c_int64), ("sam", ctypes.c_int64), ("sak", ctypes.c_int64),
        ("sbb", ctypes.c_int64), ("sbk", ctypes.c_int64), ("sbn", ctypes.c_int64),
        ("a_dtype", ctypes.c_int32), ("b_dtype", ctypes.c_int32), ("c_dtype", ctypes.c_int32),
        ("pad", ctypes.c_int32),
    ]


class GatherArgs(ctypes.Structure):
    _fields_ = [
        ("src", ctypes.c_void_p), ("idx", ctypes.c_void_p), ("out", ctypes.c_void_p),
        ("O", ctypes.c_int64), ("A", ctypes.c_int64), ("I", ctypes.c_int64), ("N", ctypes.c_int64),
        ("nthreads", ctypes.c_int64), ("mode", ctypes.c_int32), ("dtype", ctypes.c_int32),
    ]


class CumsumArgs(ctypes.Structure):
    _fields_ = [
        ("inp", ctypes.c_void_p), ("out", ctypes.c_void_p),
        ("O", ctypes.c_int64), ("A", ctypes.c_int64), ("N", ctypes.c_int64),
        ("in_dtype", ctypes.c_int32), ("out_dtype", ctypes.c_int32),
        ("acc_f32", ctypes.c_int32), ("pad", ctypes.c_int32),
    ]


class Copy16Args(ctypes.Structure):
    _fields_ = [("src", ctypes.c_void_p), ("dst", ctypes.c_void_p),
                ("n16", ctypes.c_int64), ("nthreads", ctypes.c_int64)]


def copy16(src_ptr: int, dst_ptr: int, nbytes: int) -> Launch:
    """Streaming device copy of ``nbytes`` (multiple of 16, 16-byte aligned)."""
    if nbytes % 16 or src_ptr % 16 or dst_ptr % 16:
        raise LaunchError("copy16 needs 16-byte aligned pointers and a multiple of 16 bytes")
    n16 = nbytes // 16
    grid = max(1, min((n16 + 255) // 256, 1 << 20))
    return Launch("generic", "nk_copy16", (grid, 1, 1), (256, 1, 1),
                  Copy16Args(src_ptr, dst_ptr, n16, grid * 256), bytes=2 * nbytes)


class DecodeE4m3Args(ctypes.Structure):
    _fields_ = [("src", ctypes.c_void_p), ("dst", ctypes.c_void_p), ("n8", ctypes.c_int64),
                ("nthreads", ctypes.c_int64)]


def decode_e4m3(src_ptr: int, dst_ptr: int, n: int) -> Launch:
    """fp8 E4M3FN codes -> bf16 (``n`` a multiple of 8; 8- / 16-byte aligned)
    with the decode the GEMM kernel stages its fp8 operand through."""
    if n % 8 or src_ptr % 8 or dst_ptr % 16:
        raise LaunchError("decode_e4m3 needs n % 8 == 0, 8-byte aligned codes, 16-byte aligned output")
    n8 = n // 8
    grid = max(1, min((n8 + 255) // 256, 1 << 20))
    return Launch("generic", "nk_decode_e4m3_bf16", (grid, 1, 1), (256, 1, 1),
                  DecodeE4m3Args(src_ptr, dst_ptr, n8, grid * 256), bytes=3 * n)


def _grid_for(total: int, max_blocks: int = 16384) -> int:
    return max(1, min((total + 255) // 256, max_blocks))


# ---------------------------------------------------------------------------
# Affine index maps through layout nodes
# ---------------------------------------------------------------------------
def is_unit_reshape(src_shape, dst_shape) -> bool:
    """True if the reshape only inserts / removes size-1 dimensions."""
    return [s for s in src_shape if s != 1] == [s for s in dst_shape if s != 1]


def map_to_operand(node, A: np.ndarray, b: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """Given the affine map (A, b) from program index to the index of
    ``node.out``, return the map to the index of ``node.inputs[0]``."""
    op = node.op
    src = node.inputs[0]
    if op == "broadcast_in_dim":
        dims = list(node.attrs["broadcast_dimensions"])
        if not dims:
            return np.zeros((0, A.shape[1]), np.int64), np.zeros(0, np.int64)
        return A[dims, :].copy(), b[dims].copy()
    if op == "transpose":
        perm = node.attrs["permutation"]
        A2 = np.zeros((src.ndim, A.shape[1]), np.int64)
        b2 = np.zeros(src.ndim, np.int64)
        for k, p in enumerate(perm):
            A2[p] = A[k]
            b2[p] = b[k]
        return A2, b2
    if op == "slice":
        st = np.asarray(node.attrs["start_indices"], np.int64)
        sd = np.asarray(node.attrs["strides"], np.int64)
        return A * sd[:, None], st + sd * b
    if op == "reverse":
        A2, b2 = A.copy(), b.copy()
        for d in node.attrs["dimensions"]:
            A2[d] = -A[d]
            b2[d] = (src.shape[d] - 1) - b[d]
        return A2, b2
    if op == "reshape":
        out = node.out
        o_dims = [i for i, s in enumerate(out.shape) if s != 1]
        i_dims = [i for i, s in enumerate(src.shape) if s != 1]
        A2 = np.zeros((src.ndim, A.shape[1]), np.int64)
        b2 = np.zeros(src.ndim, np.int64)
        for od, idim in zip(o_dims, i_dims):
            A2[idim] = A[od]
            b2[idim] = b[od]
        return A2, b2
    # elementwise: same index space
    return A, b


def is_affine_layout(node) -> bool:
    if node.op in LAYOUT_OPS:
        return True
    if node.op == "reshape":
        return is_unit_reshape(node.inputs[0].shape, node.out.shape)
    return False


# ---------------------------------------------------------------------------
# Program builder
# ---------------------------------------------------------------------------
class ProgramTooLarge(Exception):
    pass


class Program:
    """Register program over the index space ``shape``."""

    def __init__(self, shape):
        self.shape = tuple(int(s) for s in shape)
        self.instrs: List[tuple] = []  # (op, dst, a, b, c, dtype, flags, imm)
        self.inputs: List[tuple] = []  # (value, strides over program dims, offset)
        self._next_reg = 0
        self._memo: Dict[tuple, int] = {}

    def _reg(self) -> int:
        if self._next_reg >= EW_REGS:
            raise ProgramTooLarge("register file exhausted")
        r = self._next_reg
        self._next_reg += 1
        return r

    def emit(self, op, a=0, b=0, c=0, dtype=dt.float32, flags=0, imm=0.0) -> int:
        if len(self.instrs) >= EW_MAX_INSTR:
            raise ProgramTooLarge("instruction budget exhausted")
        dst = self._reg()
        self.instrs.append((op, dst, a, b, c, dtype_code(dtype), flags, float(imm)))
        return dst

    def load(self, v: Value, strides, offset) -> int:
        key = ("load", v.id, tuple(int(s) for s in strides), int(offset))
        if key in self._memo:
            return self._memo[key]
        if len(self.inputs) >= EW_MAX_IN:
            raise ProgramTooLarge("too many inputs")
        self.inputs.append((v, tuple(int(s) for s in strides), int(offset)))
        r = self.emit(OP_LOAD, dtype=v.dtype, imm=len(self.inputs) - 1)
        self._memo[key] = r
        return r


def scalar_constant(v: Value) -> Optional[float]:
    if v.node is not None and v.node.op == "constant" and v.size == 1:
        payload = v.node.attrs["value"]
        if payload.dtype.fields is not None:  # bf16 / fp8 bit patterns
            return float(dt.to_float32(payload).reshape(-1)[0])
        return float(np.asarray(payload).reshape(-1)[0])
    return None


class ProgramBuilder:
    """Builds the program computing ``root`` with loads of materialised values."""

    def __init__(self, materialized):
        self.materialized = materialized  # callable(Value) -> bool

    def build(self, root: Value, shape=None) -> Program:
        shape = root.shape if shape is None else shape
        if len(shape) > EW_MAX_RANK:
            raise LaunchError(f"elementwise rank {len(shape)} exceeds {EW_MAX_RANK}")
        prog = Program(shape)
        R = len(shape)
        A = np.eye(len(root.shape), R, dtype=np.int64) if len(root.shape) == R else None
        if A is None:
            raise LaunchError("program shape must match the root rank")
        b = np.zeros(len(root.shape), np.int64)
        r = self._emit(prog, root, A, b, top=True)
        prog.result = r
        return prog

    def _emit(self, prog: Program, v: Value, A, b, top=False) -> int:
        key = ("val", v.id, A.tobytes(), b.tobytes())
        if key in prog._memo:
            return prog._memo[key]
        node = v.node
        c = scalar_constant(v)
        if c is not None:
            r = prog.emit(OP_CONST, dtype=v.dtype, imm=c)
        elif (self.materialized(v) and not top) or node is None or node.op == "constant":
            s = contiguous_strides(v.shape)
            strides = s @ A if v.ndim else np.zeros(A.shape[1], np.int64)
            offset = int(s @ b) if v.ndim else 0
            r = prog.load(v, strides, offset)
        elif node.op == "iota":
            d = node.attrs["dimension"]
            # index along dim d is row d of the map: only pure axis maps allowed
            row, off = A[d], b[d]
            nz = np.nonzero(row)[0]
            if len(nz) == 1 and row[nz[0]] == 1 and off == 0:
                r = prog.emit(OP_IOTA, dtype=v.dtype, imm=int(nz[0]))
            elif len(nz) == 0:
                r = prog.emit(OP_CONST, dtype=v.dtype, imm=float(off))
            else:
                raise ProgramTooLarge("iota through a non-trivial index map")
        elif is_affine_layout(node):
            A2, b2 = map_to_operand(node, A, b)
            r = self._emit(prog, node.inputs[0], A2, b2)
        elif node.op == "reshape":
            # a general reshape of a non-materialised value cannot be inlined
            raise ProgramTooLarge("reshape inside an elementwise chain")
        elif node.op in UNARY_CODES:
            x = self._emit(prog, node.inputs[0], A, b)
            flags = 1 if dt.is_int(node.inputs[0].dtype) else 0
            r = prog.emit(UNARY_CODES[node.op], a=x, dtype=v.dtype, flags=flags)
        elif node.op in BINARY_CODES:
            x = self._emit(prog, node.inputs[0], A, b)
            y = self._emit(prog, node.inputs[1], A, b)
            flags = 1 if (dt.is_int(v.dtype) or dt.is_bool(v.dtype)) else 0
            r = prog.emit(BINARY_CODES[node.op], a=x, b=y, dtype=v.dtype, flags=flags)
        elif node.op == "compare":
            x = self._emit(prog, node.inputs[0], A, b)
            y = self._emit(prog, node.inputs[1], A, b)
            r = prog.emit(COMPARE_CODES[node.attrs["comparison_direction"]], a=x, b=y, dtype=dt.bool_)
        elif node.op == "select":
            p = self._emit(prog, node.inputs[0], A, b)
            x = self._emit(prog, node.inputs[1], A, b)
            y = self._emit(prog, node.inputs[2], A, b)
            r = prog.emit(OP_SELECT, a=p, b=x, c=y, dtype=v.dtype)
        else:
            raise ProgramTooLarge(f"op {node.op} is not elementwise")
        prog._memo[key] = r
        return r


class ProgramStep(Step):
    """One ``nk_ew_program`` launch writing ``shape`` elements of ``out``
    (a plain copy of a contiguous value takes the streaming copy kernel)."""

    kind = "elementwise"

    def __init__(self, desc, prog: Program, out: Value, out_dtype=None,
                 out_strides=None, out_offset: int = 0):
        ins = [v for v, _, _ in prog.inputs]
        super().__init__(desc, ins, [out])
        self.prog = prog
        self.out = out
        self.out_dtype = dt.canonical(out_dtype if out_dtype is not None else out.dtype)
        self.out_strides = (contiguous_strides(prog.shape) if out_strides is None
                            else np.asarray(out_strides, np.int64))
        self.out_offset = int(out_offset)

    def launches(self, addr):
        p = self.prog
        a = EwArgs()
        a.out = addr(self.out)
        a.out_offset = self.out_offset
        total = int(np.prod(p.shape)) if p.shape else 1
        rank = len(p.shape)
        for d in range(rank):
            a.shape[d] = p.shape[d]
            a.out_strides[d] = int(self.out_strides[d])
        a.total = total
        a.rank = rank
        a.n_in = len(p.inputs)
        a.n_instr = len(p.instrs)
        a.out_dtype = dtype_code(self.out_dtype)
        a.result_reg = p.result
        grid = _grid_for(total)
        a.nthreads = grid * 256
        for i, (v, strides, off) in enumerate(p.inputs):
            a.inp[i].ptr = addr(v) + off * v.dtype.itemsize
            for d in range(rank):
                a.inp[i].strides[d] = strides[d]
            a.inp[i].dtype = dtype_code(v.dtype)
        for k, (op, dst, x, y, z, dtc, flags, imm) in enumerate(p.instrs):
            I = a.prog[k]
            I.op, I.dst, I.a, I.b, I.c, I.dtype, I.flags, I.imm = op, dst, x, y, z, dtc, flags, imm
        if total == 0:
            return []
        if getattr(p, "flat_copy", False) and self.out_offset == 0 and self.out_dtype == p.inputs[0][0].dtype:
            src = a.inp[0].ptr
            nbytes = total * self.out_dtype.itemsize
            if nbytes % 16 == 0 and src % 16 == 0 and a.out % 16 == 0:
                return [copy16(src, a.out, nbytes)]
        return [Launch("generic", "nk_ew_program", (grid, 1, 1), (256, 1, 1), a,
                       bytes=total * self.out_dtype.itemsize)]


def strided_access(v: Value, materialized) -> Tuple[Value, np.ndarray, int]:
    """Follow affine layout ops from ``v`` down to a materialised value.
    Returns (base value, strides over v's index space, element offset)."""
    A = np.eye(v.ndim, dtype=np.int64)
    b = np.zeros(v.ndim, np.int64)
    cur = v
    while not materialized(cur) and cur.node is not None and is_affine_layout(cur.node):
        A, b = map_to_operand(cur.node, A, b)
        cur = cur.node.inputs[0]
    s = contiguous_strides(cur.shape)
    strides = s @ A if cur.ndim else np.zeros(v.ndim, np.int64)
    off = int(s @ b) if cur.ndim else 0
    return cur, strides, off


REDUCE_CODES = {"add": 0, "maximum": 1, "minimum": 2, "multiply": 3, "and": 4, "or": 5}


class ReduceStep(Step):
    kind = "reduce"

    def __init__(self, node, base: Value, strides, offset: int):
        super().__init__(f"{node.op} {node.attrs.get('computation', '')} over "
                         f"{node.attrs.get('dimensions', node.attrs.get('axis'))}", [base], [node.out])
        self.node = node
        self.base = base
        self.strides = np.asarray(strides, np.int64)
        self.offset = offset
        src = node.inputs[0]
        if node.op in ("argmax", "argmin"):
            red = (node.attrs["axis"],)
            self.code = 6 if node.op == "argmax" else 7
        else:
            red = tuple(node.attrs["dimensions"])
            self.code = REDUCE_CODES[node.attrs["computation"]]
        keep = [d for d in range(src.ndim) if d not in red]
        if len(keep) > RED_MAX_RANK or len(red) > RED_MAX_RANK:
            raise LaunchError("reduction rank too large")
        self.out_shape = [src.shape[d] for d in keep]
        self.out_str = [int(self.strides[d]) for d in keep]
        self.red_shape = [src.shape[d] for d in red]
        self.red_str = [int(self.strides[d]) for d in red]
        acc = node.attrs.get("acc_dtype")
        self.acc_f32 = 1 if (acc is not None and dt.canonical(acc) == dt.float32) else 0

    def launches(self, addr):
        a = ReduceArgs()
        a.inp = addr(self.base) + self.offset * self.base.dtype.itemsize
        a.out = addr(self.node.out)
        for i, (s, st) in enumerate(zip(self.out_shape, self.out_str)):
            a.out_shape[i], a.out_strides[i] = s, st
        for i, (s, st) in enumerate(zip(self.red_shape, self.red_str)):
            a.red_shape[i], a.red_strides[i] = s, st
        n_out = int(np.prod(self.out_shape)) if self.out_shape else 1
        n_red = int(np.prod(self.red_shape)) if self.red_shape else 1
        a.n_out, a.n_red = n_out, n_red
        a.out_rank, a.red_rank = len(self.out_shape), len(self.red_shape)
        a.op = self.code
        a.in_dtype = dtype_code(self.base.dtype)
        a.out_dtype = dtype_code(self.node.out.dtype)
        a.acc_f32 = self.acc_f32
        if n_out == 0:
            return []
        if n_out >= 2**31:
            raise LaunchError("too many reduction outputs for one launch")
        return [Launch("generic", "nk_reduce", (n_out, 1, 1), (256, 1, 1), a)]


class DotStep(Step):
    """Fallback batched dot with arbitrary operand strides (fp32 accumulate)."""

    kind = "dot"

    def __init__(self, node, lhs, rhs):
        super().__init__("dot (generic)", [lhs[0], rhs[0]], [node.out])
        self.node = node
        a_v, a_s, a_o = lhs
        b_v, b_s, b_o = rhs
        at = node.attrs
        src_a, src_b = node.inputs
        lb, rb = list(at["lhs_batch"]), list(at["rhs_batch"])
        lc, rc = list(at["lhs_contract"]), list(at["rhs_contract"])
        lf = [i for i in range(src_a.ndim) if i not in lb and i not in lc]
        rf = [i for i in range(src_b.ndim) if i not in rb and i not in rc]
        if len(lc) != 1 or len(rf) > 1 or len(lb) != len(rb):
            raise LaunchError("generic dot supports one contracting dim and a rank<=2 rhs per batch")

        def collapse(dims, shape, strides, what):
            """(size, stride) of dims merged into one; LaunchError if the
            strides do not describe one uniform axis."""
            if not dims:
                return 1, 0
            st = int(strides[dims[-1]])
            expect = st
            for i in reversed(dims):
                if shape[i] != 1 and int(strides[i]) != expect:
                    raise LaunchError(f"generic dot: {what} dims are not collapsible")
                expect *= shape[i]
            return int(np.prod([shape[i] for i in dims])), st

        self.M, self.sam = collapse(lf, src_a.shape, a_s, "lhs free")
        self.batch, self.sab = collapse(lb, src_a.shape, a_s, "lhs batch")
        _, self.sbb = collapse(rb, src_b.shape, b_s, "rhs batch")
        self.sak = int(a_s[lc[0]])
        self.K = src_a.shape[lc[0]]
        self.N = src_b.shape[rf[0]] if rf else 1
        self.sbn = int(b_s[rf[0]]) if rf else 0
        self.sbk = int(b_s[rc[0]])
        self.a_v, self.a_o, self.b_v, self.b_o = a_v, a_o, b_v, b_o

    def launches(self, addr):
        a = DotArgs()
        a.A = addr(self.a_v) + self.a_o * self.a_v.dtype.itemsize
        a.B = addr(self.b_v) + self.b_o * self.b_v.dtype.itemsize
        a.C = addr(self.node.out)
        a.batch, a.M, a.N, a.K = self.batch, self.M, self.N, self.K
        a.sab, a.sam, a.sak = self.sab, self.sam, self.sak
        a.sbb, a.sbk, a.sbn = self.sbb, self.sbk, self.sbn
        a.a_dtype = dtype_code(self.a_v.dtype)
        a.b_dtype = dtype_code(self.b_v.dtype)
        a.c_dtype = dtype_code(self.node.out.dtype)
        gx, gy = (self.N + 15) // 16, (self.M + 15) // 16
        if self.M * self.N * self.batch == 0:
            return []
        if gy > 65535 or self.batch > 65535:
            raise LaunchError("generic dot grid too large")
        return [Launch("generic", "nk_dot", (gx, gy, self.batch), (256, 1, 1), a,
                       flops=2 * self.batch * self.M * self.N * self.K)]


def axis_view(shape, axis) -> Tuple[int, int, int]:
    O = int(np.prod(shape[:axis])) if axis else 1
    N = int(np.prod(shape[axis + 1:])) if axis + 1 < len(shape) else 1
    return O, shape[axis], N


class GatherStep(Step):
    """take (0), take_along_axis (1), scatter (2), put_along_axis (3)."""

    kind = "gather"
    MODES = {"take": 0, "take_along_axis": 1, "scatter_along_axis": 2, "put_along_axis": 3}

    def __init__(self, node):
        mode = self.MODES[node.op]
        op = node.inputs
        src = op[0] if mode <= 1 else op[2]
        super().__init__(node.op, [src, op[1]], [node.out])
        self.node, self.mode, self.src, self.idx = node, mode, src, op[1]
        ax = node.attrs["axis"]
        operand = op[0]
        O, A, N = axis_view(operand.shape, ax)
        if mode in (0, 2):
            I = op[1].size
        else:
            I = op[1].shape[ax]
        self.dims = (O, A, I, N)

    def launches(self, addr):
        O, A, I, N = self.dims
        a = GatherArgs()
        a.src = addr(self.src)
        a.idx = addr(self.idx)
        a.out = addr(self.node.out)
        a.O, a.A, a.I, a.N = O, A, I, N
        total = O * I * N
        grid = _grid_for(total)
        a.nthreads = grid * 256
        a.mode = self.mode
        a.dtype = dtype_code(self.node.out.dtype)
        if total == 0:
            return []
        return [Launch("generic", "nk_gather", (grid, 1, 1), (256, 1, 1), a)]


class TopkArgs(ctypes.Structure):
    _fields_ = [("inp", ctypes.c_void_p), ("idx", ctypes.c_void_p), ("rows", ctypes.c_int64),
                ("n", ctypes.c_int64), ("k", ctypes.c_int32), ("largest", ctypes.c_int32),
                ("dtype", ctypes.c_int32), ("pad", ctypes.c_int32)]


class TopkStep(Step):
    """Indices of the k largest (or smallest) elements of each row along the
    last axis, ordered by value, ties by index (nk_topk)."""

    kind = "topk"

    def __init__(self, node):
        x = node.inputs[0]
        super().__init__("topk", [x], [node.out])
        self.node, self.x = node, x
        self.n = x.shape[-1] if x.ndim else 1
        self.rows = x.size // max(self.n, 1)

    def launches(self, addr):
        at = self.node.attrs
        if self.rows == 0:
            return []
        if self.rows >= 2**31:
            raise LaunchError("topk: too many rows")
        a = TopkArgs(addr(self.x), addr(self.node.out), self.rows, self.n, int(at["k"]),
                     1 if at["largest"] else 0, dtype_code(self.x.dtype), 0)
        return [Launch("generic", "nk_topk", (self.rows, 1, 1), (256, 1, 1), a,
                       bytes=self.rows * self.n * self.x.dtype.itemsize * int(at["k"]))]


class CumsumStep(Step):
    kind = "cumsum"

    def __init__(self, node):
        super().__init__("cumsum", [node.inputs[0]], [node.out])
        self.node = node

    def launches(self, addr):
        n = self.node
        O, A, N = axis_view(n.inputs[0].shape, n.attrs["axis"])
        a = CumsumArgs()
        a.inp, a.out = addr(n.inputs[0]), addr(n.out)
        a.O, a.A, a.N = O, A, N
        a.in_dtype, a.out_dtype = dtype_code(n.inputs[0].dtype), dtype_code(n.out.dtype)
        acc = n.attrs.get("acc_dtype")
        a.acc_f32 = 1 if acc is not None and dt.canonical(acc) == dt.float32 else 0
        lines = O * N
        if lines == 0 or A == 0:
            return []
        return [Launch("generic", "nk_cumsum", ((lines + 255) // 256, 1, 1), (256, 1, 1), a)]


def flat_copy_program(src: Value) -> Program:
    """Program copying a contiguous value element by element (rank 1)."""
    prog = Program((src.size,))
    r = prog.load(src, (1,), 0)
    prog.result = r
    prog.flat_copy = True
    return prog

