"""Pattern matchers: traced subgraphs -> fused gfx950 kernels.

Each pattern scans the live nodes of a graph and yields :class:`Match`
objects.  A match claims a set of nodes, names the values it reads
(``inputs``, materialised and contiguous) and the values it produces
(``outputs``), and emits the step(s) that replace the whole subgraph.  A
match is only accepted if none of its internal values escapes (is a graph
result or is read by a node outside the match).

Matching works on the graphs the tracer produces for ordinary NumPy code,
so it tolerates the noise NumPy tracing adds: keepdims reshapes, broadcast
of reduced rows, ``astype`` to the same dtype (a ``copy``), converts around
a low-precision input or output, commuted operands.
"""

from __future__ import annotations

from typing import Iterable, List, Optional, Set, Tuple

import numpy as np

from nkipy_amd.core import dtypes as dt
from nkipy_amd.core.backend.ir import Node, Value
from nkipy_amd.dispatch import launchers as LA
from nkipy_amd.dispatch.plan import Step

VIEW_OPS = ("reshape", "copy")


# ---------------------------------------------------------------------------
# structural helpers
# ---------------------------------------------------------------------------
def op_of(v: Value) -> str:
    return v.node.op if v.node is not None else "parameter"


def through_views(v: Value) -> Tuple[Value, List[Node]]:
    """Follow reshape / copy producers upward (data unchanged)."""
    nodes = []
    while v.node is not None and v.node.op in VIEW_OPS:
        nodes.append(v.node)
        v = v.node.inputs[0]
    return v, nodes


def scalar_value(v: Value) -> Tuple[Optional[float], List[Node]]:
    """Value of a size-1 constant reached through broadcasts / views."""
    nodes = []
    while v.node is not None and v.node.op in ("broadcast_in_dim",) + VIEW_OPS:
        nodes.append(v.node)
        v = v.node.inputs[0]
    if v.node is not None and v.node.op == "constant" and v.size == 1:
        p = v.node.attrs["value"]
        if p.dtype.fields is not None:
            val = float(dt.to_float32(p).reshape(-1)[0])
        else:
            val = float(np.asarray(p).reshape(-1)[0])
        return val, nodes + [v.node]
    return None, []


def row_broadcast(v: Value, shape) -> Optional[Tuple[Value, List[Node]]]:
    """``v`` is a per-row value broadcast along the last axis of ``shape``."""
    n = v.node
    if n is None or n.op != "broadcast_in_dim" or v.shape != tuple(shape):
        return None
    src = n.inputs[0]
    rows = tuple(shape[:-1])
    dims = tuple(n.attrs["broadcast_dimensions"])
    if dims != tuple(range(len(rows))) or src.shape != rows:
        return None
    base, vn = through_views(src)
    return base, [n] + vn


def col_broadcast(v: Value, shape) -> Optional[Tuple[Value, List[Node]]]:
    """``v`` is a vector over the last axis broadcast over the rows."""
    n = v.node
    if n is None or n.op != "broadcast_in_dim" or v.shape != tuple(shape):
        return None
    src = n.inputs[0]
    if tuple(n.attrs["broadcast_dimensions"]) != (len(shape) - 1,) or src.shape != (shape[-1],):
        return None
    base, vn = through_views(src)
    return base, [n] + vn


def reduce_last(v: Value, comp: str) -> Optional[Tuple[Value, Node]]:
    n = v.node
    if n is None or n.op != "reduce" or n.attrs["computation"] != comp:
        return None
    x = n.inputs[0]
    if tuple(n.attrs["dimensions"]) != (x.ndim - 1,):
        return None
    return x, n


class Match:
    """A claimed subgraph and the step(s) that replace it."""

    name = "match"

    def __init__(self, nodes: Iterable[Node], inputs: List[Value], outputs: List[Value]):
        self.node_list = list(dict.fromkeys(nodes))
        self.nodes: Set[int] = {id(n) for n in self.node_list}
        self.inputs = inputs
        self.outputs = outputs
        self.last: Node = None

    def validate(self, L) -> bool:
        """Internal values must not escape; sets ``last`` (emission point)."""
        if not self.node_list:
            return False
        if any(id(n) in L.covered for n in self.node_list):
            return False
        out_ids = {v.id for v in self.outputs}
        for n in self.node_list:
            v = n.out
            if v.id in out_ids:
                continue
            if v.id in L.result_ids:
                return False
            for u in L.users.get(v.id, []):
                if id(u) not in self.nodes:
                    return False
        order = {id(n): i for i, n in enumerate(L.live)}
        if any(id(n) not in order for n in self.node_list):
            return False
        self.last = max(self.node_list, key=lambda n: order[id(n)])
        return True

    def steps(self, plan) -> List[Step]:
        raise NotImplementedError

    def __repr__(self):
        return f"<{self.name} {[repr(v) for v in self.outputs]}>"


class LaunchStep(Step):
    """A step whose launch is produced by a launcher function of addresses."""

    def __init__(self, kind, desc, inputs, outputs, make):
        super().__init__(desc, inputs, outputs)
        self.kind = kind
        self._make = make

    def launches(self, addr):
        l = self._make(addr)
        return l if isinstance(l, list) else [l]


def _users_of(L, v):
    return L.users.get(v.id, [])


def _fold_output_convert(L, out: Value, allowed) -> Tuple[Value, List[Node]]:
    us = _users_of(L, out)
    if out.id not in L.result_ids and len(us) == 1 and us[0].op in ("convert", "copy") \
            and us[0].out.dtype in allowed:
        return us[0].out, [us[0]]
    return out, []


# ---------------------------------------------------------------------------
# K1a: row softmax
# ---------------------------------------------------------------------------
class SoftmaxMatch(Match):
    name = "softmax"

    def __init__(self, nodes, x: Value, y: Value, round_ops: bool = False):
        super().__init__(nodes, [x], [y])
        self.x, self.y, self.round_ops = x, y, round_ops

    def steps(self, plan):
        x, y = self.x, self.y
        n = x.shape[-1]
        rows = x.size // n

        def make(addr):
            return LA.softmax_rows(addr(x), addr(y), rows, n, x.dtype, y.dtype, round_ops=self.round_ops)

        desc = f"row softmax {rows}x{n} {dt.name(x.dtype)}->{dt.name(y.dtype)}"
        if self.round_ops:
            desc += f" (steps in {dt.name(x.dtype)})"
        return [LaunchStep("softmax", desc, [x], [y], make)]


class SoftmaxPattern:
    """exp(x - max(x, -1)) / sum(exp(x - max(x, -1)), -1), optionally with an
    fp32 upcast of a bf16/f16 input and a cast of the result.  Steps traced
    in the 16-bit input type itself are rounded to it as traced."""

    def find(self, L):
        for n in L.live:
            if n.op != "divide" or id(n) in L.covered:
                continue
            m = self._match(L, n)
            if m is not None and m.validate(L):
                yield m

    @staticmethod
    def structure(L, n) -> Optional[Tuple[Value, List[Node]]]:
        """``n`` (a divide) is a last-axis softmax of X -> (X, nodes)."""
        E, B2 = n.inputs
        shape = n.out.shape
        if not shape or shape[-1] < 1 or E.shape != shape:
            return None
        r2 = row_broadcast(B2, shape)
        if r2 is None:
            return None
        s_val, nodes_b2 = r2
        rs = reduce_last(s_val, "add")
        if rs is None or rs[0] is not E or op_of(E) != "exponential":
            return None
        sub = E.node.inputs[0]
        if op_of(sub) != "subtract":
            return None
        X, B1 = sub.node.inputs
        r1 = row_broadcast(B1, shape)
        if r1 is None:
            return None
        m_val, nodes_b1 = r1
        rm = reduce_last(m_val, "maximum")
        if rm is None or rm[0] is not X:
            return None
        return X, [n, rs[1], E.node, sub.node, rm[1]] + nodes_b1 + nodes_b2

    def _match(self, L, n):
        st = self.structure(L, n)
        if st is None:
            return None
        X, nodes = st
        sub, rm = nodes[3], nodes[4]
        # the type the steps run in: fp32 throughout, or x's 16-bit type for
        # x - max, exp, the sum and the divide alike
        step_types = {sub.out.dtype, nodes[2].out.dtype, nodes[1].out.dtype, n.out.dtype}
        if len(step_types) != 1:
            return None
        round_ops = sub.out.dtype in (dt.bfloat16, dt.float16)
        if round_ops and X.dtype != sub.out.dtype:
            return None
        x_in = X
        if op_of(X) == "convert" and X.dtype == dt.float32 and \
                X.node.inputs[0].dtype in (dt.bfloat16, dt.float16) and X.id not in L.result_ids and \
                all(id(u) in {id(sub), id(rm)} for u in _users_of(L, X)):
            x_in = X.node.inputs[0]
            nodes.append(X.node)
        out, extra = _fold_output_convert(L, n.out, (dt.bfloat16, dt.float32, dt.float16))
        nodes += extra
        try:
            LA.dtype_tag(x_in.dtype), LA.dtype_tag(out.dtype)
        except LA.LaunchError:
            return None
        if (LA.dtype_tag(x_in.dtype), LA.dtype_tag(out.dtype)) not in LA._SOFTMAX_TYPES:
            return None
        return SoftmaxMatch(nodes, x_in, out, round_ops)


# ---------------------------------------------------------------------------
# K1b: (residual +) RMSNorm
# ---------------------------------------------------------------------------
class RmsNormMatch(Match):
    name = "rmsnorm"

    def __init__(self, nodes, x, r, w, y, h_out, eps, round_h, mul_recip):
        ins = [v for v in (x, r, w) if v is not None]
        outs = [y] + ([h_out] if h_out is not None else [])
        super().__init__(nodes, ins, outs)
        self.x, self.r, self.w, self.y, self.h = x, r, w, y, h_out
        self.eps, self.round_h, self.mul_recip = eps, round_h, mul_recip

    def steps(self, plan):
        x, r, w, y, h = self.x, self.r, self.w, self.y, self.h
        n = x.shape[-1]
        rows = x.size // n

        def make(addr):
            return LA.rmsnorm_rows(addr(x), addr(y), rows, n, x.dtype, self.eps,
                                   r_ptr=addr(r) if r is not None else 0,
                                   w_ptr=addr(w) if w is not None else 0,
                                   h_ptr=addr(h) if h is not None else 0,
                                   round_h=self.round_h, mul_recip=self.mul_recip)

        desc = (f"{'residual + ' if r is not None else ''}rmsnorm {rows}x{n} {dt.name(x.dtype)}"
                f" eps={self.eps:g}{' (1/sqrt)' if self.mul_recip else ''}")
        return [LaunchStep("rmsnorm", desc, self.inputs, self.outputs, make)]


class RmsNormPattern:
    """h / sqrt(mean(h*h, -1) + eps) [* w], h = x [+ r], fp32 arithmetic on a
    bf16 / f16 / f32 storage dtype."""

    def find(self, L):
        for n in L.live:
            if n.op not in ("divide", "multiply") or id(n) in L.covered:
                continue
            m = self._match(L, n)
            if m is not None and m.validate(L):
                yield m

    def _denominator(self, L, v, shape):
        """v = row-broadcast sqrt(ms + eps) -> (ms, eps, nodes)."""
        rb = row_broadcast(v, shape)
        if rb is None:
            return None
        sq, nodes = rb
        if op_of(sq) != "sqrt":
            return None
        nodes = nodes + [sq.node]
        ad, vn = through_views(sq.node.inputs[0])
        nodes += vn
        if op_of(ad) != "add":
            return None
        nodes.append(ad.node)
        a, b = ad.node.inputs
        for ms, ep in ((a, b), (b, a)):
            eps, en = scalar_value(ep)
            if eps is not None:
                return ms, eps, nodes + en
        return None

    def _recip_denominator(self, L, v, shape):
        """v = row-broadcast 1/sqrt(ms + eps) or rsqrt(ms + eps)."""
        rb = row_broadcast(v, shape)
        if rb is None:
            return None
        inv, nodes = rb
        if op_of(inv) == "divide":
            one, on = scalar_value(inv.node.inputs[0])
            if one != 1.0:
                return None
            sq, vn = through_views(inv.node.inputs[1])
            nodes = nodes + [inv.node] + on + vn
            if op_of(sq) != "sqrt":
                return None
            target = sq.node.inputs[0]
            nodes.append(sq.node)
        elif op_of(inv) == "rsqrt":
            target = inv.node.inputs[0]
            nodes = nodes + [inv.node]
        else:
            return None
        ad, vn = through_views(target)
        nodes += vn
        if op_of(ad) != "add":
            return None
        nodes.append(ad.node)
        a, b = ad.node.inputs
        for ms, ep in ((a, b), (b, a)):
            eps, en = scalar_value(ep)
            if eps is not None:
                return ms, eps, nodes + en
        return None

    def _mean_square(self, L, ms, H, n_last):
        """ms = sum(H*H | H**2, -1) / n  (or * 1/n) -> nodes."""
        ms, nodes = through_views(ms)
        if op_of(ms) not in ("divide", "multiply"):
            return None
        s, c = ms.node.inputs
        cnt, cn = scalar_value(c)
        if cnt is None:
            return None
        if ms.node.op == "divide" and abs(cnt - n_last) > 1e-6 * n_last:
            return None
        if ms.node.op == "multiply" and abs(cnt * n_last - 1.0) > 1e-6:
            return None
        nodes = nodes + [ms.node] + cn
        s, vn = through_views(s)
        nodes += vn
        rs = reduce_last(s, "add")
        if rs is None:
            return None
        sq, node_r = rs
        nodes.append(node_r)
        if op_of(sq) == "multiply" and sq.node.inputs[0] is H and sq.node.inputs[1] is H:
            return nodes + [sq.node]
        if op_of(sq) == "power" and sq.node.inputs[0] is H:
            p, pn = scalar_value(sq.node.inputs[1])
            if p == 2.0:
                return nodes + [sq.node] + pn
        return None

    def _match(self, L, q):
        shape = q.out.shape
        if not shape or q.out.dtype != dt.float32 and q.out.dtype not in (dt.bfloat16, dt.float16):
            return None
        cands = []
        if q.op == "divide":
            H, B = q.inputs
            d = self._denominator(L, B, shape)
            if d is not None:
                cands.append((H, d, False))
        else:
            for H, B in (q.inputs, q.inputs[::-1]):
                d = self._recip_denominator(L, B, shape)
                if d is not None:
                    cands.append((H, d, True))
        for H, (ms, eps, nodes), mul_recip in cands:
            if H.shape != shape:
                continue
            msn = self._mean_square(L, ms, H, shape[-1])
            if msn is None:
                continue
            nodes = [q] + nodes + msn
            m = self._finish(L, q, H, nodes, eps, mul_recip)
            if m is not None:
                return m
        return None

    def _finish(self, L, q, H, nodes, eps, mul_recip):
        shape = q.out.shape
        # storage dtype T and the fp32 upcast of h (astype to the same
        # dtype traces as a copy: look through it)
        while op_of(H) == "copy" and H.node.inputs[0].shape == shape:
            nodes = nodes + [H.node]
            H = H.node.inputs[0]
        if H.dtype == dt.float32 and op_of(H) == "convert" and \
                H.node.inputs[0].dtype in (dt.bfloat16, dt.float16):
            Hs = H.node.inputs[0]
            T = Hs.dtype
            nodes = nodes + [H.node]
        elif H.dtype in (dt.float32, dt.bfloat16, dt.float16):
            Hs = H
            T = H.dtype
        else:
            return None
        # residual
        x, r, h_out, round_h = Hs, None, None, True
        if op_of(Hs) == "add" and id(Hs.node) not in L.covered and \
                Hs.node.inputs[0].shape == shape and Hs.node.inputs[1].shape == shape:
            a, b = Hs.node.inputs
            if a.dtype == T and b.dtype == T:
                x, r = a, b
                round_h = True
            elif T == dt.float32 and op_of(a) == "convert" and op_of(b) == "convert" and \
                    a.node.inputs[0].dtype == b.node.inputs[0].dtype and \
                    a.node.inputs[0].dtype in (dt.bfloat16, dt.float16) and \
                    all(id(u) == id(Hs.node) for u in _users_of(L, a)) and \
                    all(id(u) == id(Hs.node) for u in _users_of(L, b)):
                # residual added in fp32 after upcasting both operands
                x, r = a.node.inputs[0], b.node.inputs[0]
                T = x.dtype
                round_h = False
                nodes = nodes + [a.node, b.node]
            if r is not None:
                nodes = nodes + [Hs.node]
                escapes = Hs.id in L.result_ids or any(
                    id(u) not in {id(k) for k in nodes} for u in _users_of(L, Hs))
                if escapes:
                    if not round_h:
                        return None  # fp32 sum is not the storage dtype of the output
                    h_out = Hs
        # weight
        y, w = q.out, None
        us = _users_of(L, q.out)
        if q.out.id not in L.result_ids and len(us) == 1 and us[0].op == "multiply":
            mnode = us[0]
            other = mnode.inputs[1] if mnode.inputs[0] is q.out else mnode.inputs[0]
            cb = col_broadcast(other, shape)
            if cb is not None:
                wv, wn = cb
                wnodes = list(wn)
                if wv.dtype == dt.float32 and op_of(wv) == "convert" and wv.node.inputs[0].dtype == T:
                    wnodes.append(wv.node)
                    wv = wv.node.inputs[0]
                if wv.dtype == T:
                    w = wv
                    y = mnode.out
                    nodes = nodes + [mnode] + wnodes
        out, extra = _fold_output_convert(L, y, (T,))
        nodes += extra
        if out.dtype != T:
            return None
        try:
            LA.dtype_tag(T)
        except LA.LaunchError:
            return None
        return RmsNormMatch(nodes, x, r, w, out, h_out, eps, round_h, mul_recip)


_DEFAULT = []


def default_patterns():
    """The pattern list the lowering tries, in order (built on first use)."""
    if not _DEFAULT:
        _DEFAULT.extend(_build_default_patterns())
    return _DEFAULT


def _build_default_patterns():
    from nkipy_amd.dispatch.patterns_attention import (
        AttentionPattern, DecodeAttentionPattern, HeadRopePattern, ProjectionPlanesFusion, QkvRopeFusion,
        RopePattern,
    )
    from nkipy_amd.dispatch.patterns_gemm import GemmPattern, SwigluPattern
    from nkipy_amd.dispatch.patterns_linattn import LinearAttentionPattern

    # larger structures first: they contain matmuls / softmaxes that smaller
    # patterns would claim; GEMMs before RMSNorm so that a residual add
    # after a projection goes into the GEMM epilogue; the RoPE of q / k then
    # folds into its QKV projection
    return [LinearAttentionPattern(), DecodeAttentionPattern(), AttentionPattern(), RopePattern(), HeadRopePattern(),
            SwigluPattern(), GemmPattern(), SoftmaxPattern(), RmsNormPattern(), QkvRopeFusion(),
            ProjectionPlanesFusion()]

