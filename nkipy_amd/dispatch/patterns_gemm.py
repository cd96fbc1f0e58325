"""GEMM patterns: traced matmuls -> the MFMA GEMM kernel (csrc/kernels/gemm.hip).

Recognised forms (all with a 2-D weight and no batch dimensions on it):

* ``x @ W``        W (K, N) row-major            -> NN
* ``x @ W.T``      W (N, K) row-major            -> NT   (torch Linear layout,
  tests/kernels/mlp_dynamo.py:9-25 uses np.transpose + matmul)
* fp8 weights dequantised in the kernel body, ``W8.astype(f32) * scale``
  with a per-output-channel scale (then optionally ``.astype(bf16)``): the
  kernel reads the fp8 codes and applies the scale in the epilogue.
* epilogues folded into the kernel: ``+ bias`` over the last axis, ``+ r``
  with a residual of the output's shape, a final ``astype``.
* SwiGLU: ``silu(g) * u`` where g and u are the two halves of one matmul
  against a fused gate_up weight split with ``np.split`` (examples/models/
  qwen3/kernels/feedforward.py:9-18) or two matmuls of the same input; silu
  written as ``g * (1 / (1 + exp(-g)))`` (feedforward.py:4-6), ``g / (1 +
  exp(-g))`` or ``g * sigmoid``.  Gate and up are computed by one kernel and
  only the bf16 product is written.

The activation must be bf16 (or a float32 upcast of bf16, which is exact);
float32 activations stay on the generic path, because the MFMA kernel reads
bf16 operands.
"""

from __future__ import annotations

from typing import List, Optional, Tuple

from nkipy_amd.core import dtypes as dt
from nkipy_amd.core.backend.ir import Node, Value
from nkipy_amd.dispatch import launchers as LA
from nkipy_amd.dispatch.plan import Slot
from nkipy_amd.dispatch.patterns import (
    LaunchStep, Match, _users_of, col_broadcast, op_of, scalar_value, through_views,
)


def _strip_converts(v: Value) -> Tuple[Value, List[Node]]:
    """Follow float converts down (used where the cast of a dequantised
    weight is absorbed into the kernel's fp32 epilogue)."""
    nodes = []
    while op_of(v) in ("convert", "copy") and dt.is_float(v.node.inputs[0].dtype):
        nodes.append(v.node)
        v = v.node.inputs[0]
    return v, nodes


_EXACT_WIDEN = {(dt.bfloat16, dt.float32), (dt.float16, dt.float32)}


def _strip_widening(v: Value) -> Tuple[Value, List[Node]]:
    """Follow converts that preserve every value (bf16 / f16 -> f32, same-dtype
    copies) down to the narrow source."""
    nodes = []
    while op_of(v) in ("convert", "copy"):
        src = v.node.inputs[0]
        if src.dtype != v.dtype and (src.dtype, v.dtype) not in _EXACT_WIDEN:
            break
        nodes.append(v.node)
        v = src
    return v, nodes


class Weight:
    """Resolved right operand: a materialised matrix, its layout and scale."""

    def __init__(self, value: Value, layout: str, nodes: List[Node], scale: Optional[Value] = None):
        self.value = value
        self.layout = layout
        self.nodes = nodes
        self.scale = scale

    @property
    def fp8(self) -> bool:
        return self.scale is not None


def _dequant(v: Value, out_axis: int) -> Optional[Tuple[Value, Value, List[Node]]]:
    """v = W8.astype(float) * scale broadcast along ``out_axis`` (optionally
    cast again) -> (W8, scale, nodes)."""
    nodes = []
    v, cn = _strip_converts(v)
    nodes += cn
    if op_of(v) != "multiply" or v.ndim != 2:
        return None
    for w, s in (v.node.inputs, v.node.inputs[::-1]):
        wb, wn = _strip_converts(w)
        if wb.dtype != dt.float8_e4m3fn or wb.shape != v.shape:
            continue
        sn = s.node
        if sn is None or sn.op != "broadcast_in_dim" or tuple(sn.attrs["broadcast_dimensions"]) != (out_axis,):
            continue
        sv, svn = through_views(sn.inputs[0])
        if sv.dtype != dt.float32 or sv.shape != (v.shape[out_axis],):
            continue
        return wb, sv, nodes + [v.node] + wn + [sn] + svn
    return None


def resolve_weight(rhs: Value) -> Optional[Weight]:
    """Right operand of a 2-D contraction (K, N) -> Weight."""
    if rhs.ndim != 2:
        return None
    base, vn = through_views(rhs)
    if op_of(base) == "transpose" and tuple(base.node.attrs["permutation"]) == (1, 0):
        src = base.node.inputs[0]
        nodes = vn + [base.node]
        dq = _dequant(src, 0)
        if dq is not None:
            w8, sc, dn = dq
            return Weight(w8, "nt", nodes + dn, sc)
        src_b, sn = _strip_widening(src)
        if src_b.dtype == dt.bfloat16:
            return Weight(src_b, "nt", nodes + sn)
        return None
    dq = _dequant(rhs, 1)
    if dq is not None:
        w8, sc, dn = dq
        return Weight(w8, "nn", dn, sc)
    b, sn = _strip_widening(rhs)
    if b.dtype == dt.bfloat16:
        return Weight(b, "nn", sn)
    return None


def _plain_dot(n: Node) -> bool:
    if n.op != "dot":
        return False
    at = n.attrs
    lhs, rhs = n.inputs
    return (not at["lhs_batch"] and not at["rhs_batch"] and rhs.ndim == 2 and lhs.ndim >= 1
            and tuple(at["lhs_contract"]) == (lhs.ndim - 1,) and tuple(at["rhs_contract"]) == (0,))


def resolve_activation(lhs: Value) -> Optional[Tuple[Value, List[Node]]]:
    x, nodes = _strip_widening(lhs)
    if x.dtype != dt.bfloat16:
        return None
    return x, nodes


class GemmMatch(Match):
    name = "gemm"

    def __init__(self, nodes, x: Value, w: Weight, out: Value, *, bias=None, resid=None,
                 up: Weight = None, up_offset: int = 0, n_out: int = None, rnd=(False, False)):
        ins = [x, w.value] + ([w.scale] if w.scale is not None else [])
        if up is not None and up.value is not w.value:
            ins.append(up.value)
        if up is not None and up.scale is not None:
            ins.append(up.scale)
        ins += [v for v in (bias, resid) if v is not None]
        super().__init__(nodes, ins, [out])
        self.x, self.w, self.out, self.bias, self.resid = x, w, out, bias, resid
        self.up, self.up_offset = up, up_offset
        self.n_out = n_out
        self.rnd = rnd
        self.split_k = True  # few rows: partial sums over K ranges
        # a head prologue that adds this projection's partial sums itself
        # (ProjectionPlanesFusion), and what it reads: (workspace slot,
        # planes, elements per plane), set at step time
        self.planes_consumer = None
        self.planes = None

    def steps(self, plan):
        x, w, out = self.x, self.w, self.out
        K = x.shape[-1]
        M = x.size // K
        N = self.n_out if self.n_out is not None else out.shape[-1]
        ldb = w.value.shape[1]
        up, off = self.up, self.up_offset
        bias, resid = self.bias, self.resid
        rnd_bias, rnd_resid = self.rnd

        # a few rows (a decode token per sequence): the split-K projection,
        # which streams the weights over the whole part; up to a tile of rows
        # (a decode batch): the MFMA kernels over K ranges, so that the
        # grid fills the part
        fp8 = w.value.dtype == dt.float8_e4m3fn
        # a projection of up to 16-32 rows: the MFMA form of the few-row
        # kernels (16-row tiles, weights streamed once)
        mfma = (self.split_k
                and (up is None or (up.layout == w.layout and up.value.dtype == w.value.dtype))
                and LA.gemv_mfma_preferred(M, N, K, up is not None, w.layout, fp8))
        small = not mfma and LA.gemv_preferred(M, w.layout, fp8)
        splitk = (self.split_k and not mfma and not small and not (fp8 and w.layout == "nn")
                  and LA.gemm_splitk_useful(M, N, K, up is not None, fp8))
        small = small or (not mfma and M <= LA.GEMV_MAX_M and not splitk)
        ws = None
        fold = False
        if mfma:
            ws = Slot(plan.add_buffer(LA.gemv_mfma_workspace_bytes(M, N, K, up is not None), "temp",
                                      "gemv.partials"))
            ks = LA.gemv_mfma_split(M, N, K, up is not None)[0]
            fold = self.planes_consumer is not None and ks <= LA.HR_MAX_PLANES and N % 8 == 0
            self.planes = (ws, ks, M * N) if fold else None
        elif small:
            ws = Slot(plan.add_buffer(LA.gemv_workspace_bytes(M, N, K, w.layout, fp8, up is not None), "temp",
                                      "gemv.partials"))
        elif splitk:
            ws = Slot(plan.add_buffer(LA.gemm_splitk_workspace_bytes(M, N, K, up is not None, fp8), "temp",
                                      "gemm.partials"))

        def make(addr):
            up_ptr = 0
            up_scale = 0
            if up is not None:
                up_ptr = addr(up.value) + off * up.value.dtype.itemsize
                up_scale = addr(up.scale) if up.scale is not None else 0
            if mfma:
                ls = LA.gemv_mfma(addr(x), addr(w.value), addr(out), M, N, K, c_dtype=out.dtype, ldb=ldb,
                                  layout=w.layout, b_dtype=w.value.dtype, ws_ptr=addr(ws),
                                  bias_ptr=addr(bias) if bias is not None else 0,
                                  scale_ptr=addr(w.scale) if w.scale is not None else 0,
                                  resid_ptr=addr(resid) if resid is not None else 0, up_ptr=up_ptr,
                                  up_scale_ptr=up_scale,
                                  round_before_bias=rnd_bias, round_before_resid=rnd_resid)
                # with a planes consumer the reduction is the head prologue's
                return ls[:1] if fold else ls
            if small:
                return LA.gemv(addr(x), addr(w.value), addr(out), M, N, K, layout=w.layout,
                               b_dtype=w.value.dtype, c_dtype=out.dtype, ldb=ldb, ws_ptr=addr(ws),
                               bias_ptr=addr(bias) if bias is not None else 0,
                               scale_ptr=addr(w.scale) if w.scale is not None else 0,
                               resid_ptr=addr(resid) if resid is not None else 0,
                               up_ptr=up_ptr, up_scale_ptr=up_scale,
                               round_before_bias=rnd_bias, round_before_resid=rnd_resid)
            if splitk:
                return LA.gemm_splitk(addr(x), addr(w.value), addr(out), M, N, K, layout=w.layout,
                                      b_dtype=w.value.dtype, c_dtype=out.dtype, ldb=ldb, ws_ptr=addr(ws),
                                      bias_ptr=addr(bias) if bias is not None else 0,
                                      scale_ptr=addr(w.scale) if w.scale is not None else 0,
                                      resid_ptr=addr(resid) if resid is not None else 0,
                                      up_ptr=up_ptr, up_scale_ptr=up_scale,
                                      round_before_bias=rnd_bias, round_before_resid=rnd_resid)
            return LA.gemm(addr(x), addr(w.value), addr(out), M, N, K, layout=w.layout,
                           b_dtype=w.value.dtype, c_dtype=out.dtype, ldb=ldb,
                           bias_ptr=addr(bias) if bias is not None else 0,
                           scale_ptr=addr(w.scale) if w.scale is not None else 0,
                           resid_ptr=addr(resid) if resid is not None else 0,
                           up_ptr=up_ptr, up_scale_ptr=up_scale,
                           round_before_bias=rnd_bias, round_before_resid=rnd_resid)

        kind = "gemm_swiglu" if up is not None else "gemm"
        desc = (f"{'swiglu ' if up is not None else ''}gemm {w.layout} M={M} N={N} K={K} "
                f"{dt.name(w.value.dtype)} -> {dt.name(out.dtype)}"
                + (" +bias" if bias is not None else "") + (" +residual" if resid is not None else "")
                + (" (partial sums to the head prologue)" if fold else ""))
        return [LaunchStep(kind, desc, self.inputs, self.outputs, make)]


class Epilogue:
    """What a GEMM's epilogue folds in, with the traced code's cast points:
    ``rnd_bias`` / ``rnd_resid`` say the running value was rounded to bf16
    (a bf16 product, an ``astype``, a bf16 add) before that add."""

    def __init__(self):
        self.bias = self.resid = None
        self.rnd_bias = self.rnd_resid = False


def _fold_epilogue(L, v: Value, nodes: List[Node]):
    """Fold single-user bias / residual adds and a final cast after ``v``."""
    ep = Epilogue()
    rounded = v.dtype == dt.bfloat16  # the product itself is stored as bf16
    while True:
        us = _users_of(L, v)
        if v.id in L.result_ids or len(us) != 1:
            break
        u = us[0]
        if u.op == "add" and u.out.dtype == v.dtype:
            other = u.inputs[1] if u.inputs[0] is v else u.inputs[0]
            cb = col_broadcast(other, v.shape)
            if ep.bias is None and ep.resid is None and cb is not None and cb[0].dtype == dt.bfloat16:
                ep.bias, ep.rnd_bias = cb[0], rounded
                nodes += [u] + cb[1]
                v = u.out
                rounded = v.dtype == dt.bfloat16
                continue
            if ep.resid is None and other.shape == v.shape and other.dtype == v.dtype and \
                    (other.node is None or other.node.op != "broadcast_in_dim"):
                ep.resid, ep.rnd_resid = other, rounded
                nodes.append(u)
                v = u.out
                rounded = v.dtype == dt.bfloat16
                continue
            break
        if u.op in ("convert", "copy") and u.out.dtype in (dt.bfloat16, dt.float32) and dt.is_float(v.dtype):
            if ep.resid is not None and u.out.dtype != v.dtype:
                break  # the residual must have the output dtype
            nodes.append(u)
            v = u.out
            rounded = rounded or v.dtype == dt.bfloat16
            continue
        break
    return v, ep


class GemmPattern:
    """``split_k=False`` keeps every projection of more than a few rows on
    one K loop per tile (the summation order of the fused rotary GEMM)."""

    def __init__(self, split_k: bool = True):
        self.split_k = split_k

    def find(self, L):
        for n in L.live:
            if id(n) in L.covered or not _plain_dot(n):
                continue
            m = self._match(L, n)
            if m is not None and m.validate(L):
                m.split_k = self.split_k
                yield m

    def _match(self, L, n: Node):
        xa = resolve_activation(n.inputs[0])
        w = resolve_weight(n.inputs[1])
        if xa is None or w is None:
            return None
        x, xn = xa
        if x.ndim < 1 or x.shape[-1] % 8:
            return None
        if w.layout == "nn" and w.value.shape[1] % 8:
            return None
        nodes = [n] + xn + w.nodes
        out, ep = _fold_epilogue(L, n.out, nodes)
        if out.dtype not in (dt.bfloat16, dt.float32):
            return None
        if ep.resid is not None and ep.resid.dtype != out.dtype:
            return None
        return GemmMatch(nodes, x, w, out, bias=ep.bias, resid=ep.resid,
                         rnd=(ep.rnd_bias, ep.rnd_resid))


# ---------------------------------------------------------------------------
# SwiGLU
# ---------------------------------------------------------------------------
def _silu_of(v: Value) -> Optional[Tuple[Value, List[Node]]]:
    """v = silu(g) -> (g, nodes); g may sit behind converts."""
    n = v.node
    if n is None:
        return None

    def sigmoid_den(d: Value, g: Value):
        # 1 + exp(-g)
        if op_of(d) != "add":
            return None
        for one, e in (d.node.inputs, d.node.inputs[::-1]):
            c, cn = scalar_value(one)
            if c == 1.0 and op_of(e) == "exponential" and op_of(e.node.inputs[0]) == "negate" \
                    and e.node.inputs[0].node.inputs[0] is g:
                return [d.node, e.node, e.node.inputs[0].node] + cn
        return None

    if n.op == "multiply":
        for g, s in (n.inputs, n.inputs[::-1]):
            if op_of(s) == "logistic" and s.node.inputs[0] is g:
                return g, [n, s.node]
            if op_of(s) == "divide":
                c, cn = scalar_value(s.node.inputs[0])
                if c == 1.0:
                    dn = sigmoid_den(s.node.inputs[1], g)
                    if dn is not None:
                        return g, [n, s.node] + cn + dn
    if n.op == "divide":
        g, d = n.inputs
        dn = sigmoid_den(d, g)
        if dn is not None:
            return g, [n] + dn
    return None


def _last_axis_half(v: Value) -> Optional[Tuple[Value, int, List[Node]]]:
    """v = mm[..., a:b] (a contiguous slice of the last axis) -> (mm, a, nodes)."""
    base, vn = through_views(v)
    if op_of(base) != "slice":
        return None
    at = base.node.attrs
    src = base.node.inputs[0]
    nd = src.ndim
    if any(s != 1 for s in at["strides"]):
        return None
    if any(at["start_indices"][i] != 0 or at["limit_indices"][i] != src.shape[i] for i in range(nd - 1)):
        return None
    return src, at["start_indices"][-1], vn + [base.node]


class SwigluPattern:
    def find(self, L):
        for n in L.live:
            if n.op != "multiply" or id(n) in L.covered:
                continue
            m = self._match(L, n)
            if m is not None and m.validate(L):
                yield m

    def _match(self, L, n: Node):
        for s_val, u_val in (n.inputs, n.inputs[::-1]):
            sl = _silu_of(s_val)
            if sl is None:
                continue
            g, snodes = sl
            g0, gcn = _strip_widening(g)
            u0, ucn = _strip_widening(u_val)
            nodes = [n] + snodes + gcn + ucn
            m = self._fused_gate_up(L, n, g0, u0, nodes) or self._two_weights(L, n, g0, u0, nodes)
            if m is not None:
                return m
        return None

    def _finish(self, L, n, nodes, x, w, up, up_off, F):
        out = n.out
        us = _users_of(L, out)
        if out.id not in L.result_ids and len(us) == 1 and us[0].op in ("convert", "copy") and \
                us[0].out.dtype == dt.bfloat16:
            nodes.append(us[0])
            out = us[0].out
        if out.dtype != dt.bfloat16:
            return None
        return GemmMatch(nodes, x, w, out, up=up, up_offset=up_off, n_out=F)

    def _fused_gate_up(self, L, n, g, u, nodes):
        gs = _last_axis_half(g)
        us = _last_axis_half(u)
        if gs is None or us is None or gs[0] is not us[0]:
            return None
        mm, g_start, gn = gs
        _, u_start, un = us
        F = g.shape[-1]
        if g_start != 0 or u_start != F or mm.shape[-1] != 2 * F or u.shape[-1] != F:
            return None
        if mm.node is None or not _plain_dot(mm.node):
            return None
        xa = resolve_activation(mm.node.inputs[0])
        w = resolve_weight(mm.node.inputs[1])
        if xa is None or w is None or w.fp8:
            return None
        x, xn = xa
        if x.shape[-1] % 8 or F % 8:
            return None
        nodes = nodes + gn + un + [mm.node] + xn + w.nodes
        # up weight: same matrix, offset by F columns (NN) or F rows (NT)
        off = F if w.layout == "nn" else F * w.value.shape[1]
        return self._finish(L, n, nodes, x, w, w, off, F)

    def _two_weights(self, L, n, g, u, nodes):
        if g.node is None or u.node is None or not _plain_dot(g.node) or not _plain_dot(u.node):
            return None
        xg = resolve_activation(g.node.inputs[0])
        xu = resolve_activation(u.node.inputs[0])
        if xg is None or xu is None or xg[0] is not xu[0]:
            return None
        wg = resolve_weight(g.node.inputs[1])
        wu = resolve_weight(u.node.inputs[1])
        if wg is None or wu is None or wg.layout != wu.layout or wg.fp8 != wu.fp8 or \
                wg.value.shape != wu.value.shape:
            return None
        x = xg[0]
        F = g.shape[-1]
        if x.shape[-1] % 8 or F % 8:
            return None
        nodes = nodes + [g.node, u.node] + xg[1] + xu[1] + wg.nodes + wu.nodes
        return self._finish(L, n, nodes, x, wg, wu, 0, F)


GEMM_PATTERNS = [SwigluPattern(), GemmPattern()]
