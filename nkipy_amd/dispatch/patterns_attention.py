"""Attention-block patterns -> csrc/kernels/rope.hip and attention.hip.

Rotary embedding, split-half form (examples/models/qwen3/kernels/rope.py:
23-48), anchored on the ``np.concatenate`` that joins the two halves::

    x0, x1 = x[..., :D/2], x[..., D/2:]          (x bf16, upcast to fp32)
    out = concatenate([x0 * cos - x1 * sin, x0 * sin + x1 * cos], -1).astype(bf16)

with fp32 cos / sin tables indexed by one position axis and the frequency
(broadcast over the other axes).

Causal softmax attention with grouped-query heads (examples/models/qwen3/
kernels/attention.py:109-140; tests/kernels/llama_decoder_dynamo.py:
180-288), anchored on the second product::

    scores = (q @ k_t) * scale      (or / c)           fp32, q / k bf16 upcast
    scores = scores + mask          mask = triu(<= -1e4, k=1), zeros below
    p = softmax(scores, -1)
    o = (p @ v)[.transpose(0, 2, 1, 3)][.reshape(..)].astype(bf16)

q, k and v are read in place through strided views (``views.resolve``):
``np.split`` of a fused QKV projection, reshapes into heads, transposes and
``np.repeat`` of the KV heads cost no copies.  The additive mask must be
large enough that exp() of a masked score underflows to exactly zero in
fp32, which makes it identical to dropping the key.
"""

from __future__ import annotations

from typing import List, Optional, Tuple

import numpy as np

from nkipy_amd.core import dtypes as dt
from nkipy_amd.core.backend.ir import Node, Value
from nkipy_amd.dispatch import launchers as LA
from nkipy_amd.dispatch.patterns import (
    LaunchStep, Match, RmsNormPattern, SoftmaxPattern, _users_of, op_of, scalar_value,
)
from nkipy_amd.dispatch.plan import Slot
from nkipy_amd.dispatch.views import View, _is_view_node, resolve

MASK_LIMIT = -1.0e4


def _contiguous(shape) -> List[int]:
    s, out = 1, []
    for n in reversed(shape):
        out.append(s)
        s *= int(n)
    return out[::-1]


def _const_payload(v: Value) -> Optional[np.ndarray]:
    if v.node is None or v.node.op != "constant":
        return None
    p = v.node.attrs["value"]
    return dt.to_float32(p) if p.dtype.fields is not None else np.asarray(p, np.float32)


def _owned(L, view: View, inside: set) -> List[Node]:
    """The view's layout nodes (and a constant base) if they feed only the match."""
    chain = list(view.nodes)
    if view.base.node is not None and view.base.node.op == "constant":
        chain.append(view.base.node)
    ids = set(inside) | {id(n) for n in chain}
    for n in chain:
        if n.out.id in L.result_ids or any(id(u) not in ids for u in _users_of(L, n.out)):
            return []
    return chain


def _bf16_view(v: Value) -> Optional[View]:
    vw = resolve(v)
    return vw if vw.base.dtype == dt.bfloat16 else None


# ---------------------------------------------------------------------------
# RoPE
# ---------------------------------------------------------------------------
class RopeMatch(Match):
    name = "rope"

    def __init__(self, nodes, x: View, x_half: int, cos: View, sin: View, roles, out: Value):
        ins = [x.base, cos.base, sin.base]
        super().__init__(nodes, list(dict.fromkeys(ins)), [out])
        self.x, self.x_half, self.cos, self.sin, self.roles, self.out = x, x_half, cos, sin, roles, out

    def steps(self, plan):
        x, cos, sin, out = self.x, self.cos, self.sin, self.out
        (B, S, H), x_str, o_str, t_ss = self.roles
        D = out.shape[-1]
        xi, ti = x.base.dtype.itemsize, 4

        def make(addr):
            return LA.rope(addr(x.base) + xi * x.offset, addr(cos.base) + ti * cos.offset,
                           addr(sin.base) + ti * sin.offset, addr(out), B, S, H, D,
                           x_str, o_str, self.x_half, t_ss)

        return [LaunchStep("rope", f"rope B={B} S={S} H={H} D={D}", self.inputs, self.outputs, make)]


class RopePattern:
    def find(self, L):
        for n in L.live:
            if n.op != "concatenate" or id(n) in L.covered:
                continue
            m = self._match(L, n)
            if m is not None and m.validate(L):
                yield m

    @staticmethod
    def _product(v: Value):
        """v = a * b with one bf16 activation view and one fp32 table view."""
        if op_of(v) != "multiply":
            return None
        for a, b in (v.node.inputs, v.node.inputs[::-1]):
            xa = _bf16_view(a)
            tb = resolve(b, widen_ok=False)
            if xa is not None and tb.base.dtype == dt.float32 and not tb.widened:
                return xa, tb, v.node
        return None

    def _match(self, L, n: Node):
        if len(n.inputs) != 2 or n.attrs["dimension"] != n.out.ndim - 1 or n.out.dtype != dt.float32:
            return None
        A, Bv = n.inputs
        nd = n.out.ndim
        half = A.shape[-1]
        if Bv.shape != A.shape or nd < 2 or nd > 4 or half % 8:
            return None
        if op_of(A) != "subtract" or op_of(Bv) != "add":
            return None
        pa = [self._product(t) for t in A.node.inputs]
        pb = [self._product(t) for t in Bv.node.inputs]
        if any(p is None for p in pa + pb):
            return None
        (x0, c0, m0), (x1, s0, m1) = pa
        key = lambda vw: (vw.base.id, vw.offset, [tuple(d) for d in vw.dims])
        # B = x0 * sin + x1 * cos, either order
        if key(pb[0][0]) == key(x0) and key(pb[1][0]) == key(x1):
            s1, c1 = pb[0][1], pb[1][1]
        elif key(pb[1][0]) == key(x0) and key(pb[0][0]) == key(x1):
            s1, c1 = pb[1][1], pb[0][1]
        else:
            return None
        if x0.base is not x1.base or [tuple(d) for d in x0.dims] != [tuple(d) for d in x1.dims]:
            return None
        x_half = x1.offset - x0.offset
        # the tables: one position axis, frequency contiguous, same content in both uses
        for ta, tb in ((c0, c1), (s0, s1)):
            pa_, pb_ = _const_payload(ta.base), _const_payload(tb.base)
            if ta.base is not tb.base:
                if pa_ is None or pb_ is None or not np.array_equal(ta.materialize_check(pa_),
                                                                    tb.materialize_check(pb_)):
                    return None
            elif key(ta) != key(tb):
                return None
        pos = [d for d in range(nd - 1) if c0.simple(d) != 0]
        if len(pos) != 1 or c0.simple(nd - 1) != 1 or x0.simple(nd - 1) != 1:
            return None
        sd = pos[0]
        if s0.simple(sd) != c0.simple(sd) or s0.simple(nd - 1) != 1 or \
                any(s0.simple(d) != 0 for d in range(nd - 1) if d != sd):
            return None
        rest = [d for d in range(nd - 1) if d != sd]
        xs = [x0.simple(d) for d in range(nd - 1)]
        if any(s is None for s in xs):
            return None
        out, tail = n.out, []
        us = _users_of(L, out)
        if out.id in L.result_ids or len(us) != 1 or us[0].op != "convert" or us[0].out.dtype != dt.bfloat16:
            return None
        tail.append(us[0])
        out = us[0].out
        ostr = _contiguous(out.shape)
        shape = out.shape
        # kernel roles: b = first other axis, h = second other axis, s = position axis
        b_ax = rest[0] if len(rest) >= 1 else None
        h_ax = rest[1] if len(rest) >= 2 else None
        size = lambda ax: shape[ax] if ax is not None else 1
        stride = lambda arr, ax: arr[ax] if ax is not None else 0
        roles = ((size(b_ax), shape[sd], size(h_ax)),
                 (stride(xs, b_ax), xs[sd], stride(xs, h_ax)),
                 (stride(ostr, b_ax), ostr[sd], stride(ostr, h_ax)),
                 c0.simple(sd))
        if c0.shape[sd] < shape[sd]:
            return None
        nodes = [n, A.node, Bv.node, m0, m1, pb[0][2], pb[1][2]] + tail
        inside = {id(q) for q in nodes}
        for vw in (c1, s1):
            if vw.base is not c0.base and vw.base is not s0.base:
                nodes += _owned(L, vw, inside)
        return RopeMatch(nodes, x0, x_half, c0, s0, roles, out)


# ---------------------------------------------------------------------------
# Per-head RMSNorm + RoPE in bf16 steps
# ---------------------------------------------------------------------------
class HeadRopeMatch(Match):
    """One or two tensors of heads (q, k) rotated with shared tables, each
    optionally normalised first: one ``nk_head_rope_bf16`` launch."""

    name = "head_rope"

    def __init__(self, nodes, inputs, outputs, members, table, bsd):
        super().__init__(nodes, inputs, outputs)
        self.members, self.table, self.bsd = members, table, bsd
        self.planes_src = None  # a GemmMatch whose partial sums this step adds (ProjectionPlanesFusion)

    def steps(self, plan):
        members, tb = self.members, self.table
        B, S, D = self.bsd

        planes = self.planes_src.planes if self.planes_src is not None else None

        def make(addr):
            specs = []
            for m in members:
                xv, nm = m["x"], m["norm"]
                o_sp, o_rows = m.get("o_pos", (0, 0))
                # the rows, or their fp32 partial sums at the same element offset
                x_ptr = addr(planes[0]) + 4 * xv.offset if planes else addr(xv.base) + 2 * xv.offset
                specs.append(LA.HeadRopeSpec(
                    x_ptr, addr(m["out"]), m["H"], m["x_str"], m["o_str"], m["x_half"],
                    norm=nm is not None, eps=nm.eps if nm is not None else 0.0,
                    w_ptr=addr(nm.w) if nm is not None and nm.w is not None else 0,
                    mul_recip=bool(nm.mul_recip) if nm is not None else False,
                    copy=m.get("copy", False), out_pos_stride=o_sp, out_positions=o_rows))
            te = 4 if tb["f32"] else 2
            return LA.head_rope(specs, addr(tb["cos"]) + te * tb["cos_off"], addr(tb["sin"]) + te * tb["sin_off"],
                                B, S, D, table_f32=tb["f32"],
                                pos_ptr=addr(tb["pos"]) if tb["pos"] is not None else 0,
                                table_row=tb["row"], table_stride=tb["ss"], table_rows=tb["rows"],
                                planes=(planes[2], planes[1]) if planes else None)

        parts = [(f"copy {m['H']} heads" if m.get("copy") else
                  f"{'rmsnorm + ' if m['norm'] is not None else ''}rope {m['H']} heads")
                 + (" -> cache row" if m.get("o_pos") else "") for m in members]
        desc = f"head rope B={B} S={S} D={D} bf16 steps: " + ", ".join(parts) + \
            (" (runtime position)" if tb["pos"] is not None else "") + \
            (f" from {planes[1]} partial-sum planes" if planes else "")
        return [LaunchStep("head_rope", desc, self.inputs, self.outputs, make)]


class HeadRopePattern:
    """Split-half RoPE whose products, sum and difference are bf16 arrays
    (examples/models/qwen3/kernels/rope.py:23-48 applied to bf16 q / k with
    the tables cast to bf16, attention.py:84-97)::

        out = concatenate([x0 * c - x1 * s, x0 * s + x1 * c], -1)     all bf16

    with c / s views of one position axis of a table that is an fp32
    constant cast to bf16, a bf16 array, or either taken at a runtime
    position (``cos[start_pos]``).  The tensors of heads rotated with the
    same tables (q and k) form one match, which also claims the table chain
    (cast, take, layout) and, for a tensor that is a per-head RMSNorm output
    read only by the rotation (attention.py:79-80), that norm and the views
    that feed it (the split of the fused QKV projection): the kernel reads
    the projection in place."""

    def find(self, L):
        members = []
        for n in L.live:
            if n.op == "concatenate" and id(n) not in L.covered:
                m = self._member(L, n)
                if m is not None:
                    members.append(m)
        groups = {}
        for m in members:
            groups.setdefault(m["tkey"], []).append(m)
        for ms in groups.values():
            i = 0
            while i < len(ms):
                match = self._build(L, ms[i:i + 2]) if i + 1 < len(ms) else None
                if match is not None:
                    i += 2
                    yield match
                    continue
                match = self._build(L, ms[i:i + 1])
                i += 1
                if match is not None:
                    yield match

    # -- one rotated tensor ----------------------------------------------
    @staticmethod
    def _key(vw: View):
        return vw.base.id, vw.offset, [tuple(d) for d in vw.dims]

    def _member(self, L, n: Node):
        if len(n.inputs) != 2 or n.out.dtype != dt.bfloat16 or n.out.ndim != 4 or n.attrs["dimension"] != 3:
            return None
        A, Bv = n.inputs
        D = n.out.shape[-1]
        half = D // 2
        if op_of(A) != "subtract" or op_of(Bv) != "add" or A.shape != Bv.shape or A.shape[-1] * 2 != D:
            return None
        if D % 16 or D > 128 or any(v.dtype != dt.bfloat16 for v in (A, Bv)):
            return None
        muls = list(A.node.inputs) + list(Bv.node.inputs)
        if any(op_of(v) != "multiply" or v.dtype != dt.bfloat16 for v in muls):
            return None
        ops = [[resolve(u, widen_ok=False) for u in v.node.inputs] for v in muls]
        if any(o.base.dtype != dt.bfloat16 for pair in ops for o in pair):
            return None
        # the activation: the base that is one operand of every product
        for xb in dict.fromkeys(o.base.id for o in ops[0]):
            sides = []
            for pair in ops:
                hit = [k for k in (0, 1) if pair[k].base.id == xb]
                if len(hit) != 1:
                    break
                sides.append((pair[hit[0]], pair[1 - hit[0]]))
            else:
                m = self._roles(L, n, sides, muls, half)
                if m is not None:
                    return m
        return None

    def _roles(self, L, n, sides, muls, half):
        (x0, c0), (x1, s0) = sides[0], sides[1]
        key = self._key
        # second half: x0 * s + x1 * c, either order
        if key(sides[2][0]) == key(x0) and key(sides[3][0]) == key(x1):
            s1, c1 = sides[2][1], sides[3][1]
        elif key(sides[3][0]) == key(x0) and key(sides[2][0]) == key(x1):
            s1, c1 = sides[3][1], sides[2][1]
        else:
            return None
        if key(c1) != key(c0) or key(s1) != key(s0) or key(c0) == key(s0):
            return None
        if [tuple(d) for d in x0.dims] != [tuple(d) for d in x1.dims]:
            return None
        B, S, H, D = n.out.shape
        xs = [x0.simple(d) for d in range(4)]
        if any(v is None for v in xs) or xs[3] != 1:
            return None
        x_half = x1.offset - x0.offset
        # tables: frequency contiguous, broadcast over batch and heads
        geo = []
        for tv in (c0, s0):
            st = [tv.simple(d) for d in range(4)]
            if any(v is None for v in st) or st[3] != 1 or st[0] != 0 or st[2] != 0:
                return None
            geo.append(st[1])
        if geo[0] != geo[1]:
            return None
        tc, ts = self._table(L, c0), self._table(L, s0)
        if tc is None or ts is None or tc["kind"] != ts["kind"] or tc["f32"] != ts["f32"] or \
                tc["pos_id"] != ts["pos_id"] or tc["row"] != ts["row"] or tc["rows"] != ts["rows"]:
            return None
        nodes = [n, n.inputs[0].node, n.inputs[1].node] + [v.node for v in muls]
        chain = []  # layout / table nodes, claimed when nothing else reads them
        for vw in (x0, x1, c0, s0, c1, s1):
            chain += vw.nodes
        chain += tc["nodes"] + ts["nodes"]
        table = {"f32": tc["f32"], "cos": tc["value"], "sin": ts["value"], "cos_off": tc["off"],
                 "sin_off": ts["off"], "pos": tc["pos"], "row": tc["row"], "rows": tc["rows"], "ss": geo[0]}
        tkey = (tc["value"].id, ts["value"].id, tc["off"], ts["off"], tc["pos_id"], geo[0], tc["f32"], B, S, D)
        return {"n": n, "nodes": nodes, "chain": chain, "x": x0, "x_str": tuple(xs[:3]), "x_half": x_half,
                "H": H, "out": n.out, "o_str": tuple(_contiguous(n.out.shape)[:3]), "norm": None,
                "bsd": (B, S, D), "table": table, "tkey": tkey}

    @staticmethod
    def _table(L, tv: View):
        """A bf16 table view: (value read by the kernel, element offset,
        fp32?, runtime row, nodes between)."""
        T = tv.base

        def cast_const(v):
            if op_of(v) == "convert" and v.dtype == dt.bfloat16 and v.node.inputs[0].dtype == dt.float32 \
                    and op_of(v.node.inputs[0]) == "constant":
                return v.node.inputs[0]
            return None

        if op_of(T) == "take" and T.node.attrs.get("axis") == 0 and T.ndim == 2:
            src, idx = T.node.inputs
            if idx.size != 1 or idx.dtype not in (dt.int32,) or src.ndim != 2 or tv.offset >= src.shape[1]:
                return None
            c = cast_const(src)
            val, f32, nodes = (c, True, [T.node, src.node]) if c is not None else (src, False, [T.node])
            if not f32 and src.dtype != dt.bfloat16:
                return None
            return {"kind": "take", "value": val, "off": tv.offset, "f32": f32, "pos": idx, "pos_id": idx.id,
                    "row": src.shape[1], "rows": src.shape[0], "nodes": nodes}
        c = cast_const(T)
        if c is not None:
            return {"kind": "table", "value": c, "off": tv.offset, "f32": True, "pos": None, "pos_id": None,
                    "row": 0, "rows": 1, "nodes": [T.node]}
        if T.dtype == dt.bfloat16:
            return {"kind": "table", "value": T, "off": tv.offset, "f32": False, "pos": None, "pos_id": None,
                    "row": 0, "rows": 1, "nodes": []}
        return None

    # -- the RMSNorm that produced a rotated tensor ------------------------
    @staticmethod
    def _norm(L, m):
        """(norm match, view of its input rows) when the rotated tensor is
        exactly the output of a per-head RMSNorm over D (no residual)."""
        X = m["x"].base
        B, S, D = m["bsd"]
        dense = tuple(_contiguous(X.shape)[:3])
        if X.shape != (B, S, m["H"], D) or m["x"].offset != 0 or m["x_half"] != D // 2 or \
                any(n > 1 and a != b for n, a, b in zip(X.shape, m["x_str"], dense)) or X.id in L.result_ids:
            return None
        cands, cur = [], X.node
        if cur is not None and cur.op == "convert":
            cur = cur.inputs[0].node
        if cur is not None and cur.op == "multiply":
            cands.append(cur)
            cands += [v.node for v in cur.inputs if v.node is not None and v.node.op in ("divide", "multiply")]
        elif cur is not None and cur.op == "divide":
            cands.append(cur)
        pat = RmsNormPattern()
        for q in cands:
            nm = pat._match(L, q)
            if nm is None or nm.y is not X or nm.r is not None or nm.x.dtype != dt.bfloat16:
                continue
            if nm.w is not None and (nm.w.dtype != dt.bfloat16 or nm.w.shape != (D,)):
                continue
            xv = resolve(nm.x, widen_ok=False)
            if xv.base.dtype != dt.bfloat16 or xv.shape != (B, S, m["H"], D):
                continue
            st = [xv.simple(d) for d in range(4)]
            if any(v is None for v in st) or st[3] != 1:
                continue
            return nm, xv, tuple(st[:3])
        return None

    # -- the match ----------------------------------------------------------
    def _build(self, L, ms):
        t0 = ms[0]["table"]
        use = []
        for m in ms:
            m = dict(m)
            nr = self._norm(L, m)
            if nr is not None:
                nm, xv, st = nr
                m.update(norm=nm, x=xv, x_str=st, x_half=m["bsd"][2] // 2)
                m["nodes"] = m["nodes"] + nm.node_list
                m["chain"] = m["chain"] + xv.nodes
            use.append(m)
        attempts = [use, [dict(m, norm=None, x=o["x"], x_str=o["x_str"], x_half=o["x_half"],
                               nodes=o["nodes"], chain=o["chain"]) for m, o in zip(use, ms)]]
        written = self._cache_writes(L, use, t0)
        if written is not None:
            attempts.insert(0, written)
        for attempt in attempts:
            match = self._claim(L, attempt, t0)
            if match is not None:
                return match
        return None

    # -- the cache writes of one decode token --------------------------------
    @staticmethod
    def _scatter(L, node, pos, B, H, D):
        """``cache[:, pos] = src`` (attention.py:101-105 with start_pos) as
        an in-place update of a cache argument the kernel's output aliases
        (the caller's buffer is written, as the scatter kernel writes it):
        (node, cache rows, output strides, runtime position stride)."""
        if node.op != "scatter_along_axis" or id(node) in L.covered or node.attrs.get("axis") != 1 or \
                node.inputs[1] is not pos:
            return None
        P, _, src = node.inputs
        if not P.is_parameter or P.dtype != dt.bfloat16 or P.ndim != 4 or P.shape[0] != B or \
                tuple(P.shape[2:]) != (H, D) or tuple(src.shape) != (B, 1, H, D):
            return None
        if len(L.users.get(P.id, [])) != 1:  # nothing else reads the cache before its update
            return None
        if not any(L.g.results[a.output_index] is node.out and f"{a.param_name}.must_alias_input" == P.name
                   for a in L.g.aliases):
            return None
        A = P.shape[1]
        return {"node": node, "src": src, "out": node.out, "o_str": (A * H * D, 0, D), "o_pos": (H * D, A)}

    def _cache_writes(self, L, ms, tb):
        """The decode form (one token, tables taken at the runtime position,
        q and a normalised k of one projection): k written into its cache
        row by the launch instead of by a scatter step, and the v heads of
        the same projection copied into theirs (a third target).  Returns
        the members with those writes, or None."""
        if len(ms) != 2 or tb["pos"] is None or ms[0]["bsd"][1] != 1:
            return None
        B, _, D = ms[0]["bsd"]
        pos = tb["pos"]
        kk = [i for i, m in enumerate(ms) if m["norm"] is not None and m["out"].id not in L.result_ids
              and len(L.users.get(m["out"].id, [])) == 1]
        for i in kk:
            km = ms[i]
            kw = self._scatter(L, L.users[km["out"].id][0], pos, B, km["H"], D)
            if kw is None or kw["src"] is not km["out"]:
                continue
            base = km["x"].base
            for n in L.live:
                if n is kw["node"] or n.op != "scatter_along_axis":
                    continue
                src = n.inputs[2]
                vv = resolve(src, widen_ok=False)
                if vv.base is not base or src.ndim != 4:
                    continue
                vw = self._scatter(L, n, pos, B, src.shape[2], D)
                if vw is None:
                    continue
                st = [vv.simple(d) for d in range(4)]
                if any(v is None for v in st) or st[3] != 1:
                    continue
                out = [dict(m) for m in ms]
                out[i].update(out=kw["out"], o_str=kw["o_str"], o_pos=kw["o_pos"],
                              nodes=km["nodes"] + [kw["node"]])
                out.append({"n": n, "nodes": [n], "chain": list(vv.nodes), "x": vv, "x_str": tuple(st[:3]),
                            "x_half": D // 2, "H": src.shape[2], "out": vw["out"], "o_str": vw["o_str"],
                            "o_pos": vw["o_pos"], "norm": None, "copy": True, "bsd": km["bsd"]})
                return out
        return None

    @staticmethod
    def _claim(L, ms, tb):
        core = []
        for m in ms:
            core += m["nodes"]
        core_ids = {id(q) for q in core}
        # layout and table nodes that nothing outside the match reads
        chain = [q for q in dict.fromkeys(q for m in ms for q in m["chain"]) if id(q) not in core_ids]
        owned = {id(q) for q in chain}
        changed = True
        while changed:
            changed = False
            for q in chain:
                if id(q) not in owned:
                    continue
                if q.out.id in L.result_ids or any(id(u) not in core_ids and id(u) not in owned
                                                   for u in L.users.get(q.out.id, [])):
                    owned.discard(id(q))
                    changed = True
        nodes = core + [q for q in chain if id(q) in owned]
        node_ids = {id(q) for q in nodes}
        inputs = []
        for m in ms:
            inputs.append(m["x"].base)
            if m["norm"] is not None and m["norm"].w is not None:
                inputs.append(m["norm"].w)
        inputs += [tb["cos"], tb["sin"]] + ([tb["pos"]] if tb["pos"] is not None else [])
        if any(v.node is not None and id(v.node) in node_ids for v in inputs):
            return None
        match = HeadRopeMatch(nodes, list(dict.fromkeys(inputs)), [m["out"] for m in ms], ms, tb, ms[0]["bsd"])
        if not match.validate(L):
            return None
        # the outputs are written at the last claimed node: nothing may read
        # them earlier
        order = {id(q): i for i, q in enumerate(L.live)}
        last = order[id(match.last)]
        for m in ms:
            if any(order.get(id(u), last + 1) <= last and id(u) not in node_ids
                   for u in L.users.get(m["out"].id, [])):
                return None
        return match


# ---------------------------------------------------------------------------
# RoPE folded into the QKV projection
# ---------------------------------------------------------------------------
class QkvRopeMatch(Match):
    """A bf16 QKV projection whose q and k heads (128 wide, columns 0 ..
    nq + nk - 1) feed only the two RoPE matches: one GEMM launch rotates them
    in its epilogue (csrc/kernels/gemm.hip, ``gemm_epilogue_rope``) and writes
    the RoPE outputs directly; the projection value keeps its remaining (v)
    columns.  Emitted where the GEMM was."""

    name = "gemm_rope"

    def __init__(self, gm, rq: RopeMatch, rk: RopeMatch, last: Node):
        ins = list(dict.fromkeys(list(gm.inputs) + [rq.cos.base, rq.sin.base]))
        super().__init__(gm.node_list + rq.node_list + rk.node_list, ins, [gm.out, rq.out, rk.out])
        self.gm, self.rq, self.rk = gm, rq, rk
        self.last = last

    def steps(self, plan):
        gm, rq, rk = self.gm, self.rq, self.rk
        x, w, out = gm.x, gm.w, gm.out
        K = x.shape[-1]
        M = x.size // K
        N = out.shape[-1]
        ldb = w.value.shape[1]
        (_, S, Hq), _, _, t_ss = rq.roles
        Hk = rk.roles[0][2]
        hd = LA.GemmRope.HEAD_DIM
        cos, sin = rq.cos, rq.sin

        def make(addr):
            rope = LA.GemmRope(addr(cos.base) + 4 * cos.offset, addr(sin.base) + 4 * sin.offset,
                               addr(rq.out), addr(rk.out), t_ss, S, Hq * hd, Hk * hd)
            return LA.gemm(addr(x), addr(w.value), addr(out), M, N, K, layout=w.layout,
                           b_dtype=w.value.dtype, c_dtype=out.dtype, ldb=ldb,
                           scale_ptr=addr(w.scale) if w.scale is not None else 0, rope=rope)

        desc = (f"gemm {w.layout} M={M} N={N} K={K} {dt.name(w.value.dtype)} -> bf16 "
                f"+rope q {Hq}x{hd} k {Hk}x{hd}")
        return [LaunchStep("gemm_rope", desc, self.inputs, self.outputs, make)]


def _first_column(vw: View, n_cols: int) -> int:
    """Smallest column of a row-major (.., n_cols) base that ``vw`` reads
    (0 when its columns may wrap into the next row)."""
    span = sum((n - 1) * s for d in vw.dims for n, s in d if n > 1 and s % n_cols)
    c = vw.offset % n_cols
    return c if c + span < n_cols else 0


class ProjectionPlanesFusion:
    """Hands the fp32 partial sums of a few-row projection straight to the
    head prologue that is its only reader (the Qwen3 decode step: the QKV
    projection of one token per sequence, then q / k norm, RoPE and the
    cache writes, examples/models/qwen3/kernels/attention.py:44-97).  The
    prologue adds the planes in the projection's reduction order
    (``LA.head_rope(planes=...)``), so the bf16 projection output is never
    written and its reduction launch is saved.  Taken only when the
    projection has no epilogue terms (no scale, bias, residual or SwiGLU)
    and writes bf16; the projection decides at step time whether its form
    has planes (``GemmMatch.planes``).  Finds nothing on its own."""

    def find(self, L):
        return iter(())

    def refine(self, L):
        from nkipy_amd.dispatch.patterns_gemm import GemmMatch

        gemms = {m.out.id: m for m in L.matches if isinstance(m, GemmMatch)}
        for hm in [m for m in L.matches if isinstance(m, HeadRopeMatch)]:
            bases = {L.match_alias.get(mb["x"].base.id, mb["x"].base).id for mb in hm.members}
            if len(bases) != 1:
                continue
            gm = gemms.get(bases.pop())
            if gm is None or not self._eligible(L, gm, hm):
                continue
            gm.planes_consumer = hm
            hm.planes_src = gm

    @staticmethod
    def _eligible(L, gm, hm) -> bool:
        out = gm.out
        if (gm.up is not None or gm.bias is not None or gm.resid is not None or gm.w.scale is not None
                or out.dtype != dt.bfloat16 or not gm.split_k or out.id in L.result_ids
                or (gm.n_out is not None and gm.n_out != out.shape[-1])):
            return False
        # every reader of the projection (through views) is the prologue
        work, seen = [out], {out.id}
        while work:
            v = work.pop()
            for u in L.users.get(v.id, ()):
                m = L.covered.get(id(u))
                if m is hm:
                    continue
                if m is None and _is_view_node(u, True) and u.out.id not in L.result_ids:
                    if u.out.id not in seen:
                        seen.add(u.out.id)
                        work.append(u.out)
                    continue
                return False
        return True


class QkvRopeFusion:
    """Merges a QKV :class:`GemmMatch` with the RoPE matches of its q and k
    heads (examples/models/qwen3/kernels/attention.py:44-66, tests/kernels/
    llama_decoder_dynamo.py:150-178: split of the fused projection into
    heads, then the split-half rotation).  Runs after every pattern has
    claimed its nodes; finds nothing on its own."""

    def find(self, L):
        return iter(())

    def refine(self, L):
        from nkipy_amd.dispatch.patterns_gemm import GemmMatch

        ropes = {}
        for m in L.matches:
            if isinstance(m, RopeMatch):
                base = L.match_alias.get(m.x.base.id, m.x.base)
                ropes.setdefault(base.id, []).append(m)
        for gm in [m for m in L.matches if isinstance(m, GemmMatch)]:
            rs = ropes.get(gm.out.id, [])
            if len(rs) != 2:
                continue
            rq, rk = sorted(rs, key=lambda r: r.x.offset)
            fused = self._fuse(L, gm, rq, rk)
            if fused is None:
                continue
            for m in (gm, rq, rk):
                L.matches.remove(m)
            L.matches.append(fused)
            for nid in fused.nodes:
                L.covered[nid] = fused

    @staticmethod
    def _fuse(L, gm, rq, rk) -> Optional[QkvRopeMatch]:
        hd = LA.GemmRope.HEAD_DIM
        out, x, w = gm.out, gm.x, gm.w
        if gm.up is not None or gm.bias is not None or gm.resid is not None or out.dtype != dt.bfloat16:
            return None
        if w.value.dtype == dt.float8_e4m3fn and w.layout == "nn":
            return None  # no 8-wave kernel
        if out.id in L.result_ids:
            return None
        K = x.shape[-1]
        M, N = x.size // K, out.shape[-1]
        col0 = 0
        for r in (rq, rk):
            (Bs, S, H), xs, os_, _ = r.roles
            if r.out.shape[-1] != hd or r.x_half != hd // 2 or Bs * S != M:
                return None
            if xs[1] != N or (H > 1 and xs[2] != hd) or (Bs > 1 and xs[0] != S * N):
                return None
            if tuple(os_) != (S * H * hd, H * hd, hd) or r.x.offset != col0:
                return None
            col0 += H * hd
        if col0 > N or rq.roles[0][1] != rk.roles[0][1] or rq.roles[3] != rk.roles[3]:
            return None
        # RopePattern fixed each table's layout (position stride roles[3],
        # frequency contiguous); the views differ only in broadcast axes
        for a, b in ((rq.cos, rk.cos), (rq.sin, rk.sin)):
            if a.offset != b.offset:
                return None
            if a.base is not b.base:  # each rotation traced its own copy of the table
                pa, pb = _const_payload(a.base), _const_payload(b.base)
                if pa is None or pb is None or not np.array_equal(pa, pb):
                    return None
            base = a.base
            if not (base.is_parameter or (base.node is not None and base.node.op == "constant")):
                return None  # the tables must exist where the GEMM runs
        # nothing but the two rotations may read the q / k columns
        allowed = (id(rq), id(rk))
        work, seen = [out], {out.id}
        while work:
            v = work.pop()
            for u in L.users.get(v.id, ()):
                m = L.covered.get(id(u))
                if m is not None and id(m) in allowed:
                    continue
                if m is None and _is_view_node(u, True):
                    if u.out.id in L.result_ids:  # a result copied out of these columns
                        vw = resolve(u.out)
                        if L.match_alias.get(vw.base.id, vw.base) is not out or _first_column(vw, N) < col0:
                            return None
                    if u.out.id not in seen:
                        seen.add(u.out.id)
                        work.append(u.out)
                    continue
                vw = resolve(v)
                if L.match_alias.get(vw.base.id, vw.base) is not out or _first_column(vw, N) < col0:
                    return None
        order = {id(n): i for i, n in enumerate(L.live)}
        return QkvRopeMatch(gm, rq, rk, gm.last if gm.last is not None else
                            max(gm.node_list, key=lambda n: order[id(n)]))


# ---------------------------------------------------------------------------
# causal GQA attention
# ---------------------------------------------------------------------------
class AttentionMatch(Match):
    name = "attention"

    def __init__(self, nodes, q: View, k: View, v: View, out: Value, dims, scale, causal, o_str,
                 score_flags: int = 0, divisor: float = None, keys: int = None):
        ins = list(dict.fromkeys([q.base, k.base, v.base]))
        super().__init__(nodes, ins, [out])
        self.q, self.k, self.v, self.out = q, k, v, out
        self.dims, self.scale, self.causal, self.o_str = dims, scale, causal, o_str
        self.score_flags, self.divisor = score_flags, divisor
        self.keys = keys if keys is not None else dims[1]

    def steps(self, plan):
        q, k, v, out = self.q, self.k, self.v, self.out
        B, S, Hq, Hkv, D, strides = self.dims

        # the bf16 softmax takes each query's max score and weight sum from
        # passes of its own
        rm = None
        if self.score_flags & LA.ATT_SOFTMAX_BF16:
            rm = Slot(plan.add_buffer(LA.attention_rowstat_bytes(B, S, Hq, self.causal), "temp",
                                      "attention.rowstat"))

        def make(addr):
            return LA.attention(addr(q.base) + 2 * q.offset, addr(k.base) + 2 * k.offset,
                                addr(v.base) + 2 * v.offset, addr(out), B, S, Hq, Hkv, D,
                                self.scale, dict(strides, o=self.o_str), causal=self.causal,
                                score_flags=self.score_flags, divisor=self.divisor,
                                rowstat_ptr=addr(rm) if rm is not None else 0)

        desc = f"{'causal ' if self.causal else ''}attention B={B} S={S} Hq={Hq} Hkv={Hkv} D={D}"
        if self.keys != S:
            desc += f" keys<{S} of {self.keys}"
        if self.score_flags:
            desc += f" score_flags={self.score_flags}"
        return [LaunchStep("attention", desc, self.inputs, self.outputs, make)]


def _qk_dot(n: Node) -> bool:
    at = n.attrs
    return (n.op == "dot" and n.out.ndim == 4 and tuple(at["lhs_batch"]) == (0, 1)
            and tuple(at["rhs_batch"]) == (0, 1) and tuple(at["lhs_contract"]) == (3,)
            and tuple(at["rhs_contract"]) == (2,))


class AttentionPattern:
    """Prefill attention in two traced forms:

    * fp32 scores (tests/kernels/llama_decoder_dynamo.py:180-288): the
      product (bf16 operands, fp32 result) scaled, plus an (S, S) causal
      mask, fp32 softmax;
    * bf16 scores over a KV cache (examples/models/qwen3/kernels/
      attention.py:109-140): the product rounded to bf16, divided by sqrt(d)
      in fp32, rounded to bf16, plus the mask rows [:S, :MAXS] of a constant
      (MAXS, MAXS) triu mask (cast to bf16), softmax in bf16, @ v over all
      MAXS cache rows.  Keys at S and beyond are masked for every query, so
      the kernel reads the first S cache rows only; the cast points of the
      score go to the kernel as ATT_* flags."""

    def find(self, L):
        for n in L.live:
            if id(n) in L.covered or not _qk_dot(n):
                continue
            m = self._match(L, n)
            if m is not None and m.validate(L):
                yield m

    @staticmethod
    def _mask(v: Value, S: int, Sk: int):
        """An additive causal mask over (b, h, s, t), t < Sk -> (view, cast
        node or None), or None.  Its base is a constant, or a constant cast
        to a float type (which keeps zeros and values <= MASK_LIMIT)."""
        mv = resolve(v, widen_ok=False)
        cast, base = None, mv.base
        if op_of(base) == "convert" and op_of(base.node.inputs[0]) == "constant" and \
                base.dtype in (dt.float32, dt.bfloat16, dt.float16):
            cast, base = base.node, base.node.inputs[0]
        payload = _const_payload(base)
        if payload is None or mv.shape[-2:] != (S, Sk) or Sk < S:
            return None
        if mv.simple(0) != 0 or mv.simple(1) != 0:
            return None
        m = mv.materialize_check(payload.reshape(base.shape))[0, 0]
        lower = np.tril(np.ones((S, Sk), bool))
        if np.any(m[lower] != 0) or np.any(m[~lower] > MASK_LIMIT):
            return None
        return mv, cast

    @staticmethod
    def _score_chain(v: Value):
        """The score before the mask -> (dot node, scale, divisor, flags,
        nodes): [convert bf16] <- (multiply | divide by a scalar) <-
        [convert f32] <- dot, or the fp32 form without casts."""
        flags, nodes = 0, []
        if op_of(v) == "convert" and v.dtype == dt.bfloat16 and v.node.inputs[0].dtype == dt.float32:
            flags |= LA.ATT_RND_SCORE
            nodes.append(v.node)
            v = v.node.inputs[0]
        if v.dtype != dt.float32:
            return None
        scale, divisor = 1.0, None
        if op_of(v) in ("multiply", "divide"):
            a, c = v.node.inputs
            if op_of(v) == "multiply" and scalar_value(a)[0] is not None:
                a, c = c, a
            cv, cn = scalar_value(c)
            if cv is None or not cv > 0:
                return None
            if op_of(v) == "divide":
                scale, divisor = 1.0 / cv, float(cv)
            else:
                scale = float(cv)
            nodes += [v.node] + cn
            v = a
        if op_of(v) == "convert" and v.dtype == dt.float32 and v.node.inputs[0].dtype == dt.bfloat16:
            nodes.append(v.node)
            v = v.node.inputs[0]
        if op_of(v) != "dot" or not _qk_dot(v.node):
            return None
        d1 = v.node
        if d1.out.dtype == dt.bfloat16:
            flags |= LA.ATT_RND_PROD
        elif d1.out.dtype != dt.float32:
            return None
        if flags and divisor is not None:
            flags |= LA.ATT_DIVIDE
        return d1, scale, divisor, flags, nodes

    def _match(self, L, n2: Node):
        p_val, kv_op = n2.inputs
        nodes = [n2]
        while op_of(p_val) in ("convert", "copy") and p_val.dtype == dt.float32:
            nodes.append(p_val.node)
            p_val = p_val.node.inputs[0]
        if op_of(p_val) != "divide" or p_val.dtype not in (dt.float32, dt.bfloat16):
            return None
        st = SoftmaxPattern.structure(L, p_val.node)
        if st is None:
            return None
        X, smx = st
        nodes += smx
        Sq, Sk = X.shape[-2], X.shape[-1]
        causal, mask_nodes = False, None
        sc = self._score_chain(X)
        if sc is None and op_of(X) == "add":
            for a, b in (X.node.inputs, X.node.inputs[::-1]):
                sc = self._score_chain(a)
                if sc is None:
                    continue
                mk = self._mask(b, Sq, Sk)
                if mk is None:
                    sc = None
                    continue
                causal = True
                nodes.append(X.node)
                mask_nodes = mk
                break
        if sc is None:
            return None
        d1, scale, divisor, score_flags, snodes = sc
        # a bf16 softmax runs on bf16 scores: the score must have been cast
        if p_val.dtype == dt.bfloat16:
            if not score_flags & LA.ATT_RND_SCORE:
                return None
            score_flags |= LA.ATT_SOFTMAX_BF16
        nodes += [d1] + snodes
        q = _bf16_view(d1.inputs[0])
        k = _bf16_view(d1.inputs[1])
        v = _bf16_view(kv_op)
        if q is None or k is None or v is None:
            return None
        B, Hq, S, D = q.shape
        # keys past the queries exist only under a causal mask, which hides them
        if Sk != S and not causal:
            return None
        if k.shape != (B, Hq, D, Sk) or v.shape != (B, Hq, Sk, D) or n2.out.shape != (B, Hq, S, D):
            return None
        qs = [q.simple(0), q.simple(2), q.simple(1)]
        kg, vg = k.grouped(1), v.grouped(1)
        ks = [k.simple(0), k.simple(3)]
        vs = [v.simple(0), v.simple(2)]
        if None in qs + ks + vs or kg is None or vg is None:
            return None
        if q.simple(3) != 1 or k.simple(2) != 1 or v.simple(3) != 1:
            return None
        if kg[0] != vg[0] or kg[2] != vg[2] or kg[0] * kg[2] != Hq:
            return None
        Hkv = kg[0]
        # output tail: transposes, casts and a reshape after the second product
        out, perm, reshaped = n2.out, [0, 1, 2, 3], False
        while True:
            us = _users_of(L, out)
            if out.id in L.result_ids or len(us) != 1:
                break
            u = us[0]
            if u.op == "transpose" and not reshaped:
                perm = [perm[p] for p in u.attrs["permutation"]]
            elif u.op in ("convert", "copy") and (u.out.dtype == out.dtype or (
                    out.dtype == dt.float32 and u.out.dtype == dt.bfloat16)):
                pass
            elif u.op == "reshape" and not reshaped:
                reshaped = True
            else:
                break
            nodes.append(u)
            out = u.out
        if out.dtype != dt.bfloat16 or perm not in ([0, 1, 2, 3], [0, 2, 1, 3]):
            return None
        logical = [(B, Hq, S, D)[p] for p in perm]
        cs = _contiguous(logical)
        pos = {ax: i for i, ax in enumerate(perm)}  # dot axis -> position in the output
        o_str = (cs[pos[0]], cs[pos[2]], cs[pos[1]])
        try:
            LA.attention(16, 16, 16, 16, B, S, Hq, Hkv, D, scale,
                         {"q": qs, "k": (ks[0], ks[1], kg[1]), "v": (vs[0], vs[1], vg[1]), "o": o_str},
                         causal=causal, score_flags=score_flags, divisor=divisor, rowstat_ptr=16)
        except LA.LaunchError:
            return None
        if any((vw.offset * 2) % 16 for vw in (q, k, v)):
            return None
        if mask_nodes:
            mv, cast = mask_nodes
            inside = {id(x) for x in nodes}
            chain = _owned(L, mv, inside)
            nodes += chain
            if cast is not None and chain:  # the cast and its constant, if only this mask reads them
                own = inside | {id(x) for x in chain}
                cnode = cast.inputs[0].node
                if cast.out.id not in L.result_ids and all(id(u) in own for u in _users_of(L, cast.out)):
                    nodes.append(cast)
                    own.add(id(cast))
                    if cnode.out.id not in L.result_ids and all(id(u) in own for u in _users_of(L, cnode.out)):
                        nodes.append(cnode)
        strides = {"q": tuple(qs), "k": (ks[0], ks[1], kg[1]), "v": (vs[0], vs[1], vg[1])}
        return AttentionMatch(nodes, q, k, v, out, (B, S, Hq, Hkv, D, strides), scale, causal, o_str,
                              score_flags, divisor, Sk)


# ---------------------------------------------------------------------------
# decode attention: one query token against a KV cache
# ---------------------------------------------------------------------------
class DecodeAttentionMatch(Match):
    name = "decode_attention"

    def __init__(self, nodes, q: View, k: View, v: View, pos: Value, out: Value, dims, scale, flags, o_str):
        ins = list(dict.fromkeys([q.base, k.base, v.base, pos]))
        super().__init__(nodes, ins, [out])
        self.q, self.k, self.v, self.pos, self.out = q, k, v, pos, out
        self.dims, self.scale, self.flags, self.o_str = dims, scale, flags, o_str

    def steps(self, plan):
        q, k, v, out, pos = self.q, self.k, self.v, self.out, self.pos
        B, Sk, Hq, Hkv, D, strides = self.dims
        ws = Slot(plan.add_buffer(LA.decode_attention_workspace_bytes(B, Sk, Hq), "temp",
                                  "decode_attention.workspace"))

        def make(addr):
            return LA.decode_attention(addr(q.base) + 2 * q.offset, addr(k.base) + 2 * k.offset,
                                       addr(v.base) + 2 * v.offset, addr(out), addr(pos), B, Sk, Hq, Hkv, D,
                                       self.scale, dict(strides, o=self.o_str), self.flags, ws_ptr=addr(ws))

        desc = f"decode attention B={B} cache={Sk} Hq={Hq} Hkv={Hkv} D={D} flags={self.flags}"
        return [LaunchStep("decode_attention", desc, self.inputs, self.outputs, make)]


class DecodeAttentionPattern:
    """The decode step of examples/models/qwen3/kernels/attention.py:100-140:
    one query position, keys and values from the (just updated) cache with
    ``np.repeat`` GQA, scores scaled and optionally cast to bf16, plus the
    causal-mask row of the runtime position, softmax, weighted values::

        s = (q @ k_t) / c  [.astype(bf16)]      q (B, H, 1, D)
        s = s + mask[start_pos, :S]             mask = triu(<= -1e4, k=1)
        o = softmax(s) @ v
    """

    def find(self, L):
        for n in L.live:
            if id(n) in L.covered or not _qk_dot(n) or n.out.shape[2:3] != (1,):
                continue
            m = self._match(L, n)
            if m is not None and m.validate(L):
                yield m

    @staticmethod
    def _mask_row(L, v: Value, Sk: int):
        """mask[pos, :Sk] broadcast over (b, h) -> (pos value, nodes), with
        the mask a causal constant and pos an int32 scalar tensor."""
        nodes = []
        while op_of(v) in ("broadcast_in_dim", "reshape"):
            nodes.append(v.node)
            v = v.node.inputs[0]
        if op_of(v) == "slice":
            at = v.node.attrs
            if any(st != 0 for st in at["start_indices"]) or any(sd != 1 for sd in at["strides"]):
                return None
            nodes.append(v.node)
            v = v.node.inputs[0]
        if op_of(v) != "take" or v.node.attrs["axis"] != 0 or v.shape[-1] != Sk:
            return None
        tk = v.node
        C, pos = tk.inputs
        if pos.dtype != dt.int32 or pos.size != 1:
            return None
        cast = None
        if op_of(C) == "convert" and op_of(C.node.inputs[0]) == "constant":
            cast, C = C.node, C.node.inputs[0]  # a float constant cast to the score dtype
        payload = _const_payload(C)
        if payload is None or payload.ndim != 2 or payload.shape[0] != payload.shape[1] or payload.shape[1] < Sk:
            return None
        m = payload[:, :Sk]
        lower = np.tril(np.ones(m.shape, bool))
        if np.any(m[lower] != 0) or np.any(m[~lower] > MASK_LIMIT):
            return None
        nodes.append(tk)
        chain = ([cast] if cast is not None else []) + [C.node]
        own = {id(tk)}
        for cn in chain:  # the cast and the constant, if only this mask uses them
            if cn.out.id in L.result_ids or any(id(u) not in own for u in _users_of(L, cn.out)):
                break
            nodes.append(cn)
            own.add(id(cn))
        return pos, nodes

    def _match(self, L, n2: Node):
        p_val, v_op = n2.inputs
        nodes = [n2]
        if op_of(p_val) != "divide" or p_val.dtype not in (dt.bfloat16, dt.float32):
            return None
        st = SoftmaxPattern.structure(L, p_val.node)
        if st is None:
            return None
        X, smx = st
        nodes += smx
        flags = LA.DEC_SOFTMAX_BF16 if p_val.dtype == dt.bfloat16 else 0
        if op_of(X) != "add":
            return None
        Sk = X.shape[-1]
        sc = mask = None
        for a, b in (X.node.inputs, X.node.inputs[::-1]):
            mk = self._mask_row(L, b, Sk)
            if mk is not None:
                sc, mask = a, mk
                break
        if sc is None:
            return None
        nodes.append(X.node)
        pos, mnodes = mask
        nodes += mnodes
        # score chain: [convert bf16] <- (divide | multiply by a scalar) <- [convert f32] <- dot
        if op_of(sc) == "convert" and sc.dtype == dt.bfloat16:
            flags |= LA.DEC_RND_SCORE
            nodes.append(sc.node)
            sc = sc.node.inputs[0]
        if op_of(sc) not in ("divide", "multiply") or sc.dtype != dt.float32:
            return None
        a, c = sc.node.inputs
        if op_of(sc) == "multiply" and scalar_value(a)[0] is not None:
            a, c = c, a
        cv, cn = scalar_value(c)
        if cv is None or not cv > 0:
            return None
        if op_of(sc) == "divide":
            flags |= LA.DEC_DIVIDE
        nodes += [sc.node] + cn
        if op_of(a) == "convert" and a.dtype == dt.float32:
            nodes.append(a.node)
            a = a.node.inputs[0]
        if not (op_of(a) == "dot" and _qk_dot(a.node)):
            return None
        d1 = a.node
        if d1.out.dtype == dt.bfloat16:
            flags |= LA.DEC_RND_PROD
        elif d1.out.dtype != dt.float32:
            return None
        nodes.append(d1)
        q = _bf16_view(d1.inputs[0])
        k = _bf16_view(d1.inputs[1])
        v = _bf16_view(v_op)
        if q is None or k is None or v is None:
            return None
        B, Hq, one, D = q.shape
        if one != 1 or k.shape != (B, Hq, D, Sk) or v.shape != (B, Hq, Sk, D) or n2.out.shape != (B, Hq, 1, D):
            return None
        qs = [q.simple(0), q.simple(1)]
        kg, vg = k.grouped(1), v.grouped(1)
        ks = [k.simple(0), k.simple(3)]
        vs = [v.simple(0), v.simple(2)]
        if None in qs + ks + vs or kg is None or vg is None:
            return None
        if q.simple(3) != 1 or k.simple(2) != 1 or v.simple(3) != 1:
            return None
        if kg[0] != vg[0] or kg[2] != vg[2] or kg[0] * kg[2] != Hq:
            return None
        Hkv = kg[0]
        # output tail: transposes / casts / one reshape (as for prefill)
        out, perm, reshaped = n2.out, [0, 1, 2, 3], False
        while True:
            us = _users_of(L, out)
            if out.id in L.result_ids or len(us) != 1:
                break
            u = us[0]
            if u.op == "transpose" and not reshaped:
                perm = [perm[pp] for pp in u.attrs["permutation"]]
            elif u.op in ("convert", "copy") and (u.out.dtype == out.dtype or (
                    out.dtype == dt.float32 and u.out.dtype == dt.bfloat16)):
                pass
            elif u.op == "reshape" and not reshaped:
                reshaped = True
            else:
                break
            nodes.append(u)
            out = u.out
        if out.dtype != dt.bfloat16 or perm not in ([0, 1, 2, 3], [0, 2, 1, 3]):
            return None
        logical = [(B, Hq, 1, D)[pp] for pp in perm]
        cs = _contiguous(logical)
        ps = {ax: i for i, ax in enumerate(perm)}
        o_str = (cs[ps[0]], cs[ps[1]])
        strides = {"q": tuple(qs), "k": (ks[0], ks[1], kg[1]), "v": (vs[0], vs[1], vg[1])}
        try:
            LA.decode_attention(16, 16, 16, 16, 16, B, Sk, Hq, Hkv, D, cv, dict(strides, o=o_str), flags, ws_ptr=16)
        except LA.LaunchError:
            return None
        if any((vw.offset * 2) % 16 for vw in (k, v)):
            return None
        return DecodeAttentionMatch(nodes, q, k, v, pos, out, (B, Sk, Hq, Hkv, D, strides), cv, flags, o_str)


ATTENTION_PATTERNS = [AttentionPattern(), RopePattern()]
