"""Chunked causal linear attention -> csrc/kernels/linattn.hip.

Matches the traced graph of the vectorised chunked kernel
(nkipy_amd/kernels/linear_attention.py), anchored on the final
normalisation ``num / den``:

    phi(x)  = where(x > 0, x + 1, exp(x))            (x = q / k upcast)
    Qf, Kf  = reshape(phi(q)), reshape(phi(k))       (B, H, n, C, D)
    V       = reshape(v)                             (B, H, n, C, Dv)
    KV      = swapaxes(Kf) @ V;  S = cumsum(KV, 2) - KV
    ks      = sum(Kf, 3);        z = cumsum(ks, 2) - ks
    A       = (Qf @ swapaxes(Kf)) * tril(ones(C, C))
    num     = Qf @ S + A @ V
    den     = sum(Qf * z[..., None, :], -1) + sum(A, -1)
    out     = (num / den).reshape(B, H, T, Dv)  [.astype(bf16)]

Every piece is verified (the mask constant must be the lower-triangular
ones matrix, both prefix sums exclusive, phi the elu+1 map); anything else
falls through to the generic lowering.
"""

from __future__ import annotations

import numpy as np

from nkipy_amd.core import dtypes as dt
from nkipy_amd.dispatch import launchers as LA
from nkipy_amd.dispatch.plan import Slot
from nkipy_amd.dispatch.patterns import LaunchStep, Match, _users_of, op_of, scalar_value, through_views


class _NoMatch(Exception):
    pass


def _expect(v, op):
    if op_of(v) != op:
        raise _NoMatch(op)
    return v.node


def _batched_dot(v, nodes):
    n = _expect(v, "dot")
    at = n.attrs
    if tuple(at["lhs_batch"]) != (0, 1, 2) or tuple(at["rhs_batch"]) != (0, 1, 2) or \
            tuple(at["lhs_contract"]) != (4,) or tuple(at["rhs_contract"]) != (3,):
        raise _NoMatch("dot dims")
    nodes.append(n)
    return n.inputs


def _swap_last(v, nodes):
    n = _expect(v, "transpose")
    if tuple(n.attrs["permutation"]) != (0, 1, 2, 4, 3):
        raise _NoMatch("swapaxes")
    nodes.append(n)
    return n.inputs[0]


def _phi_source(v, nodes):
    """v = reshape(select(x > 0, x + 1, exp(x))), x = convert(src) -> src."""
    r = _expect(v, "reshape")
    nodes.append(r)
    sel = _expect(r.inputs[0], "select")
    nodes.append(sel)
    pred, a, e = sel.inputs
    cmp_ = _expect(pred, "compare")
    if cmp_.attrs["comparison_direction"] != "GT":
        raise _NoMatch("phi compare")
    x = cmp_.inputs[0]
    zero, zn = scalar_value(cmp_.inputs[1])
    add = _expect(a, "add")
    one, on = (None, [])
    if add.inputs[0] is x:
        one, on = scalar_value(add.inputs[1])
    exp_ = _expect(e, "exponential")
    if zero != 0.0 or one != 1.0 or exp_.inputs[0] is not x:
        raise _NoMatch("phi")
    nodes += [cmp_, add, exp_] + zn + on
    if op_of(x) == "convert":
        nodes.append(x.node)
        x = x.node.inputs[0]
    return x


def _exclusive_prefix(v, nodes):
    """v = cumsum(u, axis=2) - u -> u."""
    sub = _expect(v, "subtract")
    c, u = sub.inputs
    cs = _expect(c, "cumsum")
    if cs.attrs["axis"] != 2 or cs.inputs[0] is not u:
        raise _NoMatch("prefix")
    nodes += [sub, cs]
    return u


class LinearAttentionMatch(Match):
    name = "linear_attention"

    def __init__(self, nodes, q, k, v, out):
        super().__init__(nodes, [q, k, v], [out])
        self.q, self.k, self.v, self.out = q, k, v, out

    def steps(self, plan):
        q, k, v, out = self.q, self.k, self.v, self.out
        B, H, T, D = q.shape
        # segmented scans take their prefix states from a workspace temporary
        ws_bytes = LA.linear_attention_workspace_bytes(B * H, T)
        ws = Slot(plan.add_buffer(ws_bytes, "temp", "linear_attention.prefix")) if ws_bytes else None
        # each sequence's max |v|, checked against the kernel's fp16 operand
        # window after the execution (a silent precision loss becomes an error)
        vm = Slot(plan.add_buffer(4 * B * H, "temp", "linear_attention.vmax"))
        plan.checks.append({"kind": "linattn_vmax", "buffer": vm.buffer, "offset": 0, "count": B * H,
                            "desc": f"linear attention over {B}x{H} sequences of {T}"})

        def make(addr):
            return LA.linear_attention(addr(q), addr(k), addr(v), addr(out), B * H, T, D, v.shape[-1], 64,
                                       part_ptr=addr(ws) if ws is not None else 0, vmax_ptr=addr(vm))

        return [LaunchStep("linear_attention", f"chunked causal linear attention B*H={B * H} T={T} d={D}",
                           self.inputs, self.outputs, make)]


class LinearAttentionPattern:
    def find(self, L):
        for n in L.live:
            if n.op != "divide" or id(n) in L.covered:
                continue
            try:
                m = self._match(L, n)
            except _NoMatch:
                m = None
            if m is not None and m.validate(L):
                yield m

    def _match(self, L, div):
        nodes = [div]
        num, bden = div.inputs
        if num.ndim != 5:
            raise _NoMatch("rank")
        Bb, H, n, C, Dv = num.shape
        # den: broadcast over Dv of add(sum(Qf * z), sum(A)) (keepdims views)
        bn = _expect(bden, "broadcast_in_dim")
        if tuple(bn.attrs["broadcast_dimensions"]) != (0, 1, 2, 3):
            raise _NoMatch("den broadcast")
        nodes.append(bn)
        den, vn = through_views(bn.inputs[0])
        nodes += vn
        dadd = _expect(den, "add")
        nodes.append(dadd)
        # num = Qf @ S + A @ V
        nadd = _expect(num, "add")
        nodes.append(nadd)
        qf1 = s_val = a_val = vf1 = None
        for first, second in (nadd.inputs, nadd.inputs[::-1]):
            try:
                ops1 = _batched_dot(first, [])
                ops2 = _batched_dot(second, [])
            except _NoMatch:
                continue
            if ops1[1].shape[-2] == ops1[0].shape[-1] and op_of(ops1[1]) == "subtract":
                (qf1, s_val), (a_val, vf1) = ops1, ops2
                nodes += [first.node, second.node]
                break
        if qf1 is None:
            raise _NoMatch("num")
        # S = exclusive prefix of swap(Kf) @ V
        kv = _exclusive_prefix(s_val, nodes)
        kt, vf2 = _batched_dot(kv, nodes)
        kf = _swap_last(kt, nodes)
        if vf2 is not vf1:
            raise _NoMatch("V")
        # A = (Qf @ swap(Kf)) * tril(ones)
        am = _expect(a_val, "multiply")
        nodes.append(am)
        a_dot, mask_b = am.inputs
        if op_of(a_dot) != "dot":
            a_dot, mask_b = mask_b, a_dot
        qf2, kt2 = _batched_dot(a_dot, nodes)
        if qf2 is not qf1 or _swap_last(kt2, nodes) is not kf:
            raise _NoMatch("A operands")
        mb = _expect(mask_b, "broadcast_in_dim")
        mc = _expect(mb.inputs[0], "constant")
        mask = np.asarray(mc.attrs["value"])
        if mask.shape != (C, C) or not np.array_equal(mask.astype(np.float64), np.tril(np.ones((C, C)))):
            raise _NoMatch("mask")
        nodes += [mb, mc]
        # den terms: sum(Qf * z, -1) and sum(A, -1)
        t1, t2 = dadd.inputs
        z_seen = a_seen = False
        for t in (t1, t2):
            tb, tn = through_views(t)
            nodes += tn
            red = _expect(tb, "reduce")
            if red.attrs["computation"] != "add" or tuple(red.attrs["dimensions"]) != (4,):
                raise _NoMatch("den reduce")
            nodes.append(red)
            src = red.inputs[0]
            if src is a_val:
                a_seen = True
                continue
            mul = _expect(src, "multiply")
            nodes.append(mul)
            x, zb = mul.inputs
            if x is not qf1:
                x, zb = zb, x
            if x is not qf1:
                raise _NoMatch("den q")
            zbn = _expect(zb, "broadcast_in_dim")
            if tuple(zbn.attrs["broadcast_dimensions"]) != (0, 1, 2, 4):
                raise _NoMatch("z broadcast")
            nodes.append(zbn)
            zv, zn = through_views(zbn.inputs[0])
            nodes += zn
            ks = _exclusive_prefix(zv, nodes)
            ksr = _expect(ks, "reduce")
            if ksr.attrs["computation"] != "add" or tuple(ksr.attrs["dimensions"]) != (3,) or ksr.inputs[0] is not kf:
                raise _NoMatch("ksum")
            nodes.append(ksr)
            z_seen = True
        if not (z_seen and a_seen):
            raise _NoMatch("den terms")
        # sources
        q = _phi_source(qf1, nodes)
        k = _phi_source(kf, nodes)
        vr = _expect(vf1, "reshape")
        nodes.append(vr)
        v = vr.inputs[0]
        if op_of(v) == "convert":
            nodes.append(v.node)
            v = v.node.inputs[0]
        # output: reshape back to (B, H, T, Dv), optional cast
        out = div.out
        us = _users_of(L, out)
        if out.id in L.result_ids or len(us) != 1 or us[0].op != "reshape":
            raise _NoMatch("output reshape")
        nodes.append(us[0])
        out = us[0].out
        us = _users_of(L, out)
        if out.id not in L.result_ids and len(us) == 1 and us[0].op == "convert":
            nodes.append(us[0])
            out = us[0].out
        T = n * C
        ok = (q.dtype == k.dtype == v.dtype == out.dtype == dt.bfloat16 and C == 64
              and q.shape == (Bb, H, T, 128) and k.shape == q.shape and v.shape == (Bb, H, T, 128)
              and out.shape == (Bb, H, T, 128))
        if not ok:
            raise _NoMatch("shape / dtype not supported by the kernel")
        return LinearAttentionMatch(nodes, q, k, v, out)
