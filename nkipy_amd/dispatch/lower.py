"""Lowering of a traced graph to a :class:`~nkipy_amd.dispatch.plan.Plan`.

1. Fused patterns (softmax, RMSNorm, GEMM, ...) claim subgraphs; each
   becomes one step running a hand-written gfx950 kernel.
2. Every other live node is lowered generically (see ``generic.py``):
   elementwise / layout chains become programs, the rest dedicated steps.
3. Values that must exist in memory ("materialised") get storage: kernel
   inputs and outputs are bound per call, everything else is a temporary
   owned by the loaded kernel; a reshape shares its operand's storage.

There is no CPU fallback: a node that cannot be lowered raises
``LoweringError``.
"""

from __future__ import annotations

from typing import Dict, List, Set

import numpy as np

from nkipy_amd.core import dtypes as dt
from nkipy_amd.core.backend.ir import Graph, Node, Value
from nkipy_amd.dispatch import generic as G
from nkipy_amd.dispatch.plan import Plan, Slot


class LoweringError(NotImplementedError):
    pass


CHEAP_OPS = {"convert", "copy", "negate", "abs", "compare", "select", "iota", "constant"}


def _users(live: List[Node]) -> Dict[int, List[Node]]:
    u: Dict[int, List[Node]] = {}
    for n in live:
        for v in n.inputs:
            u.setdefault(v.id, []).append(n)
    return u


class Lowering:
    def __init__(self, graph: Graph, patterns=None):
        from nkipy_amd.dispatch.patterns import default_patterns

        self.g = graph
        self.patterns = default_patterns() if patterns is None else patterns
        self.live = graph.live_nodes()
        self.users = _users(self.live)
        self.result_ids = {r.id for r in graph.results}
        self.mat: Set[int] = set()
        self.alias_reshape: Set[int] = set()  # reshape values sharing the operand's slot
        self.matches = []
        self.covered: Dict[int, object] = {}  # id(node) -> match
        self.dot_contig: Set[int] = set()  # dots that read contiguous operands
        self.match_alias: Dict[int, Value] = {}  # value inside a match -> equal output

    # ------------------------------------------------------------------
    def n_users(self, v: Value) -> int:
        return len(self.users.get(v.id, ())) + (1 if v.id in self.result_ids else 0)

    def is_mat(self, v: Value) -> bool:
        return v.id in self.mat or v.is_parameter

    def need(self, v: Value):
        if v.is_parameter:
            return
        n = v.node
        if n is not None and n.op == "reshape" and not G.is_unit_reshape(n.inputs[0].shape, v.shape):
            # general reshape: storage is the operand's
            self.alias_reshape.add(v.id)
            self.mat.add(v.id)
            self.need(n.inputs[0])
            return
        self.mat.add(v.id)

    # ------------------------------------------------------------------
    def run(self) -> Plan:
        # 1. fused patterns
        for pat in self.patterns:
            for m in pat.find(self):
                self.matches.append(m)
                for nid in m.nodes:
                    self.covered[nid] = m
        self.match_alias = self._match_aliases()
        for pat in self.patterns:
            # merges of claimed matches (e.g. RoPE into its QKV projection)
            refine = getattr(pat, "refine", None)
            if refine is not None:
                refine(self)
        self.match_alias = self._match_aliases()
        # 2. materialisation
        for r in self.g.results:
            self.need(r)
        for m in self.matches:
            for v in list(m.inputs) + list(m.outputs):
                self.need(v)
        for n in self.live:
            if id(n) in self.covered:
                continue
            self._decide(n)
        self._settle_programs()
        for n in self.live:
            if id(n) in self.covered:
                continue
            if n.op in ("reduce", "argmax", "argmin", "dot") and n.out.id in self.mat:
                accs = [G.strided_access(v, self.is_mat) for v in n.inputs]
                if n.op == "dot":
                    try:
                        G.DotStep(n, *accs)
                    except G.LaunchError:
                        # strides do not collapse: read contiguous copies
                        self.dot_contig.add(id(n))
                        for v in n.inputs:
                            self.need(v)
                        continue
                for base, _, _ in accs:
                    self.need(base)
        self._settle_programs()
        # 3. storage and 4. steps
        return self._build_plan()

    def _match_aliases(self) -> Dict[int, Value]:
        """Values inside a match that equal one of its outputs bit for bit
        (the output is a same-dtype copy / convert of them, e.g. a no-op
        ``astype`` the GEMM epilogue absorbed).  Views look through such
        copies, so another match may read the inner value; it shares the
        output's storage, which the match writes."""
        alias: Dict[int, Value] = {}
        for m in self.matches:
            outs = {v.id for v in m.outputs}
            for o in m.outputs:
                cur = o
                while (cur.node is not None and id(cur.node) in m.nodes
                       and cur.node.op in ("copy", "convert") and cur.node.inputs[0].dtype == cur.dtype):
                    src = cur.node.inputs[0]
                    if src.id in outs or src.node is None or id(src.node) not in m.nodes:
                        break
                    alias[src.id] = o
                    cur = src
        return alias

    def _decide(self, n: Node):
        op = n.op
        v = n.out
        if op == "constant":
            if v.size > 1:
                self.need(v)
            return
        if op in G.EW_OPS or G.is_affine_layout(n):
            if self.n_users(v) > 1 and op not in CHEAP_OPS and not G.is_affine_layout(n):
                self.need(v)
            return
        if op == "reshape":
            return  # materialised on demand (alias of its operand)
        self.need(v)
        if op in ("reduce", "argmax", "argmin", "dot"):
            return  # operands read through strides; bases marked later
        for x in n.inputs:
            self.need(x)

    def _settle_programs(self):
        """Materialise operands of programs that do not fit one kernel."""
        builder = G.ProgramBuilder(self.is_mat)
        changed = True
        while changed:
            changed = False
            for n in self.live:
                v = n.out
                if id(n) in self.covered or v.id not in self.mat or v.id in self.alias_reshape:
                    continue
                if not (n.op in G.EW_OPS or G.is_affine_layout(n) or n.op == "copy"):
                    continue
                try:
                    builder.build(v)
                except G.ProgramTooLarge:
                    for x in n.inputs:
                        if not self.is_mat(x):
                            self.need(x)
                            changed = True
                    if not changed:
                        raise LoweringError(f"cannot lower {n!r} into one program")

    # ------------------------------------------------------------------
    def _build_plan(self) -> Plan:
        g = self.g
        plan = Plan(g)
        slots = plan.slots
        for p in g.parameters:
            idx = plan.add_buffer(p.nbytes, "input", p.name)
            plan.input_buffers[p.name] = idx
            slots[p.id] = Slot(idx)
        copies: Dict[int, Value] = {}  # reshape result id -> source: flat copy at the reshape
        for r in g.results:
            idx = plan.add_buffer(r.nbytes, "output", r.name)
            plan.output_buffers[r.name] = idx
            slots[r.id] = Slot(idx)
        for a in g.aliases:
            plan.alias_outputs[a.param_name] = f"{a.param_name}.must_alias_input"

        # results that are reshapes: let the producer write the output buffer
        for n in reversed(self.live):
            v = n.out
            if v.id in self.alias_reshape and v.id in slots:
                src = n.inputs[0]
                if src.id not in slots and not src.is_parameter and not (
                        src.node is not None and src.node.op == "constant"):
                    slots[src.id] = slots[v.id]
                elif slots.get(src.id) is not slots[v.id]:
                    copies[v.id] = src

        # in-place aliased results: compute out of place when the mutated
        # parameter is still read after the producing node
        inplace_skip_copy: Set[int] = set()
        order = {id(n): i for i, n in enumerate(self.live)}
        param_by_name = {p.name: p for p in g.parameters}
        deferred: List[tuple] = []
        for a in g.aliases:
            res = g.results[a.output_index]
            p = param_by_name[f"{a.param_name}.must_alias_input"]
            prod = res.node
            late = prod is None or not self._reads_done_before(p, prod, order)
            if late:
                # the producer writes a staging temporary; a final copy moves
                # it into the caller's (aliased) buffer
                outv = Value(res.shape, res.dtype, None, name=res.name)
                slots[outv.id] = slots[res.id]
                slots[res.id] = Slot(plan.add_buffer(res.nbytes, "temp", f"{res.name}.staged"))
                deferred.append((res, outv))
            elif prod.op in ("dynamic_update_slice", "scatter_along_axis", "put_along_axis",
                             "scatter_strided") and prod.inputs[0] is p:
                inplace_skip_copy.add(id(prod))

        for n in self.live:
            v = n.out
            if v.id in self.mat and v.id not in slots and v.id not in self.match_alias:
                if n.op == "constant":
                    payload = n.attrs["value"]
                    idx = plan.add_buffer(v.nbytes, "const", f"const{v.id}", payload)
                elif v.id in self.alias_reshape:
                    continue
                else:
                    idx = plan.add_buffer(v.nbytes, "temp", f"t{v.id}")
                slots[v.id] = Slot(idx)
        for vid, o in self.match_alias.items():
            if vid in self.mat:
                slots[vid] = slots[o.id]
        for n in self.live:
            v = n.out
            if v.id in self.alias_reshape and v.id not in slots:
                slots[v.id] = slots[n.inputs[0].id]

        # steps in program order
        emitted = set()
        for n in self.live:
            m = self.covered.get(id(n))
            if m is not None:
                if id(m) not in emitted and n is m.last:
                    plan.steps.extend(m.steps(plan))
                    emitted.add(id(m))
                continue
            v = n.out
            if v.id in copies:
                src = copies[v.id]
                plan.steps.append(G.ProgramStep(f"copy {src!r} -> {v.name}", G.flat_copy_program(src), v))
                continue
            if v.id not in self.mat or v.id in self.alias_reshape or n.op == "constant":
                continue
            plan.steps.extend(self._lower_node(n, plan, id(n) in inplace_skip_copy))
        for m in self.matches:
            if id(m) not in emitted:
                raise LoweringError(f"pattern {m} was never emitted")
        for res, outv in deferred:
            plan.steps.append(G.ProgramStep(f"write back {res.name}", G.flat_copy_program(res), outv))
        return plan

    _INPLACE_OPS = ("dynamic_update_slice", "scatter_along_axis", "put_along_axis", "scatter_strided")

    def _reads_done_before(self, p: Value, prod: Node, order: Dict[int, int]) -> bool:
        """True when every read of parameter ``p`` happens in a step that runs
        before ``prod``'s step, so ``prod`` may overwrite ``p``'s buffer.

        A read is deferred when the reading node is not materialised (a
        fused elementwise / layout node, or a reshape sharing ``p``'s
        storage): it happens inside the step of a later consumer, so the
        consumers are followed transitively.  ``prod`` itself may read ``p``
        only as the operand it updates in place."""
        limit = order[id(prod)]
        work, seen = [p], {p.id}
        while work:
            x = work.pop()
            for u in self.users.get(x.id, ()):
                if u is prod:
                    in_place_target = (x is p and prod.op in self._INPLACE_OPS and prod.inputs[0] is p
                                       and not any(y is p for y in prod.inputs[1:]))
                    if not in_place_target:
                        return False
                    continue
                m = self.covered.get(id(u))
                if m is not None:
                    if order[id(m.last)] >= limit:
                        return False
                    continue
                v = u.out
                if v.id in self.mat and (v.id not in self.alias_reshape or v.id in self.result_ids):
                    if order[id(u)] >= limit:
                        return False
                    continue
                if v.id not in seen:  # evaluated later, inside a consumer's step
                    seen.add(v.id)
                    work.append(v)
        return True

    # ------------------------------------------------------------------
    def _lower_node(self, n: Node, plan: Plan, inplace: bool) -> list:
        op = n.op
        v = n.out
        builder = G.ProgramBuilder(self.is_mat)
        if op in G.EW_OPS or G.is_affine_layout(n) or op == "copy":
            return [G.ProgramStep(op, builder.build(v), v)]
        if op in ("reduce", "argmax", "argmin"):
            base, strides, off = G.strided_access(n.inputs[0], self.is_mat)
            return [G.ReduceStep(n, base, strides, off)]
        if op == "dot":
            if id(n) in self.dot_contig:
                lhs, rhs = [(v, G.contiguous_strides(v.shape), 0) for v in n.inputs]
            else:
                lhs = G.strided_access(n.inputs[0], self.is_mat)
                rhs = G.strided_access(n.inputs[1], self.is_mat)
            return [G.DotStep(n, lhs, rhs)]
        if op in ("take", "take_along_axis"):
            return [G.GatherStep(n)]
        if op in ("scatter_along_axis", "put_along_axis"):
            steps = [] if inplace else [self._copy(n.inputs[0], v)]
            return steps + [G.GatherStep(n)]
        if op == "cumsum":
            return [G.CumsumStep(n)]
        if op == "topk":
            return [G.TopkStep(n)]
        if op == "concatenate":
            ax = n.attrs["dimension"]
            s = G.contiguous_strides(v.shape)
            steps, pos = [], 0
            for x in n.inputs:
                prog = builder.build(x) if not self.is_mat(x) else self._load_prog(x)
                steps.append(G.ProgramStep("concatenate part", prog, v, out_strides=s,
                                           out_offset=int(pos * s[ax])))
                pos += x.shape[ax]
            return steps
        if op == "pad":
            x, pv = n.inputs
            s = G.contiguous_strides(v.shape)
            fill = G.Program(v.shape)
            c = G.scalar_constant(pv)
            fill.result = fill.emit(G.OP_CONST, dtype=v.dtype, imm=c if c is not None else 0.0)
            off = int(sum(l * st for l, st in zip(n.attrs["low"], s)))
            return [G.ProgramStep("pad fill", fill, v),
                    G.ProgramStep("pad interior", self._load_prog(x), v, out_strides=s, out_offset=off)]
        if op == "reverse":
            return [G.ProgramStep(op, builder.build(v), v)]
        if op == "dynamic_update_slice":
            operand, upd = n.inputs
            s = G.contiguous_strides(v.shape)
            off = int(sum(a * st for a, st in zip(n.attrs["start"], s)))
            steps = [] if inplace else [self._copy(operand, v)]
            return steps + [G.ProgramStep("update slice", self._load_prog(upd), v,
                                          out_strides=s, out_offset=off)]
        if op == "scatter_strided":
            operand, upd = n.inputs
            s = G.contiguous_strides(v.shape)
            ostr, off = [], 0
            for d, ix in enumerate(n.attrs["indices_per_dim"]):
                step = (ix[1] - ix[0]) if len(ix) > 1 else 1
                if any(ix[k + 1] - ix[k] != step for k in range(len(ix) - 1)) or step <= 0:
                    raise LoweringError("scatter_strided needs arithmetic index progressions")
                ostr.append(step * int(s[d]))
                off += ix[0] * int(s[d])
            steps = [] if inplace else [self._copy(operand, v)]
            return steps + [G.ProgramStep("strided update", self._load_prog(upd), v,
                                          out_strides=ostr, out_offset=off)]
        raise LoweringError(f"no device lowering for op '{op}' ({n!r})")

    def _load_prog(self, x: Value) -> G.Program:
        if self.is_mat(x):
            prog = G.Program(x.shape)
            prog.result = prog.load(x, G.contiguous_strides(x.shape), 0)
            return prog
        return G.ProgramBuilder(self.is_mat).build(x)

    def _copy(self, src: Value, dst: Value) -> G.ProgramStep:
        return G.ProgramStep("copy", self._load_prog(src), dst)


def lower(graph: Graph, patterns=None) -> Plan:
    return Lowering(graph, patterns).run()
