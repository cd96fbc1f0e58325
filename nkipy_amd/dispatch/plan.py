"""Kernel plans: the lowered form of a traced graph.

A :class:`Plan` is a list of :class:`Step` objects over a set of device
buffers.  Buffers are the kernel's inputs and outputs (bound per call to
the caller's device tensors), temporaries (allocated once per loaded
kernel) and constants (uploaded once).  Each graph value that is
materialised lives in a :class:`Slot` -- a buffer plus a byte offset; a
reshape shares its operand's slot.

A step turns slot addresses into :class:`~nkipy_amd.dispatch.launchers.Launch`
objects.  :class:`PlanExecutor` binds a plan to concrete buffers once per
distinct set of argument addresses and replays the packed launches with a
single ``nkh_launch_batch`` call, so the per-call host cost does not grow
with argument validation or Python dispatch (the per-call work the
reference does in SpikeModel.__call__, spike/src/spike/spike_model.py:228-268).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Callable, Dict, List, Optional

import numpy as np

from nkipy_amd.core import dtypes as dt
from nkipy_amd.core.backend.ir import Graph, Value
from nkipy_amd.dispatch.launchers import Launch


@dataclass
class BufferSpec:
    index: int
    nbytes: int
    kind: str  # "input" | "output" | "temp" | "const"
    name: str = ""
    data: Optional[np.ndarray] = None  # constant payload (raw bytes view)


@dataclass
class Slot:
    buffer: int
    offset: int = 0


class Step:
    """One lowered unit of work: one or more kernel launches."""

    kind = "step"

    def __init__(self, desc: str, inputs: List[Value], outputs: List[Value]):
        self.desc = desc
        self.inputs = inputs
        self.outputs = outputs

    def launches(self, addr: Callable[[Value], int]) -> List[Launch]:
        raise NotImplementedError

    def describe(self) -> dict:
        return {
            "kind": self.kind,
            "desc": self.desc,
            "inputs": [repr(v) for v in self.inputs],
            "outputs": [repr(v) for v in self.outputs],
        }


@dataclass
class Plan:
    graph: Graph
    buffers: List[BufferSpec] = field(default_factory=list)
    slots: Dict[int, Slot] = field(default_factory=dict)
    steps: List[Step] = field(default_factory=list)
    # name -> buffer index
    input_buffers: Dict[str, int] = field(default_factory=dict)
    output_buffers: Dict[str, int] = field(default_factory=dict)
    # output name -> input name whose buffer it must reuse (aliasing)
    alias_outputs: Dict[str, str] = field(default_factory=dict)
    # host-side checks of words the kernels leave in temporaries, run after
    # an execution completes: {"kind", "buffer", "offset", "count", "desc"}
    checks: List[dict] = field(default_factory=list)

    def add_buffer(self, nbytes: int, kind: str, name: str = "", data=None) -> int:
        b = BufferSpec(len(self.buffers), int(nbytes), kind, name, data)
        self.buffers.append(b)
        return b.index

    def slot(self, v: Value) -> Slot:
        try:
            return self.slots[v.id]
        except KeyError:
            raise KeyError(f"value {v!r} has no storage in the plan") from None

    @property
    def kernel_kinds(self) -> List[str]:
        return [s.kind for s in self.steps]

    def describe(self) -> dict:
        return {
            "graph": self.graph.name,
            "buffers": [
                {"index": b.index, "kind": b.kind, "name": b.name, "nbytes": b.nbytes}
                for b in self.buffers
            ],
            "steps": [s.describe() for s in self.steps],
        }

    def summary(self) -> str:
        lines = [f"plan {self.graph.name}: {len(self.steps)} steps, "
                 f"{sum(1 for b in self.buffers if b.kind == 'temp')} temporaries"]
        for s in self.steps:
            lines.append(f"  [{s.kind}] {s.desc}")
        return "\n".join(lines)


class BoundPlan:
    """Launches of a plan with every address resolved, packed for replay."""

    def __init__(self, launches: List[Launch], rt):
        self.launches = launches
        self.rt = rt
        n = len(launches)
        fns = [l.function(rt) for l in launches]
        blobs = []
        for f, l in zip(fns, launches):
            f.check_block(l.block)
            blobs.append(f.check_args(l.args))
        offsets, off = [], 0
        for b in blobs:
            offsets.append(off)
            off += (len(b) + 15) // 16 * 16
        buf = bytearray(off)
        for o, b in zip(offsets, blobs):
            buf[o:o + len(b)] = b
        vp = ctypes.c_void_p
        u = ctypes.c_uint
        sz = ctypes.c_size_t
        self._n = n
        self._fns = (vp * n)(*[f.handle for f in fns])
        self._grids = (u * (3 * n))(*[g for l in launches for g in l.grid])
        self._blocks = (u * (3 * n))(*[b for l in launches for b in l.block])
        self._shared = (u * n)(*[l.shared for l in launches])
        self._kernargs = bytes(buf)
        self._offsets = (sz * n)(*offsets)
        self._sizes = (sz * n)(*[len(b) for b in blobs])
        self._graph = None

    def run(self):
        from nkipy_amd.runtime.hip import _check, check_current

        check_current(self.rt, "plan")
        if self._n == 0:
            return
        _check(
            self.rt.lib.nkh_launch_batch(
                self._n, self._fns, self._grids, self._blocks, self._shared,
                self._kernargs, self._offsets, self._sizes,
            ),
            "plan launch",
        )

    def run_graph(self):
        """The launches replayed as one HIP graph, captured on the first call
        (``nkh_graph_create``): one host call per execution, whatever the
        launch count.  The graph holds copies of the packed argument blocks,
        so it stays valid as long as the addresses bound here do."""
        from nkipy_amd.runtime.hip import _check, check_current

        check_current(self.rt, "plan")
        if self._n == 0:
            return
        if self._graph is None:
            h = ctypes.c_void_p()
            _check(
                self.rt.lib.nkh_graph_create(
                    self._n, self._fns, self._grids, self._blocks, self._shared,
                    self._kernargs, self._offsets, self._sizes, ctypes.byref(h),
                ),
                "plan graph capture",
            )
            self._graph = h.value
        _check(self.rt.lib.nkh_graph_launch(ctypes.c_void_p(self._graph)), "plan graph launch")

    def release_graph(self):
        """Destroys the captured graph, if any (the runtime drains its stream
        first); a runtime already shut down released it itself."""
        from nkipy_amd.runtime.hip import _check

        g, self._graph = self._graph, None
        if g is not None and not self.rt.is_closed:
            _check(self.rt.lib.nkh_graph_destroy(ctypes.c_void_p(g)), "plan graph release")

    def run_range(self, start: int, stop: int):
        """Launches ``start .. stop-1`` of the plan (all of them: ``run``)."""
        from nkipy_amd.runtime.hip import _check, check_current

        check_current(self.rt, "plan")
        if not 0 <= start <= stop <= self._n:
            raise IndexError(f"launch range {start}..{stop} outside 0..{self._n}")
        if stop == start:
            return
        vp, u, sz = ctypes.c_void_p, ctypes.c_uint, ctypes.c_size_t

        def at(arr, ctype, i):
            return ctypes.cast(ctypes.addressof(arr) + i * ctypes.sizeof(ctype), ctypes.POINTER(ctype))

        _check(
            self.rt.lib.nkh_launch_batch(
                stop - start, at(self._fns, vp, start), at(self._grids, u, 3 * start),
                at(self._blocks, u, 3 * start), at(self._shared, u, start),
                self._kernargs, at(self._offsets, sz, start), at(self._sizes, sz, start),
            ),
            "plan launch",
        )


def _check_linattn_vmax(words, desc):
    from nkipy_amd.dispatch.launchers import check_linear_attention_vmax

    check_linear_attention_vmax(words, desc or "linear attention")


# check kind -> function(words, description) raising on a failed check
CHECKS: Dict[str, Callable] = {"linattn_vmax": _check_linattn_vmax}


class PlanExecutor:
    """Owns a plan's temporaries and constants and runs it on bound I/O.

    ``plan`` is a lowered :class:`Plan` or a loaded relocatable artefact
    (:class:`nkipy_amd.dispatch.artifact.RelocatablePlan`); an artefact binds
    by patching addresses, and falls back to ``lower_fn()`` (the full plan,
    lowered on first need) for I/O addresses that are not 256-byte aligned."""

    def __init__(self, plan, lower_fn=None):
        from nkipy_amd.runtime.device_tensor import DeviceBuffer
        from nkipy_amd.runtime.hip import get_runtime

        self.plan = plan
        self.lower_fn = lower_fn
        self._full: Optional[Plan] = plan if isinstance(plan, Plan) else None
        self.rt = get_runtime()
        self._owned: Dict[int, DeviceBuffer] = {}
        pname = plan.graph.name if isinstance(plan, Plan) else plan.name
        for b in plan.buffers:
            if b.kind in ("temp", "const"):
                buf = DeviceBuffer(max(b.nbytes, 16), name=f"{pname}:{b.kind}{b.index}")
                if b.kind == "const" and b.data is not None and b.data.nbytes:
                    raw = np.ascontiguousarray(dt.numpy_storage(np.ascontiguousarray(b.data)))
                    buf.write(raw.ctypes.data, raw.nbytes)
                self._owned[b.index] = buf
        self._bound: Dict[tuple, BoundPlan] = {}

    def _full_plan(self) -> Plan:
        from nkipy_amd.runtime.hip import SpikeError

        if self._full is None:
            if self.lower_fn is None:
                raise SpikeError("this kernel was loaded from its artefact alone: its I/O must be 256-byte "
                                 "aligned device buffers")
            full = self.lower_fn()
            if [(b.index, b.kind, b.nbytes) for b in full.buffers] != \
                    [(b.index, b.kind, b.nbytes) for b in self.plan.buffers]:
                raise SpikeError("the lowered plan does not match the loaded artefact")
            self._full = full
        return self._full

    def _bind(self, bases: Dict[int, int]) -> BoundPlan:
        if not isinstance(self.plan, Plan) and all(
                bases[i] % 256 == 0 for i in list(self.plan.input_buffers.values())
                + list(self.plan.output_buffers.values())):
            return self.plan.bind(bases, self.rt)
        plan = self._full_plan()

        def addr(v) -> int:
            # a graph value, or a Slot of a step's own workspace temporary
            s = v if isinstance(v, Slot) else plan.slot(v)
            return bases[s.buffer] + s.offset

        launches: List[Launch] = []
        for st in plan.steps:
            launches.extend(st.launches(addr))
        return BoundPlan(launches, self.rt)

    def bind(self, io_ptrs: Dict[str, int]) -> BoundPlan:
        """``io_ptrs``: input / output name -> device address."""
        from nkipy_amd.runtime.hip import check_current

        check_current(self.rt, "plan")
        key = tuple(sorted(io_ptrs.items()))
        bp = self._bound.get(key)
        if bp is None:
            plan = self.plan
            bases: Dict[int, int] = {i: b.ptr for i, b in self._owned.items()}
            for name, idx in plan.input_buffers.items():
                bases[idx] = io_ptrs[name]
            for name, idx in plan.output_buffers.items():
                bases[idx] = io_ptrs[name]
            if len(self._bound) > 64:
                self._release_graphs()
                self._bound.clear()
            bp = self._bind(bases)
            self._bound[key] = bp
        return bp

    def run(self, io_ptrs: Dict[str, int], graph: bool = False):
        bp = self.bind(io_ptrs)
        if graph:
            bp.run_graph()
        else:
            bp.run()

    def run_checks(self):
        """The plan's host-side checks (:data:`CHECKS`) over what the last
        completed execution left in their temporaries; the caller has
        synchronised."""
        for c in getattr(self.plan, "checks", ()):
            buf = self._owned[c["buffer"]]
            count = int(c["count"])
            words = np.empty(count, np.uint32)
            self.rt.d2h(words.ctypes.data, buf.ptr + int(c["offset"]), 4 * count)
            CHECKS[c["kind"]](words, c.get("desc", ""))

    def _release_graphs(self):
        for bp in self._bound.values():
            bp.release_graph()

    def forget(self):
        """Drop every bound launch list and owned buffer without touching the
        device (the runtime they belong to is gone)."""
        self._owned.clear()
        self._bound.clear()

    def close(self):
        self._release_graphs()
        for b in self._owned.values():
            b.free()
        self._owned.clear()
        self._bound.clear()
