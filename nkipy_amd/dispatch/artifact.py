"""Compiled-kernel artefacts: a lowered plan in relocatable form, written to
disk and loaded back by graph hash.

This is the role the NEFF file plays in the reference: ``DeviceKernel``
keeps it under ``build_dir/<name>_<content hash>/`` and a later process that
traces the same graph loads it instead of compiling again
(nkipy/src/nkipy/runtime/device_kernel.py:258-295).  Here "compiling" is the
pattern lowering of the traced graph; the artefact stores its result as
the packed kernel-argument blocks of every launch, with the byte offsets of
the device addresses inside them (relocations), so binding a loaded
artefact to new buffers is a patch of those addresses, with no tracing
state, launcher logic or lowering involved.

Relocations are found by lowering the plan's launches twice, against two
synthetic address spaces, and diffing the argument blocks: every 8-byte
field that differs must be (synthetic base of some buffer + the same
offset) in both, and every other byte must be equal.  A plan whose launch
arguments encode addresses in any other way is not relocatable and is not
written (the kernel still runs; it is just not cached on disk).  The
synthetic bases are 1 MiB aligned, so the launchers' alignment-dependent
choices (16-byte vector access) come out as for any 256-byte-aligned
buffer; a bind with an I/O address that is not 256-byte aligned therefore
goes back to the full lowering.

An artefact is used only while it is current: same format, same lowering
code (a digest of ``nkipy_amd/dispatch/*.py``) and the same gfx950 code
objects (digests of the ``.hsaco`` files its launches use).
"""

from __future__ import annotations

import hashlib
import json
import os
from dataclasses import dataclass
from pathlib import Path
from typing import Dict, List, Optional, Tuple

import numpy as np

from nkipy_amd import _build
from nkipy_amd.core import dtypes as dt
from nkipy_amd.dispatch.launchers import Launch
from nkipy_amd.dispatch.plan import BoundPlan, BufferSpec, Plan, Slot

FORMAT = 1
BACKEND_ID = "nkipy-hip-gfx950"
SYN_BASES = (0x5A5A << 32, 0x6B6B << 32)  # two synthetic address spaces, 18 TB apart
WINDOW = 1 << 20  # synthetic buffer windows are 1 MiB aligned with >= 1 MiB slack
IO_ALIGN = 256


class NotRelocatable(ValueError):
    pass


_digest_cache: Dict[str, str] = {}


def lowering_sources() -> List[Path]:
    """The files whose content decides a plan's launches and argument blocks:
    the lowering itself, plus the dtype table (item sizes and the dtype codes
    packed into argument blocks) and the IR the patterns match on."""
    pkg = Path(__file__).resolve().parent
    core = pkg.parent / "core"
    return sorted(pkg.glob("*.py")) + [core / "dtypes.py", core / "backend" / "ir.py"]


def lowering_digest() -> str:
    """Digest of the lowering code: a change to it invalidates artefacts."""
    key = "__lowering__"
    if key not in _digest_cache:
        h = hashlib.sha256()
        for p in lowering_sources():
            h.update(p.name.encode())
            h.update(p.read_bytes())
        _digest_cache[key] = h.hexdigest()[:16]
    return _digest_cache[key]


def module_digest(module: str) -> Optional[str]:
    """Digest of a code object and its manifest (None if it is not built)."""
    path = _build.hsaco_path(module)
    if not path.exists():
        return None
    st = path.stat()
    key = f"{path}:{st.st_mtime_ns}:{st.st_size}"
    if key not in _digest_cache:
        h = hashlib.sha256(path.read_bytes())
        man = path.with_suffix(".json")
        if man.exists():
            h.update(man.read_bytes())
        _digest_cache[key] = h.hexdigest()[:16]
    return _digest_cache[key]


@dataclass
class LaunchRecord:
    kind: str
    module: str
    symbol: str
    grid: Tuple[int, int, int]
    block: Tuple[int, int, int]
    shared: int
    blob: bytes  # argument block with every relocated address zeroed
    relocs: List[Tuple[int, int, int]]  # (byte offset, buffer index, offset into the buffer)
    bytes: int = 0
    flops: int = 0

    def patched(self, bases: Dict[int, int]) -> bytes:
        b = bytearray(self.blob)
        for off, buf, delta in self.relocs:
            b[off:off + 8] = (bases[buf] + delta).to_bytes(8, "little")
        return bytes(b)


def _windows(plan_buffers, base: int) -> Dict[int, int]:
    bases, cur = {}, base
    for b in plan_buffers:
        bases[b.index] = cur
        cur += (max(b.nbytes, 16) + 2 * WINDOW - 1) // WINDOW * WINDOW
    return bases


def _lowered_launches(plan: Plan, bases: Dict[int, int]):
    def addr(v) -> int:
        s = v if isinstance(v, Slot) else plan.slot(v)
        return bases[s.buffer] + s.offset

    return [(st.kind, l) for st in plan.steps for l in st.launches(addr)]


class RelocatablePlan:
    """A lowered plan as relocatable launch records plus its buffers and the
    kernel's I/O contract; drop-in for :class:`Plan` in an executor."""

    def __init__(self, *, name, buffers, input_buffers, output_buffers, alias_outputs, steps, records, io,
                 modules, lowering, checks=()):
        self.name = name
        self.buffers: List[BufferSpec] = buffers
        self.input_buffers: Dict[str, int] = input_buffers
        self.output_buffers: Dict[str, int] = output_buffers
        self.alias_outputs: Dict[str, str] = alias_outputs
        self.step_info: List[dict] = steps
        self.records: List[LaunchRecord] = records
        self.io: dict = io
        self.modules: Dict[str, Optional[str]] = modules
        self.lowering = lowering
        self.checks: List[dict] = [dict(c) for c in checks]

    # -- Plan-like surface ---------------------------------------------
    @property
    def kernel_kinds(self) -> List[str]:
        return [s["kind"] for s in self.step_info]

    def describe(self) -> dict:
        return {"graph": self.name,
                "buffers": [{"index": b.index, "kind": b.kind, "name": b.name, "nbytes": b.nbytes}
                            for b in self.buffers],
                "steps": self.step_info}

    def summary(self) -> str:
        lines = [f"plan {self.name} (loaded artefact): {len(self.step_info)} steps, "
                 f"{sum(1 for b in self.buffers if b.kind == 'temp')} temporaries"]
        lines += [f"  [{s['kind']}] {s['desc']}" for s in self.step_info]
        return "\n".join(lines)

    # -- construction ----------------------------------------------------
    @classmethod
    def from_plan(cls, plan: Plan, io: dict) -> "RelocatablePlan":
        ba, bb = _windows(plan.buffers, SYN_BASES[0]), _windows(plan.buffers, SYN_BASES[1])
        spans = sorted((ba[i], ba[i] + ((max(b.nbytes, 16) + 2 * WINDOW - 1) // WINDOW * WINDOW), i)
                       for i, b in ((b.index, b) for b in plan.buffers))
        la, lb = _lowered_launches(plan, ba), _lowered_launches(plan, bb)
        if len(la) != len(lb):
            raise NotRelocatable("launch count depends on addresses")
        records = []
        for (kind, a), (_, b) in zip(la, lb):
            if (a.module, a.symbol, tuple(a.grid), tuple(a.block), a.shared) != \
                    (b.module, b.symbol, tuple(b.grid), tuple(b.block), b.shared):
                raise NotRelocatable(f"launch {a.symbol} changes with addresses")
            A = bytearray(a.args if isinstance(a.args, (bytes, bytearray)) else bytes(a.args))
            B = bytearray(b.args if isinstance(b.args, (bytes, bytearray)) else bytes(b.args))
            if len(A) != len(B):
                raise NotRelocatable(f"argument size of {a.symbol} changes with addresses")
            relocs = []
            for off in range(0, len(A) - 7, 8):
                va = int.from_bytes(A[off:off + 8], "little")
                vb = int.from_bytes(B[off:off + 8], "little")
                if va == vb:
                    continue
                hit = next((i for lo, hi, i in spans if lo <= va < hi), None)
                if hit is None or vb - bb[hit] != va - ba[hit]:
                    raise NotRelocatable(f"field at byte {off} of {a.symbol} is not a buffer address")
                relocs.append((off, hit, va - ba[hit]))
                A[off:off + 8] = bytes(8)
                B[off:off + 8] = bytes(8)
            if A != B:
                raise NotRelocatable(f"{a.symbol} encodes addresses outside 8-byte fields")
            records.append(LaunchRecord(kind, a.module, a.symbol, tuple(a.grid), tuple(a.block), int(a.shared),
                                        bytes(A), relocs, int(a.bytes), int(a.flops)))
        modules = {r.module: module_digest(r.module) for r in records}
        return cls(name=plan.graph.name, buffers=list(plan.buffers), input_buffers=dict(plan.input_buffers),
                   output_buffers=dict(plan.output_buffers), alias_outputs=dict(plan.alias_outputs),
                   steps=[{"kind": s["kind"], "desc": s["desc"]} for s in plan.describe()["steps"]],
                   records=records, io=io, modules=modules, lowering=lowering_digest(),
                   checks=list(getattr(plan, "checks", ())))

    # -- binding ---------------------------------------------------------
    def blobs(self, bases: Dict[int, int]) -> List[bytes]:
        return [r.patched(bases) for r in self.records]

    def bind(self, bases: Dict[int, int], rt) -> BoundPlan:
        launches = [Launch(r.module, r.symbol, r.grid, r.block, blob, r.shared, bytes=r.bytes, flops=r.flops)
                    for r, blob in zip(self.records, self.blobs(bases))]
        return BoundPlan(launches, rt)

    def is_current(self) -> bool:
        return self.lowering == lowering_digest() and all(
            d is not None and module_digest(m) == d for m, d in self.modules.items())

    # -- persistence -----------------------------------------------------
    def save(self, path: str):
        path = Path(path)
        path.parent.mkdir(parents=True, exist_ok=True)
        bufs = []
        for b in self.buffers:
            e = {"index": b.index, "nbytes": b.nbytes, "kind": b.kind, "name": b.name, "data": None}
            if b.kind == "const" and b.data is not None:
                raw = np.ascontiguousarray(dt.numpy_storage(np.ascontiguousarray(b.data))).reshape(-1).view(np.uint8)
                fname = f"{path.stem}.const{b.index}.npy"
                # written under a temporary name and renamed, like the JSON:
                # a concurrent reader sees the old payload or the new one
                part = path.parent / (fname + f".{os.getpid()}.tmp")
                with open(part, "wb") as f:
                    np.save(f, raw, allow_pickle=False)
                os.replace(part, path.parent / fname)
                e["data"] = fname
                e["sha256"] = hashlib.sha256(raw.tobytes()).hexdigest()
            bufs.append(e)
        doc = {
            "format": FORMAT, "backend": BACKEND_ID, "lowering": self.lowering, "modules": self.modules,
            "name": self.name, "io": self.io, "buffers": bufs,
            "input_buffers": self.input_buffers, "output_buffers": self.output_buffers,
            "alias_outputs": self.alias_outputs, "steps": self.step_info, "checks": self.checks,
            "launches": [{"kind": r.kind, "module": r.module, "symbol": r.symbol, "grid": list(r.grid),
                          "block": list(r.block), "shared": r.shared, "args": r.blob.hex(),
                          "relocs": [list(x) for x in r.relocs], "bytes": r.bytes, "flops": r.flops}
                         for r in self.records],
        }
        tmp = path.with_suffix(path.suffix + f".{os.getpid()}.tmp")
        tmp.write_text(json.dumps(doc, indent=1))
        os.replace(tmp, path)

    @classmethod
    def load(cls, path: str) -> "RelocatablePlan":
        path = Path(path)
        doc = json.loads(path.read_text())
        if doc.get("format") != FORMAT or doc.get("backend") != BACKEND_ID or "launches" not in doc:
            raise NotRelocatable(f"{path} is not a relocatable plan of this backend")
        bufs = []
        for e in doc["buffers"]:
            data = None
            if e.get("data"):
                data = np.load(path.parent / e["data"], allow_pickle=False)
                want = e.get("sha256")
                if want is not None and hashlib.sha256(np.ascontiguousarray(data).tobytes()).hexdigest() != want:
                    raise NotRelocatable(f"{path}: constant payload {e['data']} does not match its checksum")
            bufs.append(BufferSpec(int(e["index"]), int(e["nbytes"]), e["kind"], e["name"], data))
        records = [LaunchRecord(r["kind"], r["module"], r["symbol"], tuple(r["grid"]), tuple(r["block"]),
                                int(r["shared"]), bytes.fromhex(r["args"]), [tuple(x) for x in r["relocs"]],
                                int(r["bytes"]), int(r["flops"])) for r in doc["launches"]]
        return cls(name=doc["name"], buffers=bufs, input_buffers={k: int(v) for k, v in doc["input_buffers"].items()},
                   output_buffers={k: int(v) for k, v in doc["output_buffers"].items()},
                   alias_outputs=dict(doc["alias_outputs"]), steps=doc["steps"], records=records, io=doc["io"],
                   modules=doc["modules"], lowering=doc["lowering"], checks=doc.get("checks", []))


def io_contract(graph) -> dict:
    """The kernel's I/O names, shapes and dtypes and its aliases (what a
    loaded artefact must match, and what a graph-less load serves)."""
    return {
        "inputs": [[p.name, list(p.shape), dt.name(p.dtype)] for p in graph.parameters],
        "outputs": [[r.name, list(r.shape), dt.name(r.dtype)] for r in graph.results],
        "aliases": [[a.output_index, a.param_name, bool(a.is_user_returned)] for a in graph.aliases],
    }


def write_artifact(plan: Plan, graph, path: str) -> bool:
    """Write ``plan`` at ``path`` in relocatable form; False (and the plain
    description instead) when its launches are not relocatable."""
    try:
        RelocatablePlan.from_plan(plan, io_contract(graph)).save(path)
        return True
    except NotRelocatable as e:
        Path(path).parent.mkdir(parents=True, exist_ok=True)
        Path(path).write_text(json.dumps({"format": FORMAT, "backend": BACKEND_ID, "relocatable": False,
                                          "reason": str(e), **plan.describe()}, indent=1))
        return False


def try_load(path: str, graph=None) -> Optional[RelocatablePlan]:
    """A current relocatable artefact at ``path`` matching ``graph``'s I/O
    contract, or None."""
    if not os.path.exists(path):
        return None
    try:
        rp = RelocatablePlan.load(path)
    except (NotRelocatable, ValueError, KeyError, OSError):
        return None
    if not rp.is_current():
        return None
    if graph is not None and rp.io != json.loads(json.dumps(io_contract(graph))):
        return None
    return rp
