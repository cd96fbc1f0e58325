"""Compiled kernels on the device.

``DeviceKernel`` keeps the reference's entry points
(nkipy/src/nkipy/runtime/device_kernel.py:65-295 and SpikeModel,
spike/src/spike/spike_model.py:19-343):

* ``DeviceKernel.compile_and_load(kernel, *args, name=..., ...)`` traces the
  kernel on the given arguments (NumPy arrays, DeviceTensors or torch
  tensors -- only shapes and dtypes are read), lowers the graph to a plan of
  gfx950 kernels and loads it.  Loaded kernels are cached in memory by
  ``name + content hash`` (``_LOADED_KERNELS``); the lowered plan is written
  to ``build_dir/<name>_<hash>/plan.json`` in relocatable form, and a later
  process tracing the same graph loads that artefact instead of lowering
  (``nkipy_amd.dispatch.artifact``).  ``load_from_neff(path)`` loads an
  artefact without its graph.
* ``kernel(inputs, outputs=None)`` binds named DeviceTensors, validates
  names / shapes / dtypes, runs the plan and waits for it (the synchronous
  completion point of nrt_execute); with ``outputs=None`` it allocates and
  returns the outputs.
* ``kernel.benchmark(inputs, outputs, warmup_iter, benchmark_iter, mode)``
  returns a ``BenchmarkResult``; ``mode="device"`` times each execution with
  HIP events on the runtime stream, ``mode="host"`` with wall-clock time.

The SPMD / MPMD arguments keep their meaning for the compile step under
``torch.distributed`` (rank 0 traces and broadcasts the cache key in SPMD
mode).  Collective execution is outside this single-GPU backend:
``cc_enabled=True`` raises.
"""

from __future__ import annotations

import atexit
import hashlib
import json
import math
import os
import time
import types
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import numpy as np

from nkipy_amd.core import dtypes as dt
from nkipy_amd.core.compile import _get_build_dir
from nkipy_amd.core.logger import get_logger
from nkipy_amd.core.trace import NKIPyKernel, trace
from nkipy_amd.runtime.device_tensor import DeviceTensor
from nkipy_amd.runtime.hip import SpikeError, get_runtime
from nkipy_amd.runtime.hip import on_reset as hip_on_reset

logger = get_logger()

_LOADED_KERNELS: Dict[str, "DeviceKernel"] = {}


def _cleanup_kernels():
    for dk in _LOADED_KERNELS.values():
        dk.executor.forget()
    _LOADED_KERNELS.clear()


atexit.register(_cleanup_kernels)
hip_on_reset(_cleanup_kernels)

BACKEND_ID = "nkipy-hip-gfx950-v1"


def _graph_content_hash(graph, compiler_args: str = "") -> str:
    h = hashlib.sha256()
    h.update(graph.content_hash().encode())
    h.update(BACKEND_ID.encode())
    h.update((compiler_args or "").encode())
    return h.hexdigest()[:12]


def _torch_dist():
    try:
        import torch.distributed as dist

        return dist
    except ImportError:  # pragma: no cover
        return None


def _is_distributed() -> bool:
    dist = _torch_dist()
    return dist is not None and dist.is_available() and dist.is_initialized() and dist.get_world_size() > 1


@dataclass
class BenchmarkResult:
    """Result of a benchmark run (reference: spike_model.py:19-39)."""

    mean_ms: float
    min_ms: float
    max_ms: float
    std_dev_ms: float
    iterations: int
    warmup_iterations: int
    durations_ms: List[float] = field(default_factory=list)

    def __repr__(self) -> str:
        return (
            f"BenchmarkResult(mean={self.mean_ms:.4f}ms, min={self.min_ms:.4f}ms, "
            f"max={self.max_ms:.4f}ms, std_dev={self.std_dev_ms:.4f}ms, "
            f"iterations={self.iterations}, warmup_iterations={self.warmup_iterations})"
        )


def _make_benchmark_result(durations_ms: List[float], warmup: int) -> BenchmarkResult:
    n = len(durations_ms)
    mean = sum(durations_ms) / n
    var = sum((d - mean) ** 2 for d in durations_ms) / n
    return BenchmarkResult(mean, min(durations_ms), max(durations_ms), math.sqrt(var), n,
                           warmup, list(durations_ms))


@dataclass
class TensorMetadata:
    """Input / output description (reference: TensorMetadata in the bindings)."""

    size: int
    dtype: str
    shape: List[int]


class DeviceKernel:
    """A traced kernel lowered to gfx950 kernels and loaded on the device."""

    def __init__(self, graph, plan, name: str, build_path: Optional[str] = None, lower_fn=None):
        from nkipy_amd.dispatch.plan import PlanExecutor

        self.graph = graph
        self.plan = plan
        self.name = name
        self.neff_path = build_path  # name kept from the reference API
        self.executor = PlanExecutor(plan, lower_fn=lower_fn)
        self.core_id = get_runtime().device
        if graph is not None:
            ins = [(p.name, tuple(p.shape), p.dtype) for p in graph.parameters]
            outs = [(r.name, tuple(r.shape), r.dtype) for r in graph.results]
        else:  # a loaded artefact carries the I/O contract
            ins = [(n, tuple(sh), dt.canonical(d)) for n, sh, d in plan.io["inputs"]]
            outs = [(n, tuple(sh), dt.canonical(d)) for n, sh, d in plan.io["outputs"]]
        nbytes = lambda sh, d: int(np.prod(sh, dtype=np.int64)) * dt.itemsize(d)
        self.input_tensors_info = {n: TensorMetadata(nbytes(sh, d), dt.name(d), list(sh)) for n, sh, d in ins}
        self.output_tensors_info = {n: TensorMetadata(nbytes(sh, d), dt.name(d), list(sh)) for n, sh, d in outs}
        self._in_specs = {n: (sh, dt.canonical(d)) for n, sh, d in ins}
        self._out_specs = {n: (sh, dt.canonical(d)) for n, sh, d in outs}
        self._staging: Dict[str, DeviceTensor] = {}
        # I/O sets already validated -> outputs that need staging
        self._io_checked: Dict[tuple, tuple] = {}

    # ------------------------------------------------------------------
    @classmethod
    def compile_and_load(cls, kernel, *args, name=None, additional_compiler_args=None,
                         use_cached_if_exists=True, build_dir=None, target=None,
                         is_spmd=True, cc_enabled=None, rank_id=None, world_size=None,
                         **kwargs) -> "DeviceKernel":
        if name is None:
            name = kernel.__name__
        distributed = _is_distributed()
        dist = _torch_dist()
        compile_build_dir = build_dir
        if not is_spmd:
            eff_rank = rank_id if rank_id is not None else (dist.get_rank() if distributed else None)
            if eff_rank is not None:
                compile_build_dir = os.path.join(build_dir or _get_build_dir(), f"rank_{eff_rank}")

        graph, cache_key, plan_path = cls._trace_and_compile(
            kernel, name, args, kwargs, additional_compiler_args=additional_compiler_args,
            build_dir=compile_build_dir)
        if is_spmd and distributed:
            info = [cache_key]
            dist.broadcast_object_list(info, src=0)
            if info[0] != cache_key:
                raise SpikeError(
                    f"SPMD compile mismatch: rank {dist.get_rank()} traced {cache_key}, "
                    f"rank 0 traced {info[0]}; use is_spmd=False for per-rank kernels"
                )
        if use_cached_if_exists and cache_key in _LOADED_KERNELS:
            logger.info(f"Using loaded kernel: {name} (cache_key={cache_key})")
            return _LOADED_KERNELS[cache_key]
        resolved_cc = cc_enabled if cc_enabled is not None else distributed
        if resolved_cc:
            raise SpikeError("collective execution is not supported by the single-GPU HIP backend")
        if is_spmd and distributed:
            dist.barrier()
        from nkipy_amd.dispatch import artifact

        cached = artifact.try_load(plan_path, graph) if use_cached_if_exists else None
        if cached is not None:
            # the artefact of an earlier process: no lowering (the reference
            # skips neuronx-cc the same way, device_kernel.py:272-275)
            logger.info(f"Kernel found in '{plan_path}', using cached (cache_key={cache_key})")
            dk = cls(graph, cached, name, plan_path, lower_fn=lambda: cls._lower(graph))
        else:
            plan = cls._lower(graph)
            artifact.write_artifact(plan, graph, plan_path)
            dk = cls(graph, plan, name, plan_path)
        if use_cached_if_exists:
            _LOADED_KERNELS[cache_key] = dk
        return dk

    @classmethod
    def load_from_neff(cls, neff_path: str, name: Optional[str] = None, **kwargs) -> "DeviceKernel":
        """Load a compiled artefact (the plan file ``compile_and_load`` or
        ``compile_to_neff`` wrote) without its traced graph; the name is the
        reference's (device_kernel.py:91-117)."""
        from nkipy_amd.dispatch import artifact

        try:
            rp = artifact.RelocatablePlan.load(neff_path)
        except (OSError, ValueError, KeyError) as e:
            raise SpikeError(f"cannot load compiled kernel {neff_path}: {e}") from None
        if not rp.is_current():
            raise SpikeError(f"compiled kernel {neff_path} was built by other lowering code or code objects; "
                             "compile it again")
        return cls(None, rp, name or rp.name, neff_path)

    @staticmethod
    def _lower(graph):
        from nkipy_amd.dispatch.lower import lower

        return lower(graph)

    @classmethod
    def _trace_and_compile(cls, kernel, name, args, kwargs, *, additional_compiler_args=None,
                           build_dir=None, **_):
        if not isinstance(kernel, (types.FunctionType, NKIPyKernel)):
            raise NotImplementedError(f"Unsupported kernel type: {type(kernel)}")
        traced = trace(kernel) if isinstance(kernel, types.FunctionType) else kernel
        graph = traced.specialize(*args, **kwargs)
        content_hash = _graph_content_hash(graph, additional_compiler_args or "")
        cache_key = f"{name}_{content_hash}"
        out_dir = os.path.join(build_dir or _get_build_dir(), f"{name}_{content_hash}")
        return graph, cache_key, os.path.join(out_dir, "plan.json")

    @classmethod
    def load_from_graph(cls, graph, name=None) -> "DeviceKernel":
        return cls(graph, cls._lower(graph), name or graph.name)

    # ------------------------------------------------------------------
    def allocate_output_tensors(self) -> List[DeviceTensor]:
        return [DeviceTensor.empty(shape, dtype, name=k) for k, (shape, dtype) in self._out_specs.items()]

    def _validate_io(self, inputs: Dict[str, DeviceTensor], outputs: Dict[str, DeviceTensor]):
        for kind, given, specs in (("Input", inputs, self._in_specs), ("Output", outputs, self._out_specs)):
            missing = set(specs) - set(given)
            extra = set(given) - set(specs)
            if missing or extra:
                raise SpikeError(f"{kind} names do not match the kernel: missing {sorted(missing)}, "
                                 f"unexpected {sorted(extra)}")
            for k, t in given.items():
                shape, dtype = specs[k]
                if tuple(t.shape) != shape:
                    raise SpikeError(f"{kind} {k}: expected shape {shape}, got {tuple(t.shape)}")
                if dt.canonical(t.dtype) != dtype:
                    raise SpikeError(f"{kind} {k}: expected dtype {dt.name(dtype)}, got {dt.name(t.dtype)}")
        for out_name, in_name in self.plan.alias_outputs.items():
            if out_name in outputs and in_name in inputs and outputs[out_name].ptr != inputs[in_name].ptr:
                raise SpikeError(f"Output {out_name} must share the buffer of input {in_name}")

    def _io_ptrs(self, inputs, outputs) -> Dict[str, int]:
        ptrs = {k: v.ptr for k, v in inputs.items()}
        ptrs.update({k: v.ptr for k, v in outputs.items()})
        return ptrs

    def _overlapping_outputs(self, inputs, outputs) -> List[str]:
        """Outputs whose buffer overlaps an input other than the one it is
        declared to alias (e.g. a layer writing its result over its own
        input x, qwen3.py:281-338): the plan may still read that input after
        writing the output, so such outputs go through a staging buffer."""
        alias_in = self.plan.alias_outputs
        hits = []
        for on, ot in outputs.items():
            lo, hi = ot.ptr, ot.ptr + ot.nbytes
            for inn, it in inputs.items():
                if alias_in.get(on) == inn:
                    continue
                if it.ptr < hi and lo < it.ptr + it.nbytes:
                    hits.append(on)
                    break
        return hits

    def __call__(self, inputs: Dict[str, DeviceTensor], outputs: Dict[str, DeviceTensor] = None,
                 save_trace: bool = False, ntff_name: Optional[str] = None, sync: bool = True,
                 graph: bool = False):
        """Runs the kernel on ``inputs`` into ``outputs`` (allocated when
        None and returned).  ``sync`` waits for the launches and runs the
        plan's host checks; ``graph`` replays the launches as one HIP graph
        captured on the first call with these tensors (a serving loop that
        calls with the same tensors every step pays one host call per step);
        ``save_trace`` writes a per-launch profile instead."""
        auto = outputs is None
        if auto:
            outputs = {t.name: t for t in self.allocate_output_tensors()}
            for out_name, in_name in self.plan.alias_outputs.items():
                if in_name in inputs:
                    outputs[out_name] = inputs[in_name]
        # a serving loop calls with the same tensors every step: the checks
        # of names, shapes, dtypes, aliasing and overlap run once per set
        key = (tuple((k, t.ptr, t.shape, t.dtype) for k, t in inputs.items()),
               tuple((k, t.ptr, t.shape, t.dtype) for k, t in outputs.items()))
        ent = self._io_checked.get(key)
        if ent is None:
            self._validate_io(inputs, outputs)
            staged = tuple(self._overlapping_outputs(inputs, outputs))
            # the argument addresses of a set without staged outputs, formed
            # once (a private dict: nothing mutates it)
            io = None if staged else self._io_ptrs(inputs, outputs)
            if len(self._io_checked) > 64:
                self._io_checked.clear()
            ent = self._io_checked[key] = (staged, io)
        staged, io = ent
        if staged:
            run_outputs = dict(outputs)
            for on in staged:
                st = self._staging.get(on)
                if st is None or st.tensor_ref.is_freed:
                    shape, dtype = self._out_specs[on]
                    st = self._staging[on] = DeviceTensor.empty(shape, dtype, name=on)
                run_outputs[on] = st
            self._execute(self._io_ptrs(inputs, run_outputs), save_trace, ntff_name, graph)
            rt = get_runtime()
            for on in staged:
                rt.d2d(outputs[on].ptr, run_outputs[on].ptr, outputs[on].nbytes)
        else:
            self._execute(io, save_trace, ntff_name, graph)
        if sync:
            get_runtime().sync()
            # words the kernels left for the host (e.g. the linear-attention
            # operand range), checked once the execution is complete
            self.executor.run_checks()
        if auto:
            return outputs
        return None

    def trace_path(self, ntff_name: Optional[str] = None) -> str:
        """Where ``save_trace`` writes: ``ntff_name``, else beside the compiled
        artefact with its suffix replaced (spike_model.py:250-251)."""
        if ntff_name:
            return str(ntff_name)
        if self.neff_path:
            return os.path.splitext(str(self.neff_path))[0] + ".ntff"
        return f"{self.name}.ntff"

    def _execute(self, io_ptrs: Dict[str, int], save_trace: bool, ntff_name: Optional[str],
                 graph: bool = False):
        if not save_trace:
            self.executor.run(io_ptrs, graph=graph)
            return
        self._run_profiled(io_ptrs, self.trace_path(ntff_name))

    def _run_profiled(self, io_ptrs: Dict[str, int], path: str):
        """One execution with every launch bracketed by events, inside a
        roctx range named after the kernel: the profile the reference takes
        between nrt_profile_start / nrt_profile_stop (spike/src/model.cpp:
        97-103).  Writes a Chrome trace-event JSON document (one complete
        event per launch, microseconds, back to back on the runtime stream)
        to ``path`` and returns it."""
        from nkipy_amd.runtime.hip import profile_range

        rt = get_runtime()
        bound = self.executor.bind(io_ptrs)
        n = len(bound.launches)
        evs = [rt.event() for _ in range(n + 1)]
        try:
            rt.sync()
            with profile_range(f"nkipy:{self.name}") as have_roctx:
                evs[0].record()
                for i in range(n):
                    bound.run_range(i, i + 1)
                    evs[i + 1].record()
                rt.sync()
            durs = [evs[i].elapsed_ms(evs[i + 1]) * 1e3 for i in range(n)]
        finally:
            for e in evs:
                e.destroy()
        events, t = [], 0.0
        for l, d in zip(bound.launches, durs):
            args = {"module": l.module, "grid": list(l.grid), "block": list(l.block), "lds_bytes": l.shared}
            if l.bytes:
                args["bytes"] = int(l.bytes)
                args["GB_per_s"] = l.bytes / (d * 1e3) if d > 0 else None
            if l.flops:
                args["flops"] = int(l.flops)
                args["TFLOP_per_s"] = l.flops / (d * 1e6) if d > 0 else None
            events.append({"name": l.symbol, "cat": "kernel", "ph": "X", "ts": round(t, 3),
                           "dur": round(d, 3), "pid": 0, "tid": 0, "args": args})
            t += d
        doc = {"traceEvents": events, "displayTimeUnit": "ns",
               "otherData": {"kernel": self.name, "device": rt.device, "steps": list(self.plan.kernel_kinds),
                             "total_us": round(t, 3), "roctx_range": have_roctx}}
        d = os.path.dirname(os.path.abspath(path))
        os.makedirs(d, exist_ok=True)
        tmp = f"{path}.{os.getpid()}.tmp"
        with open(tmp, "w") as f:
            json.dump(doc, f, indent=1)
        os.replace(tmp, path)
        logger.info(f"wrote execution trace of {self.name} to {path}")
        return doc

    def benchmark(self, inputs, outputs=None, warmup_iter=5, benchmark_iter=5, mode: str = "device"):
        if mode not in ("device", "host"):
            raise ValueError(f"Invalid benchmark mode '{mode}'. Use 'device' or 'host'.")
        if outputs is None:
            outputs = {t.name: t for t in self.allocate_output_tensors()}
            for out_name, in_name in self.plan.alias_outputs.items():
                if in_name in inputs:
                    outputs[out_name] = inputs[in_name]
        self._validate_io(inputs, outputs)
        bound = self.executor.bind(self._io_ptrs(inputs, outputs))
        rt = get_runtime()
        for _ in range(warmup_iter):
            bound.run()
        rt.sync()
        durations = []
        if mode == "device":
            evs = [rt.event() for _ in range(benchmark_iter + 1)]
            evs[0].record()
            for i in range(benchmark_iter):
                bound.run()
                evs[i + 1].record()
            rt.sync()
            durations = [evs[i].elapsed_ms(evs[i + 1]) for i in range(benchmark_iter)]
            for e in evs:
                e.destroy()
        else:
            for _ in range(benchmark_iter):
                t0 = time.perf_counter()
                bound.run()
                rt.sync()
                durations.append((time.perf_counter() - t0) * 1e3)
        if not durations:
            raise RuntimeError("benchmark_iter must be at least 1")
        return _make_benchmark_result(durations, warmup_iter)

    def __repr__(self):
        return f"DeviceKernel('{self.name}', steps={list(self.plan.kernel_kinds)})"
