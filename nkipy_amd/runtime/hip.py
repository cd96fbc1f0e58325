"""ctypes binding of ``libnkipy_hip.so`` (declared in ``include/nkipy_hip.h``).

This module is the Python face of the native runtime that replaces the
reference's Spike/NRT stack:

* ``SpikeRuntimeError`` / ``SpikeError`` / ``NrtError`` keep the reference's
  exception hierarchy (spike/src/python_bindings.cpp:27-30).  ``NrtError`` is
  an alias of :class:`HipError`, which carries the ``hipError_t`` name the
  way NrtError carries the NRT status name (spike/src/include/error.h:23-44).
* :func:`get_runtime` returns the process-wide runtime, initialised lazily
  with double-checked locking like ``get_spike_singleton``
  (spike/src/spike/spike_singleton.py:123-147).
* ctypes releases the GIL around every foreign call, which is what the
  reference does explicitly around execute (python_bindings.cpp:121-126).
"""

from __future__ import annotations

import contextlib
import ctypes
import json
import os
import threading
from pathlib import Path
from typing import Dict, Optional, Tuple

from nkipy_amd import _build

c_int_p = ctypes.POINTER(ctypes.c_int)

NKH_OK = 0
NKH_ERR_HIP = 1
NKH_ERR_INVALID = 2
NKH_ERR_NOT_INIT = 3
NKH_ERR_BOUNDS = 4
NKH_ERR_FREED = 5
NKH_ERR_ALREADY_INIT = 6


class SpikeRuntimeError(RuntimeError):
    """Base class of every runtime error raised by the backend."""


class SpikeError(SpikeRuntimeError):
    """Runtime-level misuse: bounds, lifetime, state, argument errors."""


class HipError(SpikeRuntimeError):
    """A HIP API call failed; the message names the ``hipError_t``."""


NrtError = HipError


class KernelArgumentError(SpikeError):
    """Packed kernel arguments do not match the kernel's declared layout."""


def _bind(lib):
    vp = ctypes.c_void_p
    sz = ctypes.c_size_t
    u = ctypes.c_uint
    sigs = {
        "nkh_last_error": ([], ctypes.c_char_p),
        "nkh_init": ([ctypes.c_int], ctypes.c_int),
        "nkh_shutdown": ([], ctypes.c_int),
        "nkh_is_initialized": ([c_int_p], ctypes.c_int),
        "nkh_device_count": ([c_int_p], ctypes.c_int),
        "nkh_device_info": (
            [c_int_p, c_int_p, c_int_p, c_int_p, c_int_p, ctypes.c_char_p, sz],
            ctypes.c_int,
        ),
        "nkh_malloc": ([sz, ctypes.POINTER(vp)], ctypes.c_int),
        "nkh_free": ([vp], ctypes.c_int),
        "nkh_alloc_size": ([vp, ctypes.POINTER(sz)], ctypes.c_int),
        "nkh_memcpy_h2d": ([vp, vp, sz], ctypes.c_int),
        "nkh_memcpy_d2h": ([vp, vp, sz], ctypes.c_int),
        "nkh_memcpy_d2d": ([vp, vp, sz], ctypes.c_int),
        "nkh_memset": ([vp, ctypes.c_int, sz], ctypes.c_int),
        "nkh_module_load": ([ctypes.c_char_p, ctypes.POINTER(vp)], ctypes.c_int),
        "nkh_module_unload": ([vp], ctypes.c_int),
        "nkh_get_function": ([vp, ctypes.c_char_p, ctypes.POINTER(vp)], ctypes.c_int),
        "nkh_launch": ([vp, u, u, u, u, u, u, u, vp, sz], ctypes.c_int),
        "nkh_sync": ([], ctypes.c_int),
        "nkh_time_launch": (
            [vp, u, u, u, u, u, u, u, vp, sz, ctypes.c_int, ctypes.c_int,
             ctypes.POINTER(ctypes.c_float)],
            ctypes.c_int,
        ),
        "nkh_event_create": ([ctypes.POINTER(vp)], ctypes.c_int),
        "nkh_event_destroy": ([vp], ctypes.c_int),
        "nkh_event_record": ([vp], ctypes.c_int),
        "nkh_event_elapsed_ms": ([vp, vp, ctypes.POINTER(ctypes.c_float)], ctypes.c_int),
        "nkh_launch_batch": (
            [ctypes.c_int, ctypes.POINTER(vp), ctypes.POINTER(u), ctypes.POINTER(u),
             ctypes.POINTER(u), ctypes.c_char_p, ctypes.POINTER(sz), ctypes.POINTER(sz)],
            ctypes.c_int,
        ),
    }
    sigs["nkh_graph_create"] = (sigs["nkh_launch_batch"][0] + [ctypes.POINTER(vp)], ctypes.c_int)
    sigs["nkh_graph_launch"] = ([vp], ctypes.c_int)
    sigs["nkh_graph_destroy"] = ([vp], ctypes.c_int)
    sigs["nkh_profile_range_push"] = ([ctypes.c_char_p, c_int_p], ctypes.c_int)
    sigs["nkh_profile_range_pop"] = ([], ctypes.c_int)
    i64 = ctypes.c_int64
    sigs["nkh_linear_attention_workspace_size"] = ([i64, i64, ctypes.POINTER(sz)], ctypes.c_int)
    sigs["nkh_linear_attention"] = ([vp, vp, vp, vp, i64, i64, vp, sz], ctypes.c_int)
    sigs["nkh_linear_attention_noalloc"] = ([vp, vp, vp, vp, i64, i64], ctypes.c_int)
    for name, (argtypes, restype) in sigs.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = restype
    return lib


# Names the header declares; a test checks the built library exports each one.
EXPORTED_SYMBOLS = (
    "nkh_last_error", "nkh_init", "nkh_shutdown", "nkh_is_initialized",
    "nkh_device_count", "nkh_device_info", "nkh_malloc", "nkh_free",
    "nkh_alloc_size", "nkh_memcpy_h2d", "nkh_memcpy_d2h", "nkh_memcpy_d2d",
    "nkh_memset", "nkh_module_load", "nkh_module_unload", "nkh_get_function",
    "nkh_launch", "nkh_sync", "nkh_time_launch", "nkh_event_create",
    "nkh_event_destroy", "nkh_event_record", "nkh_event_elapsed_ms",
    "nkh_launch_batch", "nkh_linear_attention_workspace_size", "nkh_linear_attention",
    "nkh_linear_attention_noalloc", "nkh_profile_range_push", "nkh_profile_range_pop",
    "nkh_graph_create", "nkh_graph_launch", "nkh_graph_destroy",
)

_lib = None
_lib_lock = threading.Lock()


def library_path() -> Path:
    return _build.RUNTIME_LIB


def load_library():
    """Load the native runtime library (no device call is made)."""
    global _lib
    if _lib is None:
        with _lib_lock:
            if _lib is None:
                path = library_path()
                if not path.exists():
                    raise SpikeError(
                        f"native runtime {path} is not built; run "
                        "`python -c 'import __graft_entry__ as g; g.build()'` or "
                        "`python -m nkipy_amd._build`"
                    )
                _lib = _bind(ctypes.CDLL(str(path)))
    return _lib


def _check(rc: int, what: str = ""):
    if rc == NKH_OK:
        return
    msg = load_library().nkh_last_error().decode(errors="replace")
    if what:
        msg = f"{what}: {msg}"
    if rc == NKH_ERR_HIP:
        raise HipError(msg)
    raise SpikeError(msg)


def device_count() -> int:
    """Number of visible GPUs (0 when the HIP driver reports no device)."""
    n = ctypes.c_int(0)
    _check(load_library().nkh_device_count(ctypes.byref(n)), "device count")
    return n.value


class Module:
    """A loaded gfx950 code object plus its kernel manifest."""

    def __init__(self, rt: "HipRuntime", name: str, handle: int, manifest: dict):
        self.rt = rt
        self.name = name
        self.handle = handle
        self.manifest = manifest
        self._functions: Dict[str, "Function"] = {}

    def function(self, symbol: str) -> "Function":
        fn = self._functions.get(symbol)
        if fn is None:
            if symbol not in self.manifest:
                raise SpikeError(
                    f"kernel '{symbol}' is not in code object '{self.name}'"
                )
            h = ctypes.c_void_p()
            _check(
                self.rt.lib.nkh_get_function(
                    ctypes.c_void_p(self.handle), symbol.encode(), ctypes.byref(h)
                ),
                f"get_function({symbol})",
            )
            fn = Function(self.rt, symbol, h.value, self.manifest[symbol])
            self._functions[symbol] = fn
        return fn


class Function:
    """A kernel entry point; launches take a packed ctypes argument struct."""

    def __init__(self, rt: "HipRuntime", name: str, handle: int, meta: dict):
        self.rt = rt
        self.name = name
        self.handle = handle
        self.meta = meta
        self.kernarg_size = int(meta.get("explicit_size", meta["kernarg_size"]))
        if meta.get("hidden_args"):
            raise KernelArgumentError(
                f"kernel '{name}' uses hidden (implicit) arguments; kernels launched "
                "through packed argument blocks must not read gridDim/blockDim"
            )
        self.max_block = int(meta.get("max_block", 1024))

    def check_args(self, args) -> bytes:
        blob = bytes(args) if not isinstance(args, (bytes, bytearray)) else bytes(args)
        if len(blob) != self.kernarg_size:
            raise KernelArgumentError(
                f"kernel '{self.name}' takes {self.kernarg_size} bytes of arguments, "
                f"got {len(blob)}"
            )
        return blob

    def check_block(self, block):
        threads = block[0] * block[1] * block[2]
        if threads > self.max_block:
            raise KernelArgumentError(
                f"kernel '{self.name}' allows at most {self.max_block} threads per "
                f"block, got {threads}"
            )

    def launch(self, grid, block, args, shared: int = 0):
        blob = self.check_args(args)
        self.check_block(block)
        _check(
            self.rt.lib.nkh_launch(
                ctypes.c_void_p(self.handle), *grid, *block, shared, blob, len(blob)
            ),
            f"launch {self.name}",
        )

    def time(self, grid, block, args, shared: int = 0, warmup: int = 3, iters: int = 20) -> float:
        """Mean device time of one launch in milliseconds (HIP events)."""
        blob = self.check_args(args)
        self.check_block(block)
        ms = ctypes.c_float(0.0)
        _check(
            self.rt.lib.nkh_time_launch(
                ctypes.c_void_p(self.handle), *grid, *block, shared, blob, len(blob),
                warmup, iters, ctypes.byref(ms),
            ),
            f"time {self.name}",
        )
        return ms.value


class HipRuntime:
    """Process-wide native runtime: one device, one stream."""

    def __init__(self, device: int = 0):
        self.lib = load_library()
        self.device = device
        _check(self.lib.nkh_init(device), "init")
        self._modules: Dict[str, Module] = {}
        self._closed = False

    # -- lifetime -------------------------------------------------------
    def close(self):
        if not self._closed:
            self._modules.clear()
            _check(self.lib.nkh_shutdown(), "shutdown")
            self._closed = True

    @property
    def is_closed(self) -> bool:
        return self._closed

    def _live(self):
        if self._closed:
            raise SpikeError("runtime has been closed")

    # -- device info ----------------------------------------------------
    def device_info(self) -> dict:
        self._live()
        cu, clk, mclk, bus, l2 = (ctypes.c_int() for _ in range(5))
        arch = ctypes.create_string_buffer(64)
        _check(
            self.lib.nkh_device_info(
                ctypes.byref(cu), ctypes.byref(clk), ctypes.byref(mclk),
                ctypes.byref(bus), ctypes.byref(l2), arch, 64,
            ),
            "device_info",
        )
        return {
            "cu_count": cu.value,
            "clock_khz": clk.value,
            "mem_clock_khz": mclk.value,
            "mem_bus_bits": bus.value,
            "l2_bytes": l2.value,
            "arch": arch.value.decode(),
        }

    # -- memory ---------------------------------------------------------
    def malloc(self, nbytes: int) -> int:
        self._live()
        p = ctypes.c_void_p()
        _check(self.lib.nkh_malloc(max(int(nbytes), 1), ctypes.byref(p)), "malloc")
        return p.value

    def free(self, ptr: int):
        self._live()
        _check(self.lib.nkh_free(ctypes.c_void_p(ptr)), "free")

    def h2d(self, dst: int, src_addr: int, nbytes: int):
        self._live()
        _check(
            self.lib.nkh_memcpy_h2d(ctypes.c_void_p(dst), ctypes.c_void_p(src_addr), nbytes),
            "write",
        )

    def d2h(self, dst_addr: int, src: int, nbytes: int):
        self._live()
        _check(
            self.lib.nkh_memcpy_d2h(ctypes.c_void_p(dst_addr), ctypes.c_void_p(src), nbytes),
            "read",
        )

    def d2d(self, dst: int, src: int, nbytes: int):
        self._live()
        _check(
            self.lib.nkh_memcpy_d2d(ctypes.c_void_p(dst), ctypes.c_void_p(src), nbytes),
            "copy",
        )

    def memset(self, ptr: int, value: int, nbytes: int):
        self._live()
        _check(self.lib.nkh_memset(ctypes.c_void_p(ptr), value, nbytes), "memset")

    def sync(self):
        self._live()
        _check(self.lib.nkh_sync(), "sync")

    # -- code objects ---------------------------------------------------
    def module(self, name: str) -> Module:
        """Load (once) the code object ``nkipy_amd/lib/<name>.hsaco``."""
        self._live()
        mod = self._modules.get(name)
        if mod is None:
            path = _build.hsaco_path(name)
            manifest_path = path.with_suffix(".json")
            if not path.exists() or not manifest_path.exists():
                raise SpikeError(
                    f"code object {path} is not built; run `python -m nkipy_amd._build`"
                )
            manifest = json.loads(manifest_path.read_text())
            h = ctypes.c_void_p()
            _check(self.lib.nkh_module_load(str(path).encode(), ctypes.byref(h)),
                   f"load {path.name}")
            mod = Module(self, name, h.value, manifest)
            self._modules[name] = mod
        return mod

    def function(self, module: str, symbol: str) -> Function:
        return self.module(module).function(symbol)

    # -- events ---------------------------------------------------------
    def event(self) -> "Event":
        self._live()
        return Event(self)


@contextlib.contextmanager
def profile_range(name: str):
    """A named roctx range around the enclosed host calls (``rocprofv3
    --marker-trace`` shows it); yields whether a roctx library was found."""
    lib = load_library()
    avail = ctypes.c_int(0)
    _check(lib.nkh_profile_range_push(name.encode(), ctypes.byref(avail)), "profile_range_push")
    try:
        yield bool(avail.value)
    finally:
        _check(lib.nkh_profile_range_pop(), "profile_range_pop")


class Event:
    def __init__(self, rt: HipRuntime):
        self.rt = rt
        h = ctypes.c_void_p()
        _check(rt.lib.nkh_event_create(ctypes.byref(h)), "event_create")
        self.handle = h.value

    def record(self):
        _check(self.rt.lib.nkh_event_record(ctypes.c_void_p(self.handle)), "event_record")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        _check(
            self.rt.lib.nkh_event_elapsed_ms(
                ctypes.c_void_p(self.handle), ctypes.c_void_p(end.handle), ctypes.byref(ms)
            ),
            "event_elapsed",
        )
        return ms.value

    def destroy(self):
        if self.handle and not self.rt.is_closed:
            _check(self.rt.lib.nkh_event_destroy(ctypes.c_void_p(self.handle)), "event_destroy")
        self.handle = None


_runtime: Optional[HipRuntime] = None
_runtime_lock = threading.Lock()


def default_device() -> int:
    return int(os.environ.get("NKIPY_DEVICE", "0"))


def get_runtime() -> HipRuntime:
    """Return the process-wide runtime, creating it on first use."""
    global _runtime
    if _runtime is None or _runtime.is_closed:
        with _runtime_lock:
            if _runtime is None or _runtime.is_closed:
                _runtime = HipRuntime(default_device())
    return _runtime


_reset_hooks = []


def on_reset(fn):
    """Register ``fn()`` to run when the process-wide runtime is reset (caches
    of loaded kernels drop their handles there)."""
    _reset_hooks.append(fn)
    return fn


def reset_runtime():
    """Close the process-wide runtime (every device buffer, code object and
    loaded kernel becomes invalid)."""
    global _runtime
    with _runtime_lock:
        if _runtime is not None and not _runtime.is_closed:
            _runtime.close()
        _runtime = None
    for fn in list(_reset_hooks):
        fn()


def check_current(rt: "HipRuntime", what: str = "kernel"):
    """Raise SpikeError unless ``rt`` is the live process-wide runtime."""
    if rt.is_closed or rt is not _runtime:
        raise SpikeError(f"{what} belongs to a runtime that has been reset or closed; load it again")


def runtime_is_active() -> bool:
    return _runtime is not None and not _runtime.is_closed


def grid_block(n_blocks: int, block: int) -> Tuple[Tuple[int, int, int], Tuple[int, int, int]]:
    return (int(n_blocks), 1, 1), (int(block), 1, 1)
