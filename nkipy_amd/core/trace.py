"""Kernel tracing: ``NKIPyKernel``.

Mirrors the reference's ``NKIPyKernel`` (nkipy/src/nkipy/core/trace.py:50-250):

* ``NKIPyKernel.trace(func, backend=...)`` wraps a NumPy kernel function;
  ``specialize(*args, **kwargs)`` runs it once under a trace context with
  every array argument replaced by a traced parameter, and stores the
  recorded graph in ``._code``.
* Outputs follow the reference naming contract: a parameter mutated through
  ``__setitem__`` is renamed ``<name>.must_alias_input`` and its result takes
  the parameter's name; a mutated parameter the kernel does not return is
  appended to the results (auto-alias); a result that is a bare parameter
  gets an explicit ``copy``; the remaining results are named ``output{i}``.
* float64 / int64 / uint64 array arguments are narrowed to 32 bits with a
  warning (``_sanitize_array_dtype``, reference trace.py:25-47).

``backend`` is ``"hip"`` (the default).  ``"hlo"`` -- the reference's
default -- is accepted as a synonym so existing call sites keep working.
"""

from __future__ import annotations

import inspect
import warnings

import numpy as np

from nkipy_amd.core import dtypes as dt
from nkipy_amd.core._numpy_dispatch import register_all_numpy_apis
from nkipy_amd.core.backend import tracing
from nkipy_amd.core.backend.hip import HIPTraceContext
from nkipy_amd.core.backend.ir import AliasInfo, Graph
from nkipy_amd.core.tensor import NKIPyTensorRef

register_all_numpy_apis()

_DTYPE_DOWNCAST = {
    np.dtype("float64"): np.dtype("float32"),
    np.dtype("int64"): np.dtype("int32"),
    np.dtype("uint64"): np.dtype("uint32"),
}

TRACE_BACKENDS = ("hip", "hlo")


def _sanitize_array_dtype(arr: np.ndarray, name: str = "") -> np.ndarray:
    target = _DTYPE_DOWNCAST.get(arr.dtype)
    if target is None:
        return arr
    label = f" '{name}'" if name else ""
    warnings.warn(
        f"Input tensor{label} has dtype {arr.dtype} which is not supported by the "
        f"device. Automatically casting to {target}.",
        stacklevel=3,
    )
    return arr.astype(target)


def is_array_arg(a) -> bool:
    """Arguments that become traced parameters: NumPy arrays, device
    tensors and torch tensors (anything array-like with a shape and dtype)."""
    if isinstance(a, np.ndarray):
        return True
    mod = type(a).__module__ or ""
    if mod.startswith("torch") and hasattr(a, "shape") and hasattr(a, "dtype"):
        return True
    return hasattr(a, "shape") and hasattr(a, "dtype") and hasattr(a, "tensor_ref")


def kernel_signature(func, n_args: int, kwargs) -> inspect.Signature:
    """The kernel function's signature.  ufuncs and builtins passed as the
    kernel (np.matmul, np.where, ...) have none that ``inspect`` can read:
    they get positional parameters arg0, arg1, ... and keyword-only ones
    for the given keywords."""
    try:
        return inspect.signature(func)
    except (TypeError, ValueError):
        P = inspect.Parameter
        return inspect.Signature([P(f"arg{i}", P.POSITIONAL_ONLY) for i in range(n_args)]
                                 + [P(k, P.KEYWORD_ONLY) for k in kwargs])


def arg_shape_dtype(a):
    if isinstance(a, np.ndarray):
        return tuple(a.shape), a.dtype
    return tuple(int(s) for s in a.shape), dt.canonical(a.dtype)


class NKIPyKernel:
    """A NumPy kernel function that can be traced into a graph."""

    def __init__(self, func, backend="hip", **kwargs):
        if backend not in TRACE_BACKENDS + ("cpu",):
            raise ValueError(f"Unknown backend {backend}")
        self.func = func
        self.backend = backend
        self._code = None

    @property
    def __name__(self):
        return self.func.__name__

    def __repr__(self):
        return f"<NKIPyKernel '{self.func.__name__}' backend='{self.backend}'>"

    def __call__(self, *args, **kwargs):
        """Calling a traced kernel directly runs it as NumPy (CPU mode)."""
        return self.func(*args, **kwargs)

    def specialize(self, *args, **kwargs) -> Graph:
        if self.backend in TRACE_BACKENDS:
            return self._specialize_hip(*args, **kwargs)
        if self.backend == "cpu":
            print("CPU backend does not require specialization")
            return None
        raise ValueError(f"Unknown backend {self.backend}")

    # ------------------------------------------------------------------
    def _param(self, ctx, arg, name):
        if isinstance(arg, np.ndarray):
            arg = _sanitize_array_dtype(arg, name)
        shape, dtype = arg_shape_dtype(arg)
        dtype = _DTYPE_DOWNCAST.get(np.dtype(dtype), dtype) if not isinstance(arg, np.ndarray) else dtype
        v = ctx.add_parameter(shape, dtype, name)
        ref = NKIPyTensorRef(v, name=name)
        ref._original_parameter = v
        return ref

    def _specialize_hip(self, *args, **kwargs) -> Graph:
        graph = Graph(name=self.func.__name__)
        ctx = HIPTraceContext(graph)
        with tracing(ctx):
            sig = kernel_signature(self.func, len(args), kwargs)
            bound = sig.bind(*args, **kwargs)
            bound.apply_defaults()
            call_args, call_kwargs, params = [], {}, []
            for name, arg in bound.arguments.items():
                p = sig.parameters[name]
                if p.kind == p.VAR_POSITIONAL:
                    for i, item in enumerate(arg):
                        if is_array_arg(item):
                            ref = self._param(ctx, item, f"{name}_{i}")
                            params.append((f"{name}_{i}", ref))
                            call_args.append(ref)
                        else:
                            call_args.append(item)
                    continue
                if p.kind == p.VAR_KEYWORD:
                    for k, item in arg.items():
                        if is_array_arg(item):
                            ref = self._param(ctx, item, k)
                            params.append((k, ref))
                            call_kwargs[k] = ref
                        else:
                            call_kwargs[k] = item
                    continue
                value = arg
                if is_array_arg(arg):
                    value = self._param(ctx, arg, name)
                    params.append((name, value))
                if p.kind == p.KEYWORD_ONLY:
                    call_kwargs[name] = value
                else:
                    call_args.append(value)
            ret = self.func(*call_args, **call_kwargs)
            self._mark_outputs(ctx, graph, ret, params)
        self._code = graph
        return graph

    def _mark_outputs(self, ctx, graph: Graph, ret, params):
        if ret is None:
            ret = []
        elif not isinstance(ret, (list, tuple)):
            ret = [ret]
        ret = list(ret)
        n_user = len(ret)

        aliased = {}  # result index -> (param name, param index)
        for name, ref in params:
            if not ref._is_mutated:
                continue
            pv = ref._original_parameter
            pv.name = f"{name}.must_alias_input"
            pos = next((i for i, r in enumerate(ret) if r is ref), None)
            if pos is None:
                ret.append(ref)
                pos = len(ret) - 1
            aliased[pos] = (name, pv.parameter_id)

        for i, r in enumerate(ret):
            if not isinstance(r, NKIPyTensorRef):
                raise RuntimeError(f"Unexpected return value type: {type(r)}")
            if i in aliased:
                continue
            v = r.backend_tensor
            if v.is_parameter or any(v is ret[j].backend_tensor for j in range(i)):
                ret[i] = NKIPyTensorRef(ctx.build_op("copy", [v], v.shape, v.dtype))

        for i, r in enumerate(ret):
            v = r.backend_tensor
            if i in aliased:
                name, pidx = aliased[i]
                graph.aliases.append(AliasInfo(i, pidx, name, i < n_user))
                v.name = name
            elif not v.name:
                v.name = f"output{i}"
        graph.set_results([r.backend_tensor for r in ret])

    @classmethod
    def trace(cls, func=None, backend="hip", **kwargs):
        if func is None:
            return lambda f: cls(f, backend, **kwargs)
        return cls(func, backend, **kwargs)


trace = NKIPyKernel.trace
