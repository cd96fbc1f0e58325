"""One-shot execution of traced kernels on NumPy arrays.

``baremetal_run_traced_kernel`` keeps the reference's behaviour
(nkipy/src/nkipy/runtime/execute.py:23-178): trace on the arguments, build
the device kernel, copy the inputs in, run, copy the outputs back; results
aliased to a mutated input (``.must_alias_input``) are written back into
the caller's array, and auto-aliased results (mutated but not returned) are
left out of the return value.  Returns one array, a tuple, or None.
"""

from __future__ import annotations

import numpy as np

from nkipy_amd.core.trace import _sanitize_array_dtype, kernel_signature
from nkipy_amd.runtime.device_kernel import DeviceKernel
from nkipy_amd.runtime.device_tensor import DeviceTensor


def baremetal_run_traced_kernel(kernel, *args, artifacts_dir=None, save_trace=False,
                                additional_compiler_args="", target=None, **kwargs):
    args = tuple(_sanitize_array_dtype(a, f"arg{i}") if isinstance(a, np.ndarray) else a
                 for i, a in enumerate(args))
    kwargs = {k: _sanitize_array_dtype(v, k) if isinstance(v, np.ndarray) else v
              for k, v in kwargs.items()}
    dk = DeviceKernel.compile_and_load(kernel, *args, name=kernel.__name__,
                                       additional_compiler_args=additional_compiler_args,
                                       build_dir=artifacts_dir)
    graph = dk.graph
    sig = kernel_signature(kernel.func if hasattr(kernel, "func") else kernel, len(args), kwargs)
    bound = sig.bind(*args, **kwargs)
    bound.apply_defaults()
    arrays = {}
    for name, a in bound.arguments.items():
        p = sig.parameters[name]
        if p.kind == p.VAR_POSITIONAL:
            for i, item in enumerate(a):
                arrays[f"{name}_{i}"] = item
        elif p.kind == p.VAR_KEYWORD:
            arrays.update(a)
        else:
            arrays[name] = a

    inputs = {}
    for prm in graph.parameters:
        base = prm.name.split(".must_alias_input")[0]
        src = arrays[base]
        inputs[prm.name] = src if isinstance(src, DeviceTensor) else DeviceTensor.from_numpy(
            np.asarray(src) if not hasattr(src, "detach") else src.detach().cpu().numpy(), name=prm.name)
    alias_by_out = {a.output_index: a for a in graph.aliases}
    outputs = {}
    for i, r in enumerate(graph.results):
        if i in alias_by_out:
            outputs[r.name] = inputs[f"{alias_by_out[i].param_name}.must_alias_input"]
        else:
            outputs[r.name] = DeviceTensor.empty(r.shape, r.dtype, name=r.name)
    dk(inputs=inputs, outputs=outputs, save_trace=save_trace)

    results = []
    for i, r in enumerate(graph.results):
        host = outputs[r.name].numpy()
        if i in alias_by_out:
            dst = arrays[alias_by_out[i].param_name]
            if isinstance(dst, np.ndarray):
                np.copyto(dst, host.view(dst.dtype) if dst.dtype != host.dtype else host)
                host = dst
        results.append(host)
    auto = graph.auto_aliased_indices
    user = [r for i, r in enumerate(results) if i not in auto]
    if len(user) == 1:
        return user[0]
    if user:
        return tuple(user)
    return None
