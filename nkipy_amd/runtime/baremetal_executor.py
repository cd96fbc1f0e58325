"""``BaremetalExecutor`` and ``CompiledKernel`` (reference:
nkipy/src/nkipy/runtime/baremetal_executor.py:18-202).

A ``CompiledKernel`` pairs a traced kernel with its compiled artefact (the
plan file ``compile_to_neff`` writes).  ``BaremetalExecutor.run`` loads the
artefact as a ``DeviceKernel``, copies the NumPy arguments in, runs it,
writes aliased results back into the caller's arrays and returns the
kernel's own results (one array, a tuple, or None); ``benchmark`` returns
the ``BenchmarkResult`` of ``DeviceKernel.benchmark``.
"""

from __future__ import annotations

import os
from typing import Dict, Optional, Tuple

import numpy as np

from nkipy_amd.core.trace import kernel_signature
from nkipy_amd.runtime.device_kernel import DeviceKernel
from nkipy_amd.runtime.device_tensor import DeviceTensor


class CompiledKernel:
    def __init__(self, traced_kernel, compiled_artifact):
        self.traced_kernel = traced_kernel
        if not os.path.exists(compiled_artifact):
            raise FileNotFoundError(f"Compiled artifact not found: {compiled_artifact}")
        self.compiled_artifact = os.path.abspath(compiled_artifact)
        self.ir = traced_kernel._code


class BaremetalExecutor:
    def __init__(self, verbose: int = 0):
        self.verbose = verbose
        self._loaded: Dict[str, DeviceKernel] = {}

    def __enter__(self):
        return self

    def __exit__(self, exc_type, exc_val, exc_tb):
        self._loaded.clear()

    def _device_kernel(self, ck: CompiledKernel) -> DeviceKernel:
        dk = self._loaded.get(ck.compiled_artifact)
        if dk is None:
            dk = DeviceKernel.load_from_neff(ck.compiled_artifact, name=ck.traced_kernel.__name__)
            self._loaded[ck.compiled_artifact] = dk
        return dk

    def _prepare_io_tensors(self, ck: CompiledKernel, dk: DeviceKernel, *args,
                            **kwargs) -> Tuple[Dict[str, DeviceTensor], Dict[str, DeviceTensor], Dict[str, np.ndarray]]:
        sig = kernel_signature(ck.traced_kernel.func, len(args), kwargs)
        bound = sig.bind(*args, **kwargs)
        bound.apply_defaults()
        originals = {n: a for n, a in bound.arguments.items() if isinstance(a, np.ndarray)}
        inputs = {}
        for p in ck.ir.inputs:
            real = p.name.split(".must_alias_input")[0]
            src = originals.get(real, bound.arguments.get(real))
            inputs[p.name] = src if isinstance(src, DeviceTensor) else DeviceTensor.from_numpy(np.asarray(src),
                                                                                               name=p.name)
        outputs = {t.name: t for t in dk.allocate_output_tensors()}
        for a in ck.ir.aliases:
            outputs[ck.ir.outputs[a.output_index].name] = inputs[f"{a.param_name}.must_alias_input"]
        return inputs, outputs, originals

    def benchmark(self, compiled_kernel: CompiledKernel, *args, warmup_iterations: int = 5,
                  benchmark_iterations: int = 100, mode: str = "device", artifacts_dir: Optional[str] = None,
                  **kwargs):
        dk = self._device_kernel(compiled_kernel)
        inputs, outputs, _ = self._prepare_io_tensors(compiled_kernel, dk, *args, **kwargs)
        return dk.benchmark(inputs=inputs, outputs=outputs, warmup_iter=warmup_iterations,
                            benchmark_iter=benchmark_iterations, mode=mode)

    def run(self, compiled_kernel: CompiledKernel, *args, save_trace: bool = False,
            artifacts_dir: Optional[str] = None, **kwargs):
        dk = self._device_kernel(compiled_kernel)
        inputs, outputs, originals = self._prepare_io_tensors(compiled_kernel, dk, *args, **kwargs)
        dk(inputs=inputs, outputs=outputs, save_trace=save_trace)
        ir = compiled_kernel.ir
        for a in ir.aliases:
            host = outputs[ir.outputs[a.output_index].name].numpy()
            dst = originals.get(a.param_name)
            if dst is not None:
                np.copyto(dst, host.view(dst.dtype) if dst.dtype != host.dtype else host)
        user = [outputs[t.name].numpy() for i, t in enumerate(ir.outputs) if i not in ir.auto_aliased_indices]
        if len(user) == 1:
            return user[0]
        if user:
            return tuple(user)
        return None
