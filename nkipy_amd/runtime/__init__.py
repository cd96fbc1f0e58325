"""Device runtime: tensors, loaded kernels and the jit entry points."""

from nkipy_amd.dispatch.launchers import LinearAttentionRangeError
from nkipy_amd.runtime.baremetal_executor import BaremetalExecutor, CompiledKernel
from nkipy_amd.runtime.decorators import baremetal_jit
from nkipy_amd.runtime.device_kernel import BenchmarkResult, DeviceKernel
from nkipy_amd.runtime.device_tensor import DeviceTensor
from nkipy_amd.runtime.execute import baremetal_run_traced_kernel
from nkipy_amd.runtime.hip import HipError, NrtError, SpikeError, SpikeRuntimeError
from nkipy_amd.runtime.utils import is_gpu_available, is_neuron_compatible

__all__ = [
    "BaremetalExecutor", "CompiledKernel", "baremetal_jit", "baremetal_run_traced_kernel", "BenchmarkResult", "DeviceKernel",
    "DeviceTensor", "HipError", "LinearAttentionRangeError", "NrtError", "SpikeError", "SpikeRuntimeError",
    "is_gpu_available", "is_neuron_compatible",
]
