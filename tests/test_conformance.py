"""Conformance suite over the kernel specifications in tests/kernel_specs/.

Every module there lists ``kernel_specs`` (the interface of the reference's
tests/kernels/*.py, collected the way tests/integration/test_kernels.py:
19-93 collects them).  Each spec is

* traced and lowered on the CPU at its default shapes (no device needed:
  the reference's ``trace_and_compile`` leg);
* run on the GPU at its default inputs and compared with the same function
  run by NumPy (the reference's ``on_device_test`` leg);
* for specs whose inputs are all generated (no fixed data), swept over
  shapes and dtypes drawn inside its ``ShapeSpec`` / ``TypeSpec`` with a
  fixed seed (tests/integration/test_kernels_fuzz.py:73-123).

Bars: fp32 results |got - ref| <= 1e-4 |ref| + 1e-4 max(1, RMS(ref)) -- the
reference's CPU bar (tests/utils.py:17-18) with the absolute part scaled to
the output; fp16 results 1e-2 on both parts (its device bar, tests/utils.py:
19-20, fp16 ops being rounded per op by NumPy and once by the fused
programs); integer and boolean results exactly.
"""

import glob
import importlib
import os

import numpy as np
import pytest
from parity import assert_matches_numpy

from nkipy_amd.core.specs import TensorInputSpec
from nkipy_amd.core.trace import NKIPyKernel
from nkipy_amd.dispatch.lower import lower


def collect_kernel_specs():
    specs = {}
    here = os.path.join(os.path.dirname(__file__), "kernel_specs")
    for path in sorted(glob.glob(os.path.join(here, "*.py"))):
        mod_name = os.path.splitext(os.path.basename(path))[0]
        if mod_name == "__init__":
            continue
        mod = importlib.import_module(f"kernel_specs.{mod_name}")
        for i, spec in enumerate(getattr(mod, "kernel_specs", [])):
            specs[f"{mod_name}:{i}"] = spec
    return specs


SPECS = collect_kernel_specs()
SWEPT = {k: s for k, s in SPECS.items()
         if all(isinstance(i, TensorInputSpec) and i.default_value is None for i in s.inputs)}
SWEEP_DRAWS = 4


@pytest.mark.parametrize("name", sorted(SPECS))
def test_spec_traces_and_lowers(name):
    """Trace at the default shapes and lower to a plan of gfx950 launches."""
    spec = SPECS[name]
    assert spec.is_pure_numpy
    plan = lower(NKIPyKernel.trace(spec.function).specialize(*spec.input_stubs()))
    assert plan.steps, name
    for i, s in zip(spec.inputs, spec.input_stubs()):
        if isinstance(i, TensorInputSpec):
            assert i.shape_spec.is_valid(s.shape) and i.dtype_spec.is_valid(s.dtype), (name, i.description)


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(SPECS))
def test_spec_default_inputs(gpu, name):
    from nkipy_amd.runtime import baremetal_jit

    print(f"conformance default {name}", flush=True)
    spec = SPECS[name]
    inputs = spec.default_inputs(np.random.default_rng(0))
    for i, x in zip(spec.inputs, inputs):
        if isinstance(i, TensorInputSpec):
            assert i.shape_spec.is_valid(np.shape(x)) and i.dtype_spec.is_valid(x.dtype), (name, i.description)
    expected = spec.function(*[np.copy(x) if isinstance(x, np.ndarray) else x for x in inputs])
    got = baremetal_jit(spec.function)(*inputs)
    assert_matches_numpy(got, expected, name)


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(SWEPT))
def test_spec_sweep(gpu, name):
    """Shapes and dtypes drawn inside the spec, fixed seed per spec."""
    from nkipy_amd.runtime import baremetal_jit

    spec = SWEPT[name]
    rng = np.random.default_rng(sum(map(ord, name)))
    for draw in range(SWEEP_DRAWS):
        inputs = spec.draw_inputs(rng)
        desc = ", ".join(f"{x.dtype}{list(x.shape)}" for x in inputs)
        print(f"conformance sweep {name} draw {draw}: {desc}", flush=True)
        for i, x in zip(spec.inputs, inputs):
            assert i.shape_spec.is_valid(x.shape) and i.dtype_spec.is_valid(x.dtype)
        expected = spec.function(*[np.copy(x) for x in inputs])
        got = baremetal_jit(spec.function)(*inputs)
        assert_matches_numpy(got, expected, f"{name} draw {draw} ({desc})")
